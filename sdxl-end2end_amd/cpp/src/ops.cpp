// Ops::attention over the C ABI (see ops.hpp). Validation, eligibility errors
// and the profile label follow the reference's Ops::attention
// (src/cuda/ops_kernels.cu:1912-1973).
#include "sdxl_hip/ops.hpp"

#include "sdxl_hip/attention.h"

#include <sstream>

namespace sdxl::hip {

namespace {

std::int32_t dtype_code(ScalarType type) {
    switch (type) {
    case ScalarType::Float16: return SDXL_DTYPE_F16;
    case ScalarType::BFloat16: return SDXL_DTYPE_BF16;
    case ScalarType::Float32: return SDXL_DTYPE_F32;
    default: throw HipError("CUDA attention mismatch");
    }
}

void validate(const Tensor& query, const Tensor& key, const Tensor& value, std::size_t heads, const Tensor* key_mask) {
    if (query.rank() != 3 || key.rank() != 3 || value.shape() != key.shape() || query.type() != key.type() ||
        value.type() != key.type() ||
        (query.type() != ScalarType::Float16 && query.type() != ScalarType::BFloat16 &&
         query.type() != ScalarType::Float32) ||
        query.size(0) != key.size(0) || query.size(2) != key.size(2) || heads == 0 || query.size(2) % heads != 0)
        throw HipError("CUDA attention mismatch");
    const std::size_t head_dimension = query.size(2) / heads;
    if (head_dimension == 0 || head_dimension > 1024)
        throw HipError("CUDA attention head dimension must be in [1,1024]");
    if (key_mask != nullptr && (key_mask->type() != ScalarType::Int32 || key_mask->rank() != 2 ||
                                key_mask->size(0) != key.size(0) || key_mask->size(1) != key.size(1)))
        throw HipError("CUDA attention key mask mismatch");
}

}  // namespace

Ops::Ops(const Runtime& runtime) : runtime_(&runtime) {}

Tensor Ops::attention(const Tensor& query, const Tensor& key, const Tensor& value, std::size_t heads, bool causal,
                      const Tensor* key_mask) const {
    validate(query, key, value, heads, key_mask);
    Tensor output = Tensor::allocate(*runtime_, query.shape(), query.type());
    attention_into(query, key, value, heads, output, causal, key_mask);
    return output;
}

void Ops::attention_into(const Tensor& query, const Tensor& key, const Tensor& value, std::size_t heads,
                         Tensor& output, bool causal, const Tensor* key_mask) const {
    validate(query, key, value, heads, key_mask);
    if (output.shape() != query.shape() || output.type() != query.type()) throw HipError("CUDA attention mismatch");

    sdxl_attn_desc desc{};
    desc.batch = static_cast<std::int64_t>(query.size(0));
    desc.q_seq = static_cast<std::int64_t>(query.size(1));
    desc.k_seq = static_cast<std::int64_t>(key.size(1));
    desc.heads = static_cast<std::int64_t>(heads);
    desc.head_dim = static_cast<std::int64_t>(query.size(2) / heads);
    desc.dtype = dtype_code(query.type());
    desc.causal = causal ? 1 : 0;
    desc.backend = static_cast<std::int32_t>(runtime_->options().attention_backend);

    std::int32_t resolved = 0;
    if (sdxl_attn_resolve_backend(&desc, key_mask != nullptr, &resolved) != SDXL_STATUS_OK)
        throw HipError(sdxl_last_error());

    std::ostringstream label;
    label << "ops/attention/" << sdxl_attn_backend_name(resolved) << "/q" << query.size(1) << "_k" << key.size(1)
          << "_h" << heads << "_d" << desc.head_dim << (causal ? "_causal" : "_full");
    const int scope = runtime_->begin_profile(label.str());
    const sdxl_status status =
        sdxl_attn_fwd(&desc, query.data(), key.data(), value.data(), key_mask ? key_mask->int32_data() : nullptr,
                      output.data(), runtime_->stream());
    runtime_->end_profile(scope);
    if (status != SDXL_STATUS_OK) throw HipError(sdxl_last_error());
}

}  // namespace sdxl::hip

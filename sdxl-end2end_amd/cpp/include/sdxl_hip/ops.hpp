// Operator layer of the sdxl_hip C++20 host API: the attention entry point of
// the reference's Ops (include/sdxl/cuda/ops.hpp:92-97), implemented over the
// C ABI sdxl_attn_fwd (include/sdxl_hip/attention.h).
#pragma once

#include "sdxl_hip/runtime.hpp"
#include "sdxl_hip/tensor.hpp"

#include <cstddef>

namespace sdxl::hip {

class Ops final {
public:
    explicit Ops(const Runtime& runtime);

    // query [B, Sq, H*D], key/value [B, Sk, H*D] (fp16, bf16 or fp32, same type),
    // optional int32 key_mask [B, Sk] (0 hides a key). Returns [B, Sq, H*D] of
    // the query's type. Throws HipError with the reference's messages
    // (src/cuda/ops_kernels.cu:1914-1941). Stream-ordered, no host sync; the
    // output is allocated from the stream-ordered pool.
    [[nodiscard]] Tensor attention(const Tensor& query, const Tensor& key, const Tensor& value, std::size_t heads,
                                   bool causal = false, const Tensor* key_mask = nullptr) const;

    // Same computation into a caller-owned output (no allocation at all).
    void attention_into(const Tensor& query, const Tensor& key, const Tensor& value, std::size_t heads,
                        Tensor& output, bool causal = false, const Tensor* key_mask = nullptr) const;

private:
    const Runtime* runtime_ = nullptr;
};

}  // namespace sdxl::hip

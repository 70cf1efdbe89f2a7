// C ABI of the attention library: validation, backend selection and launch.
//
// Mirrors the host half of the reference's Ops::attention
// (src/cuda/ops_kernels.cu:1912-2010): the same shape/dtype/mask checks, the
// same eligibility errors for explicitly requested backends, then one
// stream-ordered kernel launch. No allocation and no host synchronisation.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cctype>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>

#include "../../include/sdxl_hip/attention.h"
#include "attention_kernels.hpp"
#include "capi_internal.hpp"

namespace {

thread_local std::string g_last_error;

}  // namespace

sdxl_status sdxl_hip_fail(sdxl_status status, const std::string& message) {
    g_last_error = message;
    return status;
}

int sdxl_hip_compute_units() {
    static std::atomic<int> cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int cus = cached[dev].load(std::memory_order_relaxed);
    if (cus == 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = -1;
        cached[dev].store(cus, std::memory_order_relaxed);
    }
    return cus > 0 ? cus : 0;
}

namespace {

sdxl_status fail(sdxl_status status, const std::string& message) { return sdxl_hip_fail(status, message); }

int64_t eff_stride(int64_t stride, int64_t width) { return stride == 0 ? width : stride; }

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

int compute_units() { return sdxl_hip_compute_units(); }

// Checks everything sdxl_attn_fwd checks that does not involve pointers.
sdxl_status validate_desc(const sdxl_attn_desc* d) {
    if (d == nullptr) return fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_attn: null descriptor");
    if (d->reserved != 0) return fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_attn: reserved field must be 0");
    if (d->dtype < SDXL_DTYPE_F16 || d->dtype > SDXL_DTYPE_F32)
        return fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_attn: unknown dtype");
    if (d->backend < SDXL_ATTN_AUTO || d->backend > SDXL_ATTN_WARP_ONLINE)
        return fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_attn: unknown backend");
    // Reference ops_kernels.cu:1914-1922.
    if (d->batch < 0 || d->q_seq < 0 || d->k_seq < 0 || d->heads <= 0 || d->head_dim <= 0)
        return fail(SDXL_STATUS_INVALID_SHAPE, "CUDA attention mismatch");
    if (d->head_dim > 1024)
        return fail(SDXL_STATUS_INVALID_SHAPE, "CUDA attention head dimension must be in [1,1024]");
    const int64_t width = d->heads * d->head_dim;
    const int64_t strides[4] = {d->q_row_stride, d->k_row_stride, d->v_row_stride, d->o_row_stride};
    for (int64_t s : strides) {
        if (s != 0 && s < width) return fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_attn: row stride smaller than heads*head_dim");
    }
    if (d->batch > INT32_MAX || d->q_seq > INT32_MAX || d->k_seq > INT32_MAX || d->heads > INT32_MAX)
        return fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_attn: dimension exceeds int32");
    if (!(d->scale >= 0.0f) || std::isinf(d->scale))
        return fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_attn: scale must be finite and >= 0");
    return SDXL_STATUS_OK;
}

// Fused-kernel eligibility (pointer-independent part): fp16/bf16, head_dim 64,
// every row stride a multiple of 8 elements (16-byte rows) and below 2^23
// elements (the kernel forms K/V row offsets with 24-bit multiplies).
bool fused_shape_eligible(const sdxl_attn_desc* d) {
    if (d->dtype != SDXL_DTYPE_F16 && d->dtype != SDXL_DTYPE_BF16) return false;
    if (d->head_dim != 64) return false;
    const int64_t width = d->heads * d->head_dim;
    const int64_t strides[4] = {eff_stride(d->q_row_stride, width), eff_stride(d->k_row_stride, width),
                                eff_stride(d->v_row_stride, width), eff_stride(d->o_row_stride, width)};
    for (int64_t s : strides)
        if (s % 8 != 0 || s >= (int64_t{1} << 23)) return false;
    return true;
}

sdxl_status resolve(const sdxl_attn_desc* d, bool has_mask, int32_t* out) {
    const bool fused = fused_shape_eligible(d);
    // cudnn-sdpa in the reference also refuses an explicit key mask
    // (ops_kernels.cu:1931-1937); keep that contract.
    switch (d->backend) {
    case SDXL_ATTN_CUDNN_SDPA:
        if (!fused || has_mask)
            return fail(SDXL_STATUS_UNSUPPORTED,
                        "cudnn-sdpa requires FP16/BF16, no explicit key mask, and head dimension 64 on gfx950");
        *out = SDXL_ATTN_CUDNN_SDPA;
        return SDXL_STATUS_OK;
    case SDXL_ATTN_FLASH_SM80:
        if (!fused)
            return fail(SDXL_STATUS_UNSUPPORTED,
                        "flash attention requires FP16/BF16, head dimension 64 and 16-byte aligned rows");
        *out = SDXL_ATTN_FLASH_SM80;
        return SDXL_STATUS_OK;
    case SDXL_ATTN_WARP_ONLINE:
        *out = SDXL_ATTN_WARP_ONLINE;
        return SDXL_STATUS_OK;
    default:
        *out = fused ? SDXL_ATTN_FLASH_SM80 : SDXL_ATTN_WARP_ONLINE;
        return SDXL_STATUS_OK;
    }
}

}  // namespace

extern "C" {

int32_t sdxl_abi_version(void) { return SDXL_HIP_ABI_VERSION; }

const char* sdxl_last_error(void) { return g_last_error.c_str(); }

const char* sdxl_status_string(sdxl_status status) {
    switch (status) {
    case SDXL_STATUS_OK: return "ok";
    case SDXL_STATUS_INVALID_ARGUMENT: return "invalid argument";
    case SDXL_STATUS_INVALID_SHAPE: return "invalid shape";
    case SDXL_STATUS_UNSUPPORTED: return "unsupported";
    case SDXL_STATUS_LAUNCH_FAILED: return "launch failed";
    case SDXL_STATUS_DEVICE_ERROR: return "device error";
    }
    return "unknown status";
}

const char* sdxl_attn_backend_name(int32_t backend) {
    switch (backend) {
    case SDXL_ATTN_AUTO: return "auto";
    case SDXL_ATTN_CUDNN_SDPA: return "cudnn-sdpa";
    case SDXL_ATTN_FLASH_SM80: return "flash-sm80";
    case SDXL_ATTN_WARP_ONLINE: return "warp-online";
    }
    return "unknown";
}

const char* sdxl_attn_kernel_name(int32_t resolved_backend) {
    switch (resolved_backend) {
    case SDXL_ATTN_CUDNN_SDPA:
    case SDXL_ATTN_FLASH_SM80: return "flash-gfx950";
    case SDXL_ATTN_WARP_ONLINE: return "wave-online";
    }
    return "unknown";
}

sdxl_status sdxl_attn_backend_parse(const char* name, int32_t* backend) {
    if (name == nullptr || backend == nullptr) return fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_attn: null argument");
    std::string s(name);
    for (char& ch : s) ch = static_cast<char>(std::tolower(static_cast<unsigned char>(ch)));
    if (s == "auto") { *backend = SDXL_ATTN_AUTO; return SDXL_STATUS_OK; }
    if (s == "cudnn" || s == "cudnn-sdpa" || s == "sdpa") { *backend = SDXL_ATTN_CUDNN_SDPA; return SDXL_STATUS_OK; }
    if (s == "flash" || s == "flash-sm80" || s == "flash2" || s == "flash-gfx950") {
        *backend = SDXL_ATTN_FLASH_SM80;
        return SDXL_STATUS_OK;
    }
    if (s == "warp" || s == "warp-online" || s == "reference" || s == "wave-online") {
        *backend = SDXL_ATTN_WARP_ONLINE;
        return SDXL_STATUS_OK;
    }
    return fail(SDXL_STATUS_INVALID_ARGUMENT, "attention backend must be auto, cudnn-sdpa, flash-sm80, or warp-online");
}

sdxl_status sdxl_attn_resolve_backend(const sdxl_attn_desc* desc, int32_t has_key_mask, int32_t* resolved) {
    if (resolved == nullptr) return fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_attn: null argument");
    sdxl_status st = validate_desc(desc);
    if (st != SDXL_STATUS_OK) return st;
    return resolve(desc, has_key_mask != 0, resolved);
}

sdxl_status sdxl_attn_fwd(const sdxl_attn_desc* d, const void* q, const void* k, const void* v,
                          const int32_t* key_mask, void* o, void* stream) {
    sdxl_status st = validate_desc(d);
    if (st != SDXL_STATUS_OK) return st;
    int32_t backend = 0;
    st = resolve(d, key_mask != nullptr, &backend);
    if (st != SDXL_STATUS_OK) return st;
    if (d->batch == 0 || d->q_seq == 0) return SDXL_STATUS_OK;  // empty output
    if (q == nullptr || o == nullptr || (d->k_seq > 0 && (k == nullptr || v == nullptr)))
        return fail(SDXL_STATUS_INVALID_ARGUMENT, "sdxl_attn: null tensor pointer");

    const int64_t width = d->heads * d->head_dim;
    const float scale = d->scale > 0.0f ? d->scale : 1.0f / std::sqrt(static_cast<float>(d->head_dim));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);

    if (backend != SDXL_ATTN_WARP_ONLINE) {
        if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) {
            if (d->backend != SDXL_ATTN_AUTO)
                return fail(SDXL_STATUS_UNSUPPORTED, "flash attention requires 16-byte aligned q/k/v/o");
            backend = SDXL_ATTN_WARP_ONLINE;
        }
    }

    // The fused kernels form exp2 arguments as c * S and shift raw scores by
    // m / c (c = scale * log2 e); a scale so small that 1 / c overflows runs
    // on the per-row kernel, which multiplies by the scale directly.
    const float scale_log2 = scale * 1.4426950408889634f;
    if (backend != SDXL_ATTN_WARP_ONLINE && !std::isfinite(1.0f / scale_log2)) backend = SDXL_ATTN_WARP_ONLINE;

    hipError_t err;
    if (backend == SDXL_ATTN_WARP_ONLINE) {
        sdxl_hip::OnlineAttentionParams p{};
        p.q = q; p.k = k; p.v = v; p.key_mask = key_mask; p.o = o;
        p.q_row_stride = eff_stride(d->q_row_stride, width);
        p.k_row_stride = eff_stride(d->k_row_stride, width);
        p.v_row_stride = eff_stride(d->v_row_stride, width);
        p.o_row_stride = eff_stride(d->o_row_stride, width);
        p.batch = (int32_t)d->batch; p.q_seq = (int32_t)d->q_seq; p.k_seq = (int32_t)d->k_seq;
        p.heads = (int32_t)d->heads; p.head_dim = (int32_t)d->head_dim; p.causal = d->causal != 0;
        p.scale = scale;
        // FP32 at head_dim 512 (the VAE's attention) runs on the fp32 matrix
        // cores when the call allows (auto backend, no mask, non-causal,
        // aligned rows); an explicit warp-online request keeps the per-row kernel.
        if (d->backend == SDXL_ATTN_AUTO && sdxl_hip::attention_f32_d512_eligible(p, d->dtype))
            err = sdxl_hip::launch_attention_f32_d512(p, compute_units(), s);
        else err = sdxl_hip::launch_online_attention(p, d->dtype, s);
    } else {
        sdxl_hip::FusedAttentionParams p{};
        p.q = q; p.k = k; p.v = v; p.key_mask = key_mask; p.o = o;
        p.q_row_stride = eff_stride(d->q_row_stride, width);
        p.k_row_stride = eff_stride(d->k_row_stride, width);
        p.v_row_stride = eff_stride(d->v_row_stride, width);
        p.o_row_stride = eff_stride(d->o_row_stride, width);
        p.batch = (int32_t)d->batch; p.q_seq = (int32_t)d->q_seq; p.k_seq = (int32_t)d->k_seq;
        p.heads = (int32_t)d->heads; p.causal = d->causal != 0;
        p.scale_log2 = scale_log2;
        p.inv_scale_log2 = 1.0f / scale_log2;
        const int64_t blocks = ((d->q_seq + sdxl_hip::fused_attention_block_queries() - 1) /
                                sdxl_hip::fused_attention_block_queries()) * d->heads * d->batch;
        if (blocks > INT32_MAX) return fail(SDXL_STATUS_INVALID_SHAPE, "sdxl_attn: grid too large");
        err = sdxl_hip::launch_fused_attention_d64(p, d->dtype == SDXL_DTYPE_BF16, compute_units(), s);
    }
    if (err != hipSuccess)
        return fail(SDXL_STATUS_LAUNCH_FAILED, std::string("sdxl_attn launch: ") + hipGetErrorString(err));
    return SDXL_STATUS_OK;
}

}  // extern "C"

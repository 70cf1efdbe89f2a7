/*
 * sdxl_hip attention C ABI: the drop-in boundary for the SDXL UNet
 * SpatialTransformer attention on MI355X (gfx950).
 *
 * Plain C: pointers, sizes and status codes only. The stream argument is a
 * hipStream_t passed as void* so that FFI callers (ctypes, cgo, JNI) need no
 * HIP headers. Device pointers are HIP device memory.
 *
 * Tensor layout (all of q, k, v, o): row-major [batch, seq, row_stride] with
 * head h occupying elements [h*head_dim, (h+1)*head_dim) of each row, i.e. the
 * [B, S, H*D] "BSHD" storage the reference passes between its linears and its
 * attention (reference src/cuda/flash_attention_sm80.cu:81-83,
 * src/unet.cpp:463). A row stride larger than heads*head_dim lets q/k/v be
 * column slices of one fused [B, S, 3*H*D] projection output.
 */
#ifndef SDXL_HIP_ATTENTION_H
#define SDXL_HIP_ATTENTION_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SDXL_HIP_ABI_VERSION 2

typedef enum sdxl_status {
    SDXL_STATUS_OK = 0,
    SDXL_STATUS_INVALID_ARGUMENT = 1, /* null pointer, unknown enum value */
    SDXL_STATUS_INVALID_SHAPE = 2,    /* shape/stride/dtype mismatch ("CUDA attention mismatch") */
    SDXL_STATUS_UNSUPPORTED = 3,      /* requested backend not eligible for this call */
    SDXL_STATUS_LAUNCH_FAILED = 4,    /* hipGetLastError after the launch was not hipSuccess */
    SDXL_STATUS_DEVICE_ERROR = 5      /* device query failed (no GPU, wrong architecture) */
} sdxl_status;

typedef enum sdxl_dtype {
    SDXL_DTYPE_F16 = 0,
    SDXL_DTYPE_BF16 = 1,
    SDXL_DTYPE_F32 = 2,
    SDXL_DTYPE_E4M3 = 3 /* FP8 E4M3 (finite-only, bias 7): linear weights only */
} sdxl_dtype;

/* Backend selection. Values and accepted spellings mirror the reference's
 * AttentionBackend (include/sdxl/cuda/runtime.hpp:53-58,
 * src/cuda/runtime.cpp:61-77). On MI355X:
 *   CUDNN_SDPA and FLASH_SM80 both run the fused gfx950 MFMA kernel
 *     (the reference's vendor FA-2 graph and in-tree tiled kernel are the
 *     two "fast" backends it replaces);
 *   WARP_ONLINE runs the wave64 online-softmax kernel (the reference's
 *     correctness fallback, any head_dim <= 1024, f16/bf16/f32);
 *   AUTO picks the fused kernel whenever it is eligible, else WARP_ONLINE,
 *     whose unmasked non-causal FP32 calls at head_dim 512 (the VAE) run a
 *     tiled fp32 matrix-core kernel instead of the per-row one. */
typedef enum sdxl_attn_backend {
    SDXL_ATTN_AUTO = 0,
    SDXL_ATTN_CUDNN_SDPA = 1,
    SDXL_ATTN_FLASH_SM80 = 2,
    SDXL_ATTN_WARP_ONLINE = 3
} sdxl_attn_backend;

typedef struct sdxl_attn_desc {
    int64_t batch;
    int64_t q_seq;
    int64_t k_seq;
    int64_t heads;
    int64_t head_dim;
    /* Row strides in elements; 0 means heads*head_dim (contiguous BSHD). */
    int64_t q_row_stride;
    int64_t k_row_stride;
    int64_t v_row_stride;
    int64_t o_row_stride;
    int32_t dtype;    /* sdxl_dtype, same for q, k, v and o */
    int32_t causal;   /* nonzero: key j visible to query i only when j <= i */
    int32_t backend;  /* sdxl_attn_backend */
    int32_t reserved; /* must be 0 */
    float scale;      /* softmax scale; 0 means 1/sqrt(head_dim) */
} sdxl_attn_desc;

/* Forward attention: o = softmax(q k^T * scale [masked]) v, per (batch, head).
 * Replaces Ops::attention (reference include/sdxl/cuda/ops.hpp:92-97,
 * src/cuda/ops_kernels.cu:1912-2010) and the backend launchers
 * launch_flash_attention_sm80_hdim64 (src/cuda/flash_attention_sm80.hpp:13-20)
 * and launch_cudnn_frontend_sdpa (src/cuda/cudnn_sdpa.hpp:13-20).
 * key_mask: nullable int32 [batch, k_seq]; 0 hides that key (reference
 * ops_kernels.cu:1923-1926). A query row with no visible key produces zeros.
 * Stream-ordered and asynchronous: no allocation, no host synchronisation,
 * safe to capture in a HIP graph. The output buffer is caller-owned. */
sdxl_status sdxl_attn_fwd(const sdxl_attn_desc* desc, const void* q, const void* k,
                          const void* v, const int32_t* key_mask, void* o, void* stream);

/* Resolves desc->backend (AUTO included) to the backend sdxl_attn_fwd would
 * run, or returns the eligibility error sdxl_attn_fwd would return
 * (reference ops_kernels.cu:1928-1952). Host only: no device call. */
sdxl_status sdxl_attn_resolve_backend(const sdxl_attn_desc* desc, int32_t has_key_mask,
                                      int32_t* resolved_backend);

/* Parses a backend name with the reference's spellings
 * (src/cuda/runtime.cpp:61-77): auto | cudnn, cudnn-sdpa, sdpa |
 * flash, flash-sm80, flash2 | warp, warp-online, reference, plus the native
 * names flash-gfx950 and wave-online. Case-insensitive. Unknown names return
 * SDXL_STATUS_INVALID_ARGUMENT with the reference's message. */
sdxl_status sdxl_attn_backend_parse(const char* name, int32_t* backend);

/* Canonical name of a backend (reference attention_backend_name,
 * src/cuda/runtime.cpp:79-87), or "unknown". */
const char* sdxl_attn_backend_name(int32_t backend);

/* Name of the kernel family a resolved backend runs on this device:
 * "flash-gfx950" or "wave-online". Under the auto backend, unmasked non-causal
 * FP32 calls at head_dim 512 (the VAE's attention) resolve to the online
 * family but run its fp32 matrix-core kernel. */
const char* sdxl_attn_kernel_name(int32_t resolved_backend);

const char* sdxl_status_string(sdxl_status status);

/* Message of the last failing call on this thread ("" if none). */
const char* sdxl_last_error(void);

int32_t sdxl_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SDXL_HIP_ATTENTION_H */

/* C ABI of the transformer attention sublayer on MI355X (gfx950).
 *
 * The reference's UNet transformer block runs, for its self-attention
 * sublayer (src/cuda/unet.cpp:106-118):
 *   normalized = Ops::layer_norm(hidden, norm1.weight, norm1.bias)     eps 1e-5
 *   q, k, v    = Ops::linear(normalized, to_q / to_k / to_v.weight)     no bias
 *   attention  = Ops::attention(q, k, v, heads)
 *   attention  = Ops::linear(attention, to_out.0.weight, &to_out.0.bias)
 *   Ops::add_in_place(hidden, attention)
 * These entry points provide each step (sdxl_layer_norm, sdxl_linear) and the
 * whole sublayer in one call (sdxl_attn_sublayer), with q/k/v as one fused
 * projection against the row-concatenated weight [3W, W]. Linear weights are
 * fp16 or FP8 E4M3 with per-output-channel fp32 scales (the reference's
 * weight-only FP8 path, src/cuda/fp8_kernels.cu:52-245). fp32 accumulation,
 * fp16 storage between steps. All calls are stream-ordered, allocate nothing
 * and never synchronise. Errors as in attention.h (sdxl_last_error()).
 */
#ifndef SDXL_HIP_SUBLAYER_H
#define SDXL_HIP_SUBLAYER_H

#include <stddef.h>
#include <stdint.h>

#include "attention.h"

#ifdef __cplusplus
extern "C" {
#endif

/* LayerNorm over the last dim (Ops::layer_norm, src/cuda/ops_kernels.cu:1428-1460;
 * CPU semantics src/unet.cpp:237-263): y = (x - mean) / sqrt(var + eps) * gamma + beta,
 * two-pass centred variance, fp16 x/gamma/beta/y, fp32 maths. width even, at most
 * 2048 (SDXL: 320, 640, 1280, 2048). eps 0 means 1e-5. Row strides in
 * elements (0 = width). y may equal x. */
sdxl_status sdxl_layer_norm(int64_t rows, int64_t width, const void* x, int64_t x_row_stride,
                            const void* gamma, const void* beta, float eps, void* y,
                            int64_t y_row_stride, void* stream);

/* LayerNorm as sdxl_layer_norm, output quantised for the fp8 projection: the
 * normalised row (fp32) becomes E4M3 codes q [rows, width] (row stride in bytes,
 * 0 = width) with a per-row fp32 scale q_scale [rows] = amax > 0 ?
 * max(amax / 448, 1e-12) : 1, code = E4M3(y / scale) rounded to nearest even and
 * saturated to +-448 (the rule of sdxl_quantize_e4m3_rows). No counterpart in the
 * reference (its FP8 path quantises weights only); feeds sdxl_linear_e4m3. */
sdxl_status sdxl_layer_norm_e4m3(int64_t rows, int64_t width, const void* x, int64_t x_row_stride,
                                 const void* gamma, const void* beta, float eps, uint8_t* q,
                                 int64_t q_row_stride, float* q_scale, void* stream);
typedef struct sdxl_linear_desc {
    int64_t m; /* rows of a and c */
    int64_t n; /* output features (rows of w) */
    int64_t k; /* input features */
    /* Row strides in elements; 0 means dense (k for a and w, n for c and residual). */
    int64_t a_row_stride;
    int64_t w_row_stride;
    int64_t c_row_stride;
    int64_t residual_row_stride;
    int32_t w_dtype; /* SDXL_DTYPE_F16 or SDXL_DTYPE_E4M3; a, c, bias, residual are fp16 */
    int32_t reserved; /* must be 0 */
} sdxl_linear_desc;

/* c = (a . w^T) * w_scale + bias + residual (Ops::linear, src/cuda/ops_blas.cpp;
 * CPU semantics src/unet.cpp:202-222 plus add_in_place). w is [n, k] row-major
 * (the reference's [out, in] storage). w_scale: per-output-channel fp32 scales,
 * required for E4M3 weights (dequantised weight = code * scale), optional (NULL = 1)
 * for fp16. bias [n] and residual [m, n] are optional (NULL). residual may equal c.
 * Requires k % 64 == 0, n % 4 == 0, 16-byte aligned a/w rows and w_scale, 8-byte
 * aligned c/bias/residual rows (SDXL widths all qualify). */
sdxl_status sdxl_linear(const sdxl_linear_desc* desc, const void* a, const void* w, const float* w_scale,
                        const void* bias, const void* residual, void* c, void* stream);
/* sdxl_linear with FP8 activations on the fp8 matrix cores:
 * c = (a . w^T) * a_scale[m] * w_scale[n] + bias + residual, a E4M3 codes [m, k]
 * (desc->a_row_stride in bytes) with per-row fp32 scales a_scale [m] (as written by
 * sdxl_layer_norm_e4m3), w E4M3 [n, k] with w_scale [n] (desc->w_dtype must be
 * SDXL_DTYPE_E4M3). fp32 accumulation of exact fp8 products. Same shape and
 * alignment rules as sdxl_linear. No counterpart in the reference (weight-only FP8
 * there, src/cuda/fp8_kernels.cu:52-245); the optional fp8 QKV projection. */
sdxl_status sdxl_linear_e4m3(const sdxl_linear_desc* desc, const uint8_t* a, const float* a_scale, const void* w,
                             const float* w_scale, const void* bias, const void* residual, void* c,
                             void* stream);

/* Per-output-channel E4M3 quantisation of an fp16 weight [rows, cols] (the
 * reference's FP8 weight packing, src/cuda/weights.cu:119-170): scale[r] =
 * amax_r > 0 ? max(amax_r / 448, 1e-12) : 1 over finite values; q = E4M3(w / scale)
 * rounded to nearest even, saturated to +-448. */
sdxl_status sdxl_quantize_e4m3_rows(int64_t rows, int64_t cols, const void* w, uint8_t* q, float* scales,
                                    void* stream);

/* LayerNorm fused into the projection that consumes it, for the transformer
 * block's norm1 -> q|k|v (reference src/cuda/unet.cpp:106-112: Ops::layer_norm,
 * src/cuda/ops_kernels.cu:1428-1460, then Ops::linear on FP8 weights,
 * src/cuda/fp8_kernels.cu:52-245): c = LN(x) . w^T * w_scale (+ bias), with LN(x)
 * rounded to fp16 exactly as sdxl_layer_norm rounds it and the same fp32 sums as
 * sdxl_linear, so c equals sdxl_layer_norm followed by sdxl_linear bit for bit;
 * the normalised rows never reach HBM. desc as sdxl_linear (k = width, a_row_stride
 * = x row stride; w_dtype must be SDXL_DTYPE_E4M3; residual_row_stride 0). eps 0
 * means 1e-5. SDXL_STATUS_UNSUPPORTED unless k == 640 or k == 1280, n % 128 == 0, 16-byte
 * aligned x rows, gamma, beta and w rows, 8-byte aligned c rows. */
sdxl_status sdxl_layer_norm_linear(const sdxl_linear_desc* desc, const void* x, const void* gamma,
                                   const void* beta, float eps, const void* w, const float* w_scale,
                                   const void* bias, void* c, void* stream);

/* sdxl_layer_norm_linear with FP8 activations on the fp8 matrix cores: the LayerNorm rounds each
 * normalised row to E4M3 codes with its per-row scale exactly as sdxl_layer_norm_e4m3 does, and
 * c = codes . w^T * row_scale * w_scale (+ bias), the same bits as sdxl_layer_norm_e4m3 followed by
 * sdxl_linear_e4m3; neither the codes nor the scales reach HBM. No counterpart in the reference
 * (weight-only FP8 there): the fused form of the optional fp8 QKV projection. Same arguments and
 * shape rules as sdxl_layer_norm_linear. */
sdxl_status sdxl_layer_norm_linear_e4m3(const sdxl_linear_desc* desc, const void* x, const void* gamma,
                                        const void* beta, float eps, const void* w, const float* w_scale,
                                        const void* bias, void* c, void* stream);

typedef struct sdxl_sublayer_desc {
    int64_t batch;
    int64_t seq;
    int64_t heads;     /* width = heads * 64 */
    int32_t w_qkv_dtype; /* SDXL_DTYPE_F16 or SDXL_DTYPE_E4M3 */
    int32_t attn_backend; /* sdxl_attn_backend for the attention step */
    float ln_eps;      /* 0 means 1e-5 */
    /* Activations of the QKV projection: SDXL_DTYPE_F16 (0: the reference's
     * weight-only FP8, fp16 MFMA) or SDXL_DTYPE_E4M3 (LayerNorm quantises its
     * output per row and the projection runs on the fp8 matrix cores; needs E4M3
     * w_qkv). */
    int32_t qkv_activations;
    /* 0: the LayerNorm runs inside the q|k|v projection (sdxl_layer_norm_linear, or
     * sdxl_layer_norm_linear_e4m3 with E4M3 activations) where that kernel takes the
     * shape (E4M3 w_qkv, width 640 or 1280) and is the faster choice (at most two
     * workgroups per 64-row block: the level-1 blocks, not the level-2 ones), else
     * as its own launch; 1: always its own
     * launch. Same results either way. */
    int32_t ln_fusion;
} sdxl_sublayer_desc;

/* Workspace the sublayer needs: batch * seq * width * 8 bytes (normalised
 * hidden / attention output, then the fused q|k|v projection). */
size_t sdxl_attn_sublayer_workspace_bytes(const sdxl_sublayer_desc* desc);

/* y = x + to_out(attention(split_heads(LN(x) . w_qkv^T))) for hidden x [B, S, W]
 * fp16: LayerNorm (gamma, beta [W]), fused q|k|v projection (w_qkv [3W, W] = to_q,
 * to_k, to_v rows concatenated; w_qkv_scale [3W] for E4M3), head-dim-64 attention,
 * output projection (w_out [W, W] fp16, b_out [W]) with the residual added in its
 * epilogue. y may equal x. workspace: sdxl_attn_sublayer_workspace_bytes, 256-byte
 * aligned. */
sdxl_status sdxl_attn_sublayer(const sdxl_sublayer_desc* desc, const void* x, const void* ln_gamma,
                               const void* ln_beta, const void* w_qkv, const float* w_qkv_scale,
                               const void* w_out, const void* b_out, void* y, void* workspace,
                               size_t workspace_bytes, void* stream);

/* Allocation-free form of sdxl_attn_sublayer. No counterpart in the reference:
 * for callers that cannot allocate device memory or take a workspace (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * workspace is a fixed device-resident array of
 * sdxl_attn_sublayer_noalloc_max_workspace_bytes() (80 MiB) per GPU, held until the
 * process ends; calls whose sdxl_attn_sublayer_workspace_bytes exceed it fail with
 * SDXL_STATUS_INVALID_SHAPE (e.g. [2, 4096, 640] needs 40 MiB, [4, 3840, 640]
 * 75 MiB). Every call on one GPU shares that array: calls that overlap on one GPU
 * (concurrent streams, or threads without ordering) race. Allocates nothing, no
 * host synchronisation; the first call on a device looks up the array's address.
 * The array is part of the library's code object: a process that loads the library
 * reserves its 80 MiB on every GPU it runs one of the library's kernels on, whether
 * or not it calls this entry point. Arguments and results as sdxl_attn_sublayer. */
size_t sdxl_attn_sublayer_noalloc_max_workspace_bytes(void);
sdxl_status sdxl_attn_sublayer_noalloc(const sdxl_sublayer_desc* desc, const void* x, const void* ln_gamma,
                                       const void* ln_beta, const void* w_qkv, const float* w_qkv_scale,
                                       const void* w_out, const void* b_out, void* y, void* stream);

typedef struct sdxl_cross_sublayer_desc {
    int64_t batch;
    int64_t seq;
    int64_t heads;       /* width = heads * 64 */
    int64_t ctx_len;     /* context tokens (77 for SDXL's CLIP context) */
    int32_t w_q_dtype;   /* SDXL_DTYPE_F16 or SDXL_DTYPE_E4M3 */
    int32_t attn_backend; /* sdxl_attn_backend for the attention step */
    float ln_eps;        /* 0 means 1e-5 */
    int32_t q_activations; /* SDXL_DTYPE_F16 or SDXL_DTYPE_E4M3 (fp8 MFMA; E4M3 w_q) */
} sdxl_cross_sublayer_desc;

/* Workspace the cross-attention sublayer needs: batch * seq * width * 4 bytes
 * (normalised hidden / attention output, then the query projection). */
size_t sdxl_cross_attn_sublayer_workspace_bytes(const sdxl_cross_sublayer_desc* desc);

/* The cross-attention half of the reference's transformer block
 * (src/cuda/unet.cpp:120-131): y = x + to_out(attention(LN(x) . w_q^T, K, V)) for
 * hidden x [B, S, W] fp16. kv [B, ctx_len, 2W] fp16 holds K | V of the context,
 * projected once per request (the context is constant over the sampler steps):
 * sdxl_linear of encoder_hidden_states [B * ctx_len, C] against the row-concatenated
 * [to_k; to_v] weight [2W, C]. kv_row_stride in elements (0 = 2W). w_q [W, W] fp16 or
 * E4M3 (+ w_q_scale [W]); w_out [W, W] fp16, b_out [W]; the residual is added in
 * the output projection's epilogue. y may equal x. workspace:
 * sdxl_cross_attn_sublayer_workspace_bytes, 256-byte aligned. */
sdxl_status sdxl_cross_attn_sublayer(const sdxl_cross_sublayer_desc* desc, const void* x, const void* ln_gamma,
                                     const void* ln_beta, const void* w_q, const float* w_q_scale,
                                     const void* kv, int64_t kv_row_stride, const void* w_out,
                                     const void* b_out, void* y, void* workspace, size_t workspace_bytes,
                                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SDXL_HIP_SUBLAYER_H */

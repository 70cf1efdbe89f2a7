// Internal launch interface of the sublayer kernels (sublayer.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attention_kernels.hpp"  // kStreamOutBytes

namespace sdxl_hip {

// c[m, n] = w_scale[n] * sum_k a[m, k] * w[n, k] + bias[n] + residual[m, n]
// a, c, bias, residual fp16; w fp16 or E4M3 codes; strides in elements.
// Requires k % 64 == 0, n % 4 == 0, 16-byte aligned a/w rows, 8-byte
// aligned c/bias/residual rows, 16-byte aligned w_scale.
struct LinearParams {
    const void* a;
    const void* w;
    const float* w_scale;   // nullable: 1
    const void* bias;       // nullable
    const void* residual;   // nullable
    const float* a_scale;   // nullable; set: a holds E4M3 codes with per-row scales (w must be E4M3)
    void* c;
    int64_t lda, ldw, ldr, ldc;
    int32_t m, n, k;
    int32_t m_blocks, n_blocks;  // filled by the launcher
    int32_t group_m;             // filled by the launcher: m blocks per task group
    // Query projection fused with the 77-token cross-attention
    // (launch_q_cross_attention only): kv [batch, ctx_len, ldkv] holds K in
    // columns 0 .. n-1 and V in n .. 2n-1; c receives the attention output.
    const void* kv;
    int64_t ldkv;
    int32_t ctx_len, seq;
    float scale_log2;
};
// compute_units: CUs of the device (tile-size choice).
hipError_t launch_linear(const LinearParams& params, bool w_fp8, int compute_units, hipStream_t stream);
// K-split form for fp16 weights (64 x 160 tiles, the four waves of a tile each
// over a quarter of every K stage): used by launch_linear when it applies.
// Requires a residual (output projections), n % 8 == 0, 16-byte aligned rows
// and pointers (a, w, c, residual, bias, w_scale) and one round of tiles on
// compute_units CUs.
bool linear_ksplit_supported(const LinearParams& params, bool w_fp8, int compute_units);
hipError_t launch_linear_ksplit(const LinearParams& params, hipStream_t stream);
// q = a w^T (64 x 128 tiles, one 32-row block of one head per wave), then
// softmax(q k^T * scale) v per head, written to c. Requires seq % 64 == 0,
// n % 128 == 0 (heads of 64), 65 <= ctx_len <= 80, k % 64 == 0, no bias or
// residual, and a grid that is resident at once on compute_units CUs.
bool q_cross_attention_supported(const LinearParams& params, bool w_fp8, int compute_units);
hipError_t launch_q_cross_attention(const LinearParams& params, bool w_fp8, int compute_units, hipStream_t stream);

struct LayerNormParams {
    const void* x;
    const void* gamma;
    const void* beta;
    void* y;
    float* y_scale;  // nullable; set: y receives E4M3 codes (row stride ldy bytes) and per-row scales
    int64_t rows;
    int64_t ldx, ldy;
    int32_t width;  // even, <= 2048
    float eps;
};
hipError_t launch_layer_norm(const LayerNormParams& params, hipStream_t stream);

// LayerNorm fused with a projection on E4M3 weights (k = 640):
// c[m, n] = w_scale[n] * sum_k LN(x)[m, k] * w[n, k] + bias[n], LN(x) rounded to
// fp16 exactly as launch_layer_norm rounds it. Requires n % 128 == 0, 16-byte
// aligned x rows, gamma, beta and w rows (ldw % 16 == 0), 8-byte aligned c
// rows; strides in elements (w: bytes).
struct LnLinearParams {
    const void* x;
    const void* gamma;
    const void* beta;
    const uint8_t* w;
    const float* w_scale;
    const void* bias;  // nullable
    void* c;
    int64_t ldx, ldw, ldc;
    int32_t m, n, k;
    float eps;
    int32_t a_fp8;  // nonzero: the LayerNorm rounds its rows to E4M3 codes with per-row scales (as
                    // launch_layer_norm's E4M3 output) and the projection runs on the fp8 matrix cores
    int32_t m_blocks, n_split, chunks;  // filled by the launcher
};
bool ln_linear_supported(const LnLinearParams& params);
// Whether the fused kernel is the faster choice over LayerNorm + projection as two
// launches: it is when at most two workgroups share a 64-row block (each of them
// normalises the block's rows again): 8192 rows of width 640 on 256 CUs, not 2048
// rows of width 1280 (measured 27.1 / 42.1 us against 4.1 + 15.9 / 3.8 + 23.6 us).
bool ln_linear_preferred(const LnLinearParams& params, int compute_units);
hipError_t launch_ln_linear(const LnLinearParams& params, int compute_units, hipStream_t stream);

struct QuantizeParams {
    const void* w;   // fp16 [rows, cols]
    uint8_t* q;      // E4M3 [rows, cols]
    float* scales;   // [rows]
    int64_t rows, cols;
};
hipError_t launch_quantize_e4m3_rows(const QuantizeParams& params, hipStream_t stream);

}  // namespace sdxl_hip

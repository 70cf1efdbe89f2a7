// Internal launch interface between the C ABI (capi.cpp) and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sdxl_hip {

// Waves per workgroup of the fused kernel (32 query rows per wave).
constexpr int kFusedWaves = 4;
// Outputs of at least this many bytes are written with non-temporal stores:
// they stream to memory instead of occupying L2 (measured faster for the
// 10-40 MB outputs of the level-1 shapes; smaller outputs, read back by the
// next kernel of a sublayer, were faster with ordinary stores).
constexpr int64_t kStreamOutBytes = int64_t{8} << 20;
// Key sequences up to this length run the one-pass short-key kernel (K/V wholly in LDS).
constexpr int kShortKeysMax = 128;

struct FusedAttentionParams {
    const void* q;
    const void* k;
    const void* v;
    const int32_t* key_mask;  // nullable [batch, k_seq]
    void* o;
    int64_t q_row_stride;  // elements
    int64_t k_row_stride;
    int64_t v_row_stride;
    int64_t o_row_stride;
    int32_t batch;
    int32_t q_seq;
    int32_t k_seq;
    int32_t heads;
    int32_t causal;
    int32_t q_blocks;      // filled by the launcher
    int32_t total_blocks;  // filled by the launcher
    float scale_log2;      // softmax scale * log2(e)
    float inv_scale_log2;  // 1 / scale_log2 (finite)
    int32_t whole_units;   // filled by the launcher: 128-row workgroups (ids first)
    int32_t split_units;   // filled by the launcher: 64-row key-split workgroups
    int32_t short_chunk_blocks;  // filled by the short-key launchers: query blocks (32 or 16 rows) per workgroup
    int32_t short_chunks;        // filled by the short-key launcher: workgroups per (batch, head)
    int32_t mixed_total;         // filled by the launcher: 32-row blocks of the call (mixed kind)
    int32_t mixed_wgs;           // filled by the launcher: mixed workgroups
};

// head_dim 64, fp16 or bf16 storage, 16-byte aligned rows.
// compute_units: CUs of the device (0 if unknown; disables key-split workgroups).
hipError_t launch_fused_attention_d64(const FusedAttentionParams& params, bool is_bf16, int compute_units,
                                      hipStream_t stream);
int fused_attention_block_queries();
// Whether a short-key call (k_seq <= kShortKeysMax) with blocks32 32-row query
// blocks in all runs on 16-row blocks (at most 1.5 32-row blocks per CU).
bool short_keys_16_row_blocks(int64_t blocks32, int compute_units);

struct OnlineAttentionParams {
    const void* q;
    const void* k;
    const void* v;
    const int32_t* key_mask;
    void* o;
    int64_t q_row_stride;
    int64_t k_row_stride;
    int64_t v_row_stride;
    int64_t o_row_stride;
    int32_t batch;
    int32_t q_seq;
    int32_t k_seq;
    int32_t heads;
    int32_t head_dim;  // 1 .. 1024
    int32_t causal;
    float scale;
};

// dtype: 0 f16, 1 bf16, 2 f32 (sdxl_dtype values).
hipError_t launch_online_attention(const OnlineAttentionParams& params, int dtype, hipStream_t stream);

// FP32 head_dim 512 on the fp32 matrix cores (the VAE mid-block attention):
// non-causal, unmasked, 16-byte aligned rows. Same parameters as the online kernel.
bool attention_f32_d512_eligible(const OnlineAttentionParams& params, int dtype);
hipError_t launch_attention_f32_d512(const OnlineAttentionParams& params, int compute_units, hipStream_t stream);

}  // namespace sdxl_hip

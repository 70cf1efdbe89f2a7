// Wave64 online-softmax attention: the correctness fallback backend.
//
// Replaces the reference's warp-online kernel (src/cuda/ops_kernels.cu:491-556)
// and its generic FP16/FP32 kernels (:560-630, :1355-1419), which together
// serve every head_dim and the FP32 VAE head (D = 512). Same semantics:
// online softmax over keys with expf, optional int32 key mask, causal
// visibility key <= query, output acc * (1 / max(l, 1e-20)), so a row with no
// visible key is zero.
//
// MI355X mapping: one wave64 per (b, h, query) row, four rows per workgroup.
// Keys go in chunks of 64, one key per lane: each lane forms its full dot
// product q.k (q staged in LDS, pre-scaled), the chunk max and sum are wave
// reductions, and the output accumulation switches to one channel per lane
// (channels lane, lane+64, ... up to 1024), broadcasting each key's
// probability with v_readlane. No shared memory barriers: every wave works
// alone.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attention_kernels.hpp"

namespace sdxl_hip {
namespace {

constexpr int kMaxHeadDim = 1024;
constexpr int kMaxChannelsPerLane = kMaxHeadDim / 64;
constexpr int kRowsPerBlock = 4;

template <typename T>
__device__ __forceinline__ float load_f(const T* p) {
    return (float)(*p);
}

template <typename T>
__device__ __forceinline__ void store_f(T* p, float v) {
    *p = (T)v;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
    return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}

template <typename T>
__global__ __launch_bounds__(64 * kRowsPerBlock) void online_attention_kernel(OnlineAttentionParams p) {
    __shared__ float q_lds[kRowsPerBlock][kMaxHeadDim];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t rows = (int64_t)p.batch * p.heads * p.q_seq;
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + wave;
    if (row >= rows) return;  // whole wave exits; no block-level barrier below
    const int query = (int)(row % p.q_seq);
    const int h = (int)((row / p.q_seq) % p.heads);
    const int b = (int)(row / ((int64_t)p.q_seq * p.heads));
    const int D = p.head_dim;

    const T* qrow = (const T*)p.q + ((int64_t)b * p.q_seq + query) * p.q_row_stride + (int64_t)h * D;
    const T* kb = (const T*)p.k + (int64_t)b * p.k_seq * p.k_row_stride + (int64_t)h * D;
    const T* vb = (const T*)p.v + (int64_t)b * p.k_seq * p.v_row_stride + (int64_t)h * D;
    T* orow = (T*)p.o + ((int64_t)b * p.q_seq + query) * p.o_row_stride + (int64_t)h * D;

    float* qs = q_lds[wave];
    for (int d = lane; d < D; d += 64) qs[d] = load_f(qrow + d);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const int n_ch = (D + 63) >> 6;
    float acc[kMaxChannelsPerLane];
#pragma unroll
    for (int t = 0; t < kMaxChannelsPerLane; ++t) acc[t] = 0.0f;
    float m = -__builtin_inff();
    float l = 0.0f;

    int n_keys = p.k_seq;
    if (p.causal) n_keys = n_keys < query + 1 ? n_keys : query + 1;

    for (int k0 = 0; k0 < n_keys; k0 += 64) {
        const int key = k0 + lane;
        bool visible = key < n_keys;
        if (visible && p.key_mask != nullptr) visible = p.key_mask[(int64_t)b * p.k_seq + key] != 0;
        float s = -__builtin_inff();
        if (visible) {
            const T* krow = kb + (int64_t)key * p.k_row_stride;
            float dot = 0.0f;
            for (int d = 0; d < D; ++d) dot += qs[d] * load_f(krow + d);
            s = dot * p.scale;
        }
        const float m_new = fmaxf(m, wave_max(s));
        if (m_new == -__builtin_inff()) continue;  // nothing visible yet
        const float alpha = m == -__builtin_inff() ? 0.0f : expf(m - m_new);
        const float pr = visible ? expf(s - m_new) : 0.0f;
        l = l * alpha + wave_sum(pr);
        m = m_new;
        const int chunk = n_keys - k0 < 64 ? n_keys - k0 : 64;
#pragma unroll
        for (int t = 0; t < kMaxChannelsPerLane; ++t) {
            if (t < n_ch) acc[t] *= alpha;
        }
        for (int j = 0; j < chunk; ++j) {
            const float pj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pr), j));
            const T* vrow = vb + (int64_t)(k0 + j) * p.v_row_stride;
#pragma unroll
            for (int t = 0; t < kMaxChannelsPerLane; ++t) {
                const int d = lane + 64 * t;
                if (t < n_ch && d < D) acc[t] += pj * load_f(vrow + d);
            }
        }
    }
    const float inv = 1.0f / fmaxf(l, 1.0e-20f);
#pragma unroll
    for (int t = 0; t < kMaxChannelsPerLane; ++t) {
        const int d = lane + 64 * t;
        if (t < n_ch && d < D) store_f(orow + d, acc[t] * inv);
    }
}

}  // namespace

hipError_t launch_online_attention(const OnlineAttentionParams& p, int dtype, hipStream_t stream) {
    const int64_t rows = (int64_t)p.batch * p.heads * p.q_seq;
    if (rows == 0) return hipSuccess;
    const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    if (blocks > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    const dim3 grid((unsigned)blocks), block(64 * kRowsPerBlock);
    switch (dtype) {
    case 0: hipLaunchKernelGGL(online_attention_kernel<_Float16>, grid, block, 0, stream, p); break;
    case 1: hipLaunchKernelGGL(online_attention_kernel<__bf16>, grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL(online_attention_kernel<float>, grid, block, 0, stream, p); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace sdxl_hip

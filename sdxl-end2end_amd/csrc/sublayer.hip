// Kernels of the transformer attention sublayer around the fused attention:
// LayerNorm, linear projections (fp16 or FP8 E4M3 weights) and the per-row
// E4M3 weight quantizer, for gfx950 (MI355X, CDNA4).
//
// Replaces, on the UNet attention sublayer (src/cuda/unet.cpp:106-118):
//   Ops::layer_norm            src/cuda/ops_kernels.cu:185-257, :1428-1460
//   Ops::linear (fp16)         src/cuda/ops_blas.cpp (cuBLASLt, fp16 accumulate)
//   Ops::linear (FP8 weights)  src/cuda/fp8_kernels.cu:52-245 (weight-only
//                              E4M3 with per-output-channel scales)
//   FP8 weight packing         src/cuda/weights.cu:119-170
//
// Linear y[m, n] = s[n] * sum_k a[m, k] w[n, k] (+ bias[n]) (+ r[m, n]):
//   one workgroup = 4 wave64s = a 128 x 128 output tile; K in stages of 64.
//   A (activations, fp16, K-contiguous rows) and fp16 W stream HBM -> LDS
//   with global_load_lds_dwordx4 (no VGPR staging); E4M3 W goes through
//   registers and is decoded to fp16 on the way into LDS (v_cvt_scalef32_pk_
//   f16_fp8, scale 1: every E4M3 value is exact in fp16), so the per-row
//   scale s[n] is applied once, in fp32, in the epilogue. Each wave computes a
//   64 x 64 block as 2 x 2 v_mfma_f32_32x32x16_f16 tiles in transposed form
//   (W rows as the A operand), so that every lane ends up holding 4
//   consecutive output columns of one row: the epilogue reads bias/residual
//   and writes y with 8-byte accesses. fp32 accumulation, one rounding to fp16.
//   LDS rows are 128 B with the chunk swizzle of the attention kernel
//   (conflict-free 16-byte operand reads).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sublayer_kernels.hpp"

namespace sdxl_hip {
namespace {

typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x8 lds_i16x8;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) char lds_char;

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kRowBytes = kBK * 2;              // 128: one fp16 tile row
constexpr int kTileBytes = 128 * kRowBytes;     // 16 KiB

__device__ __forceinline__ int rev3(int x) { return ((x & 1) << 2) | (x & 2) | ((x >> 2) & 1); }
__device__ __forceinline__ int swz(int row) { return rev3((row >> 1) & 7); }

__device__ __forceinline__ f32x16 mfma32(i16x8 a, i16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_char*)p; }

// 1-KiB HBM -> LDS transfer (lane l: 16 bytes from base + voff to lds + 16 l);
// see the attention kernel for the ordering argument (explicit waits and
// barriers, no memory clobber).
__device__ __forceinline__ void lds_dma16(const char* base, uint32_t voff, uint32_t lds) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint64_t ub = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    base = (const char*)(uintptr_t)ub;
    lds = __builtin_amdgcn_readfirstlane(lds);
    asm volatile(
        "s_mov_b32 m0, %2\n\t"
        "s_nop 4\n\t"
        "global_load_lds_dwordx4 %0, %1"
        :
        : "v"(voff), "s"(base), "s"(lds));
}

__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0070); }  // vmcnt(0)

// Four E4M3 codes -> four fp16 values (exact).
__device__ __forceinline__ uint2 e4m3x4_to_f16(uint32_t x) {
    const f16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, false);
    const f16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, true);
    return uint2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}

template <bool kWFp8>
__global__ __launch_bounds__(256, 2) void linear_kernel(LinearParams p) {
    __shared__ __attribute__((aligned(16))) char abuf[2][kTileBytes];
    __shared__ __attribute__((aligned(16))) char wbuf[2][kTileBytes];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hf = lane >> 5, col = lane & 31;

    // Tasks in row-major (m block, n block) order, each XCD taking one
    // contiguous range: the workgroups sharing an A block run together and
    // read it from their XCD's L2.
    int task;
    {
        const int n = p.m_blocks * p.n_blocks;
        const int id = blockIdx.x;
        const int xcd = id & 7, slot = id >> 3;
        const int per = n >> 3, extra = n & 7;
        task = xcd * per + (xcd < extra ? xcd : extra) + slot;
    }
    const int mb = task / p.n_blocks, nb = task % p.n_blocks;
    const int m0 = mb * kBM, n0 = nb * kBN;
    const int n_stages = p.k / kBK;

    const char* abase = (const char*)p.a;
    const char* wbase = (const char*)p.w;
    const int64_t lda_b = p.lda * 2;
    const int64_t ldw_b = kWFp8 ? p.ldw : p.ldw * 2;

    // ---- stage loads. A (and fp16 W): 16 1-KiB transfers per operand and
    // stage, 4 per wave; transfer n covers tile rows 8n .. 8n+7, lane l the
    // row 8n + l/8 and global chunk (l%8) ^ swz(row), landing in its slot.
    auto issue_dma = [&](const char* gbase, int64_t ld_b, int row0, int rows, int k0, char* buf)
                         __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = wave * 4 + j;
            const int row = 8 * n + (lane >> 3);
            const int lrow = min(row, rows - 1 - row0);  // rows past the end re-read the last row
            const char* tile_base = gbase + (int64_t)row0 * ld_b + (int64_t)k0 * 2;
            const uint32_t off = (uint32_t)(lrow * ld_b) + (uint32_t)(((lane & 7) ^ swz(row)) << 4);
            lds_dma16(tile_base, off, lds_addr(buf + 8 * n * kRowBytes));
        }
    };
    // E4M3 W: thread t loads 32 codes (row t/2, k half t%2) into registers ...
    const int wq_row = threadIdx.x >> 1, wq_half = threadIdx.x & 1;
    const char* wq_src = wbase + (int64_t)min(n0 + wq_row, p.n - 1) * ldw_b + wq_half * 32;
    u32x4 wq[2];
    auto load_wq = [&](int k0) __attribute__((always_inline)) {
        const u32x4* src = (const u32x4*)(wq_src + k0);
        wq[0] = src[0];
        wq[1] = src[1];
    };
    // ... and stores them decoded as four 16-byte chunks of its tile row.
    auto store_wq = [&](char* buf) __attribute__((always_inline)) {
        char* row = buf + wq_row * kRowBytes;
        const int s = swz(wq_row);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint2 lo = e4m3x4_to_f16(wq[c >> 1][2 * (c & 1)]);
            const uint2 hi = e4m3x4_to_f16(wq[c >> 1][2 * (c & 1) + 1]);
            *(lds_u32x4*)(row + (((4 * wq_half + c) ^ s) << 4)) = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
    };
    auto issue_stage = [&](int s) __attribute__((always_inline)) {
        issue_dma(abase, lda_b, m0, p.m, s * kBK, abuf[s & 1]);
        if constexpr (kWFp8) load_wq(s * kBK);
        else issue_dma(wbase, ldw_b, n0, p.n, s * kBK, wbuf[s & 1]);
    };

    // ---- wave block: 64 (M) x 64 (N) at (wm, wn); acc[j][i] = C^T tile of
    // n-tile j and m-tile i.
    const int wm = wave & 1, wn = wave >> 1;
    f32x16 acc[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;
    int a_off[2], w_off[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int ar = wm * 64 + 32 * t + col, wr = wn * 64 + 32 * t + col;
        a_off[t] = ar * kRowBytes;
        w_off[t] = wr * kRowBytes;
    }
    const int a_swz[2] = {swz(wm * 64 + col), swz(wm * 64 + 32 + col)};
    const int w_swz[2] = {swz(wn * 64 + col), swz(wn * 64 + 32 + col)};

    issue_stage(0);
    if constexpr (kWFp8) {
        store_wq(wbuf[0]);
    }
    wait_vmem_all();
    __syncthreads();
    for (int s = 0; s < n_stages; ++s) {
        const bool more = s + 1 < n_stages;
        if (more) issue_stage(s + 1);
        const char* ab = abuf[s & 1];
        const char* wb = wbuf[s & 1];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            i16x8 aop[2], wop[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                aop[t] = *(const lds_i16x8*)(ab + a_off[t] + (((2 * ks + hf) ^ a_swz[t]) << 4));
                wop[t] = *(const lds_i16x8*)(wb + w_off[t] + (((2 * ks + hf) ^ w_swz[t]) << 4));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 2; ++i) acc[j][i] = mfma32(wop[j], aop[i], acc[j][i]);
        }
        if constexpr (kWFp8) {
            if (more) store_wq(wbuf[(s + 1) & 1]);
        }
        wait_vmem_all();
        __syncthreads();
    }

    // ---- epilogue. acc[j][i][4u + q]: output row m = m0 + wm*64 + 32i + col,
    // column n = n0 + wn*64 + 32j + 8u + 4hf + q.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int m = m0 + wm * 64 + 32 * i + col;
        if (m >= p.m) continue;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int n = n0 + wn * 64 + 32 * j + 8 * u + 4 * hf;
                if (n >= p.n) continue;
                float v[4] = {acc[j][i][4 * u], acc[j][i][4 * u + 1], acc[j][i][4 * u + 2], acc[j][i][4 * u + 3]};
                if (p.w_scale != nullptr) {
                    const float4 sc = *(const float4*)(p.w_scale + n);
                    v[0] *= sc.x, v[1] *= sc.y, v[2] *= sc.z, v[3] *= sc.w;
                }
                if (p.bias != nullptr) {
                    const f16x4 bb = *(const f16x4*)((const _Float16*)p.bias + n);
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[q] += (float)bb[q];
                }
                if (p.residual != nullptr) {
                    const f16x4 rr = *(const f16x4*)((const _Float16*)p.residual + (int64_t)m * p.ldr + n);
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[q] += (float)rr[q];
                }
                const f16x4 out = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
                *(f16x4*)((_Float16*)p.c + (int64_t)m * p.ldc + n) = out;
            }
    }
}

// LayerNorm over rows of `width` (even, at most 2048): one wave per row, the
// row held in registers (up to 32 values per lane, as fp16 pairs); two-pass
// centred variance as the reference (ops_kernels.cu:225-257), fp32 maths, one
// rounding to fp16. Sums are wave-tree reductions (order differs from the
// reference's block reduction by rounding only).
constexpr int kLnMaxPer = 16;  // half2 pairs per lane: width <= 2048

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

__global__ __launch_bounds__(256) void layer_norm_kernel(LayerNormParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // wave-uniform; no barrier in this kernel
    const int pairs = p.width / 2;
    const f16x2* x = (const f16x2*)((const _Float16*)p.x + row * p.ldx);
    const f16x2* g = (const f16x2*)p.gamma;
    const f16x2* bt = (const f16x2*)p.beta;
    float v[2 * kLnMaxPer];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kLnMaxPer; ++j) {
        if (lane + 64 * j < pairs) {
            const f16x2 h = x[lane + 64 * j];
            v[2 * j] = (float)h[0];
            v[2 * j + 1] = (float)h[1];
            sum += v[2 * j] + v[2 * j + 1];
        }
    }
    const float inv_w = 1.0f / (float)p.width;
    const float mean = wave_sum(sum) * inv_w;
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < kLnMaxPer; ++j) {
        if (lane + 64 * j < pairs) {
            const float d0 = v[2 * j] - mean, d1 = v[2 * j + 1] - mean;
            sq += d0 * d0 + d1 * d1;
        }
    }
    const float var = fmaxf(wave_sum(sq) * inv_w, 0.0f);
    const float inv = 1.0f / sqrtf(var + p.eps);
    f16x2* y = (f16x2*)((_Float16*)p.y + row * p.ldy);
#pragma unroll
    for (int j = 0; j < kLnMaxPer; ++j) {
        if (lane + 64 * j < pairs) {
            const int c = lane + 64 * j;
            const f16x2 gg = g[c], bb = bt[c];
            const float y0 = (v[2 * j] - mean) * inv * (float)gg[0] + (float)bb[0];
            const float y1 = (v[2 * j + 1] - mean) * inv * (float)gg[1] + (float)bb[1];
            y[c] = f16x2{(_Float16)y0, (_Float16)y1};
        }
    }
}

// Per-row E4M3 quantization of an fp16 weight [rows, cols] (reference
// src/cuda/weights.cu:119-170): amax over the finite values of the row, scale
// = amax > 0 ? max(amax / 448, 1e-12) : 1, code = E4M3(w / scale) rounded to
// nearest even, saturated to +-448. One wave per row.
__global__ __launch_bounds__(256) void quantize_e4m3_rows_kernel(QuantizeParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;
    const _Float16* w = (const _Float16*)p.w + row * p.cols;
    float amax = 0.0f;
    for (int64_t c = lane; c < p.cols; c += 64) {
        const float a = fabsf((float)w[c]);
        if (__builtin_isfinite(a)) amax = fmaxf(amax, a);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    const float scale = amax > 0.0f ? fmaxf(amax / 448.0f, 1.0e-12f) : 1.0f;
    if (lane == 0) p.scales[row] = scale;
    uint8_t* q = p.q + row * p.cols;
    for (int64_t c = lane; c < p.cols; c += 64) {
        float x = (float)w[c] / scale;
        x = x != x ? x : fminf(fmaxf(x, -448.0f), 448.0f);
        const uint32_t packed = __builtin_amdgcn_cvt_pk_fp8_f32(x, 0.0f, 0u, false);
        q[c] = (uint8_t)(packed & 0xFFu);
    }
}

}  // namespace

hipError_t launch_linear(const LinearParams& params_in, bool w_fp8, hipStream_t stream) {
    LinearParams p = params_in;
    p.m_blocks = (p.m + kBM - 1) / kBM;
    p.n_blocks = (p.n + kBN - 1) / kBN;
    const int64_t tasks = (int64_t)p.m_blocks * p.n_blocks;
    if (tasks == 0) return hipSuccess;
    if (tasks > 0x7FFFFFFF || p.k % kBK != 0 || p.n % 4 != 0) return hipErrorInvalidValue;
    const dim3 grid((unsigned)tasks), block(256);
    if (w_fp8) hipLaunchKernelGGL(linear_kernel<true>, grid, block, 0, stream, p);
    else hipLaunchKernelGGL(linear_kernel<false>, grid, block, 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_layer_norm(const LayerNormParams& p, hipStream_t stream) {
    if (p.rows == 0) return hipSuccess;
    if (p.width % 2 != 0 || p.width > 128 * kLnMaxPer) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((p.rows + 3) / 4)), block(256);
    hipLaunchKernelGGL(layer_norm_kernel, grid, block, 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_quantize_e4m3_rows(const QuantizeParams& p, hipStream_t stream) {
    if (p.rows == 0) return hipSuccess;
    const dim3 grid((unsigned)((p.rows + 3) / 4)), block(256);
    hipLaunchKernelGGL(quantize_e4m3_rows_kernel, grid, block, 0, stream, p);
    return hipGetLastError();
}

}  // namespace sdxl_hip

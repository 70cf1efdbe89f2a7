// FP32 attention at head dimension 512 on the fp32 matrix cores.
//
// The SDXL VAE decoder's mid-block attention is single-head with the head
// width equal to the 512 channels, in FP32 (reference src/cuda/vae.cpp:65-99,
// dispatched to generic_online_attention_f32_kernel,
// src/cuda/ops_kernels.cu:1355-1419: one block per query, keys one by one).
// At a 128x128 latent that is 16384 tokens: 550 GFLOP per call, which the
// per-row online kernels run at ~3 TFLOP/s. This kernel is a tiled online
// softmax on v_mfma_f32_32x32x2_f32 with the same semantics (exact fp32
// products, fp32 accumulation, softmax with a running maximum, output divided
// by max(sum, 1e-20)); non-causal, unmasked calls with 16-byte aligned rows.
//
// Work split: a workgroup = 8 waves = 64 queries of one (batch, head): wave
// w = 4 qt + dq owns query tile qt (32 rows) and head-dimension quarter dq
// (128 dims) of the output, O^T[d][q] in 4 MFMA tiles (64 VGPRs). Per block
// of 32 keys:
//   * the 32 x 512 fp32 K tile (64 KiB) moves HBM -> LDS by DMA, double
//     buffered (128 KiB), chunks XOR-swizzled by row so that the 32 rows'
//     16-byte reads at one column hit distinct banks;
//   * each wave forms the partial scores S^T = K[:, dq] Q[:, dq]^T over its
//     128 dims (64 MFMAs), the four partials of a query tile are summed in a
//     fixed order through LDS (16 KiB per tile, 32 KiB), so every wave of the
//     tile holds the same full scores;
//   * online softmax per query (the C layout gives each lane one query with
//     16 of the 32 keys; the other 16 sit in lane l ^ 32);
//   * O^T[d][q] += V^T P^T for the wave's 128 dims (64 MFMAs): V rows come
//     straight from global memory (lane l reads 4 consecutive dims of one key
//     row: the 4 accumulator tiles hold dims 128 dq + 4 m + t, t = 0..3), and
//     P^T from the score registers, MFMA j pairing the keys held in register
//     j by the two lane halves (the reduction order over keys is free).
// The reduction order over the head dimension in S is likewise permuted
// (MFMA j of group g pairs dims 8g + j and 8g + 4 + j), so every lane loads
// its K and Q operands as 16-byte chunks.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attention_kernels.hpp"

namespace sdxl_hip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
typedef __attribute__((address_space(3))) float lds_float;

constexpr int kDim = 512;
constexpr int kKeys = 32;                        // keys per block
constexpr int kRowBytes = kDim * 4;              // 2 KiB per K row
constexpr int kTileBytes = kKeys * kRowBytes;    // 64 KiB per K tile
constexpr int kPartFloats = 16 * 64;             // one wave's partial scores

__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_char*)p; }

// One 1-KiB HBM -> LDS transfer: lane l copies 16 bytes from base + voff to
// LDS byte lds + 16 l (base and lds wave-uniform, M0 holds the destination).
// Inline assembly keeps the compiler from ordering it against LDS reads or
// waiting on it; the kernel orders it explicitly (vmcnt(0) and a barrier
// before a tile is read, the transfer into a buffer only after the barrier
// that ends the buffer's previous reads).
__device__ __forceinline__ void lds_dma16(const char* base, uint32_t voff, uint32_t lds) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint64_t ub = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    base = (const char*)(uintptr_t)ub;
    lds = __builtin_amdgcn_readfirstlane(lds);
    asm volatile(
        "s_nop 4\n\t"
        "global_load_lds_dwordx4 %0, %1"
        :
        : "v"(voff), "s"(base), "{m0}"(lds));
}

__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0070); }  // vmcnt(0)

__device__ __forceinline__ float xhalf_max(float x) { return fmaxf(x, __shfl_xor(x, 32, 64)); }
__device__ __forceinline__ float xhalf_sum(float x) { return x + __shfl_xor(x, 32, 64); }

// Physical 16-byte chunk of logical chunk c (0..127) in K row r: the low four
// bits are XORed with r & 15, so 16 rows read at one logical chunk land in 16
// distinct 16-byte bank groups.
__device__ __forceinline__ int kchunk(int c, int r) { return c ^ (r & 15); }

template <int N> struct FloatVec;
template <> struct FloatVec<2> { typedef float type __attribute__((ext_vector_type(2))); };
template <> struct FloatVec<4> { typedef float type __attribute__((ext_vector_type(4))); };

// kQTiles = 32-query tiles per workgroup, kSlices = slices of the head
// dimension (512 / kSlices dims per wave): (2, 4) = 8 waves for calls with at
// least as many 64-query blocks as CUs, else (1, 4) = 4 waves (measured at
// 4096 tokens: 0.71 ms; (1, 8), two waves per SIMD on one query tile, 0.85).
template <int kQTiles, int kSlices>
__global__ __launch_bounds__(kQTiles * kSlices * 64, 1) void attention_f32_d512_kernel(OnlineAttentionParams p, int q_blocks) {
    constexpr int kWaves = kQTiles * kSlices;
    constexpr int kPerWave = 64 / kWaves;  // 1-KiB K transfers per wave and tile
    constexpr int kSD = kDim / kSlices;    // dims per wave
    constexpr int kTD = kSD / 32;          // accumulator tiles per wave (dims kSD dq + kTD m + t)
    constexpr int kG = kSD / 8;            // 4-MFMA groups of the partial scores
    typedef typename FloatVec<kTD>::type vtype;
    static_assert(kWaves * kPartFloats * 4 + 2 * kTileBytes <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(16))) char kbuf[2][kTileBytes];
    __shared__ __attribute__((aligned(16))) float part[kWaves][kPartFloats];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int qt = wave / kSlices, dq = wave % kSlices;
    const int hf = lane >> 5, col = lane & 31;

    const int bh = blockIdx.x / q_blocks;
    const int q0 = (blockIdx.x % q_blocks) * (32 * kQTiles) + 32 * qt;
    const int h = bh % p.heads, b = bh / p.heads;
    const float* qbase = (const float*)p.q + ((int64_t)b * p.q_seq * p.q_row_stride + (int64_t)h * kDim);
    const char* kbase = (const char*)((const float*)p.k + ((int64_t)b * p.k_seq * p.k_row_stride + (int64_t)h * kDim));
    const float* vbase = (const float*)p.v + ((int64_t)b * p.k_seq * p.v_row_stride + (int64_t)h * kDim);
    float* obase = (float*)p.o + ((int64_t)b * p.q_seq * p.o_row_stride + (int64_t)h * kDim);
    const int n_blocks = (p.k_seq + kKeys - 1) / kKeys;
    const uint32_t k_stride_b = (uint32_t)(p.k_row_stride * 4);

    // K tile of key block t into buffer buf: 64 transfers of 1 KiB, kPerWave
    // per wave; transfer n fills physical chunks 64 (n & 1) .. +63 of row n >> 1.
    // Rows past k_seq re-read the last key (their scores are masked).
    auto issue_k = [&](int t, int buf) __attribute__((always_inline)) {
        const char* src = kbase + (int64_t)t * kKeys * p.k_row_stride * 4;
        const int last = p.k_seq - 1 - t * kKeys;
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int n = wave * kPerWave + j;
            const int row = n >> 1;
            const int c = kchunk(64 * (n & 1) + lane, row);
            const uint32_t off = (uint32_t)min(row, last) * k_stride_b + (uint32_t)(c << 4);
            lds_dma16(src, off, lds_addr(&kbuf[buf][0] + 1024 * n));
        }
    };
    issue_k(0, 0);

    // Q^T operand: lane holds query q0 + col, dims kSD dq + 8g + 4hf .. +3 in
    // qop[g] (MFMA j of group g takes element j).
    f32x4 qop[kG];
    {
        const float* qrow = qbase + (int64_t)min(q0 + col, p.q_seq - 1) * p.q_row_stride + kSD * dq + 4 * hf;
#pragma unroll
        for (int g = 0; g < kG; ++g) qop[g] = *(const f32x4*)(qrow + 8 * g);
    }

    const float c = p.scale * 1.4426950408889634f;  // scores to log2 units
    f32x16 o[kTD];
#pragma unroll
    for (int t = 0; t < kTD; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[t][i] = 0.0f;
    float m_run = -__builtin_inff();  // running maximum (log2 units) of this lane's query
    float l_run = 0.0f;               // this lane's half of the running sum
    const float* vcol = vbase + kSD * dq + kTD * col;
    // K operand address: lane reads row col, logical chunk (kSD / 4) dq + 2g + hf.
    const int krow_off = col * kRowBytes;

    for (int t = 0; t < n_blocks; ++t) {
        const int buf = t & 1;
        wait_vmem_all();  // this wave's part of K(t) landed
        __syncthreads();  // all of K(t); every wave is done with K(t - 1) and the partial scores
        if (t + 1 < n_blocks) issue_k(t + 1, buf ^ 1);

        // V rows of this block for PV: register j holds key 8(j >> 2) + 4hf +
        // (j & 3), dims kSD dq + kTD col .. +kTD-1. The first half is loaded now (in
        // flight during S), the second after S (in flight during the score
        // reduction, the softmax and the first half of PV).
        vtype vop[16];
        auto load_v = [&](int j0) __attribute__((always_inline)) {
            const int key0 = t * kKeys;
#pragma unroll
            for (int j = j0; j < j0 + 8; ++j) {
                const int key = min(key0 + 8 * (j >> 2) + 4 * hf + (j & 3), p.k_seq - 1);
                vop[j] = *(const vtype*)(vcol + (int64_t)key * p.v_row_stride);
            }
        };
        load_v(0);

        // partial S^T over this wave's kSD dims
        // two accumulator chains (even and odd groups), summed after: at 16384
        // tokens 5.12 -> 5.00 ms against one chain (the same interleave in the
        // 16-query kernel measured slower, 399 -> 416 us at 4096 tokens)
        f32x16 s, s_odd;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = s_odd[i] = 0.0f;
        const char* kt = &kbuf[buf][0] + krow_off;
#pragma unroll
        for (int g = 0; g < kG; g += 2) {
            const f32x4 kop0 = *(const lds_f32x4*)(kt + (kchunk((kSD / 4) * dq + 2 * g + hf, col) << 4));
            const f32x4 kop1 = *(const lds_f32x4*)(kt + (kchunk((kSD / 4) * dq + 2 * (g + 1) + hf, col) << 4));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kop0[j], qop[g][j], s, 0, 0, 0);
                s_odd = __builtin_amdgcn_mfma_f32_32x32x2f32(kop1[j], qop[g + 1][j], s_odd, 0, 0, 0);
            }
        }
        s += s_odd;
        load_v(8);
        float* mine = &part[wave][0];
#pragma unroll
        for (int i = 0; i < 16; ++i) mine[i * 64 + lane] = s[i];
        __syncthreads();
        // full scores: the tile's partials in dq order (the same sum in every wave of the tile)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float acc = part[kSlices * qt][i * 64 + lane];
#pragma unroll
            for (int w = 1; w < kSlices; ++w) acc += part[kSlices * qt + w][i * 64 + lane];
            s[i] = acc;
        }

        // keys past k_seq: element i is key t*32 + 8(i >> 2) + 4hf + (i & 3)
        const int lim = p.k_seq - t * kKeys - 4 * hf;
        if (lim < 32) {
#pragma unroll
            for (int i = 0; i < 16; ++i) s[i] = 8 * (i >> 2) + (i & 3) < lim ? s[i] : -__builtin_inff();
        }
        float mx = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[i]);
        mx = xhalf_max(mx) * c;
        const float m_new = fmaxf(m_run, mx);  // finite: every block holds a visible key
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first block
        m_run = m_new;
        float pr[16];
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], c, -m_new));
            sum += pr[i];
        }
        l_run = l_run * alpha + sum;
#pragma unroll
        for (int tt = 0; tt < kTD; ++tt)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[tt][i] *= alpha;

        // O^T[d][q] += V^T P^T: tile tt holds dims kSD dq + kTD m + tt
#pragma unroll
        for (int j = 0; j < 16; ++j)
#pragma unroll
            for (int tt = 0; tt < kTD; ++tt) o[tt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vop[j][tt], pr[j], o[tt], 0, 0, 0);
    }

    // ---- normalise and store: lane holds rows m = 8(i >> 2) + 4hf + (i & 3)
    // of each tile for query q0 + col, i.e. dims kSD dq + kTD m .. +kTD-1.
    const float inv = 1.0f / fmaxf(xhalf_sum(l_run), 1.0e-20f);
    if (q0 + col < p.q_seq) {
        float* orow = obase + (int64_t)(q0 + col) * p.o_row_stride + kSD * dq;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = 8 * (i >> 2) + 4 * hf + (i & 3);
            vtype w;
#pragma unroll
            for (int tt = 0; tt < kTD; ++tt) w[tt] = o[tt][i] * inv;
            *(vtype*)(orow + kTD * m) = w;
        }
    }
}

// Variant for calls with fewer 32-query tiles than CUs (the VAE at a 64x64
// latent, 4096 tokens: 128 tiles): 16-query workgroups on
// v_mfma_f32_16x16x4_f32, 4 waves = 4 slices of 128 dims, so twice as many
// workgroups fill the CUs. Same algorithm and order of operations as above
// per key block; the 16x16 C layout gives lane l query l & 15 and keys
// 4 (l >> 4) .. +3 of each 16-key half, so the row maximum and sum take two
// lane exchanges (l ^ 16, l ^ 32). Index maps (free reduction orders):
//   S: MFMA j of group g pairs dim 16 g + 4 (l >> 4) + j of the slice (K and
//      Q operands are 16-byte chunks);
//   PV: score register r (key 16 (r >> 2) + 4 (l >> 4) + (r & 3)) is the B
//      operand of MFMA r; accumulator tile tt row m holds dim 8 m + tt of the
//      slice, so lane l loads dims 8 (l & 15) .. +7 of its key row (32 bytes)
//      and stores 8 consecutive dims per register.
__global__ __launch_bounds__(256, 1) void attention_f32_d512_q16_kernel(OnlineAttentionParams p, int q_blocks) {
    constexpr int kWaves = 4;
    constexpr int kPerWave = 64 / kWaves;
    constexpr int kSD = kDim / kWaves;  // 128 dims per wave
    static_assert(kWaves * 8 * 64 * 4 + 2 * kTileBytes <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(16))) char kbuf[2][kTileBytes];
    __shared__ __attribute__((aligned(16))) float part[kWaves][8 * 64];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int dq = wave;
    const int qc = lane & 15, kq = lane >> 4;

    const int bh = blockIdx.x / q_blocks;
    const int q0 = (blockIdx.x % q_blocks) * 16;
    const int h = bh % p.heads, b = bh / p.heads;
    const float* qbase = (const float*)p.q + ((int64_t)b * p.q_seq * p.q_row_stride + (int64_t)h * kDim);
    const char* kbase = (const char*)((const float*)p.k + ((int64_t)b * p.k_seq * p.k_row_stride + (int64_t)h * kDim));
    const float* vbase = (const float*)p.v + ((int64_t)b * p.k_seq * p.v_row_stride + (int64_t)h * kDim);
    float* obase = (float*)p.o + ((int64_t)b * p.q_seq * p.o_row_stride + (int64_t)h * kDim);
    const int n_blocks = (p.k_seq + kKeys - 1) / kKeys;
    const uint32_t k_stride_b = (uint32_t)(p.k_row_stride * 4);

    // K tile of key block t into buffer buf (as in the 32-query kernel).
    auto issue_k = [&](int t, int buf) __attribute__((always_inline)) {
        const char* src = kbase + (int64_t)t * kKeys * p.k_row_stride * 4;
        const int last = p.k_seq - 1 - t * kKeys;
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int n = wave * kPerWave + j;
            const int row = n >> 1;
            const int c = kchunk(64 * (n & 1) + lane, row);
            const uint32_t off = (uint32_t)min(row, last) * k_stride_b + (uint32_t)(c << 4);
            lds_dma16(src, off, lds_addr(&kbuf[buf][0] + 1024 * n));
        }
    };
    issue_k(0, 0);

    // Q operand: query q0 + qc, dims kSD dq + 16 g + 4 kq .. +3 in qop[g].
    f32x4 qop[8];
    {
        const float* qrow = qbase + (int64_t)min(q0 + qc, p.q_seq - 1) * p.q_row_stride + kSD * dq + 4 * kq;
#pragma unroll
        for (int g = 0; g < 8; ++g) qop[g] = *(const f32x4*)(qrow + 16 * g);
    }

    const float c = p.scale * 1.4426950408889634f;  // scores to log2 units
    f32x4 o[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) o[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -__builtin_inff();
    float l_run = 0.0f;  // this lane's quarter of the running sum
    const float* vcol = vbase + kSD * dq + 8 * qc;

    for (int t = 0; t < n_blocks; ++t) {
        const int buf = t & 1;
        wait_vmem_all();
        __syncthreads();
        if (t + 1 < n_blocks) issue_k(t + 1, buf ^ 1);

        // V operands: register r holds key t*32 + 16 (r >> 2) + 4 kq + (r & 3),
        // dims kSD dq + 8 qc .. +7 (two 16-byte halves).
        f32x4 vop[8][2];
        auto load_v = [&](int r0) __attribute__((always_inline)) {
#pragma unroll
            for (int r = r0; r < r0 + 4; ++r) {
                const int key = min(t * kKeys + 16 * (r >> 2) + 4 * kq + (r & 3), p.k_seq - 1);
                const float* src = vcol + (int64_t)key * p.v_row_stride;
                vop[r][0] = *(const f32x4*)src;
                vop[r][1] = *(const f32x4*)(src + 4);
            }
        };
        load_v(0);

        f32x4 s[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            s[kt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            const int row = 16 * kt + qc;
            const char* krow = &kbuf[buf][0] + row * kRowBytes;
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                const f32x4 kop = *(const lds_f32x4*)(krow + (kchunk((kSD / 4) * dq + 4 * g + kq, row) << 4));
#pragma unroll
                for (int j = 0; j < 4; ++j) s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kop[j], qop[g][j], s[kt], 0, 0, 0);
            }
        }
        load_v(4);
        float* mine = &part[wave][0];
#pragma unroll
        for (int i = 0; i < 8; ++i) mine[i * 64 + lane] = s[i >> 2][i & 3];
        __syncthreads();
        // full scores: the partials summed in slice order
        float sc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float acc = part[0][i * 64 + lane];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) acc += part[w][i * 64 + lane];
            sc[i] = acc;
        }

        // keys past k_seq: score i is key t*32 + 16 (i >> 2) + 4 kq + (i & 3)
        const int lim = p.k_seq - t * kKeys - 4 * kq;
        if (lim < 32) {
#pragma unroll
            for (int i = 0; i < 8; ++i) sc[i] = 16 * (i >> 2) + (i & 3) < lim ? sc[i] : -__builtin_inff();
        }
        float mx = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < 8; ++i) mx = fmaxf(mx, sc[i]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * c;
        const float m_new = fmaxf(m_run, mx);  // finite: every block holds a visible key
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        float pr[8];
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            pr[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i], c, -m_new));
            sum += pr[i];
        }
        l_run = l_run * alpha + sum;
#pragma unroll
        for (int tt = 0; tt < 8; ++tt) o[tt] *= alpha;

#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int tt = 0; tt < 8; ++tt)
                o[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vop[r][tt >> 2][tt & 3], pr[r], o[tt], 0, 0, 0);
    }

    // ---- normalise and store: register i of tile tt is dim kSD dq + 8 (4 kq + i) + tt.
    float l = l_run + __shfl_xor(l_run, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const float inv = 1.0f / fmaxf(l, 1.0e-20f);
    if (q0 + qc < p.q_seq) {
        float* orow = obase + (int64_t)(q0 + qc) * p.o_row_stride + kSD * dq + 32 * kq;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x4 lo = {o[0][i] * inv, o[1][i] * inv, o[2][i] * inv, o[3][i] * inv};
            const f32x4 hi = {o[4][i] * inv, o[5][i] * inv, o[6][i] * inv, o[7][i] * inv};
            *(f32x4*)(orow + 8 * i) = lo;
            *(f32x4*)(orow + 8 * i + 4) = hi;
        }
    }
}

}  // namespace

bool attention_f32_d512_eligible(const OnlineAttentionParams& p, int dtype) {
    auto a16 = [](const void* x) { return ((uintptr_t)x & 15) == 0; };
    return dtype == 2 && p.head_dim == kDim && !p.causal && p.key_mask == nullptr && p.k_seq > 0 &&
           p.q_row_stride % 4 == 0 && p.k_row_stride % 4 == 0 && p.v_row_stride % 4 == 0 && p.o_row_stride % 4 == 0 &&
           a16(p.q) && a16(p.k) && a16(p.v) && a16(p.o) &&
           (int64_t)kKeys * p.k_row_stride * 4 < (int64_t{1} << 31);
}

hipError_t launch_attention_f32_d512(const OnlineAttentionParams& p, int compute_units, hipStream_t stream) {
    if (p.batch == 0 || p.q_seq == 0) return hipSuccess;
    // 64-query workgroups (waves: 2 query tiles x 4 dim slices) when they
    // fill the CUs; else 32-query workgroups (1 x 4): twice the workgroups,
    // each K tile staged for half as many queries; and when even those leave
    // CUs idle, 16-query workgroups on the 16x16 matrix-core tiles.
    const int64_t heads_total = (int64_t)p.heads * p.batch;
    const int64_t blocks64 = (p.q_seq + 63) / 64 * heads_total;
    const int cus = compute_units > 0 ? compute_units : 256;
    const bool wide = blocks64 >= cus;
    const bool q16 = !wide && (p.q_seq + 31) / 32 * heads_total < cus;
    const int rows = wide ? 64 : q16 ? 16 : 32;
    const int64_t q_blocks = (p.q_seq + rows - 1) / rows;
    const int64_t grid = q_blocks * heads_total;
    if (grid > INT32_MAX) return hipErrorInvalidValue;
    if (q16) hipLaunchKernelGGL(attention_f32_d512_q16_kernel, dim3((unsigned)grid), dim3(256), 0, stream, p, (int)q_blocks);
    else if (wide) hipLaunchKernelGGL((attention_f32_d512_kernel<2, 4>), dim3((unsigned)grid), dim3(512), 0, stream, p, (int)q_blocks);
    else hipLaunchKernelGGL((attention_f32_d512_kernel<1, 4>), dim3((unsigned)grid), dim3(256), 0, stream, p, (int)q_blocks);
    return hipGetLastError();
}

}  // namespace sdxl_hip

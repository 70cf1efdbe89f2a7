// Fused forward attention for head_dim 64 on gfx950 (MI355X, CDNA4).
//
// Replaces the reference's in-tree tiled kernel
// (src/cuda/flash_attention_sm80.cu:45-221) and its cuDNN SDPA backend
// (src/cuda/cudnn_sdpa.cpp:44-168): o = softmax(q k^T * scale) v per
// (batch, head), online softmax, no score matrix in memory.
//
// Work decomposition
//   One workgroup = kWaves wave64s = kWaves*32 query rows of one (b, h).
//   Every wave owns 32 query rows and walks all keys in tiles of 64.
//   K and V tiles (64 keys x 64 dims, fp16/bf16) are staged in LDS, double
//   buffered, and shared by the workgroup's waves.
//
// Per wave and key tile (MFMA v_mfma_f32_32x32x16_{f16,bf16}):
//   S^T[key][q] = K Q^T     : A = K rows from LDS (16 B per lane),
//                             B = Q^T from registers (loaded once);
//                             C layout puts one query per lane column, so the
//                             row max / row sum are in-lane plus one
//                             lane<->lane+32 exchange (v_permlane32_swap).
//   P = exp2(S*scale*log2e - m)  in fp32, packed to fp16/bf16 (v_cvt_pk_*).
//   O^T[d][q] += V^T P^T    : A = V^T built with ds_read_b64_tr_b16 straight
//                             from the row-major V tile (no transpose pass),
//                             B = P^T from the S^T accumulator registers
//                             (no LDS round trip).
//   Lazy rescaling: the running max used in exp2 only moves when a row's tile
//   max exceeds it by more than 2^8, so O is rescaled almost never after the
//   first tile (P then lies in [0, 256], exact enough in fp16/bf16).
//
// LDS layout per stage: K[64][64] then V[64][64] elements, 128 B rows, the
// eight 16-byte chunks of row r stored at chunk ^ rev3(r & 7). That swizzle
// makes both the 16 B K-operand reads (8 consecutive rows, one chunk) and the
// transposing V reads (4 rows, 2 chunks per 16-lane group) bank-conflict free.
// Tiles move HBM -> LDS with global_load_lds_dwordx4 (no VGPR staging); each
// lane picks the global chunk that lands in its swizzled LDS slot.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attention_kernels.hpp"

namespace sdxl_hip {
namespace {

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) i16x8 lds_i16x8;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kHeadDim = 64;
constexpr int kKeyTile = 64;
constexpr int kRowBytes = kHeadDim * 2;                // 128
constexpr int kTileBytes = kKeyTile * kRowBytes;       // 8 KiB
constexpr int kStageBytes = 2 * kTileBytes;            // K + V
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleThreshold = 8.0f;              // log2 units

__device__ __forceinline__ int rev3(int x) { return ((x & 1) << 2) | (x & 2) | ((x >> 2) & 1); }

template <bool IsBf16>
__device__ __forceinline__ f32x16 mfma32(i16x8 a, i16x8 b, f32x16 c) {
    if constexpr (IsBf16) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
}

// Packs two fp32 values into one dword of fp16/bf16 (round to nearest even).
template <bool IsBf16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (IsBf16) {
        bf16x2 v = {(__bf16)a, (__bf16)b};
        return __builtin_bit_cast(uint32_t, v);
    } else {
        f16x2 v = {(_Float16)a, (_Float16)b};
        return __builtin_bit_cast(uint32_t, v);
    }
}

// Sum of the two packed values, added to acc in fp32.
template <bool IsBf16>
__device__ __forceinline__ float sum2(uint32_t packed, float acc) {
    if constexpr (IsBf16) {
        const uint32_t lo = packed << 16, hi = packed & 0xFFFF0000u;
        return acc + __builtin_bit_cast(float, lo) + __builtin_bit_cast(float, hi);
    } else {
        const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, packed), one, acc, false);
    }
}

// Exchange with lane l ^ 32 (the other half of the wave holds the other keys
// of the same query). ds_bpermute: the permlane32 swap builtin is folded
// incorrectly by this compiler when both operands are the same value.
__device__ __forceinline__ float xhalf_max(float x) { return fmaxf(x, __shfl_xor(x, 32, 64)); }

__device__ __forceinline__ float xhalf_sum(float x) { return x + __shfl_xor(x, 32, 64); }

// Stages one 64-key tile of K and V into LDS. The 16 1-KiB load instructions
// (8 for K, 8 for V) are split evenly over the workgroup's waves; instruction
// n covers rows 8*(n%8) .. 8*(n%8)+7 of K (n < 8) or V (n >= 8). Rows past
// k_seq are clamped to the last key: their scores are masked to -inf, so they
// contribute exactly 0 and the clamp only keeps the loaded values finite.
template <int kWaves>
__device__ __forceinline__ void stage_tile(const char* __restrict__ kbase, const char* __restrict__ vbase,
                                           int64_t k_stride_bytes, int64_t v_stride_bytes, int key0,
                                           int k_seq, char* lds_stage, int wave, int lane) {
    constexpr int kPerWave = 16 / kWaves;
    const int row_in_group = lane >> 3;
    const int chunk_slot = lane & 7;
#pragma unroll
    for (int j = 0; j < kPerWave; ++j) {
        const int n = wave * kPerWave + j;
        const bool is_v = n >= 8;
        const int row = 8 * (n & 7) + row_in_group;
        int key = key0 + row;
        key = key < k_seq ? key : k_seq - 1;
        const int chunk = chunk_slot ^ rev3(row & 7);
        const char* src = (is_v ? vbase + (int64_t)key * v_stride_bytes : kbase + (int64_t)key * k_stride_bytes) +
                          chunk * 16;
        char* dst = lds_stage + (is_v ? kTileBytes : 0) + 8 * (n & 7) * kRowBytes;
        __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)dst, 16, 0, 0);
    }
}

template <int kWaves, bool IsBf16>
__global__ __launch_bounds__(kWaves * 64) void fused_attention_d64_kernel(FusedAttentionParams p) {
    constexpr int kBlockQueries = kWaves * 32;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int hf = lane >> 5;   // which half of the wave
    const int col = lane & 31;  // query column of this lane in the 32x32 tiles

    // XCD-aware task order: the hardware deals workgroup ids round robin over
    // the 8 XCDs, so give each XCD one contiguous range of tasks (consecutive
    // query blocks of the same head share K/V in that XCD's L2).
    int task;
    {
        const int n = p.total_blocks;
        const int id = blockIdx.x;
        const int xcd = id & 7, slot = id >> 3;
        const int per = n >> 3, extra = n & 7;
        task = xcd * per + (xcd < extra ? xcd : extra) + slot;
    }
    const int qblk = task % p.q_blocks;
    const int bh = task / p.q_blocks;
    const int h = bh % p.heads;
    const int b = bh / p.heads;

    const int64_t elem = 2;
    const char* qbase = (const char*)p.q + ((int64_t)b * p.q_seq * p.q_row_stride + (int64_t)h * kHeadDim) * elem;
    const char* kbase = (const char*)p.k + ((int64_t)b * p.k_seq * p.k_row_stride + (int64_t)h * kHeadDim) * elem;
    const char* vbase = (const char*)p.v + ((int64_t)b * p.k_seq * p.v_row_stride + (int64_t)h * kHeadDim) * elem;
    char* obase = (char*)p.o + ((int64_t)b * p.q_seq * p.o_row_stride + (int64_t)h * kHeadDim) * elem;
    const int64_t ks_bytes = p.k_row_stride * elem, vs_bytes = p.v_row_stride * elem;

    const int q0 = qblk * kBlockQueries + wave * 32;
    const int my_query = q0 + col;

    // Q^T operand: lane holds dims 16*ks + 8*hf .. +7 of its query row.
    i16x8 qop[4];
    if (my_query < p.q_seq) {
        const i16x8* qrow = (const i16x8*)(qbase + (int64_t)my_query * p.q_row_stride * elem);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qop[ks] = qrow[2 * ks + hf];
    } else {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qop[ks] = i16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }

    // Key range. Causal: keys beyond the block's last query are never visible.
    int n_keys = p.k_seq;
    if (p.causal) {
        const int last_query = qblk * kBlockQueries + kBlockQueries - 1;
        n_keys = n_keys < last_query + 1 ? n_keys : last_query + 1;
    }
    const int n_tiles = (n_keys + kKeyTile - 1) / kKeyTile;
    // Tiles below full_tiles need no masking unless a key mask is given or, for
    // causal calls, the tile reaches past this wave's first query.
    const int full_tiles = p.key_mask != nullptr ? 0 : p.k_seq / kKeyTile;

    // Per-lane LDS byte offsets.
    // K operand: row 32g + col, chunk (2ks + hf) ^ rev3(col & 7).
    const int k_swz = rev3(col & 7);
    // V^T operand via transposing reads: inside each 16-lane group, lane
    // r = 4j + qd supplies the address of key (4*hf + j) (+8 for the second
    // read), dims 32dt + 16*((lane>>4)&1) + 4qd .. +3.
    const int g16 = lane & 15;
    const int tr_j = g16 >> 2, tr_qd = g16 & 3;
    const int tr_key = 4 * hf + tr_j;
    const int tr_swz = rev3(tr_key);
    int v_off[2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
        const int chunk = 4 * dt + 2 * ((lane >> 4) & 1) + (tr_qd >> 1);
        v_off[dt] = kTileBytes + tr_key * kRowBytes + ((chunk ^ tr_swz) << 4) + ((tr_qd & 1) << 3);
    }

    f32x16 acc[2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] = 0.0f;
    float m_run = -__builtin_inff();
    float l_run = 0.0f;
    const float c = p.scale_log2;

    __shared__ __attribute__((aligned(16))) char stage0[kStageBytes];
    __shared__ __attribute__((aligned(16))) char stage1[kStageBytes];

    auto tile = [&](const char* stage, char* next, int t) {
        __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0): this lane's loads of tile t have landed
        __syncthreads();                     // ... and every other lane's; tile t-1 fully consumed
        // Key-mask word of this lane's key in tile t; issued before the prefetch so
        // that its wait does not also wait for the next tile's loads.
        int mask_word = 1;
        if (p.key_mask != nullptr) {
            const int key = t * kKeyTile + lane;
            mask_word = key < p.k_seq ? p.key_mask[(int64_t)b * p.k_seq + key] : 0;
        }
        if (t + 1 < n_tiles)
            stage_tile<kWaves>(kbase, vbase, ks_bytes, vs_bytes, (t + 1) * kKeyTile, p.k_seq, next, wave, lane);

        // ---- S^T = K Q^T for the two 32-key groups of the tile.
        f32x16 s[2];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
#pragma unroll
            for (int i = 0; i < 16; ++i) s[g][i] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int off = (32 * g + col) * kRowBytes + (((2 * ks + hf) ^ k_swz) << 4);
                const i16x8 kop = *(const lds_i16x8*)(stage + off);
                s[g] = mfma32<IsBf16>(kop, qop[ks], s[g]);
            }
        }

        // ---- masking (ragged tail, key mask, causal), only on tiles that need it.
        // vis bit j = key key0 + j exists and is not masked out (wave-uniform).
        if (t >= full_tiles || (p.causal && t * kKeyTile + kKeyTile - 1 > q0)) {
            const int key0 = t * kKeyTile;
            uint64_t vis = ~0ull;
            if (key0 + kKeyTile > p.k_seq) vis = (1ull << (p.k_seq - key0)) - 1ull;
            if (p.key_mask != nullptr) vis &= __builtin_amdgcn_ballot_w64(mask_word != 0);
            const uint32_t lane_vis = (uint32_t)(vis >> (4 * hf)) ;
            const uint32_t lane_vis_hi = (uint32_t)(vis >> (32 + 4 * hf));
            // causal: key key0 + kk + 4hf visible iff <= my_query
            const int causal_lim = p.causal ? my_query - key0 - 4 * hf : 0x7FFFFFFF;
#pragma unroll
            for (int g = 0; g < 2; ++g)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int kk = (i >> 2) * 8 + (i & 3);  // key offset within group, minus 4hf
                    const uint32_t bits = g ? lane_vis_hi : lane_vis;
                    const bool ok = ((bits >> kk) & 1u) && (32 * g + kk <= causal_lim);
                    s[g][i] = ok ? s[g][i] : -__builtin_inff();
                }
        }

        // ---- online softmax (per lane: one query, 32 of the tile's keys)
        float mx = fmaxf(s[0][0], s[0][1]);
#pragma unroll
        for (int i = 2; i < 16; ++i) mx = fmaxf(mx, s[0][i]);
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[1][i]);
        mx = xhalf_max(mx);
        const float m_tile = mx * c;
        const bool need = m_tile > m_run + kRescaleThreshold;
        if (__builtin_amdgcn_ballot_w64(need)) {
            const float m_new = need ? m_tile : m_run;
            const float alpha = need ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;
            l_run *= alpha;
            m_run = m_new;
        }
        const float neg_m = m_run == -__builtin_inff() ? 0.0f : -m_run;

        uint32_t pk[2][8];
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[g][2 * i], c, neg_m));
                const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[g][2 * i + 1], c, neg_m));
                pk[g][i] = pack2<IsBf16>(p0, p1);
                l_run = sum2<IsBf16>(pk[g][i], l_run);
            }

        // ---- O^T += V^T P^T
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int ss = 0; ss < 2; ++ss) {
                const i16x8 pop = __builtin_bit_cast(
                    i16x8, (uint32_t __attribute__((ext_vector_type(4)))){pk[g][4 * ss], pk[g][4 * ss + 1],
                                                                           pk[g][4 * ss + 2], pk[g][4 * ss + 3]});
                const int key_off = (32 * g + 16 * ss) * kRowBytes;
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) {
                    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_i16x4*)(stage + v_off[dt] + key_off));
                    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_i16x4*)(stage + v_off[dt] + key_off + 8 * kRowBytes));
                    const i16x8 vop = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    acc[dt] = mfma32<IsBf16>(vop, pop, acc[dt]);
                }
            }
    };

    if (n_tiles > 0) stage_tile<kWaves>(kbase, vbase, ks_bytes, vs_bytes, 0, p.k_seq, stage0, wave, lane);
    for (int t = 0; t < n_tiles; t += 2) {
        tile(stage0, stage1, t);
        if (t + 1 < n_tiles) tile(stage1, stage0, t + 1);
    }

    // ---- epilogue: normalise, convert, store. Lane holds, for d-tile dt,
    // dims 32dt + 8u + 4hf + (0..3) of its query in acc[dt][4u .. 4u+3].
    const float l_tot = xhalf_sum(l_run);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (my_query < p.q_seq) {
        char* orow = obase + (int64_t)my_query * p.o_row_stride * elem;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t w0 = pack2<IsBf16>(acc[dt][4 * u] * inv, acc[dt][4 * u + 1] * inv);
                const uint32_t w1 = pack2<IsBf16>(acc[dt][4 * u + 2] * inv, acc[dt][4 * u + 3] * inv);
                const int d = 32 * dt + 8 * u + 4 * hf;
                *(uint2*)(orow + d * 2) = uint2{w0, w1};
            }
    }
}

}  // namespace

int fused_attention_block_queries() { return 32 * kFusedWaves; }

hipError_t launch_fused_attention_d64(const FusedAttentionParams& params_in, bool is_bf16, hipStream_t stream) {
    FusedAttentionParams p = params_in;
    constexpr int kBlockQueries = 32 * kFusedWaves;
    p.q_blocks = (p.q_seq + kBlockQueries - 1) / kBlockQueries;
    p.total_blocks = p.q_blocks * p.heads * p.batch;
    if (p.total_blocks == 0) return hipSuccess;
    const size_t lds_bytes = 0;  // static LDS: two stages of K+V
    if (is_bf16) {
        hipLaunchKernelGGL((fused_attention_d64_kernel<kFusedWaves, true>), dim3(p.total_blocks),
                           dim3(64 * kFusedWaves), lds_bytes, stream, p);
    } else {
        hipLaunchKernelGGL((fused_attention_d64_kernel<kFusedWaves, false>), dim3(p.total_blocks),
                           dim3(64 * kFusedWaves), lds_bytes, stream, p);
    }
    return hipGetLastError();
}

}  // namespace sdxl_hip

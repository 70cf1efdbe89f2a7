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
// eight 16-byte chunks of row r stored at chunk ^ swz(r), swz(r) =
// rev3((r >> 1) & 7). The LDS serves 256 B (64 banks x 4 B) per cycle: a
// 16 B K-operand read covers 16 consecutive rows in one chunk per cycle (rows
// of equal parity must get distinct swizzles), a transposing V read covers 4
// rows x 64 B per cycle (rows r and r+2 must fall in opposite chunk halves).
// swz satisfies both, so neither read pattern has bank conflicts.
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
__device__ __forceinline__ int swz(int row) { return rev3((row >> 1) & 7); }

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

// Stages 64-key tiles of K and V into LDS. The 16 1-KiB load instructions of
// a tile (8 for K, 8 for V) are split evenly over the workgroup's waves;
// instruction n covers rows 8*(n%8) .. 8*(n%8)+7 of K (n < 8) or V (n >= 8),
// lane l the row 8*(n%8) + l/8 and the global chunk (l%8) ^ swz(row), so that
// it lands in its swizzled LDS slot. Addresses are a wave-uniform tile base
// plus a per-lane 32-bit offset fixed for the whole loop. In a tile that runs
// past k_seq the rows are clamped to the last key: their scores are masked to
// -inf, so they contribute exactly 0; the clamp only keeps the values finite.
template <int kWaves>
struct TileLoader {
    static constexpr int kPerWave = 16 / kWaves;
    const char* base[kPerWave];  // K or V pointer (wave-uniform)
    int64_t stride[kPerWave];    // row stride in bytes (wave-uniform)
    int lds_off[kPerWave];       // byte offset inside a stage (wave-uniform)
    uint32_t voff[kPerWave];     // per-lane offset from the tile base

    __device__ __forceinline__ void init(const char* kbase, const char* vbase, int64_t ks, int64_t vs, int wave,
                                         int lane) {
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const int n = wave * kPerWave + j;
            const bool is_v = n >= 8;
            base[j] = is_v ? vbase : kbase;
            stride[j] = is_v ? vs : ks;
            lds_off[j] = (is_v ? kTileBytes : 0) + 8 * (n & 7) * kRowBytes;
            const int row = 8 * (n & 7) + (lane >> 3);
            voff[j] = (uint32_t)(row * stride[j]) + (uint32_t)(((lane & 7) ^ swz(row)) << 4);
        }
    }

    template <bool kClamp>
    __device__ __forceinline__ void load(char* stage, int key0, int k_seq, int wave, int lane) const {
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const char* tile_base = base[j] + (int64_t)key0 * stride[j];
            uint32_t off = voff[j];
            if constexpr (kClamp) {
                const int row = 8 * ((wave * kPerWave + j) & 7) + (lane >> 3);
                const int key = key0 + row < k_seq ? row : k_seq - 1 - key0;
                off = (uint32_t)(key * stride[j]) + (uint32_t)(((lane & 7) ^ swz(row)) << 4);
            }
            __builtin_amdgcn_global_load_lds((const void*)(tile_base + off), (lds_void*)(stage + lds_off[j]), 16, 0, 0);
        }
    }

    // Loads tile t (keys 64t ..) clamping only when the tile is partial.
    __device__ __forceinline__ void load_tile(char* stage, int t, int k_seq, int wave, int lane) const {
        const int key0 = t * kKeyTile;
        if (key0 + kKeyTile <= k_seq) load<false>(stage, key0, k_seq, wave, lane);
        else load<true>(stage, key0, k_seq, wave, lane);
    }
};

template <int kWaves, bool IsBf16, bool kMaskAll>
__global__ __launch_bounds__(kWaves * 64, 3) void fused_attention_d64_kernel(FusedAttentionParams p) {
    constexpr int kBlockQueries = kWaves * 32;
    __shared__ __attribute__((aligned(16))) char stage0[kStageBytes];
    __shared__ __attribute__((aligned(16))) char stage1[kStageBytes];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
    // Tiles [0, n_plain) run without any masking code: they are complete and
    // there is no key mask / causal limit (kMaskAll covers those calls).
    const int n_plain = kMaskAll ? 0 : n_keys / kKeyTile;

    // Per-lane LDS byte offsets.
    // K operand: row 32g + col, chunk (2ks + hf) ^ swz(col).
    const int k_off = col * kRowBytes;
    const int k_swz = swz(col);
    // V^T operand via transposing reads: inside each 16-lane group, lane
    // r = 4j + qd supplies the address of key row 4*hf + j (+8 for the second
    // read, which flips bit 0 of the swizzle), dims 32dt + 16*((lane>>4)&1) + 4qd .. +3.
    const int g16 = lane & 15;
    const int tr_j = g16 >> 2, tr_qd = g16 & 3;
    const int tr_key = 4 * hf + tr_j;
    int v_off[2][2];  // [dt][second read]
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
        const int chunk = 4 * dt + 2 * ((lane >> 4) & 1) + (tr_qd >> 1);
#pragma unroll
        for (int hi = 0; hi < 2; ++hi)
            v_off[dt][hi] = kTileBytes + (tr_key + 8 * hi) * kRowBytes + ((chunk ^ swz(tr_key + 8 * hi)) << 4) +
                            ((tr_qd & 1) << 3);
    }

    f32x16 acc[2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] = 0.0f;
    float m_run = -__builtin_inff();
    float l_run = 0.0f;
    const float c = p.scale_log2;

    TileLoader<kWaves> loader;
    loader.init(kbase, vbase, ks_bytes, vs_bytes, wave, lane);

    auto tile = [&]<bool kMasked>(const char* stage, char* next, int t) {
        __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0): this lane's loads of tile t have landed
        __syncthreads();                     // ... and every other lane's; tile t-1 fully consumed
        // Key-mask word of this lane's key in tile t; issued before the prefetch so
        // that its wait does not also wait for the next tile's loads.
        int mask_word = 1;
        if (kMasked && p.key_mask != nullptr) {
            const int key = t * kKeyTile + lane;
            mask_word = key < p.k_seq ? p.key_mask[(int64_t)b * p.k_seq + key] : 0;
        }
        if (t + 1 < n_tiles) loader.load_tile(next, t + 1, p.k_seq, wave, lane);

        // ---- S^T = K Q^T for the two 32-key groups of the tile.
        i16x8 kop[2][4];
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                kop[g][ks] = *(const lds_i16x8*)(stage + k_off + 32 * g * kRowBytes + (((2 * ks + hf) ^ k_swz) << 4));
        f32x16 s[2];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
#pragma unroll
            for (int i = 0; i < 16; ++i) s[g][i] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) s[g] = mfma32<IsBf16>(kop[g][ks], qop[ks], s[g]);
        }

        // ---- masking (ragged tail, key mask, causal) on the tiles that need it.
        // vis bit j = key key0 + j exists and is not masked out (wave-uniform).
        if constexpr (kMasked) {
            const int key0 = t * kKeyTile;
            uint64_t vis = ~0ull;
            if (key0 + kKeyTile > p.k_seq) vis = (1ull << (p.k_seq - key0)) - 1ull;
            if (p.key_mask != nullptr) vis &= __builtin_amdgcn_ballot_w64(mask_word != 0);
            const uint32_t lane_vis = (uint32_t)(vis >> (4 * hf));
            const uint32_t lane_vis_hi = (uint32_t)(vis >> (32 + 4 * hf));
            // causal: key key0 + 32g + kk + 4hf is visible iff <= my_query
            const int causal_lim = p.causal ? my_query - key0 - 4 * hf : 0x7FFFFFFF;
#pragma unroll
            for (int g = 0; g < 2; ++g)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int kk = (i >> 2) * 8 + (i & 3);
                    const uint32_t bits = g ? lane_vis_hi : lane_vis;
                    const bool ok = ((bits >> kk) & 1u) && (32 * g + kk <= causal_lim);
                    s[g][i] = ok ? s[g][i] : -__builtin_inff();
                }
        }

        // ---- V^T operands (independent of the softmax: issue early)
        i16x8 vop[2][2][2];
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int ss = 0; ss < 2; ++ss)
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) {
                    const char* base = stage + (32 * g + 16 * ss) * kRowBytes;
                    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + v_off[dt][0]));
                    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + v_off[dt][1]));
                    vop[g][ss][dt] = i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
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
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) acc[dt] = mfma32<IsBf16>(vop[g][ss][dt], pop, acc[dt]);
            }
    };

    // Tile t lives in stage (t & 1). Plain tiles first (unrolled by two so both
    // LDS buffers are static), then the masked remainder.
    if (n_tiles > 0) loader.load_tile(stage0, 0, p.k_seq, wave, lane);
    int t = 0;
    for (; t + 1 < n_plain; t += 2) {
        tile.template operator()<false>(stage0, stage1, t);
        tile.template operator()<false>(stage1, stage0, t + 1);
    }
    if (t < n_plain) {
        tile.template operator()<false>(stage0, stage1, t);
        ++t;
        if (t < n_tiles) {
            tile.template operator()<true>(stage1, stage0, t);
            ++t;
        }
    }
    for (; t < n_tiles; t += 2) {
        tile.template operator()<true>(stage0, stage1, t);
        if (t + 1 < n_tiles) tile.template operator()<true>(stage1, stage0, t + 1);
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
    const bool mask_all = p.causal || p.key_mask != nullptr;
    const dim3 grid(p.total_blocks), block(64 * kFusedWaves);
    if (is_bf16) {
        if (mask_all) hipLaunchKernelGGL((fused_attention_d64_kernel<kFusedWaves, true, true>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((fused_attention_d64_kernel<kFusedWaves, true, false>), grid, block, 0, stream, p);
    } else {
        if (mask_all) hipLaunchKernelGGL((fused_attention_d64_kernel<kFusedWaves, false, true>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((fused_attention_d64_kernel<kFusedWaves, false, false>), grid, block, 0, stream, p);
    }
    return hipGetLastError();
}

}  // namespace sdxl_hip

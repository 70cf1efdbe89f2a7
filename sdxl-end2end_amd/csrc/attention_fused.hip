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

// Multiplies eight packed fp16/bf16 values by c (round to nearest even).
// Element-wise on a typed vector: writing dwords of a uint32 vector in a loop
// while bit-casting its elements miscompiles with this toolchain.
template <bool IsBf16>
__device__ __forceinline__ i16x8 scale_operand(i16x8 x, float c) {
    if constexpr (IsBf16) {
        const bf16x8 v = __builtin_bit_cast(bf16x8, x);
        bf16x8 r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = (__bf16)((float)v[i] * c);
        return __builtin_bit_cast(i16x8, r);
    } else {
        const f16x8 v = __builtin_bit_cast(f16x8, x);
        f16x8 r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = (_Float16)((float)v[i] * c);
        return __builtin_bit_cast(i16x8, r);
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
// a K tile plus a V tile are split evenly over the workgroup's waves;
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
    uint32_t voff[kPerWave];     // per-lane offset from the tile base

    __device__ __forceinline__ static bool is_v(int wave, int j) { return wave * kPerWave + j >= 8; }
    __device__ __forceinline__ static int lds_off(int wave, int j) { return 8 * ((wave * kPerWave + j) & 7) * kRowBytes; }

    __device__ __forceinline__ void init(const char* kbase, const char* vbase, int64_t ks, int64_t vs, int wave,
                                         int lane) {
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            base[j] = is_v(wave, j) ? vbase : kbase;
            stride[j] = is_v(wave, j) ? vs : ks;
            const int row = 8 * ((wave * kPerWave + j) & 7) + (lane >> 3);
            voff[j] = (uint32_t)(row * stride[j]) + (uint32_t)(((lane & 7) ^ swz(row)) << 4);
        }
    }

    __device__ __forceinline__ void load_one(char* buf, int j, int tile, int k_seq, int wave, int lane) const {
        const int key0 = tile * kKeyTile;
        const char* tile_base = base[j] + (int64_t)key0 * stride[j];
        uint32_t off = voff[j];
        if (key0 + kKeyTile > k_seq) {  // partial tile: clamp rows (wave-uniform branch)
            const int row = 8 * ((wave * kPerWave + j) & 7) + (lane >> 3);
            const int key = key0 + row < k_seq ? row : k_seq - 1 - key0;
            off = (uint32_t)(key * stride[j]) + (uint32_t)(((lane & 7) ^ swz(row)) << 4);
        }
        __builtin_amdgcn_global_load_lds((const void*)(tile_base + off), (lds_void*)(buf + lds_off(wave, j)), 16, 0,
                                         0);
    }

    // K tile k_tile into kbuf and V tile v_tile into vbuf; negative or
    // out-of-range tiles are skipped.
    __device__ __forceinline__ void load(char* kbuf, int k_tile, char* vbuf, int v_tile, int n_tiles, int k_seq,
                                         int wave, int lane) const {
#pragma unroll
        for (int j = 0; j < kPerWave; ++j) {
            const bool v = is_v(wave, j);
            const int tile = v ? v_tile : k_tile;
            if (tile >= 0 && tile < n_tiles) load_one(v ? vbuf : kbuf, j, tile, k_seq, wave, lane);
        }
    }
};

template <int kWaves, bool IsBf16, bool kMaskAll>
__global__ __launch_bounds__(kWaves * 64, 2) void fused_attention_d64_kernel(FusedAttentionParams p) {
    constexpr int kBlockQueries = kWaves * 32;
    // K and V tiles are double buffered at different phases: while tile t's V
    // and tile t+1's K are read, tile t+2's K and tile t+1's V are loaded.
    __shared__ __attribute__((aligned(16))) char kbuf0[kTileBytes];
    __shared__ __attribute__((aligned(16))) char kbuf1[kTileBytes];
    __shared__ __attribute__((aligned(16))) char vbuf0[kTileBytes];
    __shared__ __attribute__((aligned(16))) char vbuf1[kTileBytes];

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

    const float c = p.scale_log2;
    // Q^T operand, pre-scaled by scale*log2(e) so that the MFMA yields scores
    // directly in log2 units: lane holds dims 16*ks + 8*hf .. +7 of its query.
    i16x8 qop[4];
    if (my_query < p.q_seq) {
        const i16x8* qrow = (const i16x8*)(qbase + (int64_t)my_query * p.q_row_stride * elem);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qop[ks] = scale_operand<IsBf16>(qrow[2 * ks + hf], c);
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
    // Tiles [0, n_plain) are complete and need no mask (kMaskAll covers key-mask
    // and causal calls, where every tile is masked).
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
            v_off[dt][hi] = (tr_key + 8 * hi) * kRowBytes + ((chunk ^ swz(tr_key + 8 * hi)) << 4) + ((tr_qd & 1) << 3);
    }

    // Online-softmax state of this lane's query (shared by lanes l and l^32).
    //   m_run     anchor in log2 units; scores enter exp2 as s*c - m_run, which
    //             the QK^T MFMA produces directly by starting from neg_m = -m_run.
    //   anchored  m_run has been set from a finite tile maximum.
    // The anchor only moves on an exact-maximum pass: always for the first tile
    // and for masked tiles, otherwise only when a tile's sum of probabilities
    // exceeds 2^14 (some score rose more than ~9 above the anchor) or is not
    // finite. Probabilities therefore stay below 2^16 in fp16/bf16; the anchor
    // never exceeds the true running maximum, so nothing underflows that the
    // exact algorithm would keep.
    f32x16 acc[2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] = 0.0f;
    float m_run = 0.0f;
    bool anchored = false;
    float l_run = 0.0f;
    f32x16 neg_m;
#pragma unroll
    for (int i = 0; i < 16; ++i) neg_m[i] = 0.0f;

    TileLoader<kWaves> loader;
    loader.init(kbase, vbase, ks_bytes, vs_bytes, wave, lane);

    // S^T = K Q^T - m_run for the two 32-key groups of the K tile in kb.
    auto scores = [&](const char* kb, f32x16 (&sc)[2]) {
        i16x8 kop[2][4];
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                kop[g][ks] = *(const lds_i16x8*)(kb + k_off + 32 * g * kRowBytes + (((2 * ks + hf) ^ k_swz) << 4));
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            sc[g] = mfma32<IsBf16>(kop[g][0], qop[0], neg_m);
#pragma unroll
            for (int ks = 1; ks < 4; ++ks) sc[g] = mfma32<IsBf16>(kop[g][ks], qop[ks], sc[g]);
        }
    };

    // Exact-maximum pass over scores sc (relative to m_run): moves the anchor
    // where needed, rescales O and l, leaves sc relative to the new anchor and
    // returns the per-lane shift (for scores already computed with the old one).
    auto exact_max = [&](f32x16 (&sc)[2]) -> float {
        float mx = fmaxf(sc[0][0], sc[0][1]);
#pragma unroll
        for (int i = 2; i < 16; ++i) mx = fmaxf(mx, sc[0][i]);
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sc[1][i]);
        mx = xhalf_max(mx);
        // anchored rows move up only; unanchored rows take any finite maximum
        const bool move = anchored ? mx > 0.0f : mx > -__builtin_inff();
        const float shift = move ? mx : 0.0f;
        const float alpha = anchored ? __builtin_amdgcn_exp2f(-shift) : 0.0f;
        anchored = anchored || move;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;
        l_run *= alpha;
        m_run += shift;
#pragma unroll
        for (int i = 0; i < 16; ++i) neg_m[i] = -m_run;
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int i = 0; i < 16; ++i) sc[g][i] -= shift;
        return shift;
    };

    f32x16 s[2];  // scores of the current tile

    // One pipelined step: tile t's softmax and PV, overlapped with tile t+1's QK^T.
    // kr: K of tile t+1, vr: V of tile t; kw/vw receive K of t+2 / V of t+1.
    auto step = [&]<bool kMasked, bool kExact>(const char* kr, const char* vr, char* kw, char* vw, int t) {
        __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0): K(t+1), V(t) of this lane landed
        __syncthreads();                     // ... for every lane; step t-1 fully done with kw, vw
        int mask_word = 1;
        if (kMasked && p.key_mask != nullptr) {
            const int key = t * kKeyTile + lane;
            mask_word = key < p.k_seq ? p.key_mask[(int64_t)b * p.k_seq + key] : 0;
        }
        loader.load(kw, t + 2, vw, t + 1, n_tiles, p.k_seq, wave, lane);

        // Next tile's scores (independent of this tile's softmax; stale data when
        // t + 1 == n_tiles, never used then).
        f32x16 s_next[2];
        scores(kr, s_next);

        // ---- masking (ragged tail, key mask, causal) of tile t.
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

        // ---- softmax numerators P = exp2(s) and their sum
        auto rebase_next = [&](float shift) {
#pragma unroll
            for (int g = 0; g < 2; ++g)
#pragma unroll
                for (int i = 0; i < 16; ++i) s_next[g][i] -= shift;
        };
        if constexpr (kExact || kMasked) rebase_next(exact_max(s));
        uint32_t pk[2][8];
        float l_tile;
        auto exponentiate = [&]() {
            l_tile = 0.0f;
#pragma unroll
            for (int g = 0; g < 2; ++g)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    pk[g][i] = pack2<IsBf16>(__builtin_amdgcn_exp2f(s[g][2 * i]), __builtin_amdgcn_exp2f(s[g][2 * i + 1]));
                    l_tile = sum2<IsBf16>(pk[g][i], l_tile);
                }
        };
        exponentiate();
        if constexpr (!kExact && !kMasked) {
            // A score rose far above the anchor (sum > 2^14, or inf/NaN): redo this
            // tile with an exact maximum. Rare: scores must exceed the first
            // tile's maximum by about 9 (log2 units).
            if (__builtin_amdgcn_ballot_w64(!(l_tile <= 16384.0f))) {
                rebase_next(exact_max(s));
                exponentiate();
            }
        }
        l_run += l_tile;

        // ---- O^T += V^T P^T
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int ss = 0; ss < 2; ++ss) {
                const i16x8 pop = __builtin_bit_cast(
                    i16x8, (uint32_t __attribute__((ext_vector_type(4)))){pk[g][4 * ss], pk[g][4 * ss + 1],
                                                                           pk[g][4 * ss + 2], pk[g][4 * ss + 3]});
                const char* base = vr + (32 * g + 16 * ss) * kRowBytes;
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) {
                    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + v_off[dt][0]));
                    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + v_off[dt][1]));
                    const i16x8 vop = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    acc[dt] = mfma32<IsBf16>(vop, pop, acc[dt]);
                }
            }
#pragma unroll
        for (int g = 0; g < 2; ++g) s[g] = s_next[g];
    };

    // Prologue: K(0), V(0), K(1) in flight, then tile 0's scores.
    if (n_tiles > 0) {
        loader.load(kbuf0, 0, vbuf0, 0, n_tiles, p.k_seq, wave, lane);
        loader.load(kbuf1, 1, vbuf1, -1, n_tiles, p.k_seq, wave, lane);
        __builtin_amdgcn_s_waitcnt(0x0070);
        __syncthreads();
        scores(kbuf0, s);
    }
    // Step t reads K[(t+1)&1], V[t&1] and fills K[t&1], V[(t+1)&1]; unrolled by
    // two so that every LDS buffer is a static object. Step 0 anchors the
    // softmax; plain tiles follow, then the masked remainder.
    int t = 0;
    if (n_plain > 0) {
        step.template operator()<false, true>(kbuf1, vbuf0, kbuf0, vbuf1, 0);
        t = 1;
        for (; t + 1 < n_plain; t += 2) {
            step.template operator()<false, false>(kbuf0, vbuf1, kbuf1, vbuf0, t);
            step.template operator()<false, false>(kbuf1, vbuf0, kbuf0, vbuf1, t + 1);
        }
        if (t < n_plain) {  // t odd
            step.template operator()<false, false>(kbuf0, vbuf1, kbuf1, vbuf0, t);
            ++t;
        }
    }
    if ((t & 1) && t < n_tiles) {
        step.template operator()<true, true>(kbuf0, vbuf1, kbuf1, vbuf0, t);
        ++t;
    }
    for (; t < n_tiles; t += 2) {
        step.template operator()<true, true>(kbuf1, vbuf0, kbuf0, vbuf1, t);
        if (t + 1 < n_tiles) step.template operator()<true, true>(kbuf0, vbuf1, kbuf1, vbuf0, t + 1);
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

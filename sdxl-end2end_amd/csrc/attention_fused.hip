// Fused forward attention for head_dim 64 on gfx950 (MI355X, CDNA4).
//
// Replaces the reference's in-tree tiled kernel
// (src/cuda/flash_attention_sm80.cu:45-221) and its cuDNN SDPA backend
// (src/cuda/cudnn_sdpa.cpp:44-168): o = softmax(q k^T * scale) v per
// (batch, head), online softmax, no score matrix in memory.
//
// Work decomposition
//   One workgroup = kWaves wave64s = kWaves*32 query rows of one (b, h).
//   Every wave owns 32 query rows and walks all keys in tiles of 64 keys,
//   each tile in two groups of 32 keys. K and V tiles (64 keys x 64 dims) are
//   staged in LDS and shared by the workgroup's waves.
//
// Per wave and 32-key group (MFMA v_mfma_f32_32x32x16_{f16,bf16}):
//   S^T[key][q] = K Q^T - m/c : A = K rows from LDS (16 B per lane); B = Q^T
//                             from registers as stored (exact products); the
//                             accumulator starts at -m/c (m: the softmax
//                             anchor in log2 units, c = scale*log2(e)). The C
//                             layout puts one query per lane column: row sums
//                             stay in-lane (plus one lane<->lane+32 exchange).
//   P = exp2(c S)            one fp32 multiply and v_exp_f32 per score, packed
//                             to fp16/bf16 (v_cvt_pk_*), row sums in fp32
//                             (before rounding). Q is not pre-scaled: rounding
//                             q*c to fp16 costs 2^-12 of every score, which at
//                             logits of a few tens exceeds the output bar.
//   O^T[d][q] += V^T P^T    : A = V^T built with ds_read_b64_tr_b16 straight
//                             from the row-major V tile (no transpose pass),
//                             B = P^T from the registers holding P.
//   Software pipelining: the next group's QK^T MFMAs are issued before the
//   current group's exp2 work, so the matrix cores and the VALU overlap inside
//   each wave; only two 32-key score blocks are live.
//
// Softmax anchoring: the anchor m only moves on an exact-maximum pass, which
// runs for the first group, for masked groups, and when a group's sum of
// probabilities exceeds 2^14 or is not finite (a score rose ~9 above the
// anchor in log2 units). Probabilities stay below 2^16, representable in fp16
// and bf16; the anchor never exceeds the true running maximum, so nothing
// underflows that the exact algorithm keeps. With the reference's inputs the
// exact pass runs once per row.
//
// LDS: two K tiles and two V tiles (32 KiB). While tile t is consumed (its V,
// and K of t+1 for the next groups' operands), K of t+2 and V of t+1 stream
// in, so each load has a full tile of compute to land. Rows are 128 B; the eight 16-byte
// chunks of row r sit at chunk ^ swz(r), swz(r) = rev3((r >> 1) & 7). The LDS
// serves 256 B (64 banks x 4 B) per cycle: a 16 B K-operand read covers 16
// consecutive rows of one chunk per cycle (rows of equal parity need distinct
// swizzles) and a transposing V read covers 4 rows x 64 B per cycle (rows r
// and r+2 must fall in opposite chunk halves); swz satisfies both.
// Tiles move HBM -> LDS with global_load_lds_dwordx4 (no VGPR staging), each
// lane loading the global chunk that lands in its swizzled slot.
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
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) i16x8 lds_i16x8;
typedef __attribute__((address_space(3))) char lds_char;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;

constexpr int kHeadDim = 64;
constexpr int kKeyTile = 64;
constexpr int kRowBytes = kHeadDim * 2;           // 128
constexpr int kTileBytes = kKeyTile * kRowBytes;  // 8 KiB
constexpr int kKRing = 2;
constexpr int kVRing = 2;
constexpr float kOverflowSum = 16384.0f;          // 2^14

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

// Sum of eight fp32 probabilities as a depth-3 tree.
__device__ __forceinline__ float sum8(const float* e) {
    return ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
}

// Sum of the eight packed fp16/bf16 probabilities in pk[0..3] (fp32
// accumulation, v_dot2 against ones): the row sum of exactly the values the
// P.V product uses, four instructions instead of seven adds.
template <bool IsBf16>
__device__ __forceinline__ float sum8_packed(const uint32_t* pk) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (IsBf16) {
            const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
            s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk[i]), one, s, false);
        } else {
            const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
            s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pk[i]), one, s, false);
        }
    }
    return s;
}

// Exchange with lane l ^ 32 (the other half of the wave holds the other keys
// of the same query). ds_bpermute: the permlane32 swap builtin is folded
// incorrectly by this compiler when both operands are the same value.
__device__ __forceinline__ float xhalf_max(float x) { return fmaxf(x, __shfl_xor(x, 32, 64)); }

__device__ __forceinline__ float xhalf_sum(float x) { return x + __shfl_xor(x, 32, 64); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const lds_char*)p;
}

// One 1-KiB HBM -> LDS transfer: lane l copies 16 bytes from base + voff to
// LDS byte lds + 16*l. Issued as inline assembly so that the compiler neither
// treats later LDS reads as possible aliases of the transfer nor waits for
// earlier transfers before issuing the next (which a memory clobber causes).
// Ordering is explicit instead: the volatile statement stays in program order
// with the s_waitcnt and s_barrier builtins around it, a transfer never
// targets a buffer read in the same tile, and every tile begins with
// vmcnt(0) + barrier before its buffers are read. M0 holds the wave-uniform
// LDS destination, bound through an {m0} operand constraint so that the
// compiler itself sets M0 and knows its value.
__device__ __forceinline__ void lds_dma16(const char* base, uint32_t voff, uint32_t lds) {
    // base and lds are wave-uniform by construction; readfirstlane makes that
    // explicit so that they are allocated to SGPRs as the instruction requires.
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

__device__ __forceinline__ void wait_vmem4() { __builtin_amdgcn_s_waitcnt(0x0074); }     // vmcnt(4)

__device__ __forceinline__ void wait_vmem2() { __builtin_amdgcn_s_waitcnt(0x0072); }     // vmcnt(2)

// Output store: non-temporal (streams to memory instead of staying in L2)
// for large outputs, else ordinary. A compile-time choice: with a run-time
// flag the compiler merges both branches into one ordinary store.
template <bool kNt, typename T>
__device__ __forceinline__ void store_out(T v, T* ptr) {
    if constexpr (kNt) __builtin_nontemporal_store(v, ptr);
    else *ptr = v;
}

// Workgroup kinds of the fused kernel.
constexpr int kKindWhole = 0;  // 4 waves: 128 query rows, all keys
constexpr int kKindSplit = 1;  // 4 waves: 64 query rows, each row block's keys in two halves
constexpr int kKindSplit2 = 4;  // as kKindSplit with 64 keys of each half per stage (64 KiB of LDS)
constexpr int kKindMixed = 2;  // 12 waves: 10 consecutive 32-row blocks, 8 whole + 2 split in groups
constexpr int kKindMixed2 = 5;  // as kKindMixed for calls whose workgroups can span two heads
constexpr int kMixedFull = 8;    // waves of a mixed workgroup that take one row block and all keys
constexpr int kMixedBlocks = 10; // 32-row blocks per mixed workgroup
// Output staging after the key loop (merge slots, then 4 KiB per storing
// wave) fits in the stage buffers of each kind.
static_assert(2 * 34 * 64 * 4 + 2 * 32 * kRowBytes <= (kKRing + kVRing) * kTileBytes, "key-split epilogue staging");
static_assert(4 * 32 * kRowBytes <= (kKRing + kVRing) * kTileBytes, "whole epilogue staging");
static_assert(2 * 34 * 64 * 4 + (kMixedFull + 2) * 32 * kRowBytes <= 2 * (kKRing + kVRing) * kTileBytes, "mixed epilogue staging");

// The kernel body for one workgroup kind.
template <int kWaves, bool IsBf16, bool kMaskAll, int kKind>
__device__ __attribute__((always_inline)) inline void attention_body(const FusedAttentionParams& p,
                                                                     char (*ring)[kTileBytes]) {
    constexpr bool split2 = kKind == kKindSplit2;
    constexpr bool split = kKind == kKindSplit || split2;  // row assignment, merge and epilogue
    constexpr bool mixed = kKind == kKindMixed || kKind == kKindMixed2;
    constexpr int kBlockQueries = kWaves * 32;
    constexpr int kLoadsPerWave = 16 / kWaves;  // 1-KiB transfers per wave and tile (K and V), 4-wave kinds

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hf = lane >> 5;   // which half of the wave
    const int col = lane & 31;  // query column of this lane in the 32x32 tiles

    // Workgroup kinds. Whole: 128 query rows (4 waves x 32), all keys.
    // Key-split (ids >= whole_units): 64 query rows; wave w takes rows
    // 32 (w & 1) .. +31 and key half w >> 1, and the two halves of each row
    // block are merged through LDS at the end (split2, in the 64-KiB kernel:
    // each stage holds 64 keys of each half, so a wave steps through two
    // groups per stage as a whole wave does). Mixing the kinds lets a call
    // fill the resident workgroup slots evenly (see the launcher).
    // Mixed (one 12-wave workgroup per CU, three waves per SIMD): row blocks
    // 10i .. 10i + 9 of the flattened (batch, head, block) order; waves 0-7
    // take blocks 10i + w with all keys, waves 8-11 take blocks 10i + 8 + (w-8)/2
    // with 32-key group (w-8)%2 of every tile, merged through LDS at the end.
    // Waves w, w+4, w+8 share a SIMD, so every SIMD carries two whole blocks
    // and one half: 2.5 blocks per SIMD, the same in every tile step. One
    // staging of each K/V tile serves 10 row blocks (4 in the 4-wave kinds).
    // A workgroup spanning two heads stages both heads' tiles.
    // XCD-aware order within each kind: the hardware deals workgroup ids round
    // robin over the 8 XCDs, so each XCD gets one contiguous range of tasks
    // (row blocks of the same head share K/V in that XCD's L2).
    int task;
    {
        const int n = mixed ? p.mixed_wgs : split ? p.split_units : p.whole_units;
        const int id = split ? (int)blockIdx.x - p.whole_units : (int)blockIdx.x;
        const int xcd = id & 7, slot = id >> 3;
        const int per = n >> 3, extra = n & 7;
        task = xcd * per + (xcd < extra ? xcd : extra) + slot;
    }
    int khalf = split ? wave >> 1 : 0;  // key half (split) or key group (mixed half waves)
    bool half_wave = split;             // one 32-key group per tile step
    bool active = true;                 // a row block exists (mixed: the last workgroup may be short)
    int nsets = 1, set = 0, bh_set[2] = {0, 0};
    int bh, q0;
    if constexpr (mixed) {
        const int first = task * kMixedBlocks;
        half_wave = wave >= kMixedFull;
        const int my = half_wave ? first + kMixedFull + ((wave - kMixedFull) >> 1) : first + wave;
        khalf = half_wave ? (wave - kMixedFull) & 1 : 0;
        active = my < p.mixed_total;
        const int blk = min(my, p.mixed_total - 1);
        bh = blk / p.q_blocks;  // q_blocks: 32-row blocks per head
        q0 = (blk % p.q_blocks) * 32;
        bh_set[0] = first / p.q_blocks;
        bh_set[1] = min(first + kMixedBlocks - 1, p.mixed_total - 1) / p.q_blocks;
        nsets = bh_set[1] != bh_set[0] ? 2 : 1;
        set = bh == bh_set[0] ? 0 : 1;
    } else if constexpr (!split) {
        bh = task / p.q_blocks;
        q0 = (task % p.q_blocks) * kBlockQueries + wave * 32;
    } else {
        const int blocks64 = p.q_seq / 64;  // q_seq % 128 == 0 for key-split calls
        const int gb = 2 * p.whole_units + task;
        bh = gb / blocks64;
        q0 = (gb % blocks64) * 64 + (wave & 1) * 32;
    }
    const int qblk = q0 / kBlockQueries;
    char (*kring)[kTileBytes] = ring + (mixed ? 4 * set : 0);
    char (*vring)[kTileBytes] = kring + kKRing;
    const int h = bh % p.heads;
    const int b = bh / p.heads;

    const int64_t elem = 2;
    const char* qbase = (const char*)p.q + ((int64_t)b * p.q_seq * p.q_row_stride + (int64_t)h * kHeadDim) * elem;
    const char* kbase = (const char*)p.k + ((int64_t)b * p.k_seq * p.k_row_stride + (int64_t)h * kHeadDim) * elem;
    const char* vbase = (const char*)p.v + ((int64_t)b * p.k_seq * p.v_row_stride + (int64_t)h * kHeadDim) * elem;
    char* obase = (char*)p.o + ((int64_t)b * p.q_seq * p.o_row_stride + (int64_t)h * kHeadDim) * elem;
    const int64_t ks_bytes = p.k_row_stride * elem, vs_bytes = p.v_row_stride * elem;

    const int my_query = q0 + col;

    // Scores leave the MFMA unscaled (exact products, fp32 sums); exp2
    // arguments are c * S with c = scale*log2(e) > 0 (checked on the host).
    const float c = p.scale_log2;
    const float ic = p.inv_scale_log2;  // 1 / c, finite (checked on the host)
    // Q^T operand as stored: lane holds dims 16*ks + 8*hf .. +7 of its query.
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
    // Key-split calls: stage t holds keys 32t .. +31 of each half (rows 0-31
    // half 0, rows 32-63 half 1); k_seq % 64 == 0.
    const int half_keys = p.k_seq / 2;
    const int n_tiles = split2 ? p.k_seq / (2 * kKeyTile)
                               : (split || mixed) ? p.k_seq / kKeyTile : (n_keys + kKeyTile - 1) / kKeyTile;
    // Tiles [0, n_plain) are complete and need no mask (kMaskAll covers key-mask
    // and causal calls, where every tile is masked).
    const int n_plain = kMaskAll ? 0 : n_keys / kKeyTile;

    // ---- tile transfers: the 16 1-KiB transfers of a K tile plus a V tile are
    // split over the waves; transfer n covers the 8-row slab n%8 (rows
    // 8*(n%8) .. +7) of K (n < 8) or V (n >= 8); lane l takes slab row l/8 and
    // the global chunk (l%8) ^ swz(row), which lands in its swizzled slot.
    // With row = 8 s + l/8, swz(row) depends only on l and the parity of the
    // slab s, so a transfer's global offset is a per-lane part for its slab
    // parity, computed once (24-bit multiplies: row strides are below 2^24
    // bytes, checked on the host), plus 8 s rows added to the scalar base.
    auto lane_off = [&](int parity, int64_t stride) __attribute__((always_inline)) -> uint32_t {
        const int sw = rev3((4 * parity + (lane >> 4)) & 7);
        return __umul24((uint32_t)(lane >> 3), (uint32_t)stride) + (uint32_t)(((lane & 7) ^ sw) << 4);
    };

    // Whole and key-split workgroups: wave w issues the four K (w < 2) or V
    // (w >= 2) slabs of parity w & 1, i.e. slabs 2j + (w & 1), j = 0..3: one
    // per-lane offset per wave. Issues the transfers of K tile kt and V tile vt
    // (skipping tiles out of range); rows past the end of a partial last tile
    // re-read the last key (per-lane clamp, the slow form).
    const int64_t whole_stride = wave < 2 ? ks_bytes : vs_bytes;
    const uint32_t whole_off = (!mixed) ? lane_off(wave & 1, whole_stride) : 0u;
    auto issue = [&](int kt, int vt) __attribute__((always_inline)) {
        const bool is_v = wave >= 2;
        const int tile = is_v ? vt : kt;
        if (tile < 0 || tile >= n_tiles) return;
        const int key0 = tile * kKeyTile;
        const char* buf = is_v ? vring[tile % kVRing] : kring[tile % kKRing];
        if (key0 + kKeyTile <= p.k_seq) {
#pragma unroll
            for (int j = 0; j < kLoadsPerWave; ++j) {
                const int slab = 2 * j + (wave & 1);
                const char* slab_base = (is_v ? vbase : kbase) + (int64_t)(key0 + 8 * slab) * whole_stride;
                lds_dma16(slab_base, whole_off, lds_addr(buf + 8 * slab * kRowBytes));
            }
        } else {
            const char* tile_base = (is_v ? vbase : kbase) + (int64_t)key0 * whole_stride;
#pragma unroll
            for (int j = 0; j < kLoadsPerWave; ++j) {
                const int slab = 2 * j + (wave & 1);
                const int row = 8 * slab + (lane >> 3);
                const int key = min(row, p.k_seq - 1 - key0);  // clamp rows of a partial tile
                const uint32_t off =
                    __umul24((uint32_t)key, (uint32_t)whole_stride) + (uint32_t)(((lane & 7) ^ swz(row)) << 4);
                lds_dma16(tile_base, off, lds_addr(buf + 8 * slab * kRowBytes));
            }
        }
    };

    // Key-split stages: slab s covers 8 rows of one key half (slabs 0-3 half
    // 0, 4-7 half 1); stage t holds keys 32t .. +31 of each half.
    auto issue_split = [&](int kt, int vt) __attribute__((always_inline)) {
        const bool is_v = wave >= 2;
        const int tile = is_v ? vt : kt;
        if (tile < 0 || tile >= n_tiles) return;
        const char* buf = is_v ? vring[tile % kVRing] : kring[tile % kKRing];
#pragma unroll
        for (int j = 0; j < kLoadsPerWave; ++j) {
            const int slab = 2 * j + (wave & 1), half = slab >> 2;
            const char* slab_base =
                (is_v ? vbase : kbase) + (int64_t)(half * half_keys + 32 * tile + 8 * (slab & 3)) * whole_stride;
            lds_dma16(slab_base, whole_off, lds_addr(buf + 8 * slab * kRowBytes));
        }
    };

    // Key-split stages of 64 keys per half (split2): stage t holds keys
    // 64t .. +63 of half 0 in rows 0-63 and of half 1 in rows 64-127 of a
    // 128-row buffer (two consecutive tiles); slab n covers rows 8n .. 8n+7.
    auto issue_split2 = [&](int kt, int vt) __attribute__((always_inline)) {
        const bool is_v = wave >= 2;
        const int tile = is_v ? vt : kt;
        if (tile < 0 || tile >= n_tiles) return;
        // byte offset, not an indexed choice of buffers (which the compiler
        // turned into a pointer table in scratch, read under vmcnt waits)
        const char* buf = &ring[0][0] + (2 * ((is_v ? kKRing : 0) + (tile & 1))) * kTileBytes;
#pragma unroll
        for (int j = 0; j < 2 * kLoadsPerWave; ++j) {
            const int slab = 2 * j + (wave & 1), half = slab >> 3;
            const char* slab_base =
                (is_v ? vbase : kbase) + (int64_t)(half * half_keys + 64 * tile + 8 * (slab & 7)) * whole_stride;
            lds_dma16(slab_base, whole_off, lds_addr(buf + 8 * slab * kRowBytes));
        }
    };

    // Mixed workgroups: the 16 transfers of each staged head go to the four
    // half waves (two K slabs each: 8 + i takes slabs i and i + 4), which
    // have one group per tile step against the whole waves' two and so slack
    // at every barrier, and to the eight whole waves (V slab w each): the
    // issue of a transfer holds its wave for tens of cycles, and whole waves
    // then issue one instead of two (c3 90.9 -> 88.2 us; moving V to the half
    // waves as well measured no faster). Every wave's slabs have parity w & 1,
    // one per-lane offset per wave; k_seq % 64 == 0. The head index is a
    // compile-time loop variable so the base pointers stay scalars.
    const char* set_k0 = (const char*)p.k + ((int64_t)(bh_set[0] / p.heads) * p.k_seq * p.k_row_stride +
                                             (int64_t)(bh_set[0] % p.heads) * kHeadDim) * elem;
    const char* set_k1 = (const char*)p.k + ((int64_t)(bh_set[1] / p.heads) * p.k_seq * p.k_row_stride +
                                             (int64_t)(bh_set[1] % p.heads) * kHeadDim) * elem;
    const char* set_v0 = (const char*)p.v + ((int64_t)(bh_set[0] / p.heads) * p.k_seq * p.v_row_stride +
                                             (int64_t)(bh_set[0] % p.heads) * kHeadDim) * elem;
    const char* set_v1 = (const char*)p.v + ((int64_t)(bh_set[1] / p.heads) * p.k_seq * p.v_row_stride +
                                             (int64_t)(bh_set[1] % p.heads) * kHeadDim) * elem;
    // kKindMixed2 (calls whose blocks per head are not a multiple of 10, so
    // that some workgroups stage two heads, nsets == 2, with twice the
    // transfers): the second head's V slabs go to the half waves as well (half
    // wave 8 + i takes V slabs p + 4r and p + 4r + 2, p = i & 1, r = i >> 1), so
    // that the whole waves still issue one transfer per tile step (c3 86.2 ->
    // 85.0 us). A kind of its own: the extra code in the common kind measured
    // 0.8-1.6 % slower on calls where no workgroup spans two heads.
    constexpr bool v1_on_half = kKind == kKindMixed2;
    const bool mixed_v = wave < kMixedFull;
    const int64_t mixed_stride = mixed_v ? vs_bytes : ks_bytes;
    const uint32_t mixed_off = mixed ? lane_off(wave & 1, mixed_stride) : 0u;
    auto issue_mixed = [&](int kt, int vt) __attribute__((always_inline)) {
        const int tile = mixed_v ? vt : kt;
        if constexpr (!v1_on_half) {
            if (tile < 0 || tile >= n_tiles) return;
#pragma unroll
            for (int sidx = 0; sidx < 2; ++sidx) {
                if (sidx == 1 && nsets == 1) break;
                const char* base = mixed_v ? (sidx ? set_v1 : set_v0) : (sidx ? set_k1 : set_k0);
                const char* buf = mixed_v ? ring[4 * sidx + kKRing + tile % kVRing] : ring[4 * sidx + tile % kKRing];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    if (j == 1 && mixed_v) break;
                    const int slab = mixed_v ? wave : (wave - kMixedFull) + 4 * j;
                    const char* slab_base = base + (int64_t)(tile * kKeyTile + 8 * slab) * mixed_stride;
                    lds_dma16(slab_base, mixed_off, lds_addr(buf + 8 * slab * kRowBytes));
                }
            }
        } else {
            if (tile >= 0 && tile < n_tiles) {
#pragma unroll
                for (int sidx = 0; sidx < 2; ++sidx) {
                    if (sidx == 1 && (nsets == 1 || mixed_v)) break;
                    const char* base = mixed_v ? set_v0 : (sidx ? set_k1 : set_k0);
                    const char* buf = mixed_v ? ring[kKRing + tile % kVRing] : ring[4 * sidx + tile % kKRing];
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        if (j == 1 && mixed_v) break;
                        const int slab = mixed_v ? wave : (wave - kMixedFull) + 4 * j;
                        const char* slab_base = base + (int64_t)(tile * kKeyTile + 8 * slab) * mixed_stride;
                        lds_dma16(slab_base, mixed_off, lds_addr(buf + 8 * slab * kRowBytes));
                    }
                }
            }
            if (!mixed_v && nsets == 2 && vt >= 0 && vt < n_tiles) {
                const int i = wave - kMixedFull;
                char* buf = ring[4 + kKRing + vt % kVRing];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int slab = (i & 1) + 4 * (i >> 1) + 2 * j;
                    const char* slab_base = set_v1 + (int64_t)(vt * kKeyTile + 8 * slab) * vs_bytes;
                    lds_dma16(slab_base, mixed_off, lds_addr(buf + 8 * slab * kRowBytes));
                }
            }
        }
    };

    // ---- per-lane LDS byte offsets.
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

    // ---- online-softmax state of this lane's query (shared by lanes l, l^32).
    f32x16 acc[2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] = 0.0f;
    float m_run = 0.0f;     // anchor, log2 units
    bool anchored = false;  // m_run came from a finite maximum
    float l_run = 0.0f;
    // Accumulator seed of QK^T: -m_run in every entry. Loop-carried; the
    // rare anchor update rewrites it in place (tied asm operands) so that the
    // join after that path needs no copies.
    f32x16 neg_m;
#pragma unroll
    for (int i = 0; i < 16; ++i) neg_m[i] = 0.0f;

    // K operands (4 x 16 B) of key group g of the K tile in kb.
    auto load_k = [&](const char* kb, int g, i16x8 (&kop)[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            kop[ks] = *(const lds_i16x8*)(kb + k_off + 32 * g * kRowBytes + (((2 * ks + hf) ^ k_swz) << 4));
    };
    // V^T operands of 16-key half ss of key group g of the V tile in vb: [dt].
    auto load_v = [&](const char* vb, int g, int ss, i16x8 (&vop)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
            const char* base = vb + (32 * g + 16 * ss) * kRowBytes;
            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + v_off[dt][0]));
            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + v_off[dt][1]));
            vop[dt] = i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
    };

    // Exact-maximum pass over the exp2 arguments sc[i0, i1) (scaled scores,
    // relative to m_run): moves the anchor where needed (anchored rows move up
    // only, unanchored rows take any finite maximum), rescales O and l and
    // returns the shift (log2 units) every exp2 argument formed against the
    // old anchor must subtract; raw (unscaled) scores subtract shift / c
    // (times ic = 1 / c).
    auto exact_max = [&](const f32x16& sc, int i0, int i1) __attribute__((always_inline)) -> float {
        float mx = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (i >= i0 && i < i1) mx = fmaxf(mx, sc[i]);
        mx = xhalf_max(mx);
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
        const float nm = -m_run * ic;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float x = neg_m[i];
            asm volatile("v_mov_b32 %0, %1" : "+v"(x) : "v"(nm));
            neg_m[i] = x;
        }
        return shift;
    };

    // One pipelined group step (32 keys of tile t, group g; s_cur holds its
    // exp2 arguments c * S - m, scaled in place during the previous step).
    // Overlapped inside the wave: the next group's QK^T chain (K operands in
    // kop, prefetched one step earlier) runs on the matrix core while this
    // group's exponentials run on the VALU; P.V of each 16-key half follows as
    // soon as its probabilities are packed. The instruction order is pinned
    // with scheduling barriers so that every dependent MFMA has independent
    // VALU work issued between it and its predecessor (in-order issue would
    // otherwise stall the wave on the chain). At the end, the K operands of
    // the group after next (tile buffer kn2, group g2) are prefetched into kop.
    // kMasked/kExact: exact maximum over the whole group first (masked tiles,
    // first tile); otherwise each half is checked for overflow after the fact.
    auto group_step = [&]<bool kMasked, bool kExact, bool kPrefetchK = true>(f32x16& s_cur, f32x16& s_next, i16x8 (&kop)[4], const char* vb,
                                                     int g, int t, uint64_t vis, const char* kn2, int g2,
                                                     bool have_next) __attribute__((always_inline)) {
        // V^T operands of both 16-key halves in their own registers; the second
        // half's are read in slot 3, two slots ahead of their MFMAs (read just
        // before them, c3 94.1 -> 93.8 us, c1 17.1 -> 16.9 us)
        i16x8 vop[2], vop1[2];
        load_v(vb, g, 0, vop);
        if constexpr (kMasked) {
            const int key0 = t * kKeyTile + 32 * g;
            const uint32_t lane_vis = (uint32_t)(vis >> (32 * g + 4 * hf));
            // causal: key key0 + kk + 4hf is visible iff <= my_query
            const int causal_lim = p.causal ? my_query - key0 - 4 * hf : 0x7FFFFFFF;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int kk = (i >> 2) * 8 + (i & 3);
                const bool ok = ((lane_vis >> kk) & 1u) && (kk <= causal_lim);
                s_cur[i] = ok ? s_cur[i] : -__builtin_inff();
            }
        }
        if constexpr (kMasked || kExact) {
            const float shift = exact_max(s_cur, 0, 16);
#pragma unroll
            for (int i = 0; i < 16; ++i) s_cur[i] -= shift;
        }
        float e[16];
        uint32_t pk[8];
        constexpr bool kCheck = !kMasked && !kExact;

        // Eight slots, each one MFMA followed by about its duration (32 cycles)
        // of VALU work that does not depend on it, pinned with scheduling
        // barriers: the wave keeps issuing while the matrix core runs, and the
        // dependent QK^T chain always has a slot between its links. The next
        // group's raw scores are scaled in slots 6-8, after its chain is done.
        // 1: QK1 | exp 0-3
        s_next = mfma32<IsBf16>(kop[0], qop[0], neg_m);
#pragma unroll
        for (int i = 0; i < 4; ++i) e[i] = __builtin_amdgcn_exp2f(s_cur[i]);
        __builtin_amdgcn_sched_barrier(0);
        // 2: QK2 | exp 4-7
        s_next = mfma32<IsBf16>(kop[1], qop[1], s_next);
#pragma unroll
        for (int i = 4; i < 8; ++i) e[i] = __builtin_amdgcn_exp2f(s_cur[i]);
        __builtin_amdgcn_sched_barrier(0);
        // 3: QK3 | V^T operands of half 1; pack + row sum of half 0, overflow check
        s_next = mfma32<IsBf16>(kop[2], qop[2], s_next);
        load_v(vb, g, 1, vop1);
#pragma unroll
        for (int i = 0; i < 4; ++i) pk[i] = pack2<IsBf16>(e[2 * i], e[2 * i + 1]);
        float l_a = sum8_packed<IsBf16>(pk);
        if constexpr (kCheck) {
            // Half 0 rose far above the anchor (sum > 2^14, or inf/NaN): exact
            // maximum over it and recompute. Rare.
            if (__builtin_expect(__builtin_amdgcn_ballot_w64(!(l_a <= kOverflowSum)) != 0, 0)) {
                const float shift = exact_max(s_cur, 0, 8);
                const float raw_shift = shift * ic;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    s_cur[i] -= shift;
                    s_next[i] -= raw_shift;  // partial QK^T sum seeded with the old anchor
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) e[i] = __builtin_amdgcn_exp2f(s_cur[i]);
#pragma unroll
                for (int i = 0; i < 4; ++i) pk[i] = pack2<IsBf16>(e[2 * i], e[2 * i + 1]);
                l_a = sum8_packed<IsBf16>(pk);
            }
        }
        l_run += l_a;
        __builtin_amdgcn_sched_barrier(0);
        // 4: QK4 | exp 8-11
        s_next = mfma32<IsBf16>(kop[3], qop[3], s_next);
#pragma unroll
        for (int i = 8; i < 12; ++i) e[i] = __builtin_amdgcn_exp2f(s_cur[i]);
        __builtin_amdgcn_sched_barrier(0);
        // 5: PV half 0, d 0-31 | exp 12-15; K operands of the group after next
        // (unconditional: stale data past the last tile is never used)
        const i16x8 p0 = __builtin_bit_cast(i16x8, u32x4{pk[0], pk[1], pk[2], pk[3]});
        acc[0] = mfma32<IsBf16>(vop[0], p0, acc[0]);
#pragma unroll
        for (int i = 12; i < 16; ++i) e[i] = __builtin_amdgcn_exp2f(s_cur[i]);
        if constexpr (kPrefetchK) load_k(kn2, g2, kop);
        __builtin_amdgcn_sched_barrier(0);
        // 6: PV half 0, d 32-63 | pack + row sum of half 1, overflow check
        acc[1] = mfma32<IsBf16>(vop[1], p0, acc[1]);
#pragma unroll
        for (int i = 4; i < 8; ++i) pk[i] = pack2<IsBf16>(e[2 * i], e[2 * i + 1]);
        float l_b = sum8_packed<IsBf16>(pk + 4);
        if constexpr (kCheck) {
            if (__builtin_expect(__builtin_amdgcn_ballot_w64(!(l_b <= kOverflowSum)) != 0, 0)) {
                const float shift = exact_max(s_cur, 8, 16);
                const float raw_shift = shift * ic;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    s_cur[i] -= shift;
                    s_next[i] -= raw_shift;
                }
#pragma unroll
                for (int i = 8; i < 16; ++i) e[i] = __builtin_amdgcn_exp2f(s_cur[i]);
#pragma unroll
                for (int i = 4; i < 8; ++i) pk[i] = pack2<IsBf16>(e[2 * i], e[2 * i + 1]);
                l_b = sum8_packed<IsBf16>(pk + 4);
            }
        }
        l_run += l_b;
        __builtin_amdgcn_sched_barrier(0);
        // 7: PV half 1, d 0-31 | scale the next group's scores 0-7
        const i16x8 p1 = __builtin_bit_cast(i16x8, u32x4{pk[4], pk[5], pk[6], pk[7]});
        acc[0] = mfma32<IsBf16>(vop1[0], p1, acc[0]);
#pragma unroll
        for (int i = 0; i < 8; ++i) s_next[i] *= c;
        __builtin_amdgcn_sched_barrier(0);
        // 8: PV half 1, d 32-63 | scale the next group's scores 8-15
        acc[1] = mfma32<IsBf16>(vop1[1], p1, acc[1]);
#pragma unroll
        for (int i = 8; i < 16; ++i) s_next[i] *= c;
        (void)have_next;
    };

    // ---- main loop. Step j = 2t + g handles key group g of tile t; it needs
    // K operands of group j+1 (loaded in step j-1) and V(t), and prefetches the
    // K operands of group j+2 from K(t+1). Tile t starts K(t+2), V(t+1): two K
    // and two V buffers suffice. sa/sb: scores of groups 0/1.
    f32x16 sa, sb;
    i16x8 kop[4];
    if constexpr (split && !split2) {
        // ---- key-split workgroup: one 32-key group per stage and wave (group
        // khalf of the stage buffers). The group after next lies in a stage not
        // yet resident, so each stage loads the next group's K operands at its
        // start instead of prefetching them a step earlier.
        issue_split(0, 0);
        issue_split(1, -1);
        wait_vmem_all();
        __syncthreads();
        load_k(kring[0], khalf, kop);
        sa = mfma32<IsBf16>(kop[0], qop[0], neg_m);
#pragma unroll
        for (int ks = 1; ks < 4; ++ks) sa = mfma32<IsBf16>(kop[ks], qop[ks], sa);
#pragma unroll
        for (int i = 0; i < 16; ++i) sa[i] *= c;  // exp2 arguments of the first group
        auto stage = [&]<bool kFirst, bool kOdd>(int t) __attribute__((always_inline)) {
            wait_vmem_all();  // this lane's transfers of K(t+1), V(t) landed
            __syncthreads();  // ... and every lane's; stage t-1 fully consumed
            issue_split(t + 2, t + 1);
            load_k(kring[kOdd ? 0 : 1], khalf, kop);  // K(t+1) (stale past the end, unused)
            const char* v_t = vring[kOdd ? 1 : 0];
            if constexpr (kOdd) group_step.template operator()<false, kFirst, false>(sb, sa, kop, v_t, khalf, t, ~0ull, v_t, 0, true);
            else group_step.template operator()<false, kFirst, false>(sa, sb, kop, v_t, khalf, t, ~0ull, v_t, 0, true);
        };
        int t = 0;
        if (n_tiles > 0) {
            stage.template operator()<true, false>(0);
            for (t = 1; t + 1 < n_tiles; t += 2) {
                stage.template operator()<false, true>(t);
                stage.template operator()<false, false>(t + 1);
            }
            if (t < n_tiles) stage.template operator()<false, true>(t);
        }
    } else if constexpr (split2) {
        // ---- key-split workgroup with 64 keys of each half per stage: each
        // wave steps through two groups per stage as a whole wave does (its
        // half's rows of the 128-row stage buffers), so the K operands of the
        // group after next are prefetched across stages as in the whole kind.
        const int hrow = khalf * 64 * kRowBytes;
        issue_split2(0, 0);
        issue_split2(1, -1);
        wait_vmem_all();
        __syncthreads();
        load_k(&ring[0][0] + hrow, 0, kop);
        sa = mfma32<IsBf16>(kop[0], qop[0], neg_m);
#pragma unroll
        for (int ks = 1; ks < 4; ++ks) sa = mfma32<IsBf16>(kop[ks], qop[ks], sa);
#pragma unroll
        for (int i = 0; i < 16; ++i) sa[i] *= c;  // exp2 arguments of the first group
        load_k(&ring[0][0] + hrow, 1, kop);
        auto stage2 = [&]<bool kFirst, bool kOdd>(int t) __attribute__((always_inline)) {
            wait_vmem_all();  // this lane's transfers of K(t+1), V(t) landed
            __syncthreads();  // ... and every lane's; stage t-1 fully consumed
            issue_split2(t + 2, t + 1);
            const char* v_t = &ring[2 * (kKRing + (kOdd ? 1 : 0))][0] + hrow;
            const char* k_t1 = &ring[2 * (kOdd ? 0 : 1)][0] + hrow;
            group_step.template operator()<false, kFirst>(sa, sb, kop, v_t, 0, t, ~0ull, k_t1, 0, true);
            group_step.template operator()<false, false>(sb, sa, kop, v_t, 1, t, ~0ull, k_t1, 1, true);
        };
        int t = 0;
        if (n_tiles > 0) {
            stage2.template operator()<true, false>(0);
            for (t = 1; t + 1 < n_tiles; t += 2) {
                stage2.template operator()<false, true>(t);
                stage2.template operator()<false, false>(t + 1);
            }
            if (t < n_tiles) stage2.template operator()<false, true>(t);
        }
    } else if constexpr (mixed) {
        // ---- mixed workgroup: whole waves step through both groups of every
        // tile (as the whole kind), half waves through group khalf of every
        // tile (as the key-split kind); one barrier per tile step for all.
        issue_mixed(0, 0);
        issue_mixed(1, -1);
        wait_vmem_all();
        __syncthreads();
        load_k(kring[0], khalf, kop);
        sa = mfma32<IsBf16>(kop[0], qop[0], neg_m);
#pragma unroll
        for (int ks = 1; ks < 4; ++ks) sa = mfma32<IsBf16>(kop[ks], qop[ks], sa);
#pragma unroll
        for (int i = 0; i < 16; ++i) sa[i] *= c;  // exp2 arguments of the first group
        if (!half_wave) load_k(kring[0], 1, kop);
        // Whole and half waves run separate loops (same barrier sequence), so
        // each keeps its own register allocation.
        auto whole_step = [&]<bool kFirst, bool kOdd>(int t) __attribute__((always_inline)) {
            wait_vmem_all();  // this lane's transfers of K(t+1), V(t) landed
            __syncthreads();  // ... and every lane's; step t-1 fully consumed
            issue_mixed(t + 2, t + 1);
            const char* v_t = vring[kOdd ? 1 : 0];
            const char* k_t1 = kring[kOdd ? 0 : 1];
            group_step.template operator()<false, kFirst>(sa, sb, kop, v_t, 0, t, ~0ull, k_t1, 0, true);
            group_step.template operator()<false, false>(sb, sa, kop, v_t, 1, t, ~0ull, k_t1, 1, true);
        };
        auto half_step = [&]<bool kFirst, bool kOdd>(int t) __attribute__((always_inline)) {
            wait_vmem_all();
            __syncthreads();
            issue_mixed(t + 2, t + 1);
            const char* v_t = vring[kOdd ? 1 : 0];
            load_k(kring[kOdd ? 0 : 1], khalf, kop);  // K(t+1) (stale past the end, unused)
            if constexpr (kOdd) group_step.template operator()<false, kFirst, false>(sb, sa, kop, v_t, khalf, t, ~0ull, v_t, 0, true);
            else group_step.template operator()<false, kFirst, false>(sa, sb, kop, v_t, khalf, t, ~0ull, v_t, 0, true);
        };
        // n_tiles >= 1 (k_seq >= 64)
        if (!half_wave) {
            whole_step.template operator()<true, false>(0);
            int t = 1;
            for (; t + 1 < n_tiles; t += 2) {
                whole_step.template operator()<false, true>(t);
                whole_step.template operator()<false, false>(t + 1);
            }
            if (t < n_tiles) whole_step.template operator()<false, true>(t);
        } else {
            half_step.template operator()<true, false>(0);
            int t = 1;
            for (; t + 1 < n_tiles; t += 2) {
                half_step.template operator()<false, true>(t);
                half_step.template operator()<false, false>(t + 1);
            }
            if (t < n_tiles) half_step.template operator()<false, true>(t);
        }
    } else {
    if (n_tiles > 0) {
        issue(0, 0);
        issue(1, -1);
        wait_vmem_all();
        __syncthreads();
        load_k(kring[0], 0, kop);
        sa = mfma32<IsBf16>(kop[0], qop[0], neg_m);
#pragma unroll
        for (int ks = 1; ks < 4; ++ks) sa = mfma32<IsBf16>(kop[ks], qop[ks], sa);
#pragma unroll
        for (int i = 0; i < 16; ++i) sa[i] *= c;  // exp2 arguments of the first group
        load_k(kring[0], 1, kop);
    }
    // kOdd: parity of t, so that every ring slot below is a compile-time
    // offset (folded into the LDS instructions' immediates).
    auto tile = [&]<bool kMasked, bool kFirst, bool kOdd>(int t) __attribute__((always_inline)) {
        wait_vmem_all();  // this lane's transfers of K(t+1), V(t) landed
        __syncthreads();  // ... and every lane's; tile t-1 fully consumed
        uint64_t vis = ~0ull;
        if constexpr (kMasked) {
            // vis bit j: key 64t + j exists and is not masked out (wave-uniform).
            const int key0 = t * kKeyTile;
            if (p.key_mask != nullptr) {
                const int key = key0 + lane;
                const int word = key < p.k_seq ? p.key_mask[(int64_t)b * p.k_seq + key] : 0;
                vis = __builtin_amdgcn_ballot_w64(word != 0);
            }
            if (key0 + kKeyTile > p.k_seq) vis &= (1ull << (p.k_seq - key0)) - 1ull;
        }
        issue(t + 2, t + 1);
        const char* v_t = vring[kOdd ? 1 : 0];
        const char* k_t1 = kring[kOdd ? 0 : 1];
        group_step.template operator()<kMasked, kMasked || kFirst>(sa, sb, kop, v_t, 0, t, vis, k_t1, 0, true);
        group_step.template operator()<kMasked, kMasked>(sb, sa, kop, v_t, 1, t, vis, k_t1, 1, true);
    };
    int t = 0;
    if (n_plain > 0) {
        tile.template operator()<false, true, false>(0);
        for (t = 1; t + 1 < n_plain; t += 2) {
            tile.template operator()<false, false, true>(t);
            tile.template operator()<false, false, false>(t + 1);
        }
        if (t < n_plain) {
            tile.template operator()<false, false, true>(t);
            ++t;
        }
    }
    if ((t & 1) && t < n_tiles) {
        tile.template operator()<true, false, true>(t);
        ++t;
    }
    for (; t < n_tiles; t += 2) {
        tile.template operator()<true, false, false>(t);
        if (t + 1 < n_tiles) tile.template operator()<true, false, true>(t + 1);
    }

    }  // whole workgroup

    if constexpr (split || mixed) {
        // ---- merge the two key parts of each split row block: the part-1
        // wave parks (O, anchor, row sum) in LDS, the part-0 wave combines in
        // fixed order and stores.
        __syncthreads();  // every wave is done with the stage buffers
        const int slot = split ? (wave & 1) : (wave - kMixedFull) >> 1;
        float* park = (float*)&ring[0][0] + (half_wave ? slot : 0) * (34 * 64) + lane;
        const bool parks = half_wave && khalf == 1;
        if (parks) {
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) park[(16 * dt + i) * 64] = acc[dt][i];
            park[32 * 64] = anchored ? m_run : -__builtin_inff();
            park[33 * 64] = l_run;
        }
        __syncthreads();
        if (parks) return;
        if (half_wave) {
            const float m0 = anchored ? m_run : -__builtin_inff();
            const float m1 = park[32 * 64];
            const float mx = fmaxf(m0, m1);
            // Scale factors 2^(m - mx); an empty part (-inf) weighs 0.
            const float a0 = m0 == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m0 - mx);
            const float a1 = m1 == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m1 - mx);
#pragma unroll
            for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[dt][i] = acc[dt][i] * a0 + park[(16 * dt + i) * 64] * a1;
            l_run = l_run * a0 + park[33 * 64] * a1;
        }
    }

    // ---- epilogue: normalise, convert, and write the wave's 32 output rows
    // to LDS (a wave-private 4 KiB buffer past the merge slots, 16-byte
    // chunks XOR-swizzled by row as the K tiles), then store whole 128-byte
    // row segments (8 lanes per row) with non-temporal stores. Lane holds,
    // for d-tile dt, dims 32dt + 8u + 4hf + (0..3) of its query in
    // acc[dt][4u .. 4u+3], i.e. half hf of 16-byte chunk 4dt + u.
    if constexpr (!split && !mixed) __syncthreads();  // every wave is done with the stage buffers
    const float l_tot = xhalf_sum(l_run);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (active) {
        constexpr int kParkBytes = 2 * 34 * 64 * 4;  // merge slots (split and mixed kinds)
        const int stage = mixed ? (half_wave ? kMixedFull + ((wave - kMixedFull) >> 1) : wave) : split ? (wave & 1) : wave;
        char* sbuf = &ring[0][0] + ((split || mixed) ? kParkBytes : 0) + stage * (32 * kRowBytes);
        const int sw = swz(col);
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t w0 = pack2<IsBf16>(acc[dt][4 * u] * inv, acc[dt][4 * u + 1] * inv);
                const uint32_t w1 = pack2<IsBf16>(acc[dt][4 * u + 2] * inv, acc[dt][4 * u + 3] * inv);
                *(lds_u32x2*)(sbuf + col * kRowBytes + (((4 * dt + u) ^ sw) << 4) + 8 * hf) = u32x2{w0, w1};
            }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = 8 * j + (lane >> 3);
            const u32x4 w = *(const lds_u32x4*)(sbuf + row * kRowBytes + (((lane & 7) ^ swz(row)) << 4));
            if (q0 + row < p.q_seq)
                store_out<mixed>(w, (u32x4*)(obase + (int64_t)(q0 + row) * p.o_row_stride * elem + 16 * (lane & 7)));
        }
    }
}

// Whole and key-split workgroups share one kernel (one grid); each kind is
// a separate instantiation of the body, so neither constrains the other's
// register allocation. K ring then V ring in one array (the key-split merge
// reuses all of it).
template <int kWaves, bool IsBf16, bool kMaskAll>
__global__ __launch_bounds__(kWaves * 64, 3) void fused_attention_d64_kernel(FusedAttentionParams p) {
    __shared__ __attribute__((aligned(16))) char ring[kKRing + kVRing][kTileBytes];
    if constexpr (!kMaskAll) {
        if ((int)blockIdx.x >= p.whole_units) {
            attention_body<kWaves, IsBf16, false, kKindSplit>(p, ring);
            return;
        }
    }
    attention_body<kWaves, IsBf16, kMaskAll, kKindWhole>(p, ring);
}

// Whole workgroups with split2 key-split ones (64 KiB of LDS: two per CU),
// for single-round grids of at most two workgroups per CU.
template <bool IsBf16>
__global__ __launch_bounds__(4 * 64, 2) void fused_attention_d64_wide_kernel(FusedAttentionParams p) {
    __shared__ __attribute__((aligned(16))) char ring[2 * (kKRing + kVRing)][kTileBytes];
    if ((int)blockIdx.x >= p.whole_units) {
        attention_body<4, IsBf16, false, kKindSplit2>(p, ring);
        return;
    }
    attention_body<4, IsBf16, false, kKindWhole>(p, ring);
}

// Mixed workgroups: 12 waves, one workgroup per CU; K and V rings for up to
// two heads (the key-part merge reuses the first of them).
template <bool IsBf16, int kKind = kKindMixed>
__global__ __launch_bounds__(12 * 64, 3) void fused_attention_d64_mixed_kernel(FusedAttentionParams p) {
    __shared__ __attribute__((aligned(16))) char ring[2 * (kKRing + kVRing)][kTileBytes];
    attention_body<12, IsBf16, false, kKind>(p, ring);
}

// ---- short key sequences (k_seq <= 128: the 77-token cross-attention, CLIP).
// One workgroup owns a chunk of consecutive 32-row query blocks of one
// (batch, head): it stages that head's whole K and V (at most 128 rows each)
// in LDS once, then each wave walks its blocks (w, w + kWaves, ...) computing
// the exact softmax in one pass (no running anchor, no rescaling):
// S^T = K Q^T for all key groups, one maximum, exp2, one sum, O^T = V^T P^T.
// A wave's block is one dependent chain (Q -> scores -> max -> exp2 -> PV ->
// output) of about 1.5 us, so throughput comes from residency: the kernel
// keeps ~110 VGPRs and 40 KiB of LDS per 4-wave workgroup (3 key groups) so
// that four waves share each SIMD. The next block's Q rows are transferred
// into the wave's LDS buffer as soon as the current block's output has left
// it for registers, overlapping that block's stores.
// Q is used as stored and the scale is folded into one fma per exp2
// argument. Keys past k_seq get a -inf accumulator seed in the last group;
// when that group holds at most 16 keys (kHalf, e.g. 77 = 64 + 13) its upper
// half is skipped in the exponentials and in PV.
// kGroups = ceil(k_seq / 32). Visibility per key: key < k_seq, key mask,
// causal (key <= query); a row with no visible key is 0 (reference
// src/cuda/flash_attention_sm80.cu:214-219).
// Workgroups per CU: LDS takes 16 + 8 groups KiB per workgroup; 96 keys
// without the half group need more than 128 VGPRs.
constexpr int short_keys_occupancy(int groups, bool half) { return groups == 4 || (groups == 3 && !half) ? 3 : 4; }

template <bool IsBf16, int kGroups, bool kHalf, bool kMasked, int kWaves, bool kNt>
__global__ __launch_bounds__(kWaves * 64, short_keys_occupancy(kGroups, kHalf)) void short_keys_attention_d64_kernel(FusedAttentionParams p) {
    constexpr int kRows = 32 * kGroups;
    constexpr int kLastN = kHalf ? 8 : 16;  // elements of the last group's scores in use (kHalf: keys 0-15 of it)
    constexpr int kPerWave = 8 * kGroups / kWaves;  // 1-KiB transfers per wave (4 kGroups for K, 4 kGroups for V)
    constexpr int kBlockBytes = 32 * kRowBytes;
    __shared__ __attribute__((aligned(16))) char kbuf[kRows * kRowBytes];
    __shared__ __attribute__((aligned(16))) char vbuf[kRows * kRowBytes];
    __shared__ __attribute__((aligned(16))) char qobuf[kWaves * kBlockBytes];  // per-wave Q / O staging

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hf = lane >> 5;
    const int col = lane & 31;
    // XCD-aware order: workgroup ids are dealt round robin over the 8 XCDs;
    // each XCD takes a contiguous range of chunks, so the chunks of one head
    // read its K/V through one L2.
    int task;
    {
        const int n = p.total_blocks, id = (int)blockIdx.x;
        const int xcd = id & 7, slot = id >> 3, per = n >> 3, extra = n & 7;
        task = xcd * per + (xcd < extra ? xcd : extra) + slot;
    }
    const int bh = task / p.short_chunks;
    const int blk_begin = (task % p.short_chunks) * p.short_chunk_blocks;
    const int blk_end = min(blk_begin + p.short_chunk_blocks, p.q_blocks);
    const int h = bh % p.heads;
    const int b = bh / p.heads;
    const int64_t elem = 2;
    const char* qbase = (const char*)p.q + ((int64_t)b * p.q_seq * p.q_row_stride + (int64_t)h * kHeadDim) * elem;
    const char* kbase = (const char*)p.k + ((int64_t)b * p.k_seq * p.k_row_stride + (int64_t)h * kHeadDim) * elem;
    const char* vbase = (const char*)p.v + ((int64_t)b * p.k_seq * p.v_row_stride + (int64_t)h * kHeadDim) * elem;
    char* obase = (char*)p.o + ((int64_t)b * p.q_seq * p.o_row_stride + (int64_t)h * kHeadDim) * elem;

    // K/V rows into LDS (swizzled 128-byte rows as in the tiled kernel); rows
    // past k_seq re-read the last key and are never visible.
#pragma unroll
    for (int j = 0; j < kPerWave; ++j) {
        const int n = wave * kPerWave + j;
        const bool is_v = n >= 4 * kGroups;
        const int r8 = is_v ? n - 4 * kGroups : n;
        const int row = 8 * r8 + (lane >> 3);
        const int key = min(row, p.k_seq - 1);
        const uint32_t stride = (uint32_t)((is_v ? p.v_row_stride : p.k_row_stride) * elem);
        const uint32_t off = __umul24((uint32_t)key, stride) + (uint32_t)(((lane & 7) ^ swz(row)) << 4);
        lds_dma16(is_v ? vbase : kbase, off, lds_addr((is_v ? vbuf : kbuf) + 8 * r8 * kRowBytes));
    }

    // Q rows move HBM -> LDS by DMA into the wave's block buffer (whole
    // 128-byte row segments, 8 lanes per row: coalesced), stored swizzled as
    // the K tiles; rows past q_seq re-read the last row and are never stored.
    // The output leaves through the same buffer. A wave's blocks are
    // blk_begin + wave + kWaves i, i < n_mine.
    char* const wbuf = qobuf + wave * kBlockBytes;
    const int first = blk_begin + wave;
    const int n_mine = first < blk_end ? (blk_end - first + kWaves - 1) / kWaves : 0;
    const uint32_t q_stride_b = (uint32_t)(p.q_row_stride * elem);
    auto issue_q = [&](int i) __attribute__((always_inline)) {
        const int blk = first + kWaves * i;
        const char* src = qbase + (int64_t)(32 * blk) * p.q_row_stride * elem;
        const int last = p.q_seq - 1 - 32 * blk;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = 8 * j + (lane >> 3);
            const uint32_t off = __umul24((uint32_t)min(row, last), q_stride_b) + (uint32_t)(((lane & 7) ^ swz(row)) << 4);
            lds_dma16(src, off, lds_addr(wbuf + 8 * j * kRowBytes));
        }
    };
    if (n_mine > 0) issue_q(0);
    // Visibility words of keys lane and lane + 64 (wave-uniform ballots):
    // key < k_seq and, with a key mask, mask != 0.
    uint64_t vis_word[2] = {~0ull, ~0ull};
    if constexpr (kMasked) {
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const int key = 64 * w + lane;
            const bool ok = key < p.k_seq && (p.key_mask == nullptr || p.key_mask[(int64_t)b * p.k_seq + key] != 0);
            vis_word[w] = __builtin_amdgcn_ballot_w64(ok);
        }
    }
    // K and V landed (block 0's Q, issued after them, may still fly)
    if (n_mine > 0) wait_vmem4();
    else wait_vmem_all();
    __syncthreads();

    const int k_swz = swz(col);
    const int g16 = lane & 15;
    const int tr_key = 4 * hf + (g16 >> 2), tr_qd = g16 & 3;
    int v_off[2][2];  // [dt][second read]
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
        const int chunk = 4 * dt + 2 * ((lane >> 4) & 1) + (tr_qd >> 1);
#pragma unroll
        for (int hi = 0; hi < 2; ++hi)
            v_off[dt][hi] = (tr_key + 8 * hi) * kRowBytes + ((chunk ^ swz(tr_key + 8 * hi)) << 4) + ((tr_qd & 1) << 3);
    }
    const float c = p.scale_log2;
    // Accumulator seed of the last key group: -inf for keys past k_seq, so
    // that the scores of those keys come out of the MFMA as -inf.
    f32x16 seed_last;
    {
        const int lim = p.k_seq - 32 * (kGroups - 1) - 4 * hf;
#pragma unroll
        for (int i = 0; i < 16; ++i) seed_last[i] = 8 * (i >> 2) + (i & 3) < lim ? 0.0f : -__builtin_inff();
    }

    for (int i = 0; i < n_mine; ++i) {
        const int blk = first + kWaves * i;
        const int my_query = 32 * blk + col;
        // Block i's transfer was issued before block i - 1's 4 stores (and
        // block 0's after K and V).
        if (i == 0) wait_vmem_all();
        else wait_vmem4();
        // Q^T operand: lane holds dims 16ks + 8hf .. +7 of query row col (used
        // as stored: the softmax scale is applied in fp32 to the scores, folded
        // into the exp2 argument).
        i16x8 qop[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qop[ks] = *(const lds_i16x8*)(wbuf + col * kRowBytes + (((2 * ks + hf) ^ k_swz) << 4));

        // S^T[key][q] = K Q^T (unscaled), key group g: lane holds keys
        // 32g + 8(i >> 2) + 4hf + (i & 3) of its query in s[g][i]. The groups'
        // chains are interleaved so the matrix pipe always has independent work.
        auto k_operand = [&](int g, int ks) __attribute__((always_inline)) {
            return *(const lds_i16x8*)(kbuf + (32 * g + col) * kRowBytes + (((2 * ks + hf) ^ k_swz) << 4));
        };
        f32x16 s[kGroups];
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            f32x16 z;
#pragma unroll
            for (int i = 0; i < 16; ++i) z[i] = 0.0f;
            s[g] = mfma32<IsBf16>(k_operand(g, 0), qop[0], g == kGroups - 1 ? seed_last : z);
        }
#pragma unroll
        for (int ks = 1; ks < 4; ++ks)
#pragma unroll
            for (int g = 0; g < kGroups; ++g) s[g] = mfma32<IsBf16>(k_operand(g, ks), qop[ks], s[g]);
        if constexpr (kMasked) {
            // element i of group g is key 32g + 4hf + kk, kk = 8(i >> 2) + (i & 3)
            const int causal_lim = p.causal ? my_query - 4 * hf : 0x7FFFFFFF;
#pragma unroll
            for (int g = 0; g < kGroups; ++g) {
                const uint32_t lane_vis = (uint32_t)(vis_word[g >> 1] >> (32 * (g & 1) + 4 * hf));
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int kk = 8 * (i >> 2) + (i & 3);
                    const bool ok = ((lane_vis >> kk) & 1u) && 32 * g + kk <= causal_lim;
                    s[g][i] = ok ? s[g][i] : -__builtin_inff();
                }
            }
        }
        float mx = -__builtin_inff();
#pragma unroll
        for (int g = 0; g < kGroups; ++g)
#pragma unroll
            for (int i = 0; i < (g == kGroups - 1 ? kLastN : 16); ++i) mx = fmaxf(mx, s[g][i]);
        mx = xhalf_max(mx);
        // p = 2^(c s - c max), c = scale log2(e); no visible key: every p is 0
        const float neg_cm = mx == -__builtin_inff() ? 0.0f : -c * mx;

        // O^T = V^T P^T, one accumulator per d tile; V^T operands by
        // transposing LDS reads (addresses as in the tiled kernel).
        f32x16 out[2];
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) out[dt][i] = 0.0f;
        float l = 0.0f;
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            // kHalf: keys 16-31 of the last group are all past k_seq; their
            // probabilities and PV step are skipped.
            constexpr int kSteps = 2;
            const int n_ss = (kHalf && g == kGroups - 1) ? 1 : kSteps;
            float e[16];
#pragma unroll
            for (int i = 0; i < 16; ++i)
                e[i] = i < 8 * n_ss ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[g][i], c, neg_cm)) : 0.0f;
            l += n_ss == 2 ? sum8(e) + sum8(e + 8) : sum8(e);
#pragma unroll
            for (int ss = 0; ss < n_ss; ++ss) {
                const i16x8 pop = __builtin_bit_cast(
                    i16x8, u32x4{pack2<IsBf16>(e[8 * ss], e[8 * ss + 1]), pack2<IsBf16>(e[8 * ss + 2], e[8 * ss + 3]),
                                 pack2<IsBf16>(e[8 * ss + 4], e[8 * ss + 5]), pack2<IsBf16>(e[8 * ss + 6], e[8 * ss + 7])});
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) {
                    const char* base = vbuf + (32 * g + 16 * ss) * kRowBytes;
                    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + v_off[dt][0]));
                    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + v_off[dt][1]));
                    out[dt] = mfma32<IsBf16>(i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}, pop, out[dt]);
                }
            }
        }
        const float l_tot = xhalf_sum(l);
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        // O rows through the staging buffer (its Q rows are consumed): lane
        // holds dims 32dt + 8u + 4hf .. +3 of row col, i.e. half hf of chunk
        // 4dt + u; then whole row segments to HBM.
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t w0 = pack2<IsBf16>(out[dt][4 * u] * inv, out[dt][4 * u + 1] * inv);
                const uint32_t w1 = pack2<IsBf16>(out[dt][4 * u + 2] * inv, out[dt][4 * u + 3] * inv);
                *(lds_u32x2*)(wbuf + col * kRowBytes + (((4 * dt + u) ^ k_swz) << 4) + 8 * hf) = u32x2{w0, w1};
            }
        u32x4 orow[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = 8 * j + (lane >> 3);
            orow[j] = *(const lds_u32x4*)(wbuf + row * kRowBytes + (((lane & 7) ^ swz(row)) << 4));
        }
        // the buffer is free once its output rows are in registers
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (i + 1 < n_mine) issue_q(i + 1);
        // Whole 128-byte row segments per 8 lanes; non-temporal for large
        // outputs (measured [4,10,3840,77] 11.4 -> 9.8 us).
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = 8 * j + (lane >> 3);
            if (32 * blk + row < p.q_seq)
                store_out<kNt>(orow[j], (u32x4*)(obase + (int64_t)(32 * blk + row) * p.o_row_stride * elem + 16 * (lane & 7)));
        }
    }
}

template <bool IsBf16, bool kMasked>
hipError_t launch_short_keys(FusedAttentionParams p, int compute_units, hipStream_t stream) {
    // Chunks: about as many workgroups as fit on the device at once (four per
    // CU, or three), each a run of consecutive 32-row
    // blocks of one head, a whole number of blocks per wave. Measured on the
    // 77-token shapes against 1-3 per CU and fixed chunks of 4-12 blocks:
    // [2,10,4096] 8.4 -> 7.2 us, [4,20,960] 8.3 -> 7.0 us at two per CU.
    constexpr int kWaves = 4;
    const int groups = (p.k_seq + 31) / 32;
    // kHalf when the last 32-key group holds at most 16 keys
    const bool half = (p.k_seq - 1) % 32 < 16;
    const int per_cu = short_keys_occupancy(groups, half);
    p.q_blocks = (p.q_seq + 31) / 32;
    const int64_t heads_total = (int64_t)p.heads * p.batch;
    const int64_t all_blocks = (int64_t)p.q_blocks * heads_total;
    const int64_t target_wgs = (int64_t)(compute_units > 0 ? compute_units : 256) * per_cu;
    int64_t chunk = (all_blocks + target_wgs - 1) / target_wgs;
    chunk = (chunk + kWaves - 1) / kWaves * kWaves;  // whole rounds of the workgroup's waves
    chunk = chunk > p.q_blocks ? p.q_blocks : chunk;
    p.short_chunk_blocks = (int32_t)chunk;
    p.short_chunks = (int32_t)((p.q_blocks + chunk - 1) / chunk);
    const int64_t grid_size = heads_total * p.short_chunks;
    if (grid_size > INT32_MAX) return hipErrorInvalidValue;
    p.total_blocks = (int32_t)grid_size;
    const dim3 grid(p.total_blocks), block(64 * kWaves);
    // non-temporal output stores for large outputs
    const bool nt = (int64_t)p.batch * p.q_seq * p.heads * kHeadDim * 2 >= kStreamOutBytes;
#define SDXL_SK_LAUNCH(G, H)                                                                                        \
    do {                                                                                                            \
        if (nt) hipLaunchKernelGGL((short_keys_attention_d64_kernel<IsBf16, G, H, kMasked, kWaves, true>), grid, block, 0, stream, p); \
        else hipLaunchKernelGGL((short_keys_attention_d64_kernel<IsBf16, G, H, kMasked, kWaves, false>), grid, block, 0, stream, p); \
    } while (0)
    switch (groups) {
    case 1: if (half) SDXL_SK_LAUNCH(1, true); else SDXL_SK_LAUNCH(1, false); break;
    case 2: if (half) SDXL_SK_LAUNCH(2, true); else SDXL_SK_LAUNCH(2, false); break;
    case 3: if (half) SDXL_SK_LAUNCH(3, true); else SDXL_SK_LAUNCH(3, false); break;
    default: if (half) SDXL_SK_LAUNCH(4, true); else SDXL_SK_LAUNCH(4, false); break;
    }
#undef SDXL_SK_LAUNCH
    return hipGetLastError();
}


// ---- short key sequences, 16-row blocks (v_mfma_f32_16x16x32). The same
// algorithm as short_keys_attention_d64_kernel with half the query rows per
// wave block: a block's dependent chain (scores, maximum, exponentials, PV,
// output) is about half as long and there are twice as many blocks, for
// calls whose 32-row blocks would leave most SIMDs without a wave (CLIP's
// 77-token self-attention: 72 blocks).
// Per block and 16-key tile t (kTiles = ceil(k_seq / 16)): S^T tile = K_t Q^T
// (two MFMAs over d = 64); lane l holds query l & 15 and keys
// 16t + 4(l >> 4) + i, i < 4, in s[t][i]. O^T = V^T P^T runs over pairs of
// tiles (32 keys per MFMA; the probability operand of lane group g is keys
// 4g..4g+3 of the first tile and of the second, so the V^T operand is two
// transposing LDS reads of those key rows); an odd last tile takes a step
// whose second half has zero probabilities. Keys past k_seq get a -inf
// accumulator seed in the last tile. Visibility per key: key < k_seq, key mask, causal (key <= query);
// a row with no visible key is 0 (reference
// src/cuda/flash_attention_sm80.cu:214-219).
template <bool IsBf16>
__device__ __forceinline__ f32x4 mfma16x32(i16x8 a, i16x8 b, f32x4 c) {
    if constexpr (IsBf16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Workgroups per CU: LDS is 4 kTiles + 8 KiB per workgroup.
constexpr int short16_occupancy(int tiles) { return tiles <= 5 ? 5 : 4; }

template <bool IsBf16, int kTiles, bool kMasked, int kWaves, bool kNt>
__global__ __launch_bounds__(kWaves * 64, short16_occupancy(kTiles)) void short_keys16_attention_d64_kernel(FusedAttentionParams p) {
    constexpr int kRows = 16 * kTiles;
    constexpr int kPerWave = 4 * kTiles / kWaves;  // 1-KiB K/V transfers per wave
    constexpr int kBlockBytes = 16 * kRowBytes;
    __shared__ __attribute__((aligned(16))) char kbuf[kRows * kRowBytes];
    __shared__ __attribute__((aligned(16))) char vbuf[kRows * kRowBytes];
    __shared__ __attribute__((aligned(16))) char qobuf[kWaves * kBlockBytes];  // per-wave Q / O staging

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4;   // lane group: keys 4g..4g+3 of each tile
    const int r16 = lane & 15; // query row of the block
    int task;
    {
        const int n = p.total_blocks, id = (int)blockIdx.x;
        const int xcd = id & 7, slot = id >> 3, per = n >> 3, extra = n & 7;
        task = xcd * per + (xcd < extra ? xcd : extra) + slot;
    }
    const int bh = task / p.short_chunks;
    const int blk_begin = (task % p.short_chunks) * p.short_chunk_blocks;
    const int blk_end = min(blk_begin + p.short_chunk_blocks, p.q_blocks);
    const int h = bh % p.heads;
    const int b = bh / p.heads;
    const int64_t elem = 2;
    const char* qbase = (const char*)p.q + ((int64_t)b * p.q_seq * p.q_row_stride + (int64_t)h * kHeadDim) * elem;
    const char* kbase = (const char*)p.k + ((int64_t)b * p.k_seq * p.k_row_stride + (int64_t)h * kHeadDim) * elem;
    const char* vbase = (const char*)p.v + ((int64_t)b * p.k_seq * p.v_row_stride + (int64_t)h * kHeadDim) * elem;
    char* obase = (char*)p.o + ((int64_t)b * p.q_seq * p.o_row_stride + (int64_t)h * kHeadDim) * elem;

    // K/V rows into LDS (swizzled 128-byte rows); rows past k_seq re-read the
    // last key and are never visible.
#pragma unroll
    for (int j = 0; j < kPerWave; ++j) {
        const int n = wave * kPerWave + j;
        const bool is_v = n >= 2 * kTiles;
        const int r8 = is_v ? n - 2 * kTiles : n;
        const int row = 8 * r8 + (lane >> 3);
        const int key = min(row, p.k_seq - 1);
        const uint32_t stride = (uint32_t)((is_v ? p.v_row_stride : p.k_row_stride) * elem);
        const uint32_t off = __umul24((uint32_t)key, stride) + (uint32_t)(((lane & 7) ^ swz(row)) << 4);
        lds_dma16(is_v ? vbase : kbase, off, lds_addr((is_v ? vbuf : kbuf) + 8 * r8 * kRowBytes));
    }

    // Q rows by DMA into the wave's staging buffer (two 1-KiB transfers per
    // block); rows past q_seq re-read the last row and are never stored. A
    // wave's blocks are blk_begin + wave + kWaves i, i < n_mine.
    char* const wbuf = qobuf + wave * kBlockBytes;
    const int first = blk_begin + wave;
    const int n_mine = first < blk_end ? (blk_end - first + kWaves - 1) / kWaves : 0;
    const uint32_t q_stride_b = (uint32_t)(p.q_row_stride * elem);
    auto issue_q = [&](int i) __attribute__((always_inline)) {
        const int blk = first + kWaves * i;
        const char* src = qbase + (int64_t)(16 * blk) * p.q_row_stride * elem;
        const int last = p.q_seq - 1 - 16 * blk;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int row = 8 * j + (lane >> 3);
            const uint32_t off = __umul24((uint32_t)min(row, last), q_stride_b) + (uint32_t)(((lane & 7) ^ swz(row)) << 4);
            lds_dma16(src, off, lds_addr(wbuf + 8 * j * kRowBytes));
        }
    };
    if (n_mine > 0) issue_q(0);
    uint64_t vis_word[2] = {~0ull, ~0ull};
    if constexpr (kMasked) {
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const int key = 64 * w + lane;
            const bool ok = key < p.k_seq && (p.key_mask == nullptr || p.key_mask[(int64_t)b * p.k_seq + key] != 0);
            vis_word[w] = __builtin_amdgcn_ballot_w64(ok);
        }
    }
    // K and V landed (block 0's two Q transfers, issued after them, may fly)
    if (n_mine > 0) wait_vmem2();
    else wait_vmem_all();
    __syncthreads();

    const int k_swz = swz(r16);
    int v_off[4];  // transposing V reads: key row 4g + (r16 >> 2), dims 16dt + 4(r16 & 3)
    {
        const int row = 4 * g + (r16 >> 2);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
            v_off[dt] = row * kRowBytes + (((2 * dt + ((r16 & 3) >> 1)) ^ swz(row)) << 4) + ((r16 & 1) << 3);
    }
    const float c = p.scale_log2;
    f32x4 seed_last;
#pragma unroll
    for (int i = 0; i < 4; ++i) seed_last[i] = 16 * (kTiles - 1) + 4 * g + i < p.k_seq ? 0.0f : -__builtin_inff();

    for (int i = 0; i < n_mine; ++i) {
        const int blk = first + kWaves * i;
        const int my_query = 16 * blk + r16;
        // Block i's transfers were issued before block i - 1's 2 stores.
        if (i == 0) wait_vmem_all();
        else wait_vmem2();
        i16x8 qop[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) qop[ks] = *(const lds_i16x8*)(wbuf + r16 * kRowBytes + (((4 * ks + g) ^ k_swz) << 4));
        auto k_operand = [&](int t, int ks) __attribute__((always_inline)) {
            return *(const lds_i16x8*)(kbuf + (16 * t + r16) * kRowBytes + (((4 * ks + g) ^ k_swz) << 4));
        };
        f32x4 s[kTiles];
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
            s[t] = mfma16x32<IsBf16>(k_operand(t, 0), qop[0], t == kTiles - 1 ? seed_last : z);
        }
#pragma unroll
        for (int t = 0; t < kTiles; ++t) s[t] = mfma16x32<IsBf16>(k_operand(t, 1), qop[1], s[t]);
        if constexpr (kMasked) {
            const int causal_lim = p.causal ? my_query - 4 * g : 0x7FFFFFFF;
#pragma unroll
            for (int t = 0; t < kTiles; ++t) {
                const uint32_t lane_vis = (uint32_t)(vis_word[t >> 2] >> (16 * (t & 3) + 4 * g));
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool ok = ((lane_vis >> e) & 1u) && 16 * t + e <= causal_lim;
                    s[t][e] = ok ? s[t][e] : -__builtin_inff();
                }
            }
        }
        float mx = -__builtin_inff();
#pragma unroll
        for (int t = 0; t < kTiles; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) mx = fmaxf(mx, s[t][e]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = xhalf_max(mx);
        const float neg_cm = mx == -__builtin_inff() ? 0.0f : -c * mx;

        f32x4 out[4];
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) out[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        float l = 0.0f;
        uint32_t pk[kTiles][2];
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            float e[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) e[u] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][u], c, neg_cm));
            l += (e[0] + e[1]) + (e[2] + e[3]);
            pk[t][0] = pack2<IsBf16>(e[0], e[1]);
            pk[t][1] = pack2<IsBf16>(e[2], e[3]);
        }
#pragma unroll
        for (int ss = 0; ss < kTiles / 2; ++ss) {
            const i16x8 pop = __builtin_bit_cast(i16x8, u32x4{pk[2 * ss][0], pk[2 * ss][1], pk[2 * ss + 1][0], pk[2 * ss + 1][1]});
            const char* base = vbuf + 32 * ss * kRowBytes;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + v_off[dt]));
                const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + 16 * kRowBytes + v_off[dt]));
                out[dt] = mfma16x32<IsBf16>(i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}, pop, out[dt]);
            }
        }
        if constexpr (kTiles % 2 == 1) {
            // odd last tile: a 32-key step whose second half has zero
            // probabilities (the V operand repeats the tile's rows, finite)
            const i16x8 pop = __builtin_bit_cast(i16x8, u32x4{pk[kTiles - 1][0], pk[kTiles - 1][1], 0u, 0u});
            const char* base = vbuf + 16 * (kTiles - 1) * kRowBytes;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + v_off[dt]));
                out[dt] = mfma16x32<IsBf16>(i16x8{lo[0], lo[1], lo[2], lo[3], lo[0], lo[1], lo[2], lo[3]}, pop, out[dt]);
            }
        }
        l += __shfl_xor(l, 16, 64);
        const float l_tot = xhalf_sum(l);
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        // O rows through the staging buffer: lane holds dims 16dt + 4g .. +3
        // of row r16 (half g & 1 of chunk 2dt + (g >> 1)).
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const uint32_t w0 = pack2<IsBf16>(out[dt][0] * inv, out[dt][1] * inv);
            const uint32_t w1 = pack2<IsBf16>(out[dt][2] * inv, out[dt][3] * inv);
            *(lds_u32x2*)(wbuf + r16 * kRowBytes + (((2 * dt + (g >> 1)) ^ k_swz) << 4) + 8 * (g & 1)) = u32x2{w0, w1};
        }
        u32x4 orow[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int row = 8 * j + (lane >> 3);
            orow[j] = *(const lds_u32x4*)(wbuf + row * kRowBytes + (((lane & 7) ^ swz(row)) << 4));
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (i + 1 < n_mine) issue_q(i + 1);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int row = 8 * j + (lane >> 3);
            if (16 * blk + row < p.q_seq)
                store_out<kNt>(orow[j], (u32x4*)(obase + (int64_t)(16 * blk + row) * p.o_row_stride * elem + 16 * (lane & 7)));
        }
    }
}

template <bool IsBf16, bool kMasked>
hipError_t launch_short_keys16(FusedAttentionParams p, int compute_units, hipStream_t stream) {
    constexpr int kWaves = 4;
    const int tiles = (p.k_seq + 15) / 16;
    const int per_cu = short16_occupancy(tiles);
    p.q_blocks = (p.q_seq + 15) / 16;
    const int64_t heads_total = (int64_t)p.heads * p.batch;
    const int64_t all_blocks = (int64_t)p.q_blocks * heads_total;
    const int64_t target_wgs = (int64_t)(compute_units > 0 ? compute_units : 256) * per_cu;
    int64_t chunk = (all_blocks + target_wgs - 1) / target_wgs;
    chunk = (chunk + kWaves - 1) / kWaves * kWaves;
    chunk = chunk > p.q_blocks ? p.q_blocks : chunk;
    p.short_chunk_blocks = (int32_t)chunk;
    p.short_chunks = (int32_t)((p.q_blocks + chunk - 1) / chunk);
    const int64_t grid_size = heads_total * p.short_chunks;
    if (grid_size > INT32_MAX) return hipErrorInvalidValue;
    p.total_blocks = (int32_t)grid_size;
    const dim3 grid(p.total_blocks), block(64 * kWaves);
    const bool nt = (int64_t)p.batch * p.q_seq * p.heads * kHeadDim * 2 >= kStreamOutBytes;
#define SDXL_SK16_LAUNCH(T)                                                                                          \
    do {                                                                                                             \
        if (nt) hipLaunchKernelGGL((short_keys16_attention_d64_kernel<IsBf16, T, kMasked, kWaves, true>), grid, block, 0, stream, p); \
        else hipLaunchKernelGGL((short_keys16_attention_d64_kernel<IsBf16, T, kMasked, kWaves, false>), grid, block, 0, stream, p); \
    } while (0)
    switch (tiles) {
    case 1: SDXL_SK16_LAUNCH(1); break;
    case 2: SDXL_SK16_LAUNCH(2); break;
    case 3: SDXL_SK16_LAUNCH(3); break;
    case 4: SDXL_SK16_LAUNCH(4); break;
    case 5: SDXL_SK16_LAUNCH(5); break;
    case 6: SDXL_SK16_LAUNCH(6); break;
    case 7: SDXL_SK16_LAUNCH(7); break;
    default: SDXL_SK16_LAUNCH(8); break;
    }
#undef SDXL_SK16_LAUNCH
    return hipGetLastError();
}

}  // namespace

int fused_attention_block_queries() { return 32 * kFusedWaves; }

bool short_keys_16_row_blocks(int64_t blocks32, int compute_units) {
    return compute_units > 0 && 2 * blocks32 <= 3 * (int64_t)compute_units;
}

hipError_t launch_fused_attention_d64(const FusedAttentionParams& params_in, bool is_bf16, int compute_units,
                                      hipStream_t stream) {
    FusedAttentionParams p = params_in;
    constexpr int kBlockQueries = 32 * kFusedWaves;
    p.q_blocks = (p.q_seq + kBlockQueries - 1) / kBlockQueries;
    p.total_blocks = p.q_blocks * p.heads * p.batch;
    if (p.total_blocks == 0) return hipSuccess;
    if (p.k_seq > 0 && p.k_seq <= kShortKeysMax) {
        const bool masked = p.causal || p.key_mask != nullptr;
        // Grids of at most 1.5 32-row blocks per CU run 16-row blocks (twice
        // the waves in flight): CLIP's [2,12,77,77] 4.65 -> 3.56 us,
        // [2,20,256,77] 3.65 -> 3.27 us; from [2,20,512,77] (2.5 per CU) the
        // 32-row kernel is as fast or faster (3.86 vs 3.97 us).
        if (short_keys_16_row_blocks((int64_t)((p.q_seq + 31) / 32) * p.heads * p.batch, compute_units)) {
            if (is_bf16) return masked ? launch_short_keys16<true, true>(p, compute_units, stream) : launch_short_keys16<true, false>(p, compute_units, stream);
            return masked ? launch_short_keys16<false, true>(p, compute_units, stream) : launch_short_keys16<false, false>(p, compute_units, stream);
        }
        if (is_bf16) return masked ? launch_short_keys<true, true>(p, compute_units, stream) : launch_short_keys<true, false>(p, compute_units, stream);
        return masked ? launch_short_keys<false, true>(p, compute_units, stream) : launch_short_keys<false, false>(p, compute_units, stream);
    }
    // Work split. Three workgroups are resident per CU (occupancy 3, one wave
    // per SIMD each), S = 3 CUs slots. With U 128-row units, the rounds that
    // fill every slot run whole workgroups; the remaining R = U mod S units are
    // re-cut so that the last round is balanced: part of them becomes
    // key-split workgroups (64 rows, each wave half the keys: half the work of
    // a whole one), see below.
    // The hardware deals ids x, x + CUs, x + 2 CUs to one CU, so with whole
    // workgroups first every CU of the last round gets the same mix.
    // Non-causal, unmasked calls with q_seq % 128 == 0 and k_seq % 64 == 0.
    p.whole_units = p.total_blocks;
    p.split_units = 0;
    bool wide = false;  // whole + split2 workgroups on the 64-KiB kernel
    const int64_t slots = (int64_t)compute_units * 3;
    const int64_t units = p.total_blocks;
    if (compute_units > 0 && !p.causal && p.key_mask == nullptr && p.q_seq % 128 == 0 && p.k_seq % 64 == 0 &&
        p.k_seq > 0 && units % slots != 0) {
        const int64_t full = units - units % slots, rem = units % slots;
        // Whole workgroups do more per transfer and per barrier than two
        // key-split ones (two groups per tile step, one staging per 4 blocks):
        // with q = rem / CUs >= 1, q whole workgroups per CU and the other
        // rem - q CUs units as key-split ones keep the same most-loaded CU
        // (q + 1/2 blocks per SIMD) as the all-split cut, while three
        // workgroups per CU suffice (c1 [2,20,1024,1024] 18.5 -> 17.4 us,
        // [2,10,2048,2048] 32.4 -> 30.5 us; below one unit per CU, whole
        // workgroups alone measured slower).
        const int64_t q = compute_units > 0 ? rem / compute_units : 0, r = rem - q * compute_units;
        if (q >= 1 && q + (2 * r + compute_units - 1) / compute_units <= 3) {
            p.whole_units = (int32_t)(full + q * compute_units);
            p.split_units = (int32_t)(2 * r);
            // one round of at most two workgroups per CU: key-split workgroups
            // with 64 keys of each half per stage
            wide = full == 0 && q == 1 && 2 * r <= compute_units && p.k_seq % 128 == 0;
        } else if (2 * rem >= slots) {
            p.whole_units = (int32_t)(full + 2 * rem - slots);
            p.split_units = (int32_t)(2 * slots - 2 * rem);
        } else {
            p.whole_units = (int32_t)full;
            p.split_units = (int32_t)(2 * rem);
            // one round of at most two key-split workgroups per CU: the 64-KiB
            // kind too ([1,10,1024,1024] 11.5 -> 10.9 us)
            wide = full == 0 && rem <= compute_units && p.k_seq % 128 == 0;
        }
    }
    const bool mask_all = p.causal || p.key_mask != nullptr;
    // Mixed 12-wave workgroups (10 row blocks each, one per CU at a time) when
    // their rounds carry at most 10% more blocks per CU than an even share:
    // per SIMD 2.5 blocks with one K/V staging per 10 blocks. Measured against
    // the 4-wave grids in one process: [2,10,4096] 92.5 vs 94.0 us (exact
    // fit), [4,20,960] 26.5 vs 29.5 us (240 of 256 CUs busy), [4,10,3840]
    // 157.9 vs 169.9 us (two rounds, 480 workgroups).
    if (compute_units > 0 && !mask_all && p.k_seq % 64 == 0 && p.k_seq > 0) {
        const int64_t qb32 = (p.q_seq + 31) / 32;
        const int64_t total = qb32 * p.heads * p.batch;
        const int64_t wgs = (total + kMixedBlocks - 1) / kMixedBlocks;
        const int64_t rounds = (wgs + compute_units - 1) / compute_units;
        if (qb32 >= kMixedBlocks && wgs <= INT32_MAX &&
            (double)(rounds * kMixedBlocks) <= 1.10 * (double)total / (double)compute_units) {
            p.q_blocks = (int32_t)qb32;
            p.mixed_total = (int32_t)total;
            p.mixed_wgs = (int32_t)wgs;
            // workgroups span two heads unless every head holds a whole number of
            // them (the two-head kind takes K and V of one row stride: the half
            // waves' V transfers reuse their K offsets)
            const bool spans = qb32 % kMixedBlocks != 0 && p.heads * p.batch > 1 && p.k_row_stride == p.v_row_stride;
            const dim3 g(p.mixed_wgs), b(768);
            if (spans) {
                if (is_bf16) hipLaunchKernelGGL((fused_attention_d64_mixed_kernel<true, kKindMixed2>), g, b, 0, stream, p);
                else hipLaunchKernelGGL((fused_attention_d64_mixed_kernel<false, kKindMixed2>), g, b, 0, stream, p);
            } else {
                if (is_bf16) hipLaunchKernelGGL((fused_attention_d64_mixed_kernel<true>), g, b, 0, stream, p);
                else hipLaunchKernelGGL((fused_attention_d64_mixed_kernel<false>), g, b, 0, stream, p);
            }
            return hipGetLastError();
        }
    }
    const dim3 grid(p.whole_units + p.split_units), block(64 * kFusedWaves);
    if (wide) {
        if (is_bf16) hipLaunchKernelGGL((fused_attention_d64_wide_kernel<true>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((fused_attention_d64_wide_kernel<false>), grid, block, 0, stream, p);
        return hipGetLastError();
    }
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

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
//
// FP8 activations (E4M3 codes with per-row scales, from the E4M3 LayerNorm)
// times E4M3 weights run on the gfx950 fp8 matrix cores
// (v_mfma_f32_32x32x64_f8f6f4, twice the fp16 rate): both operands stay as
// codes in 64-byte LDS rows and one MFMA covers a whole 64-deep K stage; the
// epilogue applies a_scale[m] * w_scale[n] in fp32. No reference counterpart
// (its FP8 path is weight-only); an optional mode of the QKV projection.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "sublayer_device.hpp"
#include "sublayer_kernels.hpp"

namespace sdxl_hip {
namespace {

// One workgroup = 4 waves in a 2 x 2 arrangement = a (64 kTM) x 128 output
// tile (kTM = 1, 2 or 4); each wave computes (32 kTM) x 64 as kTM x 2 MFMA tiles. kRing LDS
// stages of kBK = 64 columns of K: stage s + kRing - 1 is requested while
// stage s is consumed (prefetch distance kRing - 1 stages), so that a stage's
// transfers have MFMA work to land behind. E4M3 weights stay as codes in LDS
// (64-byte rows, chunk swizzle (row >> 2) & 3) and are decoded when the
// operand is read; fp16 weights use the A-operand layout. kAFp8 (with kWFp8):
// E4M3 activations in 64-byte rows, fp8 MFMA.
// kKvG > 0: the query projection of the cross-attention (64 x 128 tiles, so
// each wave's 32 x 64 block is one 32-row query block of one head) fused
// with the attention over kKvG 32-key groups of context (kKvHalf: the last
// group holds at most 16 keys); see the epilogue.
// kProd: the workgroup has kWM x kWN more waves that only issue the stage
// transfers (wave w + kWM kWN issues compute wave w's), so the compute waves
// never stall on a transfer's issue and the producers' issue overlaps the
// MFMA work of their SIMD.
template <bool kWFp8, bool kAFp8, int kTM, int kRing, int kOcc, bool kNt, int kWM = 2, int kKvG = 0, bool kKvHalf = false,
          int kWN = 2, bool kProd = false>
__global__ __launch_bounds__(64 * kWM * kWN * (kProd ? 2 : 1), kOcc) void linear_kernel(LinearParams p) {
    static_assert(!kAFp8 || kWFp8, "E4M3 activations need E4M3 weights");
    static_assert(!kProd || kKvG == 0, "producer waves: plain projections only");
    static_assert(kKvG == 0 || kWN == 2, "the cross-attention form uses 128-column tiles");
    constexpr int kBMt = 64 * kTM;
    constexpr int kBNt = 64 * kWN;             // tile columns
    constexpr int kWaves = kWM * kWN;          // kWM waves along M x kWN along N
    constexpr int kTMw = kBMt / (32 * kWM);    // 32-row MFMA tiles per wave
    static_assert(kTMw >= 1 && kTMw * 32 * kWM == kBMt, "wave tiling");
    constexpr int kWRowBytes = kWFp8 ? 64 : kRowBytes;
    constexpr int kARowBytes = kAFp8 ? 64 : kRowBytes;
    constexpr int kATileBytes = kBMt * kARowBytes;
    constexpr int kWTileBytes = kBNt * kWRowBytes;
    constexpr int kAXfers = kATileBytes / 1024 / kWaves;  // 1-KiB A transfers per wave and stage
    constexpr int kWXfers = kWTileBytes / 1024 / kWaves;
    static_assert(kAXfers * kWaves * 1024 == kATileBytes && kWXfers * kWaves * 1024 == kWTileBytes,
                  "every 1-KiB transfer of a stage has a wave");
    constexpr int kLoadsPerStage = kAXfers + kWXfers;
    // Stage st: A tile at smem[st], W tile right after it. The epilogue
    // reuses the array.
    // (at least the epilogue's 4 x 32 x 256 bytes of staging)
    constexpr int kStageBytes = kATileBytes + kWTileBytes;
    constexpr int kSmemStages = kRing * kStageBytes >= kWaves * 32 * 256 ? kRing : (kWaves * 32 * 256 + kStageBytes - 1) / kStageBytes;
    __shared__ __attribute__((aligned(16))) char smem[kSmemStages][kStageBytes];
    // V rows of the tile's two heads (cross-attention form), swizzled 128-byte
    // rows: every row a key group reads (kKvHalf: 16 of the last group's 32)
    constexpr int kVRows = kKvG > 0 ? 32 * (kKvG - 1) + (kKvHalf ? 16 : 32) : 1;
    __shared__ __attribute__((aligned(16))) char vbuf[2 * kVRows * kRowBytes];

    const int lane = threadIdx.x & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool producer = kProd && wave_id >= kWaves;
    const int wave = kProd ? wave_id % kWaves : wave_id;  // compute wave (or the one a producer serves)
    const int hf = lane >> 5, col = lane & 31;

    // Tasks in groups of group_m m blocks (within a group m varies fastest,
    // then n), each XCD taking one contiguous range of tasks: an XCD's
    // resident workgroups cover a group_m x (range / group_m) rectangle of
    // output tiles, whose A rows and W rows together fit its L2 better than
    // a row of the output.
    int task;
    {
        const int n = p.m_blocks * p.n_blocks;
        const int id = blockIdx.x;
        const int xcd = id & 7, slot = id >> 3;
        const int per = n >> 3, extra = n & 7;
        task = xcd * per + (xcd < extra ? xcd : extra) + slot;
    }
    int mb, nb;
    {
        const int in_group = p.group_m * p.n_blocks;
        const int first_m = (task / in_group) * p.group_m;
        const int rows = min(p.m_blocks - first_m, p.group_m);
        const int r = task % in_group;
        mb = first_m + r % rows;
        nb = r / rows;
    }
    const int m0 = mb * kBMt, n0 = nb * kBNt;
    const int n_stages = p.k / kBK;

    const int64_t lda_b = kAFp8 ? p.lda : p.lda * 2;
    const char* abase = (const char*)p.a + (int64_t)m0 * lda_b;
    const int64_t ldw_b = kWFp8 ? p.ldw : p.ldw * 2;
    const char* wbase = (const char*)p.w + (int64_t)n0 * ldw_b;
    const int a_rows = p.m - 1 - m0, w_rows = p.n - 1 - n0;  // last valid tile row

    // Epilogue column constants, loaded now so that their latency hides under
    // the main loop: lane l finishes columns 4(l%16) .. +3 of its wave block.
    const int wm = wave % kWM, wn = wave / kWM;
    const int ec = lane & 15;
    const int en = n0 + wn * 64 + 4 * ec;
    const bool en_ok = en < p.n;
    float4 e_scale = {1.0f, 1.0f, 1.0f, 1.0f}, e_bias = {0.0f, 0.0f, 0.0f, 0.0f};
    if (en_ok && p.w_scale != nullptr) e_scale = *(const float4*)(p.w_scale + en);
    if (en_ok && p.bias != nullptr) {
        const f16x4 bb = *(const f16x4*)((const _Float16*)p.bias + en);
        e_bias = float4{(float)bb[0], (float)bb[1], (float)bb[2], (float)bb[3]};
    }

    // ---- stage transfers (rows past the end re-read the last row).
    // 128-byte rows (A, fp16 W): transfer n covers rows 8n .. 8n+7; lane l
    // takes row 8n + l/8 and global chunk (l%8) ^ swz(row), its slot's chunk.
    auto dma_rows128 = [&](const char* gbase, int64_t ld_b, int last, int kbyte, char* buf, int n)
                           __attribute__((always_inline)) {
        const int row = 8 * n + (lane >> 3);
        const uint32_t off = (uint32_t)(min(row, last) * ld_b) + (uint32_t)(((lane & 7) ^ swz(row)) << 4);
        lds_dma16(gbase + kbyte, off, lds_addr(buf + 8 * n * kRowBytes));
    };
    // 64-byte rows (E4M3 W): transfer n covers rows 16n .. 16n+15; lane l takes
    // row 16n + l/4 and global chunk (l%4) ^ ((row >> 2) & 3).
    auto dma_rows64 = [&](const char* gbase, int64_t ld_b, int last, int kbyte, char* buf, int n)
                          __attribute__((always_inline)) {
        const int row = 16 * n + (lane >> 2);
        const uint32_t off = (uint32_t)(min(row, last) * ld_b) + (uint32_t)(((lane & 3) ^ ((row >> 2) & 3)) << 4);
        lds_dma16(gbase + kbyte, off, lds_addr(buf + 16 * n * 64));
    };
    auto issue_stage = [&](int st) __attribute__((always_inline)) {
        char* ab = smem[st % kRing];
        char* wb = smem[st % kRing] + kATileBytes;
        if constexpr (kAFp8) {
#pragma unroll
            for (int j = 0; j < kAXfers; ++j) dma_rows64(abase, lda_b, a_rows, st * kBK, ab, wave * kAXfers + j);
        } else {
#pragma unroll
            for (int j = 0; j < kAXfers; ++j) dma_rows128(abase, lda_b, a_rows, st * kBK * 2, ab, wave * kAXfers + j);
        }
        if constexpr (kWFp8) {
#pragma unroll
            for (int j = 0; j < kWXfers; ++j) dma_rows64(wbase, ldw_b, w_rows, st * kBK, wb, wave * kWXfers + j);
        } else {
#pragma unroll
            for (int j = 0; j < kWXfers; ++j) dma_rows128(wbase, ldw_b, w_rows, st * kBK * 2, wb, wave * kWXfers + j);
        }
    };

    // ---- wave block: rows wm*32kTM .. +32kTM, columns wn*64 .. +64;
    // acc[j][i] = C^T tile of n-tile j and m-tile i.
    f32x16 acc[2][kTMw];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < kTMw; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;
    int a_off[kTMw], a_swz[kTMw], w_off[2], w_swz[2];
#pragma unroll
    for (int t = 0; t < kTMw; ++t) {
        const int ar = wm * 32 * kTMw + 32 * t + col;
        a_off[t] = ar * kARowBytes;
        a_swz[t] = kAFp8 ? (ar >> 2) & 3 : swz(ar);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int wr = wn * 64 + 32 * t + col;
        w_off[t] = wr * kWRowBytes;
        w_swz[t] = kWFp8 ? (wr >> 2) & 3 : swz(wr);
    }

    // Cross-attention form: the wave's K operands go to registers and both
    // heads' V rows to LDS now, ahead of the stages (older loads: the stage
    // waits cover them), so their latency hides under the main loop.
    i16x8 kreg[kKvG > 0 ? kKvG : 1][4];
    if constexpr (kKvG > 0) {
        const int64_t ldkv_b = p.ldkv * 2;
        const char* kvb = (const char*)p.kv + (int64_t)(m0 / p.seq) * p.ctx_len * ldkv_b;
        const char* kh = kvb + (int64_t)(n0 + wn * 64) * 2;
#pragma unroll
        for (int g = 0; g < kKvG; ++g) {
            const int key = min(32 * g + col, p.ctx_len - 1);  // rows past ctx_len: never visible
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) kreg[g][ks] = *(const i16x8*)(kh + key * ldkv_b + (2 * ks + hf) * 16);
        }
        constexpr int kVXfers = 2 * kVRows / 8 / kWaves;  // 1-KiB transfers per wave
        static_assert(kVXfers * kWaves * 8 == 2 * kVRows, "V transfers");
        const char* vb0 = kvb + (int64_t)(p.n + n0) * 2;
#pragma unroll
        for (int j = 0; j < kVXfers; ++j) {
            const int t = wave * kVXfers + j;
            const int hl = t / (kVRows / 8), r8 = t % (kVRows / 8);
            const int row = 8 * r8 + (lane >> 3);
            const uint32_t off =
                (uint32_t)(min(row, p.ctx_len - 1) * ldkv_b) + (uint32_t)(((lane & 7) ^ swz(row)) << 4);
            lds_dma16(vb0 + hl * 128, off, lds_addr(vbuf + (hl * kVRows + 8 * r8) * kRowBytes));
        }
    }
    auto wait_stage = [&](int s) __attribute__((always_inline)) {
        // Stage s landed (this wave's transfers; later stages may still fly)
        const int later = min(n_stages - 1 - s, kRing - 2);
        if constexpr (kRing >= 4) {
            if (later >= 2) wait_vmem<2 * kLoadsPerStage>();
            else if (later == 1) wait_vmem<kLoadsPerStage>();
            else wait_vmem<0>();
        } else if constexpr (kRing == 3) {
            if (later >= 1) wait_vmem<kLoadsPerStage>();
            else wait_vmem<0>();
        } else {
            wait_vmem<0>();
        }
    };
    if constexpr (kProd) {
        if (producer) {
            // the compute waves' barrier sequence: one per stage, one before the epilogue
#pragma unroll
            for (int st = 0; st < kRing - 1; ++st)
                if (st < n_stages) issue_stage(st);
            for (int s = 0; s < n_stages; ++s) {
                wait_stage(s);
                __syncthreads();
                if (s + kRing - 1 < n_stages) issue_stage(s + kRing - 1);
            }
            __syncthreads();
            return;
        }
    } else {
#pragma unroll
        for (int st = 0; st < kRing - 1; ++st)
            if (st < n_stages) issue_stage(st);
    }
    for (int s = 0; s < n_stages; ++s) {
        if constexpr (!kProd) wait_stage(s);
        __syncthreads();  // stage s landed for every wave, and stage s - 1's buffers are free
        if constexpr (!kProd) {
            if (s + kRing - 1 < n_stages) issue_stage(s + kRing - 1);
        }
        const char* ab = smem[s % kRing];
        const char* wb = smem[s % kRing] + kATileBytes;
        if constexpr (kAFp8) {
            // one fp8 MFMA per tile pair covers the stage: lane reads bytes
            // 32hf .. +31 (chunks 2hf, 2hf + 1) of its W row and A row.
            auto op32 = [&](const char* tile, int off, int sw) __attribute__((always_inline)) {
                const u32x4 lo = *(const lds_u32x4*)(tile + off + (((2 * hf) ^ sw) << 4));
                const u32x4 hi = *(const lds_u32x4*)(tile + off + (((2 * hf + 1) ^ sw) << 4));
                return __builtin_bit_cast(i32x8, u32x4x2{lo, hi});
            };
            i32x8 wop8[2], aop8[kTMw];
#pragma unroll
            for (int t = 0; t < 2; ++t) wop8[t] = op32(wb, w_off[t], w_swz[t]);
#pragma unroll
            for (int t = 0; t < kTMw; ++t) aop8[t] = op32(ab, a_off[t], a_swz[t]);
#pragma unroll
            for (int i = 0; i < kTMw; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[j][i] = mfma32_fp8(wop8[j], aop8[i], acc[j][i]);
            continue;
        }
        // K order inside a stage: step ks = 2 pp + q (pp = 0, 1; q = 0, 1) has
        // lane half hf supply the 8 columns 32 pp + 16 hf + 8 q .. +7 of its row
        // (any order the A and W operands share gives the same sum). Over the two
        // steps of a pair a lane then needs 16 consecutive columns: one 16-byte
        // read of E4M3 weight codes per pair (a 64-byte code row holds four such
        // chunks, swizzled by (row >> 2) & 3, so every 16 lanes of a read hit
        // all 64 banks), where 8-byte reads per step left half the banks idle.
        // Operands of step ks + 1 are read from LDS while step ks's MFMAs run
        // (two register sets), so the LDS latency is not exposed at one or two
        // waves per SIMD. E4M3 weights are decoded just before their step.
        i16x8 aop[2][kTMw];
        u32x4 wraw[2][2];  // fp16: the step's operand; E4M3: the pair's 16 codes
        auto read_ops = [&](int ks, i16x8 (&a)[kTMw], u32x4 (&w)[2]) __attribute__((always_inline)) {
            const int pp = ks >> 1, q = ks & 1;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                if constexpr (kWFp8) {
                    if (q == 0) w[t] = *(const lds_u32x4*)(wb + w_off[t] + (((2 * pp + hf) ^ w_swz[t]) << 4));
                } else {
                    w[t] = __builtin_bit_cast(
                        u32x4, *(const lds_i16x8*)(wb + w_off[t] + (((4 * pp + 2 * hf + q) ^ w_swz[t]) << 4)));
                }
            }
#pragma unroll
            for (int t = 0; t < kTMw; ++t)
                a[t] = *(const lds_i16x8*)(ab + a_off[t] + (((4 * pp + 2 * hf + q) ^ a_swz[t]) << 4));
        };
        read_ops(0, aop[0], wraw[0]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int cur = ks & 1;
            // E4M3: the pair's codes are read at its first step, into the set
            // of that step's parity
            const int wset = kWFp8 ? ((ks >> 1) & 1) : cur;
            if (ks < 3) read_ops(ks + 1, aop[cur ^ 1], wraw[kWFp8 ? (((ks + 1) >> 1) & 1) : cur ^ 1]);
            __builtin_amdgcn_sched_barrier(0);  // keep the next step's reads ahead of this step's MFMAs
            i16x8 wop[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                if constexpr (kWFp8) {
                    const int d = 2 * (ks & 1);  // dwords 0-1: step 2pp, dwords 2-3: step 2pp + 1
                    const uint2 lo = e4m3x4_to_f16(wraw[wset][t][d]), hi = e4m3x4_to_f16(wraw[wset][t][d + 1]);
                    wop[t] = __builtin_bit_cast(i16x8, u32x4{lo.x, lo.y, hi.x, hi.y});
                } else {
                    wop[t] = __builtin_bit_cast(i16x8, wraw[cur][t]);
                }
            }
#pragma unroll
            for (int i = 0; i < kTMw; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[j][i] = mfma32(wop[j], aop[cur][i], acc[j][i]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // ---- epilogue, one m-tile (32 rows) at a time through LDS so that HBM
    // sees whole rows: the wave parks the tile's 32 x 64 fp32 block row-major
    // (256-byte rows, 16-byte chunk c of row r at c ^ (r & 15): conflict-free
    // for 16 lanes of distinct rows), then reads it back with lane l owning
    // columns 4(l%16) .. +3 of rows 4it + l/16: residual loads and output
    // stores are 128-byte row segments per 16 lanes. The tile's 8 residual
    // loads are all issued before its staging. acc[j][i][4u + q] is row
    // 32i + col, column 32j + 8u + 4hf + q of the wave block.
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
    char* eb = &smem[0][0] + wave * (32 * 256);
    static_assert(sizeof(smem) >= kWaves * 32 * 256, "epilogue staging fits in the stage buffers");
    __syncthreads();  // every wave is done with the stage buffers
    if constexpr (kKvG > 0) {
        // ---- cross-attention epilogue. (1) The wave's fp16 query block,
        // computed exactly as the plain epilogue would store it (same parking,
        // scale and rounding), goes to LDS as 32 swizzled 128-byte rows.
        static_assert(kTMw == 1 && kWM == 2, "one 32 x 64 query block per wave");
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = 8 * j + 2 * u + hf;
                *(lds_f32x4*)(eb + col * 256 + ((c ^ (col & 15)) << 4)) =
                    f32x4{acc[j][0][4 * u], acc[j][0][4 * u + 1], acc[j][0][4 * u + 2], acc[j][0][4 * u + 3]};
            }
        const int rq0 = m0 + wm * 32 + (lane >> 4);
        uint2 qv[8];
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const int r = 4 * it + (lane >> 4);
            const float rs = kAFp8 ? p.a_scale[rq0 + 4 * it] : 1.0f;
            const f32x4 a = *(const lds_f32x4*)(eb + r * 256 + ((ec ^ (r & 15)) << 4));
            // fp32 value first, then fp16 (as the plain epilogue and the
            // reference round): the empty asm keeps the compiler from
            // rounding the fma straight to fp16 in one step
            f32x4 v = {a[0] * rs * e_scale.x + e_bias.x, a[1] * rs * e_scale.y + e_bias.y,
                       a[2] * rs * e_scale.z + e_bias.z, a[3] * rs * e_scale.w + e_bias.w};
            asm volatile("" : "+v"(v));
            const f16x4 h = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
            qv[it] = __builtin_bit_cast(uint2, h);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // parked values read before the rows are reused
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const int r = 4 * it + (lane >> 4);
            *(lds_u32x2*)(eb + r * kRowBytes + (((ec >> 1) ^ swz(r)) << 4) + 8 * (ec & 1)) = u32x2{qv[it].x, qv[it].y};
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        // (2) One-pass exact softmax over the ctx_len keys (the short-key
        // attention's block step): S^T = K Q^T with K from registers, one
        // maximum, exp2, one sum, O^T = V^T P^T with V^T by transposing reads.
        const int k_swz = swz(col);
        i16x8 qop[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qop[ks] = *(const lds_i16x8*)(eb + col * kRowBytes + (((2 * ks + hf) ^ k_swz) << 4));
        f32x16 seed_last;
        {
            const int lim = p.ctx_len - 32 * (kKvG - 1) - 4 * hf;
#pragma unroll
            for (int i = 0; i < 16; ++i) seed_last[i] = 8 * (i >> 2) + (i & 3) < lim ? 0.0f : -__builtin_inff();
        }
        f32x16 s[kKvG];
#pragma unroll
        for (int g = 0; g < kKvG; ++g) {
            f32x16 z = {};
            s[g] = mfma32(kreg[g][0], qop[0], g == kKvG - 1 ? seed_last : z);
        }
#pragma unroll
        for (int ks = 1; ks < 4; ++ks)
#pragma unroll
            for (int g = 0; g < kKvG; ++g) s[g] = mfma32(kreg[g][ks], qop[ks], s[g]);
        constexpr int kLastN = kKvHalf ? 8 : 16;
        float mx = -__builtin_inff();
#pragma unroll
        for (int g = 0; g < kKvG; ++g)
#pragma unroll
            for (int i = 0; i < (g == kKvG - 1 ? kLastN : 16); ++i) mx = fmaxf(mx, s[g][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float c = p.scale_log2;
        const float neg_cm = -c * mx;  // ctx_len > 0: every row has a visible key
        const int g16 = lane & 15;
        const int tr_key = 4 * hf + (g16 >> 2), tr_qd = g16 & 3;
        int v_off[2][2];
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
            const int chunk = 4 * dt + 2 * ((lane >> 4) & 1) + (tr_qd >> 1);
#pragma unroll
            for (int hi = 0; hi < 2; ++hi)
                v_off[dt][hi] = (tr_key + 8 * hi) * kRowBytes + ((chunk ^ swz(tr_key + 8 * hi)) << 4) + ((tr_qd & 1) << 3);
        }
        const char* vh = vbuf + wn * (kVRows * kRowBytes);
        f32x16 out[2] = {};
        float l = 0.0f;
#pragma unroll
        for (int g = 0; g < kKvG; ++g) {
            const int n_ss = (kKvHalf && g == kKvG - 1) ? 1 : 2;
            float e[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) e[i] = i < 8 * n_ss ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[g][i], c, neg_cm)) : 0.0f;
            float ls = 0.0f;
#pragma unroll
            for (int h8 = 0; h8 < 2; ++h8)
                if (h8 < n_ss)
                    ls += ((e[8 * h8] + e[8 * h8 + 1]) + (e[8 * h8 + 2] + e[8 * h8 + 3])) +
                          ((e[8 * h8 + 4] + e[8 * h8 + 5]) + (e[8 * h8 + 6] + e[8 * h8 + 7]));
            l += ls;
#pragma unroll
            for (int ss = 0; ss < n_ss; ++ss) {
                u32x4 pw;
#pragma unroll
                for (int w2 = 0; w2 < 4; ++w2) {
                    const f16x2 pr = {(_Float16)e[8 * ss + 2 * w2], (_Float16)e[8 * ss + 2 * w2 + 1]};
                    pw[w2] = __builtin_bit_cast(uint32_t, pr);
                }
                const i16x8 pop = __builtin_bit_cast(i16x8, pw);
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) {
                    const char* base = vh + (32 * g + 16 * ss) * kRowBytes;
                    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + v_off[dt][0]));
                    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(base + v_off[dt][1]));
                    out[dt] = mfma32(i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}, pop, out[dt]);
                }
            }
        }
        const float l_tot = l + __shfl_xor(l, 32, 64);
        const float inv = 1.0f / l_tot;
        // (3) Output rows through the same buffer (the query rows are in
        // registers), then whole 128-byte row segments per 8 lanes.
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const f16x2 w0 = {(_Float16)(out[dt][4 * u] * inv), (_Float16)(out[dt][4 * u + 1] * inv)};
                const f16x2 w1 = {(_Float16)(out[dt][4 * u + 2] * inv), (_Float16)(out[dt][4 * u + 3] * inv)};
                *(lds_u32x2*)(eb + col * kRowBytes + (((4 * dt + u) ^ k_swz) << 4) + 8 * hf) =
                    u32x2{__builtin_bit_cast(uint32_t, w0), __builtin_bit_cast(uint32_t, w1)};
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        _Float16* ob = (_Float16*)p.c + (int64_t)(m0 + wm * 32) * p.ldc + n0 + wn * 64 + 8 * (lane & 7);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int row = 8 * j + (lane >> 3);
            const u32x4 w = *(const lds_u32x4*)(eb + row * kRowBytes + (((lane & 7) ^ swz(row)) << 4));
            store_out<kNt>(w, (u32x4*)(ob + (int64_t)row * p.ldc));
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < kTMw; ++i) {
        const int rm0 = m0 + wm * 32 * kTMw + 32 * i + (lane >> 4);  // row of iteration it: rm0 + 4 it
        f16x4 res[8];
        float rs[8];  // activation scale of the row (1 for fp16 activations)
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            res[it] = f16x4{0, 0, 0, 0};
            rs[it] = kAFp8 ? p.a_scale[min(rm0 + 4 * it, p.m - 1)] : 1.0f;
        }
        if (p.residual != nullptr && en_ok) {
#pragma unroll
            for (int it = 0; it < 8; ++it) {
                const int m = min(rm0 + 4 * it, p.m - 1);
                res[it] = *(const f16x4*)((const _Float16*)p.residual + (int64_t)m * p.ldr + en);
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int c = 8 * j + 2 * u + hf;
                *(lds_f32x4*)(eb + col * 256 + ((c ^ (col & 15)) << 4)) =
                    f32x4{acc[j][i][4 * u], acc[j][i][4 * u + 1], acc[j][i][4 * u + 2], acc[j][i][4 * u + 3]};
            }
        if (en_ok) {
#pragma unroll
            for (int it = 0; it < 8; ++it) {
                const int r = 4 * it + (lane >> 4);
                const int m = rm0 + 4 * it;
                if (m < p.m) {
                    const f32x4 a = *(const lds_f32x4*)(eb + r * 256 + ((ec ^ (r & 15)) << 4));
                    const float v0 = a[0] * rs[it] * e_scale.x + e_bias.x + (float)res[it][0];
                    const float v1 = a[1] * rs[it] * e_scale.y + e_bias.y + (float)res[it][1];
                    const float v2 = a[2] * rs[it] * e_scale.z + e_bias.z + (float)res[it][2];
                    const float v3 = a[3] * rs[it] * e_scale.w + e_bias.w + (float)res[it][3];
                    store_out<kNt>(f16x4{(_Float16)v0, (_Float16)v1, (_Float16)v2, (_Float16)v3},
                                   (f16x4*)((_Float16*)p.c + (int64_t)m * p.ldc + en));
                }
            }
        }
    }
}

// LayerNorm over rows of `width` (even, at most 2048): one wave per row, the
// row held in registers (up to 32 values per lane, as fp16 pairs); two-pass
// centred variance as the reference (ops_kernels.cu:225-257), fp32 maths, one
// rounding to fp16. Sums are wave-tree reductions (order differs from the
// reference's block reduction by rounding only).
constexpr int kLnMaxPer = 16;  // half2 pairs per lane: width <= 2048

// Sum over the wave: DPP butterflies inside each 16-lane row (quad_perm
// [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror pair every lane with one
// from the other half at each level), then the four row sums through
// readlane. Result in every lane.
template <int kCtrl>
__device__ __forceinline__ float dpp_pair_add(float x) {
    const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, false);
    return x + __builtin_bit_cast(float, moved);
}
__device__ __forceinline__ float wave_sum(float x) {
    x = dpp_pair_add<0xB1>(x);   // quad_perm [1,0,3,2]
    x = dpp_pair_add<0x4E>(x);   // quad_perm [2,3,0,1]
    x = dpp_pair_add<0x141>(x);  // row_half_mirror
    x = dpp_pair_add<0x140>(x);  // row_mirror
    const int b = __builtin_bit_cast(int, x);
    return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
           (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}

// kPer fp16 pairs per lane (width <= 128 kPer): straight-line code, every
// load issued before the first use (indices clamped, values masked), so one
// memory round trip covers the row.
// kE4M3: the normalised row (fp32) is quantised to E4M3 codes with a per-row
// scale max(amax / 448, 1e-12) (1 for an all-zero row), round to nearest even,
// saturated to +-448 (the weight quantiser's rule), for the fp8 projection.
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}

template <int kPer, bool kE4M3, bool kNt>
__global__ __launch_bounds__(256) void layer_norm_kernel(LayerNormParams p) {
#pragma clang fp contract(off)  // every operation rounded on its own, as the reference's CPU LayerNorm
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // wave-uniform; no barrier in this kernel
    const int pairs = p.width / 2;
    const f16x2* x = (const f16x2*)((const _Float16*)p.x + row * p.ldx);
    const f16x2* g = (const f16x2*)p.gamma;
    const f16x2* bt = (const f16x2*)p.beta;
    f16x2 h[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) h[j] = x[min(lane + 64 * j, pairs - 1)];
    float v[2 * kPer];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const bool ok = lane + 64 * j < pairs;
        v[2 * j] = ok ? (float)h[j][0] : 0.0f;
        v[2 * j + 1] = ok ? (float)h[j][1] : 0.0f;
        sum += v[2 * j] + v[2 * j + 1];
    }
    const float mean = wave_sum(sum) / (float)p.width;
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        if (lane + 64 * j < pairs) {
            const float d0 = v[2 * j] - mean, d1 = v[2 * j + 1] - mean;
            sq += d0 * d0 + d1 * d1;
        }
    }
    const float var = fmaxf(wave_sum(sq) / (float)p.width, 0.0f);
    const float inv = 1.0f / sqrtf(var + p.eps);
    if constexpr (kE4M3) {
        float yv[2 * kPer];
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int c = lane + 64 * j;
            const f16x2 gg = g[min(c, pairs - 1)], bb = bt[min(c, pairs - 1)];
            yv[2 * j] = (v[2 * j] - mean) * inv * (float)gg[0] + (float)bb[0];
            yv[2 * j + 1] = (v[2 * j + 1] - mean) * inv * (float)gg[1] + (float)bb[1];
            if (c < pairs) amax = fmaxf(amax, fmaxf(fabsf(yv[2 * j]), fabsf(yv[2 * j + 1])));
        }
        amax = wave_max(amax);
        const float scale = amax > 0.0f ? fmaxf(amax / 448.0f, 1.0e-12f) : 1.0f;
        if (lane == 0) p.y_scale[row] = scale;
        uint16_t* q = (uint16_t*)((uint8_t*)p.y + row * p.ldy);
        // y / scale correctly rounded, as the weight quantiser divides, from
        // the correctly rounded reciprocal r (one division per row) and one
        // Markstein correction per value: q = y r, e = y - q scale (exact by
        // fma), q + e r rounds to the nearest quotient.
        const float r = 1.0f / scale;
        auto quot = [&](float y) __attribute__((always_inline)) {
            const float q0 = y * r;
            return __builtin_fmaf(__builtin_fmaf(-q0, scale, y), r, q0);
        };
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int c = lane + 64 * j;
            if (c < pairs) {
                const float q0 = fminf(fmaxf(quot(yv[2 * j]), -448.0f), 448.0f);
                const float q1 = fminf(fmaxf(quot(yv[2 * j + 1]), -448.0f), 448.0f);
                store_out<kNt>((uint16_t)(__builtin_amdgcn_cvt_pk_fp8_f32(q0, q1, 0u, false) & 0xFFFFu), q + c);
            }
        }
        return;
    }
    f16x2* y = (f16x2*)((_Float16*)p.y + row * p.ldy);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int c = lane + 64 * j;
        if (c < pairs) {
            const f16x2 gg = g[c], bb = bt[c];
            const float y0 = (v[2 * j] - mean) * inv * (float)gg[0] + (float)bb[0];
            const float y1 = (v[2 * j + 1] - mean) * inv * (float)gg[1] + (float)bb[1];
            store_out<kNt>(f16x2{(_Float16)y0, (_Float16)y1}, y + c);
        }
    }
}

// LayerNorm (fp16 output) for widths that are a multiple of 8 with 16-byte
// aligned rows: lane l holds chunks l, l + 64, .. of 8 values (16-byte loads
// and stores), otherwise as layer_norm_kernel (same two-pass centred variance,
// fp32 maths, one rounding). kChunks = ceil(width / 512).
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
// Two-pass statistics of one row held as 16-byte chunks (lane l: chunks l,
// l + 64, ..; chunks past the row masked to zero): the values in fp32, the
// mean and 1 / sqrt(var + eps). Shared by the LayerNorm kernels so that every
// LayerNorm in this file rounds identically.
template <int kChunks>
__device__ __forceinline__ void ln_row_stats_v8(const f16x8v (&h)[kChunks], int lane, int chunks, int width, float eps,
                                                float (&v)[8 * kChunks], float& mean, float& inv) {
#pragma clang fp contract(off)  // every operation rounded on its own, as the reference's CPU LayerNorm
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
        const bool ok = lane + 64 * j < chunks;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            v[8 * j + e] = ok ? (float)h[j][e] : 0.0f;
            sum += v[8 * j + e];
        }
    }
    mean = wave_sum(sum) / (float)width;
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
        if (lane + 64 * j < chunks) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float d = v[8 * j + e] - mean;
                sq += d * d;
            }
        }
    }
    const float var = fmaxf(wave_sum(sq) / (float)width, 0.0f);
    inv = 1.0f / sqrtf(var + eps);
}

// One normalised value in fp32: ((v - mean) * inv) * gamma + beta, each
// operation rounded on its own (no fused multiply-add), as the reference's CPU
// LayerNorm computes it.
__device__ __forceinline__ float ln_affine(float v, float mean, float inv, _Float16 g, _Float16 b) {
#pragma clang fp contract(off)
    return (v - mean) * inv * (float)g + (float)b;
}

// One normalised chunk, rounded once to fp16.
__device__ __forceinline__ f16x8v ln_out_v8(const float* v, float mean, float inv, f16x8v gg, f16x8v bb) {
#pragma clang fp contract(off)
    f16x8v o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (_Float16)ln_affine(v[e], mean, inv, gg[e], bb[e]);
    return o;
}

// Sum over each 16-lane row of the wave (DPP butterfly: quad_perm [1,0,3,2],
// [2,3,0,1], row_half_mirror, row_mirror); every lane of a row ends with the
// same value (each step adds two partial sums, commutatively).
__device__ __forceinline__ float row16_sum(float x) {
    x = dpp_pair_add<0xB1>(x);
    x = dpp_pair_add<0x4E>(x);
    x = dpp_pair_add<0x141>(x);
    x = dpp_pair_add<0x140>(x);
    return x;
}

// Maximum over each 16-lane row of the wave (the same DPP pattern as row16_sum).
template <int kCtrl>
__device__ __forceinline__ float dpp_pair_max(float x) {
    const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, false);
    return fmaxf(x, __builtin_bit_cast(float, moved));
}
__device__ __forceinline__ float row16_max(float x) {
    x = dpp_pair_max<0xB1>(x);
    x = dpp_pair_max<0x4E>(x);
    x = dpp_pair_max<0x141>(x);
    x = dpp_pair_max<0x140>(x);
    return x;
}

// Sum over each 32-lane half of the wave: the 16-lane butterfly, then the two
// 16-lane rows of a half exchanged (commutative, so both hold the same value).
__device__ __forceinline__ float row32_sum(float x) {
    x = row16_sum(x);
    return x + __shfl_xor(x, 16, 64);
}

// LayerNorm statistics of 64 / kLanes rows per wave (kLanes = 16 or 32 lanes
// per row) for widths 8 kLanes kCpl: lane l works on row l / kLanes and holds
// its 16-byte chunks l % kLanes + kLanes i (i < kCpl), so every lane is busy and
// a row's sums stay inside its lane group. Two-pass centred variance in fp32
// (the reference's form, ops_kernels.cu:225-257): the sum by v_dot2 of fp16
// pairs against ones (exact products, fp32 accumulation), the centred values
// x - mean straight from fp16 (one fused multiply-add with 1, the exact
// difference rounded once), their squares by fused multiply-adds. d receives
// the centred values.
template <int kCpl, int kLanes = 16>
__device__ __forceinline__ void ln_rows4_stats(const f16x8v (&h)[kCpl], float eps, float (&d)[8 * kCpl], float& inv) {
    static_assert(kLanes == 16 || kLanes == 32, "16 or 32 lanes per row");
    constexpr int kWidth = 8 * kLanes * kCpl;
    auto rsum = [](float x) __attribute__((always_inline)) { return kLanes == 16 ? row16_sum(x) : row32_sum(x); };
    const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kCpl; ++i)
#pragma unroll
        for (int e = 0; e < 8; e += 2)
            sum = __builtin_amdgcn_fdot2(f16x2{h[i][e], h[i][e + 1]}, ones, sum, false);
    const float mean = rsum(sum) / (float)kWidth;
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < kCpl; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            d[8 * i + e] = __builtin_fmaf((float)h[i][e], 1.0f, -mean);
            sq = __builtin_fmaf(d[8 * i + e], d[8 * i + e], sq);
        }
    const float var = fmaxf(rsum(sq) / (float)kWidth, 0.0f);
    inv = 1.0f / sqrtf(var + eps);
}

// One normalised value of the four-rows form in fp32: (d * inv) * gamma + beta
// with the last two as one fused multiply-add.
__device__ __forceinline__ float ln4_affine(float d, float inv, _Float16 g, _Float16 b) {
    return __builtin_fmaf(d * inv, (float)g, (float)b);
}

// fp16 LayerNorm of 64 / kLanes rows per wave (ln_rows4_stats); writes the
// normalised chunks through put(i, chunk index, value). Each value is rounded to
// fp32 and then to fp16 (the empty asm keeps the compiler from folding the fma
// and the conversion into one v_fma_mix rounding, which it may do in one
// caller and not in another).
template <int kCpl, int kLanes = 16, typename Put>
__device__ __forceinline__ void ln_rows4(const f16x8v (&h)[kCpl], const f16x8v (&gg)[kCpl], const f16x8v (&bb)[kCpl],
                                         float eps, Put&& put) {
    float d[8 * kCpl];
    float inv;
    ln_rows4_stats<kCpl, kLanes>(h, eps, d, inv);
    const int j = threadIdx.x & (kLanes - 1);
#pragma unroll
    for (int i = 0; i < kCpl; ++i) {
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = ln4_affine(d[8 * i + e], inv, gg[i][e], bb[i][e]);
        asm volatile("" : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]), "+v"(y[4]), "+v"(y[5]), "+v"(y[6]), "+v"(y[7]));
        f16x8v o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (_Float16)y[e];
        put(i, j + kLanes * i, o);
    }
}

// E4M3 codes of four values y / scale (r = 1 / scale, correctly rounded): the
// quotient from the reciprocal plus one Markstein correction (the correctly
// rounded quotient), saturated to +-448, rounded to nearest even.
__device__ __forceinline__ uint32_t e4m3_code4(const float* y4, float scale, float r) {
    float q[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float q0 = y4[e] * r;
        q[e] = fminf(fmaxf(__builtin_fmaf(__builtin_fmaf(-q0, scale, y4[e]), r, q0), -448.0f), 448.0f);
    }
    const uint32_t lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0u, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
}

// E4M3 LayerNorm of 64 / kLanes rows per wave: the normalised fp32 row
// (ln4_affine), its scale max(amax / 448, 1e-12) (1 for an all-zero row) and
// the codes E4M3(y / scale) (the weight quantiser's rule). put(i, chunk index,
// 8 codes as two dwords); returns the row's scale (the same in all lanes of
// the row).
template <int kCpl, int kLanes = 16, typename Put>
__device__ __forceinline__ float ln_rows4_e4m3(const f16x8v (&h)[kCpl], const f16x8v (&gg)[kCpl],
                                               const f16x8v (&bb)[kCpl], float eps, Put&& put) {
    float v[8 * kCpl];
    float inv;
    ln_rows4_stats<kCpl, kLanes>(h, eps, v, inv);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kCpl; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            v[8 * i + e] = ln4_affine(v[8 * i + e], inv, gg[i][e], bb[i][e]);
            amax = fmaxf(amax, fabsf(v[8 * i + e]));
        }
    amax = row16_max(amax);
    if constexpr (kLanes == 32) amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    const float scale = amax > 0.0f ? fmaxf(amax / 448.0f, 1.0e-12f) : 1.0f;
    const float r = 1.0f / scale;
    const int j = threadIdx.x & (kLanes - 1);
#pragma unroll
    for (int i = 0; i < kCpl; ++i)
        put(i, j + kLanes * i, u32x2{e4m3_code4(v + 8 * i, scale, r), e4m3_code4(v + 8 * i + 4, scale, r)});
    return scale;
}

// fp16 LayerNorm for widths 128 kCpl: 16 rows per 256-thread block, four per
// wave (ln_rows4).
template <int kCpl, bool kNt>
__global__ __launch_bounds__(256) void layer_norm_r4_kernel(LayerNormParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int64_t r = row < p.rows ? row : p.rows - 1;  // rows past the end repeat the last (not stored)
    const int j = lane & 15;
    const f16x8v* x = (const f16x8v*)((const _Float16*)p.x + r * p.ldx);
    const f16x8v* g = (const f16x8v*)p.gamma;
    const f16x8v* bt = (const f16x8v*)p.beta;
    f16x8v h[kCpl], gg[kCpl], bb[kCpl];
#pragma unroll
    for (int i = 0; i < kCpl; ++i) {
        h[i] = x[j + 16 * i];
        gg[i] = g[j + 16 * i];
        bb[i] = bt[j + 16 * i];
    }
    f16x8v* y = (f16x8v*)((_Float16*)p.y + r * p.ldy);
    ln_rows4<kCpl>(h, gg, bb, p.eps, [&](int, int c, f16x8v o) __attribute__((always_inline)) {
        if (row < p.rows) store_out<kNt>(o, y + c);
    });
}

// fp16 LayerNorm for widths 256 kCpl: 8 rows per 256-thread block, two per
// wave with 32 lanes per row (the level-2 rows, 1280 = 256 x 5, hold as many
// values per lane as the width-640 rows in the four-rows form).
template <int kCpl, bool kNt>
__global__ __launch_bounds__(256) void layer_norm_r2_kernel(LayerNormParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int64_t r = row < p.rows ? row : p.rows - 1;  // rows past the end repeat the last (not stored)
    const int j = lane & 31;
    const f16x8v* x = (const f16x8v*)((const _Float16*)p.x + r * p.ldx);
    const f16x8v* g = (const f16x8v*)p.gamma;
    const f16x8v* bt = (const f16x8v*)p.beta;
    f16x8v h[kCpl], gg[kCpl], bb[kCpl];
#pragma unroll
    for (int i = 0; i < kCpl; ++i) {
        h[i] = x[j + 32 * i];
        gg[i] = g[j + 32 * i];
        bb[i] = bt[j + 32 * i];
    }
    f16x8v* y = (f16x8v*)((_Float16*)p.y + r * p.ldy);
    ln_rows4<kCpl, 32>(h, gg, bb, p.eps, [&](int, int c, f16x8v o) __attribute__((always_inline)) {
        if (row < p.rows) store_out<kNt>(o, y + c);
    });
}

// E4M3 LayerNorm for widths 256 kCpl, two rows per wave (32 lanes per row).
template <int kCpl, bool kNt>
__global__ __launch_bounds__(256) void layer_norm_r2_e4m3_kernel(LayerNormParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int64_t r = row < p.rows ? row : p.rows - 1;  // rows past the end repeat the last (not stored)
    const int j = lane & 31;
    const f16x8v* x = (const f16x8v*)((const _Float16*)p.x + r * p.ldx);
    const f16x8v* g = (const f16x8v*)p.gamma;
    const f16x8v* bt = (const f16x8v*)p.beta;
    f16x8v h[kCpl], gg[kCpl], bb[kCpl];
#pragma unroll
    for (int i = 0; i < kCpl; ++i) {
        h[i] = x[j + 32 * i];
        gg[i] = g[j + 32 * i];
        bb[i] = bt[j + 32 * i];
    }
    u32x2* y = (u32x2*)((uint8_t*)p.y + r * p.ldy);
    const float scale = ln_rows4_e4m3<kCpl, 32>(h, gg, bb, p.eps, [&](int, int c, u32x2 codes) __attribute__((always_inline)) {
        if (row < p.rows) store_out<kNt>(codes, y + c);
    });
    if (row < p.rows && j == 0) p.y_scale[row] = scale;
}

// E4M3 LayerNorm (codes + per-row scales) for widths 128 kCpl, four rows per
// wave (ln_rows4_e4m3).
template <int kCpl, bool kNt>
__global__ __launch_bounds__(256) void layer_norm_r4_e4m3_kernel(LayerNormParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int64_t r = row < p.rows ? row : p.rows - 1;  // rows past the end repeat the last (not stored)
    const int j = lane & 15;
    const f16x8v* x = (const f16x8v*)((const _Float16*)p.x + r * p.ldx);
    const f16x8v* g = (const f16x8v*)p.gamma;
    const f16x8v* bt = (const f16x8v*)p.beta;
    f16x8v h[kCpl], gg[kCpl], bb[kCpl];
#pragma unroll
    for (int i = 0; i < kCpl; ++i) {
        h[i] = x[j + 16 * i];
        gg[i] = g[j + 16 * i];
        bb[i] = bt[j + 16 * i];
    }
    u32x2* y = (u32x2*)((uint8_t*)p.y + r * p.ldy);
    const float scale = ln_rows4_e4m3<kCpl>(h, gg, bb, p.eps, [&](int, int c, u32x2 codes) __attribute__((always_inline)) {
        if (row < p.rows) store_out<kNt>(codes, y + c);
    });
    if (row < p.rows && j == 0) p.y_scale[row] = scale;
}

template <int kChunks, bool kNt, bool kE4M3>
__global__ __launch_bounds__(256) void layer_norm_v8_kernel(LayerNormParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // wave-uniform; no barrier in this kernel
    const int chunks = p.width / 8;
    const f16x8v* x = (const f16x8v*)((const _Float16*)p.x + row * p.ldx);
    f16x8v h[kChunks];
#pragma unroll
    for (int j = 0; j < kChunks; ++j) h[j] = x[min(lane + 64 * j, chunks - 1)];
    float v[8 * kChunks];
    float mean, inv;
    ln_row_stats_v8<kChunks>(h, lane, chunks, p.width, p.eps, v, mean, inv);
    const f16x8v* g = (const f16x8v*)p.gamma;
    const f16x8v* bt = (const f16x8v*)p.beta;
    if constexpr (kE4M3) {
        // as layer_norm_kernel's E4M3 form: row amax, scale, correctly rounded
        // quotients (reciprocal + one Markstein correction), 8 codes per lane
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            const int c = min(lane + 64 * j, chunks - 1);
            const f16x8v gg = g[c], bb = bt[c];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[8 * j + e] = ln_affine(v[8 * j + e], mean, inv, gg[e], bb[e]);
            if (lane + 64 * j < chunks)
#pragma unroll
                for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[8 * j + e]));
        }
        amax = wave_max(amax);
        const float scale = amax > 0.0f ? fmaxf(amax / 448.0f, 1.0e-12f) : 1.0f;
        if (lane == 0) p.y_scale[row] = scale;
        const float r = 1.0f / scale;
        auto code4 = [&](const float* y4) __attribute__((always_inline)) {
            float q[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float q0 = y4[e] * r;
                q[e] = fminf(fmaxf(__builtin_fmaf(__builtin_fmaf(-q0, scale, y4[e]), r, q0), -448.0f), 448.0f);
            }
            const uint32_t lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0u, false);
            return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
        };
        typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
        u32x2v* yq = (u32x2v*)((uint8_t*)p.y + row * p.ldy);
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            const int c = lane + 64 * j;
            if (c < chunks) store_out<kNt>(u32x2v{code4(v + 8 * j), code4(v + 8 * j + 4)}, yq + c);
        }
        return;
    }
    f16x8v* y = (f16x8v*)((_Float16*)p.y + row * p.ldy);
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
        const int c = lane + 64 * j;
        if (c < chunks) {
            store_out<kNt>(ln_out_v8(v + 8 * j, mean, inv, g[c], bt[c]), y + c);
        }
    }
}

// LayerNorm fused into the projection that consumes it, for K = kK input
// features (640: level 1, 1280: level 2) and E4M3 weights (the transformer
// block's norm1 -> q|k|v and norm2 -> q, src/cuda/unet.cpp:106-112,120-124):
// c[m, n] = w_scale[n] * sum_k LN(x)[m, k] w[n, k] (+ bias[n]), with LN(x)
// exactly as the standalone LayerNorm kernel of that width rounds it.
//
// One workgroup of 8 waves per CU (two per SIMD) owns 64 rows and a range of
// 128-column chunks of the output. Prologue: the rows are normalised once with
// the standalone LayerNorm's code for the width (640: ln_rows4, four rows per
// wave-quarter of 16 lanes; 1280: two rows per wave-half of 32 lanes) into LDS,
// then each wave takes its 32 rows' normalised values into registers as MFMA
// operands (kK / 16 steps of 8 values: 160 VGPRs at kK = 640), so the
// activations never go back to HBM. At kK = 1280 with fp16 activations
// (kSplitA) the registers hold K columns 0-639 and LDS keeps columns 640-1279
// of all 64 rows for the whole kernel (80 KiB), read per K step in the second
// half of every chunk. kAFp8: the LayerNorm rounds each row to E4M3 codes with
// a per-row scale (ln_rows4_e4m3, the standalone E4M3 LayerNorm's code; kK
// codes per row: 80 VGPRs at 640, 160 at 1280) and the projection runs on
// v_mfma_f32_32x32x64_f8f6f4 with the weight codes as read (no decode), as
// linear_kernel's fp8 form. Main loop: the E4M3 weight rows of each chunk
// stream HBM/L2 -> LDS by global_load_lds_dwordx4 in 128-column K stages (two
// 64-byte-row sub-stages, linear_kernel's layout) through a ring of three
// (prefetch distance two, one barrier per stage); wave (wm, wn) computes rows
// 32 wm .. +31 x columns 32 wn .. +31 of a chunk as one chain of kK / 16
// v_mfma_f32_32x32x16_f16 over linear_kernel's K order, operand layouts and
// code decode (fp8: one MFMA per 64-column sub-stage), so the fp32 sums equal
// that kernel's. At the end of a chunk each wave rounds its 32 x 32 block to
// fp16 (scale, bias: linear_kernel's epilogue arithmetic) into a 2-KiB LDS
// staging; the block is stored as 64-byte row segments during the next
// chunk's second stage, so the stores drain under MFMA work instead of in one
// burst at the end. Per-column scales and bias sit in LDS, and every lane
// stores (rows past m repeat row m - 1 with its own value), so the
// vector-memory operations in the loop are a fixed sequence and every wait
// counts exactly the transfers it needs.
template <int kK>
constexpr int ln_linear_max_cols() { return kK > 640 ? 1024 : 2048; }  // output columns per workgroup

template <int kK, bool kAFp8, bool kNt>
__global__ __launch_bounds__(512, 1) void ln_linear_kernel(LnLinearParams p) {
    constexpr int kStages = kK / 128;        // 128-column K stages per chunk
    constexpr int kSteps = kK / 16;          // MFMA K steps
    constexpr int kStageBytes = 2 * 128 * 64;  // two sub-stages of 128 code rows x 64 bytes
    constexpr int kRing = 3;
    constexpr int kLanes = kK > 640 ? 32 : 16;   // lanes per row in the LayerNorm (the standalone kernel's)
    constexpr int kCpl = kK / (8 * kLanes);      // 16-byte fp16 chunks per lane and row
    constexpr int kRowsPerGroup = 64 / kLanes;   // rows per wave and LayerNorm call
    constexpr int kGroups = 8 / kRowsPerGroup;   // LayerNorm calls per wave (8 rows)
    constexpr bool kSplitA = !kAFp8 && kK > 640;  // K columns 640.. from LDS
    constexpr int kRegSteps = kSplitA ? 40 : kSteps;  // K steps held in registers (fp16)
    constexpr int kHalfChunks = 80;               // 16-byte chunks of 640 fp16 columns
    constexpr int kARow = kAFp8 ? kK : (kSplitA ? 2 * 640 : 2 * kK);  // bytes of one row in abuf
    constexpr int kMaxCols = ln_linear_max_cols<kK>();
    constexpr int kStgBytes = 32 * 32 * 2;        // one wave's fp16 32 x 32 staging
    static_assert(kK % 128 == 0 && kCpl * 8 * kLanes == kK, "width");
    static_assert(kSplitA || 8 * kStgBytes <= 64 * kARow, "epilogue staging fits in the row buffer");
    __shared__ __attribute__((aligned(16))) char ring[kRing][kStageBytes];
    __shared__ __attribute__((aligned(16))) char abuf[64 * kARow];
    __shared__ __attribute__((aligned(16))) char stg_own[kSplitA ? 8 * kStgBytes : 16];
    __shared__ __attribute__((aligned(16))) float sc_lds[kMaxCols];
    __shared__ __attribute__((aligned(16))) float bias_lds[kMaxCols];
    __shared__ float rs_lds[64];  // E4M3 activations: the rows' scales

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hf = lane >> 5, col = lane & 31;
    const int wm = wave & 1, wn = wave >> 1;

    // XCD-aware task order (as linear_kernel): the n_split tasks of a row block
    // are consecutive, so they run on one XCD and share its rows in L2.
    int task;
    {
        const int n = p.m_blocks * p.n_split;
        const int id = blockIdx.x;
        const int xcd = id & 7, slot = id >> 3;
        const int per = n >> 3, extra = n & 7;
        task = xcd * per + (xcd < extra ? xcd : extra) + slot;
    }
    const int mb = task / p.n_split, ns = task % p.n_split;
    const int m0 = mb * 64;
    const int c_begin = (int)((int64_t)ns * p.chunks / p.n_split);
    const int c_end = (int)((int64_t)(ns + 1) * p.chunks / p.n_split);
    const int nch = c_end - c_begin;  // >= 1: n_split <= chunks
    const int G = nch * kStages;      // K stages of the workgroup

    // Weight transfers of stage g (chunk c_begin + g / kStages, K stage
    // g % kStages): wave w moves code rows 16 w .. +15 of both sub-stages;
    // lane l takes row 16 w + l / 4 and global chunk (l % 4) ^ ((row >> 2) & 3),
    // the slot the readers expect, so its offset is the same for every stage.
    const int dma_row = 16 * wave + (lane >> 2);
    const uint32_t w_lane_off =
        (uint32_t)(dma_row * p.ldw) + (uint32_t)(((lane & 3) ^ ((dma_row >> 2) & 3)) << 4);
    auto issue_stage = [&](int g) __attribute__((always_inline)) {
        const int chunk = c_begin + g / kStages, st = g % kStages;
        const char* base = (const char*)p.w + (int64_t)chunk * 128 * p.ldw + st * 128;
        char* buf = ring[g % kRing];
        lds_dma16(base, w_lane_off, lds_addr(buf + wave * 1024));
        lds_dma16(base + 64, w_lane_off, lds_addr(buf + 8192 + wave * 1024));
    };
    issue_stage(0);
    if (G > 1) issue_stage(1);

    // Per-column scales and bias of the workgroup's columns: loaded now, with
    // the rows below, and written to LDS after the LayerNorm (one memory round
    // trip for both).
    constexpr int kColsPerThread = kMaxCols / 512;
    float sc_reg[kColsPerThread], bias_reg[kColsPerThread];
    {
        const int n0 = c_begin * 128, ncols = nch * 128;
#pragma unroll
        for (int k = 0; k < kColsPerThread; ++k) {
            const int i = threadIdx.x + 512 * k;
            sc_reg[k] = i < ncols ? p.w_scale[n0 + i] : 0.0f;
            bias_reg[k] = i < ncols && p.bias != nullptr ? (float)((const _Float16*)p.bias)[n0 + i] : 0.0f;
        }
    }

    // ---- LayerNorm of the block's 64 rows: wave w takes rows 8 w .. +7 as
    // kGroups calls of the standalone kernel's code (rows past m repeat row
    // m - 1). fp16 rows: 16-byte chunk c of row r at slot c ^ (r & 15); with
    // kSplitA, chunks 0-79 (columns 0-639) go to LDS now and chunks 80-159 are
    // kept in registers until the first half has been taken into operand
    // registers, then written over it.
    constexpr int kKeep = kSplitA ? 3 : 1;  // chunks i = 2, 3, 4 of a lane may lie past column 640
    f16x8v keep[kGroups][kKeep];
    {
        const int j = lane & (kLanes - 1);
        const f16x8v* g = (const f16x8v*)p.gamma;
        const f16x8v* bt = (const f16x8v*)p.beta;
        f16x8v gg[kCpl], bb[kCpl];
#pragma unroll
        for (int i = 0; i < kCpl; ++i) {
            gg[i] = g[j + kLanes * i];
            bb[i] = bt[j + kLanes * i];
        }
        // rows loaded two calls at a time (all loads of a pair issued before its first use)
#pragma unroll
        for (int g2 = 0; g2 < kGroups; g2 += 2) {
            f16x8v h[2][kCpl];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int gm = min(m0 + 8 * wave + kRowsPerGroup * (g2 + u) + lane / kLanes, p.m - 1);
                const f16x8v* xr = (const f16x8v*)((const _Float16*)p.x + (int64_t)gm * p.ldx);
#pragma unroll
                for (int i = 0; i < kCpl; ++i) h[u][i] = xr[j + kLanes * i];
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int grp = g2 + u;
                const int r = 8 * wave + kRowsPerGroup * grp + lane / kLanes;
                if constexpr (kAFp8) {
                    // E4M3 rows (ln_rows4_e4m3, the standalone E4M3 LayerNorm's code):
                    // the 8 codes of fp16 chunk c at byte 8c, 16-byte slots swizzled
                    // by r & 7
                    const float sc = ln_rows4_e4m3<kCpl, kLanes>(h[u], gg, bb, p.eps,
                                                                 [&](int, int c, u32x2 codes) __attribute__((always_inline)) {
                        *(lds_u32x2*)(abuf + r * kARow + (((c >> 1) ^ (r & 7)) << 4) + 8 * (c & 1)) = codes;
                    });
                    if (j == 0) rs_lds[r] = sc;
                } else {
                    ln_rows4<kCpl, kLanes>(h[u], gg, bb, p.eps, [&](int i, int c, f16x8v o) __attribute__((always_inline)) {
                        if (!kSplitA || c < kHalfChunks)
                            *(__attribute__((address_space(3))) f16x8v*)(abuf + r * kARow + ((c ^ (r & 15)) << 4)) = o;
                        if constexpr (kSplitA) {
                            if (i >= 2) keep[grp][i - 2] = o;
                        }
                    });
                }
            }
        }
    }
#pragma unroll
    for (int k = 0; k < kColsPerThread; ++k) {
        sc_lds[threadIdx.x + 512 * k] = sc_reg[k];
        bias_lds[threadIdx.x + 512 * k] = bias_reg[k];
    }
    __syncthreads();
    // Activation operands of the wave's rows: step ks = 4 s + 2 pp + q (s: 64-column
    // sub-stage) takes columns 64 s + 32 pp + 16 hf + 8 q .. +7 (linear_kernel's K order),
    // i.e. 16-byte chunk a_chunk(ks) of the row.
    // E4M3 activations: one fp8 MFMA per 64-column sub-stage s, the lane
    // supplying bytes 64 s + 32 hf .. +31 of its row (linear_kernel's fp8 order).
    const int ar = 32 * wm + col;
    auto a_chunk = [&](int ks) __attribute__((always_inline)) {
        return 8 * (ks >> 2) + 4 * ((ks >> 1) & 1) + 2 * hf + (ks & 1);
    };
    i16x8 aop[kAFp8 ? 1 : kRegSteps];
    i32x8 aop8[kAFp8 ? kK / 64 : 1];
    if constexpr (kAFp8) {
#pragma unroll
        for (int s8 = 0; s8 < kK / 64; ++s8) {
            const u32x4 lo = *(const lds_u32x4*)(abuf + ar * kARow + (((4 * s8 + 2 * hf) ^ (ar & 7)) << 4));
            const u32x4 hi = *(const lds_u32x4*)(abuf + ar * kARow + (((4 * s8 + 2 * hf + 1) ^ (ar & 7)) << 4));
            aop8[s8] = __builtin_bit_cast(i32x8, u32x4x2{lo, hi});
        }
    } else {
#pragma unroll
        for (int ks = 0; ks < kRegSteps; ++ks)
            aop[ks] = *(const lds_i16x8*)(abuf + ar * kARow + ((a_chunk(ks) ^ (ar & 15)) << 4));
    }
    __syncthreads();  // kSplitA: the row buffer takes columns 640-1279; else it becomes the epilogue staging
    if constexpr (kSplitA) {
        const int j = lane & (kLanes - 1);
#pragma unroll
        for (int grp = 0; grp < kGroups; ++grp) {
            const int r = 8 * wave + kRowsPerGroup * grp + lane / kLanes;
#pragma unroll
            for (int i = 2; i < kCpl; ++i) {
                const int c = j + kLanes * i;
                if (c >= kHalfChunks)
                    *(__attribute__((address_space(3))) f16x8v*)(abuf + r * kARow + (((c - kHalfChunks) ^ (r & 15)) << 4)) =
                        keep[grp][i - 2];
            }
        }
        __syncthreads();
    }
    (void)keep;

    const int wr = 32 * wn + col;  // weight row of this lane within a chunk
    const int w_off = wr * 64, w_swz = (wr >> 2) & 3;
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
    char* stg = (kSplitA ? stg_own : abuf) + wave * kStgBytes;
    // Epilogue of one chunk's 32 x 32 block, in two parts: park() at the end of
    // the chunk forms the outputs ((sum x row scale) then scale and bias in one
    // fused multiply-add, fp32, then fp16: linear_kernel's epilogue rounding)
    // and writes them to the wave's staging (64-byte fp16 rows, 8-byte unit v
    // of row r at v ^ ((r >> 2) & 7): conflict-free in both directions; acc[4u
    // + q] is row col, column 8u + 4hf + q); store() reads them back during
    // the next chunk with lane l on columns 4 (l % 8) .. +3 of rows l / 8 + 8 it
    // and stores: exactly four stores per lane.
    auto park = [&](const f32x16& a, int ci) __attribute__((always_inline)) {
        const float rs = kAFp8 ? rs_lds[ar] : 1.0f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int lc = ci * 128 + 32 * wn + 8 * u + 4 * hf;  // column within the workgroup's range
            const f32x4 e_scale = *(const lds_f32x4*)(sc_lds + lc);
            const f32x4 e_bias = *(const lds_f32x4*)(bias_lds + lc);
            f32x4 v = {a[4 * u], a[4 * u + 1], a[4 * u + 2], a[4 * u + 3]};
            if constexpr (kAFp8) v = f32x4{v[0] * rs, v[1] * rs, v[2] * rs, v[3] * rs};
            // the empty asm keeps the compiler from rounding the fma straight to
            // fp16 (v_fma_mix)
            f32x4 o = {__builtin_fmaf(v[0], e_scale[0], e_bias[0]), __builtin_fmaf(v[1], e_scale[1], e_bias[1]),
                       __builtin_fmaf(v[2], e_scale[2], e_bias[2]), __builtin_fmaf(v[3], e_scale[3], e_bias[3])};
            asm volatile("" : "+v"(o));
            const f16x4 h4 = {(_Float16)o[0], (_Float16)o[1], (_Float16)o[2], (_Float16)o[3]};
            *(lds_u32x2*)(stg + col * 64 + (((2 * u + hf) ^ ((col >> 2) & 7)) << 3)) = __builtin_bit_cast(u32x2, h4);
        }
    };
    // (32-bit element offsets: m * ldc + n < 2^31, checked on the host)
    auto store = [&](int ci) __attribute__((always_inline)) {
        const int en = (c_begin + ci) * 128 + 32 * wn + 4 * (lane & 7);
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int r = (lane >> 3) + 8 * it;
            const int m = min(m0 + 32 * wm + r, p.m - 1);
            const u32x2 v = *(const lds_u32x2*)(stg + r * 64 + (((lane & 7) ^ ((r >> 2) & 7)) << 3));
            const uint32_t off = (uint32_t)m * (uint32_t)p.ldc + (uint32_t)en;
            store_out<kNt>(__builtin_bit_cast(f16x4, v), (f16x4*)((_Float16*)p.c + off));
        }
    };

    // Waits before stage g: the vector-memory operations issued after stage
    // g's transfers are stage g + 1's two transfers (when it exists) and, in
    // K stages 2 and 3 of every chunk but the first, the previous chunk's four
    // output stores (issued in K stage 1): vmcnt counts them in issue order.
    auto wait_stage = [&](bool next, bool stores) __attribute__((always_inline)) {
        if (stores) {
            if (next) wait_vmem<6>();
            else wait_vmem<4>();
        } else {
            if (next) wait_vmem<2>();
            else wait_vmem<0>();
        }
    };

    for (int ci = 0; ci < nch; ++ci) {
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int st = 0; st < kStages; ++st) {
            const int g = ci * kStages + st;
            wait_stage(g + 1 < G, ci > 0 && (st == 2 || st == 3));
            __syncthreads();  // stage g landed for every wave; stage g - 1's buffer is free
            if (g + 2 < G) issue_stage(g + 2);
            const char* cur = ring[g % kRing];
            // fp16 activations: pair pr = (sub-stage pr / 2, K pair pr % 2), the
            // lane's 16 codes of two K steps; E4M3 activations: pr = (sub-stage pr
            // / 2, half pr % 2) of the lane's 32 code bytes 32 hf .. +31
            auto read_w = [&](int pr) __attribute__((always_inline)) {
                const int chunk = kAFp8 ? 2 * hf + (pr & 1) : 2 * (pr & 1) + hf;
                return *(const lds_u32x4*)(cur + (pr >> 1) * 8192 + w_off + ((chunk ^ w_swz) << 4));
            };
            if constexpr (kAFp8) {
                // both sub-stages' 32 code bytes per lane, then one fp8 MFMA each
                u32x4 wq[4];
#pragma unroll
                for (int pr = 0; pr < 4; ++pr) wq[pr] = read_w(pr);
#pragma unroll
                for (int sub = 0; sub < 2; ++sub) {
                    acc = mfma32_fp8(__builtin_bit_cast(i32x8, u32x4x2{wq[2 * sub], wq[2 * sub + 1]}),
                                     aop8[2 * st + sub], acc);
                    if (st == 1 && sub == 0 && ci > 0) {
                        store(ci - 1);
                        asm volatile("" ::: "memory");  // as below
                    }
                }
                continue;
            }
            // activation operands of K step ks: registers, or (kSplitA, second
            // half of the chunk) the LDS rows
            const bool lds_a = kSplitA && st >= kStages / 2;
            auto read_a = [&](int ks) __attribute__((always_inline)) -> i16x8 {
                return *(const lds_i16x8*)(abuf + ar * kARow + (((a_chunk(ks) - kHalfChunks) ^ (ar & 15)) << 4));
            };
            // code reads two pairs ahead of their MFMAs; LDS activations (kSplitA,
            // second half of the chunk) at the pair's start
            u32x4 wq[4];
            wq[0] = read_w(0);
            wq[1] = read_w(1);
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) {
                if (pr + 2 < 4) wq[pr + 2] = read_w(pr + 2);
                i16x8 aq[2];
                if (lds_a) {
#pragma unroll
                    for (int q = 0; q < 2; ++q) aq[q] = read_a(8 * st + 2 * pr + q);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const uint2 lo = e4m3x4_to_f16(wq[pr][2 * q]), hi = e4m3x4_to_f16(wq[pr][2 * q + 1]);
                    const int ks = 8 * st + 2 * pr + q;
                    const i16x8 a_op = lds_a ? aq[q] : aop[ks < kRegSteps ? ks : 0];
                    acc = mfma32(__builtin_bit_cast(i16x8, u32x4{lo.x, lo.y, hi.x, hi.y}), a_op, acc);
                }
                if (st == 1 && pr == 1 && ci > 0) {
                    store(ci - 1);
                    // the stores stay here, ahead of the next stage's wait,
                    // which counts them (a compiler barrier only)
                    asm volatile("" ::: "memory");
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        park(acc, ci);  // the wave's staging was read back in this chunk's K stage 1
    }
    store(nch - 1);
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

hipError_t launch_linear(const LinearParams& params_in, bool w_fp8, int compute_units, hipStream_t stream) {
    LinearParams p = params_in;
    const bool a_fp8 = p.a_scale != nullptr;
    if (a_fp8 && !w_fp8) return hipErrorInvalidValue;
    if (p.m == 0 || p.n == 0) return hipSuccess;
    if (p.k % kBK != 0 || p.n % 4 != 0) return hipErrorInvalidValue;
    p.n_blocks = (p.n + kBN - 1) / kBN;
    // Row-tile height: 256 (twice the MFMA work per staged byte, E4M3 weights)
    // when those tiles still give at least 80% of the resident workgroups (two
    // per CU) work; else 128, unless 128-row tiles fill less than 70% of them,
    // then 64 (measured: 2048 x 1280 x 1280 18.3 -> 15.2 us fp16, 12.2 -> 10.0
    // fp8; 8192 x 640 x 640 E4M3 weights 15.3 -> 13.2 us).
    const int64_t slots = (int64_t)(compute_units > 0 ? compute_units : 256) * 2;
    const int64_t tall = (int64_t)((p.m + 255) / 256) * p.n_blocks;
    const int64_t mid = (int64_t)((p.m + 127) / 128) * p.n_blocks;
    const bool use_tall = w_fp8 && tall * 5 >= slots * 4;
    const bool use_short = !use_tall && mid * 10 < slots * 7;
    p.m_blocks = use_tall ? (p.m + 255) / 256 : use_short ? (p.m + 63) / 64 : (p.m + 127) / 128;
    const int64_t tasks = (int64_t)p.m_blocks * p.n_blocks;
    if (tasks > 0x7FFFFFFF) return hipErrorInvalidValue;
    // Task groups of 8 m blocks for M >= 4096, row-major (groups of 1) below.
    // Measured in the sublayer chains, where A is the previous kernel's fresh
    // output: configs[3] (M = 8192) 142.4 -> 140.6 us with groups of 8, the
    // level-2 cross sublayer (M = 2048) 44.0 -> 46.6 us, although each of its
    // projections alone ran 5-8 % faster (1, 4, 8, 16 and sqrt-balanced group
    // sizes tried on the standalone projections).
    p.group_m = p.m < 4096 ? 1 : p.m_blocks < 8 ? p.m_blocks : 8;
    const dim3 grid((unsigned)tasks), block(256);
    // non-temporal output stores for large outputs
    const bool nt = (int64_t)p.m * p.n * 2 >= kStreamOutBytes;
#define SDXL_LIN(WF, AF, TM, RING)                                                                              \
    do {                                                                                                        \
        if (nt) hipLaunchKernelGGL((linear_kernel<WF, AF, TM, RING, 2, true>), grid, block, 0, stream, p);      \
        else hipLaunchKernelGGL((linear_kernel<WF, AF, TM, RING, 2, false>), grid, block, 0, stream, p);        \
    } while (0)
    // ... with four producer waves (512 threads)
#define SDXL_LIN_PROD(WF, AF, TM, RING, OCC)                                                                    \
    do {                                                                                                        \
        const dim3 bp(512);                                                                                     \
        if (nt) hipLaunchKernelGGL((linear_kernel<WF, AF, TM, RING, OCC, true, 2, 0, false, 2, true>), grid, bp, 0, stream, p); \
        else hipLaunchKernelGGL((linear_kernel<WF, AF, TM, RING, OCC, false, 2, 0, false, 2, true>), grid, bp, 0, stream, p); \
    } while (0)
    // E4M3 weights: 256 x 128 tiles of 8 waves (4 x 2, each 64 x 64; two
    // workgroups per CU) when those tiles give at least 90 % of the CUs one:
    // each staged W tile serves twice the rows, four waves share each SIMD.
    // Measured: 8192 x 1920 x 640 with E4M3 activations 19.9 -> 16.7 us, fp16
    // activations 30-32 -> 27.5-30 us (configs[3] sublayer stage 29.5 -> 24.9);
    // 2048 x 3840 x 1280 19.2 -> 16.3 and 28.2 -> 26.6 us. With fewer tiles
    // (the out-projections) they ran slower; fp16 weights (48-KiB stages, one
    // workgroup per CU) measured within 2 %, so those keep the 4-wave grids.
    // Below 4096 rows with at least 512 columns the eight waves take 128 x 256
    // tiles instead (2 x 4 waves): per K stage 16 KiB of A and 16 KiB of
    // weight codes against 32 + 8 KiB for the same MFMA work, and the
    // transfers' issue is what the loop waits on (2048 x 3840 x 1280 28.1 ->
    // 27.4 us; 8192-row projections unchanged, so they keep 256 x 128).
    if (w_fp8 && p.m < 4096 && p.n >= 512 &&
        (int64_t)((p.m + 127) / 128) * ((p.n + 255) / 256) * 10 >= (int64_t)(compute_units > 0 ? compute_units : 256) * 9) {
        p.m_blocks = (p.m + 127) / 128;
        p.n_blocks = (p.n + 255) / 256;
        p.group_m = 1;
        const dim3 g8((unsigned)((int64_t)p.m_blocks * p.n_blocks)), b8(512);
        if (a_fp8) {
            if (nt) hipLaunchKernelGGL((linear_kernel<true, true, 2, 3, 2, true, 2, 0, false, 4>), g8, b8, 0, stream, p);
            else hipLaunchKernelGGL((linear_kernel<true, true, 2, 3, 2, false, 2, 0, false, 4>), g8, b8, 0, stream, p);
        } else {
            if (nt) hipLaunchKernelGGL((linear_kernel<true, false, 2, 2, 2, true, 2, 0, false, 4>), g8, b8, 0, stream, p);
            else hipLaunchKernelGGL((linear_kernel<true, false, 2, 2, 2, false, 2, 0, false, 4>), g8, b8, 0, stream, p);
        }
        return hipGetLastError();
    }
    if (w_fp8 && (int64_t)((p.m + 255) / 256) * p.n_blocks * 10 >= (int64_t)(compute_units > 0 ? compute_units : 256) * 9) {
        p.m_blocks = (p.m + 255) / 256;
        p.group_m = p.m < 4096 ? 1 : p.m_blocks < 8 ? p.m_blocks : 8;
        const dim3 g8((unsigned)((int64_t)p.m_blocks * p.n_blocks)), b8(512);
        if (a_fp8) {
            if (nt) hipLaunchKernelGGL((linear_kernel<true, true, 4, 3, 2, true, 4>), g8, b8, 0, stream, p);
            else hipLaunchKernelGGL((linear_kernel<true, true, 4, 3, 2, false, 4>), g8, b8, 0, stream, p);
        } else {
            if (nt) hipLaunchKernelGGL((linear_kernel<true, false, 4, 2, 2, true, 4>), g8, b8, 0, stream, p);
            else hipLaunchKernelGGL((linear_kernel<true, false, 4, 2, 2, false, 4>), g8, b8, 0, stream, p);
        }
        return hipGetLastError();
    }
    // 64-row tiles of few workgroups per CU (the level-2 projections, the
    // per-request context K/V projection) wait on their stage transfers
    // (rocprof: 59 % of wave time in s_waitcnt, 11 % MFMA-busy on the
    // level-2 out-projection): there producer waves issue the transfers and,
    // with fp16 weights, a deeper ring requests each stage further ahead.
    // Measured (graph replay, fp16 weights): one round of tiles, ring of four
    // (96 KiB: one workgroup per CU) + producers: context K/V [154, 2048] x
    // [2048, 2560] 20.8 -> 12.0 us, x [2048, 1280] 15.3 -> 11.1 us; at most
    // 1.25 tiles per CU, ring of three + producers: 2048 x 1280 x 1280 + bias +
    // residual 16.5 -> 15.0 us; E4M3 weights, producers on the two-stage
    // ring: 13.1 -> 12.6 us (2048 x 1280 x 1280), context K/V 15.6 -> 12.0 us.
    // With more tiles per CU (8192 x 640 x 640, 3840 x 1280 x 1280) both
    // measured slower than the plain four-wave kernel.
    // one round of fp16-weight tiles: the K-split kernel (linear_ksplit.hip);
    // measured 2048 x 1280 x 1280 + bias + residual 15.6 -> 13.8 us
    if (linear_ksplit_supported(p, w_fp8, compute_units)) return launch_linear_ksplit(p, stream);
    const int cus_lin = compute_units > 0 ? compute_units : 256;
    const bool one_round = tasks <= cus_lin, few = tasks * 4 <= (int64_t)cus_lin * 5;
    if (a_fp8) {
        if (use_tall) SDXL_LIN(true, true, 4, 3);
        else if (use_short) SDXL_LIN(true, true, 1, 2);
        else SDXL_LIN(true, true, 2, 3);
    } else if (w_fp8) {
        if (use_tall) SDXL_LIN(true, false, 4, 2);
        else if (use_short && few) SDXL_LIN_PROD(true, false, 1, 2, 2);
        else if (use_short) SDXL_LIN(true, false, 1, 2);
        else SDXL_LIN(true, false, 2, 3);
    } else {
        if (use_short && one_round) SDXL_LIN_PROD(false, false, 1, 4, 1);
        else if (use_short && few) SDXL_LIN_PROD(false, false, 1, 3, 2);
        else if (use_short) SDXL_LIN(false, false, 1, 2);
        else SDXL_LIN(false, false, 2, 2);
    }
#undef SDXL_LIN_PROD
#undef SDXL_LIN
    return hipGetLastError();
}

// Workgroups of the fused kernel resident per CU (LDS: 52 KiB with E4M3
// weights and fp16 activations, 56 or 68 KiB otherwise).
int q_cross_attention_per_cu(bool w_fp8, bool a_fp8) { return w_fp8 && !a_fp8 ? 3 : 2; }

bool q_cross_attention_supported(const LinearParams& p, bool w_fp8, int compute_units) {
    // one round: a second round of a few workgroups costs more than the
    // saved launch and query round trip
    const int64_t tasks = p.m > 0 ? (int64_t)(p.m / 64) * (p.n / 128) : 0;
    if (compute_units <= 0 || tasks > (int64_t)q_cross_attention_per_cu(w_fp8, p.a_scale != nullptr) * compute_units)
        return false;
    // the fused form computes the attention as the 32-row short-key kernel
    // does; calls that the attention dispatch gives 16-row blocks stay
    // separate, so that both forms give the same bits
    if (p.m <= 0 || short_keys_16_row_blocks((int64_t)(p.m / 32) * (p.n / 64), compute_units)) return false;
    return p.m > 0 && p.seq > 0 && p.seq % 64 == 0 && p.m % p.seq == 0 && p.n % 128 == 0 && p.k % kBK == 0 &&
           p.ctx_len >= 65 && p.ctx_len <= 80 && p.kv != nullptr && p.bias == nullptr && p.residual == nullptr &&
           p.ldkv >= 2 * (int64_t)p.n && p.ldkv % 8 == 0 && ((uintptr_t)p.kv & 15) == 0 && p.ldc % 8 == 0 &&
           (int64_t)p.ctx_len * p.ldkv * 2 <= 0x7FFFFFFF &&  // V-row transfer offsets are 32-bit
           ((uintptr_t)p.c & 15) == 0 && (int64_t)(p.m / 64) * (p.n / 128) <= 0x7FFFFFFF;
}

hipError_t launch_q_cross_attention(const LinearParams& params_in, bool w_fp8, int compute_units, hipStream_t stream) {
    LinearParams p = params_in;
    const bool a_fp8 = p.a_scale != nullptr;
    if (!q_cross_attention_supported(p, w_fp8, compute_units) || (a_fp8 && !w_fp8)) return hipErrorInvalidValue;
    // 64 x 128 tiles in row-major task order; 65-80 keys are three 32-key
    // groups, the last holding at most 16.
    p.m_blocks = p.m / 64;
    p.n_blocks = p.n / kBN;
    p.group_m = 1;
    const dim3 grid((unsigned)((int64_t)p.m_blocks * p.n_blocks)), block(256);
    const bool nt = (int64_t)p.m * p.n * 2 >= kStreamOutBytes;
#define SDXL_QX(WF, AF)                                                                                              \
    do {                                                                                                             \
        if (nt) hipLaunchKernelGGL((linear_kernel<WF, AF, 1, 2, 2, true, 2, 3, true>), grid, block, 0, stream, p);  \
        else hipLaunchKernelGGL((linear_kernel<WF, AF, 1, 2, 2, false, 2, 3, true>), grid, block, 0, stream, p);    \
    } while (0)
    if (a_fp8) SDXL_QX(true, true);
    else if (w_fp8) SDXL_QX(true, false);
    else SDXL_QX(false, false);
#undef SDXL_QX
    return hipGetLastError();
}

bool ln_linear_supported(const LnLinearParams& p) {
    return (p.k == 640 || p.k == 1280) && p.m > 0 && p.n >= 128 && p.n % 128 == 0 && p.ldx % 8 == 0 && ((uintptr_t)p.x & 15) == 0 &&
           ((uintptr_t)p.gamma & 15) == 0 && ((uintptr_t)p.beta & 15) == 0 && p.ldw % 16 == 0 &&
           ((uintptr_t)p.w & 15) == 0 && p.w_scale != nullptr && ((uintptr_t)p.w_scale & 3) == 0 &&
           (p.bias == nullptr || ((uintptr_t)p.bias & 1) == 0) && p.ldc % 4 == 0 && ((uintptr_t)p.c & 7) == 0 &&
           p.ldw * 128 <= 0x7FFFFFFF &&  // 32-bit transfer offsets
           (int64_t)(p.m - 1) * p.ldc + p.n <= 0x7FFFFFFF;  // 32-bit output offsets
}

// Work split of the fused LayerNorm projection: one workgroup per CU (144-152
// KiB of LDS), row blocks of 64, and the output columns split so that the
// grid fills the CUs once (at most ln_linear_max_cols columns per workgroup).
// Every workgroup of a row block normalises its 64 rows.
static void ln_linear_split(LnLinearParams& p, int compute_units) {
    const int cus = compute_units > 0 ? compute_units : 256;
    const int max_cols = p.k > 640 ? ln_linear_max_cols<1280>() : ln_linear_max_cols<640>();
    p.m_blocks = (p.m + 63) / 64;
    p.chunks = p.n / 128;
    const int min_split = (p.chunks * 128 + max_cols - 1) / max_cols;
    const int fill = p.m_blocks >= cus ? 1 : cus / p.m_blocks;
    p.n_split = std::min(p.chunks, std::max(min_split, fill));
}

bool ln_linear_preferred(const LnLinearParams& params, int compute_units) {
    if (!ln_linear_supported(params)) return false;
    LnLinearParams p = params;
    ln_linear_split(p, compute_units);
    return p.n_split <= 2;
}

hipError_t launch_ln_linear(const LnLinearParams& params_in, int compute_units, hipStream_t stream) {
    LnLinearParams p = params_in;
    if (!ln_linear_supported(p)) return hipErrorInvalidValue;
    ln_linear_split(p, compute_units);
    const int64_t tasks = (int64_t)p.m_blocks * p.n_split;
    if (tasks > 0x7FFFFFFF) return hipErrorInvalidValue;
    const dim3 grid((unsigned)tasks), block(512);
    const bool nt = (int64_t)p.m * p.n * 2 >= kStreamOutBytes;
#define SDXL_LNL(K)                                                                                       \
    do {                                                                                                  \
        if (p.a_fp8) {                                                                                    \
            if (nt) hipLaunchKernelGGL((ln_linear_kernel<K, true, true>), grid, block, 0, stream, p);    \
            else hipLaunchKernelGGL((ln_linear_kernel<K, true, false>), grid, block, 0, stream, p);      \
        } else {                                                                                          \
            if (nt) hipLaunchKernelGGL((ln_linear_kernel<K, false, true>), grid, block, 0, stream, p);   \
            else hipLaunchKernelGGL((ln_linear_kernel<K, false, false>), grid, block, 0, stream, p);     \
        }                                                                                                 \
    } while (0)
    if (p.k == 640) SDXL_LNL(640);
    else SDXL_LNL(1280);
#undef SDXL_LNL
    return hipGetLastError();
}

hipError_t launch_layer_norm(const LayerNormParams& params_in, hipStream_t stream) {
    LayerNormParams p = params_in;
    if (p.rows == 0) return hipSuccess;
    if (p.width % 2 != 0 || p.width <= 0 || p.width > 128 * kLnMaxPer) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((p.rows + 3) / 4)), block(256);
    const bool e4m3 = p.y_scale != nullptr;
    const bool nt = p.rows * p.width * (e4m3 ? 1 : 2) >= kStreamOutBytes;  // non-temporal stores for large outputs
    // 16-byte form: width % 8 == 0, 16-byte aligned input rows, 16-byte (fp16)
    // or 8-byte (E4M3) aligned output rows. Measured: fp16 [2048, 1280] 4.9 ->
    // 4.0 us, [8192, 640] unchanged; E4M3 [2048, 1280] 4.7 -> 4.3 us,
    // [1024, 2048] 4.5 -> 4.1 us, but width 640 (80 chunks: a quarter of the
    // lanes take two) 7.3 -> 7.6 us, so E4M3 rows narrower than 1024 keep the
    // pair kernel.
    // Four rows per wave (the form the fused LayerNorm projection shares) for
    // fp16 output at widths 128 .. 640 in steps of 128: configs[3]'s [8192, 640]
    // 5.65 -> 4.45 us (every lane busy: 80 chunks over 64 lanes left three
    // quarters of them idle in the second pass); at width 1280 (160 VGPRs,
    // occupancy 3) it measured 4.7 against 4.1-4.3 us, so wider rows keep the
    // 16-byte kernel below.
    if (!e4m3 && p.width % 128 == 0 && p.width <= 640 && p.ldx % 8 == 0 && ((uintptr_t)p.x & 15) == 0 &&
        ((uintptr_t)p.gamma & 15) == 0 && ((uintptr_t)p.beta & 15) == 0 && p.ldy % 8 == 0 &&
        ((uintptr_t)p.y & 15) == 0) {
        const dim3 g16((unsigned)((p.rows + 15) / 16));
        switch (p.width / 128) {
#define SDXL_LNR4(n)                                                                            \
    case n:                                                                                     \
        if (nt) hipLaunchKernelGGL((layer_norm_r4_kernel<n, true>), g16, block, 0, stream, p);  \
        else hipLaunchKernelGGL((layer_norm_r4_kernel<n, false>), g16, block, 0, stream, p);    \
        break;
            SDXL_LNR4(1) SDXL_LNR4(2) SDXL_LNR4(3) SDXL_LNR4(4) SDXL_LNR4(5)
#undef SDXL_LNR4
        }
        return hipGetLastError();
    }
    // Two rows per wave (32 lanes per row) for fp16 widths 768 .. 1280 in steps of
    // 256 (the level-2 rows).
    if (!e4m3 && p.width % 256 == 0 && p.width > 640 && p.width <= 1280 && p.ldx % 8 == 0 &&
        ((uintptr_t)p.x & 15) == 0 && ((uintptr_t)p.gamma & 15) == 0 && ((uintptr_t)p.beta & 15) == 0 &&
        p.ldy % 8 == 0 && ((uintptr_t)p.y & 15) == 0) {
        const dim3 g8((unsigned)((p.rows + 7) / 8));
        switch (p.width / 256) {
#define SDXL_LNR2(n)                                                                            \
    case n:                                                                                     \
        if (nt) hipLaunchKernelGGL((layer_norm_r2_kernel<n, true>), g8, block, 0, stream, p);   \
        else hipLaunchKernelGGL((layer_norm_r2_kernel<n, false>), g8, block, 0, stream, p);     \
        break;
            SDXL_LNR2(3) SDXL_LNR2(4) SDXL_LNR2(5)
#undef SDXL_LNR2
        }
        return hipGetLastError();
    }
    if (e4m3 && p.width % 256 == 0 && p.width > 640 && p.width <= 1280 && p.ldx % 8 == 0 &&
        ((uintptr_t)p.x & 15) == 0 && ((uintptr_t)p.gamma & 15) == 0 && ((uintptr_t)p.beta & 15) == 0 &&
        p.ldy % 8 == 0 && ((uintptr_t)p.y & 7) == 0) {
        const dim3 g8((unsigned)((p.rows + 7) / 8));
        switch (p.width / 256) {
#define SDXL_LNR2E(n)                                                                               \
    case n:                                                                                         \
        if (nt) hipLaunchKernelGGL((layer_norm_r2_e4m3_kernel<n, true>), g8, block, 0, stream, p);  \
        else hipLaunchKernelGGL((layer_norm_r2_e4m3_kernel<n, false>), g8, block, 0, stream, p);    \
        break;
            SDXL_LNR2E(3) SDXL_LNR2E(4) SDXL_LNR2E(5)
#undef SDXL_LNR2E
        }
        return hipGetLastError();
    }
    // E4M3 rows of widths 128 .. 640 in the same four-rows-per-wave form (the
    // fused E4M3 LayerNorm projection shares its code).
    if (e4m3 && p.width % 128 == 0 && p.width <= 640 && p.ldx % 8 == 0 && ((uintptr_t)p.x & 15) == 0 &&
        ((uintptr_t)p.gamma & 15) == 0 && ((uintptr_t)p.beta & 15) == 0 && p.ldy % 8 == 0 &&
        ((uintptr_t)p.y & 7) == 0) {
        const dim3 g16((unsigned)((p.rows + 15) / 16));
        switch (p.width / 128) {
#define SDXL_LNR4E(n)                                                                                \
    case n:                                                                                          \
        if (nt) hipLaunchKernelGGL((layer_norm_r4_e4m3_kernel<n, true>), g16, block, 0, stream, p);  \
        else hipLaunchKernelGGL((layer_norm_r4_e4m3_kernel<n, false>), g16, block, 0, stream, p);    \
        break;
            SDXL_LNR4E(1) SDXL_LNR4E(2) SDXL_LNR4E(3) SDXL_LNR4E(4) SDXL_LNR4E(5)
#undef SDXL_LNR4E
        }
        return hipGetLastError();
    }
    const bool v8 = p.width % 8 == 0 && p.ldx % 8 == 0 && ((uintptr_t)p.x & 15) == 0 &&
                    ((uintptr_t)p.gamma & 15) == 0 && ((uintptr_t)p.beta & 15) == 0 &&
                    (e4m3 ? p.width >= 1024 && p.ldy % 8 == 0 && ((uintptr_t)p.y & 7) == 0
                          : p.ldy % 8 == 0 && ((uintptr_t)p.y & 15) == 0);
    if (v8) {
        switch ((p.width + 511) / 512) {
#define SDXL_LN8(n)                                                                                   \
    if (e4m3 && nt) hipLaunchKernelGGL((layer_norm_v8_kernel<n, true, true>), grid, block, 0, stream, p);       \
    else if (e4m3) hipLaunchKernelGGL((layer_norm_v8_kernel<n, false, true>), grid, block, 0, stream, p);      \
    else if (nt) hipLaunchKernelGGL((layer_norm_v8_kernel<n, true, false>), grid, block, 0, stream, p);        \
    else hipLaunchKernelGGL((layer_norm_v8_kernel<n, false, false>), grid, block, 0, stream, p);
        case 1: SDXL_LN8(1) break;
        case 2: SDXL_LN8(2) break;
        case 3: SDXL_LN8(3) break;
        default: SDXL_LN8(4) break;
#undef SDXL_LN8
        }
        return hipGetLastError();
    }
    switch ((p.width + 127) / 128) {
#define SDXL_LN_CASE(n)                                                                   \
    case n:                                                                               \
        if (e4m3 && nt) hipLaunchKernelGGL((layer_norm_kernel<n, true, true>), grid, block, 0, stream, p);   \
        else if (e4m3) hipLaunchKernelGGL((layer_norm_kernel<n, true, false>), grid, block, 0, stream, p);   \
        else if (nt) hipLaunchKernelGGL((layer_norm_kernel<n, false, true>), grid, block, 0, stream, p);     \
        else hipLaunchKernelGGL((layer_norm_kernel<n, false, false>), grid, block, 0, stream, p);           \
        break;
        SDXL_LN_CASE(1) SDXL_LN_CASE(2) SDXL_LN_CASE(3) SDXL_LN_CASE(4) SDXL_LN_CASE(5) SDXL_LN_CASE(6)
        SDXL_LN_CASE(7) SDXL_LN_CASE(8) SDXL_LN_CASE(9) SDXL_LN_CASE(10) SDXL_LN_CASE(11) SDXL_LN_CASE(12)
        SDXL_LN_CASE(13) SDXL_LN_CASE(14) SDXL_LN_CASE(15) SDXL_LN_CASE(16)
#undef SDXL_LN_CASE
    }
    return hipGetLastError();
}

hipError_t launch_quantize_e4m3_rows(const QuantizeParams& p, hipStream_t stream) {
    if (p.rows == 0) return hipSuccess;
    const dim3 grid((unsigned)((p.rows + 3) / 4)), block(256);
    hipLaunchKernelGGL(quantize_e4m3_rows_kernel, grid, block, 0, stream, p);
    return hipGetLastError();
}

}  // namespace sdxl_hip

// K-split projection kernel for fp16 weights (the level-2 output projections
// of the UNet attention sublayers, 2048 x 1280 x 1280 + bias + residual,
// src/cuda/unet.cpp:114-118, :128-131, which the reference runs through
// cuBLASLt, src/cuda/ops_blas.cpp:244-386). Built on its own because its 160 fp32 accumulators per wave stay
// in the accumulation registers: with the MFMA results forced into the
// architectural VGPRs (the flag the other sublayer kernels build with) the
// compiler shuffles them between the two register files on every K stage.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sublayer_device.hpp"
#include "sublayer_kernels.hpp"

namespace sdxl_hip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;

// K-split projection for fp16 weights: one workgroup = 4 waves = a
// (32 kMT) x (32 kNT) output tile (64 x 160: the level-2 projections cut
// into exactly one tile per CU of a 256-CU device). Every
// 64-deep K stage of the tile (A rows, then W rows, 128-byte swizzled rows as
// linear_kernel stages them) is staged once, and wave w takes the 16-deep
// slice w of every stage for the whole tile: each wave reads each of its
// kMT + kNT operands once per stage for kMT kNT MFMAs (a 2 x 2 arrangement
// of 32 x 64 wave blocks reads 3 per 2). The operands of stage s are read
// while the MFMAs of stage s - 1 run (two register sets), and the next
// stage's transfers are issued between those MFMAs. The four partial tiles
// are summed through LDS in a fixed order, ((p0 + p1) + p2) + p3, and the
// epilogue (scale, bias, residual, one rounding to fp16) is linear_kernel's,
// with 16-byte residual loads and output stores.
template <int kMT, int kNT, int kRing, bool kNt>
__global__ __launch_bounds__(256, 1) void linear_ksplit_kernel(LinearParams p) {
    constexpr int kBMt = 32 * kMT, kBNt = 32 * kNT;
    constexpr int kStageBytes = (kBMt + kBNt) * kRowBytes;
    constexpr int kXfers = (kBMt + kBNt) / 8 / 4;  // 1-KiB transfers per wave and stage
    static_assert(kXfers == kMT + kNT, "every transfer of a stage has a wave");
    constexpr int kPartRow = kBNt * 4;           // bytes of one partial row (fp32)
    constexpr int kPartBytes = 32 * kPartRow;    // one wave's partial m-tile
    constexpr int kSmemBytes = kRing * kStageBytes > 4 * kMT * kPartBytes ? kRing * kStageBytes : 4 * kMT * kPartBytes;
    static_assert(kSmemBytes <= 160 * 1024, "LDS of one CU");
    __shared__ __attribute__((aligned(16))) char smem_raw[kSmemBytes];  // the stages, then the partials
    auto smem = [&](int st) __attribute__((always_inline)) { return smem_raw + st * kStageBytes; };

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hf = lane >> 5, col = lane & 31;

    // tasks: as linear_kernel (contiguous range per XCD, groups of group_m m blocks)
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
    const int64_t lda_b = p.lda * 2, ldw_b = p.ldw * 2;
    const char* abase = (const char*)p.a + (int64_t)m0 * lda_b;
    const char* wbase = (const char*)p.w + (int64_t)n0 * ldw_b;
    const int a_rows = p.m - 1 - m0, w_rows = p.n - 1 - n0;

    // transfers of the wave in every stage: A row blocks kMT wave + j (j <
    // kMT) and W row blocks kNT wave + j - kMT (8 rows of 128 bytes each; lane
    // l takes row 8 blk + l / 8 and global chunk (l % 8) ^ swz(row), its slot's
    // chunk); rows past the end re-read the last row. The per-lane offsets do
    // not depend on the stage.
    uint32_t voff[kXfers];
#pragma unroll
    for (int j = 0; j < kXfers; ++j) {
        const bool is_a = j < kMT;
        const int row = 8 * (is_a ? kMT * wave + j : kNT * wave + j - kMT) + (lane >> 3);
        voff[j] = (uint32_t)(min(row, is_a ? a_rows : w_rows) * (is_a ? lda_b : ldw_b)) +
                  (uint32_t)(((lane & 7) ^ swz(row)) << 4);
    }
    auto issue = [&](int st, int j) __attribute__((always_inline)) {
        const bool is_a = j < kMT;
        const int blk = is_a ? kMT * wave + j : kBMt / 8 + kNT * wave + j - kMT;
        lds_dma16((is_a ? abase : wbase) + st * kBK * 2, voff[j], lds_addr(smem(st % kRing) + blk * 8 * kRowBytes));
    };

    f32x16 acc[kNT][kMT];
#pragma unroll
    for (int j = 0; j < kNT; ++j)
#pragma unroll
        for (int i = 0; i < kMT; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;
    // the wave's 16-byte chunk of every row it reads: K columns 16 wave + 8 hf
    int a_off[kMT], w_off[kNT];
#pragma unroll
    for (int i = 0; i < kMT; ++i) {
        const int r = 32 * i + col;
        a_off[i] = r * kRowBytes + (((2 * wave + hf) ^ swz(r)) << 4);
    }
#pragma unroll
    for (int j = 0; j < kNT; ++j) {
        const int r = kBMt + 32 * j + col;  // W rows follow the A rows; swz depends on r % 16 only
        w_off[j] = r * kRowBytes + (((2 * wave + hf) ^ swz(r)) << 4);
    }
    i16x8 aop[2][kMT], wop[2][kNT];
    auto read_ops = [&](int s, int set) __attribute__((always_inline)) {
        const char* b = smem(s % kRing);
#pragma unroll
        for (int j = 0; j < kNT; ++j) wop[set][j] = *(const lds_i16x8*)(b + w_off[j]);
#pragma unroll
        for (int i = 0; i < kMT; ++i) aop[set][i] = *(const lds_i16x8*)(b + a_off[i]);
    };
    // MFMAs of the operand set, with the transfers of stage `next` (if any)
    // issued one after each MFMA
    auto mfmas = [&](int set, int next) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < kNT * kMT; ++q) {
            const int j = q / kMT, i = q % kMT;
            acc[j][i] = mfma32(wop[set][j], aop[set][i], acc[j][i]);
            if (q < kXfers && next >= 0) issue(next, q);
        }
        if constexpr (kXfers > kNT * kMT) {
#pragma unroll
            for (int q = kNT * kMT; q < kXfers; ++q)
                if (next >= 0) issue(next, q);
        }
    };
    auto wait_stage = [&](int s) __attribute__((always_inline)) {
        const int later = min(n_stages - 1 - s, kRing - 2);
        if constexpr (kRing >= 4) {
            if (later >= 2) wait_vmem<2 * kXfers>();
            else if (later == 1) wait_vmem<kXfers>();
            else wait_vmem<0>();
        } else if constexpr (kRing == 3) {
            if (later >= 1) wait_vmem<kXfers>();
            else wait_vmem<0>();
        } else {
            wait_vmem<0>();
        }
    };

    // epilogue operands, requested first so that their latency hides under
    // the loop. Wave w finishes rows 8w .. 8w + 7 of both 32-row m-tiles:
    // lane l takes row r = 4 (l / 16) + (l / 4) % 4 of those 16 (m-tile r / 8,
    // row 8w + r % 8) and, in item it (it < kIt), the 8 columns 8 dc .. 8 dc +
    // 7 with dc = 4 it + l % 4: residual loads and output stores are 16 bytes
    // per lane, 64 contiguous bytes per row, and the partial reads of every 16
    // lanes (4 rows x 4 column groups) hit 16 distinct bank groups.
    static_assert(kMT == 2, "16 rows per wave in the epilogue");
    constexpr int kDC = 4 * kNT;                 // 8-column groups per row
    constexpr int kIt = kDC / 4;
    const int er = 4 * (lane >> 4) + ((lane >> 2) & 3);
    const int ei = er >> 3, erow = 8 * wave + (er & 7);
    f32x4 e_scale[kIt][2];
    f16x8 e_bias[kIt], res[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int dc = 4 * it + (lane & 3);
        const int en = min(n0 + 8 * dc, p.n - 8);
        const int m = min(m0 + 32 * ei + erow, p.m - 1);
        if (p.w_scale != nullptr) {
            e_scale[it][0] = *(const f32x4*)(p.w_scale + en);
            e_scale[it][1] = *(const f32x4*)(p.w_scale + en + 4);
        } else {
            e_scale[it][0] = e_scale[it][1] = f32x4{1.0f, 1.0f, 1.0f, 1.0f};
        }
        e_bias[it] = p.bias != nullptr ? *(const f16x8*)((const _Float16*)p.bias + en) : f16x8{};
        res[it] = p.residual != nullptr ? *(const f16x8*)((const _Float16*)p.residual + (int64_t)m * p.ldr + en) : f16x8{};
    }

#pragma unroll
    for (int st = 0; st < kRing - 1; ++st)
        if (st < n_stages)
#pragma unroll
            for (int j = 0; j < kXfers; ++j) issue(st, j);
    // step s: stage s landed for every wave (and every wave's reads of stage
    // s - 1 are done, so its buffer takes stage s + kRing - 1); read stage s's
    // operands into set s & 1, then run stage s - 1's MFMAs with the next
    // stage's transfers between them. Steps go in pairs so that the sets are
    // fixed registers.
    auto land = [&](int s) __attribute__((always_inline)) {
        wait_stage(s);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };
    auto step = [&](int s, int set) __attribute__((always_inline)) {
        land(s);
        read_ops(s, set);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(set ^ 1, s + kRing - 1 < n_stages ? s + kRing - 1 : -1);
        __builtin_amdgcn_sched_barrier(0);
    };
    if (n_stages > 0) {
        land(0);
        read_ops(0, 0);
        if (kRing - 1 < n_stages)
#pragma unroll
            for (int q = 0; q < kXfers; ++q) issue(kRing - 1, q);
    }
    int s = 1;
    for (; s + 1 < n_stages; s += 2) {
        step(s, 1);
        step(s + 1, 0);
    }
    if (s < n_stages) {
        step(s, 1);
        mfmas(1, -1);
    } else if (n_stages > 0) {
        mfmas(0, -1);
    }

    // ---- the four partial tiles through LDS (all of them at once: 4 x 40 KiB
    // per 32-row m-tile, the whole 160 KiB). Wave w parks its partial
    // row-major, 16-byte chunk c of row r of m-tile i at c ^ sw(i, r) with
    // sw = ((r >> 1) & 7) ^ 4i: conflict-free for the 16 rows of a parking
    // write and for the readers' 4 rows (two m-tiles) x 4 chunk pairs;
    // acc[j][i][4u + q] is row 32i + col, column 32j + 8u + 4hf + q of the tile.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();  // every wave is done with the stage buffers
    {
#pragma unroll
        for (int i = 0; i < kMT; ++i) {
            char* mine = smem_raw + (i * 4 + wave) * kPartBytes;
            const int psw = ((col >> 1) & 7) ^ (4 * i);
#pragma unroll
            for (int j = 0; j < kNT; ++j)
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int c = 8 * j + 2 * u + hf;
                    *(lds_f32x4*)(mine + col * kPartRow + ((c ^ psw) << 4)) =
                        f32x4{acc[j][i][4 * u], acc[j][i][4 * u + 1], acc[j][i][4 * u + 2], acc[j][i][4 * u + 3]};
                }
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int dc = 4 * it + (lane & 3);
        const int m = m0 + 32 * ei + erow, en = n0 + 8 * dc;
        const char* part = smem_raw + ei * 4 * kPartBytes + erow * kPartRow;
        const int sw = ((erow >> 1) & 7) ^ (4 * ei);
        f32x4 a[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int off = ((2 * dc + h) ^ sw) << 4;
            const f32x4 p0 = *(const lds_f32x4*)(part + off);
            const f32x4 p1 = *(const lds_f32x4*)(part + kPartBytes + off);
            const f32x4 p2 = *(const lds_f32x4*)(part + 2 * kPartBytes + off);
            const f32x4 p3 = *(const lds_f32x4*)(part + 3 * kPartBytes + off);
            a[h] = ((p0 + p1) + p2) + p3;
        }
        if (m < p.m && en < p.n) {
            f16x8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = a[e >> 2][e & 3] * e_scale[it][e >> 2][e & 3] + (float)e_bias[it][e] + (float)res[it][e];
                o[e] = (_Float16)v;
            }
            store_out<kNt>(o, (f16x8*)((_Float16*)p.c + (int64_t)m * p.ldc + en));
        }
    }
}

}  // namespace

bool linear_ksplit_supported(const LinearParams& p, bool w_fp8, int compute_units) {
    // output projections only (a residual): projections without one (the
    // query projection) keep linear_kernel's accumulation order, which the
    // fused query projection + cross-attention reproduces bit for bit
    if (w_fp8 || p.a_scale != nullptr || p.residual == nullptr || compute_units <= 0 || p.m <= 0 || p.n <= 0)
        return false;
    // one round of 64 x 160 tiles that fills at least 90 % of the CUs (the
    // level-2 projections, 2048 x 1280: 256 tiles); with fewer tiles, or
    // several per CU, the 64 x 128 kernels measured faster
    const int64_t tasks = (int64_t)((p.m + 63) / 64) * ((p.n + 159) / 160);
    if (tasks > compute_units || tasks * 10 < (int64_t)compute_units * 9) return false;
    auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
    return p.n % 8 == 0 && p.k % kBK == 0 && p.k > 0 && p.ldc % 8 == 0 && al16(p.c) && p.lda % 8 == 0 &&
           p.ldw % 8 == 0 && al16(p.a) && al16(p.w) && p.ldr % 8 == 0 && al16(p.residual) &&
           (p.bias == nullptr || al16(p.bias)) && (p.w_scale == nullptr || al16(p.w_scale)) &&
           (int64_t)(p.m - 1) * p.lda * 2 + p.k * 2 <= 0xFFFFFFFFll && (int64_t)(p.n - 1) * p.ldw * 2 + p.k * 2 <= 0xFFFFFFFFll;
}

hipError_t launch_linear_ksplit(const LinearParams& params_in, hipStream_t stream) {
    LinearParams p = params_in;
    p.m_blocks = (p.m + 63) / 64;
    p.n_blocks = (p.n + 159) / 160;
    // an XCD's 32 workgroups take 8 m blocks x 4 n blocks (2048 x 1280: 1.3 MB
    // of A rows and 1.6 MB of W rows per XCD's L2)
    p.group_m = p.m_blocks < 8 ? p.m_blocks : 8;
    const dim3 grid((unsigned)((int64_t)p.m_blocks * p.n_blocks)), block(256);
    if ((int64_t)p.m * p.n * 2 >= kStreamOutBytes)
        hipLaunchKernelGGL((linear_ksplit_kernel<2, 5, 4, true>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((linear_ksplit_kernel<2, 5, 4, false>), grid, block, 0, stream, p);
    return hipGetLastError();
}

}  // namespace sdxl_hip

// Device helpers shared by the sublayer kernels (sublayer.hip,
// linear_ksplit.hip): vector types, the 128-byte row swizzle, the fp16 and fp8
// MFMAs, the HBM -> LDS transfer, E4M3 decode, output stores and vmcnt waits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sdxl_hip {
namespace {

typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
struct u32x4x2 {
    u32x4 lo, hi;
};
typedef __attribute__((address_space(3))) i16x8 lds_i16x8;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;
typedef __attribute__((address_space(3))) char lds_char;

constexpr int kBN = 128, kBK = 64;
constexpr int kRowBytes = kBK * 2;              // 128: one fp16 tile row

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
        "s_nop 4\n\t"
        "global_load_lds_dwordx4 %0, %1"
        :
        : "v"(voff), "s"(base), "{m0}"(lds));
}

// Four E4M3 codes -> four fp16 values (exact).
__device__ __forceinline__ uint2 e4m3x4_to_f16(uint32_t x) {
    const f16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, false);
    const f16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, true);
    return uint2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}

// s_waitcnt vmcnt(n) (lgkmcnt(0), expcnt untouched) for a compile-time n < 64.
// Output store: non-temporal (streams to memory instead of staying in L2)
// for large outputs, else ordinary. A compile-time choice: with a run-time
// flag the compiler merges both branches into one ordinary store.
template <bool kNt, typename T>
__device__ __forceinline__ void store_out(T v, T* ptr) {
    if constexpr (kNt) __builtin_nontemporal_store(v, ptr);
    else *ptr = v;
}

template <int N>
__device__ __forceinline__ void wait_vmem() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70);
}

// E4M3 x E4M3 MFMA, 32 x 32 x 64: each lane supplies 32 consecutive K bytes of
// its row of A and of B. The hardware's K order inside an operand is the same
// for A and B, so any fixed byte order that both operands share gives the
// same sum.
__device__ __forceinline__ f32x16 mfma32_fp8(i32x8 a, i32x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

}  // namespace
}  // namespace sdxl_hip

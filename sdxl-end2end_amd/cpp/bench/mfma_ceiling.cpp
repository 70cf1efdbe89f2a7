// MFMA throughput ceiling of the device on random vs zero operands.
//
// Four independent v_mfma_f32_32x32x16_f16 chains per wave, operands held in
// registers (no memory traffic in the loop), 8 workgroups of 4 waves per CU.
// The instruction stream is identical for both operand sets; the difference
// in throughput is the clock the device sustains under the power drawn by
// toggling operands. The attention kernel's achieved rate is read against the
// random-operand figure.
//
// Usage: bin/sdxl_hip_mfma_ceiling [iterations]
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define CHECK(x)                                                                          \
    do {                                                                                  \
        hipError_t e_ = (x);                                                              \
        if (e_ != hipSuccess) {                                                           \
            std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));           \
            std::exit(1);                                                                 \
        }                                                                                 \
    } while (0)

__global__ __launch_bounds__(256) void mfma_loop(const f16x8* in, float* out, int iters, int zero_b) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    const f16x8 a = in[t & 4095];
    f16x8 b = in[(t * 7 + 3) & 4095];
    if (zero_b) b = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int i = 0; i < iters; ++i) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, b, c3, 0, 0, 0);
    }
    float s = 0.0f;
    for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
    out[t] = s;
}

}  // namespace

int main(int argc, char** argv) {
    const int iters = argc > 1 ? std::atoi(argv[1]) : 4000;
    hipDeviceProp_t prop;
    CHECK(hipGetDeviceProperties(&prop, 0));
    const int n = 4096;
    std::vector<_Float16> host(n * 8);
    unsigned s = 1;
    for (auto& x : host) {  // uniform in [-2, 2)
        s = s * 1664525u + 1013904223u;
        x = (_Float16)((float)((s >> 9) % 2000) / 500.0f - 2.0f);
    }
    f16x8* in;
    float* out;
    const int blocks = prop.multiProcessorCount * 8;
    CHECK(hipMalloc(&in, n * sizeof(f16x8)));
    CHECK(hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)));
    CHECK(hipMemcpy(in, host.data(), n * sizeof(f16x8), hipMemcpyHostToDevice));
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    const double flops = (double)blocks * 4 * iters * 4 * 2.0 * 32 * 32 * 16;
    for (int zero = 0; zero < 2; ++zero) {
        hipLaunchKernelGGL(mfma_loop, dim3(blocks), dim3(256), 0, 0, in, out, iters, zero);  // warm-up
        CHECK(hipDeviceSynchronize());
        float best = 1e30f;
        for (int rep = 0; rep < 5; ++rep) {
            CHECK(hipEventRecord(e0));
            hipLaunchKernelGGL(mfma_loop, dim3(blocks), dim3(256), 0, 0, in, out, iters, zero);
            CHECK(hipEventRecord(e1));
            CHECK(hipEventSynchronize(e1));
            float ms;
            CHECK(hipEventElapsedTime(&ms, e0, e1));
            best = ms < best ? ms : best;
        }
        std::printf("{\"operands\": \"%s\", \"cus\": %d, \"ms\": %.4f, \"tflops\": %.1f}\n",
                    zero ? "zero_b" : "random", prop.multiProcessorCount, best, flops / best / 1e9);
    }
    CHECK(hipFree(in));
    CHECK(hipFree(out));
    return 0;
}

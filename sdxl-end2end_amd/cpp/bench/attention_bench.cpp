// Attention micro-benchmark with the reference's command line
// (src/attention_bench.cu:103-146, shapes in ATTENTION_BENCHMARK.bat):
//   sdxl_hip_attention_bench [q_seq=4096] [k_seq=q_seq] [heads=10] [batch=2] [iterations=10]
// Inputs are the reference's sinusoids (sin(i*f)/4, f = 0.0013/0.0017/0.0007,
// attention_bench.cu:19-30). Times the fused backend (flash-sm80 spelling) and
// wave-online, each with hipEvents around `iterations` calls after warm-up,
// and prints max-abs / RMS of fused vs wave-online, like the reference.
#include "sdxl_hip/ops.hpp"

#include <algorithm>
#include <cmath>
#include <iomanip>
#include <iostream>
#include <string>

namespace {

using namespace sdxl::hip;

FloatTensor make_input(std::size_t batch, std::size_t sequence, std::size_t width, float frequency) {
    FloatTensor t;
    t.shape = {batch, sequence, width};
    t.values.resize(batch * sequence * width);
    for (std::size_t i = 0; i < t.values.size(); ++i) t.values[i] = std::sin(static_cast<float>(i) * frequency) * 0.25F;
    return t;
}

struct Result {
    double milliseconds = 0.0;
    FloatTensor output;
};

Result run(AttentionBackend backend, const FloatTensor& q, const FloatTensor& k, const FloatTensor& v, std::size_t heads,
           int warmup, int iterations) {
    RuntimeOptions options;
    options.attention_backend = backend;
    Runtime runtime(options);
    Ops ops(runtime);
    auto qd = Tensor::from_host_f32(runtime, q), kd = Tensor::from_host_f32(runtime, k), vd = Tensor::from_host_f32(runtime, v);
    Tensor out = Tensor::allocate(runtime, q.shape, ScalarType::Float16);
    for (int i = 0; i < warmup; ++i) ops.attention_into(qd, kd, vd, heads, out);
    runtime.synchronize();
    hipEvent_t start = nullptr, stop = nullptr;
    SDXL_HIP_CHECK(hipEventCreate(&start));
    SDXL_HIP_CHECK(hipEventCreate(&stop));
    SDXL_HIP_CHECK(hipEventRecord(start, runtime.stream()));
    for (int i = 0; i < iterations; ++i) ops.attention_into(qd, kd, vd, heads, out);
    SDXL_HIP_CHECK(hipEventRecord(stop, runtime.stream()));
    SDXL_HIP_CHECK(hipEventSynchronize(stop));
    float ms = 0.0F;
    SDXL_HIP_CHECK(hipEventElapsedTime(&ms, start, stop));
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
    return {static_cast<double>(ms) / iterations, out.to_host_f32(runtime)};
}

}  // namespace

int main(int argc, char** argv) {
    try {
        const std::size_t q_seq = argc > 1 ? std::stoull(argv[1]) : 4096;
        const std::size_t k_seq = argc > 2 ? std::stoull(argv[2]) : q_seq;
        const std::size_t heads = argc > 3 ? std::stoull(argv[3]) : 10;
        const std::size_t batch = argc > 4 ? std::stoull(argv[4]) : 2;
        const int iterations = argc > 5 ? std::stoi(argv[5]) : 10;
        const std::size_t width = heads * 64;
        const auto q = make_input(batch, q_seq, width, 0.0013F);
        const auto k = make_input(batch, k_seq, width, 0.0017F);
        const auto v = make_input(batch, k_seq, width, 0.0007F);
        const Result flash = run(AttentionBackend::FlashSM80, q, k, v, heads, 2, iterations);
        const Result warp = run(AttentionBackend::WarpOnline, q, k, v, heads, 1, std::max(1, std::min(iterations, 3)));
        double max_abs = 0.0, sq = 0.0;
        for (std::size_t i = 0; i < flash.output.values.size(); ++i) {
            const double d = static_cast<double>(flash.output.values[i]) - warp.output.values[i];
            max_abs = std::max(max_abs, std::fabs(d));
            sq += d * d;
        }
        const double rms = flash.output.values.empty() ? 0.0 : std::sqrt(sq / flash.output.values.size());
        const double flops = 4.0 * batch * heads * q_seq * k_seq * 64;
        std::cout << std::fixed << std::setprecision(3) << "shape B=" << batch << " Q=" << q_seq << " K=" << k_seq
                  << " H=" << heads << " D=64\n"
                  << "flash-gfx950: " << flash.milliseconds << " ms (" << flops / (flash.milliseconds * 1e9)
                  << " TFLOP/s)\n"
                  << "wave-online: " << warp.milliseconds << " ms\n"
                  << "flash vs wave: " << (warp.milliseconds / flash.milliseconds) << "x\n"
                  << std::setprecision(6) << "flash error: max_abs=" << max_abs << " rms=" << rms << "\n";
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "Error: " << e.what() << '\n';
        return 1;
    }
}

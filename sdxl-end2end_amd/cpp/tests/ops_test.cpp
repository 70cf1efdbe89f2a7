// CTest-style test of the sdxl_hip C++20 host API, mirroring the attention
// cases of the reference's tests/cuda/cuda_ops_test.cu:427-502 plus its
// host-side error paths (src/cuda/runtime.cpp:61-77, ops_kernels.cu:1914-1941).
//
//   sdxl_hip_ops_test              all cases (needs a GPU)
//   sdxl_hip_ops_test --host-only  cases that need no device
// Exit status 0 on success; the first failure throws and exits 1.
#include "sdxl_hip/ops.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <iostream>
#include <string>
#include <vector>

namespace {

using namespace sdxl::hip;

void require(bool condition, const std::string& what) {
    if (!condition) throw std::runtime_error("check failed: " + what);
}

void require_close(float actual, float expected, float tolerance, const std::string& what) {
    if (!(std::fabs(actual - expected) <= tolerance))
        throw std::runtime_error(what + ": expected " + std::to_string(expected) + " got " + std::to_string(actual));
}

template <typename F>
void require_throws(F&& fn, const std::string& message_part, const std::string& what) {
    try {
        fn();
    } catch (const HipError& e) {
        if (std::string(e.what()).find(message_part) == std::string::npos)
            throw std::runtime_error(what + ": wrong message: " + e.what());
        return;
    }
    throw std::runtime_error(what + ": no HipError thrown");
}

void host_cases() {
    require(parse_attention_backend("auto") == AttentionBackend::Auto, "auto");
    for (const char* s : {"cudnn", "cudnn-sdpa", "sdpa", "CUDNN"})
        require(parse_attention_backend(s) == AttentionBackend::CuDnnSDPA, s);
    for (const char* s : {"flash", "flash-sm80", "flash2", "flash-gfx950"})
        require(parse_attention_backend(s) == AttentionBackend::FlashSM80, s);
    for (const char* s : {"warp", "warp-online", "reference", "wave-online"})
        require(parse_attention_backend(s) == AttentionBackend::WarpOnline, s);
    require_throws([] { (void)parse_attention_backend("triton"); },
                   "attention backend must be auto, cudnn-sdpa, flash-sm80, or warp-online", "unknown backend");
    require(std::string(attention_backend_name(AttentionBackend::FlashSM80)) == "flash-sm80", "name");
    require(std::string(attention_backend_name(AttentionBackend::WarpOnline)) == "warp-online", "name");
    // host conversions used by Tensor::from_host_f32
    require(float_to_half(1.0F) == 0x3C00 && float_to_half(-2.0F) == 0xC000, "half");
    require(float_to_half(65520.0F) == 0x7C00 && float_to_half(1.0F + 1.0F / 2048.0F) == 0x3C00, "half rounding");
    require(half_to_float(0x0001) == std::ldexp(1.0F, -24), "half subnormal");
    require(float_to_bf16(1.0F) == 0x3F80 && bf16_to_float(0x3F80) == 1.0F, "bf16");
    std::cout << "host cases passed\n";
}

FloatTensor filled(std::vector<std::size_t> shape, const std::function<float(std::size_t)>& f) {
    FloatTensor t;
    t.shape = std::move(shape);
    std::size_t n = 1;
    for (auto d : t.shape) n *= d;
    t.values.resize(n);
    for (std::size_t i = 0; i < n; ++i) t.values[i] = f(i);
    return t;
}

void device_cases() {
    Runtime runtime;
    Ops ops(runtime);

    // cuda_ops_test.cu:427-439: q = k = 0, v rows 2 and 4 -> every output 3.0 (auto backend).
    FloatTensor q = filled({1, 2, 64}, [](std::size_t) { return 0.0F; });
    FloatTensor v = filled({1, 2, 64}, [](std::size_t i) { return i < 64 ? 2.0F : 4.0F; });
    auto qd = Tensor::from_host_f32(runtime, q);
    auto kd = Tensor::from_host_f32(runtime, q);
    auto vd = Tensor::from_host_f32(runtime, v);
    for (float x : ops.attention(qd, kd, vd, 1, false).to_host_f32(runtime).values) require_close(x, 3.0F, 0.02F, "attention");

    // cuda_ops_test.cu:441-482: flash vs warp-online on [1, 64, 2x64], per element 0.04.
    const auto qc = filled({1, 64, 128}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.013F) * 0.25F; });
    const auto kc = filled({1, 64, 128}, [](std::size_t i) { return std::cos(static_cast<float>(i) * 0.017F) * 0.25F; });
    const auto vc = filled({1, 64, 128}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.007F); });
    RuntimeOptions flash_options;
    flash_options.attention_backend = AttentionBackend::FlashSM80;
    flash_options.profile = true;
    Runtime flash_runtime(flash_options);
    Ops flash_ops(flash_runtime);
    const auto flash = flash_ops.attention(Tensor::from_host_f32(flash_runtime, qc), Tensor::from_host_f32(flash_runtime, kc),
                                           Tensor::from_host_f32(flash_runtime, vc), 2, false)
                           .to_host_f32(flash_runtime);
    RuntimeOptions warp_options;
    warp_options.attention_backend = AttentionBackend::WarpOnline;
    Runtime warp_runtime(warp_options);
    Ops warp_ops(warp_runtime);
    const auto warp = warp_ops.attention(Tensor::from_host_f32(warp_runtime, qc), Tensor::from_host_f32(warp_runtime, kc),
                                         Tensor::from_host_f32(warp_runtime, vc), 2, false)
                          .to_host_f32(warp_runtime);
    require(flash.values.size() == warp.values.size(), "flash/warp shape");
    for (std::size_t i = 0; i < flash.values.size(); ++i) require_close(flash.values[i], warp.values[i], 0.04F, "flash vs warp");
    // profile label grammar (ops_kernels.cu:1956-1961)
    const auto records = flash_runtime.profile_records();
    require(records.size() == 1 && records[0].label == "ops/attention/flash-sm80/q64_k64_h2_d64_full", "profile label");
    require(records[0].milliseconds >= 0.0F, "profile time");

    // cuda_ops_test.cu:484-502: FP32, D = 512 (VAE head), uniform case 3.0 +- 1e-3.
    FloatTensor qv = filled({1, 2, 512}, [](std::size_t) { return 0.0F; });
    FloatTensor vv = filled({1, 2, 512}, [](std::size_t i) { return i < 512 ? 2.0F : 4.0F; });
    const auto vae = ops.attention(Tensor::from_host_f32(runtime, qv, ScalarType::Float32),
                                   Tensor::from_host_f32(runtime, qv, ScalarType::Float32),
                                   Tensor::from_host_f32(runtime, vv, ScalarType::Float32), 1, false)
                         .to_host_f32(runtime);
    for (float x : vae.values) require_close(x, 3.0F, 1.0e-3F, "VAE FP32 attention");

    // causal + key mask through the fused backend: row 0 sees only key 0.
    const auto kq = filled({1, 5, 64}, [](std::size_t i) { return std::sin(static_cast<float>(i)); });
    const auto kv = filled({1, 5, 64}, [](std::size_t i) { return static_cast<float>(i / 64); });
    auto mask = Tensor::from_host_i32(runtime, {1, 5}, {1, 1, 0, 1, 1});
    const auto causal = flash_ops.attention(Tensor::from_host_f32(flash_runtime, kq), Tensor::from_host_f32(flash_runtime, kq),
                                            Tensor::from_host_f32(flash_runtime, kv), 1, true, &mask)
                            .to_host_f32(flash_runtime);
    for (std::size_t d = 0; d < 64; ++d) require_close(causal.values[d], 0.0F, 1e-3F, "causal row 0 = v row 0");

    // error paths (ops_kernels.cu:1914-1941)
    require_throws([&] { (void)ops.attention(qd, kd, Tensor::from_host_f32(runtime, filled({1, 3, 64}, [](std::size_t) { return 0.0F; })), 1); },
                   "CUDA attention mismatch", "value shape");
    require_throws([&] { (void)ops.attention(qd, kd, vd, 3); }, "CUDA attention mismatch", "heads");
    auto bad_mask = Tensor::from_host_i32(runtime, {1, 3}, {1, 1, 1});
    require_throws([&] { (void)ops.attention(qd, kd, vd, 1, false, &bad_mask); }, "key mask mismatch", "mask shape");
    RuntimeOptions cudnn_options;
    cudnn_options.attention_backend = AttentionBackend::CuDnnSDPA;
    Runtime cudnn_runtime(cudnn_options);
    Ops cudnn_ops(cudnn_runtime);
    auto good_mask = Tensor::from_host_i32(cudnn_runtime, {1, 2}, {1, 1});
    auto q2 = Tensor::from_host_f32(cudnn_runtime, q);
    auto v2 = Tensor::from_host_f32(cudnn_runtime, v);
    require_throws([&] { (void)cudnn_ops.attention(q2, q2, v2, 1, false, &good_mask); }, "cudnn-sdpa requires",
                   "cudnn-sdpa with mask");
    for (float x : cudnn_ops.attention(q2, q2, v2, 1).to_host_f32(cudnn_runtime).values)
        require_close(x, 3.0F, 0.02F, "cudnn-sdpa spelling runs the fused kernel");
    std::cout << "device cases passed\n";
}

}  // namespace

int main(int argc, char** argv) {
    try {
        host_cases();
        if (argc > 1 && std::strcmp(argv[1], "--host-only") == 0) return 0;
        device_cases();
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "FAILED: " << e.what() << '\n';
        return 1;
    }
}

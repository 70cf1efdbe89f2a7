// CTest-style test of the sdxl_hip C++20 host API, mirroring the attention
// cases of the reference's tests/cuda/cuda_ops_test.cu:427-502 plus its
// host-side error paths (src/cuda/runtime.cpp:61-77, ops_kernels.cu:1914-1941).
//
//   sdxl_hip_ops_test              all cases (needs a GPU)
//   sdxl_hip_ops_test --host-only  cases that need no device
// Exit status 0 on success; the first failure throws and exits 1.
#include "sdxl_hip/ops.hpp"

#include <algorithm>
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
    // E4M3 decode (src/unet.cpp:91-119): 1.0, max 448, smallest subnormal 2^-9, NaN code
    require(e4m3_to_float(0x38) == 1.0F && e4m3_to_float(0x7E) == 448.0F && e4m3_to_float(0xFE) == -448.0F, "e4m3");
    require(e4m3_to_float(0x01) == std::ldexp(1.0F, -9) && std::isnan(e4m3_to_float(0x7F)), "e4m3 edges");
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

// Host fp32 references of the sublayer operators (src/unet.cpp:202-263).
std::vector<float> host_layer_norm(const FloatTensor& x, std::size_t W) {
    std::vector<float> y(x.values.size());
    for (std::size_t r = 0; r < x.values.size() / W; ++r) {
        const float* s = x.values.data() + r * W;
        float mean = 0.0F, var = 0.0F;
        for (std::size_t i = 0; i < W; ++i) mean += s[i];
        mean /= static_cast<float>(W);
        for (std::size_t i = 0; i < W; ++i) var += (s[i] - mean) * (s[i] - mean);
        const float inv = 1.0F / std::sqrt(var / static_cast<float>(W) + 1.0e-5F);
        for (std::size_t i = 0; i < W; ++i) y[r * W + i] = (s[i] - mean) * inv;
    }
    return y;
}

std::vector<float> host_linear(const std::vector<float>& x, const std::vector<float>& w, std::size_t rows,
                               std::size_t n, std::size_t k) {
    std::vector<float> y(rows * n, 0.0F);
    for (std::size_t r = 0; r < rows; ++r)
        for (std::size_t o = 0; o < n; ++o) {
            float acc = 0.0F;
            for (std::size_t i = 0; i < k; ++i) acc += x[r * k + i] * w[o * k + i];
            y[r * n + o] = acc;
        }
    return y;
}

void sublayer_cases() {
    Runtime runtime;
    Ops ops(runtime);
    const std::size_t rows = 96, W = 128, N = 192;
    const auto x = filled({2, rows / 2, W}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.37F) * 2.0F; });
    const auto ones = filled({W}, [](std::size_t) { return 1.0F; });
    const auto zeros = filled({W}, [](std::size_t) { return 0.0F; });
    auto xd = Tensor::from_host_f32(runtime, x);
    const auto ln = ops.layer_norm(xd, Tensor::from_host_f32(runtime, ones), Tensor::from_host_f32(runtime, zeros))
                        .to_host_f32(runtime);
    const auto ln_ref = host_layer_norm(x, W);
    for (std::size_t i = 0; i < ln_ref.size(); ++i)
        require_close(ln.values[i], ln_ref[i], std::fabs(ln_ref[i]) * 1e-3F + 1e-4F, "layer_norm");

    const auto w = filled({N, W}, [](std::size_t i) { return std::cos(static_cast<float>(i) * 0.11F) * 0.05F; });
    auto wd = Tensor::from_host_f32(runtime, w);
    const auto lin = ops.linear(xd, wd).to_host_f32(runtime);
    const auto lin_ref = host_linear(x.values, Tensor::from_host_f32(runtime, w).to_host_f32(runtime).values, rows, N, W);
    for (std::size_t i = 0; i < lin_ref.size(); ++i)
        require_close(lin.values[i], lin_ref[i], std::fabs(lin_ref[i]) * 1e-3F + 1e-3F, "linear fp16");

    const auto packed = ops.pack_e4m3(wd);
    require(packed.type() == ScalarType::Float8E4M3 && packed.dequant_scale_count() == N, "pack_e4m3");
    auto scales = std::vector<float>(N);
    SDXL_HIP_CHECK(hipMemcpy(scales.data(), packed.dequant_scale_data(), N * 4, hipMemcpyDeviceToHost));
    auto deq = packed.to_host_f32(runtime).values;
    for (std::size_t o = 0; o < N; ++o)
        for (std::size_t i = 0; i < W; ++i) deq[o * W + i] *= scales[o];
    const auto lin8 = ops.linear(xd, packed).to_host_f32(runtime);
    const auto lin8_ref = host_linear(x.values, deq, rows, N, W);
    for (std::size_t i = 0; i < lin8_ref.size(); ++i)
        require_close(lin8.values[i], lin8_ref[i], std::fabs(lin8_ref[i]) * 1e-3F + 1e-3F, "linear e4m3");
    require_throws([&] { (void)ops.linear(xd, Tensor::from_host_f32(runtime, filled({N, 64}, [](std::size_t) { return 0.0F; }))); },
                   "linear feature mismatch", "linear shape");
    require_throws([&] { (void)ops.layer_norm(xd, wd, wd); }, "CUDA layer norm shape/type mismatch", "layer_norm shape");

    // layer_norm_linear at width 640 (the fused kernel) equals layer_norm -> linear bit for bit
    {
        const std::size_t W6 = 640, N6 = 1920;
        const auto x6 = filled({2, rows / 2, W6}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.29F) * 1.5F; });
        const auto g6 = filled({W6}, [](std::size_t i) { return 1.0F + 0.25F * std::cos(static_cast<float>(i)); });
        const auto b6 = filled({W6}, [](std::size_t i) { return 0.1F * std::sin(static_cast<float>(i)); });
        const auto w6 = filled({N6, W6}, [](std::size_t i) { return std::cos(static_cast<float>(i) * 0.013F) * 0.04F; });
        auto x6d = Tensor::from_host_f32(runtime, x6);
        auto g6d = Tensor::from_host_f32(runtime, g6), b6d = Tensor::from_host_f32(runtime, b6);
        const auto w6p = ops.pack_e4m3(Tensor::from_host_f32(runtime, w6));
        const auto fused = ops.layer_norm_linear(x6d, g6d, b6d, w6p).to_host_f32(runtime);
        const auto comp = ops.linear(ops.layer_norm(x6d, g6d, b6d), w6p).to_host_f32(runtime);
        require(fused.values.size() == comp.values.size(), "layer_norm_linear shape");
        for (std::size_t i = 0; i < comp.values.size(); ++i)
            require(std::memcmp(&fused.values[i], &comp.values[i], sizeof(float)) == 0,
                    "layer_norm_linear equals layer_norm -> linear");
        // fp16 weight (no fused kernel): the two calls
        auto onesd = Tensor::from_host_f32(runtime, ones), zerosd = Tensor::from_host_f32(runtime, zeros);
        const auto unfused = ops.layer_norm_linear(xd, onesd, zerosd, wd).to_host_f32(runtime);
        const auto unfused_ref = ops.linear(ops.layer_norm(xd, onesd, zerosd), wd).to_host_f32(runtime);
        for (std::size_t i = 0; i < unfused_ref.values.size(); ++i)
            require(std::memcmp(&unfused.values[i], &unfused_ref.values[i], sizeof(float)) == 0,
                    "layer_norm_linear with an fp16 weight equals the two calls");
    }

    // attention_sublayer == layer_norm -> linear(qkv) -> attention -> linear_residual_into
    const std::size_t heads = 2;
    const auto wq = filled({3 * W, W}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.013F) * 0.06F; });
    const auto wo = filled({W, W}, [](std::size_t i) { return std::cos(static_cast<float>(i) * 0.029F) * 0.06F; });
    const auto bo = filled({W}, [](std::size_t i) { return 0.01F * static_cast<float>(i % 7); });
    const auto qkv8 = ops.pack_e4m3(Tensor::from_host_f32(runtime, wq));
    auto wod = Tensor::from_host_f32(runtime, wo);
    auto bod = Tensor::from_host_f32(runtime, bo);
    auto gd = Tensor::from_host_f32(runtime, ones);
    auto bd = Tensor::from_host_f32(runtime, zeros);
    auto fused = Tensor::from_host_f32(runtime, x);
    ops.attention_sublayer(fused, gd, bd, qkv8, wod, bod, heads);
    auto step = Tensor::from_host_f32(runtime, x);
    const auto n = ops.layer_norm(step, gd, bd);
    const auto qkv = ops.linear(n, qkv8).to_host_f32(runtime);  // [2, 48, 3W] on the host, split below
    FloatTensor qh{{2, rows / 2, W}, {}}, kh{{2, rows / 2, W}, {}}, vh{{2, rows / 2, W}, {}};
    for (std::size_t r = 0; r < rows; ++r)
        for (std::size_t c = 0; c < W; ++c) {
            qh.values.push_back(qkv.values[r * 3 * W + c]);
            kh.values.push_back(qkv.values[r * 3 * W + W + c]);
            vh.values.push_back(qkv.values[r * 3 * W + 2 * W + c]);
        }
    const auto attn = ops.attention(Tensor::from_host_f32(runtime, qh), Tensor::from_host_f32(runtime, kh),
                                    Tensor::from_host_f32(runtime, vh), heads);
    ops.linear_residual_into(attn, wod, &bod, step);
    const auto a = fused.to_host_f32(runtime).values, b = step.to_host_f32(runtime).values;
    for (std::size_t i = 0; i < a.size(); ++i) require(a[i] == b[i], "attention_sublayer == composition");
    // fp8 activations (E4M3 LayerNorm output, fp8 MFMA projection): close to the fp16-activation result
    auto fused8 = Tensor::from_host_f32(runtime, x);
    ops.attention_sublayer(fused8, gd, bd, qkv8, wod, bod, heads, /*fp8_activations=*/true);
    const auto a8 = fused8.to_host_f32(runtime).values;
    for (std::size_t i = 0; i < a.size(); ++i) require_close(a8[i], a[i], 2e-2F, "sublayer fp8 activations");
    const auto qkv16 = Tensor::from_host_f32(runtime, wq);
    require_throws([&] { ops.attention_sublayer(fused8, gd, bd, qkv16, wod, bod, heads, true); },
                   "FP8 activations require a packed E4M3 qkv weight", "fp8 activations need E4M3 weights");
    // cross_attention_sublayer == layer_norm -> linear(q) -> attention(q, K, V of the projected
    // context) -> linear_residual_into (the block's second half, unet.cpp:120-131)
    const std::size_t ctx_len = 77, ctx_dim = 128;
    const auto ctx = filled({2, ctx_len, ctx_dim}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.031F); });
    const auto wk = filled({W, ctx_dim}, [](std::size_t i) { return std::cos(static_cast<float>(i) * 0.011F) * 0.08F; });
    const auto wv = filled({W, ctx_dim}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.019F) * 0.08F; });
    const auto wq1 = filled({W, W}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.023F) * 0.06F; });
    auto ctxd = Tensor::from_host_f32(runtime, ctx);
    const auto kv = ops.linear(ctxd, ops.concat_rows(Tensor::from_host_f32(runtime, wk), Tensor::from_host_f32(runtime, wv)));
    const auto wqd = Tensor::from_host_f32(runtime, wq1);
    auto crossed = Tensor::from_host_f32(runtime, x);
    ops.cross_attention_sublayer(crossed, gd, bd, wqd, kv, wod, bod, heads);
    auto cstep = Tensor::from_host_f32(runtime, x);
    const auto cq = ops.linear(ops.layer_norm(cstep, gd, bd), wqd);
    const auto kvh = kv.to_host_f32(runtime);
    FloatTensor kh2{{2, ctx_len, W}, {}}, vh2{{2, ctx_len, W}, {}};
    for (std::size_t r = 0; r < 2 * ctx_len; ++r)
        for (std::size_t c = 0; c < W; ++c) {
            kh2.values.push_back(kvh.values[r * 2 * W + c]);
            vh2.values.push_back(kvh.values[r * 2 * W + W + c]);
        }
    const auto cattn = ops.attention(cq, Tensor::from_host_f32(runtime, kh2), Tensor::from_host_f32(runtime, vh2), heads);
    ops.linear_residual_into(cattn, wod, &bod, cstep);
    const auto ca = crossed.to_host_f32(runtime).values, cb = cstep.to_host_f32(runtime).values;
    for (std::size_t i = 0; i < ca.size(); ++i) require(ca[i] == cb[i], "cross_attention_sublayer == composition");
    std::cout << "sublayer cases passed\n";
}

// The level-2 out-projection shape ([2, 1024, 1280] x [1280, 1280]^T + bias, added into the hidden
// state: the K-split kernel on a 256-CU device): sampled rows against the host fp32 reference of the
// fp16-rounded operands.
void out_projection_cases() {
    Runtime runtime;
    Ops ops(runtime);
    const std::size_t rows = 2048, W = 1280;
    const auto a = filled({2, rows / 2, W}, [](std::size_t i) { return std::sin(static_cast<float>(i % 9973) * 0.37F); });
    const auto w = filled({W, W}, [](std::size_t i) { return std::cos(static_cast<float>(i % 7919) * 0.11F) * 0.03F; });
    const auto b = filled({W}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.7F) * 0.1F; });
    const auto h = filled({2, rows / 2, W}, [](std::size_t i) { return std::cos(static_cast<float>(i % 6007) * 0.05F); });
    const auto ad = Tensor::from_host_f32(runtime, a);
    const auto wd = Tensor::from_host_f32(runtime, w);
    const auto bd = Tensor::from_host_f32(runtime, b);
    auto hd = Tensor::from_host_f32(runtime, h);
    const auto a16 = ad.to_host_f32(runtime).values, w16 = wd.to_host_f32(runtime).values;
    const auto b16 = bd.to_host_f32(runtime).values, h16 = hd.to_host_f32(runtime).values;
    ops.linear_residual_into(ad, wd, &bd, hd);
    const auto got = hd.to_host_f32(runtime).values;
    for (std::size_t r : {std::size_t{0}, std::size_t{1}, std::size_t{63}, std::size_t{64}, std::size_t{1023},
                          std::size_t{1500}, rows - 1}) {
        const auto ref = host_linear(std::vector<float>(a16.begin() + r * W, a16.begin() + (r + 1) * W), w16, 1, W, W);
        for (std::size_t o = 0; o < W; ++o) {
            const float e = ref[o] + b16[o] + h16[r * W + o];
            require_close(got[r * W + o], e, std::fabs(e) * 1e-3F + 1e-3F, "out-projection");
        }
    }
    std::cout << "out-projection cases passed\n";
}

// Ops::attention itself (allocating its output) captured in a HIP graph: after
// one warm-up call the arena serves the output from its cache, so the capture
// makes no driver allocation; replays with eager work between them reproduce
// the eager result bit for bit; the block stays held until the graph is gone.
void graph_capture_cases() {
    Runtime runtime;
    Ops ops(runtime);
    const auto qh = filled({2, 256, 128}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.37F); });
    const auto kh = filled({2, 300, 128}, [](std::size_t i) { return std::cos(static_cast<float>(i) * 0.11F); });
    const auto vh = filled({2, 300, 128}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.05F + 1.0F); });
    const auto q = Tensor::from_host_f32(runtime, qh);
    const auto k = Tensor::from_host_f32(runtime, kh);
    const auto v = Tensor::from_host_f32(runtime, vh);
    const auto eager = ops.attention(q, k, v, 2).to_host_f32(runtime);  // warm-up: its block returns to the cache
    const auto before = runtime.memory_arena_stats();
    require(before.cached_bytes >= q.bytes(), "output block cached after the eager call");

    runtime.begin_graph_allocation_capture();
    hipGraph_t graph = nullptr;
    SDXL_HIP_CHECK(hipStreamBeginCapture(runtime.stream(), hipStreamCaptureModeGlobal));
    Tensor out = ops.attention(q, k, v, 2);
    SDXL_HIP_CHECK(hipStreamEndCapture(runtime.stream(), &graph));
    runtime.end_graph_allocation_capture();
    const auto during = runtime.memory_arena_stats();
    require(during.driver_allocations == before.driver_allocations, "no hipMalloc inside the capture");
    require(during.cache_hits == before.cache_hits + 1, "capture served from the arena cache");

    hipGraphExec_t exec = nullptr;
    SDXL_HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    for (int replay = 0; replay < 4; ++replay) {
        SDXL_HIP_CHECK(hipMemsetAsync(out.data(), 0xFF, out.bytes(), runtime.stream()));  // NaN fill, not captured
        SDXL_HIP_CHECK(hipGraphLaunch(exec, runtime.stream()));
        const auto got = out.to_host_f32(runtime);
        require(got.values.size() == eager.values.size(), "graph output shape");
        for (std::size_t i = 0; i < got.values.size(); ++i)
            require(std::memcmp(&got.values[i], &eager.values[i], sizeof(float)) == 0, "graph replay equals eager");
        (void)ops.attention(k, k, v, 2);  // unrelated eager work between replays
    }
    SDXL_HIP_CHECK(hipGraphExecDestroy(exec));
    SDXL_HIP_CHECK(hipGraphDestroy(graph));
    const std::size_t held_bytes = out.bytes();
    out = Tensor();
    require(runtime.memory_arena_stats().graph_held_bytes >= held_bytes, "captured block held after its tensor died");
    runtime.release_graph_allocations();
    const auto released = runtime.memory_arena_stats();
    require(released.graph_held_bytes == 0, "held blocks released");
    runtime.trim_memory_arena();
    require(runtime.memory_arena_stats().cached_bytes == 0, "trim frees the cache");

    // x = f(x) inside the capture: the input tensor x (allocated before the capture) dies inside
    // the captured sequence. Its block must stay out of the cache while the graph exists, or the
    // next eager tensor of that size would take it and replays would read that tensor as x.
    {
        Tensor x = Tensor::from_host_f32(runtime, qh);
        const auto x_eager = ops.attention(x, k, v, 2).to_host_f32(runtime);  // warm-up: the output size is cached
        runtime.begin_graph_allocation_capture();
        hipGraph_t g2 = nullptr;
        SDXL_HIP_CHECK(hipStreamBeginCapture(runtime.stream(), hipStreamCaptureModeGlobal));
        Tensor y = ops.attention(x, k, v, 2);
        x = Tensor();  // the input's last reference dies inside the capture
        SDXL_HIP_CHECK(hipStreamEndCapture(runtime.stream(), &g2));
        runtime.end_graph_allocation_capture();
        const auto other_host = filled({2, 256, 128}, [](std::size_t i) { return std::cos(static_cast<float>(i) * 0.29F); });
        const Tensor other = Tensor::from_host_f32(runtime, other_host);  // same size as x, allocated eagerly
        const auto other_before = other.to_host_f32(runtime);
        hipGraphExec_t exec2 = nullptr;
        SDXL_HIP_CHECK(hipGraphInstantiate(&exec2, g2, nullptr, nullptr, 0));
        for (int replay = 0; replay < 3; ++replay) {
            SDXL_HIP_CHECK(hipGraphLaunch(exec2, runtime.stream()));
            const auto got = y.to_host_f32(runtime);
            for (std::size_t i = 0; i < got.values.size(); ++i)
                require(std::memcmp(&got.values[i], &x_eager.values[i], sizeof(float)) == 0,
                        "replay reads the freed input, not the eager tensor of its size");
            const auto other_now = other.to_host_f32(runtime);
            for (std::size_t i = 0; i < other_now.values.size(); ++i)
                require(std::memcmp(&other_now.values[i], &other_before.values[i], sizeof(float)) == 0,
                        "eager tensor intact across replays");
        }
        SDXL_HIP_CHECK(hipGraphExecDestroy(exec2));
        SDXL_HIP_CHECK(hipGraphDestroy(g2));
        y = Tensor();
        runtime.release_graph_allocations();
        require(runtime.memory_arena_stats().graph_held_bytes == 0, "held blocks released");
    }

    // a size with no cached block inside a capture window: a clear error, no driver allocation
    {
        runtime.begin_graph_allocation_capture();
        bool threw = false;
        try {
            (void)runtime.allocate_device(123457);
        } catch (const HipError&) {
            threw = true;
        }
        runtime.end_graph_allocation_capture();
        require(threw, "cache miss inside a capture window throws");
    }
    std::cout << "graph capture cases passed\n";
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
    // random FP32 D = 512 (the fp32 matrix-core kernel) against a float64 host softmax
    const std::size_t vs = 70;
    const auto vq = filled({1, vs, 512}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.37F); });
    const auto vk = filled({1, vs, 512}, [](std::size_t i) { return std::cos(static_cast<float>(i) * 0.11F); });
    const auto vvv = filled({1, vs, 512}, [](std::size_t i) { return std::sin(static_cast<float>(i) * 0.05F + 1.0F); });
    const auto vae_rand = ops.attention(Tensor::from_host_f32(runtime, vq, ScalarType::Float32),
                                        Tensor::from_host_f32(runtime, vk, ScalarType::Float32),
                                        Tensor::from_host_f32(runtime, vvv, ScalarType::Float32), 1, false)
                              .to_host_f32(runtime);
    for (std::size_t r = 0; r < vs; ++r) {
        std::vector<double> sc(vs);
        double mx = -1e300, den = 0.0;
        for (std::size_t c = 0; c < vs; ++c) {
            double dot = 0.0;
            for (std::size_t d = 0; d < 512; ++d) dot += (double)vq.values[r * 512 + d] * vk.values[c * 512 + d];
            sc[c] = dot / std::sqrt(512.0);
            mx = std::max(mx, sc[c]);
        }
        for (auto& x : sc) den += (x = std::exp(x - mx));
        for (std::size_t d = 0; d < 512; ++d) {
            double o = 0.0;
            for (std::size_t c = 0; c < vs; ++c) o += sc[c] * vvv.values[c * 512 + d];
            require_close(vae_rand.values[r * 512 + d], static_cast<float>(o / den), 1.0e-5F, "VAE FP32 random");
        }
    }

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
    graph_capture_cases();
    std::cout << "device cases passed\n";
    sublayer_cases();
    out_projection_cases();
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

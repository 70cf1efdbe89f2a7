// Container-only harness that compiles the reference's own CPU attention,
// LayerNorm and linear (src/unet.cpp:202-263, :440-481 of
// Apache0ne/sdxl-end2end) into oracle/_ref/libref_attention.so.
//
// TEST INFRASTRUCTURE ONLY: used to validate the C restatement in
// attention_oracle.c and as the "reference" CPU baseline. The reference
// sources are compiled where they lie (this file includes src/unet.cpp by
// path so its anonymous-namespace functions are reachable); nothing from the
// reference is copied into this repository.
#include "unet.cpp"

#include <cstring>

namespace {

sdxl::FloatTensor make3(const float* data, std::size_t a, std::size_t b, std::size_t c) {
    sdxl::FloatTensor t;
    t.shape = {a, b, c};
    t.values.assign(data, data + a * b * c);
    return t;
}

sdxl::TensorView f32_view(const float* data, std::vector<std::uint64_t> shape) {
    sdxl::TensorView view;
    view.data = reinterpret_cast<const std::byte*>(data);
    view.dtype = sdxl::DType::F32;
    view.shape = shape;
    std::vector<std::int64_t> strides(shape.size());
    std::int64_t stride = 4;
    for (std::size_t i = shape.size(); i-- > 0;) {
        strides[i] = stride;
        stride *= static_cast<std::int64_t>(shape[i]);
    }
    view.strides_bytes = strides;
    view.storage_bytes = static_cast<std::uint64_t>(stride);
    view.source_key = "ref_harness";
    return view;
}

}  // namespace

extern "C" int ref_full_attention(const float* q, const float* k, const float* v, float* o, std::size_t batch,
                                  std::size_t q_seq, std::size_t k_seq, std::size_t heads, std::size_t head_dim) {
    try {
        const std::size_t width = heads * head_dim;
        auto out = sdxl::full_attention(make3(q, batch, q_seq, width), make3(k, batch, k_seq, width),
                                        make3(v, batch, k_seq, width), heads);
        std::memcpy(o, out.values.data(), out.values.size() * sizeof(float));
        return 0;
    } catch (...) {
        return 1;
    }
}

extern "C" int ref_layer_norm(const float* x, const float* w, const float* b, float* y, std::size_t rows,
                              std::size_t width, float eps) {
    try {
        auto out = sdxl::layer_norm_last_dim(make3(x, 1, rows, width), f32_view(w, {width}), f32_view(b, {width}), eps);
        std::memcpy(y, out.values.data(), out.values.size() * sizeof(float));
        return 0;
    } catch (...) {
        return 1;
    }
}

extern "C" int ref_linear(const float* x, const float* weight, const float* bias, float* y, std::size_t rows,
                          std::size_t in_features, std::size_t out_features) {
    try {
        auto wv = f32_view(weight, {out_features, in_features});
        sdxl::TensorView bv;
        if (bias) bv = f32_view(bias, {out_features});
        auto out = sdxl::linear_3d(make3(x, 1, rows, in_features), wv, bias ? &bv : nullptr);
        std::memcpy(y, out.values.data(), out.values.size() * sizeof(float));
        return 0;
    } catch (...) {
        return 1;
    }
}

// One UNet transformer block, src/unet.cpp:495-523 (`transformer_block`), run
// on a model graph declared by the reference itself (SDXLModel, src/sdxl.cpp)
// whose block parameters are bound to caller-provided fp32 arrays. The block
// is the first one in the graph whose channel count equals `width`.
// weights: norm1 w/b, attn1 q/k/v/out w, out b, norm2 w/b, attn2 q w,
// k/v w [width, ctx_dim], out w, out b, norm3 w/b, ff0 w [8 width, width],
// ff0 b, ff2 w [width, 4 width], ff2 b (the reference's parameter order).
extern "C" int ref_transformer_block(const float* x, const float* ctx, const float* const* weights, float* y,
                                     std::size_t batch, std::size_t seq, std::size_t width, std::size_t ctx_len,
                                     std::size_t ctx_dim, std::size_t heads) {
    try {
        static sdxl::SDXLModel model;
        static const char* suffixes[] = {
            "norm1.weight", "norm1.bias", "attn1.to_q.weight", "attn1.to_k.weight", "attn1.to_v.weight",
            "attn1.to_out.0.weight", "attn1.to_out.0.bias", "norm2.weight", "norm2.bias", "attn2.to_q.weight",
            "attn2.to_k.weight", "attn2.to_v.weight", "attn2.to_out.0.weight", "attn2.to_out.0.bias",
            "norm3.weight", "norm3.bias", "ff.net.0.proj.weight", "ff.net.0.proj.bias", "ff.net.2.weight",
            "ff.net.2.bias"};
        std::string prefix;
        for (const auto& [name, slot] : model.graph().parameter_index()) {
            const std::string tail = ".transformer_blocks.0.attn1.to_q.weight";
            if (name.size() > tail.size() && name.compare(name.size() - tail.size(), tail.size(), tail) == 0 &&
                slot->expected_shape[0] == width &&
                model.graph().find_parameter(name.substr(0, name.size() - 17) + "attn2.to_k.weight")->expected_shape[1] == ctx_dim &&
                (prefix.empty() || name < prefix))
                prefix = name.substr(0, name.size() - 18);
        }
        if (prefix.empty()) return 2;
        for (int i = 0; i < 20; ++i) {
            sdxl::ParameterSlot* slot = model.graph().find_parameter(prefix + "." + suffixes[i]);
            if (slot == nullptr) return 3;
            slot->tensor = f32_view(weights[i], slot->expected_shape);
        }
        auto out = sdxl::transformer_block(model, prefix, make3(x, batch, seq, width), make3(ctx, batch, ctx_len, ctx_dim),
                                           heads);
        std::memcpy(y, out.values.data(), out.values.size() * sizeof(float));
        return 0;
    } catch (...) {
        return 1;
    }
}

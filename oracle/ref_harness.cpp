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

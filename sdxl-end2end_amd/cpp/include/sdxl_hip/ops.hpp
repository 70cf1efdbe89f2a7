// Operator layer of the sdxl_hip C++20 host API: the attention entry point of
// the reference's Ops (include/sdxl/cuda/ops.hpp:92-97) and the operators of
// the UNet transformer block's attention sublayer (layer_norm, linear with
// fp16 or FP8 E4M3 weights, FP8 weight packing), implemented over the C ABI
// (include/sdxl_hip/attention.h, sublayer.h).
#pragma once

#include "sdxl_hip/runtime.hpp"
#include "sdxl_hip/tensor.hpp"

#include <cstddef>

namespace sdxl::hip {

class Ops final {
public:
    explicit Ops(const Runtime& runtime);

    // query [B, Sq, H*D], key/value [B, Sk, H*D] (fp16, bf16 or fp32, same type),
    // optional int32 key_mask [B, Sk] (0 hides a key). Returns [B, Sq, H*D] of
    // the query's type. Throws HipError with the reference's messages
    // (src/cuda/ops_kernels.cu:1914-1941). Stream-ordered, no host sync; the
    // output is allocated from the stream-ordered pool.
    [[nodiscard]] Tensor attention(const Tensor& query, const Tensor& key, const Tensor& value, std::size_t heads,
                                   bool causal = false, const Tensor* key_mask = nullptr) const;

    // Same computation into a caller-owned output (no allocation at all).
    void attention_into(const Tensor& query, const Tensor& key, const Tensor& value, std::size_t heads,
                        Tensor& output, bool causal = false, const Tensor* key_mask = nullptr) const;

    // LayerNorm over the last dim (reference Ops::layer_norm, ops_kernels.cu:1428-1460):
    // fp16 input [..., W], weight/bias [W]; W even, <= 2048.
    [[nodiscard]] Tensor layer_norm(const Tensor& input, const Tensor& weight, const Tensor& bias,
                                    float epsilon = 1.0e-5F) const;

    // input . weight^T + bias (reference Ops::linear): fp16 input [..., K], weight [N, K]
    // fp16 or Float8E4M3 with attached per-output-channel scales (pack_e4m3), optional
    // fp16 bias [N]. K % 64 == 0, N % 4 == 0.
    [[nodiscard]] Tensor linear(const Tensor& input, const Tensor& weight, const Tensor* bias = nullptr) const;

    // linear(layer_norm(input, norm_weight, norm_bias, epsilon), weight, bias) — the
    // transformer block's norm -> projection (unet.cpp:106-112) — in one launch where the
    // fused kernel takes the shape and is faster (Float8E4M3 weight, width 640, N % 128 == 0:
    // the level-1 q|k|v; at width 1280 the two launches are faster), else as the two calls;
    // the same result either way.
    [[nodiscard]] Tensor layer_norm_linear(const Tensor& input, const Tensor& norm_weight, const Tensor& norm_bias,
                                           const Tensor& weight, const Tensor* bias = nullptr,
                                           float epsilon = 1.0e-5F) const;

    // hidden += input . weight^T + bias in one pass (the reference's linear followed by
    // add_in_place, unet.cpp:114-118, with the residual added in the linear's epilogue).
    void linear_residual_into(const Tensor& input, const Tensor& weight, const Tensor* bias, Tensor& hidden) const;

    // Per-output-channel E4M3 packing of an fp16 weight [N, K] (reference
    // src/cuda/weights.cu:119-170): returns the codes with their scales attached.
    [[nodiscard]] Tensor pack_e4m3(const Tensor& weight) const;

    // Rows of q, k, v projection weights [W, W] concatenated into [3W, W]
    // (fp16), the fused QKV weight attention_sublayer takes.
    [[nodiscard]] Tensor concat_rows(const Tensor& a, const Tensor& b, const Tensor& c) const;
    // Two-weight form: [to_k; to_v] [2W, C], the context K|V projection's weight.
    [[nodiscard]] Tensor concat_rows(const Tensor& a, const Tensor& b) const;

    // hidden += to_out(attention(LN(hidden) . qkv_weight^T)) in place: the self-attention
    // half of the reference's UNet::transformer_block (src/cuda/unet.cpp:106-118) with q/k/v
    // as one projection. hidden fp16 [B, S, 64 heads]; qkv_weight [3W, W] fp16 or packed
    // E4M3; out_weight [W, W] fp16; out_bias [W]. fp8_activations (packed E4M3 qkv_weight
    // only): LayerNorm quantises its output per row to E4M3 and the projection runs on the
    // fp8 matrix cores (no counterpart in the reference, whose FP8 path is weight-only).
    void attention_sublayer(Tensor& hidden, const Tensor& norm_weight, const Tensor& norm_bias,
                            const Tensor& qkv_weight, const Tensor& out_weight, const Tensor& out_bias,
                            std::size_t heads, bool fp8_activations = false) const;

    // hidden += to_out(attention(LN(hidden) . q_weight^T, K, V)) in place: the cross-attention
    // half of the reference's transformer block (src/cuda/unet.cpp:120-131). context_kv
    // [B, L, 2W] fp16 holds K | V of encoder_hidden_states, projected once per request:
    // linear(context, concat_rows(to_k, to_v)). q_weight [W, W] fp16 or packed E4M3.
    void cross_attention_sublayer(Tensor& hidden, const Tensor& norm_weight, const Tensor& norm_bias,
                                  const Tensor& q_weight, const Tensor& context_kv, const Tensor& out_weight,
                                  const Tensor& out_bias, std::size_t heads, bool fp8_activations = false) const;

private:
    const Runtime* runtime_ = nullptr;
};

}  // namespace sdxl::hip

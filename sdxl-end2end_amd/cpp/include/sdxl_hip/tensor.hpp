// Owning device tensor of the sdxl_hip C++20 host API.
//
// Mirrors the parts of the reference's Tensor (include/sdxl/cuda/tensor.hpp:64-157)
// the attention path uses: shape/type queries, allocation, host upload with
// FP32 -> FP16 conversion on the host (round to nearest even, as
// Tensor::from_host_f32 does, src/cuda/tensor.cu:237-250) and download.
#pragma once

#include "sdxl_hip/runtime.hpp"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

namespace sdxl::hip {

// Float8E4M3: finite-only E4M3 codes (bias 7), used for linear weights with an
// attached per-output-channel dequantisation scale (the reference's FP8 weights).
enum class ScalarType : std::uint8_t { Float16, BFloat16, Float32, Int32, Float8E4M3 };

[[nodiscard]] std::size_t scalar_size(ScalarType type) noexcept;

// Host FP32 tensor (the reference's sdxl::FloatTensor).
struct FloatTensor {
    std::vector<std::size_t> shape;
    std::vector<float> values;
};

// IEEE conversions used for host uploads (round to nearest, ties to even).
[[nodiscard]] std::uint16_t float_to_half(float value) noexcept;
[[nodiscard]] float half_to_float(std::uint16_t bits) noexcept;
[[nodiscard]] std::uint16_t float_to_bf16(float value) noexcept;
[[nodiscard]] float bf16_to_float(std::uint16_t bits) noexcept;
// E4M3 code -> value (sign, 4-bit exponent bias 7, 3-bit mantissa, subnormals;
// 0x7F/0xFF are NaN), the reference's decode (src/unet.cpp:91-119).
[[nodiscard]] float e4m3_to_float(std::uint8_t bits) noexcept;

class Tensor final {
public:
    Tensor() = default;

    [[nodiscard]] static Tensor allocate(const Runtime& runtime, std::vector<std::size_t> shape, ScalarType type);
    [[nodiscard]] static Tensor from_host_f32(const Runtime& runtime, const FloatTensor& host,
                                              ScalarType type = ScalarType::Float16);
    [[nodiscard]] static Tensor from_host_i32(const Runtime& runtime, std::vector<std::size_t> shape,
                                              const std::vector<std::int32_t>& values);
    [[nodiscard]] FloatTensor to_host_f32(const Runtime& runtime) const;

    [[nodiscard]] const std::vector<std::size_t>& shape() const noexcept { return shape_; }
    [[nodiscard]] std::size_t rank() const noexcept { return shape_.size(); }
    [[nodiscard]] std::size_t size(std::size_t dim) const { return shape_.at(dim); }
    [[nodiscard]] std::size_t elements() const noexcept;
    [[nodiscard]] std::size_t bytes() const noexcept { return elements() * scalar_size(type_); }
    [[nodiscard]] ScalarType type() const noexcept { return type_; }
    [[nodiscard]] void* data() const noexcept { return data_.get(); }
    [[nodiscard]] const std::int32_t* int32_data() const;

    // Dequantisation scales of an FP8 tensor (fp32, one per output channel or
    // one for the tensor), as the reference's Tensor::attach_dequant_scale.
    void attach_dequant_scale(Tensor scale);
    [[nodiscard]] bool has_dequant_scale() const noexcept { return scale_ != nullptr; }
    [[nodiscard]] const float* dequant_scale_data() const;
    [[nodiscard]] std::size_t dequant_scale_count() const noexcept { return scale_ ? scale_->elements() : 0; }

private:
    std::shared_ptr<void> data_;
    std::shared_ptr<Tensor> scale_;
    std::vector<std::size_t> shape_;
    ScalarType type_ = ScalarType::Float16;
};

}  // namespace sdxl::hip

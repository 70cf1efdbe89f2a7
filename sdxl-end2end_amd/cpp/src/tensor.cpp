// Device tensor and host conversions (see tensor.hpp).
#include "sdxl_hip/tensor.hpp"

#include <bit>
#include <cmath>
#include <limits>
#include <cstring>
#include <functional>
#include <numeric>

namespace sdxl::hip {

std::size_t scalar_size(ScalarType type) noexcept {
    switch (type) {
    case ScalarType::Float16:
    case ScalarType::BFloat16: return 2;
    case ScalarType::Float32:
    case ScalarType::Int32: return 4;
    case ScalarType::Float8E4M3: return 1;
    }
    return 0;
}

float e4m3_to_float(std::uint8_t bits) noexcept {
    const std::uint32_t exponent = (bits >> 3) & 0xFU, mantissa = bits & 0x7U;
    float value;
    if ((bits & 0x7FU) == 0x7FU) value = std::numeric_limits<float>::quiet_NaN();
    else if (exponent == 0) value = std::ldexp(static_cast<float>(mantissa) / 8.0F, -6);
    else value = std::ldexp(1.0F + static_cast<float>(mantissa) / 8.0F, static_cast<int>(exponent) - 7);
    return (bits & 0x80U) ? -value : value;
}

void Tensor::attach_dequant_scale(Tensor scale) {
    if (scale.type() != ScalarType::Float32 || scale.rank() != 1)
        throw HipError("FP8 weight has invalid scaling metadata");
    scale_ = std::make_shared<Tensor>(std::move(scale));
}

const float* Tensor::dequant_scale_data() const {
    if (!scale_) throw HipError("FP8 weight has invalid scaling metadata");
    return static_cast<const float*>(scale_->data());
}

// binary32 -> binary16, round to nearest even; overflow to infinity, NaN kept quiet.
std::uint16_t float_to_half(float value) noexcept {
    const std::uint32_t x = std::bit_cast<std::uint32_t>(value);
    const std::uint32_t sign = (x >> 16) & 0x8000U;
    const std::uint32_t mag = x & 0x7FFFFFFFU;
    if (mag >= 0x7F800000U) return static_cast<std::uint16_t>(sign | 0x7C00U | (mag > 0x7F800000U ? 0x200U : 0U));
    if (mag >= 0x477FF000U) return static_cast<std::uint16_t>(sign | 0x7C00U);  // rounds past 65504
    if (mag < 0x38800000U) {                                                   // half subnormal range
        if (mag < 0x33000000U) return static_cast<std::uint16_t>(sign);
        const std::uint32_t exponent = mag >> 23;
        const std::uint32_t mantissa = (mag & 0x7FFFFFU) | 0x800000U;
        const std::uint32_t shift = 126U - exponent;
        std::uint32_t q = mantissa >> shift;
        const std::uint32_t rest = mantissa & ((1U << shift) - 1U);
        const std::uint32_t half = 1U << (shift - 1U);
        if (rest > half || (rest == half && (q & 1U))) ++q;
        return static_cast<std::uint16_t>(sign | q);
    }
    std::uint32_t q = ((((mag >> 23) - 112U) << 10) | ((mag & 0x7FFFFFU) >> 13));
    const std::uint32_t rest = mag & 0x1FFFU;
    if (rest > 0x1000U || (rest == 0x1000U && (q & 1U))) ++q;
    return static_cast<std::uint16_t>(sign | q);
}

float half_to_float(std::uint16_t bits) noexcept {
    const std::uint32_t sign = static_cast<std::uint32_t>(bits & 0x8000U) << 16;
    std::uint32_t exponent = (bits >> 10) & 0x1FU;
    std::uint32_t mantissa = bits & 0x3FFU;
    std::uint32_t out = 0;
    if (exponent == 0) {
        if (mantissa == 0) {
            out = sign;
        } else {
            int e = -14;
            while ((mantissa & 0x400U) == 0) {
                mantissa <<= 1;
                --e;
            }
            out = sign | (static_cast<std::uint32_t>(e + 127) << 23) | ((mantissa & 0x3FFU) << 13);
        }
    } else if (exponent == 0x1FU) {
        out = sign | 0x7F800000U | (mantissa << 13);
    } else {
        out = sign | ((exponent + 112U) << 23) | (mantissa << 13);
    }
    return std::bit_cast<float>(out);
}

std::uint16_t float_to_bf16(float value) noexcept {
    std::uint32_t x = std::bit_cast<std::uint32_t>(value);
    if ((x & 0x7FFFFFFFU) > 0x7F800000U) return static_cast<std::uint16_t>((x >> 16) | 0x40U);
    x += 0x7FFFU + ((x >> 16) & 1U);
    return static_cast<std::uint16_t>(x >> 16);
}

float bf16_to_float(std::uint16_t bits) noexcept { return std::bit_cast<float>(static_cast<std::uint32_t>(bits) << 16); }

std::size_t Tensor::elements() const noexcept {
    return std::accumulate(shape_.begin(), shape_.end(), std::size_t{1}, std::multiplies<>());
}

const std::int32_t* Tensor::int32_data() const {
    if (type_ != ScalarType::Int32) throw HipError("tensor is not int32");
    return static_cast<const std::int32_t*>(data_.get());
}

Tensor Tensor::allocate(const Runtime& runtime, std::vector<std::size_t> shape, ScalarType type) {
    Tensor t;
    t.shape_ = std::move(shape);
    t.type_ = type;
    t.data_ = runtime.allocate_device(t.bytes());  // the runtime's caching arena
    return t;
}

Tensor Tensor::from_host_f32(const Runtime& runtime, const FloatTensor& host, ScalarType type) {
    Tensor t = allocate(runtime, host.shape, type);
    if (host.values.size() != t.elements()) throw HipError("host tensor shape/value count mismatch");
    if (t.elements() == 0) return t;
    if (type == ScalarType::Float32) {
        SDXL_HIP_CHECK(hipMemcpyAsync(t.data(), host.values.data(), t.bytes(), hipMemcpyHostToDevice, runtime.stream()));
        runtime.synchronize();
        return t;
    }
    if (type == ScalarType::Int32) throw HipError("use from_host_i32 for int32 tensors");
    if (type == ScalarType::Float8E4M3) throw HipError("use Ops::pack_e4m3 for FP8 weights");
    std::vector<std::uint16_t> bits(host.values.size());
    for (std::size_t i = 0; i < bits.size(); ++i)
        bits[i] = type == ScalarType::Float16 ? float_to_half(host.values[i]) : float_to_bf16(host.values[i]);
    SDXL_HIP_CHECK(hipMemcpyAsync(t.data(), bits.data(), t.bytes(), hipMemcpyHostToDevice, runtime.stream()));
    runtime.synchronize();  // the staging vector dies here
    return t;
}

Tensor Tensor::from_host_i32(const Runtime& runtime, std::vector<std::size_t> shape,
                             const std::vector<std::int32_t>& values) {
    Tensor t = allocate(runtime, std::move(shape), ScalarType::Int32);
    if (values.size() != t.elements()) throw HipError("host tensor shape/value count mismatch");
    if (t.elements() == 0) return t;
    SDXL_HIP_CHECK(hipMemcpyAsync(t.data(), values.data(), t.bytes(), hipMemcpyHostToDevice, runtime.stream()));
    runtime.synchronize();
    return t;
}

FloatTensor Tensor::to_host_f32(const Runtime& runtime) const {
    FloatTensor host;
    host.shape = shape_;
    host.values.resize(elements());
    if (host.values.empty()) return host;
    if (type_ == ScalarType::Float32) {
        SDXL_HIP_CHECK(hipMemcpyAsync(host.values.data(), data(), bytes(), hipMemcpyDeviceToHost, runtime.stream()));
        runtime.synchronize();
        return host;
    }
    if (type_ == ScalarType::Float8E4M3) {
        std::vector<std::uint8_t> codes(elements());
        SDXL_HIP_CHECK(hipMemcpyAsync(codes.data(), data(), bytes(), hipMemcpyDeviceToHost, runtime.stream()));
        runtime.synchronize();
        for (std::size_t i = 0; i < codes.size(); ++i) host.values[i] = e4m3_to_float(codes[i]);
        return host;
    }
    if (type_ == ScalarType::Int32) {
        std::vector<std::int32_t> tmp(elements());
        SDXL_HIP_CHECK(hipMemcpyAsync(tmp.data(), data(), bytes(), hipMemcpyDeviceToHost, runtime.stream()));
        runtime.synchronize();
        for (std::size_t i = 0; i < tmp.size(); ++i) host.values[i] = static_cast<float>(tmp[i]);
        return host;
    }
    std::vector<std::uint16_t> bits(elements());
    SDXL_HIP_CHECK(hipMemcpyAsync(bits.data(), data(), bytes(), hipMemcpyDeviceToHost, runtime.stream()));
    runtime.synchronize();
    for (std::size_t i = 0; i < bits.size(); ++i)
        host.values[i] = type_ == ScalarType::Float16 ? half_to_float(bits[i]) : bf16_to_float(bits[i]);
    return host;
}

}  // namespace sdxl::hip

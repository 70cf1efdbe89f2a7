// Runtime, backend parsing and profiling scopes (see runtime.hpp).
#include "sdxl_hip/runtime.hpp"

#include "sdxl_hip/attention.h"

#include <sstream>

namespace sdxl::hip {

void check_hip(hipError_t status, std::string_view expression, std::string_view file, int line) {
    if (status == hipSuccess) return;
    std::ostringstream message;
    message << "HIP error " << hipGetErrorName(status) << " (" << hipGetErrorString(status) << ") at " << file << ':'
            << line << ": " << expression;
    throw HipError(message.str());
}

// Spellings and the error text live in the C ABI (sdxl_attn_backend_parse),
// which follows the reference's parse_attention_backend (src/cuda/runtime.cpp:61-77).
AttentionBackend parse_attention_backend(std::string_view value) {
    const std::string text(value);
    std::int32_t backend = 0;
    if (sdxl_attn_backend_parse(text.c_str(), &backend) != SDXL_STATUS_OK) throw HipError(sdxl_last_error());
    return static_cast<AttentionBackend>(backend);
}

const char* attention_backend_name(AttentionBackend backend) noexcept {
    return sdxl_attn_backend_name(static_cast<std::int32_t>(backend));
}

struct RuntimeState {
    RuntimeOptions options;
    hipStream_t stream = nullptr;
    struct Scope {
        std::string label;
        hipEvent_t start = nullptr;
        hipEvent_t stop = nullptr;
    };
    std::vector<Scope> scopes;
};

Runtime::Runtime(RuntimeOptions options) : state_(std::make_unique<RuntimeState>()) {
    state_->options = options;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) throw HipError("no HIP device available");
    if (options.device < 0 || options.device >= count) throw HipError("HIP device index out of range");
    SDXL_HIP_CHECK(hipSetDevice(options.device));
    SDXL_HIP_CHECK(hipStreamCreateWithFlags(&state_->stream, hipStreamNonBlocking));
}

Runtime::~Runtime() {
    if (!state_) return;
    (void)hipSetDevice(state_->options.device);
    if (state_->stream != nullptr) (void)hipStreamSynchronize(state_->stream);
    for (auto& scope : state_->scopes) {
        if (scope.start) (void)hipEventDestroy(scope.start);
        if (scope.stop) (void)hipEventDestroy(scope.stop);
    }
    if (state_->stream != nullptr) (void)hipStreamDestroy(state_->stream);
}

hipStream_t Runtime::stream() const noexcept { return state_->stream; }
int Runtime::device() const noexcept { return state_->options.device; }
const RuntimeOptions& Runtime::options() const noexcept { return state_->options; }

void Runtime::synchronize() const { SDXL_HIP_CHECK(hipStreamSynchronize(state_->stream)); }

int Runtime::begin_profile(std::string label) const {
    if (!state_->options.profile) return -1;
    RuntimeState::Scope scope;
    scope.label = std::move(label);
    SDXL_HIP_CHECK(hipEventCreate(&scope.start));
    SDXL_HIP_CHECK(hipEventCreate(&scope.stop));
    SDXL_HIP_CHECK(hipEventRecord(scope.start, state_->stream));
    state_->scopes.push_back(std::move(scope));
    return static_cast<int>(state_->scopes.size()) - 1;
}

void Runtime::end_profile(int id) const {
    if (id < 0) return;
    SDXL_HIP_CHECK(hipEventRecord(state_->scopes.at(static_cast<std::size_t>(id)).stop, state_->stream));
}

std::vector<ProfileRecord> Runtime::profile_records() const {
    synchronize();
    std::vector<ProfileRecord> records;
    for (auto& scope : state_->scopes) {
        float ms = 0.0F;
        SDXL_HIP_CHECK(hipEventElapsedTime(&ms, scope.start, scope.stop));
        records.push_back({scope.label, ms});
        (void)hipEventDestroy(scope.start);
        (void)hipEventDestroy(scope.stop);
    }
    state_->scopes.clear();
    return records;
}

}  // namespace sdxl::hip

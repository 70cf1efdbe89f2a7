// Runtime, backend parsing and profiling scopes (see runtime.hpp).
#include "sdxl_hip/runtime.hpp"

#include "sdxl_hip/attention.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <unordered_map>
#include <unordered_set>

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

// Caching device-memory arena. Shared by the Runtime and by every block it
// handed out (the deleters keep it alive), so tensors may outlive the Runtime.
struct DeviceArena {
    std::mutex mu;
    int device = 0;
    std::size_t cache_limit = 0;
    std::multimap<std::size_t, void*> free_blocks;           // size -> block
    std::unordered_map<void*, std::size_t> capture_blocks;   // allocated inside a capture window, live
    std::vector<std::pair<void*, std::size_t>> graph_held;   // freed, still used by captured graphs
    bool capturing = false;
    MemoryArenaStats stats;

    static std::size_t granule(std::size_t bytes) { return (bytes + 255) & ~std::size_t{255}; }

    void* take(std::size_t bytes) {
        std::lock_guard<std::mutex> lock(mu);
        void* p = nullptr;
        auto it = free_blocks.find(bytes);
        if (it != free_blocks.end()) {
            p = it->second;
            free_blocks.erase(it);
            stats.cached_bytes -= bytes;
            ++stats.cache_hits;
        } else {
            // A driver allocation cannot be recorded into a stream capture: inside the
            // capture window every block must come from the cache.
            if (capturing)
                throw HipError("device arena: no cached block of " + std::to_string(bytes) +
                               " bytes inside a HIP graph capture window (run the captured sequence once "
                               "eagerly first, so that its blocks are cached)");
            SDXL_HIP_CHECK(hipSetDevice(device));
            hipError_t status = hipMalloc(&p, bytes);
            if (status == hipErrorOutOfMemory && !free_blocks.empty()) {
                // cached blocks of other sizes hold the memory: return them to the driver, retry once
                (void)hipGetLastError();
                for (auto& [size, q] : free_blocks) (void)hipFree(q);
                free_blocks.clear();
                stats.cached_bytes = 0;
                status = hipMalloc(&p, bytes);
            }
            SDXL_HIP_CHECK(status);
            ++stats.driver_allocations;
        }
        stats.live_bytes += bytes;
        stats.peak_live_bytes = std::max(stats.peak_live_bytes, stats.live_bytes);
        if (capturing) capture_blocks.emplace(p, bytes);
        return p;
    }

    void give_back(void* p, std::size_t bytes) noexcept {
        std::lock_guard<std::mutex> lock(mu);
        stats.live_bytes -= bytes;
        // Held for captured graphs: blocks allocated inside a capture window (replays
        // write them), and every block freed inside one, wherever it was allocated (a
        // graph input whose tensor dies during the captured sequence, x = f(x), is still
        // read by replays). Nothing is freed to the driver or re-cached meanwhile.
        if (capture_blocks.erase(p) != 0 || capturing) {
            graph_held.emplace_back(p, bytes);
            stats.graph_held_bytes += bytes;
            return;
        }
        cache_or_free(p, bytes);
    }

    void cache_or_free(void* p, std::size_t bytes) noexcept {  // caller holds mu
        if (stats.cached_bytes + bytes <= cache_limit) {
            free_blocks.emplace(bytes, p);
            stats.cached_bytes += bytes;
        } else {
            (void)hipSetDevice(device);
            (void)hipFree(p);
        }
    }

    void trim() noexcept {
        std::lock_guard<std::mutex> lock(mu);
        (void)hipSetDevice(device);
        for (auto& [bytes, p] : free_blocks) (void)hipFree(p);
        free_blocks.clear();
        stats.cached_bytes = 0;
    }

    ~DeviceArena() {
        (void)hipSetDevice(device);
        for (auto& [bytes, p] : free_blocks) (void)hipFree(p);
        for (auto& [p, bytes] : graph_held) (void)hipFree(p);
    }
};

struct RuntimeState {
    RuntimeOptions options;
    std::shared_ptr<DeviceArena> arena;
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
    state_->arena = std::make_shared<DeviceArena>();
    state_->arena->device = options.device;
    state_->arena->cache_limit = options.arena_cache_limit_bytes;
}

std::shared_ptr<void> Runtime::allocate_device(std::size_t bytes) const {
    if (bytes == 0) return std::shared_ptr<void>();
    const std::size_t size = DeviceArena::granule(bytes);
    std::shared_ptr<DeviceArena> arena = state_->arena;
    void* p = arena->take(size);
    return std::shared_ptr<void>(p, [arena, size](void* q) { arena->give_back(q, size); });
}

MemoryArenaStats Runtime::memory_arena_stats() const noexcept {
    std::lock_guard<std::mutex> lock(state_->arena->mu);
    return state_->arena->stats;
}

void Runtime::trim_memory_arena() const { state_->arena->trim(); }

void Runtime::begin_graph_allocation_capture() const {
    std::lock_guard<std::mutex> lock(state_->arena->mu);
    if (state_->arena->capturing) throw HipError("HIP graph allocation capture is already active");
    state_->arena->capturing = true;
}

void Runtime::end_graph_allocation_capture() const noexcept {
    std::lock_guard<std::mutex> lock(state_->arena->mu);
    state_->arena->capturing = false;
}

void Runtime::release_graph_allocations() const {
    DeviceArena& a = *state_->arena;
    std::lock_guard<std::mutex> lock(a.mu);
    for (auto& [p, bytes] : a.graph_held) {
        a.stats.graph_held_bytes -= bytes;
        a.cache_or_free(p, bytes);
    }
    a.graph_held.clear();
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

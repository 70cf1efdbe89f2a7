// Runtime, error and backend-selection types of the sdxl_hip C++20 host API.
//
// Mirrors the reference's include/sdxl/cuda/runtime.hpp (AttentionBackend at
// :53-58, parse/name at :60-61, RuntimeOptions::attention_backend at :96,
// Runtime at :127-161) for the attention path: one device, one stream per
// Runtime, exceptions for every failure.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace sdxl::hip {

// Thrown for every failure (reference CudaError, runtime.hpp:18-21).
class HipError final : public std::runtime_error {
public:
    explicit HipError(const std::string& message) : std::runtime_error(message) {}
};

void check_hip(hipError_t status, std::string_view expression, std::string_view file, int line);
#define SDXL_HIP_CHECK(expr) ::sdxl::hip::check_hip((expr), #expr, __FILE__, __LINE__)

// Same enumerators and spellings as the reference. On MI355X CuDnnSDPA and
// FlashSM80 both run the fused gfx950 kernel (flash-gfx950); WarpOnline runs
// the wave64 online-softmax kernel; Auto picks the fused kernel whenever it is
// eligible (head_dim 64, fp16/bf16), else WarpOnline.
enum class AttentionBackend : std::uint8_t { Auto, CuDnnSDPA, FlashSM80, WarpOnline };

[[nodiscard]] AttentionBackend parse_attention_backend(std::string_view value);
[[nodiscard]] const char* attention_backend_name(AttentionBackend backend) noexcept;

struct RuntimeOptions {
    int device = 0;
    AttentionBackend attention_backend = AttentionBackend::Auto;
    // Record an event pair around every Ops call (reference ProfileScope,
    // include/sdxl/cuda/profiler.hpp:32-53); read with Runtime::profile_records().
    bool profile = false;
    // Bytes of freed device blocks the arena keeps for reuse (reference
    // RuntimeOptions::arena_cache_limit_bytes, runtime.hpp:80); 0 frees at once.
    std::size_t arena_cache_limit_bytes = std::numeric_limits<std::size_t>::max();
};

// Device-memory arena counters (reference MemoryArenaStats, runtime.hpp:114-125).
struct MemoryArenaStats {
    std::size_t live_bytes = 0;         // held by live tensors
    std::size_t cached_bytes = 0;       // freed blocks kept for reuse
    std::size_t peak_live_bytes = 0;
    std::size_t driver_allocations = 0; // hipMalloc calls
    std::size_t cache_hits = 0;         // allocations served from the cache
    std::size_t graph_held_bytes = 0;   // freed blocks a captured graph may still use
};

struct ProfileRecord {
    std::string label;
    float milliseconds = 0.0F;
};

struct RuntimeState;

class Runtime final {
public:
    explicit Runtime(RuntimeOptions options = {});
    ~Runtime();
    Runtime(const Runtime&) = delete;
    Runtime& operator=(const Runtime&) = delete;
    Runtime(Runtime&&) noexcept = default;
    Runtime& operator=(Runtime&&) noexcept = default;

    [[nodiscard]] hipStream_t stream() const noexcept;
    [[nodiscard]] int device() const noexcept;
    [[nodiscard]] const RuntimeOptions& options() const noexcept;
    void synchronize() const;

    // Opens an event-pair scope on the runtime stream; returns an id for end_profile.
    // No-op (returns -1) unless RuntimeOptions::profile is set. Never synchronises.
    [[nodiscard]] int begin_profile(std::string label) const;
    void end_profile(int id) const;
    // Synchronises and resolves every recorded scope, in order.
    [[nodiscard]] std::vector<ProfileRecord> profile_records() const;

    // Device memory for tensors: a caching arena of exact-size blocks (256-byte
    // granules). A freed block returns to the cache (up to the option's limit)
    // and a later allocation of the same size reuses it without a hipMalloc, so
    // a call sequence repeated after one warm-up pass allocates nothing from
    // the driver. The deleter of the returned pointer gives the block back.
    [[nodiscard]] std::shared_ptr<void> allocate_device(std::size_t bytes) const;
    [[nodiscard]] MemoryArenaStats memory_arena_stats() const noexcept;
    // Frees every cached block (hipFree); live and graph-held blocks stay.
    void trim_memory_arena() const;

    // HIP graph capture of Ops calls (reference runtime.hpp:153-157). Between
    // begin and end, allocations must be served from the cache (run the
    // sequence once eagerly first): a size with no cached block throws
    // HipError, since no driver allocation can be recorded into the capture.
    // Every block allocated in this window, and every block freed in it (a
    // graph input whose tensor dies inside the captured sequence), is held
    // when its tensor is freed instead of re-entering the cache, because
    // replays of the captured graph keep reading and writing it.
    // release_graph_allocations() returns the held blocks to the cache once
    // the graphs that use them are destroyed. Outside a capture, a hipMalloc
    // that runs out of memory frees the cached blocks and retries once.
    void begin_graph_allocation_capture() const;
    void end_graph_allocation_capture() const noexcept;
    void release_graph_allocations() const;

private:
    std::unique_ptr<RuntimeState> state_;
};

}  // namespace sdxl::hip

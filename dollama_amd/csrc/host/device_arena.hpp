// VRAM bump arena with mark / rewind (LIFO scopes), reserve / release and
// allocation statistics.
//
// Keeps the API surface of the reference's device arena
// (src/kernels/device_arena.cuh:108-297): DeviceArenaId {UNet, VAE,
// UNetPersist}, DeviceArenaMark, DeviceArenaStats, device_arena_{mark,alloc,
// rewind,reserve,release,release_noexcept,stats,reset_counters,
// first_chunk_bytes,pool_enabled} and the RAII DeviceArenaScope.  Behaviour:
//   - chunks are device allocations obtained through dlm_malloc; a rewind
//     never frees chunks, so a steady-state forward performs no allocation;
//   - allocations are 256-byte aligned (kDeviceArenaAlign);
//   - one owner thread at a time; another thread may take ownership only
//     while the arena holds no live allocation, otherwise the call throws
//     (reference device_arena.cu:161-184);
//   - DOLLAMA_POOL=0 turns the pool off: every alloc is its own dlm_malloc
//     and a rewind frees what was allocated after the mark.
#pragma once

#include <cstddef>
#include <cstdint>

namespace dollama {

enum class DeviceArenaId : int { UNet = 0, VAE = 1, UNetPersist = 2 };
static constexpr int kDeviceArenaCount = 3;
static constexpr size_t kDeviceArenaAlign = 256;

const char* device_arena_name(DeviceArenaId id);

struct DeviceArenaMark {
  DeviceArenaId id = DeviceArenaId::UNet;
  size_t chunk = 0;
  size_t offset = 0;
  size_t fallback_count = 0;
  size_t req_bytes = 0;
};

struct DeviceArenaStats {
  uint64_t cuda_malloc_calls = 0;  // device allocations made (cumulative)
  uint64_t cuda_free_calls = 0;    // device frees made (cumulative)
  uint64_t chunk_alloc_calls = 0;  // new chunks (pool mode, cumulative)
  uint64_t alloc_calls = 0;        // alloc() calls (cumulative)
  size_t total_capacity = 0;       // bytes held in chunks now
  size_t live_chunks = 0;
  size_t bytes_in_use = 0;         // bump-cursor based
  size_t peak_bytes_in_use = 0;
  size_t live_request_bytes = 0;   // aligned bytes of live allocations
  size_t peak_request_bytes = 0;
  size_t reserved_bytes = 0;
};

bool device_arena_pool_enabled();
DeviceArenaMark device_arena_mark(DeviceArenaId id);
void* device_arena_alloc(DeviceArenaId id, size_t bytes);
void device_arena_rewind(const DeviceArenaMark& mark);
void device_arena_reserve(DeviceArenaId id, size_t bytes);
void device_arena_release(DeviceArenaId id);
bool device_arena_release_noexcept(DeviceArenaId id) noexcept;
DeviceArenaStats device_arena_stats(DeviceArenaId id);
void device_arena_reset_counters(DeviceArenaId id);
size_t device_arena_first_chunk_bytes(DeviceArenaId id);
// Fill every byte the arena holds (all chunks) with `pattern`, synchronously;
// throws std::runtime_error while allocations are live.  A determinism check:
// scratch that a computation reads before writing shows up as a changed
// result after the arena was filled with different patterns.
void device_arena_fill(DeviceArenaId id, int pattern);
// Changes whenever the arena's chunk list changes (new chunk, reserve,
// release): equal epoch and equal mark mean that the same sequence of
// allocations returns the same addresses (used to reuse captured graphs).
uint64_t device_arena_epoch(DeviceArenaId id);

class DeviceArenaScope {
 public:
  explicit DeviceArenaScope(DeviceArenaId id) : mark_(device_arena_mark(id)) {}
  ~DeviceArenaScope() {
    try {
      device_arena_rewind(mark_);
    } catch (...) {
    }
  }
  DeviceArenaScope(const DeviceArenaScope&) = delete;
  DeviceArenaScope& operator=(const DeviceArenaScope&) = delete;

  template <typename T>
  T* alloc(size_t count) {
    return static_cast<T*>(device_arena_alloc(mark_.id, count * sizeof(T)));
  }
  void* alloc_bytes(size_t bytes) { return device_arena_alloc(mark_.id, bytes); }
  DeviceArenaId id() const { return mark_.id; }

 private:
  DeviceArenaMark mark_;
};

}  // namespace dollama

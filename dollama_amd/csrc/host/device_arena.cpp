// Device arena implementation (see device_arena.hpp for the contract).
#include "device_arena.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "check.hpp"

namespace dollama {
namespace {

constexpr size_t kMinChunk = size_t(64) << 20;  // 64 MiB

struct Chunk {
  void* ptr = nullptr;
  size_t bytes = 0;
};

struct Arena {
  std::mutex mu;
  std::vector<Chunk> chunks;
  size_t cur_chunk = 0;   // chunk the cursor is in
  size_t cur_off = 0;     // cursor within cur_chunk
  size_t reserved = 0;
  std::thread::id owner{};
  bool has_owner = false;
  // pool-off mode: every allocation is a separate block, freed on rewind
  std::vector<void*> direct;
  DeviceArenaStats st;
  uint64_t epoch = 0;  // bumped whenever the chunk list changes
};

Arena g_arenas[kDeviceArenaCount];

Arena& arena(DeviceArenaId id) {
  const int i = static_cast<int>(id);
  if (i < 0 || i >= kDeviceArenaCount) throw std::invalid_argument("device_arena: bad id");
  return g_arenas[i];
}

size_t align_up(size_t x) { return (x + kDeviceArenaAlign - 1) & ~(kDeviceArenaAlign - 1); }

bool live(const Arena& a) { return a.st.live_request_bytes != 0 || !a.direct.empty(); }

// Enforce the single-owner rule; ownership moves only when quiescent.
void claim(Arena& a, DeviceArenaId id) {
  const auto me = std::this_thread::get_id();
  if (!a.has_owner) {
    a.owner = me;
    a.has_owner = true;
    return;
  }
  if (a.owner == me) return;
  if (live(a))
    throw std::runtime_error(std::string("device_arena: arena ") + device_arena_name(id) +
                             " used from a second thread while allocations are live");
  a.owner = me;
}

size_t bytes_before(const Arena& a, size_t chunk, size_t off) {
  size_t b = off;
  for (size_t i = 0; i < chunk && i < a.chunks.size(); ++i) b += a.chunks[i].bytes;
  return b;
}

}  // namespace

const char* device_arena_name(DeviceArenaId id) {
  switch (id) {
    case DeviceArenaId::UNet: return "UNet";
    case DeviceArenaId::VAE: return "VAE";
    case DeviceArenaId::UNetPersist: return "UNetPersist";
  }
  return "?";
}

bool device_arena_pool_enabled() {
  static const bool enabled = [] {
    const char* v = std::getenv("DOLLAMA_POOL");
    return !(v && std::strcmp(v, "0") == 0);
  }();
  return enabled;
}

DeviceArenaMark device_arena_mark(DeviceArenaId id) {
  Arena& a = arena(id);
  std::lock_guard<std::mutex> lock(a.mu);
  claim(a, id);
  DeviceArenaMark m;
  m.id = id;
  m.chunk = a.cur_chunk;
  m.offset = a.cur_off;
  m.fallback_count = a.direct.size();
  m.req_bytes = a.st.live_request_bytes;
  return m;
}

void* device_arena_alloc(DeviceArenaId id, size_t bytes) {
  Arena& a = arena(id);
  std::lock_guard<std::mutex> lock(a.mu);
  claim(a, id);
  const size_t need = align_up(bytes == 0 ? 1 : bytes);
  a.st.alloc_calls++;
  if (!device_arena_pool_enabled()) {
    void* p = nullptr;
    DLM_CALL(dlm_malloc(&p, need));
    a.st.cuda_malloc_calls++;
    a.direct.push_back(p);
    a.st.live_request_bytes += need;
    a.st.peak_request_bytes = std::max(a.st.peak_request_bytes, a.st.live_request_bytes);
    return p;
  }
  // find room from the cursor onward
  while (true) {
    if (a.cur_chunk < a.chunks.size()) {
      Chunk& c = a.chunks[a.cur_chunk];
      if (a.cur_off + need <= c.bytes) {
        void* p = static_cast<char*>(c.ptr) + a.cur_off;
        a.cur_off += need;
        a.st.live_request_bytes += need;
        a.st.peak_request_bytes = std::max(a.st.peak_request_bytes, a.st.live_request_bytes);
        a.st.bytes_in_use = bytes_before(a, a.cur_chunk, a.cur_off);
        a.st.peak_bytes_in_use = std::max(a.st.peak_bytes_in_use, a.st.bytes_in_use);
        return p;
      }
      if (a.cur_chunk + 1 < a.chunks.size()) {
        a.cur_chunk++;
        a.cur_off = 0;
        continue;
      }
    }
    // append a new chunk large enough for this request
    Chunk c;
    c.bytes = std::max(need, a.chunks.empty() ? std::max(kMinChunk, a.reserved) : kMinChunk);
    DLM_CALL(dlm_malloc(&c.ptr, c.bytes));
    a.st.cuda_malloc_calls++;
    a.st.chunk_alloc_calls++;
    a.chunks.push_back(c);
    a.epoch++;
    a.st.total_capacity += c.bytes;
    a.st.live_chunks = a.chunks.size();
    a.cur_chunk = a.chunks.size() - 1;
    a.cur_off = 0;
  }
}

uint64_t device_arena_epoch(DeviceArenaId id) {
  Arena& a = arena(id);
  std::lock_guard<std::mutex> lock(a.mu);
  // pool-off mode hands out fresh blocks on every allocation: no two calls
  // see the same addresses, so every call is a new epoch
  return device_arena_pool_enabled() ? a.epoch : ++a.epoch;
}

void device_arena_rewind(const DeviceArenaMark& m) {
  Arena& a = arena(m.id);
  std::lock_guard<std::mutex> lock(a.mu);
  claim(a, m.id);
  if (!device_arena_pool_enabled()) {
    while (a.direct.size() > m.fallback_count) {
      DLM_CALL(dlm_free(a.direct.back()));
      a.st.cuda_free_calls++;
      a.direct.pop_back();
    }
  } else {
    if (m.chunk > a.cur_chunk || (m.chunk == a.cur_chunk && m.offset > a.cur_off))
      throw std::runtime_error("device_arena_rewind: mark is ahead of the cursor (non-LIFO use)");
    a.cur_chunk = m.chunk;
    a.cur_off = m.offset;
    a.st.bytes_in_use = bytes_before(a, a.cur_chunk, a.cur_off);
  }
  a.st.live_request_bytes = m.req_bytes;
}

void device_arena_reserve(DeviceArenaId id, size_t bytes) {
  Arena& a = arena(id);
  std::lock_guard<std::mutex> lock(a.mu);
  claim(a, id);
  // with the pool off there are no chunks to replace: a no-op, as in the
  // reference (device_arena.cu reserve under DOLLAMA_POOL=0)
  if (!device_arena_pool_enabled()) return;
  if (live(a)) throw std::runtime_error("device_arena_reserve: arena is not quiescent");
  a.reserved = bytes;
  if (!a.chunks.empty() && a.chunks.front().bytes >= bytes) return;
  for (Chunk& c : a.chunks) {
    DLM_CALL(dlm_free(c.ptr));
    a.st.cuda_free_calls++;
  }
  a.chunks.clear();
  a.epoch++;
  a.st.total_capacity = 0;
  Chunk c;
  c.bytes = std::max(align_up(bytes), kDeviceArenaAlign);
  DLM_CALL(dlm_malloc(&c.ptr, c.bytes));
  a.st.cuda_malloc_calls++;
  a.st.chunk_alloc_calls++;
  a.chunks.push_back(c);
  a.st.total_capacity = c.bytes;
  a.st.live_chunks = 1;
  a.cur_chunk = 0;
  a.cur_off = 0;
  a.st.reserved_bytes = c.bytes;
}

void device_arena_release(DeviceArenaId id) {
  Arena& a = arena(id);
  std::lock_guard<std::mutex> lock(a.mu);
  claim(a, id);
  if (live(a)) throw std::runtime_error("device_arena_release: arena is not quiescent");
  for (Chunk& c : a.chunks) {
    DLM_CALL(dlm_free(c.ptr));
    a.st.cuda_free_calls++;
  }
  a.chunks.clear();
  a.epoch++;
  a.cur_chunk = 0;
  a.cur_off = 0;
  a.st.total_capacity = 0;
  a.st.live_chunks = 0;
  a.st.bytes_in_use = 0;
  a.st.reserved_bytes = 0;
}

void device_arena_fill(DeviceArenaId id, int pattern) {
  Arena& a = arena(id);
  std::lock_guard<std::mutex> lock(a.mu);
  claim(a, id);
  if (live(a)) throw std::runtime_error("device_arena_fill: arena is not quiescent");
  for (const Chunk& c : a.chunks) DLM_CALL(dlm_memset_async(c.ptr, pattern & 0xFF, c.bytes, nullptr));
  DLM_CALL(dlm_device_synchronize());
}

bool device_arena_release_noexcept(DeviceArenaId id) noexcept {
  try {
    device_arena_release(id);
    return true;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "[device_arena] release of %s refused: %s\n", device_arena_name(id), e.what());
    return false;
  }
}

DeviceArenaStats device_arena_stats(DeviceArenaId id) {
  Arena& a = arena(id);
  std::lock_guard<std::mutex> lock(a.mu);
  return a.st;
}

void device_arena_reset_counters(DeviceArenaId id) {
  Arena& a = arena(id);
  std::lock_guard<std::mutex> lock(a.mu);
  a.st.cuda_malloc_calls = 0;
  a.st.cuda_free_calls = 0;
  a.st.chunk_alloc_calls = 0;
  a.st.alloc_calls = 0;
  a.st.peak_bytes_in_use = a.st.bytes_in_use;
  a.st.peak_request_bytes = a.st.live_request_bytes;
}

size_t device_arena_first_chunk_bytes(DeviceArenaId id) {
  Arena& a = arena(id);
  std::lock_guard<std::mutex> lock(a.mu);
  return a.chunks.empty() ? 0 : a.chunks.front().bytes;
}

}  // namespace dollama

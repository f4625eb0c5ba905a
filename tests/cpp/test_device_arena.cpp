// Contract checks of the device arena (host/device_arena.hpp), following the
// cases of the reference's src/tests/test_device_arena.cu: LIFO rewind,
// alignment, steady state, arena isolation, release / reserve, the owner
// thread rule, release_noexcept, scope RAII, reserve overflow with live
// pointers, the quiescence rule of reserve, fill, and the DOLLAMA_POOL=0
// variant (run this program a second time with that variable set).
// Needs a GPU (the arena's chunks are device memory).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <thread>
#include <vector>

#include "device_arena.hpp"
#include "dlm.h"

using namespace dollama;

static int g_fail = 0;
#define EXPECT(cond)                                                  \
  do {                                                                \
    if (!(cond)) {                                                    \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);     \
      ++g_fail;                                                       \
    }                                                                 \
  } while (0)

template <typename F>
static bool throws(F&& f) {
  try {
    f();
  } catch (const std::exception&) {
    return true;
  }
  return false;
}

static void fill(void* p, int v, size_t n) {
  EXPECT(dlm_memset_async(p, v, n, nullptr) == DLM_OK);
  EXPECT(dlm_device_synchronize() == DLM_OK);
}
static bool holds(const void* p, int v, size_t n) {
  std::vector<unsigned char> h(n);
  if (dlm_memcpy(h.data(), p, n, 1) != DLM_OK) return false;
  for (unsigned char c : h)
    if (c != (unsigned char)v) return false;
  return true;
}

static const bool kPool = device_arena_pool_enabled();

static void test_lifo_and_alignment() {
  const DeviceArenaId id = DeviceArenaId::UNet;
  DeviceArenaMark m0 = device_arena_mark(id);
  void* a = device_arena_alloc(id, 1000);
  void* b = device_arena_alloc(id, 1);
  EXPECT(((uintptr_t)a % kDeviceArenaAlign) == 0 && ((uintptr_t)b % kDeviceArenaAlign) == 0);
  DeviceArenaMark m1 = device_arena_mark(id);
  void* c = device_arena_alloc(id, 4096);
  device_arena_rewind(m1);
  void* c2 = device_arena_alloc(id, 4096);
  if (kPool) {
    EXPECT(c2 == c);  // the rewound region is handed out again
    EXPECT((char*)b - (char*)a == 1024);
  }
  device_arena_rewind(m1);
  device_arena_rewind(m0);
  if (kPool) {
    // a mark that is ahead of the cursor (non-LIFO use) is refused
    EXPECT(throws([&] { device_arena_rewind(m1); }));
  }
  EXPECT(device_arena_stats(id).live_request_bytes == 0);
}

static void test_steady_state() {
  const DeviceArenaId id = DeviceArenaId::UNet;
  auto pass = [&] {
    DeviceArenaScope sc(id);
    for (int i = 0; i < 8; ++i) (void)sc.alloc<float>(size_t(1) << 18);
  };
  pass();
  device_arena_reset_counters(id);
  for (int r = 0; r < 3; ++r) pass();
  const DeviceArenaStats s = device_arena_stats(id);
  EXPECT(s.alloc_calls == 24);
  if (kPool)
    EXPECT(s.cuda_malloc_calls == 0);  // warm passes reuse the chunks
  else
    EXPECT(s.cuda_malloc_calls == 24 && s.cuda_free_calls == 24);
  EXPECT(s.live_request_bytes == 0);
}

static void test_isolation() {
  DeviceArenaMark mu = device_arena_mark(DeviceArenaId::UNet);
  DeviceArenaMark mv = device_arena_mark(DeviceArenaId::VAE);
  void* u = device_arena_alloc(DeviceArenaId::UNet, 1 << 20);
  void* v = device_arena_alloc(DeviceArenaId::VAE, 1 << 20);
  EXPECT(u != v);
  fill(u, 0x11, 1 << 20);
  fill(v, 0x22, 1 << 20);
  device_arena_rewind(mv);
  EXPECT(holds(u, 0x11, 1 << 20));  // rewinding VAE leaves UNet's allocation alone
  EXPECT(device_arena_stats(DeviceArenaId::VAE).live_request_bytes == 0);
  EXPECT(device_arena_stats(DeviceArenaId::UNet).live_request_bytes >= (1u << 20));
  device_arena_rewind(mu);
}

static void test_thread_guard() {
  const DeviceArenaId id = DeviceArenaId::UNet;
  DeviceArenaMark m = device_arena_mark(id);
  void* p = device_arena_alloc(id, 1024);
  EXPECT(p != nullptr);
  bool threw_alloc = false, threw_mark = false;
  std::thread t1([&] { threw_alloc = throws([&] { (void)device_arena_alloc(id, 1024); }); });
  t1.join();
  std::thread t2([&] { threw_mark = throws([&] { (void)device_arena_mark(id); }); });
  t2.join();
  EXPECT(threw_alloc && threw_mark);  // a second thread while allocations are live
  device_arena_rewind(m);
  // quiescent: ownership moves to the next thread, then back
  bool handoff = false;
  std::thread t3([&] {
    handoff = !throws([&] {
      DeviceArenaScope sc(id);
      void* q = sc.alloc_bytes(4096);
      if (!q) throw std::runtime_error("null");
    });
  });
  t3.join();
  EXPECT(handoff);
  EXPECT(!throws([&] {
    DeviceArenaScope sc(id);
    (void)sc.alloc_bytes(64);
  }));
}

static void test_release_and_noexcept() {
  const DeviceArenaId id = DeviceArenaId::VAE;
  DeviceArenaMark m = device_arena_mark(id);
  (void)device_arena_alloc(id, 1 << 20);
  EXPECT(throws([&] { device_arena_release(id); }));
  EXPECT(!device_arena_release_noexcept(id));
  device_arena_rewind(m);
  EXPECT(device_arena_release_noexcept(id));
  const DeviceArenaStats s = device_arena_stats(id);
  EXPECT(s.total_capacity == 0 && s.live_chunks == 0);
  EXPECT(device_arena_first_chunk_bytes(id) == 0);
  // usable again after release
  DeviceArenaScope sc(id);
  void* p = sc.alloc_bytes(4 << 20);
  fill(p, 0x33, 4 << 20);
  EXPECT(holds(p, 0x33, 4 << 20));
}

static void test_scope_raii() {
  const DeviceArenaId id = DeviceArenaId::UNet;
  const size_t before = device_arena_stats(id).live_request_bytes;
  {
    DeviceArenaScope a(id);
    (void)a.alloc<uint16_t>(1000);
    {
      DeviceArenaScope b(id);
      (void)b.alloc<float>(5000);
      EXPECT(device_arena_stats(id).live_request_bytes > before);
    }
    EXPECT(device_arena_stats(id).live_request_bytes == before + 2048);
  }
  EXPECT(device_arena_stats(id).live_request_bytes == before);
}

static void test_reserve() {
  const DeviceArenaId id = DeviceArenaId::UNetPersist;
  device_arena_release(id);
  // reserve while live: refused with the pool on (it would free live chunks),
  // a no-op with the pool off
  DeviceArenaMark m = device_arena_mark(id);
  (void)device_arena_alloc(id, 4 << 20);
  const bool threw = throws([&] { device_arena_reserve(id, size_t(256) << 20); });
  EXPECT(kPool ? threw : !threw);
  device_arena_rewind(m);
  EXPECT(!throws([&] { device_arena_reserve(id, size_t(96) << 20); }));
  if (!kPool) return;
  EXPECT(device_arena_first_chunk_bytes(id) >= (size_t(96) << 20));
  device_arena_reset_counters(id);
  {
    // fits in the reserved chunk: no chunk growth
    DeviceArenaScope sc(id);
    for (int i = 0; i < 4; ++i) (void)sc.alloc_bytes(size_t(16) << 20);
  }
  EXPECT(device_arena_stats(id).chunk_alloc_calls == 0);
  // overflow: a further chunk is added, live pointers keep their contents
  DeviceArenaMark m2 = device_arena_mark(id);
  std::vector<void*> ps;
  for (int i = 0; i < 8; ++i) {
    void* p = device_arena_alloc(id, size_t(16) << 20);
    fill(p, 0x40 + i, size_t(16) << 20);
    ps.push_back(p);
  }
  bool intact = true;
  for (int i = 0; i < 8; ++i) intact = intact && holds(ps[i], 0x40 + i, size_t(16) << 20);
  EXPECT(intact);
  EXPECT(device_arena_stats(id).chunk_alloc_calls >= 1);
  device_arena_rewind(m2);
  device_arena_release(id);
}

static void test_fill() {
  const DeviceArenaId id = DeviceArenaId::UNet;
  DeviceArenaMark m = device_arena_mark(id);
  void* p = device_arena_alloc(id, 1 << 20);
  EXPECT(throws([&] { device_arena_fill(id, 0xFF); }));  // live allocations
  device_arena_rewind(m);
  if (!kPool) return;
  device_arena_fill(id, 0x5A);
  DeviceArenaMark m2 = device_arena_mark(id);
  void* q = device_arena_alloc(id, 1 << 20);
  EXPECT(q == p && holds(q, 0x5A, 1 << 20));
  device_arena_rewind(m2);
}

int main() {
  int n = 0;
  if (dlm_get_device_count(&n) != DLM_OK || n <= 0) {
    std::printf("FAIL: no GPU\n");
    return 1;
  }
  test_lifo_and_alignment();
  test_steady_state();
  test_isolation();
  test_thread_guard();
  test_release_and_noexcept();
  test_scope_raii();
  test_reserve();
  test_fill();
  std::printf("pool=%d: %d failure(s)\n", kPool ? 1 : 0, g_fail);
  return g_fail == 0 ? 0 : 1;
}

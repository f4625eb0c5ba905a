// Contract checks of dollama::Tensor and the allocators (host/tensor.hpp,
// host/allocator.hpp), following the cases of the reference's own
// src/tests/test_tensor.cpp and src/tests/test_allocator.cpp.
// Usage: test_tensor_allocator cpu   (no GPU visible: fallback / throw paths)
//        test_tensor_allocator gpu   (GPU present: pinned + device round trip)
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "allocator.hpp"
#include "tensor.hpp"

using namespace dollama;

static int g_fail = 0;
#define EXPECT(cond)                                                  \
  do {                                                                \
    if (!(cond)) {                                                    \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);     \
      ++g_fail;                                                       \
    }                                                                 \
  } while (0)

template <typename E, typename F>
static bool throws(F&& f) {
  try {
    f();
  } catch (const E&) {
    return true;
  } catch (...) {
    return false;
  }
  return false;
}

static void tensor_cases() {
  Tensor t({2, 3, 4});
  EXPECT(t.numel() == 24 && t.ndim() == 3 && t.dim(1) == 3 && t.nbytes() == 24 * sizeof(float));
  EXPECT(t.device() == Device::CPU);
  EXPECT(throws<std::out_of_range>([&] { (void)t.dim(3); }));
  bool zero = true;
  for (size_t i = 0; i < t.numel(); ++i) zero = zero && t.data()[i] == 0.0f;
  EXPECT(zero);
  for (size_t i = 0; i < t.numel(); ++i) t.data()[i] = 1.5f * (float)i;
  const Tensor& ct = t;
  EXPECT(ct.data()[7] == 10.5f);
  EXPECT(t.data_ptr() == static_cast<void*>(t.data()));

  Tensor p({5}, Device::PINNED);
  EXPECT(p.numel() == 5 && p.data() != nullptr && p.data()[4] == 0.0f);

  Tensor empty;
  EXPECT(empty.numel() == 0 && empty.nbytes() == 0 && empty.ndim() == 0);

  for (Device d : {Device::CUDA, Device::NPU}) {
    Tensor g({8, 8}, d);
    EXPECT(g.numel() == 64 && g.nbytes() == 256);
    EXPECT(throws<std::logic_error>([&] { (void)g.data(); }));
    EXPECT(throws<std::logic_error>([&] { (void)static_cast<const Tensor&>(g).data(); }));
    EXPECT(throws<std::logic_error>([&] { (void)g.data_ptr(); }));
    int x = 0;
    g.set_data_ptr(&x);
    EXPECT(g.data_ptr() == &x);
  }
  // an external pointer also overrides host storage
  Tensor h({3});
  float ext[3] = {1, 2, 3};
  h.set_data_ptr(ext);
  EXPECT(h.data_ptr() == ext);
}

static void buffer_cases() {
  void* raw = PinnedAllocator::alloc(1024);
  EXPECT(raw != nullptr);
  std::memset(raw, 0xA5, 1024);
  PinnedAllocator::free(raw);
  PinnedAllocator::free(nullptr);

  PinnedBuffer a(512);
  void* orig = a.get();
  EXPECT(orig != nullptr && a.size() == 512);
  PinnedBuffer b(std::move(a));
  EXPECT(b.get() == orig && b.size() == 512 && a.get() == nullptr && a.size() == 0);
  PinnedBuffer c(128);
  c = std::move(b);
  EXPECT(c.get() == orig && c.size() == 512 && b.get() == nullptr && b.size() == 0);
  PinnedBuffer& self = c;
  c = std::move(self);
  EXPECT(c.get() == orig && c.size() == 512);
  static_cast<unsigned char*>(c.get())[511] = 7;
  EXPECT(static_cast<unsigned char*>(c.get())[511] == 7);
}

static void cpu_only_cases() {
  // no GPU visible: device allocations are refused with std::runtime_error
  EXPECT(throws<std::runtime_error>([] { (void)CudaAllocator::alloc(1); }));
  EXPECT(throws<std::runtime_error>([] { CudaBuffer b(16); }));
  CudaAllocator::free(nullptr);
}

static void gpu_cases() {
  const size_t n = 1 << 20;
  CudaBuffer dev(n * sizeof(float));
  EXPECT(dev.get() != nullptr && dev.size() == n * sizeof(float));
  PinnedBuffer up(n * sizeof(float)), down(n * sizeof(float));
  float* u = static_cast<float*>(up.get());
  for (size_t i = 0; i < n; ++i) u[i] = (float)i * 0.25f - 7.0f;
  EXPECT(dlm_memcpy(dev.get(), up.get(), dev.size(), 0) == DLM_OK);
  std::memset(down.get(), 0, down.size());
  EXPECT(dlm_memcpy(down.get(), dev.get(), dev.size(), 1) == DLM_OK);
  EXPECT(std::memcmp(up.get(), down.get(), up.size()) == 0);
  // a device Tensor views the buffer
  Tensor t({1024, 1024}, Device::CUDA);
  t.set_data_ptr(dev.get());
  EXPECT(t.data_ptr() == dev.get() && t.nbytes() == dev.size());
  // move semantics with device memory: the old owner no longer frees it
  CudaBuffer moved(std::move(dev));
  EXPECT(moved.get() != nullptr && dev.get() == nullptr);
  CudaBuffer other(64);
  other = std::move(moved);
  EXPECT(other.size() == n * sizeof(float));
  EXPECT(throws<std::runtime_error>([] { (void)CudaAllocator::alloc(size_t(1) << 62); }));
}

int main(int argc, char** argv) {
  const std::string mode = argc > 1 ? argv[1] : "cpu";
  tensor_cases();
  buffer_cases();
  if (mode == "gpu") {
    int count = 0;
    if (dlm_get_device_count(&count) != DLM_OK || count <= 0) {
      std::printf("FAIL: gpu mode without a GPU\n");
      return 1;
    }
    gpu_cases();
  } else {
    cpu_only_cases();
  }
  std::printf("%s: %d failure(s)\n", mode.c_str(), g_fail);
  return g_fail == 0 ? 0 : 1;
}

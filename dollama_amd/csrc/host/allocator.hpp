// Host-pinned and GPU allocators with an RAII owner: the reference's
// allocator surface (src/core/allocator.hpp:16-130: PinnedAllocator,
// CudaAllocator, UniqueBuffer, PinnedBuffer, CudaBuffer), same names and
// error behaviour, over this library's C ABI (dlm_host_malloc_pinned /
// dlm_malloc, include/dlm.h) instead of the CUDA runtime.
//
// - PinnedAllocator::alloc returns page-locked host memory (hipHostMalloc)
//   when a GPU is present; in a process that sees no GPU it returns ordinary
//   host memory, as the reference's build without a GPU runtime does.
// - CudaAllocator::alloc returns GPU device memory; it throws
//   std::runtime_error when the allocation fails or no GPU is present.
// - free() of either never throws; free(nullptr) is a no-op.
#pragma once

#include <cstddef>
#include <new>
#include <stdexcept>
#include <string>

#include "dlm.h"

namespace dollama {

namespace detail {
// Whether this process sees a GPU (fixed for the process's lifetime, so alloc
// and free of PinnedAllocator always take the same branch).
inline bool gpu_present() {
  static const bool present = [] {
    int n = 0;
    return dlm_get_device_count(&n) == DLM_OK && n > 0;
  }();
  return present;
}
}  // namespace detail

struct PinnedAllocator {
  static void* alloc(size_t bytes) {
    if (!detail::gpu_present()) return ::operator new(bytes);
    void* p = nullptr;
    if (dlm_host_malloc_pinned(&p, bytes) != DLM_OK)
      throw std::runtime_error(std::string("PinnedAllocator: ") + dlm_last_error());
    return p;
  }
  static void free(void* ptr) noexcept {
    if (!ptr) return;
    if (!detail::gpu_present()) {
      ::operator delete(ptr);
      return;
    }
    (void)dlm_host_free_pinned(ptr);
  }
};

struct CudaAllocator {
  static void* alloc(size_t bytes) {
    if (!detail::gpu_present()) throw std::runtime_error("CudaAllocator: no GPU present");
    void* p = nullptr;
    if (dlm_malloc(&p, bytes) != DLM_OK)
      throw std::runtime_error(std::string("CudaAllocator: ") + dlm_last_error());
    return p;
  }
  static void free(void* ptr) noexcept {
    if (ptr) (void)dlm_free(ptr);
  }
};

// Owns one allocation of Alloc; move-only.  A moved-from buffer holds
// nullptr and size 0; move assignment frees the target's old block first.
template <typename Alloc>
class UniqueBuffer {
 public:
  explicit UniqueBuffer(size_t bytes) : ptr_(Alloc::alloc(bytes)), bytes_(bytes) {}
  ~UniqueBuffer() { Alloc::free(ptr_); }

  UniqueBuffer(const UniqueBuffer&) = delete;
  UniqueBuffer& operator=(const UniqueBuffer&) = delete;

  UniqueBuffer(UniqueBuffer&& o) noexcept : ptr_(o.ptr_), bytes_(o.bytes_) {
    o.ptr_ = nullptr;
    o.bytes_ = 0;
  }
  UniqueBuffer& operator=(UniqueBuffer&& o) noexcept {
    if (this != &o) {
      Alloc::free(ptr_);
      ptr_ = o.ptr_;
      bytes_ = o.bytes_;
      o.ptr_ = nullptr;
      o.bytes_ = 0;
    }
    return *this;
  }

  void* get() const noexcept { return ptr_; }
  size_t size() const noexcept { return bytes_; }

 private:
  void* ptr_ = nullptr;
  size_t bytes_ = 0;
};

using PinnedBuffer = UniqueBuffer<PinnedAllocator>;
using CudaBuffer = UniqueBuffer<CudaAllocator>;

}  // namespace dollama

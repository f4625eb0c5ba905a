// Device / Tensor: the host-side tensor type callers of the reference pass
// around (reference src/core/tensor.hpp:9-119), with the same names, members
// and error behaviour so that code written against it compiles unchanged.
//
// A Tensor is a shape plus either host storage (Device::CPU, Device::PINNED:
// fp32 elements owned by the tensor, zero-filled on construction) or a
// borrowed external pointer (Device::CUDA = GPU device memory, Device::NPU),
// set with set_data_ptr() after the memory was obtained elsewhere (e.g. a
// CudaBuffer from allocator.hpp).  Host storage of a PINNED tensor is ordinary
// host memory, as in the reference; page-locked staging buffers come from
// PinnedBuffer.
#pragma once

#include <cstddef>
#include <stdexcept>
#include <utility>
#include <vector>

namespace dollama {

enum class Device {
  CPU,     // host heap
  PINNED,  // host memory meant for DMA transfers
  CUDA,    // GPU device memory (HBM of the MI355X here; the name is the reference's)
  NPU,     // external accelerator memory
};

class Tensor {
 public:
  Tensor() = default;
  explicit Tensor(std::vector<size_t> shape, Device dev = Device::CPU)
      : shape_(std::move(shape)), device_(dev) {
    if (on_host()) host_.resize(numel(), 0.0f);
  }

  // Product of the dimensions; an empty shape has no elements.
  size_t numel() const noexcept {
    if (shape_.empty()) return 0;
    size_t n = 1;
    for (size_t d : shape_) n *= d;
    return n;
  }
  const std::vector<size_t>& shape() const noexcept { return shape_; }
  size_t ndim() const noexcept { return shape_.size(); }
  // Throws std::out_of_range for i >= ndim().
  size_t dim(size_t i) const { return shape_.at(i); }

  // Host elements; std::logic_error for a CUDA / NPU tensor.
  float* data() {
    require_host();
    return host_.data();
  }
  const float* data() const {
    require_host();
    return host_.data();
  }

  // Point the tensor at memory it does not own (device or external memory).
  void set_data_ptr(void* ptr) noexcept { ext_ = ptr; }

  // The external pointer when one is set, else the host storage;
  // std::logic_error for a CUDA / NPU tensor that was never given one.
  void* data_ptr() {
    if (ext_) return ext_;
    if (!on_host())
      throw std::logic_error("Tensor::data_ptr(): device tensor without set_data_ptr()");
    return host_.data();
  }

  Device device() const noexcept { return device_; }
  // Bytes of numel() fp32 elements.
  size_t nbytes() const noexcept { return numel() * sizeof(float); }

 private:
  bool on_host() const noexcept { return device_ == Device::CPU || device_ == Device::PINNED; }
  void require_host() const {
    if (!on_host()) throw std::logic_error("Tensor::data(): only CPU / PINNED tensors hold host data");
  }

  std::vector<size_t> shape_;
  std::vector<float> host_;
  void* ext_ = nullptr;
  Device device_ = Device::CPU;
};

}  // namespace dollama

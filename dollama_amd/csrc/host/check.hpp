// Status-to-exception bridge for the C++ host layer.
//
// The host layer reaches HIP only through the C ABI of include/dlm.h; a
// non-zero status becomes std::runtime_error carrying dlm_last_error() and
// the call site, as the reference's CUDA_CHECK does
// (reference src/kernels/utils.cuh:17-45).
#pragma once

#include <stdexcept>
#include <string>

#include "dlm.h"

namespace dollama {

[[noreturn]] inline void throw_dlm(int status, const char* expr, const char* file, int line) {
  throw std::runtime_error(std::string("dlm call failed (status ") + std::to_string(status) +
                           "): " + expr + " at " + file + ":" + std::to_string(line) + ": " +
                           dlm_last_error());
}

}  // namespace dollama

#define DLM_CALL(expr)                                                   \
  do {                                                                   \
    const int st_ = (expr);                                              \
    if (st_ != DLM_OK) ::dollama::throw_dlm(st_, #expr, __FILE__, __LINE__); \
  } while (0)

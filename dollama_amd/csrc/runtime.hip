// Error state, device memory, streams and events of the C ABI.
//
// Replaces the reference's CUDA_CHECK / std::runtime_error reporting
// (src/kernels/utils.cuh:17-45) with int status codes plus a thread-local
// message, and its cudaMalloc/cudaMemcpy call sites
// (src/core/allocator.hpp:16-130, src/kernels/device_arena.cu) with
// dlm_malloc / dlm_memcpy.
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "common.hpp"
#include "dlm_tuning.h"

namespace dlm {

static thread_local std::string g_last_error;
static thread_local const char* g_last_kernel = "";

static thread_local int g_last_dims[4] = {0, 0, 0, 0};

void note_kernel(const char* name) {
  g_last_kernel = name ? name : "";
  g_last_dims[0] = g_last_dims[1] = g_last_dims[2] = g_last_dims[3] = 0;
}
void note_dims(int M, int N, int K, int flags) {
  g_last_dims[0] = M;
  g_last_dims[1] = N;
  g_last_dims[2] = K;
  g_last_dims[3] = flags;
}

ProfArm& prof_arm() {
  static thread_local ProfArm a;
  return a;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what, const char* file, int line) {
  char buf[512];
  std::snprintf(buf, sizeof(buf), "HIP error %d (%s) in %s at %s:%d", (int)e,
                hipGetErrorString(e), what, file, line);
  g_last_error = buf;
  return e == hipErrorOutOfMemory ? DLM_ERR_OUT_OF_MEMORY : DLM_ERR_HIP;
}

// Grow-only staging per (device, stream, slot) for the reference-layout entry
// points that stage NCHW <-> NHWC copies.  Launches on one stream run in order
// and share that stream's slots; another stream gets its own, so calls on two
// streams never race on one buffer.  Growth synchronises the device before
// freeing the old block, so stream-ordered users never see it vanish.
// Bounded: when a request would take the device's total above
// kScratchDeviceCap, the device is synchronised and every slot of the other
// streams on it is freed first (they are re-created on their next use), so a
// caller that cycles through many streams does not accumulate a set per
// stream.  dlm_scratch_release(stream) frees one stream's slots explicitly
// (for a stream about to be destroyed: its handle may be reused by a new
// stream).
namespace {
struct ScratchSlot {
  void* ptr = nullptr;
  size_t bytes = 0;
};
constexpr size_t kScratchDeviceCap = size_t(2) << 30;
std::mutex g_scratch_mu;
std::map<std::tuple<int, hipStream_t, int>, ScratchSlot> g_scratch;

size_t device_total(int dev) {
  size_t t = 0;
  for (const auto& kv : g_scratch)
    if (std::get<0>(kv.first) == dev) t += kv.second.bytes;
  return t;
}

// frees the slots of `dev` whose stream is not `keep`; the caller holds the
// lock and has synchronised the device
bool evict_other_streams(int dev, hipStream_t keep) {
  bool ok = true;
  for (auto it = g_scratch.begin(); it != g_scratch.end();) {
    if (std::get<0>(it->first) == dev && std::get<1>(it->first) != keep) {
      if (it->second.ptr && hipFree(it->second.ptr) != hipSuccess) ok = false;
      it = g_scratch.erase(it);
    } else {
      ++it;
    }
  }
  return ok;
}
}  // namespace

void* scratch_slot(size_t bytes, int slot, hipStream_t stream, int* status) {
  *status = DLM_OK;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    *status = fail(DLM_ERR_HIP, "scratch: hipGetDevice failed");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchSlot& s = g_scratch[{dev, stream, slot}];
  if (s.bytes >= bytes && s.ptr) return s.ptr;
  size_t want = bytes < 256 ? 256 : bytes;
  want = (want + 0xFFFFF) & ~size_t(0xFFFFF);  // round to 1 MiB
  const bool over = device_total(dev) - s.bytes + want > kScratchDeviceCap;
  if (s.ptr || over) {
    if (hipDeviceSynchronize() != hipSuccess) {
      *status = fail(DLM_ERR_HIP, "scratch: device synchronisation failed");
      return nullptr;
    }
  }
  if (s.ptr) {
    if (hipFree(s.ptr) != hipSuccess) {
      *status = fail(DLM_ERR_HIP, "scratch: release of old block failed");
      return nullptr;
    }
    s.ptr = nullptr;
    s.bytes = 0;
  }
  if (over && !evict_other_streams(dev, stream)) {
    *status = fail(DLM_ERR_HIP, "scratch: release of other streams' blocks failed");
    return nullptr;
  }
  ScratchSlot& t = g_scratch[{dev, stream, slot}];  // eviction never erases this stream's slots
  if (hipMalloc(&t.ptr, want) != hipSuccess) {
    t.ptr = nullptr;
    *status = fail(DLM_ERR_OUT_OF_MEMORY, "scratch: hipMalloc of " + std::to_string(want) + " bytes failed");
    return nullptr;
  }
  t.bytes = want;
  return t.ptr;
}

int scratch_release(hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  bool any = false;
  for (const auto& kv : g_scratch) any |= std::get<1>(kv.first) == stream;
  if (!any) return DLM_OK;
  if (hipStreamSynchronize(stream) != hipSuccess) return fail(DLM_ERR_HIP, "scratch: stream synchronisation failed");
  for (auto it = g_scratch.begin(); it != g_scratch.end();) {
    if (std::get<1>(it->first) == stream) {
      if (it->second.ptr && hipFree(it->second.ptr) != hipSuccess) return fail(DLM_ERR_HIP, "scratch: hipFree failed");
      it = g_scratch.erase(it);
    } else {
      ++it;
    }
  }
  return DLM_OK;
}

size_t scratch_bytes() {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  size_t t = 0;
  for (const auto& kv : g_scratch) t += kv.second.bytes;
  return t;
}

// Counter calibration kernel: every wave issues `iters` rounds of eight
// v_mfma_f32_32x32x16_f16 on four independent accumulators, operands in
// registers and no memory traffic in the loop (8 x 32768 FLOP per round), so
// a profiler's MFMA counters can be read against a known MFMA rate.
__global__ void __launch_bounds__(256) mfma_probe_kernel(float* out, int iters) {
  const int lane = threadIdx.x & 63;
  f16x8 a, b;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    a[t] = (f16)(0.001f * (float)(lane + t));
    b[t] = (f16)(0.002f * (float)(lane - t));
  }
  f32x16 c0{}, c1{}, c2{}, c3{};
  for (int i = 0; i < iters; ++i) {
    c0 = mfma32x32x16(a, b, c0);
    c1 = mfma32x32x16(b, a, c1);
    c2 = mfma32x32x16(a, a, c2);
    c3 = mfma32x32x16(b, b, c3);
    c0 = mfma32x32x16(a, b, c0);
    c1 = mfma32x32x16(b, a, c1);
    c2 = mfma32x32x16(a, a, c2);
    c3 = mfma32x32x16(b, b, c3);
  }
  float sum = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) sum += c0[e] + c1[e] + c2[e] + c3[e];
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = sum;
}

}  // namespace dlm

extern "C" {

int dlm_mfma_probe(int blocks, int iters, float* out, void* stream) {
  if (blocks <= 0 || iters <= 0) return DLM_OK;
  DLM_REQUIRE(out != nullptr, "out is NULL");
  DLM_LAUNCH("mfma_probe_kernel", dlm::mfma_probe_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
             out, iters);
  DLM_LAUNCH_CHECK();
  return DLM_OK;
}

const char* dlm_last_error(void) { return dlm::g_last_error.c_str(); }

int dlm_scratch_release(void* stream) {
  const int st = dlm::scratch_release((hipStream_t)stream);
  if (st != DLM_OK) return st;
  return dlm::split_workspace_release((hipStream_t)stream);
}

int dlm_scratch_bytes(size_t* bytes) {
  DLM_REQUIRE(bytes != nullptr, "bytes is NULL");
  *bytes = dlm::scratch_bytes() + dlm::split_workspace_bytes();
  return DLM_OK;
}

void dlm_set_last_error(const char* msg) { dlm::g_last_error = msg ? msg : ""; }

const char* dlm_last_kernel(int reset) {
  const char* k = dlm::g_last_kernel;
  if (reset) dlm::note_kernel("");
  return k;
}

int dlm_prof_arm(void* start, void* stop) {
  DLM_REQUIRE(start != nullptr && stop != nullptr, "start / stop event is NULL");
  dlm::ProfArm& p = dlm::prof_arm();
  p.start = (hipEvent_t)start;
  p.stop = (hipEvent_t)stop;
  p.launched = 0;
  return DLM_OK;
}

int dlm_prof_disarm(void) {
  dlm::ProfArm& p = dlm::prof_arm();
  const int n = p.launched;
  p = dlm::ProfArm{};
  return n;
}

int dlm_last_kernel_dims(int* dims) {
  DLM_REQUIRE(dims != nullptr, "dims is NULL");
  for (int i = 0; i < 4; ++i) dims[i] = dlm::g_last_dims[i];
  return DLM_OK;
}

int dlm_get_device_count(int* count) {
  DLM_REQUIRE(count != nullptr, "count is NULL");
  DLM_HIP(hipGetDeviceCount(count));
  return DLM_OK;
}

int dlm_set_device(int device) {
  DLM_HIP(hipSetDevice(device));
  return DLM_OK;
}

int dlm_device_arch(char* buf, int buflen) {
  DLM_REQUIRE(buf != nullptr && buflen > 0, "bad buffer");
  int dev = 0;
  DLM_HIP(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  DLM_HIP(hipGetDeviceProperties(&prop, dev));
  std::snprintf(buf, (size_t)buflen, "%s", prop.gcnArchName);
  return DLM_OK;
}

int dlm_malloc(void** ptr, size_t bytes) {
  DLM_REQUIRE(ptr != nullptr, "ptr is NULL");
  *ptr = nullptr;
  if (bytes == 0) return DLM_OK;
  DLM_HIP(hipMalloc(ptr, bytes));
  return DLM_OK;
}

int dlm_free(void* ptr) {
  if (ptr == nullptr) return DLM_OK;
  DLM_HIP(hipFree(ptr));
  return DLM_OK;
}

int dlm_host_malloc_pinned(void** ptr, size_t bytes) {
  DLM_REQUIRE(ptr != nullptr, "ptr is NULL");
  *ptr = nullptr;
  if (bytes == 0) return DLM_OK;
  DLM_HIP(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
  return DLM_OK;
}

int dlm_host_free_pinned(void* ptr) {
  if (ptr == nullptr) return DLM_OK;
  DLM_HIP(hipHostFree(ptr));
  return DLM_OK;
}

static hipMemcpyKind to_kind(int kind) {
  switch (kind) {
    case 0: return hipMemcpyHostToDevice;
    case 1: return hipMemcpyDeviceToHost;
    case 2: return hipMemcpyDeviceToDevice;
    default: return hipMemcpyDefault;
  }
}

int dlm_memcpy(void* dst, const void* src, size_t bytes, int kind) {
  if (bytes == 0) return DLM_OK;
  DLM_REQUIRE(dst && src, "NULL pointer");
  DLM_HIP(hipMemcpy(dst, src, bytes, to_kind(kind)));
  return DLM_OK;
}

int dlm_memcpy_async(void* dst, const void* src, size_t bytes, int kind, void* stream) {
  if (bytes == 0) return DLM_OK;
  DLM_REQUIRE(dst && src, "NULL pointer");
  DLM_HIP(hipMemcpyAsync(dst, src, bytes, to_kind(kind), (hipStream_t)stream));
  return DLM_OK;
}

int dlm_memset_async(void* dst, int value, size_t bytes, void* stream) {
  if (bytes == 0) return DLM_OK;
  DLM_REQUIRE(dst != nullptr, "NULL pointer");
  DLM_HIP(hipMemsetAsync(dst, value, bytes, (hipStream_t)stream));
  return DLM_OK;
}

int dlm_device_synchronize(void) {
  DLM_HIP(hipDeviceSynchronize());
  return DLM_OK;
}

int dlm_mem_get_info(size_t* free_bytes, size_t* total_bytes) {
  DLM_REQUIRE(free_bytes && total_bytes, "NULL pointer");
  DLM_HIP(hipMemGetInfo(free_bytes, total_bytes));
  return DLM_OK;
}

int dlm_stream_create(void** stream) {
  DLM_REQUIRE(stream != nullptr, "stream is NULL");
  hipStream_t s = nullptr;
  DLM_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = (void*)s;
  return DLM_OK;
}

int dlm_stream_destroy(void* stream) {
  if (stream == nullptr) return DLM_OK;
  DLM_HIP(hipStreamDestroy((hipStream_t)stream));
  return DLM_OK;
}

int dlm_stream_synchronize(void* stream) {
  DLM_HIP(hipStreamSynchronize((hipStream_t)stream));
  return DLM_OK;
}

int dlm_graph_begin_capture(void* stream) {
  DLM_REQUIRE(stream != nullptr, "graph capture needs a created stream (not the null stream)");
  DLM_HIP(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
  return DLM_OK;
}

int dlm_graph_end_capture(void* stream, void** exec) {
  DLM_REQUIRE(stream && exec, "NULL argument");
  *exec = nullptr;
  hipGraph_t g = nullptr;
  DLM_HIP(hipStreamEndCapture((hipStream_t)stream, &g));
  if (!g) return dlm::fail(DLM_ERR_HIP, "graph capture produced no graph");
  hipGraphExec_t e = nullptr;
  const hipError_t st = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (st != hipSuccess) return dlm::fail(DLM_ERR_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(st));
  *exec = (void*)e;
  return DLM_OK;
}

int dlm_graph_launch(void* exec, void* stream) {
  DLM_REQUIRE(exec != nullptr, "exec is NULL");
  DLM_HIP(hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)stream));
  return DLM_OK;
}

int dlm_graph_destroy(void* exec) {
  if (exec == nullptr) return DLM_OK;
  DLM_HIP(hipGraphExecDestroy((hipGraphExec_t)exec));
  return DLM_OK;
}

int dlm_event_create(void** event) {
  DLM_REQUIRE(event != nullptr, "event is NULL");
  hipEvent_t e = nullptr;
  DLM_HIP(hipEventCreate(&e));
  *event = (void*)e;
  return DLM_OK;
}

int dlm_event_destroy(void* event) {
  if (event == nullptr) return DLM_OK;
  DLM_HIP(hipEventDestroy((hipEvent_t)event));
  return DLM_OK;
}

int dlm_event_record(void* event, void* stream) {
  DLM_REQUIRE(event != nullptr, "event is NULL");
  DLM_HIP(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
  return DLM_OK;
}

int dlm_event_synchronize(void* event) {
  DLM_REQUIRE(event != nullptr, "event is NULL");
  DLM_HIP(hipEventSynchronize((hipEvent_t)event));
  return DLM_OK;
}

int dlm_event_elapsed_ms(float* ms, void* start, void* stop) {
  DLM_REQUIRE(ms && start && stop, "NULL argument");
  DLM_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
  return DLM_OK;
}

}  // extern "C"

// Fences: cross-stream and cross-process ordering of swaps without events.
//
// The reference orders a swap after moves enqueued by other worker
// processes with CUDA interprocess events: the producer records an event
// created with cudaEventInterprocess and exports its handle
// (aegaeon/worker.py:2331,2349); the consumer rebuilds it and calls
// cudaStreamWaitEvent (aegaeon/worker.py:2351-2394, aegaeon/utils.py:263-288).
// The HIP runtime this library runs on creates such events and exports their
// handles but refuses to record them (hipEventRecord returns
// hipErrorInvalidValue), so the ordering is built from stream-ordered
// memory operations instead:
//
//   * a fence word is a 64-bit counter in device memory; a page of them can
//     be shared between processes with a HIP IPC memory handle;
//   * aegkv_fence_signal enqueues a one-wave kernel that raises a word to a
//     value (atomic max, release at system scope) once every earlier
//     operation on the stream has finished;
//   * aegkv_fence_wait enqueues a one-wave kernel that polls a word (acquire
//     at system scope) until it reaches a value, so every later operation on
//     the stream runs after the signal. The poll is bounded by a wall-clock
//     budget: a wait that runs out ends anyway and sets a caller-provided
//     flag word to 1, so no wave ever spins forever.
//
// Every memory operation here is a vector-memory load, store or atomic.
//
// A host-side view of the same counts serves a controller that only polls
// completion on the CPU (the reference's BlockManager rebuilds the workers'
// events and polls cudaEventQuery before it frees source blocks,
// aegaeon/block_manager.py:804-851): aegkv_fence_publish enqueues a host
// function that raises a host word, which may live in a file mapping shared
// by every process, and aegkv_fence_host_wait reads it with a bounded wait.

#include <hip/hip_runtime.h>
#include "aegkv.h"
#include "errors.h"

#include <chrono>
#include <cstdint>
#include <mutex>
#include <map>
#include <thread>

namespace {

#define fail aegkv_set_error

// Report a failed HIP call and clear the runtime's last-error state, which
// would otherwise make a later launch check report this failure again.
int hip_fail(hipError_t e, const char* what) {
  (void)hipGetLastError();
  return fail(static_cast<int>(e), "%s failed: %s (%d)", what, hipGetErrorString(e),
              static_cast<int>(e));
}

#define FENCE_HIP(call)                              \
  do {                                               \
    hipError_t e_ = (call);                          \
    if (e_ != hipSuccess) return hip_fail(e_, #call); \
  } while (0)

// Longest budget a wait may ask for (10 minutes).
constexpr int64_t kMaxWaitMicros = int64_t(600) * 1000 * 1000;

__global__ void __launch_bounds__(64) fence_signal_kernel(uint64_t* word, uint64_t value) {
  if (threadIdx.x == 0)
    (void)__hip_atomic_fetch_max(word, value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ void __launch_bounds__(64) fence_wait_kernel(const uint64_t* word, uint64_t value,
                                                        uint64_t budget_ticks,
                                                        uint64_t* timed_out) {
  if (threadIdx.x != 0) return;
  const uint64_t start = wall_clock64();
  for (;;) {
    const uint64_t seen = __hip_atomic_load(word, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
    if (seen >= value) return;
    if (wall_clock64() - start > budget_ticks) {
      __hip_atomic_store(timed_out, uint64_t(1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      return;
    }
    __builtin_amdgcn_s_sleep(8);
  }
}

// A fence word must be 8-byte aligned memory the current device can access:
// device memory (including memory opened from another process's IPC
// handle) or mapped pinned host memory.
int check_word(const void* p, const char* what) {
  if (!p) return fail(AEGKV_EINVAL, "%s is null", what);
  if (reinterpret_cast<uintptr_t>(p) & 7u)
    return fail(AEGKV_EINVAL, "%s must be 8-byte aligned", what);
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(AEGKV_EINVAL, "%s is not memory the HIP runtime knows", what);
  }
  if (attr.type == hipMemoryTypeDevice) return 0;
  if (attr.type == hipMemoryTypeHost && attr.devicePointer != nullptr) return 0;
  return fail(AEGKV_EINVAL, "%s must be device memory or mapped pinned host memory", what);
}

std::mutex g_rate_mu;
std::map<int, int64_t> g_rate_khz;

int wall_clock_khz(int64_t* out) {
  int dev = -1;
  FENCE_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_rate_mu);
  auto it = g_rate_khz.find(dev);
  if (it == g_rate_khz.end()) {
    int khz = 0;
    FENCE_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
    if (khz <= 0) return fail(AEGKV_EINVAL, "device %d reports no wall-clock rate", dev);
    it = g_rate_khz.emplace(dev, khz).first;
  }
  *out = it->second;
  return 0;
}

// Raise *word to at least value (release), from any host thread.
void host_word_max(uint64_t* word, uint64_t value) {
  uint64_t seen = __atomic_load_n(word, __ATOMIC_RELAXED);
  while (seen < value &&
         !__atomic_compare_exchange_n(word, &seen, value, true, __ATOMIC_RELEASE,
                                      __ATOMIC_RELAXED)) {
  }
}

struct Publish {
  uint64_t* word;
  uint64_t value;
};

// Runs on the runtime's host-function thread once the stream reaches it.
void publish_cb(void* data) {
  Publish* p = static_cast<Publish*>(data);
  host_word_max(p->word, p->value);
  delete p;
}

int check_host_word(const void* p) {
  if (!p) return fail(AEGKV_EINVAL, "host fence word is null");
  if (reinterpret_cast<uintptr_t>(p) & 7u)
    return fail(AEGKV_EINVAL, "host fence word must be 8-byte aligned");
  return 0;
}

}  // namespace

extern "C" {

int aegkv_fence_publish(uint64_t* host_word, uint64_t value, hipStream_t stream) {
  aegkv_clear_error();
  int rc = check_host_word(host_word);
  if (rc) return rc;
  if (value == 0 || value >= (uint64_t(1) << 63))
    return fail(AEGKV_EINVAL, "fence values are positive and below 2^63");
  // The callback frees its record, so a graph replaying it would use a
  // freed record: refuse a capturing stream.
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(stream, &status);
  if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
  if (status != hipStreamCaptureStatusNone)
    return fail(AEGKV_EINVAL, "fence publish cannot be captured into a graph");
  Publish* p = new Publish{host_word, value};
  e = hipLaunchHostFunc(stream, publish_cb, p);
  if (e != hipSuccess) {
    delete p;
    return hip_fail(e, "hipLaunchHostFunc(fence publish)");
  }
  return 0;
}

int aegkv_fence_host_wait(const uint64_t* host_word, uint64_t value, int64_t timeout_us) {
  aegkv_clear_error();
  int rc = check_host_word(host_word);
  if (rc) return rc;
  if (timeout_us < 0 || timeout_us > kMaxWaitMicros)
    return fail(AEGKV_ERANGE, "host fence wait timeout %lld us outside [0, %lld]",
                static_cast<long long>(timeout_us), static_cast<long long>(kMaxWaitMicros));
  const auto deadline = std::chrono::steady_clock::now() + std::chrono::microseconds(timeout_us);
  for (int polls = 0;; ++polls) {
    if (__atomic_load_n(host_word, __ATOMIC_ACQUIRE) >= value) return 1;
    if (std::chrono::steady_clock::now() >= deadline) return 0;
    // a few quick polls, then sleep in steps of at most 200 us
    if (polls < 64) std::this_thread::yield();
    else std::this_thread::sleep_for(std::chrono::microseconds(polls < 1000 ? 20 : 200));
  }
}


int aegkv_fence_signal(uint64_t* word, uint64_t value, hipStream_t stream) {
  aegkv_clear_error();
  int rc = check_word(word, "fence word");
  if (rc) return rc;
  (void)hipGetLastError();  // clear a stale error: the check below is for this launch
  hipLaunchKernelGGL(fence_signal_kernel, dim3(1), dim3(64), 0, stream, word, value);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fence_signal_kernel launch");
  return 0;
}

int aegkv_fence_wait(const uint64_t* word, uint64_t value, int64_t timeout_us,
                     uint64_t* timed_out, hipStream_t stream) {
  aegkv_clear_error();
  if (timeout_us <= 0 || timeout_us > kMaxWaitMicros)
    return fail(AEGKV_ERANGE, "fence wait timeout %lld us outside (0, %lld]",
                static_cast<long long>(timeout_us), static_cast<long long>(kMaxWaitMicros));
  int rc = check_word(word, "fence word");
  if (rc) return rc;
  rc = check_word(timed_out, "timed_out flag");
  if (rc) return rc;
  int64_t khz = 0;
  rc = wall_clock_khz(&khz);
  if (rc) return rc;
  // ticks = us * (kHz / 1000); both factors are bounded, no overflow
  const uint64_t budget = static_cast<uint64_t>(timeout_us) * static_cast<uint64_t>(khz) / 1000u;
  (void)hipGetLastError();  // clear a stale error: the check below is for this launch
  hipLaunchKernelGGL(fence_wait_kernel, dim3(1), dim3(64), 0, stream, word, value, budget,
                     timed_out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fence_wait_kernel launch");
  return 0;
}

}  // extern "C"

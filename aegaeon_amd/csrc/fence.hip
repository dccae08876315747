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
//     budget: a wait that runs out ends anyway and sets the stream's move
//     guard (a caller-provided word) to 1, so no wave ever spins forever.
//
// A failed wait must not let the stream's later moves pass for good ones.
// The reference never runs a swap before its source is ready: it waits
// without a limit (aegaeon/worker.py:2387) and stops the worker when it
// cannot get the source events (:2364-2368). Here the give-up is marked
// instead, and the mark travels with everything that reports completion:
//   * guarded moves (aegkv_swap_blocks, aegkv_migrate_blocks with a guard)
//     read the guard first and move nothing once it is set;
//   * a guarded signal raises its word to value | AEGKV_FENCE_FAILED, and a
//     wait that sees that bit sets its own stream's guard to 2, so the
//     failure follows the chain of moves across streams and processes;
//   * a guarded publish raises its host word to value | AEGKV_FENCE_FAILED,
//     which aegkv_fence_host_wait reports as 2 (failed), not as done;
//   * aegkv_guard_merge sets a consumer's guard to 2 behind its stream's
//     work when a producer's guard is set, for a consumer that waits on the
//     producer's event instead of a fence word.
// A failure is sticky: the mark stays in the words (atomic max) and the
// guard is never cleared by the library, as the reference's stopped worker
// moves nothing more.
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
constexpr uint64_t kFailed = AEGKV_FENCE_FAILED;

// Guard values a wait stores (any non-zero value stops guarded moves).
constexpr uint64_t kGuardTimedOut = 1;
constexpr uint64_t kGuardSourceFailed = 2;

__device__ __forceinline__ uint64_t load_guard(const uint64_t* guard) {
  return guard ? __hip_atomic_load(guard, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) : 0;
}

// Guards are set with plain stores, not read-modify-writes: they may live
// in pinned host memory, and any non-zero value means the same thing.
__device__ __forceinline__ void set_guard(uint64_t* guard, uint64_t why) {
  __hip_atomic_store(guard, why, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ void __launch_bounds__(64) fence_signal_kernel(uint64_t* word, uint64_t value,
                                                          const uint64_t* guard) {
  if (threadIdx.x != 0) return;
  const uint64_t v = load_guard(guard) != 0 ? (value | kFailed) : value;
  (void)__hip_atomic_fetch_max(word, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ void __launch_bounds__(64) fence_wait_kernel(const uint64_t* word, uint64_t value,
                                                        uint64_t budget_ticks, uint64_t* guard) {
  if (threadIdx.x != 0) return;
  const uint64_t start = wall_clock64();
  for (;;) {
    const uint64_t seen = __hip_atomic_load(word, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
    if (seen & kFailed) {
      set_guard(guard, kGuardSourceFailed);
      return;
    }
    if (seen >= value) return;
    if (wall_clock64() - start > budget_ticks) {
      set_guard(guard, kGuardTimedOut);
      return;
    }
    __builtin_amdgcn_s_sleep(8);
  }
}

__global__ void __launch_bounds__(64) guard_merge_kernel(uint64_t* guard, const uint64_t* source) {
  if (threadIdx.x != 0) return;
  if (load_guard(source) != 0) set_guard(guard, kGuardSourceFailed);
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
  const uint64_t* guard;  // host-readable, or null
};

// Runs on the runtime's host-function thread once the stream reaches it,
// after every earlier operation on the stream (the guard's last writer
// included) has finished.
void publish_cb(void* data) {
  Publish* p = static_cast<Publish*>(data);
  const bool failed = p->guard && __atomic_load_n(p->guard, __ATOMIC_ACQUIRE) != 0;
  host_word_max(p->word, failed ? (p->value | kFailed) : p->value);
  delete p;
}

// A guard the host function reads: pinned host memory.
int check_host_guard(const uint64_t* g) {
  if (reinterpret_cast<uintptr_t>(g) & 7u)
    return fail(AEGKV_EINVAL, "move guard must be 8-byte aligned");
  hipPointerAttribute_t attr;
  hipError_t e = hipPointerGetAttributes(&attr, g);
  if (e != hipSuccess || attr.type != hipMemoryTypeHost) {
    (void)hipGetLastError();
    return fail(AEGKV_EINVAL, "a published fence's move guard must be pinned host memory "
                "(the host function reads it)");
  }
  return 0;
}

int check_value(uint64_t value) {
  if (value == 0 || value >= kFailed)
    return fail(AEGKV_EINVAL, "fence values are positive and below 2^62 (bit 62 marks a "
                "failed move)");
  return 0;
}

int check_host_word(const void* p) {
  if (!p) return fail(AEGKV_EINVAL, "host fence word is null");
  if (reinterpret_cast<uintptr_t>(p) & 7u)
    return fail(AEGKV_EINVAL, "host fence word must be 8-byte aligned");
  return 0;
}

}  // namespace

extern "C" {

int aegkv_fence_publish(uint64_t* host_word, uint64_t value, const uint64_t* guard,
                        hipStream_t stream) {
  aegkv_clear_error();
  int rc = check_host_word(host_word);
  if (!rc) rc = check_value(value);
  if (!rc && guard) rc = check_host_guard(guard);
  if (rc) return rc;
  // The callback frees its record, so a graph replaying it would use a
  // freed record: refuse a capturing stream.
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(stream, &status);
  if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
  if (status != hipStreamCaptureStatusNone)
    return fail(AEGKV_EINVAL, "fence publish cannot be captured into a graph");
  Publish* p = new Publish{host_word, value, guard};
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
    const uint64_t seen = __atomic_load_n(host_word, __ATOMIC_ACQUIRE);
    if (seen & kFailed) return 2;
    if (seen >= value) return 1;
    if (std::chrono::steady_clock::now() >= deadline) return 0;
    // a few quick polls, then sleep in steps of at most 200 us
    if (polls < 64) std::this_thread::yield();
    else std::this_thread::sleep_for(std::chrono::microseconds(polls < 1000 ? 20 : 200));
  }
}


int aegkv_fence_signal(uint64_t* word, uint64_t value, const uint64_t* guard,
                       hipStream_t stream) {
  aegkv_clear_error();
  int rc = check_value(value);
  if (!rc) rc = check_word(word, "fence word");
  if (!rc && guard) rc = check_word(guard, "move guard");
  if (rc) return rc;
  (void)hipGetLastError();  // clear a stale error: the check below is for this launch
  hipLaunchKernelGGL(fence_signal_kernel, dim3(1), dim3(64), 0, stream, word, value, guard);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fence_signal_kernel launch");
  return 0;
}

int aegkv_fence_wait(const uint64_t* word, uint64_t value, int64_t timeout_us,
                     uint64_t* guard, hipStream_t stream) {
  aegkv_clear_error();
  if (timeout_us <= 0 || timeout_us > kMaxWaitMicros)
    return fail(AEGKV_ERANGE, "fence wait timeout %lld us outside (0, %lld]",
                static_cast<long long>(timeout_us), static_cast<long long>(kMaxWaitMicros));
  int rc = check_value(value);
  if (!rc) rc = check_word(word, "fence word");
  if (!rc) rc = check_word(guard, "move guard");
  if (rc) return rc;
  int64_t khz = 0;
  rc = wall_clock_khz(&khz);
  if (rc) return rc;
  // ticks = us * (kHz / 1000); both factors are bounded, no overflow
  const uint64_t budget = static_cast<uint64_t>(timeout_us) * static_cast<uint64_t>(khz) / 1000u;
  (void)hipGetLastError();  // clear a stale error: the check below is for this launch
  hipLaunchKernelGGL(fence_wait_kernel, dim3(1), dim3(64), 0, stream, word, value, budget,
                     guard);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "fence_wait_kernel launch");
  return 0;
}

int aegkv_guard_merge(uint64_t* guard, const uint64_t* source_guard, hipStream_t stream) {
  aegkv_clear_error();
  int rc = check_word(guard, "move guard");
  if (!rc) rc = check_word(source_guard, "source move guard");
  if (rc) return rc;
  (void)hipGetLastError();  // clear a stale error: the check below is for this launch
  hipLaunchKernelGGL(guard_merge_kernel, dim3(1), dim3(64), 0, stream, guard, source_guard);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "guard_merge_kernel launch");
  return 0;
}

}  // extern "C"

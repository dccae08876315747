// Library-driven SDMA copies for STAGED transfers (sdma.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace aegkv_sdma {

constexpr int DIR_TO_HOST = 0;
constexpr int DIR_TO_DEVICE = 1;

struct CopyRun {
  void* dst;
  const void* src;
  size_t len;
};
using CopyList = std::vector<CopyRun>;

// One lane per (device, direction, stream): its jobs run in submission
// order on a library thread that calls the HSA runtime only.
struct LaneRef {
  void* lane;
  uint64_t* slots;      // pinned start slots: job seq starts once slots[seq % slot_count] >= seq
  uint64_t slot_count;
};

// Set up the device's agents and the stream's lane on first use. Fails,
// once, with the message of an earlier failed transfer on that lane, and
// always once copies were left pending.
int lane_for(int device, int dir, hipStream_t stream, LaneRef* out);

// Queue copies that start once the job's start slot holds its number
// (*seq): the caller stores it there from its stream, in stream order,
// with aegkv_enqueue_word_store.
int submit(const LaneRef& lane, const CopyList& copies, uint64_t* seq);

// For a job whose start store could not be enqueued: skip its copies and
// let the lane go on.
void abandon(const LaneRef& lane, uint64_t seq);

// Hold the stream (a host function, no kernel) until the lane has finished
// job seq, at most 60 s; then *timed_out is set and the stream goes on.
hipError_t enqueue_wait(const LaneRef& lane, uint64_t seq, uint64_t* timed_out,
                        hipStream_t stream);

// The device's lanes, for error messages.
std::string describe(int device);

}  // namespace aegkv_sdma

// Stream-ordered store to a 64-bit word (fence.hip), for library use.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

// Enqueue a kernel that stores value into *word (release, system scope)
// once the stream's earlier work is done. For a word with one writer at a
// time, e.g. in mapped pinned host memory read by a host thread.
hipError_t aegkv_enqueue_word_store(uint64_t* word, uint64_t value, hipStream_t stream);

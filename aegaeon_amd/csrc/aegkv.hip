// libaegkv: KV-cache block movement for MI355X (gfx950).
//
// Three operations, all pure byte movement (no arithmetic on the payload):
//   * swap-out  : device K/V tiles -> composite pages of a pinned host pool
//   * swap-in   : composite host pages -> device K/V tiles
//   * copy_blocks: device block -> device block, every backing tensor
//
// One persistent "tile mover" kernel family does all of it. A work item is
// one 16 B-per-lane chunk of one (entry, segment) tile; a workgroup of 256
// lanes moves CHUNK = 256 * 16 * UNROLL bytes per item with all UNROLL loads
// issued before the first store. Items are entry-major so consecutive items
// walk one composite host page in address order (good for PCIe write
// combining and host DRAM pages); link-bound swaps run a few persistent
// workgroups that stride over the item space, HBM-bound moves one workgroup
// per item.
//
// Two host-transfer designs share the kernel:
//   DIRECT: the "host side" pointer is the pinned host pool itself (mapped
//           into the GPU address space by hipHostMalloc); the kernel's
//           loads/stores cross PCIe.
//   STAGED: the "host side" pointer is a contiguous device staging buffer
//           laid out like the host pages; hipMemcpyAsync moves merged runs
//           between staging and the host pool (the runtime runs each copy
//           as a blit kernel or on an SDMA engine).
//
// Entry-point contracts are in include/aegkv.h.

#include <hip/hip_runtime.h>
#include "aegkv.h"
#include "errors.h"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <mutex>
#include <vector>

// ---------------------------------------------------------------- errors --

namespace {
thread_local char g_err[512] = "";
}  // namespace

int aegkv_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void aegkv_clear_error() { g_err[0] = '\0'; }

namespace {

#define fail aegkv_set_error

// Report a failed HIP call and clear the runtime's last-error state, which
// would otherwise make a later launch check report this failure again.
int hip_fail(hipError_t e, const char* what) {
  (void)hipGetLastError();
  return fail(static_cast<int>(e), "%s failed: %s (%d)", what, hipGetErrorString(e),
              static_cast<int>(e));
}

#define AEGKV_HIP(call)                          \
  do {                                           \
    hipError_t e_ = (call);                      \
    if (e_ != hipSuccess) return hip_fail(e_, #call); \
  } while (0)

// --------------------------------------------------------------- tunables --

struct Tunables {
  // Swap kernels: persistent workgroups in total, per direction, each lane
  // with swap_unroll 16 B loads in flight. The swaps are link-bound: about
  // 1 MiB in flight per direction saturates PCIe, and the few workgroups
  // leave the other CUs to concurrent copies. Two loads per lane with twice
  // the workgroups keep the same bytes in flight and share the link better
  // when both directions run at once (model switch 105 -> 103 ms), at the
  // same rate for one direction alone (57.1 / 57.5 GB/s).
  int64_t swap_out_workgroups = 64;
  int64_t swap_in_workgroups = 128;
  // Swap-out into an uncached pool: alone 64-224 workgroups all reach the
  // link rate, and beside a swap-in 112 leave the swap-in more of the link
  // (with 4 loads per lane: 32 -> 56 workgroups, 108.5 -> 105 ms). Into a
  // cached pool 64 stay best alone (56.6 GB/s; 55.8 at 112) and equal
  // beside a swap-in.
  int64_t swap_out_workgroups_uncached = 112;
  int64_t staging_bytes = int64_t(512) << 20;
  int64_t auto_d2h = AEGKV_MODE_DIRECT;
  int64_t auto_h2d = AEGKV_MODE_DIRECT;
  int64_t nt_stores = 1;
  int64_t copy_wgs_per_cu = 0;   // copy_blocks: 0 = one workgroup per work item
  int64_t copy_unroll = 0;       // copy_blocks: 0 = shape from the page size
  int64_t copy_lanes = 0;        // copy_blocks with copy_unroll: 256 or 1024 lanes (0 = 1024)
  int64_t swap_shape_auto = 0;   // swap kernels: 1 = page-sized shape as copy_blocks
  int64_t swap_unroll = 2;       // swap kernels: 16 B loads per lane (256-lane shape)
  int64_t staged_workgroups = 0; // STAGED gather/scatter grid: 0 = one workgroup per item
  int64_t staged_dma_streams = 2; // STAGED copies: library streams (<= 1: caller stream)
  // STAGED over library streams: two staging chunks in flight (bit 0
  // swap-out, bit 1 swap-in), so the gather or scatter of one chunk runs
  // while another chunk's copies use the link. Qwen3-4B, 1024 blocks (GB/s
  // out / in): one call at a time 43.4 / 50.9 -> 54.3 / 55.4; swap-out and
  // swap-in at once 174 -> 121 ms for a model switch; beside a GEMM the
  // swaps end at 52 / 56 ms instead of 74 / 105. Where the host enqueues
  // far ahead with block copies between the swaps, the runtime moved the
  // swap-out's copies to SDMA and it fell to 29 GB/s (35 one chunk at a
  // time); set bit 0 off for that pattern.
  int64_t staged_overlap = 3;
  // copy_blocks, 1024-lane shapes with items of >= 32 KiB: LDS reserved per
  // workgroup so that one workgroup holds a CU (HBM copy rate +1-5 % on
  // 32-160 KiB tiles; 16 KiB items lose 14 % at one per CU, so they keep 0).
  int64_t copy_lds_bytes = int64_t(96) << 10;
  // copy_blocks: the order in which pairs reach the kernel (0: the caller's,
  // 1: by target id, 2: by source id; the checks make the result
  // order-free). By target id, a copy from one random half of a cache's
  // blocks to the other runs at 5.98 instead of 5.64 TB/s on 16 KiB tiles,
  // 5.58 instead of 5.39 on 32 KiB and within 1 % on 64-160 KiB; by source
  // id it gains about a third as much.
  int64_t copy_order = 1;
};
Tunables g_tune;
std::mutex g_tune_mu;
constexpr int64_t kMaxLdsPerWorkgroup = int64_t(160) << 10;  // gfx950: 160 KiB per CU

// Environment overrides, read once per process: AEGKV_AUTO_D2H and
// AEGKV_AUTO_H2D ("direct" or "staged") choose what mode AUTO resolves to,
// AEGKV_STAGING_BYTES (>= 1 MiB) the STAGED chunk. An invalid value makes
// every entry point that moves data fail with AEGKV_EINVAL naming it.
std::once_flag g_env_once;
char g_env_err[256] = "";

void read_env() {
  std::lock_guard<std::mutex> lk(g_tune_mu);
  auto mode = [](const char* name, int64_t* slot) {
    const char* v = std::getenv(name);
    if (!v || !*v) return;
    if (!std::strcmp(v, "direct")) *slot = AEGKV_MODE_DIRECT;
    else if (!std::strcmp(v, "staged")) *slot = AEGKV_MODE_STAGED;
    else std::snprintf(g_env_err, sizeof(g_env_err), "%s=%s: expected direct or staged", name, v);
  };
  mode("AEGKV_AUTO_D2H", &g_tune.auto_d2h);
  mode("AEGKV_AUTO_H2D", &g_tune.auto_h2d);
  const char* v = std::getenv("AEGKV_STAGING_BYTES");
  if (v && *v) {
    char* end = nullptr;
    const long long x = std::strtoll(v, &end, 10);
    if (*end != '\0' || x < (1ll << 20))
      std::snprintf(g_env_err, sizeof(g_env_err),
                    "AEGKV_STAGING_BYTES=%s: expected an integer >= 1048576", v);
    else
      g_tune.staging_bytes = x;
  }
}

int env_status() {
  std::call_once(g_env_once, read_env);
  return g_env_err[0] ? fail(AEGKV_EINVAL, "%s", g_env_err) : 0;
}

Tunables tunables() {
  std::lock_guard<std::mutex> lk(g_tune_mu);
  return g_tune;
}

// ------------------------------------------------------ device descriptors --

struct SegDesc {            // one backing tensor
  char* base;
  int64_t page_bytes;
  int64_t host_offset;
  uint64_t owner_mask;
};
static_assert(sizeof(SegDesc) == 32, "SegDesc layout");

struct EntDesc {            // one swap entry, already resolved to sides
  int64_t dev_block;        // block id in every backing tensor
  int64_t host_slot;        // host block id (DIRECT) or staging slot (STAGED)
  int32_t group;
  int32_t first;            // first kernel block of the extent
  int32_t valid;            // kernel blocks in the extent
  int32_t pad;
};
static_assert(sizeof(EntDesc) == 32, "EntDesc layout");

struct PairDesc {
  int64_t src;
  int64_t dst;
};

struct CopySeg {            // one backing tensor of a block copy
  const char* src;          // source cache's tensor
  char* dst;                // target cache's tensor (== src within one cache)
  int64_t page_bytes;
  int64_t pad;
};
static_assert(sizeof(CopySeg) == 32, "CopySeg layout");
static_assert(sizeof(PairDesc) == 16, "PairDesc layout (descriptors are whole 16-byte words)");

typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) v4u gv4u;  // global (VM) address space
typedef __attribute__((address_space(1))) char gchar;

// A kernel "shape": WG lanes per workgroup, U 16-byte loads in flight per
// lane, so one work item (chunk) is WG * 16 * U bytes.
template <int WG, int U>
struct Shape {
  static constexpr int kLanes = WG;
  static constexpr int kLoads = U;
  static constexpr int64_t kChunk = int64_t(WG) * 16 * U;
};

// Move nbytes (multiple of 16, at most one chunk) with 16 B per lane. A full
// chunk issues all U loads back to back before the first store; only a tail
// chunk pays for per-load guards.
template <int WG, int U, bool NT_STORE>
__device__ __forceinline__ void move_chunk16(const char* src, char* dst, uint32_t nbytes) {
  const gv4u* s = (const gv4u*)src;  // generic -> global address space
  gv4u* d = (gv4u*)dst;
  const uint32_t tid = threadIdx.x;
  v4u r[U];
  if (nbytes == static_cast<uint32_t>(Shape<WG, U>::kChunk)) {
#pragma unroll
    for (int u = 0; u < U; ++u) r[u] = __builtin_nontemporal_load(s + tid + u * WG);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (NT_STORE)
        __builtin_nontemporal_store(r[u], d + tid + u * WG);
      else
        d[tid + u * WG] = r[u];
    }
    return;
  }
  const uint32_t n16 = nbytes >> 4;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t i = tid + u * WG;
    if (i < n16) r[u] = __builtin_nontemporal_load(s + i);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t i = tid + u * WG;
    if (i < n16) {
      if (NT_STORE)
        __builtin_nontemporal_store(r[u], d + i);
      else
        d[i] = r[u];
    }
  }
}

// A move guard is a word a stream's fence waits set when they give up or
// see a failed source (aegkv_fence_wait). Guarded kernels read it once at
// the start, at system scope (it may live in pinned host memory), and move
// nothing when it is set.
__device__ __forceinline__ bool guard_set(const uint64_t* guard) {
  return guard != nullptr &&
         __hip_atomic_load(guard, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) != 0;
}

// Byte-granular fallback for callers whose offsets are not 16 B aligned.
template <int WG>
__device__ __forceinline__ void move_chunk_bytes(const char* src, char* dst, uint32_t nbytes) {
  const gchar* s = (const gchar*)src;
  gchar* d = (gchar*)dst;
  for (uint32_t i = threadIdx.x; i < nbytes; i += WG) d[i] = s[i];
}

// Swap tile mover. Item w -> (entry e, segment s, chunk c), entry-major.
// TO_HOST: device tile -> host side; otherwise host side -> device tile.
// The host keeps num_items + gridDim.x below 2^32 (items_fit_launch), so the
// 32-bit grid-stride loop never wraps.
template <int WG, int U, bool TO_HOST, bool VEC, bool NT_STORE>
__global__ __launch_bounds__(WG) void swap_tiles_kernel(
    const SegDesc* __restrict__ segs, const EntDesc* __restrict__ ents,
    const int64_t* __restrict__ kpp, uint32_t num_segs, uint32_t num_items,
    uint32_t chunks_per_tile, char* host_base, int64_t host_stride, int64_t host_rank_offset,
    const uint64_t* guard) {
  constexpr int64_t kChunk = Shape<WG, U>::kChunk;
  if (guard_set(guard)) return;
  for (uint32_t w = blockIdx.x; w < num_items; w += gridDim.x) {
    const uint32_t tile = w / chunks_per_tile;
    const uint32_t c = w - tile * chunks_per_tile;
    const uint32_t e = tile / num_segs;
    const uint32_t s = tile - e * num_segs;
    const EntDesc ent = ents[e];
    const SegDesc seg = segs[s];
    if (!((seg.owner_mask >> ent.group) & 1ull)) continue;
    const int64_t unit = seg.page_bytes / kpp[ent.group];
    const int64_t off = unit * ent.first;
    const int64_t len = unit * ent.valid;
    const int64_t begin = static_cast<int64_t>(c) * kChunk;
    if (begin >= len) continue;
    const uint32_t nbytes = static_cast<uint32_t>((len - begin < kChunk) ? (len - begin) : kChunk);
    char* dev = seg.base + ent.dev_block * seg.page_bytes + off + begin;
    char* host = host_base + ent.host_slot * host_stride + host_rank_offset +
                 seg.host_offset + off + begin;
    const char* src = TO_HOST ? dev : host;
    char* dst = TO_HOST ? host : dev;
    if (VEC)
      move_chunk16<WG, U, NT_STORE>(src, dst, nbytes);
    else
      move_chunk_bytes<WG>(src, dst, nbytes);
  }
}

// copy_blocks: item w -> (pair p, segment s, chunk c), pair-major: the
// workgroups running together move a few pairs across every segment (a
// segment-major walk, many pairs of one segment at a time, ran 1-9 % slower
// on 16-160 KiB tiles).
template <int WG, int U, bool VEC, bool NT_STORE>
__global__ __launch_bounds__(WG) void copy_blocks_kernel(
    const CopySeg* __restrict__ segs, const PairDesc* __restrict__ pairs, uint32_t num_segs,
    uint32_t num_items, uint32_t chunks_per_tile, const uint64_t* guard) {
  constexpr int64_t kChunk = Shape<WG, U>::kChunk;
  if (guard_set(guard)) return;
  for (uint32_t w = blockIdx.x; w < num_items; w += gridDim.x) {
    const uint32_t tile = w / chunks_per_tile;
    const uint32_t c = w - tile * chunks_per_tile;
    const uint32_t p = tile / num_segs;
    const uint32_t s = tile - p * num_segs;
    const PairDesc pr = pairs[p];
    const CopySeg seg = segs[s];
    const int64_t begin = static_cast<int64_t>(c) * kChunk;
    if (begin >= seg.page_bytes) continue;
    const uint32_t nbytes = static_cast<uint32_t>(
        (seg.page_bytes - begin < kChunk) ? (seg.page_bytes - begin) : kChunk);
    const char* src = seg.src + pr.src * seg.page_bytes + begin;
    char* dst = seg.dst + pr.dst * seg.page_bytes + begin;
    if (VEC)
      move_chunk16<WG, U, NT_STORE>(src, dst, nbytes);
    else
      move_chunk_bytes<WG>(src, dst, nbytes);
  }
}

// Measurement twins of copy_blocks_kernel (aegkv_copy_probe): the same
// item walk over the same tiles and the same grid, either reading the
// source tiles only (PROBE_READ; the loads are XOR-folded and the fold is
// stored only if it equals `magic`, so no load can be dropped and nearly
// nothing is written) or writing a fixed pattern to the target tiles only
// (PROBE_WRITE). Their rates bound what a copy of that tile pattern can
// reach on the memory system at hand.
constexpr int PROBE_READ = 1;
constexpr int PROBE_WRITE = 2;

template <int WG, int U, int KIND, bool NT_STORE>
__global__ __launch_bounds__(WG) void copy_probe_kernel(
    const CopySeg* __restrict__ segs, const PairDesc* __restrict__ pairs, uint32_t num_segs,
    uint32_t num_items, uint32_t chunks_per_tile, uint32_t* sink, uint32_t magic) {
  constexpr int64_t kChunk = Shape<WG, U>::kChunk;
  const uint32_t tid = threadIdx.x;
  v4u acc = {0u, 0u, 0u, 0u};
  const v4u pattern = {tid, blockIdx.x, 0x5a5a5a5au, magic};
  for (uint32_t w = blockIdx.x; w < num_items; w += gridDim.x) {
    const uint32_t tile = w / chunks_per_tile;
    const uint32_t c = w - tile * chunks_per_tile;
    const uint32_t p = tile / num_segs;
    const uint32_t s = tile - p * num_segs;
    const PairDesc pr = pairs[p];
    const CopySeg seg = segs[s];
    const int64_t begin = static_cast<int64_t>(c) * kChunk;
    if (begin >= seg.page_bytes) continue;
    const uint32_t n16 = static_cast<uint32_t>(
        ((seg.page_bytes - begin < kChunk) ? (seg.page_bytes - begin) : kChunk) >> 4);
    if (KIND == PROBE_READ) {
      const gv4u* src = (const gv4u*)(seg.src + pr.src * seg.page_bytes + begin);
      v4u r[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t i = tid + u * WG;
        r[u] = i < n16 ? __builtin_nontemporal_load(src + i) : v4u{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= r[u];
    } else {
      gv4u* dst = (gv4u*)(seg.dst + pr.dst * seg.page_bytes + begin);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t i = tid + u * WG;
        if (i < n16) {
          if (NT_STORE)
            __builtin_nontemporal_store(pattern, dst + i);
          else
            dst[i] = pattern;
        }
      }
    }
  }
  if (KIND == PROBE_READ) {
    const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (x == magic) sink[0] = x;
  }
}

// One contiguous slice of a weight load: `bytes` bytes from src to dst; its
// work items start at first_item.
struct SliceDesc {
  char* dst;
  const char* src;
  int64_t bytes;
  int64_t first_item;
};
static_assert(sizeof(SliceDesc) == 32, "SliceDesc layout");

// Contiguous slices, host to device (weight loads): item w -> the slice
// that holds it (the last one whose first_item <= w, found by a binary
// search over the uniform descriptor) and its chunk in that slice. Empty
// slices are dropped on the host, so every slice has at least one item.
template <int WG, int U, bool VEC, bool NT_STORE>
__global__ __launch_bounds__(WG) void slices_kernel(const SliceDesc* __restrict__ slices,
                                                    uint32_t num_slices, uint32_t num_items) {
  constexpr int64_t kChunk = Shape<WG, U>::kChunk;
  for (uint32_t w = blockIdx.x; w < num_items; w += gridDim.x) {
    uint32_t lo = 0, hi = num_slices - 1;
    while (lo < hi) {
      const uint32_t mid = (lo + hi + 1) >> 1;
      if (slices[mid].first_item <= static_cast<int64_t>(w))
        lo = mid;
      else
        hi = mid - 1;
    }
    const SliceDesc sl = slices[lo];
    const int64_t begin = (static_cast<int64_t>(w) - sl.first_item) * kChunk;
    const uint32_t nbytes =
        static_cast<uint32_t>((sl.bytes - begin < kChunk) ? (sl.bytes - begin) : kChunk);
    if (VEC)
      move_chunk16<WG, U, NT_STORE>(sl.src + begin, sl.dst + begin, nbytes);
    else
      move_chunk_bytes<WG>(sl.src + begin, sl.dst + begin, nbytes);
  }
}

// Descriptor bytes carried in one launch's kernel arguments (allocation-free
// copies): lane i stores the i-th 16 bytes. The runtime copies a launch's
// arguments when the launch is enqueued, and a graph that captures the
// launch keeps its own copy, so the host buffer they came from is free as
// soon as the launch call returns.
constexpr uint32_t kFillBytes = 2048;
struct FillArgs {
  v4u data[kFillBytes / 16];
  v4u* dst;
  uint32_t words;  // 16-byte words to store, <= kFillBytes / 16
  uint32_t pad;
};

__global__ __launch_bounds__(kFillBytes / 16) void desc_fill_kernel(FillArgs a) {
  const uint32_t i = threadIdx.x;
  if (i < a.words) a.dst[i] = a.data[i];
}

// Shapes the library instantiates. 1024-lane shapes move 16 KiB rows; a
// tile that is a multiple of 16 KiB gets the largest U dividing its row
// count, so one workgroup moves a whole tile (up to 160 KiB) with no tail
// chunk. Smaller tiles use 256-lane (4 KiB) rows.
struct ShapeSel {
  int wg;
  int u;
  int64_t chunk() const { return int64_t(wg) * 16 * u; }
};

ShapeSel auto_shape(int64_t page) {
  static const int kBigU[] = {10, 8, 6, 5, 4, 3, 2, 1};
  const int64_t row = 1024 * 16;
  if (page >= row && page % row == 0) {
    const int64_t rows = page / row;
    for (int u : kBigU)
      if (rows % u == 0) return {1024, u};
  }
  if (page >= row) return {1024, 4};
  const int64_t small_rows = (page + 4095) / 4096;
  return {256, small_rows <= 1 ? 1 : (small_rows <= 2 ? 2 : 4)};
}

bool valid_copy_unroll(int64_t u) {
  return u == 1 || u == 2 || u == 3 || u == 4 || u == 5 || u == 6 || u == 8 || u == 10;
}

// ------------------------------------------------------- per-device state --

// Stream-ordered pinned->device upload ring for call descriptors. A region
// is reused only after the event recorded behind the call that read it has
// completed, whatever stream that call ran on. Every event remembers the
// stream it was last recorded on, so that a stream about to be destroyed
// can take its events with it (forget_stream): an event is never queried,
// waited on or re-recorded after the stream that recorded it is gone. A
// region whose event was dropped that way (ev == nullptr) has completed.
struct Ring {
  char* host = nullptr;
  char* dev = nullptr;
  size_t cap = 0;
  size_t head = 0;
  struct Region {
    size_t begin, end;
    hipEvent_t ev;
    hipStream_t stream;
  };
  struct Spare {
    hipEvent_t ev;
    hipStream_t last;  // stream it was last recorded on
  };
  std::deque<Region> inflight;
  std::vector<Spare> spare;
};

constexpr int kMaxDmaStreams = 4;

struct DeviceCtx {
  int device = -1;
  int num_cus = 0;
  std::mutex mu;
  Ring ring;
  // STAGED mode: library-owned streams the per-run copies fan out over,
  // forked from and joined back into the caller's stream with events, one
  // set per direction (dma[0] swap-out, dma[1] swap-in) so a swap-out and
  // a swap-in at once do not queue their copies behind each other (with
  // one shared set, a swap-in beside a swap-out finished at 88-120 ms
  // instead of 56 ms).
  // A staged call holds the set's mutex from its first fork to its last
  // join, so its events are not re-recorded by another call in between.
  // fork_ev and kernel_ev are recorded on callers' streams; fork_on and
  // kernel_on name the stream of their last record (forget_stream).
  struct DmaSet {
    std::mutex mu;
    int streams = 0;
    hipStream_t st[kMaxDmaStreams] = {};
    hipEvent_t fork_ev = nullptr;
    hipEvent_t join_ev[2][kMaxDmaStreams] = {};  // copies done, per staging buffer
    hipEvent_t kernel_ev[2] = {};                // gather / scatter done, per staging buffer
    hipStream_t fork_on = nullptr;
    hipStream_t kernel_on[2] = {};
  } dma[2];
};

std::mutex g_ctx_mu;
std::map<int, DeviceCtx*> g_ctx;

std::mutex g_host_mu;
std::map<uintptr_t, size_t> g_host_allocs;  // live pools: start -> bytes asked for
// Uncached host memory is never returned to the runtime. Every uncached
// block hipHostMalloc gave stays mapped until the process ends, and live
// uncached pools are carved out of those blocks: a freed pool's range goes
// back to a free list (coalesced with its free neighbours in the same
// block), and a later uncached pool takes the smallest free range that fits
// before any new block is allocated. A process whose pools come and go in
// different sizes thus pins no more than its largest set of live pools,
// which keeps it under the host's cap on pinned memory.
constexpr size_t kHostPage = 4096;
std::map<uintptr_t, size_t> g_uncached_blocks;  // block base -> bytes
std::map<uintptr_t, size_t> g_uncached_pools;   // live pool start -> bytes carved
std::map<uintptr_t, size_t> g_uncached_free;    // free range start -> bytes

int get_ctx(DeviceCtx** out) {
  int dev = -1;
  AEGKV_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_ctx_mu);
  auto it = g_ctx.find(dev);
  if (it != g_ctx.end()) {
    *out = it->second;
    return 0;
  }
  auto* ctx = new DeviceCtx();
  ctx->device = dev;
  AEGKV_HIP(hipDeviceGetAttribute(&ctx->num_cus, hipDeviceAttributeMultiprocessorCount, dev));
  if (ctx->num_cus <= 0) ctx->num_cus = 1;
  // Keep stream-ordered staging memory cached in the pool between calls.
  hipMemPool_t pool = nullptr;
  if (hipDeviceGetDefaultMemPool(&pool, dev) == hipSuccess && pool) {
    uint64_t threshold = UINT64_MAX;
    (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &threshold);
  }
  (void)hipGetLastError();
  g_ctx[dev] = ctx;
  *out = ctx;
  return 0;
}

// Entry points that upload their descriptors through the host ring cannot
// be captured into a graph: a replay would copy the descriptor from the
// ring slot as a later call left it. They refuse a capturing stream before
// anything is enqueued (aegkv_copy_blocks_noalloc is the capturable copy).
int refuse_capture(hipStream_t stream) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(stream, &status);
  if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
  if (status != hipStreamCaptureStatusNone)
    return fail(AEGKV_EINVAL, "the stream is being captured: this call uploads its descriptor "
                "through a host ring that later calls reuse, so a graph replay would read "
                "another call's descriptor (aegkv_copy_blocks_noalloc can be captured)");
  return 0;
}

// Hand a completed region's event back to the spare list (caller holds
// ctx->mu; the region is popped by the caller).
void ring_retire(Ring& r, const Ring::Region& reg) {
  if (reg.ev) r.spare.push_back({reg.ev, reg.stream});
}

// True once the oldest region's reader has finished (never blocks).
bool ring_front_done(Ring& r) {
  const Ring::Region& f = r.inflight.front();
  return f.ev == nullptr || hipEventQuery(f.ev) == hipSuccess;
}

// Wait for the oldest region's reader, then retire it.
int ring_wait_front(Ring& r) {
  const Ring::Region f = r.inflight.front();
  if (f.ev) AEGKV_HIP(hipEventSynchronize(f.ev));
  ring_retire(r, f);
  r.inflight.pop_front();
  return 0;
}

int ring_grow(Ring& r, size_t need) {
  // Retire everything, then replace the buffers.
  while (!r.inflight.empty()) {
    int rc = ring_wait_front(r);
    if (rc) return rc;
  }
  if (r.host) AEGKV_HIP(hipHostFree(r.host));
  if (r.dev) AEGKV_HIP(hipFree(r.dev));
  r.host = nullptr;
  r.dev = nullptr;
  size_t cap = size_t(4) << 20;
  while (cap < need) cap <<= 1;
  AEGKV_HIP(hipHostMalloc(reinterpret_cast<void**>(&r.host), cap, hipHostMallocDefault));
  AEGKV_HIP(hipMalloc(reinterpret_cast<void**>(&r.dev), cap));
  r.cap = cap;
  r.head = 0;
  return 0;
}

// Reserve `bytes` of the ring (caller holds ctx->mu). Returns offset.
int ring_reserve(Ring& r, size_t bytes, size_t* offset) {
  bytes = (bytes + 255) & ~size_t(255);
  if (bytes == 0) bytes = 256;
  if (bytes > r.cap) {
    int rc = ring_grow(r, bytes);
    if (rc) return rc;
  }
  // Retire completed regions without blocking.
  while (!r.inflight.empty() && ring_front_done(r)) {
    ring_retire(r, r.inflight.front());
    r.inflight.pop_front();
  }
  size_t start = r.head;
  if (start + bytes > r.cap) start = 0;
  const size_t end = start + bytes;
  auto overlaps = [&](const Ring::Region& g) { return g.begin < end && start < g.end; };
  for (;;) {
    bool any = false;
    for (auto& g : r.inflight)
      if (overlaps(g)) {
        any = true;
        break;
      }
    if (!any) break;
    int rc = ring_wait_front(r);
    if (rc) return rc;
  }
  r.head = end;
  *offset = start;
  return 0;
}

int ring_commit(Ring& r, size_t offset, size_t bytes, hipStream_t stream) {
  bytes = (bytes + 255) & ~size_t(255);
  if (bytes == 0) bytes = 256;
  Ring::Spare sp{nullptr, nullptr};
  if (!r.spare.empty()) {
    sp = r.spare.back();
    r.spare.pop_back();
  } else {
    AEGKV_HIP(hipEventCreateWithFlags(&sp.ev, hipEventDisableTiming));
  }
  hipError_t e = hipEventRecord(sp.ev, stream);
  if (e != hipSuccess) {
    r.spare.push_back(sp);
    return hip_fail(e, "hipEventRecord");
  }
  r.inflight.push_back({offset, offset + bytes, sp.ev, stream});
  return 0;
}

// Drop every event this library last recorded on `stream`, which the caller
// has synchronized and is about to destroy: ring regions it read are
// complete (their events are destroyed and the regions count as done),
// spare events recorded there are destroyed, and the DMA sets' fork and
// kernel events are replaced by fresh ones.
int forget_stream(hipStream_t stream) {
  std::vector<DeviceCtx*> ctxs;
  {
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    for (auto& kv : g_ctx) ctxs.push_back(kv.second);
  }
  for (DeviceCtx* ctx : ctxs) {
    {
      std::lock_guard<std::mutex> lk(ctx->mu);
      Ring& r = ctx->ring;
      for (Ring::Region& g : r.inflight)
        if (g.ev && g.stream == stream) {
          (void)hipEventDestroy(g.ev);
          g.ev = nullptr;
        }
      auto keep = r.spare.begin();
      for (auto it = r.spare.begin(); it != r.spare.end(); ++it) {
        if (it->last == stream)
          (void)hipEventDestroy(it->ev);
        else
          *keep++ = *it;
      }
      r.spare.erase(keep, r.spare.end());
    }
    for (DeviceCtx::DmaSet& d : ctx->dma) {
      std::lock_guard<std::mutex> lk(d.mu);
      auto renew = [&](hipEvent_t* ev, hipStream_t* on) -> int {
        if (*ev == nullptr || *on != stream) return 0;
        (void)hipEventDestroy(*ev);
        *ev = nullptr;
        *on = nullptr;
        AEGKV_HIP(hipEventCreateWithFlags(ev, hipEventDisableTiming));
        return 0;
      };
      int rc = renew(&d.fork_ev, &d.fork_on);
      for (int b = 0; b < 2 && !rc; ++b) rc = renew(&d.kernel_ev[b], &d.kernel_on[b]);
      if (rc) return rc;
    }
  }
  (void)hipGetLastError();
  return 0;
}

// ------------------------------------------------------------- validation --

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Checks [ptr, ptr + bytes) lies inside one HIP device allocation.
int check_device_range(const void* ptr, int64_t bytes, const char* what) {
  if (bytes == 0) return 0;
  void* base = nullptr;
  size_t size = 0;
  hipError_t e = hipMemGetAddressRange(&base, &size, const_cast<void*>(ptr));
  if (e != hipSuccess || base == nullptr) {
    (void)hipGetLastError();
    return fail(AEGKV_EINVAL, "%s (%p) is not HIP device memory", what, ptr);
  }
  const uintptr_t b = reinterpret_cast<uintptr_t>(base);
  const uintptr_t p = reinterpret_cast<uintptr_t>(ptr);
  if (p < b || p + static_cast<uint64_t>(bytes) > b + size)
    return fail(AEGKV_ERANGE, "%s: %lld bytes at %p exceed its allocation (%zu bytes at %p)",
                what, static_cast<long long>(bytes), ptr, size, base);
  return 0;
}

// Checks a host pool is pinned and device-visible; kernels dereference it
// directly in DIRECT mode.
int check_host_range(const void* ptr, int64_t bytes, const char* what) {
  if (bytes == 0) return 0;
  {
    std::lock_guard<std::mutex> lk(g_host_mu);
    auto it = g_host_allocs.upper_bound(reinterpret_cast<uintptr_t>(ptr));
    if (it != g_host_allocs.begin()) {
      --it;
      const uintptr_t b = it->first;
      const uintptr_t p = reinterpret_cast<uintptr_t>(ptr);
      if (p >= b && p < b + it->second) {
        if (p + static_cast<uint64_t>(bytes) > b + it->second)
          return fail(AEGKV_ERANGE, "%s: %lld bytes at %p exceed its pinned pool", what,
                      static_cast<long long>(bytes), ptr);
        return 0;
      }
    }
  }
  hipPointerAttribute_t attr;
  std::memset(&attr, 0, sizeof(attr));
  hipError_t e = hipPointerGetAttributes(&attr, ptr);
  if (e != hipSuccess || attr.type != hipMemoryTypeHost) {
    (void)hipGetLastError();
    return fail(AEGKV_EINVAL, "%s (%p) is not pinned host memory (use aegkv_host_alloc)",
                what, ptr);
  }
  return 0;
}

// True when p lies in a pool from aegkv_host_alloc_flags(AEGKV_HOST_UNCACHED).
bool in_uncached_pool(const void* p) {
  std::lock_guard<std::mutex> lk(g_host_mu);
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  auto it = g_uncached_pools.upper_bound(a);
  if (it == g_uncached_pools.begin()) return false;
  --it;
  return a < it->first + it->second;
}

// ----------------------------------------------------------- launching --

// Workgroups to launch for `items` work items: at most `limit` when limit > 0
// (the kernels' grid-stride loops cover the rest), else one per item. An HSA
// dispatch counts work-items in 32 bits, so the grid is also capped at
// (2^32 - 1) / lanes.
int64_t launch_grid(int64_t limit, int64_t items, int lanes) {
  const int64_t cap = static_cast<int64_t>(UINT32_MAX) / lanes;
  int64_t g = items;
  if (limit > 0) g = std::min<int64_t>(g, limit);
  return std::max<int64_t>(1, std::min<int64_t>(g, cap));
}

// Work items one launch may hold. The kernels walk items with a 32-bit
// grid-stride loop (w += gridDim.x) and launch_grid caps a grid at
// (2^32 - 1) / lanes workgroups, so with lanes >= 256 and at most this many
// items, w + gridDim.x stays below 2^32 and the loop never wraps.
constexpr int64_t kMaxLaunchItems =
    static_cast<int64_t>(UINT32_MAX) - static_cast<int64_t>(UINT32_MAX) / 256;

// a * b * c work items, or -1 when that exceeds kMaxLaunchItems (or overflows).
int64_t launch_items(int64_t a, int64_t b, int64_t c) {
  if (a < 0 || b < 0 || c < 0) return -1;
  if (a == 0 || b == 0 || c == 0) return 0;
  if (a > kMaxLaunchItems / b) return -1;
  const int64_t ab = a * b;
  if (ab > kMaxLaunchItems / c) return -1;
  return ab * c;
}

int too_many_items(int64_t a, int64_t b, int64_t c, const char* what) {
  return fail(AEGKV_EINVAL, "%lld %s x %lld segments x %lld chunks exceed the %lld work items "
              "of one launch; split the call", static_cast<long long>(a), what,
              static_cast<long long>(b), static_cast<long long>(c),
              static_cast<long long>(kMaxLaunchItems));
}

struct SwapArgs {
  const SegDesc* segs;
  const EntDesc* ents;
  const int64_t* kpp;
  uint32_t num_segs, num_items, cpt;
  char* host_base;
  int64_t host_stride, host_rank_offset;
  const uint64_t* guard;
};

template <int WG, int U, bool TO_HOST, bool VEC, bool NT>
hipError_t launch_swap_t(int64_t grid, hipStream_t st, const SwapArgs& a) {
  (void)hipGetLastError();  // clear a stale error: the check below is for this launch
  hipLaunchKernelGGL((swap_tiles_kernel<WG, U, TO_HOST, VEC, NT>),
                     dim3(static_cast<uint32_t>(grid)), dim3(WG), 0, st, a.segs, a.ents, a.kpp,
                     a.num_segs, a.num_items, a.cpt, a.host_base, a.host_stride,
                     a.host_rank_offset, a.guard);
  return hipGetLastError();
}

template <int WG, int U>
hipError_t launch_swap_shape(bool to_host, bool nt, int64_t grid, hipStream_t st,
                             const SwapArgs& a) {
  if (to_host)
    return nt ? launch_swap_t<WG, U, true, true, true>(grid, st, a)
              : launch_swap_t<WG, U, true, true, false>(grid, st, a);
  return nt ? launch_swap_t<WG, U, false, true, true>(grid, st, a)
            : launch_swap_t<WG, U, false, true, false>(grid, st, a);
}

hipError_t launch_swap(ShapeSel sh, bool to_host, bool vec, bool nt, int64_t grid,
                       hipStream_t st, const SwapArgs& a) {
  if (!vec)
    return to_host ? launch_swap_t<256, 1, true, false, false>(grid, st, a)
                   : launch_swap_t<256, 1, false, false, false>(grid, st, a);
#define AEGKV_SW(W, UU) \
  if (sh.wg == W && sh.u == UU) return launch_swap_shape<W, UU>(to_host, nt, grid, st, a);
  AEGKV_SW(256, 1) AEGKV_SW(256, 2) AEGKV_SW(256, 4)
  AEGKV_SW(1024, 1) AEGKV_SW(1024, 2) AEGKV_SW(1024, 3) AEGKV_SW(1024, 4)
  AEGKV_SW(1024, 5) AEGKV_SW(1024, 6) AEGKV_SW(1024, 8) AEGKV_SW(1024, 10)
#undef AEGKV_SW
  return hipErrorInvalidValue;
}

// `lds`: dynamic LDS reserved per workgroup. The kernel does not use it; it
// caps how many workgroups share a CU.
template <int WG, int U, bool VEC, bool NT>
hipError_t launch_copy_t(int64_t grid, unsigned lds, hipStream_t st, const CopySeg* s,
                         const PairDesc* p, uint32_t ns, uint32_t items, uint32_t cpt,
                         const uint64_t* guard) {
  (void)hipGetLastError();  // clear a stale error: the check below is for this launch
  hipLaunchKernelGGL((copy_blocks_kernel<WG, U, VEC, NT>), dim3(static_cast<uint32_t>(grid)),
                     dim3(WG), lds, st, s, p, ns, items, cpt, guard);
  return hipGetLastError();
}

hipError_t launch_copy(ShapeSel sh, bool vec, bool nt, int64_t grid, unsigned lds,
                       hipStream_t st, const CopySeg* s, const PairDesc* p, uint32_t ns,
                       uint32_t items, uint32_t cpt, const uint64_t* guard) {
  if (!vec) return launch_copy_t<256, 1, false, false>(grid, 0, st, s, p, ns, items, cpt, guard);
#define AEGKV_CP(W, UU)                                                               \
  if (sh.wg == W && sh.u == UU)                                                       \
    return nt ? launch_copy_t<W, UU, true, true>(grid, lds, st, s, p, ns, items, cpt, guard) \
              : launch_copy_t<W, UU, true, false>(grid, lds, st, s, p, ns, items, cpt, guard);
  AEGKV_CP(256, 1) AEGKV_CP(256, 2) AEGKV_CP(256, 4) AEGKV_CP(256, 8)
  AEGKV_CP(1024, 1) AEGKV_CP(1024, 2) AEGKV_CP(1024, 3) AEGKV_CP(1024, 4)
  AEGKV_CP(1024, 5) AEGKV_CP(1024, 6) AEGKV_CP(1024, 8) AEGKV_CP(1024, 10)
#undef AEGKV_CP
  return hipErrorInvalidValue;
}

template <int WG, int U, int KIND, bool NT>
hipError_t launch_probe_t(int64_t grid, unsigned lds, hipStream_t st, const CopySeg* s,
                          const PairDesc* p, uint32_t ns, uint32_t items, uint32_t cpt,
                          uint32_t* sink, uint32_t magic) {
  (void)hipGetLastError();  // clear a stale error: the check below is for this launch
  hipLaunchKernelGGL((copy_probe_kernel<WG, U, KIND, NT>), dim3(static_cast<uint32_t>(grid)),
                     dim3(WG), lds, st, s, p, ns, items, cpt, sink, magic);
  return hipGetLastError();
}

hipError_t launch_probe(ShapeSel sh, int kind, bool nt, int64_t grid, unsigned lds,
                        hipStream_t st, const CopySeg* s, const PairDesc* p, uint32_t ns,
                        uint32_t items, uint32_t cpt, uint32_t* sink, uint32_t magic) {
#define AEGKV_PR(W, UU)                                                                     \
  if (sh.wg == W && sh.u == UU) {                                                           \
    if (kind == PROBE_READ)                                                                 \
      return launch_probe_t<W, UU, PROBE_READ, false>(grid, lds, st, s, p, ns, items, cpt,  \
                                                      sink, magic);                         \
    return nt ? launch_probe_t<W, UU, PROBE_WRITE, true>(grid, lds, st, s, p, ns, items,    \
                                                         cpt, sink, magic)                  \
              : launch_probe_t<W, UU, PROBE_WRITE, false>(grid, lds, st, s, p, ns, items,   \
                                                          cpt, sink, magic);                \
  }
  AEGKV_PR(256, 1) AEGKV_PR(256, 2) AEGKV_PR(256, 4) AEGKV_PR(256, 8)
  AEGKV_PR(1024, 1) AEGKV_PR(1024, 2) AEGKV_PR(1024, 3) AEGKV_PR(1024, 4)
  AEGKV_PR(1024, 5) AEGKV_PR(1024, 6) AEGKV_PR(1024, 8) AEGKV_PR(1024, 10)
#undef AEGKV_PR
  return hipErrorInvalidValue;
}

hipError_t launch_slices(bool vec, bool nt, int64_t grid, hipStream_t st,
                         const SliceDesc* slices, uint32_t num_slices, uint32_t items) {
  (void)hipGetLastError();  // clear a stale error: the check below is for this launch
  const dim3 g(static_cast<uint32_t>(grid));
  if (!vec)
    hipLaunchKernelGGL((slices_kernel<256, 1, false, false>), g, dim3(256), 0, st, slices,
                       num_slices, items);
  else if (nt)
    hipLaunchKernelGGL((slices_kernel<256, 2, true, true>), g, dim3(256), 0, st, slices,
                       num_slices, items);
  else
    hipLaunchKernelGGL((slices_kernel<256, 2, true, false>), g, dim3(256), 0, st, slices,
                       num_slices, items);
  return hipGetLastError();
}

// ------------------------------------------------------------ swap core --

struct SwapLayout {
  int32_t num_segments;
  void* const* bases;
  const int64_t* page_bytes;
  const int64_t* host_offsets;
  const uint64_t* owner_masks;
  int64_t device_num_blocks;
  int32_t num_groups;
  const int64_t* kpp;
  char* host_pool;
  int64_t host_num_blocks;
  int64_t host_page_bytes;
  int64_t host_rank_offset;
};

struct SwapList {
  int64_t n;
  const int64_t* src;
  const int64_t* dst;
  const int32_t* group;     // may be null: all group 0
  const int64_t* first;     // may be null: all 0
  const int64_t* valid;     // may be null: all kpp[group]
  const uint64_t* guard;    // may be null: the kernels move nothing once *guard != 0
};

bool mul_fits(int64_t a, int64_t b) { return a >= 0 && b >= 0 && (b == 0 || a <= INT64_MAX / b); }

// Argument checks that need no HIP call (run first, so a bad argument costs
// nothing on the device side). dev_vec: every device tile extent is 16 B
// aligned; host_vec: so is every host-pool extent. The 16 B kernel path needs
// both sides aligned.
int validate_layout(const SwapLayout& L, int64_t* composite_bytes, bool* dev_vec,
                    bool* host_vec) {
  if (L.num_segments <= 0) return fail(AEGKV_EINVAL, "num_segments must be positive");
  if (!L.bases || !L.page_bytes || !L.host_offsets || !L.owner_masks)
    return fail(AEGKV_EINVAL, "segment arrays must not be null");
  if (L.device_num_blocks <= 0) return fail(AEGKV_EINVAL, "device_num_blocks must be positive");
  if (L.num_groups <= 0 || L.num_groups > 64)
    return fail(AEGKV_EINVAL, "num_groups must be in [1, 64], got %d", L.num_groups);
  if (!L.kpp) return fail(AEGKV_EINVAL, "group_kernel_blocks_per_page must not be null");
  if (!L.host_pool) return fail(AEGKV_EINVAL, "host_pool must not be null");
  if (L.host_num_blocks <= 0 || L.host_page_bytes <= 0)
    return fail(AEGKV_EINVAL, "host pool geometry must be positive");
  if (!mul_fits(L.host_num_blocks, L.host_page_bytes))
    return fail(AEGKV_ERANGE, "host pool of %lld x %lld bytes overflows",
                static_cast<long long>(L.host_num_blocks),
                static_cast<long long>(L.host_page_bytes));
  if (L.host_rank_offset < 0 || L.host_rank_offset >= L.host_page_bytes)
    return fail(AEGKV_EINVAL, "host_rank_offset must be in [0, host_page_bytes)");
  for (int32_t g = 0; g < L.num_groups; ++g)
    if (L.kpp[g] <= 0 || L.kpp[g] > INT32_MAX)
      return fail(AEGKV_EINVAL, "kernel_blocks_per_page[%d]=%lld must be in [1, 2^31)", g,
                  static_cast<long long>(L.kpp[g]));
  bool v = true;
  int64_t composite = 0;
  for (int32_t s = 0; s < L.num_segments; ++s) {
    const int64_t pb = L.page_bytes[s];
    const int64_t ho = L.host_offsets[s];
    if (!L.bases[s]) return fail(AEGKV_EINVAL, "segment %d base is null", s);
    if (pb <= 0) return fail(AEGKV_EINVAL, "segment %d page_bytes must be positive", s);
    if (ho < 0) return fail(AEGKV_EINVAL, "segment %d host offset must be >= 0", s);
    if (!mul_fits(L.device_num_blocks, pb))
      return fail(AEGKV_ERANGE, "segment %d of %lld x %lld bytes overflows", s,
                  static_cast<long long>(L.device_num_blocks), static_cast<long long>(pb));
    // rank offset + host offset + page must stay inside one host page
    if (ho > L.host_page_bytes || pb > L.host_page_bytes - ho ||
        L.host_rank_offset > L.host_page_bytes - ho - pb)
      return fail(AEGKV_ERANGE,
                  "segment %d [%lld, +%lld) at rank offset %lld overruns the %lld-byte host page",
                  s, static_cast<long long>(ho), static_cast<long long>(pb),
                  static_cast<long long>(L.host_rank_offset),
                  static_cast<long long>(L.host_page_bytes));
    if (L.owner_masks[s] == 0) return fail(AEGKV_EINVAL, "segment %d has no owning group", s);
    for (int32_t g = 0; g < L.num_groups; ++g)
      if (((L.owner_masks[s] >> g) & 1ull) && pb % L.kpp[g] != 0)
        return fail(AEGKV_EEXTENT,
                    "segment %d page of %lld bytes does not split into %lld equal kernel blocks", s,
                    static_cast<long long>(pb), static_cast<long long>(L.kpp[g]));
    if (L.num_groups < 64 && (L.owner_masks[s] >> L.num_groups) != 0)
      return fail(AEGKV_ERANGE, "segment %d owner mask names a group >= %d", s, L.num_groups);
    v = v && aligned16(L.bases[s]) && pb % 16 == 0 && ho % 16 == 0;
    for (int32_t g = 0; g < L.num_groups && v; ++g)
      if ((L.owner_masks[s] >> g) & 1ull) v = (pb / L.kpp[g]) % 16 == 0;
    composite = std::max(composite, ho + pb);
  }
  *composite_bytes = composite;
  *dev_vec = v;
  *host_vec = aligned16(L.host_pool) && L.host_page_bytes % 16 == 0 &&
              L.host_rank_offset % 16 == 0;
  return 0;
}

// Pointer checks through the HIP runtime: every segment lies inside one
// device allocation, and the host pool is pinned and mapped in both modes
// (DIRECT kernels dereference it; STAGED copies of a pageable pool would be
// staged again by the runtime, so they are refused too).
int check_layout_pointers(const SwapLayout& L) {
  for (int32_t s = 0; s < L.num_segments; ++s) {
    int rc = check_device_range(L.bases[s], L.device_num_blocks * L.page_bytes[s],
                                "segment base");
    if (rc) return rc;
  }
  return check_host_range(L.host_pool, L.host_num_blocks * L.host_page_bytes, "host_pool");
}

int validate_list(const SwapLayout& L, const SwapList& E, bool is_swap_in) {
  if (E.n < 0) return fail(AEGKV_EINVAL, "num_entries must be >= 0");
  if (E.n == 0) return 0;
  if (!E.src || !E.dst) return fail(AEGKV_EINVAL, "block id arrays must not be null");
  const int64_t src_lim = is_swap_in ? L.host_num_blocks : L.device_num_blocks;
  const int64_t dst_lim = is_swap_in ? L.device_num_blocks : L.host_num_blocks;
  std::vector<uint8_t> seen(static_cast<size_t>(dst_lim), 0);
  for (int64_t i = 0; i < E.n; ++i) {
    if (E.src[i] < 0 || E.src[i] >= src_lim)
      return fail(AEGKV_ERANGE, "source block id %lld at %lld outside [0, %lld)",
                  static_cast<long long>(E.src[i]), static_cast<long long>(i),
                  static_cast<long long>(src_lim));
    if (E.dst[i] < 0 || E.dst[i] >= dst_lim)
      return fail(AEGKV_ERANGE, "target block id %lld at %lld outside [0, %lld)",
                  static_cast<long long>(E.dst[i]), static_cast<long long>(i),
                  static_cast<long long>(dst_lim));
    if (seen[static_cast<size_t>(E.dst[i])])
      return fail(AEGKV_EDUP, "target block id %lld appears twice",
                  static_cast<long long>(E.dst[i]));
    seen[static_cast<size_t>(E.dst[i])] = 1;
    const int32_t g = E.group ? E.group[i] : 0;
    if (g < 0 || g >= L.num_groups)
      return fail(AEGKV_ERANGE, "group id %d at %lld outside [0, %d)", g,
                  static_cast<long long>(i), L.num_groups);
    const int64_t k = L.kpp[g];
    const int64_t first = E.first ? E.first[i] : 0;
    const int64_t valid = E.valid ? E.valid[i] : k;
    if (first < 0 || valid < 0 || first > k || valid > k - first)
      return fail(AEGKV_EEXTENT, "kernel blocks [%lld, %lld) of entry %lld run past a page of %lld",
                  static_cast<long long>(first), static_cast<long long>(first + valid),
                  static_cast<long long>(i), static_cast<long long>(k));
  }
  return 0;
}

// Launch shape of the swap kernels: 256 lanes with the tuned loads per
// lane, or (tuning key 8) the copy's page-sized shape; bytes alone on the
// unaligned path.
ShapeSel swap_shape(const Tunables& t, bool vec, int64_t max_page) {
  if (!vec) return ShapeSel{256, 1};
  return t.swap_shape_auto ? auto_shape(max_page)
                           : ShapeSel{256, static_cast<int>(t.swap_unroll)};
}

struct Run {
  int64_t host_off;   // byte offset inside the host pool
  int64_t stage_off;  // byte offset inside staging
  int64_t len;
};

// Enqueue one descriptor upload + kernel for entries [idx...] resolved to
// the given host side. Caller holds ctx->mu.
int enqueue_swap_kernel(DeviceCtx* ctx, const SwapLayout& L, const SwapList& E,
                        const std::vector<int64_t>& order, size_t lo, size_t hi,
                        bool is_swap_in, bool staged, char* host_side, int64_t host_stride,
                        int64_t host_rank_off, bool vec, int64_t wgs, hipStream_t stream) {
  const int32_t S = L.num_segments;
  const int64_t n = static_cast<int64_t>(hi - lo);
  if (n == 0) return 0;
  const size_t seg_bytes = sizeof(SegDesc) * S;
  const size_t kpp_off = (seg_bytes + 255) & ~size_t(255);
  const size_t kpp_bytes = sizeof(int64_t) * L.num_groups;
  const size_t ent_off = (kpp_off + kpp_bytes + 255) & ~size_t(255);
  const size_t total = ent_off + sizeof(EntDesc) * n;
  size_t off = 0;
  int rc = ring_reserve(ctx->ring, total, &off);
  if (rc) return rc;
  char* h = ctx->ring.host + off;
  SegDesc* hs = reinterpret_cast<SegDesc*>(h);
  int64_t max_page = 0;
  for (int32_t s = 0; s < S; ++s) {
    hs[s].base = static_cast<char*>(L.bases[s]);
    hs[s].page_bytes = L.page_bytes[s];
    hs[s].host_offset = L.host_offsets[s];
    hs[s].owner_mask = L.owner_masks[s];
    max_page = std::max(max_page, L.page_bytes[s]);
  }
  std::memcpy(h + kpp_off, L.kpp, kpp_bytes);
  EntDesc* he = reinterpret_cast<EntDesc*>(h + ent_off);
  for (int64_t j = 0; j < n; ++j) {
    const int64_t i = order[lo + j];
    const int32_t g = E.group ? E.group[i] : 0;
    EntDesc d;
    d.dev_block = is_swap_in ? E.dst[i] : E.src[i];
    const int64_t host_id = is_swap_in ? E.src[i] : E.dst[i];
    d.host_slot = staged ? j : host_id;
    d.group = g;
    d.first = static_cast<int32_t>(E.first ? E.first[i] : 0);
    d.valid = static_cast<int32_t>(E.valid ? E.valid[i] : L.kpp[g]);
    d.pad = 0;
    he[j] = d;
  }
  char* dv = ctx->ring.dev + off;
  const Tunables t = tunables();
  const ShapeSel sh = swap_shape(t, vec, max_page);
  const int64_t cpt = (max_page + sh.chunk() - 1) / sh.chunk();
  const int64_t items = launch_items(n, S, cpt);
  if (items < 0) {
    ctx->ring.head = off;  // nothing was enqueued; hand the region back
    return too_many_items(n, S, cpt, "entries");
  }
  hipError_t e = hipMemcpyAsync(dv, h, total, hipMemcpyHostToDevice, stream);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(descriptor)");
  SwapArgs a{reinterpret_cast<const SegDesc*>(dv), reinterpret_cast<const EntDesc*>(dv + ent_off),
             reinterpret_cast<const int64_t*>(dv + kpp_off), static_cast<uint32_t>(S),
             static_cast<uint32_t>(items), static_cast<uint32_t>(cpt), host_side, host_stride,
             host_rank_off, E.guard};
  // Non-temporal stores only where the destination is HBM: plain stores to
  // the host pool measured faster (no L2 residency to avoid there).
  const bool nt = t.nt_stores != 0 && !(!is_swap_in && !staged);
  e = launch_swap(sh, !is_swap_in, vec, nt, launch_grid(wgs, items, sh.wg), stream, a);
  if (e != hipSuccess) {
    // the descriptor upload is already enqueued: retire its region in order
    (void)hipGetLastError();
    (void)ring_commit(ctx->ring, off, total, stream);
    return hip_fail(e, "swap_tiles_kernel launch");
  }
  return ring_commit(ctx->ring, off, total, stream);
}

// A staged chunk with more host runs than this counts as scattered.
constexpr size_t kManyRuns = 16;

// Runs of host bytes one staged entry moves, merged when contiguous.
void entry_runs(const SwapLayout& L, const SwapList& E, int64_t i, bool is_swap_in,
                int64_t slot, int64_t composite, std::vector<Run>& runs) {
  const int32_t g = E.group ? E.group[i] : 0;
  const int64_t k = L.kpp[g];
  const int64_t first = E.first ? E.first[i] : 0;
  const int64_t valid = E.valid ? E.valid[i] : k;
  const int64_t host_id = is_swap_in ? E.src[i] : E.dst[i];
  const int64_t host_page = host_id * L.host_page_bytes + L.host_rank_offset;
  const int64_t stage_page = slot * composite;
  for (int32_t s = 0; s < L.num_segments; ++s) {
    if (!((L.owner_masks[s] >> g) & 1ull)) continue;
    const int64_t unit = L.page_bytes[s] / k;
    const int64_t off = unit * first, len = unit * valid;
    if (len == 0) continue;
    const int64_t ho = host_page + L.host_offsets[s] + off;
    const int64_t so = stage_page + L.host_offsets[s] + off;
    if (!runs.empty()) {
      Run& r = runs.back();
      if (r.host_off + r.len == ho && r.stage_off + r.len == so) {
        r.len += len;
        continue;
      }
    }
    runs.push_back({ho, so, len});
  }
}

// A stream on a hardware queue of its own: a stream created with a CU mask
// gets a dedicated queue (here the mask enables every CU), while plain
// streams share the process's GPU_MAX_HW_QUEUES queues, and two copies whose
// streams share a queue run one after the other.
hipError_t dedicated_stream(hipStream_t* out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  int cus = 0;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  std::vector<uint32_t> mask(static_cast<size_t>((cus + 31) / 32), 0xFFFFFFFFu);
  return hipExtStreamCreateWithCUMask(out, static_cast<uint32_t>(mask.size()), mask.data());
}

// Create the DMA streams and events once (caller holds the set's mutex).
int ensure_dma(DeviceCtx::DmaSet& d, int k) {
  if (!d.fork_ev) {
    AEGKV_HIP(hipEventCreateWithFlags(&d.kernel_ev[0], hipEventDisableTiming));
    AEGKV_HIP(hipEventCreateWithFlags(&d.kernel_ev[1], hipEventDisableTiming));
    AEGKV_HIP(hipEventCreateWithFlags(&d.fork_ev, hipEventDisableTiming));
  }
  while (d.streams < k) {
    const int i = d.streams;
    AEGKV_HIP(hipStreamCreateWithFlags(&d.st[i], hipStreamNonBlocking));
    AEGKV_HIP(hipEventCreateWithFlags(&d.join_ev[0][i], hipEventDisableTiming));
    AEGKV_HIP(hipEventCreateWithFlags(&d.join_ev[1][i], hipEventDisableTiming));
    ++d.streams;
  }
  return 0;
}

hipError_t copy_run(const Run& r, bool to_device, char* staging, char* host, hipStream_t st) {
  char* s_ptr = staging + r.stage_off;
  char* h_ptr = host + r.host_off;
  const size_t len = static_cast<size_t>(r.len);
  return to_device ? hipMemcpyAsync(s_ptr, h_ptr, len, hipMemcpyHostToDevice, st)
                   : hipMemcpyAsync(h_ptr, s_ptr, len, hipMemcpyDeviceToHost, st);
}

// Copy the staged runs of one chunk between staging and the host pool over
// the k DMA streams, balanced by bytes, and record join[i] behind stream i's
// share (caller holds the set's mutex).
int runs_on_dma(DeviceCtx::DmaSet& d, int k, const std::vector<Run>& runs, bool to_device,
                char* staging, char* host, hipEvent_t* join) {
  int64_t load[kMaxDmaStreams] = {};
  for (const Run& r : runs) {
    const int i = static_cast<int>(std::min_element(load, load + k) - load);
    load[i] += r.len;
    hipError_t e = copy_run(r, to_device, staging, host, d.st[i]);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(staged run)");
  }
  for (int i = 0; i < k; ++i) AEGKV_HIP(hipEventRecord(join[i], d.st[i]));
  return 0;
}

// The gather (swap-out) or scatter (swap-in) kernel of staged chunk
// order[lo, hi) whose host side is `staging` (one composite page per entry).
// It moves HBM to HBM, so it gets a full grid, except a swap-out whose chunk
// leaves many host runs (scattered host ids, one page-sized copy each):
// there the copies measured faster beside the slower persistent grid
// (41.9 -> 50.1 GB/s), while a few large runs gain from the full grid
// (51.1 -> 55.3 GB/s).
int staged_kernel(DeviceCtx* ctx, const SwapLayout& L, const SwapList& E,
                  const std::vector<int64_t>& order, size_t lo, size_t hi, bool is_swap_in,
                  char* staging, int64_t composite, bool vec_stage, size_t num_runs,
                  const Tunables& t, hipStream_t stream) {
  const int64_t wgs = !is_swap_in && num_runs > kManyRuns ? t.swap_out_workgroups
                                                          : t.staged_workgroups;
  std::lock_guard<std::mutex> lk(ctx->mu);
  return enqueue_swap_kernel(ctx, L, E, order, lo, hi, is_swap_in, true, staging, composite, 0,
                             vec_stage, wgs, stream);
}

// Copy one chunk's runs between staging and the host pool and return the
// caller's stream to after them: on the caller's stream itself (k <= 1), or
// forked over the k DMA streams (after everything the caller's stream
// holds) and joined back, which overlaps the runtime's per-copy gaps.
int chunk_copies(DeviceCtx* ctx, int k, const std::vector<Run>& runs, bool to_device,
                 char* staging, char* host, hipStream_t stream) {
  const int dir = to_device ? 1 : 0;
  if (k <= 1) {
    for (const Run& r : runs) {
      hipError_t e = copy_run(r, to_device, staging, host, stream);
      if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(staged run)");
    }
    return 0;
  }
  DeviceCtx::DmaSet& d = ctx->dma[dir];
  std::lock_guard<std::mutex> lk(d.mu);
  int rc = ensure_dma(d, k);
  if (rc) return rc;
  d.fork_on = stream;
  AEGKV_HIP(hipEventRecord(d.fork_ev, stream));
  for (int j = 0; j < k; ++j) AEGKV_HIP(hipStreamWaitEvent(d.st[j], d.fork_ev, 0));
  rc = runs_on_dma(d, k, runs, to_device, staging, host, d.join_ev[0]);
  // join whatever was enqueued, also after a failed copy
  for (int j = 0; j < k; ++j) {
    if (rc && hipEventRecord(d.join_ev[0][j], d.st[j]) != hipSuccess) continue;
    hipError_t e = hipStreamWaitEvent(stream, d.join_ev[0][j], 0);
    if (e != hipSuccess && !rc) rc = hip_fail(e, "hipStreamWaitEvent(staged copies)");
  }
  return rc;
}

// STAGED one chunk after another, each through its own stream-ordered
// staging allocation: swap-out gathers a chunk and then copies it to the
// host, swap-in copies a chunk from the host and then scatters it.
int staged_serial(DeviceCtx* ctx, const SwapLayout& L, const SwapList& E,
                  const std::vector<int64_t>& order, bool is_swap_in, int64_t composite,
                  size_t step, bool vec_stage, const Tunables& t, int k, hipStream_t stream) {
  std::vector<Run> runs;
  for (size_t lo = 0; lo < order.size(); lo += step) {
    const size_t hi = std::min(order.size(), lo + step);
    runs.clear();
    for (size_t j = lo; j < hi; ++j)
      entry_runs(L, E, order[j], is_swap_in, static_cast<int64_t>(j - lo), composite, runs);
    void* p = nullptr;
    AEGKV_HIP(hipMallocAsync(&p, (hi - lo) * static_cast<size_t>(composite), stream));
    char* buf = static_cast<char*>(p);
    int rc = 0;
    if (is_swap_in) rc = chunk_copies(ctx, k, runs, true, buf, L.host_pool, stream);
    if (!rc)
      rc = staged_kernel(ctx, L, E, order, lo, hi, is_swap_in, buf, composite, vec_stage,
                         runs.size(), t, stream);
    if (!rc && !is_swap_in) rc = chunk_copies(ctx, k, runs, false, buf, L.host_pool, stream);
    if (rc) {
      (void)hipFreeAsync(buf, stream);
      return rc;
    }
    AEGKV_HIP(hipFreeAsync(buf, stream));
  }
  return 0;
}

// STAGED with the copies on the library's k DMA streams and two staging
// buffers, so the gather (swap-out) or scatter (swap-in) of one chunk runs
// while another chunk's copies use the link. Chunk c uses buffer b = c % 2:
//   swap-out: the caller's stream waits the copies of chunk c-2 and gathers
//             chunk c into buffer b; the DMA streams wait that gather, copy
//             the chunk to the host and record join_ev[b];
//   swap-in:  the DMA streams wait the scatter of chunk c-2, copy chunk c
//             from the host into buffer b and record join_ev[b]; the
//             caller's stream waits those and scatters the chunk.
// The DMA streams start after everything the caller's stream holds, the
// staging allocations included; the caller's stream ends after every copy
// and frees the buffers there.
int staged_overlapped(DeviceCtx* ctx, const SwapLayout& L, const SwapList& E,
                      const std::vector<int64_t>& order, bool is_swap_in, int64_t composite,
                      size_t step, bool vec_stage, const Tunables& t, int k,
                      hipStream_t stream) {
  DeviceCtx::DmaSet& d = ctx->dma[is_swap_in ? 1 : 0];
  std::lock_guard<std::mutex> lk(d.mu);
  int rc = ensure_dma(d, k);
  if (rc) return rc;
  const size_t n = order.size();
  const size_t chunks = (n + step - 1) / step;
  const int nbuf = chunks > 1 ? 2 : 1;
  const size_t buf_bytes = std::min(step, n) * static_cast<size_t>(composite);
  char* buf[2] = {nullptr, nullptr};
  for (int b = 0; b < nbuf; ++b) {
    void* p = nullptr;
    hipError_t e = hipMallocAsync(&p, buf_bytes, stream);
    if (e != hipSuccess) {
      if (b) (void)hipFreeAsync(buf[0], stream);
      return hip_fail(e, "hipMallocAsync(staging)");
    }
    buf[b] = static_cast<char*>(p);
  }
  // On a failure after work was enqueued: join every DMA stream back into
  // the caller's stream and free the buffers behind it.
  auto unwind = [&](int status) {
    for (int j = 0; j < k; ++j)
      if (hipEventRecord(d.join_ev[0][j], d.st[j]) == hipSuccess)
        (void)hipStreamWaitEvent(stream, d.join_ev[0][j], 0);
    for (int b = 0; b < nbuf; ++b) (void)hipFreeAsync(buf[b], stream);
    (void)hipGetLastError();
    return status;
  };
  // every DMA stream waits `ev`, recorded on `on` (which *ev_on notes)
  auto fan_in = [&](hipEvent_t ev, hipStream_t* ev_on, hipStream_t on) {
    *ev_on = on;
    hipError_t e = hipEventRecord(ev, on);
    for (int j = 0; j < k && e == hipSuccess; ++j) e = hipStreamWaitEvent(d.st[j], ev, 0);
    return e;
  };
  // the caller's stream waits the copies that recorded join_ev[b]
  auto join = [&](int b) {
    hipError_t e = hipSuccess;
    for (int j = 0; j < k && e == hipSuccess; ++j) e = hipStreamWaitEvent(stream, d.join_ev[b][j], 0);
    return e;
  };
  hipError_t e = fan_in(d.fork_ev, &d.fork_on, stream);
  if (e != hipSuccess) return unwind(hip_fail(e, "staged fork"));
  std::vector<Run> runs;
  for (size_t c = 0; c < chunks; ++c) {
    const size_t lo = c * step, hi = std::min(n, lo + step);
    const int b = static_cast<int>(c & 1);
    runs.clear();
    for (size_t j = lo; j < hi; ++j)
      entry_runs(L, E, order[j], is_swap_in, static_cast<int64_t>(j - lo), composite, runs);
    if (!is_swap_in) {
      if (c >= 2 && (e = join(b)) != hipSuccess)
        return unwind(hip_fail(e, "hipStreamWaitEvent(staged copies)"));
      rc = staged_kernel(ctx, L, E, order, lo, hi, false, buf[b], composite, vec_stage,
                         runs.size(), t, stream);
      if (rc) return unwind(rc);
      if ((e = fan_in(d.kernel_ev[b], &d.kernel_on[b], stream)) != hipSuccess)
        return unwind(hip_fail(e, "staged gather event"));
      rc = runs_on_dma(d, k, runs, false, buf[b], L.host_pool, d.join_ev[b]);
      if (rc) return unwind(rc);
    } else {
      for (int j = 0; c >= 2 && j < k && e == hipSuccess; ++j)
        e = hipStreamWaitEvent(d.st[j], d.kernel_ev[b], 0);
      if (e != hipSuccess) return unwind(hip_fail(e, "hipStreamWaitEvent(staged scatter)"));
      rc = runs_on_dma(d, k, runs, true, buf[b], L.host_pool, d.join_ev[b]);
      if (rc) return unwind(rc);
      if ((e = join(b)) != hipSuccess)
        return unwind(hip_fail(e, "hipStreamWaitEvent(staged copies)"));
      rc = staged_kernel(ctx, L, E, order, lo, hi, true, buf[b], composite, vec_stage,
                         runs.size(), t, stream);
      if (rc) return unwind(rc);
      d.kernel_on[b] = stream;
      if ((e = hipEventRecord(d.kernel_ev[b], stream)) != hipSuccess)
        return unwind(hip_fail(e, "staged scatter event"));
    }
  }
  // swap-out: each DMA stream's last join follows all of its earlier copies
  if (!is_swap_in && (e = join(static_cast<int>((chunks - 1) & 1))) != hipSuccess)
    return unwind(hip_fail(e, "hipStreamWaitEvent(staged copies)"));
  for (int b = 0; b < nbuf; ++b) AEGKV_HIP(hipFreeAsync(buf[b], stream));
  return 0;
}

int swap_core(const SwapLayout& L, const SwapList& E, bool is_swap_in, int mode,
              hipStream_t stream) {
  if (mode < AEGKV_MODE_AUTO || mode > AEGKV_MODE_STAGED)
    return fail(AEGKV_EINVAL, "unknown transfer mode %d", mode);
  const Tunables t = tunables();
  if (mode == AEGKV_MODE_AUTO)
    mode = static_cast<int>(is_swap_in ? t.auto_h2d : t.auto_d2h);
  const bool staged = mode == AEGKV_MODE_STAGED;
  int64_t composite = 0;
  bool dev_vec = false, host_vec = false;
  int rc = validate_layout(L, &composite, &dev_vec, &host_vec);
  if (rc) return rc;
  rc = validate_list(L, E, is_swap_in);
  if (rc) return rc;
  if (E.n == 0) return 0;
  {
    // the whole list in one launch (a staged chunk holds fewer entries)
    int64_t max_page = 0;
    for (int32_t s = 0; s < L.num_segments; ++s) max_page = std::max(max_page, L.page_bytes[s]);
    const bool vec = staged ? dev_vec && composite % 16 == 0 : dev_vec && host_vec;
    const ShapeSel sh = swap_shape(t, vec, max_page);
    const int64_t cpt = (max_page + sh.chunk() - 1) / sh.chunk();
    if (launch_items(E.n, L.num_segments, cpt) < 0)
      return too_many_items(E.n, L.num_segments, cpt, "entries");
  }
  rc = check_layout_pointers(L);
  if (rc) return rc;
  rc = refuse_capture(stream);
  if (rc) return rc;
  DeviceCtx* ctx = nullptr;
  rc = get_ctx(&ctx);
  if (rc) return rc;

  std::vector<int64_t> order(static_cast<size_t>(E.n));
  for (int64_t i = 0; i < E.n; ++i) order[static_cast<size_t>(i)] = i;

  if (!staged) {
    std::lock_guard<std::mutex> lk(ctx->mu);
    // link-bound: a few persistent workgroups
    const int64_t wgs = is_swap_in                        ? t.swap_in_workgroups
                        : in_uncached_pool(L.host_pool) ? t.swap_out_workgroups_uncached
                                                        : t.swap_out_workgroups;
    return enqueue_swap_kernel(ctx, L, E, order, 0, order.size(), is_swap_in, false,
                               L.host_pool, L.host_page_bytes, L.host_rank_offset,
                               dev_vec && host_vec, wgs, stream);
  }

  // STAGED: host-id order lets consecutive host pages merge into one DMA.
  const int64_t* host_ids = is_swap_in ? E.src : E.dst;
  std::stable_sort(order.begin(), order.end(),
                   [&](int64_t a, int64_t b) { return host_ids[a] < host_ids[b]; });
  const size_t step = static_cast<size_t>(
      std::max<int64_t>(1, std::min<int64_t>(E.n, t.staging_bytes / composite)));
  // Staging comes from hipMallocAsync (256 B aligned) with a composite stride.
  const bool vec_stage = dev_vec && composite % 16 == 0;
  const int k = static_cast<int>(std::min<int64_t>(t.staged_dma_streams, kMaxDmaStreams));
  const bool overlap = (t.staged_overlap >> (is_swap_in ? 1 : 0)) & 1;
  if (k <= 1 || !overlap)
    return staged_serial(ctx, L, E, order, is_swap_in, composite, step, vec_stage, t, k,
                         stream);
  return staged_overlapped(ctx, L, E, order, is_swap_in, composite, step, vec_stage, t, k,
                           stream);
}

// Whole-block copies from a source cache to a target cache (the same cache
// for copy_blocks), in steps shared by the allocating and the
// allocation-free entry points: layout checks, id checks, device-range
// checks, the launch shape, then descriptor upload and launch.

// Checks that need no HIP call and no memory: segment geometry and the
// 16 B path. *max_page receives the largest page.
int copy_check_layout(int32_t num_segments, void* const* src_bases, void* const* dst_bases,
                      const int64_t* page_bytes, int64_t src_num_blocks,
                      int64_t dst_num_blocks, int64_t num_pairs, const int64_t* src_ids,
                      const int64_t* dst_ids, bool same_cache, bool* vec, int64_t* max_page) {
  if (num_segments <= 0) return fail(AEGKV_EINVAL, "num_segments must be positive");
  if (!src_bases || !dst_bases || !page_bytes)
    return fail(AEGKV_EINVAL, "segment arrays must not be null");
  if (src_num_blocks <= 0 || dst_num_blocks <= 0)
    return fail(AEGKV_EINVAL, "device_num_blocks must be positive");
  if (num_pairs < 0) return fail(AEGKV_EINVAL, "num_pairs must be >= 0");
  if (num_pairs > 0 && (!src_ids || !dst_ids))
    return fail(AEGKV_EINVAL, "block id arrays must not be null");
  bool v = true;
  int64_t mp = 0;
  for (int32_t s = 0; s < num_segments; ++s) {
    if (!src_bases[s] || !dst_bases[s]) return fail(AEGKV_EINVAL, "segment %d base is null", s);
    if (page_bytes[s] <= 0)
      return fail(AEGKV_EINVAL, "segment %d page_bytes must be positive", s);
    if (!mul_fits(src_num_blocks, page_bytes[s]) || !mul_fits(dst_num_blocks, page_bytes[s]))
      return fail(AEGKV_ERANGE, "segment %d of %lld x %lld bytes overflows", s,
                  static_cast<long long>(std::max(src_num_blocks, dst_num_blocks)),
                  static_cast<long long>(page_bytes[s]));
    if (!same_cache) {
      const uintptr_t a0 = reinterpret_cast<uintptr_t>(src_bases[s]);
      const uintptr_t b0 = reinterpret_cast<uintptr_t>(dst_bases[s]);
      const uintptr_t a1 = a0 + static_cast<uint64_t>(src_num_blocks * page_bytes[s]);
      const uintptr_t b1 = b0 + static_cast<uint64_t>(dst_num_blocks * page_bytes[s]);
      if (a0 < b1 && b0 < a1)
        return fail(AEGKV_EOVERLAP,
                    "segment %d: source and target caches overlap (copy within one cache "
                    "with aegkv_copy_blocks)", s);
    }
    v = v && aligned16(src_bases[s]) && aligned16(dst_bases[s]) && page_bytes[s] % 16 == 0;
    mp = std::max(mp, page_bytes[s]);
  }
  *vec = v;
  *max_page = mp;
  return 0;
}

// Every id inside its cache (first offending pair in pair order).
int copy_check_ranges(int64_t src_num_blocks, int64_t dst_num_blocks, int64_t num_pairs,
                      const int64_t* src_ids, const int64_t* dst_ids) {
  for (int64_t i = 0; i < num_pairs; ++i) {
    const int64_t s = src_ids[i], d = dst_ids[i];
    if (s < 0 || s >= src_num_blocks || d < 0 || d >= dst_num_blocks)
      return fail(AEGKV_ERANGE, "pair %lld (%lld -> %lld) outside [0, %lld) -> [0, %lld)",
                  static_cast<long long>(i), static_cast<long long>(s),
                  static_cast<long long>(d), static_cast<long long>(src_num_blocks),
                  static_cast<long long>(dst_num_blocks));
  }
  return 0;
}

int dup_target(int64_t id) {
  return fail(AEGKV_EDUP, "target block id %lld appears twice", static_cast<long long>(id));
}

int source_is_target(int64_t id) {
  return fail(AEGKV_EOVERLAP, "block %lld is both a source and a target",
              static_cast<long long>(id));
}

// Distinct targets, and (within one cache) no source that is also a
// target, with a block-indexed map. Ids are in range.
int copy_check_ids_map(int64_t dst_num_blocks, int64_t num_pairs, const int64_t* src_ids,
                       const int64_t* dst_ids, bool same_cache) {
  std::vector<uint8_t> target(static_cast<size_t>(dst_num_blocks), 0);
  for (int64_t i = 0; i < num_pairs; ++i) {
    uint8_t& t = target[static_cast<size_t>(dst_ids[i])];
    if (t) return dup_target(dst_ids[i]);
    t = 1;
  }
  if (same_cache)
    for (int64_t i = 0; i < num_pairs; ++i)
      if (target[static_cast<size_t>(src_ids[i])]) return source_is_target(src_ids[i]);
  return 0;
}

// The same checks without memory of the block count's size: sorted copies
// of the ids in the caller's work arrays (num_pairs entries each).
int copy_check_ids_sorted(int64_t num_pairs, const int64_t* src_ids, const int64_t* dst_ids,
                          bool same_cache, int64_t* work_src, int64_t* work_dst) {
  std::copy(dst_ids, dst_ids + num_pairs, work_dst);
  std::sort(work_dst, work_dst + num_pairs);
  for (int64_t i = 1; i < num_pairs; ++i)
    if (work_dst[i] == work_dst[i - 1]) return dup_target(work_dst[i]);
  if (!same_cache) return 0;
  std::copy(src_ids, src_ids + num_pairs, work_src);
  std::sort(work_src, work_src + num_pairs);
  for (int64_t i = 0, j = 0; i < num_pairs && j < num_pairs;) {
    if (work_src[i] == work_dst[j]) return source_is_target(work_src[i]);
    if (work_src[i] < work_dst[j]) ++i;
    else ++j;
  }
  return 0;
}

int copy_check_device(int32_t num_segments, void* const* src_bases, void* const* dst_bases,
                      const int64_t* page_bytes, int64_t src_num_blocks,
                      int64_t dst_num_blocks, bool same_cache) {
  for (int32_t s = 0; s < num_segments; ++s) {
    int rc = check_device_range(src_bases[s], src_num_blocks * page_bytes[s], "segment base");
    if (rc) return rc;
    if (!same_cache) {
      rc = check_device_range(dst_bases[s], dst_num_blocks * page_bytes[s], "target segment base");
      if (rc) return rc;
    }
  }
  return 0;
}

struct CopyPlan {
  ShapeSel sh;
  bool vec;
  int64_t cpt;    // chunks per tile
  int64_t items;  // work items (pair x segment x chunk)
};

int copy_plan(const Tunables& t, bool vec, int64_t max_page, int32_t num_segments,
              int64_t num_pairs, CopyPlan* out) {
  ShapeSel sh = auto_shape(max_page);
  if (t.copy_unroll > 0)
    sh = ShapeSel{t.copy_lanes == 256 ? 256 : 1024, static_cast<int>(t.copy_unroll)};
  if (!vec) sh = ShapeSel{256, 1};
  const int64_t cpt = (max_page + sh.chunk() - 1) / sh.chunk();
  const int64_t items = launch_items(num_pairs, num_segments, cpt);
  if (items < 0) return too_many_items(num_pairs, num_segments, cpt, "pairs");
  *out = CopyPlan{sh, vec, cpt, items};
  return 0;
}

// Byte offset of the pair table after num_segments CopySeg entries.
size_t copy_pair_offset(int32_t num_segments) {
  return (sizeof(CopySeg) * static_cast<size_t>(num_segments) + 255) & ~size_t(255);
}

// Pairs in order of their target ids (by_dst) or source ids, by a stable
// least-significant-byte-first counting sort: one pass over the pairs per
// byte of the largest id, with `tmp` (num_pairs entries) as the other
// buffer. Pairs already in order are left alone.
void sort_pairs(PairDesc* a, int64_t n, bool by_dst, PairDesc* tmp) {
  auto key = [by_dst](const PairDesc& x) { return by_dst ? x.dst : x.src; };
  int64_t top = 0;
  bool sorted = true;
  for (int64_t i = 0; i < n; ++i) {
    top = std::max(top, key(a[i]));
    if (i > 0 && key(a[i]) < key(a[i - 1])) sorted = false;
  }
  if (sorted) return;
  PairDesc* from = a;
  PairDesc* to = tmp;
  for (int shift = 0; shift < 64 && (top >> shift) != 0; shift += 8) {
    int64_t start[257] = {};
    for (int64_t i = 0; i < n; ++i) ++start[((key(from[i]) >> shift) & 255) + 1];
    for (int d = 0; d < 256; ++d) start[d + 1] += start[d];
    for (int64_t i = 0; i < n; ++i) to[start[(key(from[i]) >> shift) & 255]++] = from[i];
    std::swap(from, to);
  }
  if (from != a) std::copy(from, from + n, a);
}

void pack_copy_desc(char* h, int32_t num_segments, void* const* src_bases,
                    void* const* dst_bases, const int64_t* page_bytes, int64_t num_pairs,
                    const int64_t* src_ids, const int64_t* dst_ids, int64_t order,
                    PairDesc* tmp) {
  CopySeg* hs = reinterpret_cast<CopySeg*>(h);
  for (int32_t s = 0; s < num_segments; ++s)
    hs[s] = CopySeg{static_cast<const char*>(src_bases[s]), static_cast<char*>(dst_bases[s]),
                    page_bytes[s], 0};
  PairDesc* hp = reinterpret_cast<PairDesc*>(h + copy_pair_offset(num_segments));
  for (int64_t i = 0; i < num_pairs; ++i) hp[i] = PairDesc{src_ids[i], dst_ids[i]};
  // Targets are distinct and never sources, so any order gives the same
  // result. Copies of small tiles run faster with their targets in order:
  // the workgroups running together then write near one another.
  if (order == 1 || order == 2) sort_pairs(hp, num_pairs, order == 1, tmp);
}

// What a copy call launches: the copy itself (guarded by `guard` when it is
// not null), or one of its measurement twins (aegkv_copy_probe) with the
// sink word and magic they take.
struct CopyKind {
  int probe = 0;            // 0 = copy, PROBE_READ or PROBE_WRITE
  uint32_t* sink = nullptr;
  uint32_t magic = 0;
  const uint64_t* guard = nullptr;
};

// Launch the copy kernel (or a probe twin) over descriptors already on the
// device at `dv`, with the copy's grid and LDS policy.
hipError_t copy_launch(const CopyPlan& p, const Tunables& t, int num_cus, int32_t num_segments,
                       const char* dv, hipStream_t stream, const CopyKind& kind = CopyKind()) {
  const int64_t grid = launch_grid(t.copy_wgs_per_cu * num_cus, p.items, p.sh.wg);
  const unsigned lds = p.sh.wg == 1024 && p.sh.chunk() >= (int64_t(32) << 10)
                           ? static_cast<unsigned>(t.copy_lds_bytes) : 0u;
  const CopySeg* segs = reinterpret_cast<const CopySeg*>(dv);
  const PairDesc* pairs = reinterpret_cast<const PairDesc*>(dv + copy_pair_offset(num_segments));
  const uint32_t ns = static_cast<uint32_t>(num_segments);
  const uint32_t items = static_cast<uint32_t>(p.items);
  const uint32_t cpt = static_cast<uint32_t>(p.cpt);
  if (kind.probe)
    return launch_probe(p.sh, kind.probe, t.nt_stores != 0, grid, lds, stream, segs, pairs, ns,
                        items, cpt, kind.sink, kind.magic);
  return launch_copy(p.sh, p.vec, t.nt_stores != 0, grid, lds, stream, segs, pairs, ns, items,
                     cpt, kind.guard);
}

int copy_core(int32_t num_segments, void* const* src_bases, void* const* dst_bases,
              const int64_t* page_bytes, int64_t src_num_blocks, int64_t dst_num_blocks,
              int64_t num_pairs, const int64_t* src_ids, const int64_t* dst_ids, bool same_cache,
              hipStream_t stream, const CopyKind& kind = CopyKind()) {
  bool vec = false;
  int64_t max_page = 0;
  int rc = copy_check_layout(num_segments, src_bases, dst_bases, page_bytes, src_num_blocks,
                             dst_num_blocks, num_pairs, src_ids, dst_ids, same_cache, &vec,
                             &max_page);
  if (!rc) rc = copy_check_ranges(src_num_blocks, dst_num_blocks, num_pairs, src_ids, dst_ids);
  if (!rc) rc = copy_check_ids_map(dst_num_blocks, num_pairs, src_ids, dst_ids, same_cache);
  if (rc || num_pairs == 0) return rc;
  if (kind.probe && !vec)
    return fail(AEGKV_EINVAL, "the probes move 16 B per lane: bases and pages must be "
                "16 B multiples");
  const Tunables t = tunables();
  CopyPlan plan;
  rc = copy_plan(t, vec, max_page, num_segments, num_pairs, &plan);
  if (rc) return rc;
  rc = copy_check_device(num_segments, src_bases, dst_bases, page_bytes, src_num_blocks,
                         dst_num_blocks, same_cache);
  if (rc) return rc;
  rc = refuse_capture(stream);
  if (rc) return rc;
  DeviceCtx* ctx = nullptr;
  rc = get_ctx(&ctx);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(ctx->mu);
  const size_t total = copy_pair_offset(num_segments) + sizeof(PairDesc) * num_pairs;
  size_t off = 0;
  rc = ring_reserve(ctx->ring, total, &off);
  if (rc) return rc;
  char* h = ctx->ring.host + off;
  std::vector<PairDesc> tmp(t.copy_order != 0 ? static_cast<size_t>(num_pairs) : 0);
  pack_copy_desc(h, num_segments, src_bases, dst_bases, page_bytes, num_pairs, src_ids,
                 dst_ids, t.copy_order, tmp.data());
  char* dv = ctx->ring.dev + off;
  hipError_t e = hipMemcpyAsync(dv, h, total, hipMemcpyHostToDevice, stream);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(descriptor)");
  e = copy_launch(plan, t, ctx->num_cus, num_segments, dv, stream, kind);
  if (e != hipSuccess) {
    // the descriptor upload is already enqueued: retire its region in order
    (void)hipGetLastError();
    (void)ring_commit(ctx->ring, off, total, stream);
    return hip_fail(e, kind.probe ? "copy_probe_kernel launch" : "copy_blocks_kernel launch");
  }
  return ring_commit(ctx->ring, off, total, stream);
}

// ------------------------------------------------ allocation-free copies --
//
// aegkv_copy_blocks_noalloc: aegkv_copy_blocks for callers that cannot
// allocate. The descriptor (segment table + pair table) goes to `scratch`,
// a fixed device array every GPU holds for the life of the process, instead
// of the library's upload ring; it travels in the kernel arguments of small
// fill launches (2 KiB each), so a graph that captures the call replays its
// own descriptor. The ids are checked with fixed host arrays instead of a
// block-indexed map. Nothing is allocated on the host or the device. Every
// call on a device shares that device's array, so calls that overlap on one
// device (different streams, or threads, or a graph replayed beside other
// calls) race; calls on one stream are ordered.

constexpr int32_t kNoAllocMaxSegments = 1024;
constexpr int64_t kNoAllocMaxPairs = 65536;
constexpr size_t kNoAllocBytes =
    sizeof(CopySeg) * kNoAllocMaxSegments + sizeof(PairDesc) * kNoAllocMaxPairs;  // 1.03 MiB
constexpr int kNoAllocMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

std::mutex g_noalloc_mu;                        // guards everything below
char* g_scratch_ptr[kNoAllocMaxDevices] = {};   // device address of `scratch`, per device
int g_noalloc_cus[kNoAllocMaxDevices] = {};
alignas(256) unsigned char g_noalloc_host[kNoAllocBytes];  // descriptor packing (pageable)
int64_t g_noalloc_work[2][kNoAllocMaxPairs];    // sorted id copies for the checks
PairDesc g_noalloc_order[kNoAllocMaxPairs];     // the other buffer of the pair sort

// Looks up this device's `scratch` address and CU count, once per device,
// with that device current (caller holds g_noalloc_mu). aegkv_init does it
// for every device at set-up.
int noalloc_resolve(int dev) {
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return fail(AEGKV_EINVAL, "device %d is outside the %d devices the allocation-free "
                "copy supports", dev, kNoAllocMaxDevices);
  if (g_scratch_ptr[dev]) return 0;
  void* p = nullptr;
  AEGKV_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  int cus = 0;
  AEGKV_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  g_noalloc_cus[dev] = cus > 0 ? cus : 1;
  g_scratch_ptr[dev] = static_cast<char*>(p);
  return 0;
}

// Device address of the current device's `scratch` (caller holds
// g_noalloc_mu). Without aegkv_init, the first call on a device looks it
// up, unless that call's stream is being captured: the lookup may load the
// library's code object, which must not happen inside a capture.
int noalloc_scratch(int dev, hipStream_t stream, char** out, int* num_cus) {
  if (dev < 0 || dev >= kNoAllocMaxDevices || !g_scratch_ptr[dev]) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(stream, &status);
    if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
    if (status != hipStreamCaptureStatusNone)
      return fail(AEGKV_EINVAL, "the allocation-free copy's first call on device %d is being "
                  "captured; call aegkv_init() before capturing", dev);
    int rc = noalloc_resolve(dev);
    if (rc) return rc;
  }
  *out = g_scratch_ptr[dev];
  *num_cus = g_noalloc_cus[dev];
  return 0;
}

// dst[0, bytes) <- src[0, bytes) on `stream`, kFillBytes per launch of
// desc_fill_kernel (bytes is a multiple of 16; descriptors are).
hipError_t noalloc_fill(char* dst, const unsigned char* src, size_t bytes, hipStream_t stream) {
  FillArgs a;
  a.pad = 0;
  for (size_t off = 0; off < bytes; off += kFillBytes) {
    const size_t n = std::min<size_t>(kFillBytes, bytes - off);
    std::memcpy(a.data, src + off, n);
    a.dst = reinterpret_cast<v4u*>(dst + off);
    a.words = static_cast<uint32_t>(n / 16);
    (void)hipGetLastError();  // clear a stale error: the check below is for this launch
    hipLaunchKernelGGL(desc_fill_kernel, dim3(1), dim3(kFillBytes / 16), 0, stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

int copy_noalloc(int32_t num_segments, void* const* bases, const int64_t* page_bytes,
                 int64_t num_blocks, int64_t num_pairs, const int64_t* src_ids,
                 const int64_t* dst_ids, hipStream_t stream) {
  if (num_segments > kNoAllocMaxSegments)
    return fail(AEGKV_ENOMEM, "%d segments exceed the allocation-free copy's maximum of %d "
                "(use aegkv_copy_blocks)", num_segments, kNoAllocMaxSegments);
  if (num_pairs > kNoAllocMaxPairs)
    return fail(AEGKV_ENOMEM, "%lld pairs exceed the allocation-free copy's maximum of %lld "
                "(use aegkv_copy_blocks)", static_cast<long long>(num_pairs),
                static_cast<long long>(kNoAllocMaxPairs));
  bool vec = false;
  int64_t max_page = 0;
  int rc = copy_check_layout(num_segments, bases, bases, page_bytes, num_blocks, num_blocks,
                             num_pairs, src_ids, dst_ids, true, &vec, &max_page);
  if (!rc) rc = copy_check_ranges(num_blocks, num_blocks, num_pairs, src_ids, dst_ids);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  rc = copy_check_ids_sorted(num_pairs, src_ids, dst_ids, true, g_noalloc_work[0],
                             g_noalloc_work[1]);
  if (rc || num_pairs == 0) return rc;
  const Tunables t = tunables();
  CopyPlan plan;
  rc = copy_plan(t, vec, max_page, num_segments, num_pairs, &plan);
  if (rc) return rc;
  rc = copy_check_device(num_segments, bases, bases, page_bytes, num_blocks, num_blocks, true);
  if (rc) return rc;
  int dev = -1;
  AEGKV_HIP(hipGetDevice(&dev));
  char* dv = nullptr;
  int num_cus = 0;
  rc = noalloc_scratch(dev, stream, &dv, &num_cus);
  if (rc) return rc;
  pack_copy_desc(reinterpret_cast<char*>(g_noalloc_host), num_segments, bases, bases,
                 page_bytes, num_pairs, src_ids, dst_ids, t.copy_order, g_noalloc_order);
  const size_t total = copy_pair_offset(num_segments) + sizeof(PairDesc) * num_pairs;
  // The descriptor reaches `scratch` through kernel arguments, not a copy
  // from the packing area: a copy node captured into a graph would read the
  // packing area again at every replay, after later calls rewrote it.
  hipError_t e = noalloc_fill(dv, g_noalloc_host, total, stream);
  if (e != hipSuccess) return hip_fail(e, "desc_fill_kernel launch");
  e = copy_launch(plan, t, num_cus, num_segments, dv, stream);
  if (e != hipSuccess) return hip_fail(e, "copy_blocks_kernel launch");
  return 0;
}

// Weight slices host -> device in one call (aegkv_load_slices).
int slices_core(int64_t n, void* const* dst, const void* const* src, const int64_t* bytes,
                int mode, hipStream_t stream) {
  if (n < 0) return fail(AEGKV_EINVAL, "num_slices must be >= 0");
  if (n > 0 && (!dst || !src || !bytes)) return fail(AEGKV_EINVAL, "slice arrays must not be null");
  if (mode < AEGKV_MODE_AUTO || mode > AEGKV_MODE_STAGED)
    return fail(AEGKV_EINVAL, "unknown transfer mode %d", mode);
  const Tunables t = tunables();
  if (mode == AEGKV_MODE_AUTO) mode = static_cast<int>(t.auto_h2d);
  // non-empty slices, checked; distinct targets
  std::vector<int64_t> keep;
  keep.reserve(static_cast<size_t>(n));
  bool vec = true;
  for (int64_t i = 0; i < n; ++i) {
    if (bytes[i] < 0)
      return fail(AEGKV_EINVAL, "slice %lld has %lld bytes", static_cast<long long>(i),
                  static_cast<long long>(bytes[i]));
    if (bytes[i] == 0) continue;
    if (!dst[i] || !src[i])
      return fail(AEGKV_EINVAL, "slice %lld has a null pointer", static_cast<long long>(i));
    keep.push_back(i);
    vec = vec && aligned16(dst[i]) && aligned16(src[i]) && bytes[i] % 16 == 0;
  }
  std::vector<int64_t> by_dst(keep);
  std::sort(by_dst.begin(), by_dst.end(), [&](int64_t a, int64_t b) {
    return reinterpret_cast<uintptr_t>(dst[a]) < reinterpret_cast<uintptr_t>(dst[b]);
  });
  for (size_t k = 1; k < by_dst.size(); ++k) {
    const int64_t a = by_dst[k - 1], b = by_dst[k];
    if (reinterpret_cast<uintptr_t>(dst[a]) + static_cast<uint64_t>(bytes[a]) >
        reinterpret_cast<uintptr_t>(dst[b]))
      return fail(AEGKV_EOVERLAP, "target slices %lld and %lld overlap",
                  static_cast<long long>(a), static_cast<long long>(b));
  }
  if (keep.empty()) return 0;
  const int64_t chunk = vec ? int64_t(256) * 16 * 2 : int64_t(256) * 16;
  int64_t items = 0;
  for (int64_t i : keep) {
    items += (bytes[i] + chunk - 1) / chunk;
    if (items > kMaxLaunchItems)
      return fail(AEGKV_EINVAL, "the slices need more than the %lld work items of one launch; "
                  "split the call", static_cast<long long>(kMaxLaunchItems));
  }
  for (int64_t i : keep) {
    int rc = check_device_range(dst[i], bytes[i], "target slice");
    if (!rc) rc = check_host_range(src[i], bytes[i], "source slice");
    if (rc) return rc;
  }
  if (mode == AEGKV_MODE_STAGED) {
    // the runtime's DMA copy per slice, as the reference's copy_ per slice
    for (int64_t i : keep)
      AEGKV_HIP(hipMemcpyAsync(dst[i], src[i], static_cast<size_t>(bytes[i]),
                               hipMemcpyHostToDevice, stream));
    return 0;
  }
  int rc = refuse_capture(stream);
  if (rc) return rc;
  DeviceCtx* ctx = nullptr;
  rc = get_ctx(&ctx);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(ctx->mu);
  const size_t total = sizeof(SliceDesc) * keep.size();
  size_t off = 0;
  rc = ring_reserve(ctx->ring, total, &off);
  if (rc) return rc;
  SliceDesc* h = reinterpret_cast<SliceDesc*>(ctx->ring.host + off);
  int64_t first = 0;
  for (size_t k = 0; k < keep.size(); ++k) {
    const int64_t i = keep[k];
    h[k] = SliceDesc{static_cast<char*>(dst[i]), static_cast<const char*>(src[i]), bytes[i],
                     first};
    first += (bytes[i] + chunk - 1) / chunk;
  }
  char* dv = ctx->ring.dev + off;
  hipError_t e = hipMemcpyAsync(dv, h, total, hipMemcpyHostToDevice, stream);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(descriptor)");
  e = launch_slices(vec, t.nt_stores != 0, launch_grid(t.swap_in_workgroups, items, 256), stream,
                    reinterpret_cast<const SliceDesc*>(dv), static_cast<uint32_t>(keep.size()),
                    static_cast<uint32_t>(items));
  if (e != hipSuccess) {
    (void)hipGetLastError();
    (void)ring_commit(ctx->ring, off, total, stream);
    return hip_fail(e, "slices_kernel launch");
  }
  return ring_commit(ctx->ring, off, total, stream);
}

}  // namespace

// =============================================================== C ABI ==

extern "C" {

int aegkv_abi_version(void) { return AEGKV_ABI_VERSION; }

const char* aegkv_last_error(void) { return g_err; }

int64_t aegkv_tune(int key, int64_t value) {
  (void)env_status();  // environment overrides apply before the first change
  std::lock_guard<std::mutex> lk(g_tune_mu);
  int64_t* slot = nullptr;
  switch (key) {
    case AEGKV_TUNE_SWAP_OUT_WORKGROUPS: slot = &g_tune.swap_out_workgroups; break;
    case AEGKV_TUNE_SWAP_IN_WORKGROUPS: slot = &g_tune.swap_in_workgroups; break;
    case AEGKV_TUNE_STAGING_BYTES: slot = &g_tune.staging_bytes; break;
    case AEGKV_TUNE_AUTO_D2H: slot = &g_tune.auto_d2h; break;
    case AEGKV_TUNE_AUTO_H2D: slot = &g_tune.auto_h2d; break;
    case AEGKV_TUNE_NT_STORES: slot = &g_tune.nt_stores; break;
    case AEGKV_TUNE_COPY_WGS_PER_CU: slot = &g_tune.copy_wgs_per_cu; break;
    case AEGKV_TUNE_COPY_UNROLL: slot = &g_tune.copy_unroll; break;
    case AEGKV_TUNE_COPY_LANES: slot = &g_tune.copy_lanes; break;
    case AEGKV_TUNE_SWAP_SHAPE_AUTO: slot = &g_tune.swap_shape_auto; break;
    case AEGKV_TUNE_SWAP_UNROLL: slot = &g_tune.swap_unroll; break;
    case AEGKV_TUNE_STAGED_WORKGROUPS: slot = &g_tune.staged_workgroups; break;
    case AEGKV_TUNE_STAGED_DMA_STREAMS: slot = &g_tune.staged_dma_streams; break;
    case AEGKV_TUNE_COPY_LDS_BYTES: slot = &g_tune.copy_lds_bytes; break;
    case AEGKV_TUNE_STAGED_OVERLAP: slot = &g_tune.staged_overlap; break;
    case AEGKV_TUNE_SWAP_OUT_WORKGROUPS_UNCACHED: slot = &g_tune.swap_out_workgroups_uncached; break;
    case AEGKV_TUNE_COPY_ORDER: slot = &g_tune.copy_order; break;
    default: return fail(AEGKV_EINVAL, "unknown tuning key %d", key);
  }
  const int64_t prev = *slot;
  if (value >= 0) {
    if ((key == AEGKV_TUNE_AUTO_D2H || key == AEGKV_TUNE_AUTO_H2D) &&
        value != AEGKV_MODE_DIRECT && value != AEGKV_MODE_STAGED)
      return fail(AEGKV_EINVAL, "AUTO must resolve to DIRECT or STAGED");
    if ((key == AEGKV_TUNE_SWAP_OUT_WORKGROUPS || key == AEGKV_TUNE_SWAP_IN_WORKGROUPS ||
         key == AEGKV_TUNE_SWAP_OUT_WORKGROUPS_UNCACHED) &&
        (value < 1 || value > 65536))
      return fail(AEGKV_EINVAL, "swap workgroups must be in [1, 65536]");
    if (key == AEGKV_TUNE_STAGING_BYTES && value < (int64_t(1) << 20))
      return fail(AEGKV_EINVAL, "staging must be at least 1 MiB");
    if (key == AEGKV_TUNE_COPY_WGS_PER_CU && value > 64)
      return fail(AEGKV_EINVAL, "copy workgroups per CU must be in [0, 64]");
    if (key == AEGKV_TUNE_STAGED_WORKGROUPS && value > (int64_t(1) << 24))
      return fail(AEGKV_EINVAL, "staged workgroups must be in [0, 2^24]");
    if (key == AEGKV_TUNE_SWAP_UNROLL && value != 1 && value != 2 && value != 4)
      return fail(AEGKV_EINVAL, "swap unroll must be 1, 2 or 4");
    if (key == AEGKV_TUNE_COPY_LANES && value != 0 && value != 256 && value != 1024)
      return fail(AEGKV_EINVAL, "copy lanes must be 0, 256 or 1024");
    if (key == AEGKV_TUNE_COPY_UNROLL && value != 0 && g_tune.copy_lanes == 256 &&
        value != 1 && value != 2 && value != 4 && value != 8)
      return fail(AEGKV_EINVAL, "with 256 copy lanes the unroll must be 0, 1, 2, 4 or 8");
    if (key == AEGKV_TUNE_COPY_LANES && value == 256 && g_tune.copy_unroll != 0 &&
        g_tune.copy_unroll != 1 && g_tune.copy_unroll != 2 && g_tune.copy_unroll != 4 &&
        g_tune.copy_unroll != 8)
      return fail(AEGKV_EINVAL, "256 copy lanes take an unroll of 1, 2, 4 or 8");
    if (key == AEGKV_TUNE_COPY_UNROLL && value != 0 && !valid_copy_unroll(value))
      return fail(AEGKV_EINVAL, "copy unroll must be 0 (auto) or one of 1,2,3,4,5,6,8,10");
    if (key == AEGKV_TUNE_COPY_ORDER && value > 2)
      return fail(AEGKV_EINVAL, "copy order must be 0 (as given), 1 (by target) or 2 (by source)");
    if (key == AEGKV_TUNE_STAGED_DMA_STREAMS && value > kMaxDmaStreams)
      return fail(AEGKV_EINVAL, "staged DMA streams must be in [0, %d]", kMaxDmaStreams);
    if (key == AEGKV_TUNE_COPY_LDS_BYTES && value > kMaxLdsPerWorkgroup)
      return fail(AEGKV_EINVAL, "copy LDS reservation must be in [0, %lld]",
                  static_cast<long long>(kMaxLdsPerWorkgroup));
    if (key == AEGKV_TUNE_SWAP_SHAPE_AUTO && value > 1)
      return fail(AEGKV_EINVAL, "swap shape selector is 0 or 1");
    if (key == AEGKV_TUNE_STAGED_OVERLAP && value > 3)
      return fail(AEGKV_EINVAL, "staged overlap is a 2-bit mask (0-3)");
    *slot = value;
  }
  return prev;
}

int aegkv_swap(const int64_t* source_block_ids, const int64_t* target_block_ids,
               int64_t num_ids, int is_swap_in, void* kv_cache, int64_t cache_num_blocks,
               void* kv_swap, int64_t swap_num_blocks, int64_t block_bytes, int mode,
               hipStream_t stream) {
  g_err[0] = '\0';
  if (int rc = env_status()) return rc;
  if (block_bytes <= 0) return fail(AEGKV_EINVAL, "block_bytes must be positive");
  void* bases[1] = {kv_cache};
  const int64_t page[1] = {block_bytes};
  const int64_t hoff[1] = {0};
  const uint64_t owner[1] = {1};
  const int64_t kpp[1] = {1};
  SwapLayout L{1, bases, page, hoff, owner, cache_num_blocks, 1, kpp,
               static_cast<char*>(kv_swap), swap_num_blocks, block_bytes, 0};
  SwapList E{num_ids, source_block_ids, target_block_ids, nullptr, nullptr, nullptr, nullptr};
  return swap_core(L, E, is_swap_in != 0, mode, stream);
}

int aegkv_swap_blocks(int32_t num_segments, void* const* segment_bases,
                      const int64_t* segment_page_bytes, const int64_t* segment_host_offsets,
                      const uint64_t* segment_owner_masks, int64_t device_num_blocks,
                      int32_t num_groups, const int64_t* group_kernel_blocks_per_page,
                      void* host_pool, int64_t host_num_blocks, int64_t host_page_bytes,
                      int64_t host_rank_offset, int64_t num_entries,
                      const int64_t* source_block_ids, const int64_t* target_block_ids,
                      const int32_t* group_ids, const int64_t* first_kernel_blocks,
                      const int64_t* valid_kernel_blocks, int is_swap_in, int mode,
                      const uint64_t* guard, hipStream_t stream) {
  g_err[0] = '\0';
  if (int rc = env_status()) return rc;
  if (num_entries > 0 && (!group_ids || !first_kernel_blocks || !valid_kernel_blocks))
    return fail(AEGKV_EINVAL, "entry metadata arrays must not be null");
  if (guard && (reinterpret_cast<uintptr_t>(guard) & 7u))
    return fail(AEGKV_EINVAL, "the move guard must be an 8-byte aligned word");
  SwapLayout L{num_segments, segment_bases, segment_page_bytes, segment_host_offsets,
               segment_owner_masks, device_num_blocks, num_groups,
               group_kernel_blocks_per_page, static_cast<char*>(host_pool), host_num_blocks,
               host_page_bytes, host_rank_offset};
  SwapList E{num_entries, source_block_ids, target_block_ids, group_ids, first_kernel_blocks,
             valid_kernel_blocks, guard};
  return swap_core(L, E, is_swap_in != 0, mode, stream);
}

int aegkv_copy_blocks(int32_t num_segments, void* const* segment_bases,
                      const int64_t* segment_page_bytes, int64_t device_num_blocks,
                      int64_t num_pairs, const int64_t* src_block_ids,
                      const int64_t* dst_block_ids, hipStream_t stream) {
  g_err[0] = '\0';
  if (int rc = env_status()) return rc;
  return copy_core(num_segments, segment_bases, segment_bases, segment_page_bytes,
                   device_num_blocks, device_num_blocks, num_pairs, src_block_ids,
                   dst_block_ids, true, stream);
}

int aegkv_copy_blocks_noalloc(int32_t num_segments, void* const* segment_bases,
                              const int64_t* segment_page_bytes, int64_t device_num_blocks,
                              int64_t num_pairs, const int64_t* src_block_ids,
                              const int64_t* dst_block_ids, hipStream_t stream) {
  g_err[0] = '\0';
  if (int rc = env_status()) return rc;
  return copy_noalloc(num_segments, segment_bases, segment_page_bytes, device_num_blocks,
                      num_pairs, src_block_ids, dst_block_ids, stream);
}

int aegkv_copy_probe(int kind, int32_t num_segments, void* const* segment_bases,
                     const int64_t* segment_page_bytes, int64_t device_num_blocks,
                     int64_t num_pairs, const int64_t* src_block_ids,
                     const int64_t* dst_block_ids, uint32_t* sink, uint32_t magic,
                     hipStream_t stream) {
  g_err[0] = '\0';
  if (int rc = env_status()) return rc;
  if (kind != AEGKV_PROBE_READ && kind != AEGKV_PROBE_WRITE)
    return fail(AEGKV_EINVAL, "probe kind %d is neither AEGKV_PROBE_READ nor AEGKV_PROBE_WRITE",
                kind);
  if (!sink || (reinterpret_cast<uintptr_t>(sink) & 3u))
    return fail(AEGKV_EINVAL, "the probe's sink must be a 4-byte aligned device word");
  CopyKind k;
  k.probe = kind == AEGKV_PROBE_READ ? PROBE_READ : PROBE_WRITE;
  k.sink = sink;
  k.magic = magic;
  return copy_core(num_segments, segment_bases, segment_bases, segment_page_bytes,
                   device_num_blocks, device_num_blocks, num_pairs, src_block_ids,
                   dst_block_ids, true, stream, k);
}

int aegkv_migrate_blocks(int32_t num_segments, void* const* src_segment_bases,
                         void* const* dst_segment_bases, const int64_t* segment_page_bytes,
                         int64_t src_num_blocks, int64_t dst_num_blocks, int64_t num_pairs,
                         const int64_t* src_block_ids, const int64_t* dst_block_ids,
                         const uint64_t* guard, hipStream_t stream) {
  g_err[0] = '\0';
  if (int rc = env_status()) return rc;
  if (!src_segment_bases || !dst_segment_bases)
    return fail(AEGKV_EINVAL, "segment arrays must not be null");
  if (guard && (reinterpret_cast<uintptr_t>(guard) & 7u))
    return fail(AEGKV_EINVAL, "the move guard must be an 8-byte aligned word");
  CopyKind k;
  k.guard = guard;
  return copy_core(num_segments, src_segment_bases, dst_segment_bases, segment_page_bytes,
                   src_num_blocks, dst_num_blocks, num_pairs, src_block_ids, dst_block_ids,
                   false, stream, k);
}

int aegkv_load_slices(int64_t num_slices, void* const* dst, const void* const* src,
                      const int64_t* bytes, int mode, hipStream_t stream) {
  g_err[0] = '\0';
  if (int rc = env_status()) return rc;
  return slices_core(num_slices, dst, src, bytes, mode, stream);
}

int aegkv_stream_create(hipStream_t* stream) {
  g_err[0] = '\0';
  if (!stream) return fail(AEGKV_EINVAL, "stream pointer must not be null");
  AEGKV_HIP(dedicated_stream(stream));
  return 0;
}

int aegkv_stream_create_masked(hipStream_t* stream, const uint32_t* cu_mask,
                               int32_t mask_words) {
  g_err[0] = '\0';
  if (!stream) return fail(AEGKV_EINVAL, "stream pointer must not be null");
  if (!cu_mask || mask_words <= 0) return fail(AEGKV_EINVAL, "CU mask must not be empty");
  int dev = -1, cus = 0;
  AEGKV_HIP(hipGetDevice(&dev));
  AEGKV_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  int64_t set = 0;
  for (int32_t w = 0; w < mask_words; ++w)
    for (int b = 0; b < 32; ++b)
      if ((cu_mask[w] >> b) & 1u) {
        if (int64_t(w) * 32 + b >= cus)
          return fail(AEGKV_ERANGE, "CU mask names CU %d; the device has %d", w * 32 + b, cus);
        ++set;
      }
  if (set == 0) return fail(AEGKV_EINVAL, "CU mask enables no CU");
  hipError_t e = hipExtStreamCreateWithCUMask(stream, static_cast<uint32_t>(mask_words), cu_mask);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(static_cast<int>(e),
                "hipExtStreamCreateWithCUMask refused the mask (%s); the runtime takes runs "
                "of 8 or more consecutive CUs starting at a multiple of 8",
                hipGetErrorString(e));
  }
  return 0;
}

int aegkv_stream_release(hipStream_t stream) {
  g_err[0] = '\0';
  if (!stream) return fail(AEGKV_EINVAL, "stream must not be null");
  AEGKV_HIP(hipStreamSynchronize(stream));
  return forget_stream(stream);
}

int aegkv_stream_destroy(hipStream_t stream) {
  // the stream's queued work finishes first, whatever the caller dropped,
  // and no library event stays recorded on it
  if (int rc = aegkv_stream_release(stream)) return rc;
  AEGKV_HIP(hipStreamDestroy(stream));
  return 0;
}

int aegkv_init(void) {
  g_err[0] = '\0';
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
    (void)hipGetLastError();
    return 0;  // no device: nothing to set up
  }
  int current = -1;
  AEGKV_HIP(hipGetDevice(&current));
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  // the current device first, with no device switch (a process with one
  // device never switches)
  int rc = current < kNoAllocMaxDevices ? noalloc_resolve(current) : 0;
  bool switched = false;
  for (int d = 0; d < count && d < kNoAllocMaxDevices && !rc; ++d) {
    if (d == current || g_scratch_ptr[d]) continue;
    const hipError_t e = hipSetDevice(d);
    switched = true;
    rc = e != hipSuccess ? hip_fail(e, "hipSetDevice") : noalloc_resolve(d);
  }
  if (switched) {
    const hipError_t e = hipSetDevice(current);
    if (!rc && e != hipSuccess) rc = hip_fail(e, "hipSetDevice");
  }
  return rc;
}

int aegkv_host_alloc(void** ptr, int64_t bytes) { return aegkv_host_alloc_flags(ptr, bytes, 0); }

int aegkv_host_alloc_flags(void** ptr, int64_t bytes, int flags) {
  g_err[0] = '\0';
  if (!ptr || bytes <= 0) return fail(AEGKV_EINVAL, "host_alloc needs a pointer and bytes > 0");
  if (flags & ~(AEGKV_HOST_UNCACHED | AEGKV_HOST_COHERENT))
    return fail(AEGKV_EINVAL, "unknown host_alloc flags 0x%x", flags);
  // hipHostMalloc refuses the pair; uncached memory bypasses every cache
  // already, and COHERENT is meant for cached pools
  if ((flags & AEGKV_HOST_UNCACHED) && (flags & AEGKV_HOST_COHERENT))
    return fail(AEGKV_EINVAL, "AEGKV_HOST_UNCACHED and AEGKV_HOST_COHERENT do not combine "
                "(uncached memory is coherent already)");
  const size_t n = static_cast<size_t>(bytes);
  const bool uncached = (flags & AEGKV_HOST_UNCACHED) != 0;
  unsigned hf = hipHostMallocMapped | hipHostMallocPortable;
  if (uncached) hf |= hipHostMallocUncached;
  if (flags & AEGKV_HOST_COHERENT) hf |= hipHostMallocCoherent;
  if (!uncached) {
    void* p = nullptr;
    AEGKV_HIP(hipHostMalloc(&p, n, hf));
    std::lock_guard<std::mutex> lk(g_host_mu);
    g_host_allocs[reinterpret_cast<uintptr_t>(p)] = n;
    *ptr = p;
    return 0;
  }
  const size_t want = (n + kHostPage - 1) / kHostPage * kHostPage;
  {
    // the smallest free range that fits
    std::lock_guard<std::mutex> lk(g_host_mu);
    auto best = g_uncached_free.end();
    for (auto it = g_uncached_free.begin(); it != g_uncached_free.end(); ++it)
      if (it->second >= want && (best == g_uncached_free.end() || it->second < best->second))
        best = it;
    if (best != g_uncached_free.end()) {
      const uintptr_t start = best->first;
      const size_t len = best->second;
      g_uncached_free.erase(best);
      if (len > want) g_uncached_free[start + want] = len - want;
      g_uncached_pools[start] = want;
      g_host_allocs[start] = n;
      *ptr = reinterpret_cast<void*>(start);
      return 0;
    }
  }
  void* p = nullptr;
  AEGKV_HIP(hipHostMalloc(&p, want, hf));
  std::lock_guard<std::mutex> lk(g_host_mu);
  const uintptr_t b = reinterpret_cast<uintptr_t>(p);
  g_uncached_blocks[b] = want;
  g_uncached_pools[b] = want;
  g_host_allocs[b] = n;
  *ptr = p;
  return 0;
}

int aegkv_host_usage(int64_t* pinned_bytes, int64_t* uncached_free_bytes) {
  g_err[0] = '\0';
  std::lock_guard<std::mutex> lk(g_host_mu);
  int64_t pinned = 0, free_bytes = 0;
  for (const auto& kv : g_host_allocs)
    if (!g_uncached_pools.count(kv.first)) pinned += static_cast<int64_t>(kv.second);
  for (const auto& kv : g_uncached_blocks) pinned += static_cast<int64_t>(kv.second);
  for (const auto& kv : g_uncached_free) free_bytes += static_cast<int64_t>(kv.second);
  if (pinned_bytes) *pinned_bytes = pinned;
  if (uncached_free_bytes) *uncached_free_bytes = free_bytes;
  return 0;
}

int aegkv_host_free(void* ptr) {
  g_err[0] = '\0';
  if (!ptr) return 0;
  {
    std::lock_guard<std::mutex> lk(g_host_mu);
    const uintptr_t b = reinterpret_cast<uintptr_t>(ptr);
    if (g_host_allocs.erase(b) == 0)
      return fail(AEGKV_EINVAL, "%p is not a live pool from aegkv_host_alloc", ptr);
    auto u = g_uncached_pools.find(b);
    if (u != g_uncached_pools.end()) {
      // back to the free list, merged with free neighbours of the same block
      uintptr_t start = b;
      size_t len = u->second;
      g_uncached_pools.erase(u);
      auto blk = g_uncached_blocks.upper_bound(start);
      --blk;  // the block holding the pool (every pool lies in one)
      const uintptr_t block_begin = blk->first, block_end = blk->first + blk->second;
      auto next = g_uncached_free.find(start + len);
      if (next != g_uncached_free.end() && start + len < block_end) {
        len += next->second;
        g_uncached_free.erase(next);
      }
      auto prev = g_uncached_free.lower_bound(start);
      if (prev != g_uncached_free.begin()) {
        --prev;
        if (prev->first >= block_begin && prev->first + prev->second == start) {
          prev->second += len;
          return 0;
        }
      }
      g_uncached_free[start] = len;
      return 0;
    }
  }
  AEGKV_HIP(hipHostFree(ptr));
  return 0;
}

}  // extern "C"

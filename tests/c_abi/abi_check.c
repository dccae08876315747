/*
 * A C caller of libaegkv with no Python and no torch: the drop-in boundary
 * as a C or C++ runtime would use it. Builds a small composite cache
 * (6 segments x 64 blocks x 4 KiB tiles) in device memory and a pinned host
 * pool, then checks byte for byte against plain loops on the host:
 *   1. aegkv_swap_blocks swap-out of 10 device blocks to 10 host pages,
 *   2. aegkv_swap_blocks swap-in of those pages to 10 other device blocks,
 *   3. aegkv_copy_blocks of 8 pairs,
 *   4. a rejected call (a target id out of range): negative status, a
 *      message, and nothing changed,
 *   5. a swap-in behind a set move guard: nothing moves.
 * The swap-in of step 2 runs with a clear guard (a coherent pinned word).
 * `abi_check --version` only prints the library's ABI version (no GPU).
 * Exit status 0 and the last line "c-abi ok" on success.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "aegkv.h"

#define NSEG 6
#define NBLK 64
#define TILE 4096
#define NHOST 32
#define NMOVE 10
#define NPAIR 8

static int fail_hip(hipError_t e, const char* what) {
  fprintf(stderr, "%s failed: %s\n", what, hipGetErrorString(e));
  return 2;
}

#define HIPCHK(call)                          \
  do {                                        \
    hipError_t e_ = (call);                   \
    if (e_ != hipSuccess) return fail_hip(e_, #call); \
  } while (0)

static unsigned char pattern(int seg, int blk, int i) {
  return (unsigned char)(seg * 131 + blk * 17 + i * 7 + (i >> 8));
}

/* host copy of the whole cache, segment-major */
static unsigned char want[NSEG][NBLK][TILE];
static unsigned char got[NBLK][TILE];

static int compare_cache(void* const* seg_bases, const char* step) {
  for (int s = 0; s < NSEG; ++s) {
    hipError_t e = hipMemcpy(got, seg_bases[s], sizeof(got), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return fail_hip(e, "hipMemcpy(segment)");
    if (memcmp(got, want[s], sizeof(got)) != 0) {
      fprintf(stderr, "%s: segment %d differs from the host loops\n", step, s);
      return 1;
    }
  }
  return 0;
}

int main(int argc, char** argv) {
  if (argc > 1 && strcmp(argv[1], "--version") == 0) {
    printf("aegkv ABI %d\n", aegkv_abi_version());
    return aegkv_abi_version() == AEGKV_ABI_VERSION ? 0 : 1;
  }
  HIPCHK(hipSetDevice(0));
  if (aegkv_init() != 0) {
    fprintf(stderr, "aegkv_init: %s\n", aegkv_last_error());
    return 2;
  }
  hipStream_t stream;
  HIPCHK(hipStreamCreate(&stream));

  void* seg_bases[NSEG];
  int64_t page_bytes[NSEG], host_off[NSEG];
  uint64_t owners[NSEG];
  for (int s = 0; s < NSEG; ++s) {
    for (int b = 0; b < NBLK; ++b)
      for (int i = 0; i < TILE; ++i) want[s][b][i] = pattern(s, b, i);
    HIPCHK(hipMalloc(&seg_bases[s], (size_t)NBLK * TILE));
    HIPCHK(hipMemcpy(seg_bases[s], want[s], (size_t)NBLK * TILE, hipMemcpyHostToDevice));
    page_bytes[s] = TILE;
    host_off[s] = (int64_t)s * TILE;
    owners[s] = 1; /* every segment belongs to cache group 0 */
  }
  const int64_t kpp[1] = {1}; /* one kernel block per page */
  const int64_t composite = (int64_t)NSEG * TILE;

  void* host = NULL;
  int rc = aegkv_host_alloc(&host, NHOST * composite);
  if (rc) {
    fprintf(stderr, "aegkv_host_alloc: %d %s\n", rc, aegkv_last_error());
    return 2;
  }
  memset(host, 0, (size_t)(NHOST * composite));
  unsigned char* want_host = calloc((size_t)(NHOST * composite), 1);
  if (!want_host) return 2;
  uint64_t* guard = NULL;
  rc = aegkv_host_alloc_flags((void**)&guard, 64, AEGKV_HOST_COHERENT);
  if (rc) {
    fprintf(stderr, "aegkv_host_alloc_flags(coherent): %d %s\n", rc, aegkv_last_error());
    return 2;
  }
  guard[0] = 0;

  int64_t out_src[NMOVE], out_dst[NMOVE], in_dst[NMOVE], first[NMOVE], valid[NMOVE];
  int32_t grp[NMOVE];
  for (int i = 0; i < NMOVE; ++i) {
    out_src[i] = 1 + 3 * i;             /* device blocks 1, 4, ..., 28 */
    out_dst[i] = NHOST - 1 - 2 * i;     /* host pages 31, 29, ..., 13 */
    in_dst[i] = 33 + 2 * i;             /* device blocks 33, 35, ..., 51 */
    first[i] = 0;
    valid[i] = 1;
    grp[i] = 0;
  }

  /* 1. swap-out, and the same bytes moved by host loops */
  rc = aegkv_swap_blocks(NSEG, seg_bases, page_bytes, host_off, owners, NBLK, 1, kpp, host,
                         NHOST, composite, 0, NMOVE, out_src, out_dst, grp, first, valid, 0,
                         AEGKV_MODE_AUTO, NULL, stream);
  if (rc) {
    fprintf(stderr, "swap-out: %d %s\n", rc, aegkv_last_error());
    return 1;
  }
  HIPCHK(hipStreamSynchronize(stream));
  for (int i = 0; i < NMOVE; ++i)
    for (int s = 0; s < NSEG; ++s)
      memcpy(want_host + out_dst[i] * composite + host_off[s], want[s][out_src[i]], TILE);
  if (memcmp(host, want_host, (size_t)(NHOST * composite)) != 0) {
    fprintf(stderr, "swap-out: host pool differs from the host loops\n");
    return 1;
  }

  /* 2. swap-in of those pages to other device blocks */
  rc = aegkv_swap_blocks(NSEG, seg_bases, page_bytes, host_off, owners, NBLK, 1, kpp, host,
                         NHOST, composite, 0, NMOVE, out_dst, in_dst, grp, first, valid, 1,
                         AEGKV_MODE_AUTO, guard, stream);
  if (rc) {
    fprintf(stderr, "swap-in: %d %s\n", rc, aegkv_last_error());
    return 1;
  }
  HIPCHK(hipStreamSynchronize(stream));
  for (int i = 0; i < NMOVE; ++i)
    for (int s = 0; s < NSEG; ++s)
      memcpy(want[s][in_dst[i]], want_host + out_dst[i] * composite + host_off[s], TILE);
  rc = compare_cache(seg_bases, "swap-in");
  if (rc) return rc;

  /* 3. copy_blocks: sources 2..9, targets 54..61 (disjoint, distinct) */
  int64_t csrc[NPAIR], cdst[NPAIR];
  for (int i = 0; i < NPAIR; ++i) {
    csrc[i] = 2 + i;
    cdst[i] = 54 + i;
  }
  rc = aegkv_copy_blocks(NSEG, seg_bases, page_bytes, NBLK, NPAIR, csrc, cdst, stream);
  if (rc) {
    fprintf(stderr, "copy_blocks: %d %s\n", rc, aegkv_last_error());
    return 1;
  }
  HIPCHK(hipStreamSynchronize(stream));
  for (int i = 0; i < NPAIR; ++i)
    for (int s = 0; s < NSEG; ++s) memcpy(want[s][cdst[i]], want[s][csrc[i]], TILE);
  rc = compare_cache(seg_bases, "copy_blocks");
  if (rc) return rc;

  /* 4. a target id past the cache: rejected before anything is enqueued */
  int64_t bad_dst[NPAIR];
  memcpy(bad_dst, cdst, sizeof(bad_dst));
  bad_dst[NPAIR - 1] = NBLK;
  rc = aegkv_copy_blocks(NSEG, seg_bases, page_bytes, NBLK, NPAIR, cdst, bad_dst, stream);
  if (rc >= 0 || aegkv_last_error()[0] == '\0') {
    fprintf(stderr, "out-of-range target: status %d, message \"%s\"\n", rc, aegkv_last_error());
    return 1;
  }
  printf("rejected as expected: %d %s\n", rc, aegkv_last_error());
  HIPCHK(hipStreamSynchronize(stream));
  rc = compare_cache(seg_bases, "after the rejected call");
  if (rc) return rc;

  /* 5. the guard set (as a failed fence wait would): the swap-in of the same
   * pages to blocks 0..9 moves nothing */
  __atomic_store_n(guard, 1, __ATOMIC_RELEASE);
  int64_t low[NMOVE];
  for (int i = 0; i < NMOVE; ++i) low[i] = i;
  rc = aegkv_swap_blocks(NSEG, seg_bases, page_bytes, host_off, owners, NBLK, 1, kpp, host,
                         NHOST, composite, 0, NMOVE, out_dst, low, grp, first, valid, 1,
                         AEGKV_MODE_AUTO, guard, stream);
  if (rc) {
    fprintf(stderr, "guarded swap-in: %d %s\n", rc, aegkv_last_error());
    return 1;
  }
  HIPCHK(hipStreamSynchronize(stream));
  rc = compare_cache(seg_bases, "after the guarded swap-in");
  if (rc) return rc;
  printf("guarded swap-in moved nothing\n");

  free(want_host);
  aegkv_host_free(guard);
  aegkv_host_free(host);
  for (int s = 0; s < NSEG; ++s) HIPCHK(hipFree(seg_bases[s]));
  if (aegkv_stream_release(stream) != 0) {
    fprintf(stderr, "aegkv_stream_release: %s\n", aegkv_last_error());
    return 1;
  }
  HIPCHK(hipStreamDestroy(stream));
  printf("c-abi ok\n");
  return 0;
}

/*
 * aegkv.h - C ABI of libaegkv.so, the MI355X (gfx950) KV-cache movement
 * library: paged K/V block swap-out (HBM -> pinned host), swap-in
 * (pinned host -> HBM) and in-HBM block copy.
 *
 * Conventions shared by every entry point
 *   - Plain pointers and sizes only. Device pointers are HIP device
 *     addresses on the *current* HIP device; host pool pointers must come
 *     from hipHostMalloc (aegkv_host_alloc or a pinned torch tensor).
 *   - Id arrays and metadata arrays are HOST arrays, read during the call.
 *     The library validates them completely before enqueueing anything,
 *     then uploads a compact descriptor through its own stream-ordered
 *     pinned->device ring, so the caller may reuse the arrays on return.
 *   - All work is enqueued on `stream` (a hipStream_t; torch's
 *     torch.cuda.current_stream().cuda_stream). Nothing synchronises the
 *     host except when the upload ring is full and must wait for an older
 *     call on some stream to retire.
 *   - Return value: 0 on success; a negative AEGKV_E* code for an invalid
 *     argument (nothing was enqueued); a positive hipError_t value when the
 *     HIP runtime failed. aegkv_last_error() gives a message for the
 *     calling thread's most recent failure.
 *   - The caller keeps every buffer alive until the stream has passed the
 *     enqueued work (record an event after the call and wait on it).
 *   - Calls are not for stream capture (hipGraph), except
 *     aegkv_copy_blocks_noalloc: their descriptors are copied from a host
 *     ring whose slots later calls reuse, and a replayed copy would read
 *     whatever the slot holds then. On a capturing stream they return
 *     AEGKV_EINVAL with nothing enqueued (aegkv_load_slices in STAGED mode,
 *     runtime copies from the pinned sources only, is capturable;
 *     aegkv_fence_signal and aegkv_fence_wait take their arguments by value
 *     and are too; aegkv_fence_publish refuses a capturing stream).
 */
#ifndef AEGKV_H
#define AEGKV_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AEGKV_ABI_VERSION 3

/* status codes (negative: rejected before any work was enqueued) */
#define AEGKV_OK 0
#define AEGKV_EINVAL (-1)        /* malformed argument (null, negative size) */
#define AEGKV_ERANGE (-2)        /* block id / group id outside its pool     */
#define AEGKV_EDUP (-3)          /* a target block id appears twice          */
#define AEGKV_EEXTENT (-4)       /* kernel-block extent outside the page     */
#define AEGKV_EOVERLAP (-5)      /* copy: a source is also a target, or the
                                    migration's two caches overlap          */
#define AEGKV_ENOMEM (-6)        /* output arrays too small for the rows, or
                                    a call beyond a fixed buffer's limit    */

/* host-transfer designs for swap-out / swap-in */
#define AEGKV_MODE_AUTO 0   /* library choice per direction: DIRECT unless
                               AEGKV_AUTO_D2H / AEGKV_AUTO_H2D say otherwise */
#define AEGKV_MODE_DIRECT 1 /* gather/scatter kernel reads/writes the pinned
                               host pool directly over PCIe                    */
#define AEGKV_MODE_STAGED 2 /* gather/scatter kernel <-> contiguous device
                               staging, plus hipMemcpyAsync of merged runs
                               (the runtime runs them on SDMA engines or as
                               blit kernels); leaves the CUs to concurrent
                               compute                                         */

/* Environment, read once per process before the first call:
 *   AEGKV_AUTO_D2H, AEGKV_AUTO_H2D = direct | staged   (what AUTO picks)
 *   AEGKV_STAGING_BYTES = integer >= 1048576           (STAGED chunk)
 * An invalid value makes aegkv_swap, aegkv_swap_blocks, aegkv_copy_blocks
 * and aegkv_migrate_blocks return AEGKV_EINVAL with a message naming it. */

/* tuning keys for aegkv_tune (values < 0 query without changing) */
#define AEGKV_TUNE_SWAP_OUT_WORKGROUPS 1 /* swap-out kernel: workgroups    */
#define AEGKV_TUNE_STAGING_BYTES 2   /* max device staging per chunk      */
#define AEGKV_TUNE_AUTO_D2H 3        /* mode AUTO picks for swap-out      */
#define AEGKV_TUNE_AUTO_H2D 4        /* mode AUTO picks for swap-in       */
#define AEGKV_TUNE_NT_STORES 5       /* 1: non-temporal stores to HBM     */
#define AEGKV_TUNE_COPY_WGS_PER_CU 6 /* copy_blocks grid: 0 = one workgroup
                                        per work item, else per-CU count   */
#define AEGKV_TUNE_COPY_UNROLL 7     /* copy_blocks loads per lane: 0 = from
                                        the page size, else 1-6, 8 or 10   */
#define AEGKV_TUNE_SWAP_SHAPE_AUTO 8 /* 1: swap kernels pick their shape
                                        from the page size like copy_blocks */
#define AEGKV_TUNE_SWAP_IN_WORKGROUPS 9 /* swap-in kernel: workgroups      */
#define AEGKV_TUNE_STAGED_DMA_STREAMS 10 /* STAGED copies fan out over this
                                          many library streams (0-4; <= 1:
                                          all on the caller's stream)     */
#define AEGKV_TUNE_COPY_LDS_BYTES 11 /* copy_blocks, 1024-lane shapes with
                                        >= 32 KiB items: LDS bytes reserved
                                        per workgroup (0 - 160 KiB; caps
                                        workgroups per CU; default 96 KiB) */
#define AEGKV_TUNE_SWAP_UNROLL 12    /* swap kernels: 16 B loads per lane of
                                        the 256-lane shape (1, 2 or 4;
                                        default 2)                         */
#define AEGKV_TUNE_STAGED_WORKGROUPS 13 /* STAGED gather/scatter grid (0 = one
                                           workgroup per item)             */
#define AEGKV_TUNE_STAGED_OVERLAP 14 /* STAGED over library streams: two
                                        staging chunks in flight, bit 0 for
                                        swap-out, bit 1 for swap-in
                                        (default 3)                        */
#define AEGKV_TUNE_SWAP_OUT_WORKGROUPS_UNCACHED 15 /* swap-out kernel into an
                                        uncached pool: workgroups (112)    */
/* key 16 is retired: aegkv_tune rejects it as an unknown key */
#define AEGKV_TUNE_COPY_LANES 17     /* copy_blocks with a fixed unroll (key
                                        7): 256 or 1024 lanes per workgroup
                                        (0 = 1024; 256 lanes take an unroll
                                        of 1, 2, 4 or 8)                   */
#define AEGKV_TUNE_COPY_ORDER 18     /* copy_blocks: pairs reach the kernel
                                        as given (0), sorted by target id
                                        (1, default) or by source id (2);
                                        the result does not depend on it   */

/* ABI version of the loaded library (AEGKV_ABI_VERSION). */
int aegkv_abi_version(void);

/*
 * Set-up, once per process, before the first call (optional, but needed
 * before any call made under stream capture): for every visible device,
 * with that device current, looks up the device array the allocation-free
 * copy uses (which may load the library's code object) and the device's CU
 * count, then restores the current device. Returns 0 when there is no
 * device. No counterpart in the reference.
 */
int aegkv_init(void);

/* Message for the calling thread's most recent failure ("" if none). */
const char* aegkv_last_error(void);

/* Set a tuning knob; returns the previous value (or <0 on a bad key). */
int64_t aegkv_tune(int key, int64_t value);

/*
 * Legacy whole-block swap. Replaces ops/ops.h:4-10 / ops/swap.cu:25-60
 * (`swap(source_block_ids, target_block_ids, is_swap_in, kv_cache,
 * kv_swap)`): for i < num_ids, with B = block_bytes,
 *   is_swap_in:  kv_cache[target[i]*B ..+B) <- kv_swap[source[i]*B ..+B)
 *   otherwise:   kv_swap[target[i]*B ..+B)  <- kv_cache[source[i]*B ..+B)
 * kv_cache is device memory of cache_num_blocks blocks, kv_swap a pinned
 * host pool of swap_num_blocks blocks. Unlike the reference (which checks
 * nothing and assumes 2-byte elements when deriving B, swap.cu:34), ids are
 * range-checked and duplicate targets are rejected; the caller passes B.
 */
int aegkv_swap(const int64_t* source_block_ids, const int64_t* target_block_ids,
               int64_t num_ids, int is_swap_in,
               void* kv_cache, int64_t cache_num_blocks,
               void* kv_swap, int64_t swap_num_blocks,
               int64_t block_bytes, int mode, hipStream_t stream);

/*
 * Move guards. A guard is an 8-byte aligned uint64 in mapped pinned host
 * memory (aegkv_host_alloc_flags with AEGKV_HOST_COHERENT) or device
 * memory, owned by the caller, one per stream that waits on fences.
 * aegkv_fence_wait sets it when the wait gives up (1) or when the awaited
 * word carries AEGKV_FENCE_FAILED (2); aegkv_guard_merge sets it to 2 when
 * another guard is set. The library never clears a guard. Calls that take a guard
 * read it when the stream reaches them: a guarded swap or migration then
 * moves nothing, a guarded signal or publish raises its word to
 * value | AEGKV_FENCE_FAILED. So once a wait has failed, no later move on
 * that stream reads its source and every consumer of its completion sees
 * the failure, as the reference never runs a swap before its source
 * (aegaeon/worker.py:2387) and stops the worker when the source events
 * cannot be had (:2364-2368). A STAGED swap-out that a set guard skips
 * leaves its target host pages undefined (the runtime's copies from
 * staging still run); DIRECT and swap-ins write nothing.
 */
#define AEGKV_FENCE_FAILED (1ull << 62)

/*
 * Segmented (composite-page) swap. Replaces the data-plane loop of
 * Worker.swap_blocks, aegaeon/worker.py:2265-2329, whose layout comes from
 * aegaeon/vllm_cache.py:75-101 and aegaeon/worker.py:1419-1432.
 *
 * Layout: segment s is one backing tensor viewed as
 * [device_num_blocks, segment_page_bytes[s]] bytes at segment_bases[s].
 * A host block id owns host_page_bytes bytes of host_pool (the composite
 * page times the tensor-parallel size); this rank's composite page starts
 * at host_rank_offset inside it and segment s sits at
 * segment_host_offsets[s] inside that.
 *
 * Entry e = (source_block_ids[e], target_block_ids[e], group_ids[e],
 * first_kernel_blocks[e], valid_kernel_blocks[e]). For every segment s
 * owned by group g = group_ids[e] (bit g of segment_owner_masks[s]):
 *   unit = segment_page_bytes[s] / group_kernel_blocks_per_page[g]
 *   off  = unit * first, len = unit * valid   (cache_transfer.py:138-165)
 *   host = host_pool + host_id*host_page_bytes + host_rank_offset
 *          + segment_host_offsets[s] + off
 *   dev  = segment_bases[s] + dev_id*segment_page_bytes[s] + off
 *   is_swap_in: dev[0,len) <- host[0,len)  (host_id = source, dev_id = target)
 *   otherwise:  host[0,len) <- dev[0,len)  (dev_id = source, host_id = target)
 * Entries with len == 0 and segments not owned by g move nothing.
 * guard: null, or a move guard (see above); when it is set by the time the
 * stream reaches the call, nothing moves.
 */
int aegkv_swap_blocks(int32_t num_segments, void* const* segment_bases,
                      const int64_t* segment_page_bytes,
                      const int64_t* segment_host_offsets,
                      const uint64_t* segment_owner_masks,
                      int64_t device_num_blocks,
                      int32_t num_groups,
                      const int64_t* group_kernel_blocks_per_page,
                      void* host_pool, int64_t host_num_blocks,
                      int64_t host_page_bytes, int64_t host_rank_offset,
                      int64_t num_entries,
                      const int64_t* source_block_ids,
                      const int64_t* target_block_ids,
                      const int32_t* group_ids,
                      const int64_t* first_kernel_blocks,
                      const int64_t* valid_kernel_blocks,
                      int is_swap_in, int mode, const uint64_t* guard, hipStream_t stream);

/*
 * In-HBM block copy / compaction: for every segment s and pair i,
 *   seg_s[dst[i]] := seg_s[src[i]]   (one whole block of segment_page_bytes[s]).
 * The reference has no KV copy_blocks (block_manager.py:1392-1393); its
 * in-HBM compactions are aegaeon/allocator.py:101-137 (relocate_tensors),
 * aegaeon/graph_bindings.py:60-92 and aegaeon/loader/allocator.py:288-321.
 * Targets must be distinct and disjoint from the sources (AEGKV_EDUP /
 * AEGKV_EOVERLAP otherwise), which makes the result independent of order.
 */
int aegkv_copy_blocks(int32_t num_segments, void* const* segment_bases,
                      const int64_t* segment_page_bytes,
                      int64_t device_num_blocks, int64_t num_pairs,
                      const int64_t* src_block_ids,
                      const int64_t* dst_block_ids, hipStream_t stream);

/*
 * aegkv_copy_blocks without allocating: same arguments, same checks, same
 * kernels and the same result. No counterpart in the reference; it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). The call allocates nothing on
 * the host or the device: the descriptor goes to a fixed device array of
 * 1,081,344 bytes that each GPU the library runs on holds until the process
 * ends, written there by small fill kernels whose arguments carry the
 * descriptor (2 KiB per launch; 4096 pairs over 80 segments take 34
 * launches). A graph that captures the call therefore replays the
 * descriptor it captured, whatever calls ran since. The launches cost host
 * time: measured 0.48 ms per call for 4096 pairs over 80 segments and
 * 7.0 ms for 65536 pairs, against 0.10-0.11 ms for aegkv_copy_blocks; the
 * same for up to a few hundred pairs. Limits: at most 1024
 * segments and 65536 pairs per call (AEGKV_ENOMEM beyond, nothing
 * enqueued). Every call on a device shares that device's array, which keeps
 * the last call's descriptor; nothing in it has to start at zero, since each
 * call writes the whole descriptor it reads. Calls that overlap on one
 * device (from other streams or threads, or a graph replayed beside other
 * calls) race and must be ordered by the caller; calls on one stream are
 * ordered by the stream.
 */
int aegkv_copy_blocks_noalloc(int32_t num_segments, void* const* segment_bases,
                              const int64_t* segment_page_bytes, int64_t device_num_blocks,
                              int64_t num_pairs, const int64_t* src_block_ids,
                              const int64_t* dst_block_ids, hipStream_t stream);

/*
 * Measurement only (no counterpart in the reference): the read half or the
 * write half of aegkv_copy_blocks on its own. Same arguments, checks, work
 * items, grid and launch shape as aegkv_copy_blocks; AEGKV_PROBE_READ loads
 * every source tile (the loads are folded and the fold is stored to *sink
 * only if it equals `magic`), AEGKV_PROBE_WRITE stores a fixed pattern into
 * every target tile (their previous contents are lost) and reads nothing.
 * Their rates bound what a copy over the same tiles can reach: a copy of B
 * bytes each way takes at least B/read_rate + B/write_rate. Tiles must be
 * 16 B aligned multiples of 16 B. sink: a 4-byte aligned device word.
 */
#define AEGKV_PROBE_READ 1
#define AEGKV_PROBE_WRITE 2
int aegkv_copy_probe(int kind, int32_t num_segments, void* const* segment_bases,
                     const int64_t* segment_page_bytes, int64_t device_num_blocks,
                     int64_t num_pairs, const int64_t* src_block_ids,
                     const int64_t* dst_block_ids, uint32_t* sink, uint32_t magic,
                     hipStream_t stream);

/*
 * Block migration between two caches of the same layout: for every segment
 * s and pair i,
 *   dst_seg_s[dst[i]] := src_seg_s[src[i]]   (one whole block).
 * The reference declares migration but leaves it unimplemented:
 * BlockManager._migrate_requests (aegaeon/block_manager.py:1527-1601) and
 * Worker.migrate_blocks / migrate_blocks_source / register_kvcache_mem_handles
 * (aegaeon/worker.py:2420-2445) raise NotImplementedError; their plan is
 * that the target engine's worker copies whole blocks out of the source
 * engine's cache, opened through IPC memory handles. Here the source
 * segments may be any device memory the current device can read: another
 * cache on this GPU, memory opened with hipIpcOpenMemHandle, or a peer
 * GPU's memory over xGMI once peer access is enabled. Targets must be
 * distinct (AEGKV_EDUP); the two caches must not overlap (AEGKV_EOVERLAP;
 * use aegkv_copy_blocks within one cache). Same kernel and launch shape as
 * aegkv_copy_blocks. guard: null, or a move guard; when it is set by the
 * time the stream reaches the call, nothing moves.
 */
int aegkv_migrate_blocks(int32_t num_segments, void* const* src_segment_bases,
                         void* const* dst_segment_bases, const int64_t* segment_page_bytes,
                         int64_t src_num_blocks, int64_t dst_num_blocks, int64_t num_pairs,
                         const int64_t* src_block_ids, const int64_t* dst_block_ids,
                         const uint64_t* guard, hipStream_t stream);

/*
 * Weight load on a model switch: num_slices contiguous slices, pinned host
 * -> device, dst[i][0, bytes[i]) <- src[i][0, bytes[i]), in one call.
 * Replaces QuickLoader.load_tensors_content's one
 * `slice_storage.copy_(tensors_content.tensors_storage, non_blocking=True)`
 * per tensors content (aegaeon/loader/quick_loader.py:325-340), looped over
 * a model's sharding contents by load_model_to_tensors (:297-323) inside
 * Worker.switch (aegaeon/worker.py:455-551). mode DIRECT (and AUTO when it
 * resolves to DIRECT for swap-in): one kernel reads the pinned host memory
 * over PCIe (16 B per lane when every pointer and size is a 16 B multiple);
 * mode STAGED: one hipMemcpyAsync per slice, the runtime's DMA copy. Target
 * slices must not overlap (AEGKV_EOVERLAP); sources must be pinned host
 * memory and targets device memory; empty slices are skipped.
 */
int aegkv_load_slices(int64_t num_slices, void* const* dst, const void* const* src,
                      const int64_t* bytes, int mode, hipStream_t stream);

/*
 * Transfer entries of many block tables in one call (host-only; no GPU).
 * Native form of BlockTable.transfer_entries (aegaeon/block_manager.py:
 * 446-478) over CacheGroupConfig.num_skipped_blocks / kernel_block_extent
 * (:196-266) and kernel_block_extent_for_attention_page
 * (aegaeon/cache_transfer.py:48-94).
 *
 * Cache groups g < num_groups: group_kind[g] (0 = attention, 1 = mamba_none
 * state page), group_block_size[g] and group_kernel_block_size[g] in tokens,
 * group_sliding_window[g] (<= 0: no window). Table t < num_tables has
 * processed_tokens[t] committed tokens; its group-g columns are
 * column_ids[column_offsets[t*num_groups+g] .. column_offsets[t*num_groups+g+1]),
 * -1 marking a released column. For every retained column (not released,
 * not wholly before the group's window) one row is written, in table, group,
 * column order: out_table, out_group, out_column, out_block (the column's
 * block id), out_first / out_count (the live kernel-block extent; a state
 * page is (0, 1)). Any out_* pointer may be null. *num_rows receives the
 * row count; AEGKV_ENOMEM if it would exceed max_rows.
 */
int aegkv_transfer_entries(int32_t num_groups, const int32_t* group_kind,
                           const int64_t* group_block_size,
                           const int64_t* group_kernel_block_size,
                           const int64_t* group_sliding_window, int64_t num_tables,
                           const int64_t* processed_tokens, const int64_t* column_offsets,
                           const int64_t* column_ids, int64_t max_rows, int64_t* out_table,
                           int32_t* out_group, int64_t* out_column, int64_t* out_block,
                           int64_t* out_first, int64_t* out_count, int64_t* num_rows);

/*
 * A stream on a hardware queue of its own, for the swap-in and swap-out
 * streams the reference creates with torch.cuda.Stream()
 * (aegaeon/worker.py:278-280). Plain HIP streams share the process's
 * GPU_MAX_HW_QUEUES (4) hardware queues, and work on two streams that
 * share a queue runs one after the other, so a swap-out and a swap-in
 * can lose their overlap; a stream created with a CU mask gets a queue to
 * itself (the mask here enables every CU). Default priority. It is a
 * blocking stream: it synchronizes with the legacy default (null) stream.
 * aegkv_stream_destroy waits for the stream's queued work, drops every event
 * the library recorded on it, then destroys it.
 *
 * aegkv_stream_release(stream): wait for the stream's queued work and drop
 * every event the library recorded on it (descriptor-ring and STAGED fork
 * events). Call it before destroying, by any other means, a stream that
 * library calls ran on; the library then never queries, waits on or
 * re-records an event whose stream is gone. The stream stays usable.
 */
int aegkv_stream_create(hipStream_t* stream);
int aegkv_stream_destroy(hipStream_t stream);
int aegkv_stream_release(hipStream_t stream);

/*
 * The same, on a subset of the CUs: bit i of cu_mask (mask_words 32-bit
 * words) enables CU i. Kernels launched on the stream run only there, so
 * link-bound swap waves can be kept off the CUs that HBM-bound work (block
 * copies, the model's kernels) uses on other streams. No counterpart in the
 * reference. The runtime accepts runs of 8 or more consecutive mask bits
 * that start at a multiple of 8 and refuses finer masks with a positive
 * hipError_t status; it spreads each run of 8 bits over the 8 XCDs, one CU
 * on each (measured from the hardware ids workgroups read), so a mask sets
 * how many CUs of every XCD a stream gets, not which XCDs.
 */
int aegkv_stream_create_masked(hipStream_t* stream, const uint32_t* cu_mask,
                               int32_t mask_words);

/*
 * Pinned host pool. Replaces the pinning half of the reference's host KV
 * pool set-up: Controller._init_cpu_cache (aegaeon/llm.py:1020-1040) and
 * the worker's cudaHostRegister of that mapping (aegaeon/worker.py:251-273).
 * Allocates with hipHostMalloc (mapped + portable, so kernels on every
 * device may access it). The pool is not zero-filled.
 */
int aegkv_host_alloc(void** ptr, int64_t bytes);

/*
 * As aegkv_host_alloc, with flags. AEGKV_HOST_UNCACHED allocates the pool
 * from the uncached (MTYPE UC) fine-grained system pool
 * (hipHostMallocUncached): kernel loads and stores to it bypass the GPU L2.
 * Measured on MI355X with the swap kernels: swap-out 56.6 -> 57.0 GB/s,
 * both directions at once 87 -> 90 GB/s; a blit hipMemcpyAsync is
 * unchanged. Uncached memory is never returned to the runtime before the
 * process ends: uncached pools are carved out of uncached blocks the
 * library keeps, aegkv_host_free returns a pool's range to a free list
 * (merged with free neighbours), and a later uncached pool takes the
 * smallest free range that fits before a new block is allocated. A process
 * whose pools come and go in different sizes therefore pins no more than
 * its largest set of live pools at once, which keeps it under the host's
 * cap on pinned memory. Meant for long-lived pools such as a KV host pool.
 * AEGKV_HOST_COHERENT allocates fine-grained coherent memory
 * (hipHostMallocCoherent), for words both the GPU and the host write and
 * read while kernels run, such as move guards. The two flags do not
 * combine (AEGKV_EINVAL: hipHostMalloc refuses the pair, and uncached
 * memory is coherent already).
 */
#define AEGKV_HOST_UNCACHED 1
#define AEGKV_HOST_COHERENT 2
int aegkv_host_alloc_flags(void** ptr, int64_t bytes, int flags);
/* Release a pool from aegkv_host_alloc(_flags); null is a no-op, any other
 * pointer that is not a live pool (freed twice, or not from this library)
 * is rejected with AEGKV_EINVAL. */
int aegkv_host_free(void* ptr);

/* Pinned memory this library holds, for callers that budget against the
 * host's cap: *pinned_bytes = live cached pools + every uncached block kept
 * (live or free), *uncached_free_bytes = the free part of those blocks.
 * Either pointer may be null. Host-only. No counterpart in the reference. */
int aegkv_host_usage(int64_t* pinned_bytes, int64_t* uncached_free_bytes);

/*
 * Fences: ordering a stream after work enqueued on another stream, in this
 * process or another one, without interprocess events. Replaces the
 * reference's event chaining between workers: the producer records an
 * interprocess CUDA event behind its swap and returns the handle
 * (aegaeon/worker.py:2331,2349); the consumer opens it and makes its stream
 * wait (aegaeon/worker.py:2351-2394 via aegaeon/utils.py:263-288 and
 * aegaeon/cuda_wrapper.py:43-233). The HIP runtime here refuses to record
 * interprocess events, so the same contract is kept with counters.
 *
 * A fence word is an 8-byte aligned uint64 in device memory (possibly opened
 * from another process's IPC memory handle) or in mapped pinned host memory.
 *
 * aegkv_fence_signal: once every operation enqueued on `stream` before it
 * has finished, raise *word to at least `value` (atomic max, release at
 * system scope; 0 < value < 2^62). Give each producing stream its own word
 * and signal increasing values. With a guard (may be null) that is set by
 * then, the word is raised to value | AEGKV_FENCE_FAILED instead.
 *
 * aegkv_fence_wait: every operation enqueued on `stream` after this call
 * runs after *word has reached `value` (acquire at system scope). The wait
 * gives up after `timeout_us` microseconds (0 < timeout_us <= 600 s) of
 * polling and then sets the move guard *guard to 1; a word that carries
 * AEGKV_FENCE_FAILED ends the wait at once and sets *guard to 2. Either way
 * the stream continues, and guarded calls after the wait move nothing and
 * mark their completion failed (see "Move guards"). A waiting fence
 * holds its stream's hardware queue: the signal it waits for must come from
 * another process or from a stream on a hardware queue of its own
 * (aegkv_stream_create), never from a stream that may share the waiting
 * stream's queue (plain streams share the process's few queues), or it
 * runs only after the wait has timed out.
 */
int aegkv_fence_signal(uint64_t* word, uint64_t value, const uint64_t* guard,
                       hipStream_t stream);
int aegkv_fence_wait(const uint64_t* word, uint64_t value, int64_t timeout_us,
                     uint64_t* guard, hipStream_t stream);

/*
 * Once the stream reaches it, set *guard to 2 (a source failed) when
 * *source_guard is non-zero (one single-lane kernel). For a consumer that orders its
 * stream after a producer's completion event rather than a fence word: the
 * producer's failure then stops the consumer's guarded moves too. Both are
 * move guards. No counterpart in the reference (its event waits carry no
 * failure).
 */
int aegkv_guard_merge(uint64_t* guard, const uint64_t* source_guard, hipStream_t stream);

/*
 * Host-side fence completion, for a controller that polls moves on the CPU
 * before it frees their source blocks. Replaces the controller half of the
 * reference's event chaining: BlockManager._reclaim_blocks rebuilds the
 * workers' interprocess events and polls cudaEventQuery
 * (aegaeon/block_manager.py:804-851, handles from aegaeon/utils.py:263-288).
 *
 * A host fence word is an 8-byte aligned uint64 in host memory; to be read
 * by other processes it lives in a mapping they share (a /dev/shm file).
 *
 * aegkv_fence_publish: once every operation enqueued on `stream` before it
 * has finished, raise *host_word to at least `value` (0 < value < 2^62;
 * atomic max, release). It is a host function on the stream (hipLaunchHostFunc):
 * the stream is held by the runtime, no wave waits on a CU. The mapping must
 * stay valid until the stream has passed it. With a guard (null, or a move
 * guard in pinned host memory, which the host function reads) that is set
 * by then, the word is raised to value | AEGKV_FENCE_FAILED instead.
 *
 * aegkv_fence_host_wait: on the calling thread, wait until *host_word >=
 * value (acquire), for at most timeout_us microseconds (0: look once;
 * at most 600 s). Returns 1 once reached, 2 as soon as the word carries
 * AEGKV_FENCE_FAILED (the move, or one before it on the same stream,
 * failed), 0 if neither within the time, a negative status on a bad
 * argument. No HIP call.
 */
int aegkv_fence_publish(uint64_t* host_word, uint64_t value, const uint64_t* guard,
                        hipStream_t stream);
int aegkv_fence_host_wait(const uint64_t* host_word, uint64_t value, int64_t timeout_us);

#ifdef __cplusplus
}
#endif

#endif /* AEGKV_H */

/*
 * pbe_handoff.h -- C ABI of the MI355X prefill->decode KV handoff.
 *
 * Plain C: pointers, sizes and status codes; no exceptions cross this
 * boundary and no framework types appear in the signatures. Every call returns
 * PBE_OK (0) on success, a positive code for "not yet", or a negative error;
 * pbe_last_error() gives the calling thread's last message.
 *
 * Terms (they follow the reference's shared-KV arena):
 *   half   one layer's K or V plane of one page: page_tokens*kv_heads*head_dim*elem
 *          bytes (shared_kv_arena.h:35-36, block_allocator.cpp:369-372).
 *   page   all layers' K and V of page_tokens tokens, [layer][K|V][tok][head][dim],
 *          2*layers*half bytes.
 *   block id  byte offset / half; page ids are multiples of 2*layers
 *          (split_pd_engine.cpp:76, shared_kv_arena.cpp:128,224-229).
 *   run    maximal stretch of pages whose source and destination ids both
 *          advance by one page (split_pd_engine.cpp:96-101).
 *
 * Threading: the arena, event and run-list objects may be used from any thread
 * but not concurrently on the same object; launches go to the caller's stream.
 * Lifetime: a run list holds resolved device addresses of the arena views it
 * was built for; destroy it before unmapping those views.
 */
#ifndef PBE_HANDOFF_H_
#define PBE_HANDOFF_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PBE_OK 0
#define PBE_NOT_READY 1          /* event/copy still in flight */
#define PBE_ERR_INVALID (-1)     /* rejected before any device work was queued */
#define PBE_ERR_HIP (-2)         /* a HIP call failed; see pbe_last_error() */
#define PBE_ERR_UNKNOWN (-3)     /* completion unknown: retain every resource */
#define PBE_ERR_NOMEM (-4)
#define PBE_ERR_UNSUPPORTED (-5)
#define PBE_ERR_BUSY (-6)        /* a shared resource is in use by queued work on another stream */

#define PBE_MAX_SEGMENTS 16
#define PBE_IPC_HANDLE_BYTES 64

/* Last error message of the calling thread ("" if none). */
const char* pbe_last_error(void);
/* Library version string, e.g. "pbe-handoff 1.0 gfx950". */
const char* pbe_version(void);

/* KV page geometry. elem_bytes is 2 for BF16 pools, 1 for FP8 payload pools. */
typedef struct pbe_kv_shape {
  int32_t layers;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t page_tokens;
} pbe_kv_shape;

/* One coalesced run: `pages` whole pages from src_block to dst_block. */
typedef struct pbe_run {
  int32_t src_block;
  int32_t dst_block;
  int32_t pages;
} pbe_run;

/* A process-local mapping of a (possibly segmented) arena. Byte offset o lies
 * in segment o / segment_bytes at base[seg] + o % segment_bytes. A single
 * allocation is nseg = 1, segment_bytes = bytes. Callers may fill this for
 * memory they own; pbe_arena_view() fills it for arenas made here. */
typedef struct pbe_arena_view {
  uint64_t bytes;
  uint64_t segment_bytes;
  uint32_t nseg;
  uint32_t reserved;
  void* base[PBE_MAX_SEGMENTS];
} pbe_arena_view;

/* ---- arena: owner allocation + IPC export/import ------------------------
 * Replaces run_shared_kv_owner's cudaMalloc/cudaIpcGetMemHandle
 * (shared_kv_owner.cpp:25,28) and SharedKVArenaClient's cudaIpcOpenMemHandle
 * (shared_kv_client.cpp:81). The arena is split into segments of at most
 * segment_bytes (a multiple of the page size chosen by the caller), each its
 * own hipMalloc, so every exported allocation stays below 2 GiB. */
typedef struct pbe_arena pbe_arena;

typedef struct pbe_arena_ipc {
  uint32_t version;
  uint32_t nseg;
  uint64_t bytes;
  uint64_t segment_bytes;
  uint64_t epoch;
  uint8_t gpu_uuid[16];
  uint8_t handles[PBE_MAX_SEGMENTS][PBE_IPC_HANDLE_BYTES];
} pbe_arena_ipc;

int pbe_arena_create(int device, uint64_t bytes, uint64_t segment_bytes, uint64_t epoch,
                     pbe_arena** out);
int pbe_arena_export(const pbe_arena* arena, pbe_arena_ipc* out);
/* Opens every segment in this process; fails if the exporter's GPU UUID differs
 * (shared_kv_client.cpp:72-73 checks the same). */
int pbe_arena_import(const pbe_arena_ipc* ipc, int device, pbe_arena** out);
int pbe_arena_get_view(const pbe_arena* arena, pbe_arena_view* out);
uint64_t pbe_arena_epoch(const pbe_arena* arena);
int pbe_arena_destroy(pbe_arena* arena);

/* ---- completion events ------------------------------------------------
 * In-process fences (interprocess = 0): record on one stream, wait on another
 * or query/synchronize from the host.
 * interprocess = 1 asks for a hipEventInterprocess event whose handle crosses
 * processes (the pattern of demo/cuda_ipc_event_probe.cu:24-27,70-75). The
 * HIP runtime of ROCm 7.2 creates such events but rejects hipEventRecord on
 * them, so they cannot carry a completion: pbe_event_create(.., 1, ..) and
 * pbe_event_import probe the runtime once per device and return
 * PBE_ERR_UNSUPPORTED when recording fails. Cross-process completion uses
 * pbe_signal_* below. pbe_event_export of an in-process event is
 * PBE_ERR_INVALID. */
typedef struct pbe_event pbe_event;
int pbe_event_create(int device, int interprocess, pbe_event** out);
int pbe_event_export(const pbe_event* event, uint8_t out[PBE_IPC_HANDLE_BYTES]);
int pbe_event_import(const uint8_t handle[PBE_IPC_HANDLE_BYTES], int device, pbe_event** out);
int pbe_event_record(pbe_event* event, void* stream);
int pbe_event_wait(pbe_event* event, void* stream); /* stream waits, host does not */
int pbe_event_query(pbe_event* event);              /* PBE_OK or PBE_NOT_READY */
int pbe_event_synchronize(pbe_event* event);
int pbe_event_destroy(pbe_event* event);

/* ---- IPC completion signals ------------------------------------------
 * Cross-process ordering without host round trips. A signal is a 64-bit
 * sequence word in its own small device allocation, exported with
 * hipIpcGetMemHandle. set() is a stream-ordered write (hipStreamWriteValue64)
 * that follows all earlier work on the stream; wait() makes a stream wait on
 * the GPU (hipStreamWaitValue64, >=) until the word reaches a value. This is the
 * completion protocol of the handoff: P sets "KV written" = n after its prefill
 * kernels, D's stream waits for n before the copy and then sets "copy done" = n,
 * which P waits for before retiring its pages (pattern of
 * demo/cuda_ipc_event_probe.cu:24-27,70-75 and data/ipc_pool.h:24-26). On
 * ROCm 7.2 hipEventRecord rejects hipEventInterprocess events, so interprocess
 * pbe_event objects cannot be recorded there; signals are the portable form. */
typedef struct pbe_signal pbe_signal;
int pbe_signal_create(int device, pbe_signal** out); /* starts at 0 */
int pbe_signal_export(const pbe_signal* signal, uint8_t out[PBE_IPC_HANDLE_BYTES]);
int pbe_signal_import(const uint8_t handle[PBE_IPC_HANDLE_BYTES], int device, pbe_signal** out);
int pbe_signal_set(pbe_signal* signal, uint64_t value, void* stream);
int pbe_signal_wait(pbe_signal* signal, uint64_t value, void* stream);
int pbe_signal_read(pbe_signal* signal, uint64_t* value); /* current value, host side */
int pbe_signal_destroy(pbe_signal* signal);

/* ---- host-side plan ----------------------------------------------------
 * Source id checks of copy_shared_kv (split_pd_engine.cpp:70-77): id >= 0,
 * id % (2*layers) == 0 and (id + 2*layers)*half <= arena bytes. On failure
 * *bad_index is the first offending position. */
int pbe_validate_ids(const int32_t* ids, int64_t n, const pbe_kv_shape* shape,
                     uint32_t elem_bytes, uint64_t arena_bytes, int64_t* bad_index);

/* Coalesce page-major id lists into runs (split_pd_engine.cpp:96-101). A run
 * additionally breaks where either side would cross a segment boundary
 * (segment_bytes 0 = unsegmented). `out` holds n entries. */
int pbe_build_runs(const int32_t* src_ids, const int32_t* dst_ids, int64_t n,
                   const pbe_kv_shape* shape, uint32_t elem_bytes, uint64_t segment_bytes,
                   pbe_run* out, int64_t* n_runs);

/* ---- compact page-list wire form ---------------------------------------
 * The prefill result names its KV pages once per layer as JSON integer arrays
 * (RemotePrefillResult.layers[l].src_block_ids, serving_zmq_rpc.h:80-98,
 * written by remote_prefill_result_to_json, serving_zmq_rpc.cpp:222-253);
 * copy_shared_kv then requires all of them to be identical
 * (split_pd_engine.cpp:78-79). The compact form carries the page-major list
 * once, as spans of consecutive page ids (next id = id + 2*layers), in
 * little-endian binary:
 *   pbe_page_list_header (32 bytes), then n_spans x {int32 first_block, int32 pages}.
 * `checksum` is FNV-1a (32-bit) over the header with checksum = 0 followed by
 * the spans, so any single changed byte is rejected. */
#define PBE_PAGE_LIST_MAGIC 0x50454250u /* bytes "PBEP" */
#define PBE_PAGE_LIST_VERSION 1u

typedef struct pbe_page_list_header {
  uint32_t magic;
  uint16_t version;
  uint16_t header_bytes; /* 32 */
  int32_t layers;
  int32_t n_pages;
  int32_t n_spans;
  uint32_t checksum;
  uint64_t epoch; /* shared_arena_epoch of the prefill result */
} pbe_page_list_header;

/* Bytes the encoding of `ids` takes (header + spans); 0 if ids are invalid
 * (negative, not a multiple of 2*layers, or n outside [0, INT32_MAX]). */
uint64_t pbe_page_list_bytes(const int32_t* ids, int64_t n, int32_t layers);

/* Encodes page-major block ids (each >= 0 and a multiple of 2*layers, in the
 * prefill's page order) into `out` (capacity `cap`). *out_bytes = bytes
 * written. PBE_ERR_INVALID on bad ids or too small a buffer (nothing written). */
int pbe_page_list_encode(const int32_t* ids, int64_t n, int32_t layers, uint64_t epoch, void* out,
                         uint64_t cap, uint64_t* out_bytes);

/* Checks and decodes a page list. Pass ids = NULL to read only the header
 * (*n_pages, *layers, *epoch). Otherwise `ids` holds `cap` entries and
 * receives n_pages ids. Rejects a wrong magic, version or size, a checksum
 * mismatch, spans with no pages, ids that are negative, not multiples of
 * 2*layers or beyond INT32_MAX, and span totals that differ from n_pages. */
int pbe_page_list_decode(const void* data, uint64_t bytes, int32_t* ids, int64_t cap,
                         int64_t* n_pages, int32_t* layers, uint64_t* epoch);

/* ---- device-resident run lists ----------------------------------------
 * Validated on the host (every run inside one segment of its view, no source
 * range overlapping a destination range), resolved to device addresses and
 * uploaded once; a list is reusable for any number of launches. */
typedef struct pbe_runlist pbe_runlist;

typedef struct pbe_runlist_info {
  int64_t runs;
  int64_t pages;
  uint64_t src_bytes;    /* bytes read per launch */
  uint64_t dst_bytes;    /* payload bytes written per launch */
  uint64_t scale_bytes;  /* scale bytes written per launch (FP8 per-token-head) */
  uint64_t slices;       /* work units of the launch */
} pbe_runlist_info;

/* BF16 (or any-dtype) identity copy inside/between arena views. The list
 * replaces the reference's one cudaMemcpyAsync per run (split_pd_engine.cpp:104). */
int pbe_runlist_create(const pbe_arena_view* src, const pbe_arena_view* dst,
                       const pbe_run* runs, int64_t n_runs, const pbe_kv_shape* shape,
                       uint32_t elem_bytes, int device, pbe_runlist** out);

#define PBE_FP8_SCALE_PER_TOKEN_HEAD 0 /* amax per (token, head) row, scales written */
#define PBE_FP8_SCALE_TABLE 1          /* static amax per (layer, K|V, head) */

/* Fused BF16 -> FP8 E4M3 handoff. src ids are in BF16 half units, dst ids in
 * FP8 half units (half/2). In per-token-head mode, dst_scales is the base of a
 * page-major scale pool of 2*layers*page_tokens*kv_heads fp32 per page, page
 * index = dst_block / (2*layers); it may be NULL in table mode. */
int pbe_runlist_create_fp8(const pbe_arena_view* src, const pbe_arena_view* dst,
                           void* dst_scales, uint64_t dst_scales_bytes, const pbe_run* runs,
                           int64_t n_runs, const pbe_kv_shape* shape, int device,
                           pbe_runlist** out);
int pbe_runlist_get_info(const pbe_runlist* list, pbe_runlist_info* out);
int pbe_runlist_destroy(pbe_runlist* list);

/* ---- launches (asynchronous on `stream`, a hipStream_t; NULL = default) ----
 * One kernel for every layer's K and V of every page in the list. */
int pbe_handoff_copy(const pbe_runlist* list, void* stream);
/* scale_mode PBE_FP8_SCALE_*; amax_table (device, 2*layers*kv_heads fp32,
 * index (2*layer+kv)*kv_heads+head) is read only in table mode. */
int pbe_handoff_copy_fp8(const pbe_runlist* list, int scale_mode, const float* amax_table,
                         void* stream);

/* The same launches with two caller-created hipEvent_t (timing enabled) that
 * the runtime stamps at the kernel's own start and end (hipExtLaunchKernel),
 * so hipEventElapsedTime(start, stop) is the kernel's duration. For per-
 * handoff GPU-time accounting; no counterpart in the reference. */
int pbe_handoff_copy_timed(const pbe_runlist* list, void* stream, void* start_event,
                           void* stop_event);
int pbe_handoff_copy_fp8_timed(const pbe_runlist* list, int scale_mode, const float* amax_table,
                               void* stream, void* start_event, void* stop_event);

/* ---- one-call form of copy_shared_kv's data path -----------------------
 * Validates ids against the arena (as split_pd_engine.cpp:70-77), coalesces,
 * builds a run list, launches one copy and returns the copied bytes in
 * *copied (the reference's return value, split_pd_engine.cpp:107,114). The
 * run list travels in the kernel arguments when the sources form one region
 * and it has at most 256 runs, or when it has at most 112 runs: no staging
 * copy, so such calls can be captured into a HIP graph. Longer lists go
 * through the library's staging ring (released after the launch completes on
 * `stream`); those calls refuse a capturing stream with
 * PBE_ERR_UNSUPPORTED. The call does not wait for the copy. */
int pbe_copy_shared_kv(const pbe_arena_view* arena, const int32_t* src_ids,
                       const int32_t* dst_ids, int64_t n, const pbe_kv_shape* shape,
                       int device, void* stream, uint64_t* copied);

/* ---- generic component-list copy ---------------------------------------
 * Executes an arbitrary list of (src, dst, bytes) device copies in one launch:
 * the device form of ExecuteCpuTransfer (transfer_plan.cpp:392-403) used by
 * the HIP TransferBackend. Every endpoint must be device memory of `device` or
 * pinned host memory (checked on the host); ops whose addresses and size are
 * 16-byte multiples move as 16-byte vectors, others byte by byte. No two ops
 * may write the same byte or write another op's source. The list is staged
 * into device memory owned by the library. */
typedef struct pbe_copy_op {
  uint64_t src;
  uint64_t dst;
  uint64_t bytes;
} pbe_copy_op;
int pbe_copy_ops(const pbe_copy_op* ops, int64_t n_ops, int device, void* stream);

/* ---- decode-side reader -------------------------------------------------
 * Split-K paged attention for one query token per sequence over handed-off
 * pages: the MI355X form of splitkv_batched_paged_mha_fp8_decode_cu and
 * splitkv_batched_paged_mha_fast_decode_cu (paged_mha_fast_kernel.cu:902-1076,
 * called from CudaPagedKVRuntime::decode, paged_kv_runtime.cpp:293-357), with
 * the same arithmetic: score = (q . k) * log2(e)/sqrt(head_dim) * k_scale,
 * base-2 online softmax, acc += v * (p * v_scale), output = acc / sum in BF16.
 *
 * Pages are page-major in `kv` (block id = byte offset / half, page ids are
 * multiples of 2*layers): PBE_KV_BF16 planes of 16*H*D bf16, or
 * PBE_KV_FP8_E4M3 planes of 16*H*D bytes with a page-major scale pool
 * [layer][K|V][token][head] fp32 (what pbe_handoff_copy_fp8 writes in
 * per-token-head mode). head_dim 64 or 128, page_tokens 16, q_heads a multiple
 * of kv_heads with at most 8 query heads per KV head.
 *
 * queries / outputs: bf16 [batch][q_heads][head_dim], 16-byte aligned.
 * block_tables: int32 [batch][max_blocks_per_seq]; seq_lens: int32 [batch]
 * (device memory, read by the kernel). A sequence whose table holds an id
 * outside the arena or not a page id, or whose length needs more than
 * max_blocks_per_seq blocks, gets NaN outputs (its pages are not read past
 * the failing id). splits = 0 picks pbe_paged_decode_splits(); at most 1024.
 * workspace: at least pbe_paged_decode_workspace_bytes() bytes of device
 * memory, used by this launch until it completes. Asynchronous on `stream`. */
#define PBE_KV_BF16 0
#define PBE_KV_FP8_E4M3 1
/* Split count for a decode launch on the current GPU (its CU count sets the
 * wave budget): kv_dtype as for pbe_paged_decode (FP8 pages run two waves per
 * SIMD while every split keeps at least 8 blocks, BF16 pages one; at least 4
 * blocks per split). max_blocks_per_seq here should be the block count of
 * the longest live sequence, not the block-table capacity: a table sized for
 * the maximum context would pick splits too short to keep the reader busy.
 * Size the workspace with the result. */
int32_t pbe_paged_decode_splits(int32_t batch, int32_t kv_heads, int32_t max_blocks_per_seq,
                                int32_t kv_dtype);
uint64_t pbe_paged_decode_workspace_bytes(int32_t batch, int32_t q_heads, int32_t head_dim,
                                          int32_t splits);
int pbe_paged_decode(const pbe_arena_view* kv, int32_t kv_dtype, const float* scales,
                     uint64_t scale_bytes, const pbe_kv_shape* shape, int32_t layer,
                     const void* queries, void* outputs, int32_t batch, int32_t q_heads,
                     const int32_t* block_tables, const int32_t* seq_lens,
                     int32_t max_blocks_per_seq, int32_t splits, void* workspace,
                     uint64_t workspace_bytes, int device, void* stream);

/* Allocation-free form of pbe_paged_decode. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The split-K
 * partials live in a static device array of PBE_DECODE_SCRATCH_BYTES per GPU
 * (held until the process ends) instead of a caller workspace; nothing is
 * allocated and every partial is rewritten by each call, so no clearing is
 * needed. splits = 0 takes pbe_paged_decode_splits' count, lowered until the
 * partials fit the array; an explicit split count whose partials need more
 * (pbe_paged_decode_workspace_bytes) is rejected with PBE_ERR_INVALID, as is a
 * batch too large for the array even at one split. All calls on
 * one GPU share the array, so calls must not overlap in time: issue them on
 * one stream. A call on a different stream from the previous call, while that
 * call's work has not completed, is refused with PBE_ERR_BUSY before anything
 * is queued (an event recorded after each call is queried on entry; host
 * threads are serialised by a lock). Under stream capture the guard is off:
 * the caller orders the graph's replays. The first call on a GPU resolves
 * the array's address and creates the guard event; later calls allocate
 * nothing. */
#define PBE_DECODE_SCRATCH_BYTES (8u << 20)
int pbe_paged_decode_noalloc(const pbe_arena_view* kv, int32_t kv_dtype, const float* scales,
                             uint64_t scale_bytes, const pbe_kv_shape* shape, int32_t layer,
                             const void* queries, void* outputs, int32_t batch, int32_t q_heads,
                             const int32_t* block_tables, const int32_t* seq_lens,
                             int32_t max_blocks_per_seq, int32_t splits, int device, void* stream);

/* Decode over per-layer K/V pools: the calling convention of the reference's
 * decode kernels (splitkv_batched_paged_mha_fast_decode_cu /
 * splitkv_batched_paged_mha_fp8_decode_cu, paged_mha_fast_kernel.cu:902-1076,
 * as CudaPagedKVRuntime::decode passes a KVPoolView, paged_kv_runtime.cpp:293-357).
 * Block b of the layer has its 16 token rows of K at key_pool + b*half and of V
 * at value_pool + b*half (half = 16*kv_heads*head_dim*E, rows [token][head][dim]),
 * and, for FP8, its scales at key_scales + b*16*kv_heads and
 * value_scales + b*16*kv_heads ([token][head] fp32). pool_bytes and
 * scale_pool_bytes are the bytes addressable from each pointer; a block id whose
 * rows or scales would end beyond them gives its sequence NaN outputs, as a bad
 * id does in pbe_paged_decode. Local pools (ids 0..n-1, separate K and V
 * allocations) and a shared arena's layer views (key_pool = arena +
 * 2*layer*half, value_pool = key_pool + half, page-major ids) both work. Pools
 * 16-byte aligned, scale pools 4-byte aligned; everything else as
 * pbe_paged_decode. */
int pbe_paged_decode_pools(const void* key_pool, const void* value_pool, uint64_t pool_bytes,
                           const float* key_scales, const float* value_scales,
                           uint64_t scale_pool_bytes, int32_t kv_dtype, int32_t kv_heads,
                           int32_t head_dim, const void* queries, void* outputs, int32_t batch,
                           int32_t q_heads, const int32_t* block_tables, const int32_t* seq_lens,
                           int32_t max_blocks_per_seq, int32_t splits, void* workspace,
                           uint64_t workspace_bytes, int device, void* stream);
/* One decode step of a layer in one launch pair: each sequence's new token is
 * written into its page slot and then read with the rest, as
 * pbe_scatter_kv (BF16 input) followed by pbe_paged_decode_pools would do,
 * with identical page bytes, scales and outputs. The reference runs the two
 * as separate kernels (CudaPagedKVRuntime::scatter, then the decode kernels,
 * paged_kv_runtime.cpp:207-245,293-357); this form has no counterpart there.
 *   new_keys, new_values: bf16 [batch][kv_heads][head_dim] in device memory,
 *     16-byte aligned: the K and V of each sequence's token at position
 *     seq_lens[b] - 1, i.e. row (seq_lens[b]-1) % 16 of block
 *     block_tables[b][(seq_lens[b]-1) / 16] (the slot the KVCacheManager's
 *     append_slots hands out for the step's token).
 *   Pools, scales and every other argument as pbe_paged_decode_pools; the
 *   pools are written. A sequence of length 0 writes nothing and reads as
 *   zeros; one whose last block id fails the reader's checks writes nothing
 *   and reads as NaN. */
int pbe_paged_decode_append(void* key_pool, void* value_pool, uint64_t pool_bytes,
                            float* key_scales, float* value_scales, uint64_t scale_pool_bytes,
                            int32_t kv_dtype, int32_t kv_heads, int32_t head_dim, const void* new_keys,
                            const void* new_values, const void* queries, void* outputs, int32_t batch,
                            int32_t q_heads, const int32_t* block_tables, const int32_t* seq_lens,
                            int32_t max_blocks_per_seq, int32_t splits, void* workspace,
                            uint64_t workspace_bytes, int device, void* stream);
/* The same over the page-major arena and a layer, as pbe_paged_decode takes
 * them (segmented arenas included): the new token of sequence b lands at
 * row (seq_lens[b]-1) % 16 of block block_tables[b][(seq_lens[b]-1) / 16] in
 * layer `layer`'s K and V planes, and its FP8 scales in the page-major scale
 * pool. The arena's pages and the scale pool are written (the view is
 * const because the view struct itself is not changed; the memory it names
 * is). No counterpart in the reference. */
int pbe_paged_decode_append_arena(const pbe_arena_view* kv, int32_t kv_dtype, float* scales,
                                  uint64_t scale_bytes, const pbe_kv_shape* shape, int32_t layer,
                                  const void* new_keys, const void* new_values, const void* queries,
                                  void* outputs, int32_t batch, int32_t q_heads,
                                  const int32_t* block_tables, const int32_t* seq_lens,
                                  int32_t max_blocks_per_seq, int32_t splits, void* workspace,
                                  uint64_t workspace_bytes, int device, void* stream);

/* ---- page writer ---------------------------------------------------------
 * Writes n_tokens new tokens' K and V rows into their page slots: the MI355X
 * form of scatter_kv_batch_to_pages_cu and scatter_kv_batch_to_pages_fp8_e4m3_cu
 * (scatter_kv_kernel.cuh:27-57, called from CudaPagedKVRuntime::scatter,
 * paged_kv_runtime.cpp:207-245).
 *   keys, values: [n_tokens][kv_heads*head_dim] of in_dtype (PBE_IN_BF16 or
 *     PBE_IN_F32) in device memory, 16-byte aligned, rows a multiple of 16 bytes.
 *   slot_mapping: int32 [n_tokens] in device memory, slot = block * block_size
 *     + offset. Head h of token t lands at
 *     pool + block*block_size*kv_dim*E + (offset*kv_dim + h*head_dim)*E,
 *     E the bytes of one stored element. A negative slot, or one whose row or
 *     scale would end beyond the pool sizes given, writes nothing.
 *   kv_dtype PBE_KV_BF16: plain copy, the pools hold the input type (BF16 or
 *     FP32). PBE_KV_FP8_E4M3: E4M3 bytes plus one fp32 scale per (token, head)
 *     at scales[(block*block_size + offset)*kv_heads + head]; scale = amax/448,
 *     q = E4M3(x * (448/amax)) saturated, and an all-zero row stores scale 1 and
 *     zero codes (scatter_kv_kernel.cu:166-211). FP8 needs head_dim*E_in/16 to
 *     be a power of two up to 64 (BF16 head_dim 8..512, FP32 4..256).
 * Over the shared page-major arena, a layer's planes are key_pool = arena +
 * 2*layer*half and value_pool = key_pool + half, with block ids the
 * KVCacheManager's page-major ids (its build_slot_mapping gives the slots).
 * Asynchronous on `stream`; n_tokens = 0 queues nothing. */
#define PBE_IN_BF16 0
#define PBE_IN_F32 1
int pbe_scatter_kv(const void* keys, const void* values, int32_t in_dtype, int32_t n_tokens,
                   const int32_t* slot_mapping, int32_t block_size, int32_t kv_heads,
                   int32_t head_dim, int32_t kv_dtype, void* key_pool, uint64_t key_pool_bytes,
                   void* value_pool, uint64_t value_pool_bytes, float* key_scales,
                   uint64_t key_scale_bytes, float* value_scales, uint64_t value_scale_bytes,
                   int device, void* stream);
/* One token at a slot given by value: scatter_kv_to_page_cu
 * (scatter_kv_kernel.cuh:13-24) with the block and offset as host integers, the
 * same rules as pbe_scatter_kv (FP8 pools too, which the reference routes
 * through its batched FP8 form). */
int pbe_scatter_kv_to_page(const void* keys, const void* values, int32_t in_dtype,
                           int32_t physical_block_id, int32_t offset_in_block,
                           int32_t block_size, int32_t kv_heads, int32_t head_dim,
                           int32_t kv_dtype, void* key_pool, uint64_t key_pool_bytes,
                           void* value_pool, uint64_t value_pool_bytes, float* key_scales,
                           uint64_t key_scale_bytes, float* value_scales,
                           uint64_t value_scale_bytes, int device, void* stream);

/* GPU UUID of `device` (16 bytes), as compared across processes. */
int pbe_device_uuid(int device, uint8_t out[16]);
/* The calling thread's current HIP device (the one a pool built without an
 * explicit device index lives on, as the reference's CUDA allocator uses the
 * current device: block_allocator.cpp:36-38). */
int pbe_current_device(int* device);

/* ---- streams and pointer queries for C++ host code ---------------------
 * Backends above this ABI (the HIP TransferBackend, the shared-arena
 * connector) own their streams through these calls instead of calling HIP. */
int pbe_stream_create(int device, void** out);              /* non-blocking, default priority */
int pbe_stream_destroy(int device, void* stream);
int pbe_stream_synchronize(int device, void* stream);       /* PBE_OK or PBE_ERR_UNKNOWN */
/* Makes `stream` wait for a caller-owned hipEvent_t (borrowed, not retained). */
int pbe_stream_wait_raw_event(int device, void* stream, void* hip_event);

#define PBE_PTR_UNKNOWN 0   /* pageable host or not an allocation: kernels must not touch it */
#define PBE_PTR_DEVICE 1    /* device memory; *device_out holds its GPU */
#define PBE_PTR_PINNED_HOST 2
/* Classifies [ptr, ptr+bytes): the whole span must lie in one allocation. */
int pbe_pointer_kind(const void* ptr, uint64_t bytes, int* kind, int* device_out);

#ifdef __cplusplus
}
#endif
#endif /* PBE_HANDOFF_H_ */

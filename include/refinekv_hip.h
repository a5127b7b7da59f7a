/*
 * refinekv_hip.h -- C ABI of librefinekv_hip.so, RefineKV's decode-time
 * attention path on AMD Instinct MI355X (gfx950).
 *
 * Conventions for every entry point:
 *  - Pointers are device pointers unless stated otherwise; strides are in
 *    elements; head_dim (the innermost axis) is always dense.
 *  - bfloat16 data is passed as its 16-bit pattern.
 *  - Work is enqueued on `stream` (a hipStream_t); nothing synchronizes the
 *    host, nothing allocates device memory, so every call can be captured in
 *    a HIP graph.  Calls that share a workspace must be ordered on one stream.
 *  - Return value: 0 on success, else RKV_* error code; rkv_last_error()
 *    gives a message (thread-local, valid until the next call).
 */
#ifndef REFINEKV_HIP_H
#define REFINEKV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* rkv_stream_t; /* == hipStream_t */

enum {
  RKV_OK = 0,
  RKV_INVALID_ARGUMENT = 1, /* raised as ValueError by the Python binding */
  RKV_UNSUPPORTED = 2,      /* TypeError */
  RKV_LAUNCH_FAILED = 3,    /* RuntimeError */
  RKV_WORKSPACE_TOO_SMALL = 4
};

/* GQA reduction codes (src/refinekv/kernels/runtime.py:23). */
enum { RKV_REDUCE_MEAN = 0, RKV_REDUCE_MAX = 1, RKV_REDUCE_ANY = 2 };

/* Key/value dtype codes for rkv_summary. */
enum { RKV_BF16 = 0, RKV_F16 = 1, RKV_F32 = 2 };

/* Message of the last failed call on this thread ("" after a success). */
const char* rkv_last_error(void);

/* ABI version (incremented on incompatible changes). */
int rkv_version(void);

/*
 * Prompt block summaries.  Replaces build_summary
 * (src/refinekv/summary.py:46-113; it has no accelerated backend in the
 * reference, which runs torch ops on the cache's device).
 *   keys/values: (heads, length, dim) with head/token strides, dtype RKV_*.
 *   counts: (ceil(length/block_size),) int64.
 *   key_mean, value_mean, ellipsoid: (heads, n_blocks, dim) bf16.
 *   value_norm: (heads, n_blocks) fp32; max_value_norm: (heads,) fp32.
 * dim in 32..256 (multiple of 32); block_size in {16, 32, 64}.
 */
int rkv_summary(const void* keys, int64_t k_head_stride, int64_t k_token_stride,
                const void* values, int64_t v_head_stride, int64_t v_token_stride, int dtype,
                int64_t heads, int64_t length, int64_t dim, int64_t block_size, int64_t* counts,
                void* key_mean, void* value_mean, void* ellipsoid, float* value_norm,
                float* max_value_norm, rkv_stream_t stream);

/*
 * Prompt summaries built while the prompt's keys and values are written to
 * the KV cache: rkv_summary's outputs, plus every token of keys / values
 * copied to cache_keys / cache_values (same dtype, (heads, length, dim) with
 * head/token strides, head_dim dense), from the same loads.  Replaces the
 * prefill sequence of a cache write and build_summary
 * (src/refinekv/integrations/transformers.py:529-536 over
 * src/refinekv/summary.py:46-113), which reads the prompt's K/V again.
 */
int rkv_summary_store(const void* keys, int64_t k_head_stride, int64_t k_token_stride,
                      const void* values, int64_t v_head_stride, int64_t v_token_stride,
                      int dtype, int64_t heads, int64_t length, int64_t dim, int64_t block_size,
                      void* cache_keys, int64_t ck_head_stride, int64_t ck_token_stride,
                      void* cache_values, int64_t cv_head_stride, int64_t cv_token_stride,
                      int64_t* counts, void* key_mean, void* value_mean, void* ellipsoid,
                      float* value_norm, float* max_value_norm, rkv_stream_t stream);

/* Workspace bytes needed by rkv_select / rkv_decode for this shape (device
 * memory the caller owns).  Zero-fill it when it is created: its first region
 * holds rkv_decode's hand-off counters, which count this shape's tiles (each
 * call adds the same amount), so zero-fill it again before using it for
 * another shape. */
size_t rkv_workspace_bytes(int64_t heads, int64_t group, int64_t dim, int64_t n_blocks);

/* Byte offsets inside the workspace (for tests): control (hand-off
 * counters: one 64-byte line per KV head, then a line starting with a
 * sticky u32 error word, bit 0 set if a hand-off wait gave up, and the
 * start-order ticket count, then a u64 launch count per one-launch step
 * workgroup), zf (float4 z, delta, A, th per query row and block: the
 * selection statistics and the delta-only factors of the risk), lse
 * (per-tile log-sum-exp partials), lse_slots (the same as tagged 16-byte
 * slots for the one-launch step), part_ml, part_acc (per-workgroup attention
 * partials: (m, l) and acc; tagged 16-byte slots in the one-launch step),
 * counts (per-workgroup access counts), full (per step workgroup: the tag
 * + 1 of the last launch that expanded every block of its tile), total,
 * then n_tiles, the padded row strides (elements) of zf and of the per-tile
 * arrays, and the one-launch step's workgroups per KV head (n_tiles scoring
 * tiles, then copies that repeat a tile's decision and take a share of its
 * token rows; each has a launch counter and a per-tile array entry) ->
 * out13[0..12]. */
int rkv_workspace_layout(int64_t heads, int64_t group, int64_t dim, int64_t n_blocks,
                         int64_t* out13);

/*
 * Expanded-block mask for one query.  Replaces select_blocks_triton
 * (src/refinekv/kernels/runtime.py:93-120) behind select_blocks
 * (src/refinekv/attention.py:62-73); semantics of select_blocks_reference
 * (src/refinekv/reference.py:37-47) plus an optional anchor union.
 *   query: (heads, group, dim) bf16, dense.  Summary tensors as above.
 *   anchor_mask: (heads, n_blocks) bytes 0/1 or NULL.
 *   mask_out: (heads, n_blocks) bytes 0/1 (a torch.bool tensor).
 *   risk_out (heads, group, n_blocks) fp32, stats_out (heads, group, 2) fp32
 *   (log Z, log C) and accessed_blocks (+= sum over blocks of count if
 *   expanded else 1) are optional (NULL = off).
 *   workspace: rkv_workspace_bytes() bytes, 256-byte aligned.
 */
int rkv_select(const void* query, const void* key_mean, const void* ellipsoid,
               const float* value_norm, const float* max_value_norm, int64_t heads,
               int64_t group, int64_t dim, int64_t n_blocks, int64_t block_size,
               int64_t prompt_length, float eps, int reduction, const uint8_t* anchor_mask,
               uint8_t* mask_out, float* risk_out, float* stats_out,
               unsigned long long* accessed_blocks, void* workspace, size_t workspace_bytes,
               rkv_stream_t stream);

/*
 * Prompt-anchor mask: the union of the expanded-block masks of `anchors`
 * queries.  Replaces the per-anchor loop of select_blocks calls in the
 * reference's Transformers hook (src/refinekv/integrations/
 * transformers.py:539-552) with one scoring launch over every (query, head,
 * tile) and one launch that ORs the decisions.
 *   queries: (anchors, heads, group, dim) bf16, dense.  Summary and eps /
 *   reduction as for rkv_select (each query is reduced over its own group).
 *   mask_out: (heads, n_blocks) bytes 0/1.
 *   workspace: rkv_workspace_bytes(heads * anchors, group, dim, n_blocks)
 *   bytes, 256-byte aligned, contents need no initialisation (not the
 *   rkv_decode workspace: its counters must not be overwritten).
 */
int rkv_select_anchors(const void* queries, const void* key_mean, const void* ellipsoid,
                       const float* value_norm, const float* max_value_norm, int64_t heads,
                       int64_t group, int64_t dim, int64_t n_blocks, int64_t block_size,
                       int64_t prompt_length, float eps, int reduction, int64_t anchors,
                       uint8_t* mask_out, void* workspace, size_t workspace_bytes,
                       rkv_stream_t stream);

/*
 * One decode step of RefineKV attention.  Replaces sparse_attention_triton
 * (src/refinekv/kernels/runtime.py:123-227) behind sparse_attention
 * (src/refinekv/attention.py:76-134); semantics of
 * sparse_attention_reference (src/refinekv/reference.py:50-73).
 *   key_pages/value_pages: (heads, n_blocks, block_size, dim) bf16 pages of
 *     the prompt cache; only the head stride is free (block and token
 *     strides are block_size*dim and dim).
 *   key_suffix/value_suffix: generated tokens, (heads, capacity, dim) with
 *     head/token strides; suffix_length: device int32 scalar giving the valid
 *     prefix (clamped to [0, capacity]), or NULL to use all `capacity` tokens.
 *   mask_out: (heads, n_blocks) bytes 0/1; output: (heads, group, dim) bf16.
 *   accessed_blocks: optional access counter as in rkv_select.
 */
int rkv_decode(const void* query, const void* key_mean, const void* ellipsoid,
               const void* value_mean, const float* value_norm, const float* max_value_norm,
               const void* key_pages, int64_t key_page_head_stride, const void* value_pages,
               int64_t value_page_head_stride, const void* key_suffix,
               int64_t key_suffix_head_stride, int64_t key_suffix_token_stride,
               const void* value_suffix, int64_t value_suffix_head_stride,
               int64_t value_suffix_token_stride, int64_t suffix_capacity,
               const int32_t* suffix_length, int64_t heads, int64_t group, int64_t dim,
               int64_t n_blocks, int64_t block_size, int64_t prompt_length, float eps,
               int reduction, const uint8_t* anchor_mask, uint8_t* mask_out, void* output,
               unsigned long long* accessed_blocks, void* workspace, size_t workspace_bytes,
               rkv_stream_t stream);

/*
 * Dense decode: one query token per row attends every cached token of its
 * head, with no summary.  Replaces the SDPA call of the reference's dense
 * decode (src/refinekv/integrations/transformers.py:510-520: layers below
 * full_attention_layers, and the dense baseline of speed/README.md:73):
 *   out[h, g] = softmax(query[h, g] . keys[h, t] / sqrt(dim)) @ values[h, t]
 *   over t = 0 .. L - 1.
 *   query: (heads, group, dim) bf16, contiguous; out: the same shape.
 *   keys/values: bf16, token t of head h at base + h * head_stride +
 *     t * token_stride elements (the (1, heads, capacity, dim) cache of a
 *     Transformers layer: head_stride capacity*dim, token_stride dim).
 *   length: L, or, when length_dev is given, the capacity the views cover and
 *     L = *length_dev (device int32) clamped to [0, length] (graph replays).
 *   workspace: rkv_dense_plan's bytes (per-split partials).
 * dim 32..160 step 32, group <= 16.  L = 0 gives zeros.
 */
int rkv_dense_decode(const void* query, const void* keys, int64_t key_head_stride,
                     int64_t key_token_stride, const void* values, int64_t value_head_stride,
                     int64_t value_token_stride, int64_t heads, int64_t group, int64_t dim,
                     int64_t length, const int32_t* length_dev, void* output, void* workspace,
                     size_t workspace_bytes, rkv_stream_t stream);

/* rkv_dense_decode's split of each head's tokens on the current device and
 * the workspace bytes it needs for `length` tokens (no reference
 * counterpart: SDPA allocates internally). */
int rkv_dense_plan(int64_t heads, int64_t group, int64_t dim, int64_t length, int64_t* splits,
                   size_t* workspace_bytes);

/* Profiling hook with no reference counterpart: when `events` points to 4
 * hipEvent_t handles, later rkv_select / rkv_decode calls on this thread
 * record events[0] before their first kernel and events[k] after their k-th
 * (rkv_select: score, decide; rkv_decode: the one-launch step, or score,
 * attend, merge).  NULL turns it off. */
int rkv_set_profile_events(void* events);

/* Test hook with no reference counterpart: 0 (default) lets rkv_decode run
 * one launch per step (score, decision, attention and merge in one kernel,
 * heads handed off through the workspace's counters) where the shape allows
 * it -- every query row in one attention pass and at most 256 tiles of 64
 * blocks per head -- and three kernels otherwise; 1 always uses the three
 * kernels.  Per thread. */
int rkv_set_decode_path(int path);

/*
 * rkv_decode without a caller workspace (no counterpart in the reference):
 * for callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Arguments
 * and results are rkv_decode's, minus the workspace: the library keeps one
 * 64 MiB device array per GPU for the call's intermediates (allocated with
 * the library, held until the process ends) and allocates nothing.  Shapes
 * whose rkv_workspace_bytes exceed 64 MiB - 256 bytes return
 * RKV_WORKSPACE_TOO_SMALL.  Each call first clears the array's hand-off
 * counters and slots with fill kernels on `stream`, so calls of different
 * shapes may follow each other on one stream; calls that overlap on one GPU
 * (other streams or threads) race on the shared array and must not be
 * issued.  A hand-off wait that gives up writes NaN output rows and an
 * all-expanded mask for its head, as rkv_decode does, and sets the array's
 * own status word (rkv_static_status), which no later call clears.
 */
int rkv_decode_static(const void* query, const void* key_mean, const void* ellipsoid,
                      const void* value_mean, const float* value_norm,
                      const float* max_value_norm, const void* key_pages,
                      int64_t key_page_head_stride, const void* value_pages,
                      int64_t value_page_head_stride, const void* key_suffix,
                      int64_t key_suffix_head_stride, int64_t key_suffix_token_stride,
                      const void* value_suffix, int64_t value_suffix_head_stride,
                      int64_t value_suffix_token_stride, int64_t suffix_capacity,
                      const int32_t* suffix_length, int64_t heads, int64_t group, int64_t dim,
                      int64_t n_blocks, int64_t block_size, int64_t prompt_length, float eps,
                      int reduction, const uint8_t* anchor_mask, uint8_t* mask_out,
                      void* output, unsigned long long* accessed_blocks, rkv_stream_t stream);

/* The status word of rkv_decode_static's array on the current device (part
 * of that entry point, for the same callers; no reference counterpart):
 * *status receives it (bit 0: a hand-off wait of a static call gave up since
 * the word was last cleared), with clear != 0 it is then zeroed.  Copies the
 * word to the host and synchronizes `stream` (not for graph capture). */
int rkv_static_status(uint32_t* status, int clear, rkv_stream_t stream);

/* Hand-off status of an rkv_decode workspace (no reference counterpart: the
 * reference's Triton kernels have no cross-workgroup waits).  *status
 * receives the workspace's sticky status word: bit 0 is set when a wait of
 * the one-launch step gave up after its poll limit.  The call that gave up
 * also wrote NaN to the head's output rows and marked all its blocks
 * expanded, so its result is not a plausible answer either way.  Copies the
 * word to the host and synchronizes `stream` (a debugging query: not for
 * graph capture).  The shape arguments are those the workspace was sized
 * for. */
int rkv_workspace_status(const void* workspace, size_t workspace_bytes, int64_t heads,
                         int64_t group, int64_t dim, int64_t n_blocks, uint32_t* status,
                         rkv_stream_t stream);

/* Clears the status word (one tiny kernel on `stream`). */
int rkv_workspace_clear_status(void* workspace, size_t workspace_bytes, int64_t heads,
                               int64_t group, int64_t dim, int64_t n_blocks,
                               rkv_stream_t stream);

/* Which path rkv_decode takes for this shape on the current device, for
 * tests and benchmarks (no reference counterpart): *mode_out = 0 for three
 * kernels, 1 for one launch with its whole grid resident, 2 for one launch
 * whose workgroups draw (head, workgroup) tickets in start order (grids of
 * up to two device-fulls, blocks of 64 tokens), 3 for one resident launch
 * whose workgroups score up to 4 tiles of 64 blocks each (heads with more
 * tiles than the device holds workgroups for them, query groups of at most
 * 4, head_dim <= 128). */
int rkv_decode_plan(int64_t heads, int64_t group, int64_t dim, int64_t n_blocks,
                    int64_t block_size, int* mode_out);

/* Test hook with no reference counterpart: spin_limit replaces the one-launch
 * step's poll limit per hand-off wait (0 = the default, 2^20), and a nonzero
 * skew makes every wait accept no published data, so each wait runs out its
 * limit, sets the status word and goes on (NaN output, all-expanded mask);
 * every kernel still ends.  Per thread; (0, 0) restores normal operation. */
int rkv_set_handoff_test(uint32_t spin_limit, uint32_t skew);

/* Test hook with no reference counterpart: the one-launch step's
 * speculation, 0 off, 1 (default), 2 forced (the same as 1 since it has no
 * size threshold any more; kept for the tests); other modes return
 * RKV_INVALID_ARGUMENT.  When the previous launch on a workspace expanded
 * every block of a workgroup's tile, the workgroup issues the first page
 * rows of the tile before the decision and continues from them if every
 * block expands again (else it lets them land and attends as usual): the
 * output is the same bit for bit either way.  Per thread. */
int rkv_set_speculation(int mode);

/* Test hook with no reference counterpart: applies a device scalar function
 * fn to n floats: 0 exp and 1 log as the oracle computes them (expf_,
 * logf_), 2 bf16 round trip, 3 sqrt, 4 exp and 5 log as the selection
 * kernels compute them (the hardware's transcendental unit); other fn
 * return RKV_INVALID_ARGUMENT. */
int rkv_math_probe(int fn, const float* x, float* y, int64_t n, rkv_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* REFINEKV_HIP_H */

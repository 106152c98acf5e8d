/*
 * wnw_amd.h -- C ABI of the MI355X (gfx950) decode-step attention path over
 * the flat varlen KV cache of WnW.
 *
 * Every entry point takes plain device pointers, 64-bit sizes and a
 * hipStream_t passed as `void*` (NULL = the default stream), launches
 * asynchronously on that stream, and returns an int status (WNW_OK on
 * success).  On failure wnw_last_error() returns a message for the calling
 * thread.  No entry point allocates device memory except where stated.
 *
 * Flat layout (reference: src/common/kv/flat_cache.py:46-54): per layer, K
 * and V are row-major [rows, head_dim] arrays; segment s = b * Hkv + h holds
 * the rows of (sequence b, KV head h); cu_seqlens is int32 [n_seg + 1] with
 * cu[0] = 0 and segment s = logical rows [cu[s], cu[s+1]).  An optional int64
 * seg_base[n_seg] gives the physical row of each segment's first row, so a
 * cache may keep per-segment slack and append in place; when seg_base is
 * NULL the physical row of logical row j is j (the reference's dense layout).
 *
 * Device-side bounds: kernels that follow offsets read from device memory
 * check every derived row against the row counts passed here and, instead
 * of reading out of bounds, record an error that wnw_device_error() returns.
 */
#ifndef WNW_AMD_H
#define WNW_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define WNW_OK 0
#define WNW_EINVAL 1   /* invalid argument (shape, dtype, null pointer)   */
#define WNW_EHIP 2     /* HIP runtime error                               */
#define WNW_ENOTSUP 3  /* valid but unsupported configuration             */

/* element types of K, V, q and outputs */
#define WNW_F32 0
#define WNW_F16 1
#define WNW_BF16 2

/* device error bits recorded by kernels (wnw_device_error) */
#define WNW_DEVERR_BOUNDS 1   /* an offset pointed outside the given rows  */
#define WNW_DEVERR_ORDER 2    /* cu_seqlens not non-decreasing             */
#define WNW_DEVERR_CAPACITY 4 /* in-place append beyond segment capacity   */

/* attention kernel selection (wnw_decode_attn_ex) */
#define WNW_ATTN_AUTO 0 /* MFMA kernel where supported, else VALU kernel  */
#define WNW_ATTN_MFMA 1 /* bf16/f16, head_dim 64/128, group <= 16         */
#define WNW_ATTN_VALU 2 /* any dtype, head_dim 64/128/256, group <= 16    */

/* Message describing the last failure on this thread ("" if none). */
const char* wnw_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int wnw_abi_version(void);

/*
 * Prepares the current device (allocates the 256-byte device error word).
 * Call once per device before graph capture; other entry points call it
 * lazily otherwise.
 */
int wnw_init(void);

/*
 * Reads and optionally clears the device error word of the current device.
 * Synchronizes the device.  Returns WNW_DEVERR_* bits (0 = no error) or -1
 * if the query itself failed.  No counterpart in the reference, which does
 * no validation (src/common/kv/kernels.py:22-35 reads whatever cu points to).
 */
int wnw_device_error(int clear);

/* ------------------------------------------------------------------------ */
/* Append                                                                    */
/* ------------------------------------------------------------------------ */

/*
 * Out-of-place append of one row per segment, bit-exact with the
 * reference's interleave_append (src/common/kv/kernels.py:45-73, kernel
 * :7-42):
 *   out[cu_new[s] + i] = old[cu_old[s] + i]   for i < cu_old[s+1]-cu_old[s]
 *   out[cu_new[s+1] - 1] = new_rows[s]
 * old: [total_old, head_dim]; new_rows: [n_seg, head_dim];
 * out: [total_old + n_seg, head_dim].  Unlike the reference (whose 10-step
 * binary search caps n_seg at 1024, kernels.py:22-27) any n_seg works.
 */
int wnw_interleave_append(const void* old_rows, const void* new_rows,
                          const int32_t* cu_old, const int32_t* cu_new,
                          int64_t n_seg, int64_t total_old, int64_t head_dim,
                          int dtype, void* out, void* stream);

/*
 * In-place append into a layout with per-segment slack (no reference
 * counterpart; it replaces the two full-layer copies of
 * src/algorithms/wnw/code/cache.py:506-507 for caches that keep slack).
 * For every segment s: len = cu_old[s+1] - cu_old[s];
 *   k_pool[seg_base[s] + len] = new_k[s]; v_pool[...] = new_v[s];
 *   cu_new[s] = cu_old[s] + s  (s = 0..n_seg), i.e. the reference's
 *   cu_new = cu_old + arange(n_seg + 1) (cache.py:504).
 * seg_cap[s] bounds len + 1 (WNW_DEVERR_CAPACITY otherwise, row skipped).
 * cu_new must not alias cu_old.
 */
int wnw_append_inplace(void* k_pool, void* v_pool, const void* new_k,
                       const void* new_v, const int32_t* cu_old,
                       int32_t* cu_new, const int64_t* seg_base,
                       const int32_t* seg_cap, int64_t n_seg,
                       int64_t pool_rows, int64_t head_dim, int dtype,
                       void* stream);

/* ------------------------------------------------------------------------ */
/* Compaction                                                                */
/* ------------------------------------------------------------------------ */

/*
 * Out-of-place compaction + load + append of K and V in one launch,
 * bit-exact with rebuild_append_kv (src/algorithms/wnw/code/kernels.py:
 * 375-404, kernel :407-473).  Output segment s (rows new_cu[s]..new_cu[s+1])
 * = old rows of s minus the sorted, disjoint relative ranges
 *   [evict_starts[e], evict_ends[e]) for e in [evict_offsets[s],
 *   evict_offsets[s+1]) ++ load rows [load_starts[s], +load_lens[s]) ++
 * new_k/new_v[s].  total_out = new_cu[n_seg] must be passed by the caller
 * (the reference reads it back with .item(), kernels.py:393).  max_evict is
 * the reference's MAX_EVICT bound; ranges beyond it are ignored exactly as
 * the reference's loop over range(MAX_EVICT) ignores them.  n_evict is the
 * number of entries in evict_starts/evict_ends (device-side bound).
 */
int wnw_rebuild_append_kv(const void* old_k, const void* old_v,
                          const void* new_k, const void* new_v,
                          const void* load_k, const void* load_v,
                          const int32_t* old_cu, const int32_t* new_cu,
                          const int32_t* load_starts, const int32_t* load_lens,
                          const int32_t* evict_offsets,
                          const int32_t* evict_starts,
                          const int32_t* evict_ends, int64_t n_evict,
                          int64_t n_seg, int64_t total_old, int64_t total_load,
                          int64_t total_out, int64_t max_evict,
                          int64_t head_dim, int dtype, void* out_k,
                          void* out_v, void* stream);

/*
 * Generalised compaction for a slack layout: the same per-segment
 * descriptors as wnw_rebuild_append_kv, but source and destination segments
 * are addressed by physical base arrays and only the n_list segments in
 * seg_list (each < n_seg) are rebuilt (the others are untouched); max_new_len bounds
 * new_len over the listed segments and sizes the grid.  new_len[s] is the
 * output length of segment s (evicted rows removed, loads and the optional
 * new row added).  with_new != 0 appends new_k/new_v[s] as the last row.
 * dst ranges must not overlap any src range of a listed segment.  Replaces
 * the per-layer full copy of cache.py:716-754 when only a few segments
 * change.
 */
int wnw_compact_segments(const void* src_k, const void* src_v, void* dst_k,
                         void* dst_v, const void* new_k, const void* new_v,
                         const void* load_k, const void* load_v,
                         const int32_t* seg_list, int64_t n_list,
                         int64_t n_seg, int64_t max_new_len,
                         const int64_t* src_base,
                         const int32_t* src_len,
                         const int64_t* dst_base, const int32_t* new_len,
                         const int32_t* load_starts, const int32_t* load_lens,
                         const int32_t* evict_offsets,
                         const int32_t* evict_starts,
                         const int32_t* evict_ends, int64_t n_evict,
                         int with_new, int64_t src_rows, int64_t dst_rows,
                         int64_t load_rows, int64_t head_dim, int dtype,
                         void* stream);

/* ------------------------------------------------------------------------ */
/* Decode attention (q = 1 per segment, GQA group of `group` query heads)    */
/* ------------------------------------------------------------------------ */

/*
 * Bytes of workspace wnw_decode_attn needs for n_seg segments on the
 * current device.  The workspace holds split-K partials and per-segment
 * arrival counters; it must be cleared once with wnw_workspace_init before
 * its first use and may then be reused by any number of launches on one
 * stream (every launch leaves the counters at zero).  The counters occupy the
 * first 4 * n_seg bytes (rounded up to 256): before reusing a workspace for a
 * larger n_seg than it was cleared for, clear it again.
 */
int64_t wnw_decode_attn_workspace_bytes(int64_t n_seg, int64_t group,
                                        int64_t head_dim);

/* Clears a workspace with a fill kernel (safe under graph capture). */
int wnw_workspace_init(void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Split-K GQA decode attention over the flat layout.  Same mathematics as
 * the reference's q1_decode_attn (src/common/kv/fused_attn.py:47-65, kernel
 * :9-44) and its default varlen_attn call with 0-stride GQA K/V
 * (src/algorithms/wnw/code/session.py:90-106):
 *   out[s, g, :] = softmax(scale * K_s q[s, g]) @ V_s
 * where q is [n_seg, group, head_dim] (q head h = kv * group + g,
 * session.py:81-83) and K_s/V_s are the rows of segment s.  fp32 softmax
 * and accumulation; out has the dtype of q/K/V.  An empty segment yields
 * zeros.  total_rows is an upper bound of cu_k[n_seg] (it only sizes the
 * grid); kv_rows is the number of rows allocated in k and v.
 */
int wnw_decode_attn(const void* q, const void* k, const void* v,
                    const int32_t* cu_k, const int64_t* seg_base,
                    int64_t n_seg, int64_t group, int64_t head_dim,
                    int64_t total_rows, int64_t kv_rows, float scale,
                    int dtype, void* out, void* workspace,
                    int64_t workspace_bytes, void* stream);

/*
 * wnw_decode_attn with an explicit kernel choice (WNW_ATTN_*) and an
 * explicit grid size (n_wg <= 0 selects one from the device's occupancy).
 * Used to compare the MFMA and VALU kernels under one harness.
 */
int wnw_decode_attn_ex(const void* q, const void* k, const void* v,
                       const int32_t* cu_k, const int64_t* seg_base,
                       int64_t n_seg, int64_t group, int64_t head_dim,
                       int64_t total_rows, int64_t kv_rows, float scale,
                       int dtype, void* out, void* workspace,
                       int64_t workspace_bytes, int kernel, int64_t n_wg,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WNW_AMD_H */

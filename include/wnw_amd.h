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
 * cache may keep per-segment slack, append in place and place segments in
 * any order; when seg_base is NULL the physical row of logical row j is j
 * (the reference's dense layout).
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
#define WNW_DEVERR_ORDER 2    /* cu_seqlens decreasing                     */
#define WNW_DEVERR_CAPACITY 4 /* in-place append beyond segment capacity   */

/* attention kernel selection (wnw_decode_attn_ex) */
#define WNW_ATTN_AUTO 0 /* fastest kernel that supports the arguments    */
#define WNW_ATTN_MFMA 1 /* bf16/f16, head_dim 64/128, group <= 16         */
#define WNW_ATTN_VALU 2 /* any dtype, head_dim 64/128/256, group <= 16    */
#define WNW_ATTN_STREAM 3 /* bf16/f16, head_dim 64/128, group <= 8 (AUTO's
                             choice there)                              */

/* Message describing the last failure on this thread ("" if none). */
const char* wnw_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int wnw_abi_version(void);

/*
 * Prepares the current device: resolves the address of its device error
 * word (a file-scope device array of the library, zero at load; nothing is
 * allocated).  Call once per device before graph capture; other entry
 * points call it lazily otherwise.
 */
int wnw_init(void);
/*
 * Sets up, on the current device, the kernels the decode step launches
 * outside the attention (scoring pass, chunk top-k, compaction and appends,
 * the offload channel's kernels): the runtime otherwise does it at each
 * kernel's first launch, ~1-2 ms each on MI355X, inside the first decode
 * steps.  No reference counterpart (the reference warms its Triton kernels
 * instead, src/algorithms/wnw/code/cache.py:392-484).  Always WNW_OK.
 */
int wnw_prepare_kernels(void);

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
 * wnw_interleave_append of K and V in one launch: the pair of calls
 * decode_before_attn makes (src/algorithms/wnw/code/cache.py:506-507, each
 * the reference's interleave_append, src/common/kv/kernels.py:45-73), with
 * every row's source resolved once for both tensors.  out_k / out_v as
 * wnw_interleave_append's out.
 */
int wnw_interleave_append_kv(const void* old_k, const void* old_v,
                             const void* new_k, const void* new_v,
                             const int32_t* cu_old, const int32_t* cu_new,
                             int64_t n_seg, int64_t total_old, int64_t head_dim,
                             int dtype, void* out_k, void* out_v, void* stream);

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
 * first 4 * n_seg bytes (rounded up to 256) and the partials follow them, so
 * a launch with another n_seg turns partial bytes into counters and the
 * reverse: clear the workspace again whenever n_seg changes.
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
 * zeros (as the reference's default varlen_attn path does for an empty
 * key range; no decode-time segment is ever empty, since each holds the
 * step's own row).  The kernel splits the logical rows [0, cu_k[n_seg])
 * evenly over its workgroups (it reads cu_k[n_seg] itself, so a launch
 * captured in a graph stays right as segments grow), so the cost does not
 * depend on how ragged the segments are.  total_rows, an estimate of
 * cu_k[n_seg], only sizes the grid.  kv_rows is the number of rows allocated
 * in k and v: a segment outside [0, kv_rows) sets WNW_DEVERR_BOUNDS and
 * yields NaN.  Segments may sit anywhere in k / v, in any order; decreasing
 * offsets set WNW_DEVERR_ORDER.  q, k, v and out must be 16-byte aligned.
 */
int wnw_decode_attn(const void* q, const void* k, const void* v,
                    const int32_t* cu_k, const int64_t* seg_base,
                    int64_t n_seg, int64_t group, int64_t head_dim,
                    int64_t total_rows, int64_t kv_rows, float scale,
                    int dtype, void* out, void* workspace,
                    int64_t workspace_bytes, void* stream);

/*
 * The step's append and the decode attention in one launch, for a cache
 * with per-segment slack.  Replaces decode_before_attn's two full-layer
 * interleave_append copies (src/algorithms/wnw/code/cache.py:497-515,
 * src/common/kv/kernels.py:45-73) plus the q1_decode_attn / varlen_attn
 * call (src/common/kv/fused_attn.py:47-65, src/algorithms/wnw/code/
 * session.py:90-106).  For every segment s, with len = cu_old[s+1] -
 * cu_old[s]: new_k/new_v[s] becomes row seg_base[s] + len of k_pool/v_pool,
 * cu_new = cu_old + arange(n_seg + 1) (the reference's cache.py:504), and
 * out is wnw_decode_attn over the len + 1 rows of every segment.  The
 * streaming kernel reads the new rows from new_k/new_v and writes them into
 * the pools itself (one launch); other kernels (fp32, head_dim 256, group
 * > 8) run wnw_append_inplace first.  total_rows (an estimate of
 * cu_old[n_seg] + n_seg) sizes the grid.
 * seg_cap[s] bounds len + 1 (WNW_DEVERR_CAPACITY otherwise; the row is then
 * attended but not stored).  cu_new must not alias cu_old.  new_k/new_v
 * 16-byte aligned.
 */
int wnw_decode_attn_append(const void* q, void* k_pool, void* v_pool,
                           const void* new_k, const void* new_v,
                           const int32_t* cu_old, int32_t* cu_new,
                           const int64_t* seg_base, const int32_t* seg_cap,
                           int64_t n_seg, int64_t group, int64_t head_dim,
                           int64_t total_rows, int64_t pool_rows, float scale,
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

/* Limits of wnw_decode_attn_noalloc: the size of the library's own split-K
 * scratch on each device, and the segments its counters region holds. */
#define WNW_NOALLOC_SCRATCH_BYTES (16ll << 20)
#define WNW_NOALLOC_MAX_SEG 4096

/*
 * wnw_decode_attn (AUTO kernel, grid from the device's occupancy) without a
 * workspace argument: allocates nothing, ever.  No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The split-K partials and arrival counters live in a
 * file-scope device array of the library, WNW_NOALLOC_SCRATCH_BYTES per
 * device, held until the process ends.  Limits: n_seg <= WNW_NOALLOC_MAX_SEG,
 * and (grid + n_seg) partial slots of group * (head_dim + 2) floats must fit
 * the array (n_seg 512, group 4, head_dim 128 needs ~1.6 MB); a larger call
 * returns WNW_EINVAL with the bytes it would need.  Every call on a device
 * shares that device's array, so calls that overlap on one device (other
 * streams, other threads) race: order them on one stream.  The first call on
 * a device clears the counters with a fill kernel on `stream`.
 */
int wnw_decode_attn_noalloc(const void* q, const void* k, const void* v,
                            const int32_t* cu_k, const int64_t* seg_base,
                            int64_t n_seg, int64_t group, int64_t head_dim,
                            int64_t total_rows, int64_t kv_rows, float scale,
                            int dtype, void* out, void* stream);

/* ------------------------------------------------------------------------ */
/* Class-A token scores                                                      */
/* ------------------------------------------------------------------------ */

/* Workspace of wnw_decode_attn_score: the attention workspace, the
 * per-segment softmax normalisers, then (max_audio > 0) room for the logits
 * of the scored audio rows, n_seg * group * max_audio floats.  Same clearing
 * rule as the attention workspace (wnw_workspace_init once, again whenever
 * n_seg changes).  A workspace sized with max_audio = 0 still works: the
 * scoring pass then reads the K rows again. */
int64_t wnw_decode_attn_score_workspace_bytes(int64_t n_seg, int64_t group,
                                              int64_t head_dim, int64_t max_audio);

/*
 * Decode attention + class-A score accumulation, the reference's
 * q1_decode_attn_score (src/common/kv/fused_attn.py:68-156, used for
 * "foldable" layers by WnWCache.fused_decode_attention, src/algorithms/wnw/
 * code/cache.py:546-566).  out is wnw_decode_attn's result.  Then, for every
 * segment s = b * num_kv_heads + kv with ca_kv_mask[kv] != 0 and every
 * audio row j in [audio_starts[b], audio_ends[b]) of the segment,
 *   score_acc[score_offsets[b] + j - audio_starts[b]] +=
 *       sum_g exp(scale * q[s, g] . K[row j] - m[s, g]) / l[s, g]
 * with (m, l) the final softmax max / sum of the attention itself (the
 * reference adds with atomics; here one workgroup owns each token, so the
 * sum is deterministic).  max_audio >= every audio_ends[b] - audio_starts[b]
 * (it sizes the grid); acc_len = entries of score_acc.  Audio ranges outside
 * a segment set WNW_DEVERR_BOUNDS and skip that segment.
 * When the streaming attention kernel runs (bf16/f16, head_dim 64/128,
 * group <= 8) and the workspace has room for the logits (see
 * wnw_decode_attn_score_workspace_bytes), the attention kernel keeps the
 * scaled logits of the scored rows and the scoring pass reads those instead
 * of K (4 bytes per row and head instead of 2 * head_dim).
 */
int wnw_decode_attn_score(const void* q, const void* k, const void* v,
                          const int32_t* cu_k, const int64_t* seg_base,
                          int64_t n_seg, int64_t group, int64_t head_dim,
                          int64_t total_rows, int64_t kv_rows, float scale,
                          int dtype, void* out, const int32_t* ca_kv_mask,
                          int64_t num_kv_heads, const int32_t* audio_starts,
                          const int32_t* audio_ends, float* score_acc,
                          const int32_t* score_offsets, int64_t acc_len,
                          int64_t max_audio, void* workspace,
                          int64_t workspace_bytes, void* stream);

/*
 * wnw_decode_attn_append followed by the class-A scoring of
 * wnw_decode_attn_score over the post-append segments (cu_new): the step's
 * append + q1_decode_attn_score (src/common/kv/fused_attn.py:124-156) of a
 * foldable layer (src/algorithms/wnw/code/cache.py:546-566).  Same
 * workspace as wnw_decode_attn_score.
 */
int wnw_decode_attn_score_append(
    const void* q, void* k_pool, void* v_pool, const void* new_k,
    const void* new_v, const int32_t* cu_old, int32_t* cu_new,
    const int64_t* seg_base, const int32_t* seg_cap, int64_t n_seg,
    int64_t group, int64_t head_dim, int64_t total_rows, int64_t pool_rows,
    float scale, int dtype, void* out, const int32_t* ca_kv_mask,
    int64_t num_kv_heads, const int32_t* audio_starts,
    const int32_t* audio_ends, float* score_acc, const int32_t* score_offsets,
    int64_t acc_len, int64_t max_audio, void* workspace,
    int64_t workspace_bytes, void* stream);

/* Workspace of wnw_fused_score_accumulate (partial softmax statistics). */
int64_t wnw_fused_score_workspace_bytes(int64_t n_samples, int64_t n_heads);

/*
 * The reference's fused_score_accumulate (src/algorithms/wnw/code/
 * kernels.py:302-370): for each of n_samples items with query heads
 * q[i, 0..n_heads), the softmax over K rows [seg_starts[i], seg_ends[i]) of
 * scale * q . K (the reference uses scale = head_dim^-0.5), summed over the
 * heads, is added at the audio rows [audio_starts[i], audio_ends[i])
 * (relative to seg_starts[i]) to accumulator[accum_offsets[i] + j].
 * Two launches: partial statistics over 32 row slices per item, then the
 * scoring pass over the audio rows.  k_rows = rows of k (bounds).
 */
int wnw_fused_score_accumulate(const void* q, const void* k,
                               const int32_t* seg_starts,
                               const int32_t* seg_ends,
                               const int32_t* audio_starts,
                               const int32_t* audio_ends, float* accumulator,
                               const int32_t* accum_offsets, int64_t n_samples,
                               int64_t n_heads, int64_t head_dim,
                               int64_t k_rows, int64_t acc_len,
                               int64_t max_audio, float scale, int dtype,
                               void* workspace, int64_t workspace_bytes,
                               void* stream);

/*
 * Deferred class-A scoring (no reference counterpart as such: it splits
 * q1_decode_attn_score, src/common/kv/fused_attn.py:68-156, over two
 * launches so that no launch of its own is needed).  A streaming launch
 * keeps the scaled logits of its flagged KV heads' audio rows and its final
 * softmax normalisers in a score slot; the next streaming launch scores
 * that slot into the accumulator while its own first loads are in flight
 * (one 256-token slice of one sample per workgroup), exactly as
 * wnw_decode_attn_score's scoring pass would (bit-identical sums).  A slot
 * holds [n_seg, G, 2] normalisers then [n_seg, G, max_audio] logits, fp32
 * (wnw_score_slot_bytes).
 *
 * wnw_decode_attn_append_deferred: wnw_decode_attn_append (the step's append
 * into slack + attention, one launch) that also
 *   - keeps this launch's logits and normalisers in keep_slot when keep_mask
 *     ([num_kv_heads] non-zero = scored) is given (NOT scored yet), and
 *   - scores prev_slot (kept by an earlier launch over segments prev_cu /
 *     prev_base of prev_pool_rows rows; bit h of prev_kv_bits: KV head h
 *     scored) into score_acc when prev_slot is given.
 * audio_starts / audio_ends / max_audio / score_offsets / acc_len describe
 * both launches.  Returns WNW_ENOTSUP, launching nothing, where the form
 * does not apply (not the streaming kernel's case, more than 64 segments,
 * more than 8 scored KV heads or 16 (scored KV head, query head) pairs, or
 * more 256-token slices of the samples' audio than workgroups): the
 * caller then scores with wnw_decode_attn_score_append /
 * wnw_score_kept_logits.
 * wnw_score_kept_logits: the scoring pass over a slot in a launch of its
 * own (the last launch of a step has no next launch to carry it).
 */
int64_t wnw_score_slot_bytes(int64_t n_seg, int64_t group, int64_t max_audio);
int wnw_decode_attn_append_deferred(
    const void* q, void* k_pool, void* v_pool, const void* new_k,
    const void* new_v, const int32_t* cu_old, int32_t* cu_new,
    const int64_t* seg_base, const int32_t* seg_cap, int64_t n_seg,
    int64_t group, int64_t head_dim, int64_t total_rows, int64_t pool_rows,
    float scale, int dtype, void* out, int64_t num_kv_heads,
    const int32_t* audio_starts, const int32_t* audio_ends, int64_t max_audio,
    float* score_acc, const int32_t* score_offsets, int64_t acc_len,
    const int32_t* keep_mask, float* keep_slot, uint64_t prev_kv_bits,
    const float* prev_slot, const int32_t* prev_cu, const int64_t* prev_base,
    int64_t prev_pool_rows, void* workspace, int64_t workspace_bytes,
    void* stream);
int wnw_score_kept_logits(const int32_t* kv_mask, const float* slot,
                          const int32_t* cu, const int64_t* seg_base,
                          int64_t kv_rows, int64_t n_seg, int64_t group,
                          int64_t num_kv_heads, const int32_t* audio_starts,
                          const int32_t* audio_ends, int64_t max_audio,
                          float* score_acc, const int32_t* score_offsets,
                          int64_t acc_len, void* stream);

/*
 * Chunk scores and the top-k chunk choice of the decode planner, one launch
 * for every sample: the chunk selection of src/algorithms/wnw/code/
 * cache.py:632-649 (prefix-sum chunk means, topk) in the batched form of
 * src/algorithms/wnw_cpp/code/cache.py:160-171 (-1 where a sample has fewer
 * chunks than k).  Sample b's scores are score_acc[score_offsets[b] ..
 * score_offsets[b+1]); its chunks are entries chunk_offsets[b] ..
 * chunk_offsets[b+1] of chunk_starts / chunk_ends (token bounds relative to
 * the sample's first score).  A chunk's score is the mean of its scores
 * (float64 prefix sums over the sample's scores, the chunk's sum divided by
 * max(1, length) and rounded to float32; the reference takes a float32
 * cumsum).  out_idx [n_samples, k]
 * receives each sample's k best chunks in descending order of score, equal
 * scores to the lower chunk index, -1 past the sample's chunk count.  At most
 * 8192 chunks per sample and k <= 64; bounds outside the scores set
 * WNW_DEVERR_BOUNDS (that chunk is never chosen).
 */
int wnw_chunk_topk(const float* score_acc, int64_t acc_len,
                   const int32_t* score_offsets, int64_t n_samples,
                   const int32_t* chunk_offsets, const int32_t* chunk_starts,
                   const int32_t* chunk_ends, int64_t n_chunks, int64_t k,
                   int32_t* out_idx, void* stream);

/*
 * Host->device transfer engine for a plan's offloaded rows: the gather into
 * pinned staging of src/algorithms/wnw_cpp/code/planner.cpp:113-122 and the
 * side-stream copy + wait of src/algorithms/wnw/code/cache.py:716-721 and
 * :868-881, run by a background thread with a pool of gather threads.  The
 * ranges (host rows [ranges[2r], ranges[2r+1]) of host_k / host_v, in
 * transfer order) are split into groups (ranges group_ranges[g] ..
 * group_ranges[g+1]); group by group the rows are gathered into
 * consecutive staging rows, copied (hipMemcpyAsync, the DMA engines) to the
 * same rows of dev_k / dev_v on `stream`, and an event is recorded.
 * wnw_h2d_start returns at once (after the previous start is fully issued);
 * wnw_h2d_wait makes a stream wait for one group's copy (the host blocks
 * only until that copy is issued); wnw_h2d_join waits until every group is
 * issued.  Staging is used in two alternating pairs by the caller: a start
 * waits for the copies of the start before the previous one (the last use
 * of its pair) before gathering.  At most 64 groups.  After a HIP error the
 * job's remaining groups are not gathered, their waits return the error, and
 * the engine drains the stream.  wnw_h2d_destroy returns once every issued
 * copy has finished, so the caller may then free the staging.  host_rows,
 * stg_rows and dev_rows count rows of row_bytes bytes each: every array
 * holds rows of that one size (the engine checks ranges against host_rows
 * and the gathered rows against stg_rows and dev_rows).
 */
typedef struct wnw_h2d wnw_h2d;
wnw_h2d* wnw_h2d_create(int n_workers);  /* NULL on error */
void wnw_h2d_destroy(wnw_h2d* x);
int wnw_h2d_start(wnw_h2d* x, const void* host_k, const void* host_v,
                  int64_t host_rows, const int32_t* ranges, int64_t n_ranges,
                  const int64_t* group_ranges, int n_groups, void* stg_k,
                  void* stg_v, int64_t stg_rows, void* dev_k, void* dev_v,
                  int64_t dev_rows, int64_t row_bytes, void* stream);
/*
 * wnw_h2d_start without the host gather: stage_k / stage_v are DEVICE rows
 * (stage_rows of row_bytes, at least the job's rows).  Per group, the
 * ranges are taken in host-row order and merged where they touch in host
 * memory; each merged span is copied by the DMA engines straight from
 * host_k / host_v into the group's stage rows, and a kernel on `stream` then
 * moves every range to its transfer-order rows of dev_k / dev_v before the
 * group's event (the same rows wnw_h2d_start fills).  Host rows laid out so
 * that a segment's rows of consecutive layers are adjacent make a group a
 * few large copies.  row_bytes a multiple of 16; stage and device rows
 * 16-byte aligned.  wait / join / destroy as for wnw_h2d_start; the two
 * forms may alternate on one engine.
 */
int wnw_h2d_start_direct(wnw_h2d* x, const void* host_k, const void* host_v,
                         int64_t host_rows, const int32_t* ranges,
                         int64_t n_ranges, const int64_t* group_ranges,
                         int n_groups, void* stage_k, void* stage_v,
                         int64_t stage_rows, void* dev_k, void* dev_v,
                         int64_t dev_rows, int64_t row_bytes, void* stream);
int wnw_h2d_wait(wnw_h2d* x, int group, void* stream);
int wnw_h2d_join(wnw_h2d* x);
/*
 * Set-up costs of the engine paid up front (no reference counterpart: the
 * reference's channel has none to hide): the copy streams of the direct form
 * on the current device, descriptor room for n_ranges ranges per job, the
 * DMA engines a job's copies land on (spans issued in turn on the copy
 * streams while `stream` copies too, twice: the runtime sets up an
 * engine's queue at the first copy it puts there, 6-11 ms on MI355X with
 * every copy submission of the process held meanwhile), the events of the
 * first n_groups groups (1..64) of both staging parities recorded once, and
 * an empty job through the engine's thread on `stream` (the stream later
 * jobs use).  Blocks until done; jobs may follow at once.  Without it the
 * first jobs pay these costs (tens of ms on MI355X) inside the decode
 * steps.
 */
int wnw_h2d_reserve(wnw_h2d* x, int64_t n_ranges, int n_groups, void* stream);

/* ------------------------------------------------------------------------ */
/* Host planner (CPU only; no HIP calls)                                     */
/* ------------------------------------------------------------------------ */
/*
 * Replaces the reference's pybind `Planner` class (src/algorithms/wnw_cpp/
 * code/planner.cpp:16-341; methods bound at :327-341) one call for one
 * method.  It turns each step's top-k chunk lists into the compaction
 * descriptors of wnw_rebuild_append_kv for every layer and gathers the
 * host rows to load into pinned staging.  Arrays are caller-owned int32;
 * "flattened" means row-major over the listed dimensions.  The planner keeps
 * raw pointers to the restore and staging buffers (caller keeps them alive).
 */
typedef struct wnw_planner wnw_planner;

/* Planner(L, H, B, G) (planner.cpp:18-25); NULL on bad dimensions. */
wnw_planner* wnw_planner_create(int num_layers, int num_kv_heads,
                                int batch_size, int group);
void wnw_planner_destroy(wnw_planner* p);
/* set_config (planner.cpp:27-30) */
int wnw_planner_set_config(wnw_planner* p, int top_k_chunks, int eviction_lag);
/* set_seg_count (planner.cpp:32): segments per sample, n = batch */
int wnw_planner_set_seg_count(wnw_planner* p, const int32_t* seg_count,
                              int64_t n);
/* set_chunk_to_segs (planner.cpp:34-42): CSR of chunk -> segments, sample b */
int wnw_planner_set_chunk_to_segs(wnw_planner* p, int b,
                                  const int32_t* flat_segs,
                                  const int32_t* offsets, int64_t num_chunks);
/* set_class_b (planner.cpp:44-48): class-B KV heads of one layer */
int wnw_planner_set_class_b(wnw_planner* p, int layer, const int32_t* kv_heads,
                            int64_t n);
/* set_restore_meta (planner.cpp:50-77): flattened [L][B*H][segments of the
 * sample]; host rows [cpu_s, cpu_e) and resident relative rows [gpu_s,
 * gpu_e) of each offloaded segment, -1 = none / not resident */
int wnw_planner_set_restore_meta(wnw_planner* p, const int32_t* cpu_s,
                                 const int32_t* cpu_e, const int32_t* gpu_s,
                                 const int32_t* gpu_e, int64_t n);
/* set_loaded (planner.cpp:79-84) */
int wnw_planner_set_loaded(wnw_planner* p, int b, const int32_t* segs,
                           int64_t n);
/* set_seq_lens (planner.cpp:86-95): flattened [L][B*H] segment lengths;
 * resets the eviction counters */
int wnw_planner_set_seq_lens(wnw_planner* p, const int32_t* lens, int64_t n);
/* get_loaded_segments (planner.cpp:97-99): writes up to cap ascending
 * segment ids, returns the count (-1 on error) */
int64_t wnw_planner_get_loaded_segments(wnw_planner* p, int b, int32_t* out,
                                        int64_t cap);
/* set_restore_buffers (planner.cpp:101-108): host rows and pinned staging,
 * row_bytes = head_dim * element size */
int wnw_planner_set_restore_buffers(wnw_planner* p, const void* cpu_k,
                                    const void* cpu_v, void* stg_k,
                                    void* stg_v, int64_t cpu_rows,
                                    int64_t stg_rows, int64_t row_bytes);
/* gather_restore (planner.cpp:113-122): copies the last plan's host ranges,
 * in transfer order, to the start of staging (bounds-checked) */
int wnw_planner_gather_restore(wnw_planner* p);
/*
 * compute_and_prepare (planner.cpp:124-306).  topk_idx/topk_off: CSR of the
 * chosen chunks per sample (B + 1 offsets).  Writes [L][N] load_starts,
 * load_lens, new_lens, [L][N+1] cu_new and evict_offsets (per-layer CSR),
 * [L] evict_max and [L+1] evict_layer_ptr (into the global evict list),
 * *any_change, *total_rows (rows to transfer), *n_evict and *n_ranges.  The
 * evict list and the host ranges are read with the two calls below.
 */
int wnw_planner_compute_and_prepare(
    wnw_planner* p, const int32_t* topk_idx, const int32_t* topk_off,
    int32_t* load_starts_2d, int32_t* load_lens_2d, int32_t* cu_new_2d,
    int32_t* new_lens_2d, int32_t* evict_offsets_2d, int32_t* evict_max,
    int32_t* evict_layer_ptr, int32_t* any_change, int64_t* total_rows,
    int64_t* n_evict, int64_t* n_ranges);
/* The (ev_s, ev_e) tensors of compute_and_prepare's result tuple */
int wnw_planner_get_evictions(wnw_planner* p, int32_t* starts, int32_t* ends,
                              int64_t cap);
/* The `ranges` [n, 2] tensor of compute_and_prepare's result tuple */
int wnw_planner_get_ranges(wnw_planner* p, int32_t* ranges, int64_t cap);
/* The last plan's [L+1] layer pointer into `ranges` (layer l's ranges are
 * [layer_ptr[l], layer_ptr[l+1]); all zero when nothing changed).  No
 * counterpart in the reference: the offload channel splits the ranges into
 * groups of layers with it. */
int wnw_planner_get_range_layers(wnw_planner* p, int32_t* layer_ptr,
                                 int64_t cap);
/*
 * The offload channel's plan step in one call: no counterpart in the
 * reference, which plans (planner.cpp:124-306, compute_and_prepare) and then
 * starts its side-stream copy (wnw/code/cache.py:868-881) from Python.
 * topk: [batch, k] chosen chunks per sample, -1 = none (chunk_topk's
 * output; batch = the planner's batch size, and layer_cuts[n_groups] its
 * layer count, else WNW_EINVAL before planning); the planner's outputs
 * and *any_change, *total_rows, *n_evict,
 * *n_ranges as for wnw_planner_compute_and_prepare.  Then, when the plan
 * loads rows and they fit stage_rows and dev_rows, it starts
 * wnw_h2d_start_direct of its ranges on engine x, in n_groups groups of
 * consecutive layers (group g: layers [layer_cuts[g], layer_cuts[g+1]),
 * layer_cuts[n_groups] = the planner's layer count), and sets *started to
 * 1; otherwise *started is 0 and the caller starts the transfer itself
 * (the plan stands either way).  The evict lists and ranges are read with
 * wnw_planner_get_evictions / wnw_planner_get_ranges as after
 * compute_and_prepare.  It saves the caller's round trips between the
 * planner and the engine on the step's critical path.
 */
int wnw_h2d_plan_start_direct(
    wnw_h2d* x, wnw_planner* p, const int32_t* topk, int64_t batch, int64_t k,
    int32_t* load_starts_2d, int32_t* load_lens_2d, int32_t* cu_new_2d,
    int32_t* new_lens_2d, int32_t* evict_offsets_2d, int32_t* evict_max,
    int32_t* evict_layer_ptr, const int32_t* layer_cuts, int n_groups,
    const void* host_k, const void* host_v, int64_t host_rows, void* stage_k,
    void* stage_v, int64_t stage_rows, void* dev_k, void* dev_v,
    int64_t dev_rows, int64_t row_bytes, void* stream, int32_t* any_change,
    int64_t* total_rows, int64_t* n_evict, int64_t* n_ranges,
    int32_t* started);

/* Offload channel                                                           */
/* ------------------------------------------------------------------------ */

/* 1 if the device can read both host arrays directly (pinned, mapped host
 * memory), else 0. */
int wnw_host_rows_readable(const void* host_k, const void* host_v);

/*
 * Device-side gather of planned host rows, in place of the host gather into
 * staging plus the staging copy (planner.cpp:113-122 with
 * wnw_cpp/code/cache.py:287-295; cache.py:868-881 in the Python planner).
 * For r in [r0, r1): rows [ranges[2r], ranges[2r+1]) of host_k / host_v
 * (pinned, host_rows rows of row_bytes) go to rows [dst_off[r],
 * dst_off[r+1]) of out_k / out_v (device, out_rows rows).  ranges (int32
 * [n, 2], the planner's transfer order) and dst_off (int64 [n + 1], prefix
 * sums of the range lengths) are device arrays.  Asynchronous on `stream`;
 * a range outside either array sets WNW_DEVERR_BOUNDS and is skipped.
 * Returns WNW_ENOTSUP when the device cannot read the host arrays.
 */
int wnw_gather_host_rows(const void* host_k, const void* host_v,
                         int64_t host_rows, const int32_t* ranges,
                         const int64_t* dst_off, int64_t r0, int64_t r1,
                         int64_t row_bytes, void* out_k, void* out_v,
                         int64_t out_rows, void* stream);

/* ------------------------------------------------------------------------ */
/* Measurement                                                               */
/* ------------------------------------------------------------------------ */

/*
 * Read-only streaming yardstick: reads `bytes` (a multiple of 8192) from the
 * device buffer `src` with n_wg workgroups of 256 threads, workgroup i
 * reading the i-th contiguous share.  form 2, 4 or 8: per thread two
 * batches of that many 16-byte loads in flight into registers; form 0: the
 * decode attention kernel's load path (1 KB direct-to-LDS loads, two 8 KB
 * steps in flight per wave).  sink (n_wg * 256 uint32) is written only when
 * a workgroup's XOR of what it read equals a fixed constant.  No
 * counterpart in the reference: it measures what a single launch of a given
 * size reaches when it only reads, beside the attention launch.
 */
int wnw_read_stream(const void* src, int64_t bytes, int64_t n_wg, int form,
                    void* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WNW_AMD_H */

// Split-K GQA decode attention over the flat varlen KV layout (gfx950).
//
// Mathematics (reference src/common/kv/fused_attn.py:9-44 and the varlen_attn
// call of src/algorithms/wnw/code/session.py:90-106): for every segment s and
// query head g of its GQA group,
//     out[s, g] = sum_r softmax_r(scale * q[s, g] . K[r]) * V[r]
// over the rows r of segment s.
//
// Work split ("stream-K" over the logical row space).  The logical rows
// [0, cu[n_seg]) -- segment s owns [cu[s], cu[s+1]) -- are cut into P equal
// contiguous ranges, one per workgroup, so every workgroup streams the same
// number of bytes however ragged the segment lengths are.  Logical row j of
// segment s lives at physical row base[s] + (j - cu[s]) (base = cu without
// seg_base), so segments may sit anywhere in the K/V arrays, in any order,
// with any slack between them.  A range may cover the tail of one segment,
// whole segments and the head of another; each (workgroup, segment) overlap
// is a "piece".  A piece that is a whole segment writes the output directly.
// The others write an (m, l, acc) partial to slot (p + s) -- unique because
// ranges and segments are both monotone in the logical row space -- and bump
// the segment's arrival counter; the last arriver merges the partials by
// log-sum-exp and writes the output (no second kernel launch).
//
// Fused append (streaming kernel, APPEND): every segment gains the step's
// new row, new_k/new_v[s], at physical row base[s] + len_old[s] (len_old from
// cu).  The split and the stream cover the old rows only, exactly as without
// the append; the first step of every piece also copies its segment's new
// row into LDS beside q, and the step that ends a segment takes that row as
// one of its own rows.  Such a step always has room for it: a piece that
// ends its segment and holds a multiple of 16 rows starts with a 15-row
// step.  The new rows are stored into the pools, and
// cu_out = cu + arange(n_seg + 1) written, at the end of the kernel, where
// no wait of the stream waits for their acknowledgement.
//
// Three kernels implement this split.  The streaming kernel (bf16/f16, D 64 or
// 128, G <= 8; the default there) gives each wave a quarter of its
// workgroup's range and streams it in 16-row steps straight into LDS; only a
// wave's first and last pieces can be shared, and they are merged through LDS
// after the stream.  The MFMA and VALU kernels walk the workgroup's pieces in
// order, their NW waves taking 32-row (MFMA) or 64-row (VALU) steps of each
// piece round-robin; the wave states are merged through LDS at the end of the
// piece.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "wnw_common.h"

namespace wnw {

static constexpr int kMaxGroup = 16;
static constexpr int kRing = 64;  // LDS cache of segment bounds per workgroup
static constexpr float kNegBig = -1e30f;
static constexpr float kLog2e = 1.4426950408889634f;

struct AttnParams {
  const void* q;        // [n_seg, G, D]
  const void* k;        // [phys_rows, D]
  const void* v;        // [phys_rows, D]
  const int32_t* cu;    // [n_seg + 1] logical offsets (before the append, with APPEND)
  const int64_t* base;  // [n_seg] physical first row, or null (= cu)
  void* out;            // [n_seg, G, D]
  float* part_acc;      // [slots, G, D]
  float* part_ml;       // [slots, G, 2]
  int32_t* counters;    // [n_seg]
  float* lse;           // [n_seg, G, 2] final (max, sum) of each softmax, log2 domain, or null
  int32_t* err;
  uint64_t split_inv;  // ceil(2^64 / (gridDim.x * kSplitWaves)): range bounds without a division
  int64_t phys_rows;   // rows of k / v (bounds)
  int32_t n_seg;
  int32_t G;
  float scale_log2;  // scale * log2(e)
  // Streaming kernel only, null otherwise: the scaled logits (log2 domain)
  // of the audio rows of the segments whose KV head is flagged, for the
  // class-A scoring pass: xlog[(s * G + g) * max_audio + t] for audio row t
  // (relative to audio_s[s / Hkv]) of segment s, t < max_audio.
  float* xlog;
  const int32_t* xmask;    // [Hkv] non-zero: KV head scored
  const int32_t* audio_s;  // [n_seg / Hkv] audio range of each sample, relative to its segments' starts
  const int32_t* audio_e;
  int64_t max_audio;
  int32_t Hkv;
  // APPEND only: the step's rows, the post-append offsets and the capacity
  // of each segment (rows from base[s] it may occupy)
  const void* new_k;   // [n_seg, D]
  const void* new_v;
  int32_t* cu_out;     // [n_seg + 1], must not alias cu
  const int32_t* cap;  // [n_seg]
  // Streaming kernel, direct table only, null otherwise: a previous launch's
  // kept logits (pv_xlog) and normalisers (pv_lse), scored into the class-A
  // accumulator by this launch (AttnPrevScore); audio_s / audio_e /
  // max_audio / Hkv above describe both launches.  Workgroup i takes the
  // 256 tokens of slice i = (sample, block of 256 audio tokens).
  const float* pv_xlog;
  const float* pv_lse;
  uint64_t pv_kvlist;  // the KV heads that launch scored, ascending, 8 bits each (pv_nkv of them)
  int32_t pv_nkv;
  const int32_t* pv_cu;
  const int64_t* pv_base;
  int64_t pv_kv_rows;
  float* pv_acc;
  const int32_t* pv_acc_off;
  int64_t pv_acc_len;
  int32_t pv_nblk;  // 256-token blocks per sample
  int32_t pv_slices;  // samples x pv_nblk (<= the grid)
};

// Deferred scoring of the previous launch's kept logits, before this
// launch's stream.  Workgroup i < the slice count takes slice i = (sample b,
// block of 256 audio tokens), one token per thread; the other workgroups do
// nothing of it.  At the start, beside the segment table: the sample's
// audio range and accumulator offset, lane l < 16 pair l's normalisers
// (pair = (flagged KV head i, query head g), l = i * G + g), lane 16 + i the
// bounds of flagged KV head i's segment, every thread its token's logits
// for all pairs; the accumulator entry once the offset is in.  The weights
// exp2(x - max) / sum are summed over each segment's heads, then over the
// segments, then added to the accumulator entry -- logit_score_kernel's
// order and validity rules, so the sums are bit-identical to that pass --
// and the entry is stored before the first steps are issued.
static constexpr int kPrevLogits = 16;  // pairs per sample the deferred form takes (<= 8 KV heads)
struct PrevLoads {
  float x[kPrevLogits];
  float m, l;           // lane < 16: pair `lane`'s normalisers
  int32_t c0, c1;       // lane 16 + i: flagged KV head i's segment offsets
  int64_t bv;           //   ... and physical first row
  int32_t a0, a1, off;  // the sample's audio range and accumulator offset
  float prior;          // the token's accumulator entry
  // the entry's address, and whether it is stored (bit 0), the offset is
  // valid (bit 1), the slice is its sample's first (bit 3)
  float* dst;
  int32_t flags;
};

// (called by workgroups with a slice only)
__device__ __forceinline__ int prev_slice(const AttnParams&) { return (int)blockIdx.x; }

__device__ __forceinline__ void prev_issue_head(const AttnParams& p, PrevLoads& pl) {
  const int b = prev_slice(p) / p.pv_nblk;
  pl.a0 = p.audio_s[b];
  pl.a1 = p.audio_e[b];
  pl.off = p.pv_acc_off[b];
}

__device__ __forceinline__ void prev_issue_body(const AttnParams& p, int tid, PrevLoads& pl) {
  const int lane = tid & 63;
  const int nb = p.pv_nblk, G = p.G, nkv = p.pv_nkv, Hkv = p.Hkv;
  const int sl = prev_slice(p);
  const int b = sl / nb, blk = sl - b * nb;
  const int np = nkv * G;
  {
    const int t = min(lane, np - 1), i = t / G, g = t - i * G;
    const int s = b * Hkv + (int)((p.pv_kvlist >> (8 * i)) & 0xff);
    pl.m = p.pv_lse[((int64_t)s * G + g) * 2];
    pl.l = p.pv_lse[((int64_t)s * G + g) * 2 + 1];
  }
  {
    const int i = min(max(lane - 16, 0), nkv - 1);
    const int s = b * Hkv + (int)((p.pv_kvlist >> (8 * i)) & 0xff);
    pl.c0 = p.pv_cu[s];
    pl.c1 = p.pv_cu[s + 1];
    pl.bv = p.pv_base ? p.pv_base[s] : 0;
  }
  const int64_t jc = min((int64_t)blk * 256 + tid, p.max_audio - 1);
  // pair t = (flagged KV head i, query head g) reads row (s_i G + g) of the
  // slot's logits; pairs past the count repeat the last one.  Counted, not
  // divided: the row offset advances by max_audio per pair (uniform).
  {
    const int64_t ma = p.max_audio;
    const float* xb = p.pv_xlog + jc;
    int i = 0, g = 0;
    int64_t cur = (int64_t)(b * Hkv + (int)(p.pv_kvlist & 0xff)) * G * ma, last = cur;
#pragma unroll
    for (int t = 0; t < kPrevLogits; ++t) {
      if (t < np) last = cur;
      pl.x[t] = xb[last];
      cur += ma;
      if (++g == G) {
        g = 0;
        ++i;
        cur = (int64_t)(b * Hkv + (int)((p.pv_kvlist >> (8 * min(i, 7))) & 0xff)) * G * ma;
      }
    }
  }
  // the entry, clamped into the accumulator (a bad offset is refused later)
  const int off = __builtin_amdgcn_readfirstlane(pl.off);
  float* dst = p.pv_acc + min(max((int64_t)off + jc, (int64_t)0), p.pv_acc_len - 1);
  pl.prior = *dst;
  pl.dst = dst;
  const int n_audio = pl.a1 - pl.a0;
  const int64_t j = (int64_t)blk * 256 + tid;
  const bool off_ok = off >= 0 && (int64_t)off + n_audio <= p.pv_acc_len;
  pl.flags = ((off_ok && j < n_audio && j < p.max_audio) ? 1 : 0) | (off_ok ? 2 : 0) | (blk == 0 ? 8 : 0);
}

// The token's accumulator entry (at, -1: none) and its new value, from
// loads that have arrived.
__device__ __forceinline__ void prev_finish(const AttnParams& p, int tid, const PrevLoads& pl, float*& dst,
                                            float& total) {
  dst = nullptr;
  total = 0.f;
  const int flags = __builtin_amdgcn_readfirstlane(pl.flags);  // bits 1 and 3 are uniform
  if (!(flags & 2)) {  // the accumulator cannot hold the sample's tokens
    if (tid == 0 && (flags & 8)) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
    return;
  }
  const int G = p.G, nkv = p.pv_nkv;
  const bool has_base = p.pv_base != nullptr;
  // flagged segments whose rows cover the audio range (the others are
  // skipped and reported, as the scoring pass does)
  uint32_t use = 0;
  for (int i = 0; i < nkv; ++i) {
    const int32_t c0 = __builtin_amdgcn_readlane(pl.c0, 16 + i), c1 = __builtin_amdgcn_readlane(pl.c1, 16 + i);
    const uint32_t blo = __builtin_amdgcn_readlane((uint32_t)pl.bv, 16 + i);
    const uint32_t bhi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)pl.bv >> 32), 16 + i);
    const int64_t len = (int64_t)c1 - c0;
    const int64_t base = has_base ? (int64_t)(((uint64_t)bhi << 32) | blo) : (int64_t)c0;
    const bool oob = (pl.a0 < 0) | (pl.a1 > len) | (base < 0) | (base + len > p.pv_kv_rows);
    if (!oob) use |= 1u << i;
    else if (tid == 0 && blockIdx.x == 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
  }
  // lane t holds pair t's normaliser: its reciprocal once per lane, not
  // once per pair and thread
  const float inv_lane = 1.f / pl.l;
  float sum = 0.f, sc = 0.f;
  int i = 0, g = 0;  // pair t = (flagged KV head i, query head g), uniform, counted (no division by G)
#pragma unroll
  for (int t = 0; t < kPrevLogits; ++t) {
    if (i < nkv) {
      const float m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pl.m), t));
      const float inv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv_lane), t));
      // v_exp_f32 directly, as the scoring pass: arguments are <= 0 and
      // weights below 2^-126 (flushed to zero) are negligible
      if ((use >> i) & 1) sc += __builtin_amdgcn_exp2f(pl.x[t] - m) * inv;
      if (g == G - 1) {
        sum += sc;
        sc = 0.f;
      }
    }
    if (++g == G) {
      g = 0;
      ++i;
    }
  }
  if (pl.flags & 1) {
    dst = pl.dst;
    total = pl.prior + sum;
  }
}

// side rows (256 bytes: one dword per lane) of the scored flags and audio
// ranges, per wave (direct table, logits kept)
static constexpr int kXlRows = 3;

// A 4-byte copy per lane from a 64-bit address into LDS (lane i's dword at
// lds_addr + 4 i), counted by vmcnt like the stream's loads.
__device__ __forceinline__ void dma_copy4_a64(const void* gaddr, uint32_t lds_addr) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dword %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(gaddr), "s"(lds_addr)
      : "memory");
}

// A segment is attended when its rows fit both row spaces; every piece of
// logic that decides this (owner outputs, pieces, the stream walk) uses this
// one test, so all workgroups agree on the segments they skip.
__device__ __forceinline__ bool seg_valid(int64_t lo, int64_t len, int64_t b, int64_t R, int64_t KV) {
  return len > 0 && lo >= 0 && lo + len <= R && b >= 0 && b + len <= KV;
}

// Per-workgroup schedule, shared through LDS.
struct SchedLds {
  int64_t R;       // logical rows partitioned: cu[n_seg]
  int64_t KV;      // physical rows (bounds)
  int64_t B0, B1;  // this workgroup's logical row range
  int32_t P;       // effective number of workgroups (<= R)
  int32_t s_first, s_last;
  int32_t is_last;  // combine flag broadcast
  // Set when the table is not in layout order (WNW_DEVERR_ORDER).  Every
  // workgroup reads the whole table and comes to the same verdict, so all of
  // them then skip the split-K hand-off: no arrival counter is touched and
  // the workspace stays valid for the next launch.
  int32_t order_bad;
  alignas(16) int32_t hdr[16][4];  // streaming kernel: merge slot headers (segment, length, logical start lo, hi)
  int64_t ring_base[kRing];  // physical first row
  int32_t ring_lo[kRing];    // logical first row
  int32_t ring_len[kRing];
  int32_t ring_cap[kRing];   // with APPEND: capacity
  int32_t ring_a0[kRing];    // with xlog: audio start of the segment
  int32_t ring_alen[kRing];  // with xlog: audio rows kept (0: segment not scored)
};

// The logical rows [0, R) are split over P workgroups, [floor(p R / P),
// floor((p + 1) R / P)) for workgroup p, and each workgroup's range over its
// kSplitWaves waves the same way (unit u = p * kSplitWaves + w of
// P * kSplitWaves), so wave and workgroup bounds agree.
static constexpr int kSplitWaves = 4;

// floor(u R / U) for U = gridDim.x * kSplitWaves with inv = ceil(2^64 / U):
// the high half of u R * inv, exact for n = u R < 2^64 / U (R < 2^32, U <
// 2^14): the product overshoots n / U by less than n / 2^64 < 1 / U, and
// the fraction of n / U is at most 1 - 1 / U.
__device__ __forceinline__ int64_t unit_start(int64_t u, int64_t R, uint64_t inv) {
  return (int64_t)__umul64hi((uint64_t)(u * R), inv);
}
// The workgroup whose row range holds logical row j (P <= R):
// floor(x / R) for x = (j + 1) P - 1, by a correctly rounded double division
// instead of a 64-bit integer one (~170 instructions).  Exact for
// 0 <= x < 2^52: when x / R = n - d is not an integer, d >= 1 / R, while
// the rounding error is at most n 2^-53 < 1 / R (n R <= x + R < 2^53), so the
// quotient never rounds up to n.  Here x < 2^31 * 2^14.
__device__ __forceinline__ int64_t owner_of(int64_t j, int64_t R, int64_t P) {
  return (int64_t)floor((double)((j + 1) * P - 1) / (double)R);
}
__device__ __forceinline__ int64_t effective_wgs(int64_t R, int64_t grid = gridDim.x) {
  return R > 0 ? min(grid, R) : 0;
}
// Start of split unit u (of P * kSplitWaves) for R rows: the reciprocal
// when every workgroup of the grid takes part (R >= gridDim.x), else a
// division (tiny launches; marked unlikely, so it is laid out of the
// prologue's path).
__device__ __forceinline__ int64_t split_start(int64_t u, int64_t R, int64_t P, uint64_t inv,
                                              int64_t grid = gridDim.x) {
  if (__builtin_expect(P == grid && inv != 0, 1)) return unit_start(u, R, inv);
  return (u * R) / (P * kSplitWaves);
}
// This workgroup's logical row range [B0, B1) for R rows over P workgroups.
__device__ __forceinline__ void wg_range(int64_t R, int64_t P, uint64_t inv, int64_t& B0, int64_t& B1,
                                         int64_t grid = gridDim.x) {
  const int64_t pid = blockIdx.x;
  if (pid >= P) {
    B0 = B1 = 0;
    return;
  }
  B0 = split_start(pid * kSplitWaves, R, P, inv, grid);
  B1 = split_start((pid + 1) * kSplitWaves, R, P, inv, grid);
}

// APPEND, a segment with no old rows: its only row is the new one, so every
// head's output is that V row (softmax weight 1) and its statistics are
// (logit, 1).  One thread does it all; rare, since a decode-time segment
// holds its earlier steps' rows.  With store_row the row also goes into the
// pools at physical row b.
template <typename T>
__device__ __forceinline__ void append_only_segment(const AttnParams& p, int D, int s, int64_t b, bool store_row) {
  const int G = p.G;
  const T* nk = (const T*)p.new_k + (int64_t)s * D;
  const T* nv = (const T*)p.new_v + (int64_t)s * D;
  const T* q = (const T*)p.q + (int64_t)s * G * D;
  for (int g = 0; g < G; ++g) {
    float dot = 0.f;
    for (int e = 0; e < D; ++e) dot += Elem<T>::to_f32(q, g * D + e) * Elem<T>::to_f32(nk, e);
    for (int e = 0; e < D; ++e) store_elem<T>(p.out, ((int64_t)s * G + g) * D + e, Elem<T>::to_f32(nv, e));
    if (p.lse) {
      gptr_w<float>(p.lse)[((int64_t)s * G + g) * 2] = dot * p.scale_log2;
      gptr_w<float>(p.lse)[((int64_t)s * G + g) * 2 + 1] = 1.f;
    }
  }
  if (store_row) {
    WNW_GLOBAL uint16_t* kd = gptr_w<uint16_t>(const_cast<void*>(p.k)) + b * D;
    WNW_GLOBAL uint16_t* vd = gptr_w<uint16_t>(const_cast<void*>(p.v)) + b * D;
    for (int e = 0; e < D; ++e) {
      kd[e] = ((const uint16_t*)nk)[e];
      vd[e] = ((const uint16_t*)nv)[e];
    }
  }
}

// Workgroup prologue: one pass over cu / base (all threads, independent
// loads) finds the segments whose logical rows overlap this workgroup's
// range, checks the table, and writes the outputs of empty segments (zeros)
// and of invalid ones (NaN) owned by this workgroup (segment i -> workgroup
// i % grid).  With APPEND, an empty segment's output is its new row (the
// owner stores that row into the pool too) and workgroup 0 writes cu_out.
template <typename T, int NT, bool XL = false, bool APPEND = false>
__device__ __forceinline__ void schedule(const AttnParams& p, int D, SchedLds& sl) {
  const int tid = threadIdx.x;
  const int N = p.n_seg;
  if (tid == 0) {
    sl.s_first = 0x7fffffff;
    sl.s_last = -1;
    sl.order_bad = 0;
  }
  const int64_t KV = p.phys_rows;
  const int64_t pid = blockIdx.x;
  int32_t lo[4], hi[4], cp[4];
  int64_t bs[4];
  int32_t xm[4], xa[4], xe[4];  // with xlog: KV-head flag, audio range
  const WNW_GLOBAL int32_t* cu = gptr<int32_t>(p.cu);
  const WNW_GLOBAL int64_t* basep = gptr<int64_t>(p.base);
  auto load_chunk = [&](int i0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * NT + tid;
      lo[u] = hi[u] = cp[u] = 0;
      bs[u] = 0;
      xm[u] = xa[u] = xe[u] = 0;
      if (XL && i < N) {
        xm[u] = gptr<int32_t>(p.xmask)[i % p.Hkv];
        xa[u] = gptr<int32_t>(p.audio_s)[i / p.Hkv];
        xe[u] = gptr<int32_t>(p.audio_e)[i / p.Hkv];
      }
      if (i < N) {
        lo[u] = cu[i];
        hi[u] = cu[i + 1];
        if (p.base) bs[u] = basep[i];
        if (APPEND) cp[u] = gptr<int32_t>(p.cap)[i];
      }
    }
  };
  // Ring entries are written only for segments that overlap this range;
  // an empty or invalid segment between s_first and s_last must read as
  // empty (length 0), not as what an earlier kernel left in LDS.
  if (tid < kRing) {
    sl.ring_base[tid] = 0;
    sl.ring_lo[tid] = 0;
    sl.ring_len[tid] = 0;
    sl.ring_cap[tid] = 0;
    if (XL) {
      sl.ring_a0[tid] = 0;
      sl.ring_alen[tid] = 0;
    }
  }
  // The loads of the first chunk (and of cu[N], the end of the logical rows
  // the split covers) are issued before the barrier: one global round trip
  // for n_seg <= 4 * NT.
  const int32_t cu_end = cu[N];
  load_chunk(0);
  __syncthreads();
  const int64_t R = max((int64_t)0, (int64_t)cu_end);
  const int64_t P = effective_wgs(R);
  const bool active = pid < P;
  int64_t B0, B1;
  wg_range(R, P, p.split_inv, B0, B1);
  for (int i0 = 0; i0 < N; i0 += 4 * NT) {
    if (i0 > 0) load_chunk(i0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * NT + tid;
      if (i >= N) continue;
      if (__builtin_expect(APPEND && pid == 0, 0)) {  // post-append offsets (one workgroup)
        WNW_GLOBAL int32_t* co = gptr_w<int32_t>(p.cu_out);
        co[i] = lo[u] + i;
        if (i == N - 1) co[N] = hi[u] + N;
      }
      int64_t len = (int64_t)hi[u] - lo[u];
      const int64_t b = p.base ? bs[u] : (int64_t)lo[u];
      bool neg = false;
      if (__builtin_expect(len < 0, 0)) {  // corrupt offsets: treated as an empty segment
        raise_device_error(p.err, WNW_DEVERR_ORDER);
        sl.order_bad = 1;
        len = 0;
        neg = true;
      } else if (__builtin_expect(APPEND && len + 1 > cp[u], 0)) {
        raise_device_error(p.err, WNW_DEVERR_CAPACITY);
      }
      const bool owner = (i % (int)gridDim.x) == (int)pid;
      // rare paths (error, empty segments) hinted so, to keep them out of
      // the pass's straight line: the pass runs once per launch, with the
      // instruction cache cold
      if (__builtin_expect(!seg_valid(lo[u], len, b, R, KV), 0)) {
        if (len != 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
        if (APPEND && len == 0 && !neg) {  // only the new row: it is the output
          if (owner) append_only_segment<T>(p, D, i, b, len + 1 <= cp[u] && b >= 0 && b < KV);
          continue;
        }
        if (owner) {
          const float fill = len == 0 ? 0.f : __int_as_float(0x7fc00000);
          for (int e = 0; e < p.G * D; ++e) store_elem<T>(p.out, (int64_t)i * p.G * D + e, fill);
          if (p.lse) {
            WNW_GLOBAL float* ls = gptr_w<float>(p.lse) + (int64_t)i * p.G * 2;
            for (int g = 0; g < p.G; ++g) {
              ls[2 * g] = len == 0 ? kNegBig : fill;
              ls[2 * g + 1] = len == 0 ? 0.f : fill;
            }
          }
        }
        continue;
      }
      if (active && lo[u] < B1 && lo[u] + len > B0) {
        atomicMin(&sl.s_first, i);
        atomicMax(&sl.s_last, i);
        sl.ring_base[i % kRing] = b;
        sl.ring_lo[i % kRing] = lo[u];
        sl.ring_len[i % kRing] = (int32_t)len;
        sl.ring_cap[i % kRing] = cp[u];
        if (XL) {
          sl.ring_a0[i % kRing] = xa[u];
          sl.ring_alen[i % kRing] = xm[u] ? (int32_t)max((int64_t)0, min((int64_t)xe[u] - xa[u], p.max_audio)) : 0;
        }
      }
    }
  }
  if (tid == 0) {
    sl.R = R;
    sl.KV = KV;
    sl.P = (int32_t)P;
    sl.B0 = B0;
    sl.B1 = B1;
  }
  __syncthreads();
}

struct Piece {
  int64_t seg_lo;    // logical first row of the segment
  int64_t seg_len;
  int64_t phys;      // physical row of the piece's first row
  int32_t nrows;     // rows in the piece
  bool whole;
  bool skip;         // no valid rows of this segment in the workgroup's range
};

// Workgroup-uniform values read from LDS land in VGPRs; broadcasting them
// from lane 0 puts them in SGPRs, so addresses and loop bounds derived from
// them stay scalar.
__device__ __forceinline__ int32_t uni(int32_t x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ int64_t uni(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// The MFMA and VALU kernels (no append): segment s's piece of this
// workgroup's logical range.
__device__ __forceinline__ Piece make_piece(const AttnParams& p, const SchedLds& sl, int s) {
  Piece pc;
  int64_t b, lo, len;
  if (sl.s_last - sl.s_first < kRing) {
    b = sl.ring_base[s % kRing];
    lo = sl.ring_lo[s % kRing];
    len = sl.ring_len[s % kRing];
  } else {
    const int64_t c0 = gptr<int32_t>(p.cu)[s], c1 = gptr<int32_t>(p.cu)[s + 1];
    b = p.base ? gptr<int64_t>(p.base)[s] : c0;
    lo = c0;
    len = c1 - c0;
  }
  b = uni(b);
  lo = uni(lo);
  len = uni(len);
  pc.seg_lo = lo;
  pc.seg_len = len;
  // Invalid or empty segments inside [s_first, s_last] are skipped here and
  // handled by their owner in schedule(); the condition matches it exactly.
  const int64_t B0 = uni(sl.B0), B1 = uni(sl.B1);
  pc.skip = !(seg_valid(lo, len, b, uni(sl.R), uni(sl.KV)) && lo < B1 && lo + len > B0);
  const int64_t a = max(lo, B0), e = min(lo + len, B1);
  pc.whole = (a == lo) && (e == lo + len);
  pc.phys = b + (a - lo);
  pc.nrows = pc.skip ? 0 : (int32_t)(e - a);
  return pc;
}

// Agent-scope coherent accesses (global_{load,store} sc1 on gfx950): they
// bypass the non-coherent per-XCD L2 state, so a partial written by one
// XCD is visible to a reader on another without any L2 write-back or
// invalidation of the whole cache (which a release/acquire fence costs).
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(gptr_w<float>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent2(float* p, float a, float b) {
  const uint64_t v = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
  __hip_atomic_store(gptr_w<uint64_t>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// s_waitcnt vmcnt(0): every vector memory access of this wave has completed.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// s_waitcnt vmcnt(n) (expcnt and lgkmcnt not waited on), n < 64.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | ((N & 0x30) << 10));
}

// Last-arriver merge of the np partials of one segment (slots s0 ..
// s0 + np - 1) into the output, by threads t = 0 .. nt - 1.  Every thread
// owns 4 consecutive elements of one head and reads, for a chunk of partials
// at a time, their (m, l) pairs and its accumulator quad: one memory round
// trip per chunk, no LDS and no barriers.  The reads are buffer loads with
// the sc1 policy (the agent-coherent form of a load on gfx950), one 16-byte
// and one 8-byte load per partial at a scalar offset from the segment's
// first slot.  Chunks are folded in slot order with the usual max
// rescaling, so the result is deterministic.
template <typename T>
__device__ __forceinline__ void combine_pieces(const AttnParams& p, int D, int64_t s0, int np, int64_t s, int t,
                                               int nt) {
  // the segment and its slots are wave-uniform: scalar, so the buffer
  // descriptors below live in SGPRs
  s0 = uni(s0);
  np = uni(np);
  s = uni(s);
  constexpr int QC = 16;             // partials per round trip
  constexpr int kSc1 = 16;           // buffer cache policy: sc1
  constexpr int kRsrc3 = 0x00020000;  // buffer descriptor word 3 (raw 32-bit data) on gfx9
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const int G = p.G;
  const int GD = G * D;
  const int GD4 = GD / 4;
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc(p.part_acc + s0 * GD, 0, np * GD * 4, kRsrc3);
  const __amdgpu_buffer_rsrc_t rm =
      __builtin_amdgcn_make_buffer_rsrc(p.part_ml + s0 * G * 2, 0, np * G * 8, kRsrc3);
  for (int i4 = t; i4 < GD4; i4 += nt) {
    const int g = (4 * i4) / D;
    float M = kNegBig, L = 0.f;
    f32x4 A = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int q0 = 0; q0 < np; q0 += QC) {
      f32x4 a[QC];
      u32x2 ml[QC];
#pragma unroll
      for (int k = 0; k < QC; ++k) {
        a[k] = f32x4{0.f, 0.f, 0.f, 0.f};
        ml[k] = u32x2{0u, 0u};
        if (q0 + k < np) {  // wave-uniform: no wait between the loads
          a[k] = __builtin_bit_cast(f32x4,
                                    __builtin_amdgcn_raw_buffer_load_b128(ra, i4 * 16, (q0 + k) * GD * 4, kSc1));
          ml[k] = __builtin_amdgcn_raw_buffer_load_b64(rm, g * 8, (q0 + k) * G * 8, kSc1);
        }
      }
      float Mc = M;
#pragma unroll
      for (int k = 0; k < QC; ++k)
        if (q0 + k < np) Mc = fmaxf(Mc, __uint_as_float(ml[k].x));
      const float so = __builtin_amdgcn_exp2f(M - Mc);
      L *= so;
      A *= so;
#pragma unroll
      for (int k = 0; k < QC; ++k) {
        if (q0 + k >= np) continue;
        const float wk = __builtin_amdgcn_exp2f(__uint_as_float(ml[k].x) - Mc);
        L += __uint_as_float(ml[k].y) * wk;
        A += a[k] * wk;
      }
      M = Mc;
    }
    const float inv = 1.f / L;
    const float o4[4] = {A[0] * inv, A[1] * inv, A[2] * inv, A[3] * inv};
    store_quad<T>(p.out, s * GD + 4 * i4, o4);
    if (p.lse && (4 * i4) % D == 0) {
      gptr_w<float>(p.lse)[(s * G + g) * 2] = M;
      gptr_w<float>(p.lse)[(s * G + g) * 2 + 1] = L;
    }
  }
}

// Pieces (workgroups) of the segment at logical rows [seg_lo, seg_lo + seg_len).
__device__ __forceinline__ void piece_range(const SchedLds& sl, int64_t seg_lo, int64_t seg_len, int64_t& p_first,
                                            int64_t& p_last) {
  const int64_t R = sl.R, P = sl.P;
  p_first = min(max(owner_of(seg_lo, R, P), (int64_t)0), P - 1);
  p_last = min(max(owner_of(seg_lo + seg_len - 1, R, P), p_first), P - 1);
}

// Arrival of this workgroup's partial of segment s (already written with
// agent-coherent stores and waited for, followed by a barrier): bump the
// segment's counter and return whether this was the last piece.  One thread.
__device__ __forceinline__ bool arrive(const AttnParams& p, const SchedLds& sl, int64_t seg_lo, int64_t seg_len,
                                      int s) {
  int64_t p_first, p_last;
  piece_range(sl, seg_lo, seg_len, p_first, p_last);
  const int old =
      __hip_atomic_fetch_add(gptr_w<int32_t>(p.counters) + s, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return old == (int)(p_last - p_first);
}

// The merge of segment s from its np pieces, the first held by workgroup
// p_first (by threads t = 0 .. nt - 1), and the reset of its counter for the
// next launch.
template <typename T>
__device__ __forceinline__ void combine_from(const AttnParams& p, int D, int64_t p_first, int np, int s, int t,
                                             int nt) {
  combine_pieces<T>(p, D, p_first + s /* slot of the first piece */, np, s, t, nt);
  if (t == 0) __hip_atomic_store(gptr_w<int32_t>(p.counters) + s, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The last arriver of segment s merges every partial into the output (by
// threads t = 0 .. nt - 1 of the workgroup) and resets the counter for the
// next launch.  No LDS is used.
template <typename T>
__device__ __forceinline__ void combine_segment(const AttnParams& p, int D, const SchedLds& sl, int64_t seg_lo,
                                                int64_t seg_len, int s, int t, int nt) {
  int64_t p_first, p_last;
  piece_range(sl, seg_lo, seg_len, p_first, p_last);
  combine_from<T>(p, D, p_first, (int)(p_last - p_first + 1), s, t, nt);
}

// Arrival of this workgroup's partial of segment s followed, on the last
// arrival, by the merge.  Called by all threads.
template <typename T, int NT>
__device__ __forceinline__ void arrive_and_combine(const AttnParams& p, int D, SchedLds& sl, int64_t seg_lo,
                                                   int64_t seg_len, int s) {
  if (threadIdx.x == 0) sl.is_last = !sl.order_bad && arrive(p, sl, seg_lo, seg_len, s);
  __syncthreads();
  if (!sl.is_last) return;  // workgroup-uniform
  combine_segment<T>(p, D, sl, seg_lo, seg_len, s, threadIdx.x, NT);
}

// Merge the NW wave states in LDS (layout: ml[w][g] = (m, l),
// acc[w][g][d]), then either write the final output (whole segment) or a
// partial, and run the last-arriver combine.  Called by all threads.
//
// Hand-off protocol of a split segment: every thread stores its share of
// the partial with agent-coherent stores and waits for their completion;
// after the barrier one thread bumps the segment's counter (relaxed atomic,
// coherent across XCDs).  The workgroup that sees count == pieces - 1 is the
// last arriver: all other partials were complete before their counters
// moved, so its agent-coherent loads see them.  It resets the counter for
// the next launch.
template <typename T, int NT, int NW>
__device__ __forceinline__ void finish_piece(const AttnParams& p, int D, SchedLds& sl, const Piece& pc, int s,
                                             float* mrg_ml, float* mrg_acc) {
  const int tid = threadIdx.x;
  const int G = p.G;
  const int GD = G * D;
  if (pc.whole) {
    T* o = (T*)p.out + (int64_t)s * GD;
    for (int idx = tid; idx < GD; idx += NT) {
      const int g = idx / D;
      float M = kNegBig;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, mrg_ml[(w * kMaxGroup + g) * 2]);
      float L = 0.f, A = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float sc = exp2f(mrg_ml[(w * kMaxGroup + g) * 2] - M);
        L += mrg_ml[(w * kMaxGroup + g) * 2 + 1] * sc;
        A += mrg_acc[(w * kMaxGroup + g) * D + (idx - g * D)] * sc;
      }
      store_elem<T>(o, idx, A / L);
      if (p.lse && idx - g * D == 0) {
        gptr_w<float>(p.lse)[((int64_t)s * G + g) * 2] = M;
        gptr_w<float>(p.lse)[((int64_t)s * G + g) * 2 + 1] = L;
      }
    }
    __syncthreads();  // LDS reuse by the next piece
    return;
  }
  const int64_t slot = (int64_t)blockIdx.x + s;
  float* pa = p.part_acc + slot * GD;
  float* pm = p.part_ml + slot * G * 2;
  for (int idx = tid; idx < GD; idx += NT) {
    const int g = idx / D;
    float M = kNegBig;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, mrg_ml[(w * kMaxGroup + g) * 2]);
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float sc = exp2f(mrg_ml[(w * kMaxGroup + g) * 2] - M);
      L += mrg_ml[(w * kMaxGroup + g) * 2 + 1] * sc;
      A += mrg_acc[(w * kMaxGroup + g) * D + (idx - g * D)] * sc;
    }
    st_agent(pa + idx, A);
    if (idx - g * D == 0) {
      st_agent(pm + g * 2, M);
      st_agent(pm + g * 2 + 1, L);
    }
  }
  wait_vmem();
  __syncthreads();
  arrive_and_combine<T, NT>(p, D, sl, pc.seg_lo, pc.seg_len, s);
}

// ---------------------------------------------------------------------------
// MFMA kernel (bf16 / f16 K, V, q; D = 64 or 128; G <= 16)
// ---------------------------------------------------------------------------
// Per wave and 32-row step (two 16-row tiles h = 0, 1):
//   S^T tile  = K_tile (16 x D, rows permuted by sigma) x q^T (D x 16)
//               via D/32 v_mfma_f32_16x16x32; lane l holds
//               S[row 4i + l/16 of the tile][g = l % 16], i = 0..3.
//   O^T      += V^T (D x 32 rows) x P^T (32 rows x 16)
//               via D/16 v_mfma_f32_16x16x32, with P split as hi + lo bf16
//               parts so that the weights keep ~16 mantissa bits.
// The S output layout is exactly the P^T operand layout (rows in-lane,
// g = l % 16), so P never leaves the lane; V^T is read from a padded LDS copy
// of the V rows (row pitch 288 B keeps the transposed u16 reads free of bank
// conflicts).  The accumulator lane (q, g) holds O[g][16t + 4q + i], so the
// online-softmax rescale by alpha[g] stays in-lane.
static constexpr int kStepRows = 32;

template <typename T>
struct MfmaOps;
template <>
struct MfmaOps<bf16_t> {
  __device__ static f32x4 mma(const u32x4& a, const u32x4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static uint32_t from_f32(float x) { return f32_to_bf16_bits(x); }
  __device__ static float to_f32(uint32_t h) { return __uint_as_float(h << 16); }
};
template <>
struct MfmaOps<f16_t> {
  __device__ static f32x4 mma(const u32x4& a, const u32x4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static uint32_t from_f32(float x) { return f32_to_f16_bits(x); }
  __device__ static float to_f32(uint32_t h) { return f16_bits_to_f32(h); }
};

template <int D, int NW>
struct MfmaLds {
  static constexpr int kStep = kStepRows * D * 2;  // one staged step of V
  static constexpr int kStage = NW * 2 * kStep;     // two per wave
  static constexpr int kMerge = NW * kMaxGroup * (D + 2) * 4;
  static constexpr int kBytes = kStage > kMerge ? kStage : kMerge;
};


template <typename T, int D, int NW>
__global__ __launch_bounds__(NW * 64, 2) void attn_mfma_kernel(AttnParams p) {
  constexpr int NT = NW * 64;
  constexpr int NC = D / 32;            // QK k-chunks
  constexpr int NTD = D / 16;           // PV output tiles
  constexpr int CPR = D / 8;            // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;         // rows per wave-wide LDS load
  constexpr int VO = kStepRows / RPI;   // V load instructions per step
  constexpr int KO = 2 * NC;            // K load instructions per step
  constexpr int VSTEP = MfmaLds<D, NW>::kStep;
  __shared__ SchedLds sl;
  __shared__ __attribute__((aligned(16))) uint8_t lds[MfmaLds<D, NW>::kBytes];

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index (uniform)
  const int lane = tid & 63;
  const int lq = lane >> 4;   // lane quarter
  const int lc = lane & 15;   // lane column (g for S/P, m for MFMA A rows)
  // K row of this lane inside a 16-row tile (rows permuted so that lane
  // quarter q ends up with rows 4i + q of the tile in the S output).
  const int krow = (lc & 3) * 4 + (lc >> 2);
  uint8_t* vbuf0 = lds + w * 2 * VSTEP;
  uint8_t* vbuf1 = vbuf0 + VSTEP;
  const WNW_GLOBAL uint16_t* kp = gptr<uint16_t>(p.k);
  const WNW_GLOBAL uint16_t* vp = gptr<uint16_t>(p.v);

  // Loads address a uniform base (SGPRs) plus a 32-bit per-lane offset, so
  // they use the scalar-base form and keep few VGPRs.
  // K: two register buffers per wave (MFMA A layout, straight from memory).
  auto issue_k = [&](u32x4 (&kb)[2][NC], const WNW_GLOBAL uint16_t* base, int row0, int valid) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int r = 16 * h + krow;
      r = r < valid ? r : valid - 1;
      const uint32_t off = (uint32_t)(row0 + r) * D + 8 * lq;
#pragma unroll
      for (int c = 0; c < NC; ++c)
        kb[h][c] = __builtin_nontemporal_load((const WNW_GLOBAL u32x4*)(base + off + 32 * c));
    }
  };
  // V: two LDS buffers per wave, filled by direct global->LDS loads.  Row r
  // is stored row-major with its 16-byte chunks XOR-swizzled by 2 * (r % 4),
  // so the transposed reads below (four consecutive rows per lane quarter)
  // hit distinct banks without padding.
  auto issue_v = [&](uint8_t* vb, const WNW_GLOBAL uint16_t* base, int row0, int valid) {
#pragma unroll
    for (int u = 0; u < VO; ++u) {
      const int r = u * RPI + lane / CPR;
      const int c = (lane % CPR) ^ (2 * (r & 3));
      const int rr = r < valid ? r : valid - 1;
      const uint32_t off = (uint32_t)(row0 + rr) * D + 8 * c;
      __builtin_amdgcn_global_load_lds(base + off, vb + u * 1024, 16, 0, 2 /* nt */);
    }
  };

  // Offsets first, then q, then the K/V stream: the small loads every later
  // step depends on are queued ahead of the bulk traffic, not behind it.
  schedule<T, NT>(p, D, sl);
  if (sl.s_first > sl.s_last) return;
  const int G = p.G;

  const int s_first = uni(sl.s_first), s_last = uni(sl.s_last);
  for (int s = s_first; s <= s_last; ++s) {
    const Piece pc = make_piece(p, sl, s);
    if (pc.skip) continue;  // workgroup-uniform
    const int nsteps = (pc.nrows + kStepRows - 1) / kStepRows;
    auto step_rows = [&](int st) { return min(kStepRows, pc.nrows - st * kStepRows); };
    u32x4 kA[2][NC], kB[2][NC];
    // q^T operand: lane (lq, lc) holds q[g = lc][32c + 8lq .. +8].
    u32x4 qb[NC];
    {
      const WNW_GLOBAL uint16_t* qs = gptr<uint16_t>(p.q) + (int64_t)s * G * D;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (lc < G)
          qb[c] = *(const WNW_GLOBAL u32x4*)(qs + lc * D + 32 * c + 8 * lq);
        else
          qb[c] = u32x4{0, 0, 0, 0};
      }
    }
    float m_run = kNegBig, l_run = 0.f;
    f32x4 acc[NTD];
#pragma unroll
    for (int t = 0; t < NTD; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // piece base pointers (uniform); row offsets within a piece fit in 32 bits
    const WNW_GLOBAL uint16_t* kpc = kp + pc.phys * D;
    const WNW_GLOBAL uint16_t* vpc = vp + pc.phys * D;
    __builtin_amdgcn_sched_barrier(0);
    if (w < nsteps) {
      issue_k(kA, kpc, w * kStepRows, step_rows(w));
      issue_v(vbuf0, vpc, w * kStepRows, step_rows(w));
    }
    if (w + NW < nsteps) {
      issue_k(kB, kpc, (w + NW) * kStepRows, step_rows(w + NW));
      issue_v(vbuf1, vpc, (w + NW) * kStepRows, step_rows(w + NW));
    }
    __builtin_amdgcn_sched_barrier(0);

    // One step: QK from the K registers, refill them two steps ahead,
    // softmax, wait for this step's V, PV from LDS, refill the V buffer two
    // steps ahead.  In-order issue (pinned by sched_barrier) makes the number
    // of vector-memory ops issued after this step's V loads exactly
    // (KO + VO) * has1 + KO * has2, which is what the wait allows in flight.
    auto process = [&](u32x4 (&kb)[2][NC], uint8_t* vb, int st) {
      const int valid = step_rows(st);
      const bool has1 = st + NW < nsteps;
      const bool has2 = st + 2 * NW < nsteps;
      f32x4 sacc[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        sacc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c) sacc[h] = MfmaOps<T>::mma(kb[h][c], qb[c], sacc[h]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (has2) issue_k(kb, kpc, (st + 2 * NW) * kStepRows, step_rows(st + 2 * NW));
      __builtin_amdgcn_sched_barrier(0);

      // online softmax for g = lc over the 8 rows this lane holds
      float sv[2][4];
      float mx = kNegBig;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 16 * h + 4 * i + lq;
          const float x = r < valid ? sacc[h][i] * p.scale_log2 : -INFINITY;
          sv[h][i] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, swap16(mx));
      mx = fmaxf(mx, swap32(mx));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = exp2f(m_run - m_new);
      m_run = m_new;
      float psum = 0.f;
      uint32_t phi[2][4], plo[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pv = exp2f(sv[h][i] - m_new);
          psum += pv;
          const uint32_t hb = MfmaOps<T>::from_f32(pv);
          phi[h][i] = hb;
          plo[h][i] = MfmaOps<T>::from_f32(pv - MfmaOps<T>::to_f32(hb));
        }
      l_run = l_run * alpha + psum;
#pragma unroll
      for (int t = 0; t < NTD; ++t) acc[t] *= alpha;
      // P^T operand: k-slot (lq, j): j < 4 -> tile 0 row 4j + lq, else tile 1
      u32x4 bh, bl;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        bh[j] = phi[0][2 * j] | (phi[0][2 * j + 1] << 16);
        bh[2 + j] = phi[1][2 * j] | (phi[1][2 * j + 1] << 16);
        bl[j] = plo[0][2 * j] | (plo[0][2 * j + 1] << 16);
        bl[2 + j] = plo[1][2 * j] | (plo[1][2 * j + 1] << 16);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (has1) {
        if (has2)
          wait_vmcnt<2 * KO + VO>();
        else
          wait_vmcnt<KO + VO>();
      } else {
        wait_vmcnt<0>();
      }
      __builtin_amdgcn_sched_barrier(0);
      // O^T += V^T P^T, V^T read transposed from the staged rows: element
      // (row r, dim d) is at r * 2D + ((d / 8) ^ (2 (r % 4))) * 16 + (d % 8) * 2,
      // and every row this lane reads has r % 4 == lq.
#pragma unroll
      for (int t = 0; t < NTD; ++t) {
        const uint8_t* col = vb + (((2 * t + (lc >> 3)) ^ (2 * lq)) * 16) + (lc & 7) * 2;
        uint32_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int r = (j < 4) ? (4 * j + lq) : (16 + 4 * (j - 4) + lq);
          e[j] = *(const uint16_t*)(col + r * (2 * D));
        }
        u32x4 a;
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = e[2 * j] | (e[2 * j + 1] << 16);
        acc[t] = MfmaOps<T>::mma(a, bh, acc[t]);
        acc[t] = MfmaOps<T>::mma(a, bl, acc[t]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (has2) issue_v(vb, vpc, (st + 2 * NW) * kStepRows, step_rows(st + 2 * NW));
      __builtin_amdgcn_sched_barrier(0);
    };

    for (int st = w; st < nsteps; st += 2 * NW) {
      process(kA, vbuf0, st);
      if (st + NW < nsteps) process(kB, vbuf1, st + NW);
    }
    // l over the lane quarters (same g)
    l_run += swap16(l_run);
    l_run += swap32(l_run);

    __syncthreads();  // all waves done with their V staging (aliased below)
    float* mrg_ml = (float*)lds;                        // [NW][16][2]
    float* mrg_acc = (float*)lds + NW * kMaxGroup * 2;  // [NW][16][D]
    if (lc < G) {
      if (lq == 0) {
        mrg_ml[(w * kMaxGroup + lc) * 2] = m_run;
        mrg_ml[(w * kMaxGroup + lc) * 2 + 1] = l_run;
      }
#pragma unroll
      for (int t = 0; t < NTD; ++t)
        *(f32x4*)(mrg_acc + (w * kMaxGroup + lc) * D + 16 * t + 4 * lq) = acc[t];
    }
    __syncthreads();
    finish_piece<T, NT, NW>(p, D, sl, pc, s, mrg_ml, mrg_acc);
  }
  wait_vmcnt<0>();
}

// ---------------------------------------------------------------------------
// Streaming MFMA kernel (bf16 / f16 K, V, q; D = 64 or 128; G <= 8)
// ---------------------------------------------------------------------------
// Each wave owns a contiguous quarter of its workgroup's row range and walks
// the segments overlapping it in 16-row steps, two steps in flight, without
// stopping at segment boundaries.  The K and V rows and the segment's q of a
// step are copied straight into the wave's LDS buffers by direct global->LDS
// loads issued from inline assembly, so the compiler tracks none of them and
// inserts no memory waits of its own; every wait below is explicit, with a
// count fixed per step (K, q, V: NI + QD + NI loads, in that order).
//
// Per step (16 rows):
//   S^T (16 rows x 16 heads) = K_tile x q^T: D/32 v_mfma_f32_16x16x32, the
//       K operand read row by row from LDS (16-byte chunks XOR-swizzled by
//       the row, so the 16 rows of one read hit distinct banks);
//   O^T += V^T x P^T: D/16 tiles of v_mfma_f32_16x16x16, two per tile (P
//       split into hi + lo halves); the V^T operand comes from one
//       ds_read_b64_tr_b16 per lane and tile (4 rows x 1 column each),
//       and the S output layout is already the P^T operand layout.
// A segment that lies entirely inside the wave's range is finished in the
// stream (output written at once).  Only a wave's first and last pieces can
// be shared; their states are kept in registers and merged through LDS after
// the stream, then written as an output, or as a workgroup partial that the
// last-arriver protocol combines.
static constexpr int kSRows = 16;    // rows per step
static constexpr int kMaxGroupS = 8;  // heads per group of this kernel

// 16 bytes per lane from gbase + voff into LDS at lds_addr + 16 * lane.
// M0 carries the LDS address; it is saved and restored around the load, so
// the compiler's own uses of M0 are unaffected.
__device__ __forceinline__ void dma_copy16(const void* gbase, uint32_t voff, uint32_t lds_addr) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "global_load_lds_dwordx4 %1, %2 nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(voff), "s"(gbase), "s"(lds_addr)
      : "memory");
}

// The same copy with a 64-bit address per lane (no scalar base), for a load
// whose lanes read from two different arrays.
__device__ __forceinline__ void dma_copy16_a64(const void* gaddr, uint32_t lds_addr) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(gaddr), "s"(lds_addr)
      : "memory");
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

template <typename T>
struct StreamOps;
template <>
struct StreamOps<bf16_t> {
  typedef __bf16 v4 __attribute__((ext_vector_type(4)));
  typedef short s4 __attribute__((ext_vector_type(4)));
  __device__ static f32x4 qk(const u32x4& a, const u32x4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  __device__ static uint64_t vt(const uint8_t* lds) {
    return __builtin_bit_cast(uint64_t,
                              __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) v4*)lds));
  }
  __device__ static f32x4 pv(uint64_t a, uint64_t b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4, a), __builtin_bit_cast(s4, b), c, 0, 0,
                                                     0);
  }
  __device__ static uint32_t from_f32(float x) { return f32_to_bf16_bits(x); }
  __device__ static float to_f32(uint32_t h) { return __uint_as_float(h << 16); }
  // two finite values, round to nearest even, in one v_cvt_pk_bf16_f32
  __device__ static uint32_t pack2(float a, float b) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, bf2));
  }
};
template <>
struct StreamOps<f16_t> {
  typedef _Float16 v4 __attribute__((ext_vector_type(4)));
  typedef __fp16 h4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
  __device__ static f32x4 qk(const u32x4& a, const u32x4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  __device__ static uint64_t vt(const uint8_t* lds) {
    return __builtin_bit_cast(uint64_t,
                              __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) h4*)lds));
  }
  __device__ static f32x4 pv(uint64_t a, uint64_t b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4, a), __builtin_bit_cast(v4, b), c, 0, 0, 0);
  }
  __device__ static uint32_t from_f32(float x) { return f32_to_f16_bits(x); }
  __device__ static float to_f32(uint32_t h) { return f16_bits_to_f32(h); }
  __device__ static uint32_t pack2(float a, float b) { return f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16); }
};

template <int D>
struct StreamGeom {
  static constexpr int RB = D * 2;             // bytes per row
  static constexpr int SB = kSRows * RB;       // bytes per tensor per step
  static constexpr int NI = SB / 1024;         // 1 KB loads per tensor per step
  static constexpr int RPI = 1024 / RB;        // rows per load
  static constexpr int CH = RB / 16;           // 16-byte chunks per row
  static constexpr int NC = D / 32;            // QK k-chunks
  static constexpr int NTD = D / 16;           // PV output tiles
  // Merge slot: (m, l) per head, then one accumulator row per head (the
  // slot's header lives in SchedLds::hdr).
  // Rows are DP floats apart, DP = 20 (mod 64): the (up to 8) heads a wave
  // writes in one instruction then start in different groups of 4 LDS banks.
  static constexpr int DP = D + 20;
  static constexpr int kSlot = 2 * kMaxGroupS * 4 + kMaxGroupS * DP * 4;  // merge slot bytes
};

// Fused append: new rows a wave keeps (K and V, plus the physical row) to
// store at the end of the kernel; beyond that they are stored at once.
static constexpr int kSaveRows = 4;

// q slot bytes: q's G rows, rounded to 256; with the fused append 1 KB more
// for the segment's new K and V rows (one 64-lane load).
__host__ __device__ constexpr int stream_qslot(int G, int D, bool append) {
  return ((G * D * 2 + 255) & ~255) + (append ? 1024 : 0);
}

// LDS bytes of the streaming kernel: per wave two (K, V) step buffers and two
// q slots of qslot bytes, with the fused append the kept new rows
// (kSaveRows x (K + V rows + 8-byte row index)), and side rows of 256 bytes
// (the direct table's scored flags and audio ranges, the deferred scoring's
// loads); the merge slots reuse the step buffers.
__host__ __device__ constexpr int stream_lds_bytes(int D, int NW, int qslot, bool append = false, int side_rows = 0) {
  return NW * (4 * kSRows * D * 2 + 2 * qslot + (append ? kSaveRows * (2 * D * 2 + 8) : 0) + side_rows * 256);
}
__host__ __device__ constexpr int stream_side_rows(bool xl, bool direct) { return xl && direct ? kXlRows : 0; }

// One step of a wave's stream: rows [row0, row0 + nrows) of segment s.
struct SStep {
  int64_t row0;    // physical row of the step's first row
  int64_t seg_lo;  // logical first row of the segment
  int32_t s, nrows, seg_len, qslot;
  int32_t first, last, whole;
  int32_t t0, alen;  // audio index of the first row; audio rows whose logits are kept (0: none)
  // APPEND: the step ends its segment (fewer than 16 old rows; the new row
  // is added): 1, or 2 when the table pass already found that the segment
  // has no room for the new row in the pool; 0 otherwise
  int32_t ends_seg;
  int32_t wr;  // APPEND, direct table: the segment's lane (its capacity is read when the row is kept)
};

// XL: keep the logits of the scored audio rows (p.xlog), else p.xlog is ignored.
// APPEND: append new_k / new_v[s] to every segment first (fused append).
// PV: score the previous launch's kept logits (deferred scoring; direct
// table and fused append only), an instance of its own so that the other
// launches carry none of its code or argument loads.
template <typename T, int D, int NW, int QD, bool XL, bool APPEND, bool DIRECT, bool PV = false>
// The fields read first lead the argument list as scalars: the build asks
// for 16 preloaded argument dwords (-amdgpu-kernarg-preload-count), of which
// the hardware delivers 14 in SGPRs at dispatch (the other two user SGPRs
// hold the argument pointer).  Those 14 are exactly the table, the tensors,
// the segment count and the group size packed with the grid size
// (gpack = G | grid << 8), so the table load is the kernel's first
// instruction of note and no argument or implicit-argument load (gridDim)
// precedes it; the split reciprocal and the aggregate are loaded and arrive
// while the table load is in flight.
__global__ __launch_bounds__(NW * 64, 2) void attn_stream_kernel(const int32_t* cu_arg, const int64_t* base_arg,
                                                               const int32_t* cap_arg, const void* q_arg,
                                                               const void* k_arg, const void* v_arg,
                                                               int32_t nseg_arg, int32_t gpack_arg, uint64_t inv_arg,
                                                               AttnParams p) {
  // DIRECT (n_seg <= 64, n_seg >= 1): lane s's segment bounds, loaded before
  // anything else (clamped lanes load segment n_seg - 1 and are masked by
  // the walk)
  int32_t t_lo = 0, t_hi = 0, t_cap = 0;
  int64_t t_base = 0;
  if constexpr (DIRECT) {
    const int si = min((int)(threadIdx.x & 63), nseg_arg - 1);
    t_lo = cu_arg[si];
    t_hi = cu_arg[si + 1];
    if (base_arg) t_base = base_arg[si];
    if (APPEND) t_cap = cap_arg[si];
  }
  __builtin_amdgcn_sched_barrier(0);
  const int64_t grid = (int64_t)((uint32_t)gpack_arg >> 8);
  const int32_t g_arg = gpack_arg & 0xff;
  // The argument fields the range computation and the first steps use,
  // loaded here while the table load is in flight: left to the compiler,
  // their loads sit behind the table's wait, one more round trip each.
  if constexpr (DIRECT)
    asm volatile("" ::"s"(inv_arg), "s"(p.phys_rows), "s"(p.scale_log2), "s"(p.new_k), "s"(p.new_v));
  p.q = q_arg;
  p.k = k_arg;
  p.v = v_arg;
  p.cu = cu_arg;
  p.base = base_arg;
  p.cap = cap_arg;
  p.split_inv = inv_arg;
  p.n_seg = nseg_arg;
  p.G = g_arg;
  // deferred scoring, before the stream: the sample's audio range and
  // accumulator offset, the slot's normalisers, the segments' bounds and the
  // logits go out beside the segment table, the accumulator entry once the
  // offset is in; the sums and the entry's store come before the first
  // steps are issued (workgroups with a slice only)
  PrevLoads pl;
  static_assert(!PV || (DIRECT && APPEND), "deferred scoring rides in the direct, fused-append instances");
  const bool pv_slice = PV && (int32_t)blockIdx.x < p.pv_slices;  // uniform
  if constexpr (PV) {
    if (pv_slice) {
      prev_issue_head(p, pl);
      prev_issue_body(p, (int)threadIdx.x, pl);
    }
  }
  using G_ = StreamGeom<D>;
  using Ops = StreamOps<T>;
  constexpr int NT = NW * 64;
  constexpr int RB = G_::RB, SB = G_::SB, NI = G_::NI, RPI = G_::RPI, CH = G_::CH, NC = G_::NC, NTD = G_::NTD;
  constexpr int QX = QD + (APPEND ? 1 : 0);  // first-step loads besides K and V: q (and the new row)
  constexpr int E = NI + QX + NI;  // loads per step
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
  __shared__ SchedLds sl;

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int lq = lane >> 4, lc = lane & 15;
  const int G = p.G;
  const int qbytes = G * RB;
  const int qarea = (qbytes + 255) & ~255;  // the new row (APPEND) follows q in its slot
  const int qslot = stream_qslot(G, D, APPEND);

  // the per-step load count (E) must match the group: q takes exactly QD loads
  if (QD != (qbytes + 1023) / 1024) {
    if (tid == 0 && blockIdx.x == 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
    return;
  }
  uint8_t* wbuf = dyn + w * 4 * SB;                    // K0 V0 K1 V1
  uint8_t* qbuf = dyn + NW * 4 * SB + w * 2 * qslot;   // q slot 0, 1
  // fused append: this wave's kept new rows (K | V per row), then their rows
  uint8_t* sbuf = dyn + NW * (4 * SB + 2 * qslot) + w * kSaveRows * (2 * RB + 8);
  int64_t* srow = (int64_t*)(sbuf + kSaveRows * 2 * RB);
  int nsaved = 0;
  // side rows of this wave (direct table, logits kept): the scored flag and
  // audio range of each segment
  constexpr int kSide = stream_side_rows(XL, DIRECT);
  uint8_t* side = dyn + NW * (4 * SB + 2 * qslot + (APPEND ? kSaveRows * (2 * RB + 8) : 0)) + w * kSide * 256;
  const uint32_t lds_side = __builtin_amdgcn_readfirstlane(lds_address(side));
  const int32_t* xl_rows = (const int32_t*)side;
  const uint32_t lds_w = __builtin_amdgcn_readfirstlane(lds_address(wbuf));
  const uint32_t lds_q = __builtin_amdgcn_readfirstlane(lds_address(qbuf));
  const T* kp = (const T*)p.k;
  const T* vp = (const T*)p.v;
  // rows [row0, row0 + nrows) of K or V into step buffer b, 16-byte chunks
  // swizzled by the row (K: chunk ^ (r % CH); V: chunk ^ 2 (r % 4)); rows past
  // nrows repeat the last row
  auto load_rows = [&](bool is_v, int64_t row0, int nrows, int b) {
    // wave-uniform addresses, kept scalar (the load takes them in SGPRs)
    const T* src = (const T*)uni((int64_t)(uintptr_t)((is_v ? vp : kp) + row0 * D));
    const uint32_t dst = __builtin_amdgcn_readfirstlane(lds_w + b * 2 * SB + (is_v ? SB : 0));
    nrows = uni((int32_t)nrows);
#pragma unroll
    for (int u = 0; u < NI; ++u) {
      const int r = u * RPI + lane / CH;
      const int rr = max(0, r < nrows ? r : nrows - 1);
      const int sw = is_v ? 2 * (r & 3) : r % CH;
      dma_copy16(src, (uint32_t)(rr * RB + (((lane % CH) ^ sw) * 16)), dst + u * 1024);
    }
  };
  // Up to 64 segments ("direct"): every wave reads the segment table itself,
  // one lane per segment, and issues its first steps as soon as it arrives;
  // the workgroup's checks of the table (and the outputs of empty or
  // invalid segments) follow once those loads are out.  More segments: the
  // workgroup pass of schedule() first, with its LDS cache of the bounds.
  // DIRECT is chosen by the host (n_seg <= 64); the two prologues are
  // separate instances, so neither carries the other's code and registers.
  constexpr bool direct = DIRECT;
  if (DIRECT && p.n_seg > 64) {
    if (tid == 0 && blockIdx.x == 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
    return;
  }
  const int64_t KV = p.phys_rows;
  int64_t R = 0, B0 = 0, B1 = 0;
  int s_first, s_last;
  if (direct) {  // the split range follows from the table (below)
    s_first = 0;
    s_last = p.n_seg - 1;
  } else {
    schedule<T, NT, XL, APPEND>(p, D, sl);
    if (sl.s_first > sl.s_last) return;
    R = uni(sl.R);
    B0 = uni(sl.B0);
    B1 = uni(sl.B1);
    s_first = uni(sl.s_first);
    s_last = uni(sl.s_last);
  }
  static_assert(NW == kSplitWaves, "wave ranges are units of the split");
  int64_t P_ = direct ? 0 : (int64_t)uni(sl.P);
  int64_t W0 = 0, W1 = 0;
  if (!direct && (int64_t)blockIdx.x < P_) {
    W0 = split_start((int64_t)blockIdx.x * NW + w, R, P_, p.split_inv);
    W1 = split_start((int64_t)blockIdx.x * NW + w + 1, R, P_, p.split_inv);
  }
  const bool in_ring = !direct && (s_last - s_first) < kRing;

  // ---- segment walk: a window of 64 segments, one per lane; the mask holds
  // the valid ones overlapping [W0, W1) that are not taken yet.
  int wb = s_first;
  int64_t lb = 0;  // physical first row
  int32_t llo = 0, llen = 0, lcap = 0, la0 = 0, lal = 0;  // logical first row, length, capacity
  bool lneg = false;  // the offsets of this lane's segment decrease
  uint64_t mask = 0;
  // the segments of the window that overlap this wave's range [W0, W1)
  auto window_mask = [&]() {
    // the piece [max(lo, W0), min(lo + len, W1)) must be non-empty (an empty
    // wave range inside a segment overlaps nothing)
    const bool ov = wb + lane <= s_last && seg_valid(llo, llen, lb, R, KV) &&
                    max((int64_t)llo, W0) < min((int64_t)llo + llen, W1);
    mask = __ballot(ov);
  };
  auto load_window = [&](bool with_mask) {
    const int s = wb + lane;
    lb = 0;
    llo = llen = lcap = 0;
    la0 = lal = 0;
    lneg = false;
    if (s <= s_last) {
      if (in_ring) {
        lb = sl.ring_base[s % kRing];
        llo = sl.ring_lo[s % kRing];
        llen = sl.ring_len[s % kRing];
        if (APPEND) lcap = sl.ring_cap[s % kRing];
        if (XL) {
          la0 = sl.ring_a0[s % kRing];
          lal = sl.ring_alen[s % kRing];
        }
      } else {
        // DIRECT: the one window, s = lane, loaded at entry
        const int32_t lo = DIRECT ? t_lo : p.cu[s], hi = DIRECT ? t_hi : p.cu[s + 1];
        lb = p.base ? (DIRECT ? t_base : p.base[s]) : (int64_t)lo;
        llo = lo;
        llen = hi - lo;
        lneg = llen < 0;
        if (APPEND) lcap = DIRECT ? t_cap : p.cap[s];
        if (XL && !DIRECT && p.xmask[s % p.Hkv]) {  // DIRECT: the side rows, read by process()
          la0 = p.audio_s[s / p.Hkv];
          lal = (int32_t)max((int64_t)0, min((int64_t)p.audio_e[s / p.Hkv] - la0, p.max_audio));
        }
      }
    }
    if (with_mask) window_mask();
  };
  load_window(!direct);
  if (direct) {
    // The rows the split covers end at cu[n_seg]: lane n_seg - 1 holds it.
    // Read from the table rather than passed in, so a launch captured in a
    // graph stays right as the segments grow.  Only this wave's own bounds
    // sit on the start-up path; the workgroup's follow once the first steps
    // are issued.
    R = max((int64_t)0, (int64_t)__builtin_amdgcn_readlane(llo + llen, p.n_seg - 1));
    P_ = effective_wgs(R, grid);
    if ((int64_t)blockIdx.x < P_) {
      W0 = split_start((int64_t)blockIdx.x * NW + w, R, P_, p.split_inv, grid);
      W1 = split_start((int64_t)blockIdx.x * NW + w + 1, R, P_, p.split_inv, grid);
    }
    window_mask();
  }
  // issue-side iterator: current piece [pb, pe) of segment cur_s (logical rows)
  int cur_s = 0, cur_len = 0, piece_no = 0, cur_a0 = 0, cur_al = 0, cur_k = 0;
  int64_t cur_b = 0, cur_lo = 0, pb = 0, pe = 0, irow = 0;
  bool cur_whole = false, have = false;
  // APPEND: the piece ends its segment with a multiple of 16 rows, so its
  // first step takes 15: the step that ends the segment then always has room
  // for the new row
  bool short_first = false;
  auto next_piece = [&]() {
    while (mask == 0) {
      wb += 64;
      if (wb > s_last) {
        have = false;
        return;
      }
      load_window(true);
    }
    const int k = __builtin_ctzll(mask);
    mask &= mask - 1;
    cur_s = wb + k;
    const uint32_t blo = __builtin_amdgcn_readlane((uint32_t)lb, k);
    const uint32_t bhi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)lb >> 32), k);
    cur_b = (int64_t)(((uint64_t)bhi << 32) | blo);
    cur_lo = __builtin_amdgcn_readlane(llo, k);
    cur_len = __builtin_amdgcn_readlane(llen, k);
    cur_k = k;  // the segment's lane in the window (its capacity, read by the step that ends it)
    if (XL) {
      cur_a0 = __builtin_amdgcn_readlane(la0, k);
      cur_al = __builtin_amdgcn_readlane(lal, k);
    }
    pb = max(cur_lo, W0);
    pe = min(cur_lo + cur_len, W1);
    cur_whole = cur_lo >= W0 && cur_lo + cur_len <= W1;
    short_first = APPEND && pe == cur_lo + cur_len && ((pe - pb) & (kSRows - 1)) == 0;
    irow = pb;
    have = true;
  };
  next_piece();
  auto gen = [&](SStep& st) -> bool {
    if (!have) return false;
    st.s = cur_s;
    st.seg_lo = cur_lo;
    st.seg_len = cur_len;
    st.row0 = cur_b + (irow - cur_lo);
    st.first = irow == pb;
    st.nrows = APPEND && st.first && short_first ? kSRows - 1 : (int32_t)min((int64_t)kSRows, pe - irow);
    st.whole = cur_whole;
    st.qslot = piece_no & 1;
    if (XL) {
      // DIRECT: the offset within the segment (the audio start is subtracted
      // by process(), from the side rows)
      st.t0 = (int32_t)(irow - cur_lo) - (DIRECT ? 0 : cur_a0);
      st.alen = DIRECT ? 0 : cur_al;
    }
    // With more than one window of 64 segments (the table pass), the walk
    // may move on to the next window (next_piece below) before this step is
    // processed, so the segment's capacity is read now; with the direct
    // table there is one window, and it is read only when the row is kept.
    st.ends_seg = 0;
    if (APPEND && irow + st.nrows == cur_lo + cur_len)
      st.ends_seg = (!DIRECT && cur_len + 1 > __builtin_amdgcn_readlane(lcap, cur_k)) ? 2 : 1;
    st.wr = cur_k;
    irow += st.nrows;
    st.last = irow >= pe;
    if (st.last) {
      ++piece_no;
      next_piece();
    }
    return true;
  };

  // ---- loads of one step into buffer b: K, q (+ new row), V (E loads, in
  // this order).  q is loaded for the first step of a piece only (the later
  // steps keep it in registers), so a step issues E loads with q and E - QX
  // without.  With the fused append the first step also copies the
  // segment's new K and V rows behind q (lanes 0 .. CH-1: K chunks, CH ..
  // 2CH-1: V chunks, the others repeat them), one 64-bit-addressed load.
  auto issue = [&](const SStep& st, int b) {
    load_rows(false, st.row0, st.nrows, b);
    if (st.first) {
      const T* qs = (const T*)uni((int64_t)(uintptr_t)((const T*)p.q + (int64_t)st.s * G * D));
#pragma unroll
      for (int u = 0; u < QD; ++u) {
        const int off = u * 1024 + lane * 16;
        if (off < qbytes)
          dma_copy16(qs, (uint32_t)off, __builtin_amdgcn_readfirstlane(lds_q + st.qslot * qslot + u * 1024));
      }
      if (APPEND) {
        const int c = lane % (2 * CH);
        const uint8_t* a = (const uint8_t*)(c < CH ? p.new_k : p.new_v) + (int64_t)st.s * RB + (c % CH) * 16;
        dma_copy16_a64(a, __builtin_amdgcn_readfirstlane(lds_q + st.qslot * qslot + qarea));
      }
    }
    load_rows(true, st.row0, st.nrows, b);
  };

  // ---- softmax state of the current piece, and the held (first, shared) one
  float m_run = kNegBig, l_run = 0.f;
  f32x4 acc[NTD];
  float m_h = kNegBig, l_h = 0.f;
  f32x4 acc_h[NTD];
  int32_t h_s = -1, h_len = 0;
  int64_t h_b = 0;
#pragma unroll
  for (int t = 0; t < NTD; ++t) {
    acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc_h[t] = acc[t];
  }
  int32_t c_s = -1, c_len = 0;  // the unfinished piece at the end of the stream
  int64_t c_b = 0;
  u32x4 qb[NC];

  // APPEND: a segment's new row kept for the pools (stored after the hand-off)
  // when the segment has room for it.  The row goes after the segment's old
  // rows.
  auto keep_new_row = [&](const SStep& st) {
    if (st.ends_seg != 1) return;  // wave-uniform
    if (DIRECT && st.seg_len + 1 > __builtin_amdgcn_readlane(lcap, st.wr)) return;
    const uint8_t* nrow = qbuf + st.qslot * qslot + qarea;
    const int64_t row = st.row0 + st.nrows;
    if (nsaved < kSaveRows) {  // wave-uniform
      if (lane < 2 * CH) *(u32x4*)(sbuf + nsaved * 2 * RB + lane * 16) = *(const u32x4*)(nrow + lane * 16);
      if (lane == 0) srow[nsaved] = row;
      ++nsaved;
    } else if (lane < 2 * CH) {  // keep-list full: stored now (its acknowledgement delays the next wait)
      *(WNW_GLOBAL u32x4*)(gptr_w<uint8_t>(const_cast<void*>(lane < CH ? p.k : p.v)) + row * RB +
                           (lane % CH) * 16) = *(const u32x4*)(nrow + lane * 16);
    }
  };

  auto process = [&](const SStep& st, int b, bool has_next, bool next_first) {
    uint8_t* kbuf = wbuf + b * 2 * SB;
    uint8_t* vbuf = kbuf + SB;
    __builtin_amdgcn_sched_barrier(0);
    // K (and q) of this step: its V and the next step may still load
    if (has_next && next_first)
      wait_vmcnt<NI + E>();
    else if (has_next)
      wait_vmcnt<NI + E - QX>();
    else
      wait_vmcnt<NI>();
    __builtin_amdgcn_sched_barrier(0);
    if (st.first) {  // q of this piece: operand lane (lq, lc) = q[g = lc][32c + 8lq ..]
      const uint8_t* qsl = qbuf + st.qslot * qslot;
#pragma unroll
      for (int c = 0; c < NC; ++c)
        qb[c] = lc < G ? *(const u32x4*)(qsl + lc * RB + (4 * c + lq) * 16) : u32x4{0, 0, 0, 0};
    }
    // APPEND: the step that ends its segment (fewer than 16 old rows, by the
    // cut of the piece's steps) takes the segment's new row (behind q in the
    // piece's slot) as row nrows:
    // its K chunks now, swizzled like the loaded rows, its V chunks after
    // V's wait.  The step's DMA has landed, and the buffer is this wave's
    // until the step after next is issued.
    const bool add_row = APPEND && st.ends_seg && st.nrows < kSRows;  // wave-uniform
    if (add_row && lane < CH) {
      const uint8_t* nrow = qbuf + st.qslot * qslot + qarea;
      *(u32x4*)(kbuf + st.nrows * RB + ((lane ^ (st.nrows % CH)) * 16)) = *(const u32x4*)(nrow + lane * 16);
    }
    const int nvalid = st.nrows + (add_row ? 1 : 0);
    f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const u32x4 a = *(const u32x4*)(kbuf + lc * RB + (((4 * c + lq) ^ (lc % CH)) * 16));
      sacc = Ops::qk(a, qb[c], sacc);
    }
    // online softmax for head g = lc over rows 4 lq + i
    float x[4];
    float mx = kNegBig;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = (4 * lq + i) < nvalid ? sacc[i] * p.scale_log2 : -INFINITY;
      mx = fmaxf(mx, x[i]);
    }
    int32_t x_t0 = st.t0, x_alen = st.alen;
    if constexpr (XL && DIRECT) {  // the segment's scored flag and audio range (side rows, landed)
      const int32_t xm = xl_rows[st.wr], as = xl_rows[64 + st.wr], ae = xl_rows[128 + st.wr];
      x_alen = xm ? (int32_t)max((int64_t)0, min((int64_t)ae - as, p.max_audio)) : 0;
      x_t0 = st.t0 - as;
    }
    if (XL && x_alen > 0 && x_t0 < x_alen && x_t0 + st.nrows > 0 && lc < G) {
      // rows of a scored segment's audio: keep their logits for the scoring
      // pass.  The lane's four rows are consecutive in the slot: one 16-byte
      // store (4-byte aligned) when all four are kept, else one per row.
      WNW_GLOBAL float* xl = gptr_w<float>(p.xlog) + ((int64_t)st.s * G + lc) * p.max_audio;
      const int r0 = 4 * lq, t0 = x_t0 + r0;
      if (r0 + 3 < st.nrows && t0 >= 0 && t0 + 3 < x_alen) {
        typedef float f32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
        *(WNW_GLOBAL f32x4a4*)(xl + t0) = f32x4a4{x[0], x[1], x[2], x[3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = r0 + i, t = t0 + i;
          if (r < st.nrows && t >= 0 && t < x_alen) xl[t] = x[i];
        }
      }
    }
    mx = max_x32(max_x16(mx));
    const float m_new = fmaxf(m_run, mx);
    // exp2 by v_exp_f32 directly: arguments are <= 0, and weights below
    // 2^-126 (flushed to zero) are negligible beside the maximum's 1
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    float pv[4];
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pv[i] = __builtin_amdgcn_exp2f(x[i] - m_new);
      psum += pv[i];
    }
    // P = hi + lo, each a 16-bit float: PV runs as two MFMAs with fp32-grade P
    const uint32_t h01 = Ops::pack2(pv[0], pv[1]), h23 = Ops::pack2(pv[2], pv[3]);
    const uint32_t l01 = Ops::pack2(pv[0] - Ops::to_f32(h01 & 0xffffu), pv[1] - Ops::to_f32(h01 >> 16));
    const uint32_t l23 = Ops::pack2(pv[2] - Ops::to_f32(h23 & 0xffffu), pv[3] - Ops::to_f32(h23 >> 16));
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int t = 0; t < NTD; ++t) acc[t] *= alpha;
    const uint64_t ph = (uint64_t)h01 | ((uint64_t)h23 << 32);
    const uint64_t pl = (uint64_t)l01 | ((uint64_t)l23 << 32);
    __builtin_amdgcn_sched_barrier(0);
    // V of this step: the next step may still load
    if (has_next && next_first)
      wait_vmcnt<E>();
    else if (has_next)
      wait_vmcnt<E - QX>();
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_sched_barrier(0);
    if (add_row && lane < CH) {  // the new row's V chunks as row nrows
      const uint8_t* nrow = qbuf + st.qslot * qslot + qarea;
      *(u32x4*)(vbuf + st.nrows * RB + ((lane ^ (2 * (st.nrows & 3))) * 16)) =
          *(const u32x4*)(nrow + RB + lane * 16);
    }
    // V^T operand of tile t: lane (lq, lc) addresses row 4 lq + lc / 4, columns
    // 16 t + 4 (lc % 4) .. + 3 (8 bytes of the swizzled row)
    {
      const int r = 4 * lq + (lc >> 2);
      const int sw = 2 * (r & 3);
      const uint8_t* rowp = vbuf + r * RB + (lc & 1) * 8;
#pragma unroll
      for (int t = 0; t < NTD; ++t) {
        const int chunk = (2 * t + ((lc & 3) >> 1)) ^ sw;
        const uint64_t a = Ops::vt(rowp + chunk * 16);
        acc[t] = Ops::pv(a, ph, acc[t]);
        acc[t] = Ops::pv(a, pl, acc[t]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (st.last) {
      if (APPEND && st.ends_seg) {
        keep_new_row(st);
      }
      const float l_tot = sum_x32(sum_x16(l_run));
      if (st.whole) {  // the segment lies inside this wave's range: finish it
        if (lc < G) {
          WNW_GLOBAL uint16_t* o = gptr_w<uint16_t>(p.out) + ((int64_t)st.s * G + lc) * D;
          const float inv = 1.f / l_tot;
#pragma unroll
          for (int t = 0; t < NTD; ++t) {
            const uint32_t w0 = Ops::from_f32(acc[t][0] * inv) | (Ops::from_f32(acc[t][1] * inv) << 16);
            const uint32_t w1 = Ops::from_f32(acc[t][2] * inv) | (Ops::from_f32(acc[t][3] * inv) << 16);
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            *(WNW_GLOBAL u32x2*)(o + 16 * t + 4 * lq) = u32x2{w0, w1};
          }
          if (p.lse && lq == 0) {
            WNW_GLOBAL float* ls = gptr_w<float>(p.lse) + ((int64_t)st.s * G + lc) * 2;
            ls[0] = m_run;
            ls[1] = l_tot;
          }
        }
      } else if (h_s < 0) {  // first shared piece: hold it until the end
        h_s = st.s;
        h_b = st.seg_lo;
        h_len = st.seg_len;
        m_h = m_run;
        l_h = l_tot;
#pragma unroll
        for (int t = 0; t < NTD; ++t) acc_h[t] = acc[t];
      } else {  // last shared piece: it is the end of this wave's range
        c_s = st.s;
        c_b = st.seg_lo;
        c_len = st.seg_len;
        l_run = l_tot;
        return;
      }
      m_run = kNegBig;
      l_run = 0.f;
#pragma unroll
      for (int t = 0; t < NTD; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };

  if constexpr (PV) {
    if (pv_slice) {
      float* pv_dst = nullptr;
      float pv_total = 0.f;
      prev_finish(p, tid, pl, pv_dst, pv_total);
      if (pv_dst) *gptr_w<float>(pv_dst) = pv_total;
    }
  }
  // the scored flag and audio range of each segment (lane = segment) into
  // the side rows, older than every step's loads, so the first step's waits
  // cover them (the table path does not wait for them)
  if constexpr (XL && DIRECT) {
    const int sx = min(lane, p.n_seg - 1);
    const int hkv = max(p.Hkv, 1);
    const int smp = sx / hkv;
    dma_copy4_a64(p.xmask + (sx - smp * hkv), lds_side);
    dma_copy4_a64(p.audio_s + smp, lds_side + 256);
    dma_copy4_a64(p.audio_e + smp, lds_side + 512);
  }
  // ---- the stream: two steps in flight (buffers 0 and 1 alternate)
  SStep sA, sB;
  bool hA = gen(sA);
  if (hA) issue(sA, 0);
  bool hB = hA && gen(sB);
  if (hB) issue(sB, 1);
  if (direct) {
    wg_range(R, P_, p.split_inv, B0, B1, grid);
    if (tid == 0) {  // read by the merge and the hand-off, after barriers
      sl.R = R;
      sl.KV = KV;
      sl.P = (int32_t)P_;
      sl.B0 = B0;
      sl.B1 = B1;
    }
  }
  // direct: the checks of schedule() from the table window in registers
  // (lane i holds segment i; no new loads, which would wait behind the
  // steps just issued).  Wave 0 of every workgroup; the outputs of empty
  // and invalid segments are written by workgroup i % grid.
  if (direct && w == 0) {
    const int si = lane;
    const bool in = si < p.n_seg;
    // lneg: the offsets of this segment decrease (a corrupt table, treated
    // as an empty segment)
    const int64_t len = in && !lneg ? llen : 0;
    const bool bad = in && lneg;
    if (bad) raise_device_error(p.err, WNW_DEVERR_ORDER);
    const bool any_bad = __ballot(bad) != 0;
    if (lane == 0) sl.order_bad = any_bad;
    if (in && !seg_valid(llo, len, lb, R, KV)) {
      const bool owner = (si % (int)grid) == (int)blockIdx.x;
      if (len != 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
      if (APPEND && len == 0 && !lneg) {  // only the new row: it is the output
        if (owner) append_only_segment<T>(p, D, si, lb, 1 <= lcap && lb >= 0 && lb < KV);
      } else if (owner) {
        const float fill = len == 0 ? 0.f : __int_as_float(0x7fc00000);
        for (int e = 0; e < G * D; ++e) store_elem<T>(p.out, (int64_t)si * G * D + e, fill);
        if (p.lse) {
          WNW_GLOBAL float* ls = gptr_w<float>(p.lse) + (int64_t)si * G * 2;
          for (int g = 0; g < G; ++g) {
            ls[2 * g] = len == 0 ? kNegBig : fill;
            ls[2 * g + 1] = len == 0 ? 0.f : fill;
          }
        }
      }
    }
  }
  while (hA) {
    process(sA, 0, hB, hB && sB.first);
    hA = hB && gen(sA);  // the step after sB
    if (hA) issue(sA, 0);
    if (!hB) break;
    process(sB, 1, hA, hA && sA.first);
    hB = hA && gen(sB);
    if (hB) issue(sB, 1);
    if (!hA) break;
  }
  wait_vmcnt<0>();

  // ---- shared pieces: merge the waves' states through LDS
  __syncthreads();  // every wave is done with its step buffers (reused below)
  constexpr int SLOT = G_::kSlot;
  static_assert(2 * NW * SLOT <= NW * 4 * SB, "the merge slots reuse the step buffers");
  auto slot_of = [&](int i) { return dyn + i * SLOT; };
  auto put = [&](int i, int32_t s, int64_t b, int32_t len, float m, float l, const f32x4* a) {
    uint8_t* sp = slot_of(i);
    if (lane == 0) {
      sl.hdr[i][0] = s;
      sl.hdr[i][1] = len;
      sl.hdr[i][2] = (int32_t)(uint32_t)b;
      sl.hdr[i][3] = (int32_t)(b >> 32);
    }
    if (s >= 0 && lc < G) {
      float* ml = (float*)sp;
      if (lq == 0) {
        ml[lc] = m;
        ml[kMaxGroupS + lc] = l;
      }
      float* ap = (float*)(sp + 2 * kMaxGroupS * 4) + lc * G_::DP;
#pragma unroll
      for (int t = 0; t < NTD; ++t) *(f32x4*)(ap + 16 * t + 4 * lq) = a[t];
    }
  };
  put(2 * w, h_s, h_b, h_len, m_h, l_h, acc_h);
  put(2 * w + 1, c_s, c_b, c_len, m_run, l_run, acc);
  __syncthreads();
  // Slot headers: lane i reads header i % NS (one LDS read for all of
  // them).  Slots follow the row order, and segments are disjoint and
  // ordered, so the segment numbers of the non-empty slots never decrease:
  // a slot leads its segment when its number exceeds every earlier slot's,
  // and only the segments of the first and the last non-empty slot can
  // cross the workgroup's range boundaries (those become partials for the
  // last-arriver combine; every other segment is written out).
  constexpr int NS = 2 * NW;
  static_assert(NS <= 16, "merge slot headers");
  typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
  const i32x4 hv = *(const i32x4*)sl.hdr[lane % NS];
  int32_t ss[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) ss[i] = __builtin_amdgcn_readlane(hv.x, i);
  uint32_t lead = 0;
  {
    int32_t top = -1;
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      if (ss[i] > top) lead |= 1u << i;
      top = max(top, ss[i]);
    }
  }
  int32_t ps0 = -1, ps1 = -1, pl0 = 0, pl1 = 0;
  int64_t pb0 = 0, pb1 = 0;
  if (lead) {
    const uint32_t used = (uint32_t)__ballot(lane < NS && hv.x >= 0);
    const int jf = __builtin_ctz(used), jl = 31 - __builtin_clz(used);
    auto base_of = [&](int j) {
      return (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hv.w, j) << 32) |
                       (uint32_t)__builtin_amdgcn_readlane(hv.z, j));
    };
    const int64_t bf = base_of(jf), bl = base_of(jl);
    const int32_t nf = __builtin_amdgcn_readlane(hv.y, jf), nl = __builtin_amdgcn_readlane(hv.y, jl);
    const int32_t sf = __builtin_amdgcn_readlane(hv.x, jf), sg = __builtin_amdgcn_readlane(hv.x, jl);
    if (bf < B0 || bf + nf > B1) {
      ps0 = sf;
      pb0 = bf;
      pl0 = nf;
    }
    if (sg != sf && bl + nl > B1) {
      if (ps0 < 0) {
        ps0 = sg;
        pb0 = bl;
        pl0 = nl;
      } else {
        ps1 = sg;
        pb1 = bl;
        pl1 = nl;
      }
    }
  }
  const int GD = G * D;
  const int GD4 = GD / 4;
  // Task t = (leader t / GD4, quad t % GD4) over all threads: one thread per
  // 4 consecutive elements of one head of one segment.  Every slot is read
  // (no branches between the loads, so they share one LDS round trip);
  // selects drop the other segments' slots, whatever they hold.
  const int n_lead = __builtin_popcount(lead);
  for (int t = tid; t < n_lead * GD4; t += NT) {
    const int li = t / GD4, i4 = t - li * GD4;
    uint32_t lm = lead;
    for (int r = 0; r < li; ++r) lm &= lm - 1;
    const int a = __builtin_ctz(lm);
    const i32x4 ha = *(const i32x4*)sl.hdr[a];
    const int32_t sa = ha.x, na = ha.y;
    const int64_t ba = (int64_t)(((uint64_t)(uint32_t)ha.w << 32) | (uint32_t)ha.z);
    const bool inside = ba >= B0 && ba + na <= B1;
    const int g = (4 * i4) / D;
    float mv[NS], lv[NS];
    f32x4 av[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const float* ml = (const float*)slot_of(j);
      mv[j] = ml[g];
      lv[j] = ml[kMaxGroupS + g];
      av[j] = *(const f32x4*)((const float*)(slot_of(j) + 2 * kMaxGroupS * 4) + g * G_::DP + (4 * i4 - g * D));
    }
    float M = kNegBig;
#pragma unroll
    for (int j = 0; j < NS; ++j) M = fmaxf(M, ss[j] == sa ? mv[j] : kNegBig);
    float L = 0.f;
    f32x4 A = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const bool in = ss[j] == sa;
      const float sc = in ? __builtin_amdgcn_exp2f(mv[j] - M) : 0.f;
      L += in ? lv[j] * sc : 0.f;
      A += in ? av[j] * sc : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const bool lead_elem = (4 * i4) % D == 0;
    if (inside) {
      const float inv = 1.f / L;
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      const uint32_t w0 = Ops::from_f32(A[0] * inv) | (Ops::from_f32(A[1] * inv) << 16);
      const uint32_t w1 = Ops::from_f32(A[2] * inv) | (Ops::from_f32(A[3] * inv) << 16);
      *((WNW_GLOBAL u32x2*)gptr_w<uint16_t>(p.out) + ((int64_t)sa * GD4 + i4)) = u32x2{w0, w1};
      if (p.lse && lead_elem) {
        gptr_w<float>(p.lse)[((int64_t)sa * G + g) * 2] = M;
        gptr_w<float>(p.lse)[((int64_t)sa * G + g) * 2 + 1] = L;
      }
    } else {
      const int64_t pslot = (int64_t)blockIdx.x + sa;
      st_agent2(p.part_acc + pslot * GD + 4 * i4, A[0], A[1]);
      st_agent2(p.part_acc + pslot * GD + 4 * i4 + 2, A[2], A[3]);
      if (lead_elem) st_agent2(p.part_ml + (pslot * G + g) * 2, M, L);
    }
  }
  // piece counts of the partial segments, worked out while the stores drain
  int32_t pn0 = 0, pn1 = 0;  // pieces - 1
  int64_t pf0 = 0, pf1 = 0;  // workgroup of the first piece
  {
    int64_t l;
    if (ps0 >= 0) {
      piece_range(sl, pb0, pl0, pf0, l);
      pn0 = (int32_t)(l - pf0);
    }
    if (ps1 >= 0) {
      piece_range(sl, pb1, pl1, pf1, l);
      pn1 = (int32_t)(l - pf1);
    }
  }
  wait_vmem();
  __syncthreads();  // partials complete; the slots may be overwritten below
  // Both arrivals in one atomic instruction (lanes 0 and 1 of wave 0, one
  // memory round trip); each segment whose last partial this is merges.
  if (tid < 2) {
    const int32_t ps = sl.order_bad ? -1 : (tid ? ps1 : ps0);
    bool f = false;
    if (ps >= 0)
      f = __hip_atomic_fetch_add(gptr_w<int32_t>(p.counters) + ps, 1, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT) == (tid ? pn1 : pn0);
    const uint64_t fl = __ballot(f);
    if (tid == 0) sl.is_last = (int)(fl & 3);
  }
  __syncthreads();
  if (APPEND) {
    // the kept new rows into the pools: no wait of this workgroup follows
    // (the combine below reads other memory), so their acknowledgement
    // overlaps the combine
    for (int i = 0; i < nsaved; ++i) {
      const int64_t row = uni(srow[i]);
      if (lane < 2 * CH)
        *(WNW_GLOBAL u32x4*)(gptr_w<uint8_t>(const_cast<void*>(lane < CH ? p.k : p.v)) + row * RB +
                             (lane % CH) * 16) = *(const u32x4*)(sbuf + i * 2 * RB + lane * 16);
    }
  }
  // the segments this workgroup completes are merged side by side (one
  // half of the workgroup each when there are two)
  const int last = uni(sl.is_last);
  if (last) {
    const bool both = last == 3;
    const int nt = both ? NT / 2 : NT;
    const bool k = both ? tid >= NT / 2 : last == 2;  // uniform per wave
    combine_from<T>(p, D, k ? pf1 : pf0, (k ? pn1 : pn0) + 1, k ? ps1 : ps0, both && k ? tid - NT / 2 : tid, nt);
  }
  if (APPEND) {
    // (direct table) workgroup 0's post-append offsets, last, so no wait of
    // this kernel waits for them, and the capacity check of every segment
    if (direct && blockIdx.x == 0 && w == 0 && lane < p.n_seg) {  // cu_out = cu + arange(n_seg + 1)
      WNW_GLOBAL int32_t* co = gptr_w<int32_t>(p.cu_out);
      co[lane] = llo + lane;
      if (lane == p.n_seg - 1) co[p.n_seg] = llo + llen + p.n_seg;  // llen: cu[s + 1] - cu[s], as read
      if (!lneg && llen + 1 > lcap) raise_device_error(p.err, WNW_DEVERR_CAPACITY);
    }
  }
}

// ---------------------------------------------------------------------------
// VALU kernel (any element type; D = 64, 128, 256; G <= 16)
// ---------------------------------------------------------------------------
// Per wave and 64-row step: lane r scores row r against all G heads (q staged
// in LDS as fp32), the wave takes the per-head max and sum, writes P to LDS,
// then every lane accumulates D/64 output columns over the 64 rows (V reads
// coalesced along the row).
template <int D, int NW>
struct ValuLds {
  static constexpr int kQ = kMaxGroup * D * 4;
  static constexpr int kP = NW * 64 * kMaxGroup * 4;
  static constexpr int kMerge = NW * kMaxGroup * (D + 2) * 4;
  static constexpr int kWork = kQ + kP;
  static constexpr int kBytes = kWork > kMerge ? kWork : kMerge;
};

template <typename T, int D, int NW>
__global__ __launch_bounds__(NW * 64, 2) void attn_valu_kernel(AttnParams p) {
  constexpr int NT = NW * 64;
  constexpr int E = D / 64;  // output columns per lane
  constexpr int EPC = 16 / sizeof(T);  // elements per 16-byte chunk
  __shared__ SchedLds sl;
  __shared__ __attribute__((aligned(16))) uint8_t lds[ValuLds<D, NW>::kBytes];

  schedule<T, NT>(p, D, sl);
  if (sl.s_first > sl.s_last) return;

  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int G = p.G;
  float* qf = (float*)lds;                            // [16][D]
  float* pl = (float*)(lds + ValuLds<D, NW>::kQ) + w * 64 * kMaxGroup;  // [64][16]
  const T* kp = (const T*)p.k;
  const T* vp = (const T*)p.v;

  for (int s = sl.s_first; s <= sl.s_last; ++s) {
    const Piece pc = make_piece(p, sl, s);
    if (pc.skip) continue;  // workgroup-uniform
    const T* qs = (const T*)p.q + (int64_t)s * G * D;
    for (int idx = tid; idx < G * D; idx += NT) qf[idx] = Elem<T>::to_f32(qs, idx);
    __syncthreads();

    float m_run[kMaxGroup], l_run[kMaxGroup], acc[kMaxGroup][E];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
      m_run[g] = kNegBig;
      l_run[g] = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[g][e] = 0.f;
    }
    const int nsteps = (pc.nrows + 63) / 64;
    for (int step = w; step < nsteps; step += NW) {
      const int64_t r0 = pc.phys + (int64_t)step * 64;
      const int valid = min(64, pc.nrows - step * 64);
      const int r = lane < valid ? lane : valid - 1;
      float sc[kMaxGroup];
#pragma unroll
      for (int g = 0; g < kMaxGroup; ++g) sc[g] = 0.f;
      const T* krow = kp + (r0 + r) * D;
      for (int c = 0; c < D / EPC; ++c) {
        const u32x4 wv = *(const u32x4*)(krow + c * EPC);
        float kf[8];
        if constexpr (sizeof(T) == 4) {
#pragma unroll
          for (int i = 0; i < 4; ++i) kf[i] = __uint_as_float(wv[i]);
        } else {
          unpack8(wv, kf, (T*)nullptr);
        }
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) {
          if (g < G) {
#pragma unroll
            for (int i = 0; i < EPC; ++i) sc[g] += qf[g * D + c * EPC + i] * kf[i];
          }
        }
      }
#pragma unroll
      for (int g = 0; g < kMaxGroup; ++g) {
        if (g < G) {
          const float x = lane < valid ? sc[g] * p.scale_log2 : -INFINITY;
          const float m_new = fmaxf(m_run[g], wave_max(x));
          const float alpha = exp2f(m_run[g] - m_new);
          const float pv = exp2f(x - m_new);
          l_run[g] = l_run[g] * alpha + wave_sum(pv);
          m_run[g] = m_new;
#pragma unroll
          for (int e = 0; e < E; ++e) acc[g][e] *= alpha;
          pl[lane * kMaxGroup + g] = pv;
        }
      }
      // PV: lane owns columns lane + 64 e
      for (int rr = 0; rr < valid; ++rr) {
        const T* vrow = vp + (r0 + rr) * D;
        float vf[E];
#pragma unroll
        for (int e = 0; e < E; ++e) vf[e] = Elem<T>::to_f32(vrow, lane + 64 * e);
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) {
          if (g < G) {
            const float pv = pl[rr * kMaxGroup + g];
#pragma unroll
            for (int e = 0; e < E; ++e) acc[g][e] += pv * vf[e];
          }
        }
      }
    }
    __syncthreads();  // q / P staging aliased by the merge area
    float* mrg_ml = (float*)lds;
    float* mrg_acc = (float*)lds + NW * kMaxGroup * 2;
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
      if (g < G) {
        if (lane == 0) {
          mrg_ml[(w * kMaxGroup + g) * 2] = m_run[g];
          mrg_ml[(w * kMaxGroup + g) * 2 + 1] = l_run[g];
        }
#pragma unroll
        for (int e = 0; e < E; ++e) mrg_acc[(w * kMaxGroup + g) * D + lane + 64 * e] = acc[g][e];
      }
    }
    __syncthreads();
    finish_piece<T, NT, NW>(p, D, sl, pc, s, mrg_ml, mrg_acc);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static constexpr int kNW = 4;

struct DeviceInfo {
  int cus = 0;
  int max_wg = 0;  // upper bound of workgroups per launch (sizes the workspace)
};

static DeviceInfo& device_info() {
  static std::mutex mu;
  static std::vector<DeviceInfo> infos;
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::lock_guard<std::mutex> lock(mu);
  if ((int)infos.size() <= dev) infos.resize(dev + 1);
  DeviceInfo& di = infos[dev];
  if (di.cus == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    di.cus = cus;
    di.max_wg = cus * 8;
  }
  return di;
}

struct WsLayout {
  int64_t counters, ml, acc, total;
  int64_t slots;
};

// Arrival counters for cap_seg segments first, then the (m, l) pairs and
// the accumulators of `slots` partial slots.
static WsLayout make_layout(int64_t cap_seg, int64_t slots, int64_t G, int64_t D) {
  WsLayout L;
  L.slots = slots;
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  L.counters = 0;
  L.ml = up(cap_seg * 4);
  L.acc = L.ml + up(L.slots * G * 2 * 4);
  L.total = L.acc + up(L.slots * G * D * 4);
  return L;
}

// Caller-owned workspace: sized before the grid is known, so for the
// largest grid a launch may use.
static WsLayout ws_layout(int64_t n_seg, int64_t G, int64_t D) {
  return make_layout(n_seg, device_info().max_wg + n_seg, G, D);
}

// ---------------------------------------------------------------------------
// The library's own attention scratch (wnw_decode_attn_noalloc)
// ---------------------------------------------------------------------------
// A file-scope device array: each device holds its own copy, at its own
// address, for as long as the process lives.  Host code uses only the
// per-device address from hipGetSymbolAddress (resolved once per device,
// with that device current), never the array's name.  The counters region
// is sized for WNW_NOALLOC_MAX_SEG segments whatever a call's n_seg, so
// calls with different n_seg never turn partial bytes into counters; every
// launch leaves the counters of its segments at zero, the others are never
// touched, and the array is zero at load (cleared again on first use).
static constexpr int64_t kNoAllocBytes = WNW_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t g_attn_scratch[kNoAllocBytes];

struct ScratchSlot {
  void* ptr = nullptr;
  bool cleared = false;
};

__global__ void fill_zero_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// Raises a kernel's dynamic-LDS limit once per device (the attribute is a
// property of the kernel on the device that is current when it is set).
static hipError_t set_lds_limit_once(std::vector<signed char>& done, std::mutex& mu, const void* fn, int bytes) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)done.size() <= dev) done.resize(dev + 1, 0);
  if (!done[dev]) {
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return e;
    done[dev] = 1;
  }
  return hipSuccess;
}

// Streaming kernel launch: QD = q loads per step, dynamic LDS as sized by
// stream_lds_bytes (above 64 KB, so the limit is raised once per instance
// and device).
template <typename T, int D, int QD, bool XL, bool APPEND, bool DIRECT, bool PV = false>
static hipError_t launch_stream_k(const AttnParams& ap, int64_t n_wg, hipStream_t st) {
  constexpr int side = stream_side_rows(XL, DIRECT);
  const int lds = stream_lds_bytes(D, kNW, stream_qslot(ap.G, D, APPEND), APPEND, side);
  static std::mutex mu;
  static std::vector<signed char> done;
  const hipError_t attr_err =
      set_lds_limit_once(done, mu, (const void*)&attn_stream_kernel<T, D, kNW, QD, XL, APPEND, DIRECT, PV>,
                         stream_lds_bytes(D, kNW, stream_qslot(kMaxGroupS, D, APPEND), APPEND, side));
  if (attr_err != hipSuccess) return attr_err;
  hipLaunchKernelGGL((attn_stream_kernel<T, D, kNW, QD, XL, APPEND, DIRECT, PV>), dim3((unsigned)n_wg), dim3(kNW * 64), lds,
                     st, ap.cu, ap.base, ap.cap, ap.q, ap.k, ap.v, ap.n_seg,
                     (int32_t)((uint32_t)ap.G | ((uint32_t)n_wg << 8)), ap.split_inv, ap);
  return hipGetLastError();
}

// Up to 64 segments the table is read by every wave directly (one lane per
// segment); more take the workgroup scheduling pass.
template <typename T, int D, int QD, bool XL, bool APPEND>
static hipError_t launch_stream(const AttnParams& ap, int64_t n_wg, hipStream_t st) {
  if constexpr (APPEND) {
    if (ap.pv_xlog)  // the host allows it with the direct table only
      return ap.n_seg <= 64 ? launch_stream_k<T, D, QD, XL, APPEND, true, true>(ap, n_wg, st) : hipErrorInvalidValue;
  }
  return ap.n_seg <= 64 ? launch_stream_k<T, D, QD, XL, APPEND, true>(ap, n_wg, st)
                        : launch_stream_k<T, D, QD, XL, APPEND, false>(ap, n_wg, st);
}

template <typename T, int D, int QD>
static hipError_t launch_stream_qd(const AttnParams& ap, int64_t n_wg, hipStream_t st) {
  if (ap.new_k)
    return ap.xlog ? launch_stream<T, D, QD, true, true>(ap, n_wg, st)
                   : launch_stream<T, D, QD, false, true>(ap, n_wg, st);
  return ap.xlog ? launch_stream<T, D, QD, true, false>(ap, n_wg, st)
                 : launch_stream<T, D, QD, false, false>(ap, n_wg, st);
}

template <typename T, int D>
static hipError_t launch_attn(int kernel, const AttnParams& ap, int64_t n_wg, hipStream_t st) {
  if (kernel == WNW_ATTN_STREAM) {
    if constexpr (sizeof(T) == 2 && (D == 64 || D == 128)) {
      const int qd = (ap.G * D * 2 + 1023) / 1024;
      if (ap.G <= kMaxGroupS) {
        if constexpr (D == 128)
          if (qd == 2) return launch_stream_qd<T, D, 2>(ap, n_wg, st);
        if (qd == 1) return launch_stream_qd<T, D, 1>(ap, n_wg, st);
      }
    }
    return hipErrorInvalidValue;
  }
  if (kernel == WNW_ATTN_MFMA) {
    if constexpr (sizeof(T) == 2 && (D == 64 || D == 128)) {
      hipLaunchKernelGGL((attn_mfma_kernel<T, D, kNW>), dim3((unsigned)n_wg), dim3(kNW * 64), 0, st, ap);
      return hipGetLastError();
    }
    return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL((attn_valu_kernel<T, D, kNW>), dim3((unsigned)n_wg), dim3(kNW * 64), 0, st, ap);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_attn_d(int kernel, int64_t D, const AttnParams& ap, int64_t n_wg, hipStream_t st) {
  switch (D) {
    case 64: return launch_attn<T, 64>(kernel, ap, n_wg, st);
    case 128: return launch_attn<T, 128>(kernel, ap, n_wg, st);
    case 256: return launch_attn<T, 256>(kernel, ap, n_wg, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace wnw

using namespace wnw;

extern "C" int64_t wnw_decode_attn_workspace_bytes(int64_t n_seg, int64_t group, int64_t head_dim) {
  if (n_seg < 0 || group <= 0 || head_dim <= 0) return -1;
  return ws_layout(n_seg, group, head_dim).total;
}

extern "C" int wnw_workspace_init(void* workspace, int64_t workspace_bytes, void* stream) {
  WNW_CHECK_ARG(workspace != nullptr || workspace_bytes == 0, "workspace is null");
  WNW_CHECK_ARG(workspace_bytes % 4 == 0, "workspace_bytes must be a multiple of 4");
  if (workspace_bytes == 0) return WNW_OK;
  const int64_t n = workspace_bytes / 4;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (uint32_t*)workspace, n);
  WNW_CHECK_HIP(hipGetLastError(), "workspace init launch");
  return WNW_OK;
}

namespace wnw {
// The current device's scratch address (resolved once per device; the
// counters region is cleared with a fill kernel on the first call, which
// may be under graph capture, so no memset node is recorded).
static int noalloc_scratch(hipStream_t st, void** out) {
  static std::mutex mu;
  static std::vector<ScratchSlot> slots;
  int dev = 0;
  WNW_CHECK_HIP(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lock(mu);
  if ((int)slots.size() <= dev) slots.resize(dev + 1);
  ScratchSlot& sl = slots[dev];
  if (!sl.ptr) {
    void* p = nullptr;
    WNW_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(g_attn_scratch)), "resolving the attention scratch");
    WNW_CHECK_ARG(p != nullptr, "the attention scratch has no device address");
    sl.ptr = p;
  }
  if (!sl.cleared) {
    const int64_t n = (int64_t)WNW_NOALLOC_MAX_SEG;  // counters, 4 bytes each
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, (uint32_t*)sl.ptr, n);
    WNW_CHECK_HIP(hipGetLastError(), "clearing the attention scratch counters");
    sl.cleared = true;
  }
  *out = sl.ptr;
  return WNW_OK;
}

int decode_attn_impl(const void* q, const void* k, const void* v, const int32_t* cu_k,
                     const int64_t* seg_base, int64_t n_seg, int64_t group, int64_t head_dim,
                     int64_t total_rows, int64_t kv_rows, float scale, int dtype, void* out,
                     void* workspace, int64_t workspace_bytes, int kernel, int64_t n_wg, float* lse,
                     const AttnLogits* logits, int* logits_kept, void* stream, bool noalloc,
                     const AttnAppend* app, const AttnPrevScore* prev) {
  if (logits_kept) *logits_kept = 0;
  WNW_CHECK_ARG(n_seg >= 0 && n_seg < (1ll << 30), "n_seg out of range: %lld", (long long)n_seg);
  if (n_seg == 0) return WNW_OK;
  WNW_CHECK_ARG(q && cu_k && out && (workspace || noalloc) && ((k && v) || kv_rows == 0),
                "null pointer argument");
  WNW_CHECK_ARG(group >= 1 && group <= kMaxGroup, "group must be in [1, %d], got %lld", kMaxGroup,
                (long long)group);
  WNW_CHECK_ARG(head_dim == 64 || head_dim == 128 || head_dim == 256,
                "head_dim must be 64, 128 or 256, got %lld", (long long)head_dim);
  WNW_CHECK_ARG(dtype == WNW_F32 || dtype == WNW_F16 || dtype == WNW_BF16, "bad dtype %d", dtype);
  WNW_CHECK_ARG(total_rows >= 0 && kv_rows >= 0, "negative row count");
  if (app) {
    WNW_CHECK_ARG(seg_base && app->new_k && app->new_v && app->cu_out && app->cap,
                  "the fused append needs seg_base, new rows, cu_out and seg_cap");
    WNW_CHECK_ARG((const void*)app->cu_out != (const void*)cu_k, "cu_out must not alias cu");
    WNW_CHECK_ARG(((uintptr_t)app->new_k % 16) == 0 && ((uintptr_t)app->new_v % 16) == 0,
                  "new_k and new_v must be 16-byte aligned");
  }
  WNW_CHECK_ARG(kv_rows < (1ll << 40), "kv_rows too large");
  WNW_CHECK_ARG(((uintptr_t)q % 16) == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0 &&
                    ((uintptr_t)out % 16) == 0,
                "q, k, v and out must be 16-byte aligned");
  int kern = kernel;
  if (kern == WNW_ATTN_AUTO)
    kern = (dtype != WNW_F32 && (head_dim == 64 || head_dim == 128))
               ? (group <= kMaxGroupS ? WNW_ATTN_STREAM : WNW_ATTN_MFMA)
               : WNW_ATTN_VALU;
  WNW_CHECK_ARG(kern == WNW_ATTN_MFMA || kern == WNW_ATTN_VALU || kern == WNW_ATTN_STREAM, "bad kernel id %d",
                kernel);
  if (kern == WNW_ATTN_STREAM)
    WNW_CHECK_ARG(dtype != WNW_F32 && (head_dim == 64 || head_dim == 128) && group <= kMaxGroupS,
                  "the streaming kernel needs bf16/f16, head_dim 64 or 128 and group <= %d", kMaxGroupS);
  if (kern == WNW_ATTN_MFMA)
    WNW_CHECK_ARG(dtype != WNW_F32 && (head_dim == 64 || head_dim == 128),
                  "the MFMA kernel needs bf16/f16 and head_dim 64 or 128");
  const DeviceInfo& di = device_info();
  int64_t P = n_wg;
  if (P <= 0) {
    // Balanced split of the rows, never fewer than ~64 rows per workgroup:
    // one workgroup per CU for the streaming kernel (its four waves keep
    // enough loads in flight, and fewer workgroups mean fewer partials to
    // merge), two per CU for the others.
    const int64_t by_rows = std::max<int64_t>(1, (total_rows + 63) / 64);
    P = std::min<int64_t>((int64_t)di.cus * (kern == WNW_ATTN_STREAM ? 1 : 2), by_rows);
  }
  P = std::max<int64_t>(1, std::min<int64_t>(P, di.max_wg));
  WsLayout L;
  if (noalloc) {
    WNW_CHECK_ARG(n_seg <= WNW_NOALLOC_MAX_SEG, "the no-alloc entry point takes at most %d segments, got %lld",
                  WNW_NOALLOC_MAX_SEG, (long long)n_seg);
    L = make_layout(WNW_NOALLOC_MAX_SEG, P + n_seg, group, head_dim);
    WNW_CHECK_ARG(L.total <= kNoAllocBytes,
                  "this launch needs %lld bytes of split-K scratch; the no-alloc entry point holds %lld "
                  "(fewer segments or a smaller group / head_dim fit)",
                  (long long)L.total, (long long)kNoAllocBytes);
    const int rc = noalloc_scratch((hipStream_t)stream, &workspace);
    if (rc != WNW_OK) return rc;
  } else {
    L = ws_layout(n_seg, group, head_dim);
    WNW_CHECK_ARG(workspace_bytes >= L.total, "workspace too small: %lld < %lld bytes",
                  (long long)workspace_bytes, (long long)L.total);
  }

  AttnParams ap;
  ap.q = q;
  ap.k = k;
  ap.v = v;
  ap.cu = cu_k;
  ap.base = seg_base;
  ap.out = out;
  ap.counters = (int32_t*)((char*)workspace + L.counters);
  ap.lse = lse;
  ap.part_ml = (float*)((char*)workspace + L.ml);
  ap.part_acc = (float*)((char*)workspace + L.acc);
  ap.err = device_error_word();
  ap.split_inv = ~0ull / (uint64_t)(P * kSplitWaves) + 1;  // ceil(2^64 / (P * kSplitWaves))
  ap.phys_rows = kv_rows;
  ap.n_seg = (int32_t)n_seg;
  ap.G = (int32_t)group;
  ap.scale_log2 = scale * kLog2e;
  ap.xlog = nullptr;
  ap.xmask = ap.audio_s = ap.audio_e = nullptr;
  ap.max_audio = 0;
  ap.Hkv = 1;
  ap.new_k = ap.new_v = nullptr;
  ap.cu_out = nullptr;
  ap.cap = nullptr;
  ap.pv_xlog = ap.pv_lse = nullptr;
  ap.pv_kvlist = 0;
  ap.pv_nkv = 0;
  ap.pv_slices = 0;
  ap.pv_cu = ap.pv_acc_off = nullptr;
  ap.pv_base = nullptr;
  ap.pv_acc = nullptr;
  ap.pv_kv_rows = ap.pv_acc_len = 0;
  ap.pv_nblk = 0;
  if (prev) {
    // deferred scoring rides in the streaming kernel's direct-table form
    // only, one slice of 256 tokens per workgroup: elsewhere the caller
    // scores the slot in its own launch
    WNW_CHECK_ARG(prev->xlog && prev->lse && prev->cu && prev->acc && prev->acc_off && prev->audio_s &&
                      prev->audio_e,
                  "null deferred-scoring argument");
    WNW_CHECK_ARG(prev->hkv >= 1 && n_seg % prev->hkv == 0 && prev->max_audio > 0 && prev->kv_rows >= 0 &&
                      prev->acc_len >= 0,
                  "bad deferred-scoring geometry");
    const int64_t nblk = (prev->max_audio + 255) / 256;
    int nkv = 0;
    uint64_t kvlist = 0;
    for (int h = 0; h < prev->hkv && h < 64; ++h)
      if ((prev->kv_bits >> h) & 1) {
        if (nkv < 8) kvlist |= (uint64_t)h << (8 * nkv);
        ++nkv;
      }
    WNW_CHECK_ARG(prev->hkv <= 64 && (prev->hkv == 64 || (prev->kv_bits >> prev->hkv) == 0),
                  "deferred-scoring KV heads outside [0, %d)", prev->hkv);
    if (kern != WNW_ATTN_STREAM || n_seg > 64 || nkv > 8 || nkv * group > kPrevLogits ||
        (n_seg / prev->hkv) * nblk > P) {
      set_error("deferred scoring needs the streaming kernel, at most 64 segments, at most 8 scored KV heads "
                "and %d (KV head, query head) pairs, and one 256-token slice per workgroup (%lld slices, %lld "
                "workgroups)",
                kPrevLogits, (long long)((n_seg / prev->hkv) * nblk), (long long)P);
      return WNW_ENOTSUP;
    }
    if (logits && kern == WNW_ATTN_STREAM)
      WNW_CHECK_ARG(logits->hkv == prev->hkv && logits->max_audio == prev->max_audio &&
                        logits->audio_s == prev->audio_s && logits->audio_e == prev->audio_e,
                    "the deferred scoring and this launch's logits must share the audio geometry");
    ap.pv_xlog = nkv > 0 ? prev->xlog : nullptr;  // nothing scored: nothing to do
    ap.pv_lse = prev->lse;
    ap.pv_kvlist = kvlist;
    ap.pv_nkv = nkv;
    ap.pv_slices = (int32_t)((n_seg / prev->hkv) * nblk);
    ap.pv_cu = prev->cu;
    ap.pv_base = prev->base;
    ap.pv_kv_rows = prev->kv_rows;
    ap.pv_acc = prev->acc;
    ap.pv_acc_off = prev->acc_off;
    ap.pv_acc_len = prev->acc_len;
    ap.pv_nblk = (int32_t)nblk;
    ap.audio_s = prev->audio_s;
    ap.audio_e = prev->audio_e;
    ap.max_audio = prev->max_audio;
    ap.Hkv = prev->hkv;
  }
  hipStream_t st = (hipStream_t)stream;
  if (app) {
    if (kern == WNW_ATTN_STREAM) {  // fused into the launch
      ap.new_k = app->new_k;
      ap.new_v = app->new_v;
      ap.cu_out = app->cu_out;
      ap.cap = app->cap;
    } else {  // the in-place append first, then attention over the new offsets
      const int rc = wnw_append_inplace(const_cast<void*>(k), const_cast<void*>(v), app->new_k, app->new_v, cu_k,
                                        app->cu_out, seg_base, app->cap, n_seg, kv_rows, head_dim, dtype, stream);
      if (rc != WNW_OK) return rc;
      ap.cu = app->cu_out;
    }
  }
  if (logits && kern == WNW_ATTN_STREAM) {
    WNW_CHECK_ARG(logits->xlog && logits->mask && logits->audio_s && logits->audio_e, "null logits argument");
    WNW_CHECK_ARG(logits->hkv >= 1 && n_seg % logits->hkv == 0 && logits->max_audio > 0,
                  "bad logits geometry");
    ap.xlog = logits->xlog;
    ap.xmask = logits->mask;
    ap.audio_s = logits->audio_s;
    ap.audio_e = logits->audio_e;
    ap.max_audio = logits->max_audio;
    ap.Hkv = logits->hkv;
    if (logits_kept) *logits_kept = 1;
  }
  hipError_t e = hipErrorInvalidValue;
  switch (dtype) {
    case WNW_BF16: e = launch_attn_d<bf16_t>(kern, head_dim, ap, P, st); break;
    case WNW_F16: e = launch_attn_d<f16_t>(kern, head_dim, ap, P, st); break;
    case WNW_F32: e = launch_attn_d<float>(kern, head_dim, ap, P, st); break;
  }
  WNW_CHECK_HIP(e, "decode attention launch");
  return WNW_OK;
}

}  // namespace wnw

extern "C" int wnw_decode_attn_ex(const void* q, const void* k, const void* v, const int32_t* cu_k,
                                  const int64_t* seg_base, int64_t n_seg, int64_t group,
                                  int64_t head_dim, int64_t total_rows, int64_t kv_rows, float scale,
                                  int dtype, void* out, void* workspace, int64_t workspace_bytes,
                                  int kernel, int64_t n_wg, void* stream) {
  return decode_attn_impl(q, k, v, cu_k, seg_base, n_seg, group, head_dim, total_rows, kv_rows, scale,
                          dtype, out, workspace, workspace_bytes, kernel, n_wg, nullptr, nullptr, nullptr,
                          stream, false, nullptr);
}

extern "C" int wnw_decode_attn(const void* q, const void* k, const void* v, const int32_t* cu_k,
                               const int64_t* seg_base, int64_t n_seg, int64_t group,
                               int64_t head_dim, int64_t total_rows, int64_t kv_rows, float scale,
                               int dtype, void* out, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  return wnw_decode_attn_ex(q, k, v, cu_k, seg_base, n_seg, group, head_dim, total_rows, kv_rows,
                            scale, dtype, out, workspace, workspace_bytes, WNW_ATTN_AUTO, 0, stream);
}

extern "C" int wnw_decode_attn_noalloc(const void* q, const void* k, const void* v, const int32_t* cu_k,
                                       const int64_t* seg_base, int64_t n_seg, int64_t group,
                                       int64_t head_dim, int64_t total_rows, int64_t kv_rows, float scale,
                                       int dtype, void* out, void* stream) {
  return decode_attn_impl(q, k, v, cu_k, seg_base, n_seg, group, head_dim, total_rows, kv_rows, scale,
                          dtype, out, nullptr, 0, WNW_ATTN_AUTO, 0, nullptr, nullptr, nullptr, stream, true,
                          nullptr);
}

extern "C" int wnw_decode_attn_append(const void* q, void* k_pool, void* v_pool, const void* new_k,
                                      const void* new_v, const int32_t* cu_old, int32_t* cu_new,
                                      const int64_t* seg_base, const int32_t* seg_cap, int64_t n_seg,
                                      int64_t group, int64_t head_dim, int64_t total_rows, int64_t pool_rows,
                                      float scale, int dtype, void* out, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  AttnAppend app;
  app.new_k = new_k;
  app.new_v = new_v;
  app.cu_out = cu_new;
  app.cap = seg_cap;
  return decode_attn_impl(q, k_pool, v_pool, cu_old, seg_base, n_seg, group, head_dim, total_rows, pool_rows,
                          scale, dtype, out, workspace, workspace_bytes, WNW_ATTN_AUTO, 0, nullptr, nullptr,
                          nullptr, stream, false, &app);
}

// Append and compaction kernels of the flat varlen KV layout (gfx950).
//
// All of them are row gathers: every output row is one input row (an old
// row, a row loaded from the host, or the step's new token) moved verbatim,
// so results are bit-exact by construction.  Rows move in 16-byte chunks;
// a 256-thread workgroup moves a block of consecutive output rows, so every
// wave instruction reads and writes whole contiguous row spans.
#include <algorithm>

#include "wnw_common.h"

namespace wnw {

static constexpr int kNT = 256;
static constexpr int kRows = 64;  // output rows per workgroup
static constexpr int kSegRing = 64;

// Segments overlapping one output-row block, found with one pass of
// independent loads over cu_out (the output offsets).
struct BlockSegs {
  int32_t s_first, s_last;
  int32_t out_lo[kSegRing], out_hi[kSegRing];
};

__device__ void scan_block_segments(const int32_t* cu_out, int N, int64_t B0, int64_t B1,
                                    BlockSegs& bs, int32_t* err) {
  const int tid = threadIdx.x;
  if (tid == 0) {
    bs.s_first = 0x7fffffff;
    bs.s_last = -1;
  }
  __syncthreads();
  for (int i0 = 0; i0 < N; i0 += 4 * kNT) {
    int32_t lo[4], hi[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * kNT + tid;
      lo[u] = hi[u] = 0;
      if (i < N) {
        lo[u] = cu_out[i];
        hi[u] = cu_out[i + 1];
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * kNT + tid;
      if (i >= N) continue;
      if (hi[u] < lo[u]) {
        raise_device_error(err, WNW_DEVERR_ORDER);
        continue;
      }
      // "touching" ranges: every segment between s_first and s_last
      // (empty ones included) gets a ring entry.
      if (lo[u] <= B1 && hi[u] >= B0) {
        atomicMin(&bs.s_first, i);
        atomicMax(&bs.s_last, i);
        bs.out_lo[i % kSegRing] = lo[u];
        bs.out_hi[i % kSegRing] = hi[u];
      }
    }
  }
  __syncthreads();
}

// Segment of output row j (s_first <= s <= s_last, rows are contiguous).
__device__ __forceinline__ int seg_of_row(const BlockSegs& bs, const int32_t* cu_out, int64_t j) {
  const bool ring = bs.s_last - bs.s_first < kSegRing;
  int s = bs.s_first;
  while (s < bs.s_last) {
    const int64_t hi = ring ? bs.out_hi[s % kSegRing] : cu_out[s + 1];
    if (j < hi) break;
    ++s;
  }
  return s;
}

__device__ __forceinline__ int64_t seg_lo(const BlockSegs& bs, const int32_t* cu_out, int s) {
  return (bs.s_last - bs.s_first < kSegRing) ? bs.out_lo[s % kSegRing] : cu_out[s];
}
__device__ __forceinline__ int64_t seg_hi(const BlockSegs& bs, const int32_t* cu_out, int s) {
  return (bs.s_last - bs.s_first < kSegRing) ? bs.out_hi[s % kSegRing] : cu_out[s + 1];
}

// Where each output row of a block comes from, resolved once per row by the
// block's first wave (the lookups are short chains of dependent loads), so
// that the copy loop below issues its data loads back to back.
enum RowKind : int32_t { kOld = 0, kLoad = 1, kNew = 2, kNone = 3 };
struct RowSrc {
  int64_t row[kRows];   // source row in the tensor its kind names
  int32_t kind[kRows];  // RowKind; kNone writes zeros (an error was raised)
};

// Copies the block's nrows rows: output row out_row0 + r <- row rs.row[r] of
// (k, v)[rs.kind[r]].  Each thread has four 16-byte chunks of each tensor in
// flight; a wave's loads and stores cover contiguous spans of the rows.  NT:
// non-temporal loads and stores, for copies larger than the 256 MB
// Infinity Cache, which they would only stream through (measured at cfg5:
// 859 MB per layer, 161 -> 151 us; at cfg2, 149 MB, plain accesses are
// faster: 27.5 vs 28.8 us).
template <bool KV, bool NT = false>
__device__ __forceinline__ void copy_rows(const RowSrc& rs, int nrows, int cpr, const u32x4* k0,
                                          const u32x4* v0, const u32x4* k1, const u32x4* v1,
                                          const u32x4* k2, const u32x4* v2, int64_t out_row0,
                                          u32x4* out_k, u32x4* out_v) {
  constexpr int U = 4;
  const int n = nrows * cpr;
  WNW_GLOBAL u32x4* ok = (WNW_GLOBAL u32x4*)out_k + out_row0 * cpr;
  WNW_GLOBAL u32x4* ov = KV ? (WNW_GLOBAL u32x4*)out_v + out_row0 * cpr : nullptr;
  for (int x0 = threadIdx.x; x0 < n; x0 += U * kNT) {
    u32x4 a[U], b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int x = x0 + u * kNT;
      a[u] = b[u] = u32x4{0, 0, 0, 0};
      if (x < n) {
        const int r = x / cpr;
        const int kind = rs.kind[r];
        if (kind != kNone) {
          const int64_t off = rs.row[r] * cpr + (x - r * cpr);
          const u32x4* pk = kind == kOld ? k0 : kind == kLoad ? k1 : k2;
          if (NT)
            a[u] = __builtin_nontemporal_load((const WNW_GLOBAL u32x4*)pk + off);
          else
            a[u] = ((const WNW_GLOBAL u32x4*)pk)[off];
          if (KV) {
            const u32x4* pv = kind == kOld ? v0 : kind == kLoad ? v1 : v2;
            if (NT)
              b[u] = __builtin_nontemporal_load((const WNW_GLOBAL u32x4*)pv + off);
            else
              b[u] = ((const WNW_GLOBAL u32x4*)pv)[off];
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int x = x0 + u * kNT;
      if (x < n) {
        if (NT) {
          __builtin_nontemporal_store(a[u], ok + x);
          if (KV) __builtin_nontemporal_store(b[u], ov + x);
        } else {
          ok[x] = a[u];
          if (KV) ov[x] = b[u];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// interleave_append (reference src/common/kv/kernels.py:7-73)
// ---------------------------------------------------------------------------
// KV: K and V appended in one launch (the rows' sources are resolved once
// for both tensors, as in the rebuild kernel).
template <bool KV>
__global__ __launch_bounds__(kNT) void interleave_append_kernel(
    const u32x4* __restrict__ old_rows, const u32x4* __restrict__ new_rows,
    const int32_t* __restrict__ cu_old, const int32_t* __restrict__ cu_new, int N,
    int64_t total_old, int64_t total_out, int cpr, u32x4* __restrict__ out, int32_t* err,
    const u32x4* __restrict__ old_v = nullptr, const u32x4* __restrict__ new_v = nullptr,
    u32x4* __restrict__ out_v = nullptr) {
  __shared__ BlockSegs bs;
  __shared__ RowSrc rs;
  const int64_t B0 = (int64_t)blockIdx.x * kRows;
  const int64_t B1 = min(B0 + kRows, total_out);
  const int nrows = (int)(B1 - B0);
  scan_block_segments(cu_new, N, B0, B1, bs, err);
  if ((int)threadIdx.x < nrows) {
    const int64_t j = B0 + threadIdx.x;
    int kind = kNone;
    int64_t src = 0;
    if (bs.s_first > bs.s_last || j >= seg_hi(bs, cu_new, bs.s_last) || j < seg_lo(bs, cu_new, bs.s_first)) {
      raise_device_error(err, WNW_DEVERR_BOUNDS);  // row not covered by cu_new
    } else {
      const int s = seg_of_row(bs, cu_new, j);
      const int64_t i = j - seg_lo(bs, cu_new, s);
      const int64_t olo = cu_old[s], ohi = cu_old[s + 1];
      if (i < ohi - olo) {
        src = olo + i;
        if (src >= 0 && src < total_old)
          kind = kOld;
        else
          raise_device_error(err, WNW_DEVERR_BOUNDS);
      } else {
        src = s;
        kind = kNew;
      }
    }
    rs.kind[threadIdx.x] = kind;
    rs.row[threadIdx.x] = src;
  }
  __syncthreads();
  copy_rows<KV>(rs, nrows, cpr, old_rows, old_v, nullptr, nullptr, new_rows, new_v, B0, out, out_v);
}

// ---------------------------------------------------------------------------
// rebuild_append_kv (reference src/algorithms/wnw/code/kernels.py:375-473)
// ---------------------------------------------------------------------------
struct RebuildDesc {
  const int32_t* load_starts;
  const int32_t* load_lens;
  const int32_t* evict_offsets;
  const int32_t* evict_starts;
  const int32_t* evict_ends;
  int64_t n_evict;  // entries in evict_starts / evict_ends
  int32_t max_evict;
};

// Source of row i (relative) of a rebuilt segment: a RowKind (kNone for an
// invalid descriptor: evict indices outside [0, n_evict)).  Follows the
// reference's index arithmetic exactly: kept_len subtracts the first
// min(n_evict, max_evict) ranges; an old row is found by walking those
// ranges in order, skipping each range that starts at or before the running
// source index.  The descriptor arrays reach the kernel inside a struct, so
// they are read through global-address-space pointers.
__device__ __forceinline__ int rebuild_source(const RebuildDesc& d, int s, int64_t old_len,
                                              int64_t i, int64_t& src) {
  const WNW_GLOBAL int32_t* eoff = gptr<int32_t>(d.evict_offsets);
  const WNW_GLOBAL int32_t* est = gptr<int32_t>(d.evict_starts);
  const WNW_GLOBAL int32_t* een = gptr<int32_t>(d.evict_ends);
  // every descriptor of the segment is read up front (independent loads)
  const int e0 = eoff[s];
  const int e1 = eoff[s + 1];
  const int64_t ll = gptr<int32_t>(d.load_lens)[s];
  const int64_t ls = gptr<int32_t>(d.load_starts)[s];
  const int ne = min(e1 - e0, d.max_evict);
  if (ne > 0 && (e0 < 0 || (int64_t)e0 + ne > d.n_evict)) return kNone;
  // The evict ranges are read in batches of kEB whose loads are issued
  // together (one memory round trip per batch, not per range); entries past
  // ne read the last range again and count as empty.
  constexpr int kEB = 8;
  int64_t kept = old_len;
  for (int b0 = 0; b0 < ne; b0 += kEB) {
    int32_t es[kEB], ee[kEB];
#pragma unroll
    for (int u = 0; u < kEB; ++u) {
      const int e = e0 + min(b0 + u, ne - 1);
      es[u] = est[e];
      ee[u] = een[e];
    }
#pragma unroll
    for (int u = 0; u < kEB; ++u)
      if (b0 + u < ne) kept -= (int64_t)ee[u] - es[u];
  }
  if (i < kept) {
    int64_t rel = i;
    for (int b0 = 0; b0 < ne; b0 += kEB) {
      int32_t es[kEB], ee[kEB];
#pragma unroll
      for (int u = 0; u < kEB; ++u) {
        const int e = e0 + min(b0 + u, ne - 1);
        es[u] = est[e];
        ee[u] = een[e];
      }
#pragma unroll
      for (int u = 0; u < kEB; ++u)
        if (b0 + u < ne && rel >= es[u]) rel += (int64_t)ee[u] - es[u];
    }
    src = rel;
    return kOld;
  }
  if (i < kept + ll) {
    src = ls + (i - kept);
    return kLoad;
  }
  src = s;
  return kNew;
}

template <bool NT>
__global__ __launch_bounds__(kNT) void rebuild_append_kernel(
    const u32x4* __restrict__ old_k, const u32x4* __restrict__ old_v,
    const u32x4* __restrict__ new_k, const u32x4* __restrict__ new_v,
    const u32x4* __restrict__ load_k, const u32x4* __restrict__ load_v,
    const int32_t* __restrict__ old_cu, const int32_t* __restrict__ new_cu, RebuildDesc d, int N,
    int64_t total_old, int64_t total_load, int64_t total_out, int cpr, u32x4* __restrict__ out_k,
    u32x4* __restrict__ out_v, int32_t* err) {
  __shared__ BlockSegs bs;
  __shared__ RowSrc rs;
  const int64_t B0 = (int64_t)blockIdx.x * kRows;
  const int64_t B1 = min(B0 + kRows, total_out);
  const int nrows = (int)(B1 - B0);
  scan_block_segments(new_cu, N, B0, B1, bs, err);
  if ((int)threadIdx.x < nrows) {
    const int64_t j = B0 + threadIdx.x;
    int kind = kNone;
    int64_t src = 0;
    if (bs.s_first > bs.s_last || j >= seg_hi(bs, new_cu, bs.s_last) || j < seg_lo(bs, new_cu, bs.s_first)) {
      raise_device_error(err, WNW_DEVERR_BOUNDS);
    } else {
      const int s = seg_of_row(bs, new_cu, j);
      const int64_t i = j - seg_lo(bs, new_cu, s);
      const int64_t olo = old_cu[s], ohi = old_cu[s + 1];
      kind = rebuild_source(d, s, ohi - olo, i, src);
      if (kind == kOld) {
        src += olo;
        if (src < 0 || src >= total_old) kind = kNone;
      } else if (kind == kLoad) {
        if (src < 0 || src >= total_load) kind = kNone;
      }
      if (kind == kNone) raise_device_error(err, WNW_DEVERR_BOUNDS);
    }
    rs.kind[threadIdx.x] = kind;
    rs.row[threadIdx.x] = src;
  }
  __syncthreads();
  copy_rows<true, NT>(rs, nrows, cpr, old_k, old_v, load_k, load_v, new_k, new_v, B0, out_k, out_v);
}

// ---------------------------------------------------------------------------
// compaction of listed segments between physical layouts
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kNT) void compact_segments_kernel(
    const u32x4* __restrict__ src_k, const u32x4* __restrict__ src_v, u32x4* __restrict__ dst_k,
    u32x4* __restrict__ dst_v, const u32x4* __restrict__ new_k, const u32x4* __restrict__ new_v,
    const u32x4* __restrict__ load_k, const u32x4* __restrict__ load_v,
    const int32_t* __restrict__ seg_list, int n_seg, const int64_t* __restrict__ src_base,
    const int32_t* __restrict__ src_len, const int64_t* __restrict__ dst_base,
    const int32_t* __restrict__ new_len, RebuildDesc d, int with_new, int64_t src_rows,
    int64_t dst_rows, int64_t load_rows, int cpr, int32_t* err) {
  __shared__ RowSrc rs;
  const int s = seg_list[blockIdx.y];
  if (s < 0 || s >= n_seg) {
    if (blockIdx.x == 0 && threadIdx.x == 0) raise_device_error(err, WNW_DEVERR_BOUNDS);
    return;
  }
  const int64_t nl = new_len[s];
  const int64_t r0 = (int64_t)blockIdx.x * kRows;
  if (r0 >= nl) return;
  const int64_t r1 = min(r0 + kRows, nl);
  const int nrows = (int)(r1 - r0);
  const int64_t sb = src_base[s], sl = src_len[s], db = dst_base[s];
  if (db < 0 || db + nl > dst_rows || sb < 0 || sb + sl > src_rows) {
    if (threadIdx.x == 0) raise_device_error(err, WNW_DEVERR_BOUNDS);
    return;
  }
  if ((int)threadIdx.x < nrows) {
    const int64_t i = r0 + threadIdx.x;
    int64_t src = 0;
    int kind = rebuild_source(d, s, sl, i, src);
    if (kind == kOld) {
      if (src >= 0 && src < sl)
        src += sb;
      else
        kind = kNone;
    } else if (kind == kLoad) {
      if (src < 0 || src >= load_rows) kind = kNone;
    } else if (kind == kNew) {
      if (!with_new || i != nl - 1) kind = kNone;  // only the last row is the new one
    }
    if (kind == kNone) raise_device_error(err, WNW_DEVERR_BOUNDS);
    rs.kind[threadIdx.x] = kind;
    rs.row[threadIdx.x] = src;
  }
  __syncthreads();
  copy_rows<true>(rs, nrows, cpr, src_k, src_v, load_k, load_v, new_k, new_v, db + r0, dst_k, dst_v);
}

// ---------------------------------------------------------------------------
// in-place append into per-segment slack
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kNT) void append_inplace_kernel(
    u32x4* __restrict__ k_pool, u32x4* __restrict__ v_pool, const u32x4* __restrict__ new_k,
    const u32x4* __restrict__ new_v, const int32_t* __restrict__ cu_old, int32_t* __restrict__ cu_new,
    const int64_t* __restrict__ seg_base, const int32_t* __restrict__ seg_cap, int N,
    int64_t pool_rows, int cpr, int32_t* err) {
  const int64_t x = (int64_t)blockIdx.x * kNT + threadIdx.x;
  if (x <= N) cu_new[x] = cu_old[x] + (int32_t)x;
  if (x >= (int64_t)N * cpr) return;
  const int s = (int)(x / cpr);
  const int c = (int)(x % cpr);
  const int64_t len = (int64_t)cu_old[s + 1] - cu_old[s];
  const int64_t b = seg_base[s];
  const int64_t dst = b + len;
  if (len < 0 || len + 1 > seg_cap[s]) {
    if (c == 0) raise_device_error(err, WNW_DEVERR_CAPACITY);
    return;
  }
  if (b < 0 || dst >= pool_rows) {
    if (c == 0) raise_device_error(err, WNW_DEVERR_BOUNDS);
    return;
  }
  k_pool[dst * cpr + c] = new_k[(int64_t)s * cpr + c];
  v_pool[dst * cpr + c] = new_v[(int64_t)s * cpr + c];
}

static int check_rows(int64_t head_dim, int dtype, int& cpr) {
  WNW_CHECK_ARG(dtype == WNW_F32 || dtype == WNW_F16 || dtype == WNW_BF16, "bad dtype %d", dtype);
  WNW_CHECK_ARG(head_dim > 0 && (head_dim * elem_bytes(dtype)) % 16 == 0 && head_dim <= 4096,
                "head_dim * element size must be a positive multiple of 16 bytes (head_dim %lld)",
                (long long)head_dim);
  cpr = (int)(head_dim * elem_bytes(dtype) / 16);
  return WNW_OK;
}

static bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

}  // namespace wnw

using namespace wnw;

extern "C" int wnw_interleave_append(const void* old_rows, const void* new_rows, const int32_t* cu_old,
                                     const int32_t* cu_new, int64_t n_seg, int64_t total_old,
                                     int64_t head_dim, int dtype, void* out, void* stream) {
  int cpr = 0;
  if (int rc = check_rows(head_dim, dtype, cpr)) return rc;
  WNW_CHECK_ARG(n_seg >= 0 && n_seg < (1 << 30) && total_old >= 0, "bad sizes");
  const int64_t total_out = total_old + n_seg;
  if (total_out == 0) return WNW_OK;
  WNW_CHECK_ARG(new_rows && cu_old && cu_new && out && (old_rows || total_old == 0), "null pointer argument");
  WNW_CHECK_ARG(aligned16(old_rows) && aligned16(new_rows) && aligned16(out), "rows must be 16-byte aligned");
  const int64_t blocks = (total_out + kRows - 1) / kRows;
  WNW_CHECK_ARG(blocks < (1ll << 31), "too many rows");
  hipLaunchKernelGGL(interleave_append_kernel<false>, dim3((unsigned)blocks), dim3(kNT), 0, (hipStream_t)stream,
                     (const u32x4*)old_rows, (const u32x4*)new_rows, cu_old, cu_new, (int)n_seg, total_old, total_out,
                     cpr, (u32x4*)out, device_error_word(), nullptr, nullptr, nullptr);
  WNW_CHECK_HIP(hipGetLastError(), "interleave_append launch");
  return WNW_OK;
}

extern "C" int wnw_interleave_append_kv(const void* old_k, const void* old_v, const void* new_k, const void* new_v,
                                        const int32_t* cu_old, const int32_t* cu_new, int64_t n_seg,
                                        int64_t total_old, int64_t head_dim, int dtype, void* out_k, void* out_v,
                                        void* stream) {
  int cpr = 0;
  if (int rc = check_rows(head_dim, dtype, cpr)) return rc;
  WNW_CHECK_ARG(n_seg >= 0 && n_seg < (1 << 30) && total_old >= 0, "bad sizes");
  const int64_t total_out = total_old + n_seg;
  if (total_out == 0) return WNW_OK;
  WNW_CHECK_ARG(new_k && new_v && cu_old && cu_new && out_k && out_v && ((old_k && old_v) || total_old == 0),
                "null pointer argument");
  WNW_CHECK_ARG(aligned16(old_k) && aligned16(old_v) && aligned16(new_k) && aligned16(new_v) && aligned16(out_k) &&
                    aligned16(out_v),
                "rows must be 16-byte aligned");
  const int64_t blocks = (total_out + kRows - 1) / kRows;
  WNW_CHECK_ARG(blocks < (1ll << 31), "too many rows");
  hipLaunchKernelGGL(interleave_append_kernel<true>, dim3((unsigned)blocks), dim3(kNT), 0, (hipStream_t)stream,
                     (const u32x4*)old_k, (const u32x4*)new_k, cu_old, cu_new, (int)n_seg, total_old, total_out, cpr,
                     (u32x4*)out_k, device_error_word(), (const u32x4*)old_v, (const u32x4*)new_v, (u32x4*)out_v);
  WNW_CHECK_HIP(hipGetLastError(), "interleave_append_kv launch");
  return WNW_OK;
}

extern "C" int wnw_append_inplace(void* k_pool, void* v_pool, const void* new_k, const void* new_v,
                                  const int32_t* cu_old, int32_t* cu_new, const int64_t* seg_base,
                                  const int32_t* seg_cap, int64_t n_seg, int64_t pool_rows,
                                  int64_t head_dim, int dtype, void* stream) {
  int cpr = 0;
  if (int rc = check_rows(head_dim, dtype, cpr)) return rc;
  WNW_CHECK_ARG(n_seg >= 0 && n_seg < (1 << 30), "bad n_seg");
  WNW_CHECK_ARG(k_pool && v_pool && new_k && new_v && cu_old && cu_new && seg_base && seg_cap,
                "null pointer argument");
  WNW_CHECK_ARG((const void*)cu_old != (const void*)cu_new, "cu_new must not alias cu_old");
  WNW_CHECK_ARG(aligned16(k_pool) && aligned16(v_pool) && aligned16(new_k) && aligned16(new_v),
                "rows must be 16-byte aligned");
  const int64_t nthreads = std::max<int64_t>(n_seg * cpr, n_seg + 1);
  const int64_t blocks = (nthreads + kNT - 1) / kNT;
  WNW_CHECK_ARG(blocks < (1ll << 31), "too many rows");
  hipLaunchKernelGGL(append_inplace_kernel, dim3((unsigned)blocks), dim3(kNT), 0, (hipStream_t)stream,
                     (u32x4*)k_pool, (u32x4*)v_pool, (const u32x4*)new_k, (const u32x4*)new_v, cu_old,
                     cu_new, seg_base, seg_cap, (int)n_seg, pool_rows, cpr, device_error_word());
  WNW_CHECK_HIP(hipGetLastError(), "append_inplace launch");
  return WNW_OK;
}

extern "C" int wnw_rebuild_append_kv(const void* old_k, const void* old_v, const void* new_k,
                                     const void* new_v, const void* load_k, const void* load_v,
                                     const int32_t* old_cu, const int32_t* new_cu,
                                     const int32_t* load_starts, const int32_t* load_lens,
                                     const int32_t* evict_offsets, const int32_t* evict_starts,
                                     const int32_t* evict_ends, int64_t n_evict, int64_t n_seg,
                                     int64_t total_old, int64_t total_load, int64_t total_out,
                                     int64_t max_evict,
                                     int64_t head_dim, int dtype, void* out_k, void* out_v,
                                     void* stream) {
  int cpr = 0;
  if (int rc = check_rows(head_dim, dtype, cpr)) return rc;
  WNW_CHECK_ARG(n_seg >= 0 && n_seg < (1 << 30) && total_old >= 0 && total_load >= 0 && total_out >= 0,
                "bad sizes");
  if (total_out == 0) return WNW_OK;
  WNW_CHECK_ARG(new_k && new_v && old_cu && new_cu && load_starts && load_lens && evict_offsets && out_k &&
                    out_v,
                "null pointer argument");
  WNW_CHECK_ARG((old_k && old_v) || total_old == 0, "old rows are null");
  WNW_CHECK_ARG((load_k && load_v) || total_load == 0, "load rows are null");
  WNW_CHECK_ARG(n_evict >= 0 && ((evict_starts && evict_ends) || n_evict == 0), "evict ranges are null");
  const int64_t blocks = (total_out + kRows - 1) / kRows;
  WNW_CHECK_ARG(blocks < (1ll << 31), "too many rows");
  RebuildDesc d;
  d.load_starts = load_starts;
  d.load_lens = load_lens;
  d.evict_offsets = evict_offsets;
  d.evict_starts = evict_starts;
  d.evict_ends = evict_ends;
  d.n_evict = n_evict;
  d.max_evict = (int32_t)std::max<int64_t>(std::min<int64_t>(max_evict, 1 << 30), 1);
  // rows written (K and V) beyond the Infinity Cache: non-temporal copies
  const bool nt = total_out * cpr * 16 * 2 > (256ll << 20);
  hipLaunchKernelGGL(nt ? rebuild_append_kernel<true> : rebuild_append_kernel<false>, dim3((unsigned)blocks),
                     dim3(kNT), 0, (hipStream_t)stream, (const u32x4*)old_k, (const u32x4*)old_v,
                     (const u32x4*)new_k, (const u32x4*)new_v, (const u32x4*)load_k, (const u32x4*)load_v, old_cu,
                     new_cu, d, (int)n_seg, total_old, total_load, total_out, cpr, (u32x4*)out_k, (u32x4*)out_v,
                     device_error_word());
  WNW_CHECK_HIP(hipGetLastError(), "rebuild_append_kv launch");
  return WNW_OK;
}

extern "C" int wnw_compact_segments(const void* src_k, const void* src_v, void* dst_k, void* dst_v,
                                    const void* new_k, const void* new_v, const void* load_k,
                                    const void* load_v, const int32_t* seg_list, int64_t n_list,
                                    int64_t n_seg, int64_t max_new_len, const int64_t* src_base, const int32_t* src_len,
                                    const int64_t* dst_base, const int32_t* new_len,
                                    const int32_t* load_starts, const int32_t* load_lens,
                                    const int32_t* evict_offsets, const int32_t* evict_starts,
                                    const int32_t* evict_ends, int64_t n_evict, int with_new,
                                    int64_t src_rows,
                                    int64_t dst_rows, int64_t load_rows, int64_t head_dim, int dtype,
                                    void* stream) {
  int cpr = 0;
  if (int rc = check_rows(head_dim, dtype, cpr)) return rc;
  WNW_CHECK_ARG(n_list >= 0 && n_list < 65536, "n_list must be in [0, 65535]");
  WNW_CHECK_ARG(n_seg >= 0 && n_seg < (1 << 30), "bad n_seg");
  if (n_list == 0) return WNW_OK;
  WNW_CHECK_ARG(src_k && src_v && dst_k && dst_v && seg_list && src_base && src_len && dst_base && new_len &&
                    load_starts && load_lens && evict_offsets,
                "null pointer argument");
  WNW_CHECK_ARG(!with_new || (new_k && new_v), "new rows are null");
  WNW_CHECK_ARG((load_k && load_v) || load_rows == 0, "load rows are null");
  WNW_CHECK_ARG(n_evict >= 0 && ((evict_starts && evict_ends) || n_evict == 0), "evict ranges are null");
  WNW_CHECK_ARG(dst_rows > 0, "dst_rows must be positive");
  WNW_CHECK_ARG(max_new_len >= 0 && max_new_len <= dst_rows, "max_new_len out of range");
  if (max_new_len == 0) return WNW_OK;
  RebuildDesc d;
  d.load_starts = load_starts;
  d.load_lens = load_lens;
  d.evict_offsets = evict_offsets;
  d.evict_starts = evict_starts;
  d.evict_ends = evict_ends;
  d.n_evict = n_evict;
  d.max_evict = 1 << 30;
  // grid.x covers the longest listed segment; shorter ones exit early.
  const int64_t gx = (max_new_len + kRows - 1) / kRows;
  WNW_CHECK_ARG(gx < (1ll << 31), "segment too long");
  hipLaunchKernelGGL(compact_segments_kernel, dim3((unsigned)gx, (unsigned)n_list), dim3(kNT), 0,
                     (hipStream_t)stream, (const u32x4*)src_k, (const u32x4*)src_v, (u32x4*)dst_k,
                     (u32x4*)dst_v, (const u32x4*)new_k, (const u32x4*)new_v, (const u32x4*)load_k,
                     (const u32x4*)load_v, seg_list, (int)n_seg, src_base, src_len, dst_base, new_len, d, with_new,
                     src_rows, dst_rows, load_rows, cpr, device_error_word());
  WNW_CHECK_HIP(hipGetLastError(), "compact_segments launch");
  return WNW_OK;
}

namespace wnw {
void touch_append_kernels() {
  hipFuncAttributes a;
  (void)hipFuncGetAttributes(&a, (const void*)&compact_segments_kernel);
  (void)hipFuncGetAttributes(&a, (const void*)&append_inplace_kernel);
  (void)hipFuncGetAttributes(&a, (const void*)&rebuild_append_kernel<false>);
  (void)hipFuncGetAttributes(&a, (const void*)&interleave_append_kernel<true>);
}
}  // namespace wnw

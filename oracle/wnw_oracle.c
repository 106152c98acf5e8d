/*
 * CPU oracle of the decode-step attention path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker (or the timed CPU baseline),
 * never as a product path.  Each function restates one reference
 * computation in plain C, citing the reference file:line it follows
 * (paths relative to the WnW source tree).
 *
 * Element types: 0 = f32, 1 = f16, 2 = bf16 (as in include/wnw_amd.h).
 * Row gathers move raw bytes, so they are exact for every type.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static size_t esize(int dtype) { return dtype == 0 ? 4 : 2; }

static double elem_to_f64(const void* base, int64_t i, int dtype) {
  if (dtype == 0) return (double)((const float*)base)[i];
  uint16_t h = ((const uint16_t*)base)[i];
  if (dtype == 2) {
    uint32_t u = ((uint32_t)h) << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
  }
  /* IEEE half -> double, all cases (subnormals, inf, nan) */
  int sign = (h >> 15) & 1, ex = (h >> 10) & 0x1f, man = h & 0x3ff;
  double v;
  if (ex == 0)
    v = ldexp((double)man, -24);
  else if (ex == 31)
    v = man ? NAN : INFINITY;
  else
    v = ldexp((double)(man | 0x400), ex - 25);
  return sign ? -v : v;
}

/*
 * Decode attention for q = 1 per segment, GQA group G, in float64:
 *   out[s, g, :] = sum_r softmax_r(scale * <q[s, g], K[r]>) V[r]
 * over rows r in [cu[s], cu[s+1]) (the physical row is base[s] + r - cu[s]
 * when base != NULL).  Follows q1_decode_attn
 * (src/common/kv/fused_attn.py:9-44: per-segment softmax over all cached
 * keys, no mask, q head h = kv * G + g) and the varlen_attn call of
 * src/algorithms/wnw/code/session.py:81-106 (q_flat [B*Hkv, G, D], K/V
 * broadcast over the group).  Two-pass softmax with exact max.  Empty
 * segments give zeros.  Returns 0, or -1 on inconsistent offsets.
 */
int oracle_decode_attn(const void* q, const void* k, const void* v,
                       const int32_t* cu, const int64_t* base, int64_t n_seg,
                       int64_t G, int64_t D, double scale, int dtype,
                       int64_t kv_rows, double* out) {
  double* sc = NULL;
  int64_t cap = 0;
  for (int64_t s = 0; s < n_seg; ++s) {
    int64_t lo = cu[s], hi = cu[s + 1];
    if (hi < lo) {
      free(sc);
      return -1;
    }
    int64_t n = hi - lo;
    int64_t b = base ? base[s] : lo;
    if (b < 0 || b + n > kv_rows) {
      free(sc);
      return -1;
    }
    if (n > cap) {
      free(sc);
      cap = n;
      sc = (double*)malloc(sizeof(double) * cap);
      if (!sc) return -1;
    }
    for (int64_t g = 0; g < G; ++g) {
      double* o = out + (s * G + g) * D;
      for (int64_t d = 0; d < D; ++d) o[d] = 0.0;
      if (n == 0) continue;
      const int64_t qoff = (s * G + g) * D;
      double mx = -INFINITY;
      for (int64_t r = 0; r < n; ++r) {
        double acc = 0.0;
        for (int64_t d = 0; d < D; ++d)
          acc += elem_to_f64(q, qoff + d, dtype) * elem_to_f64(k, (b + r) * D + d, dtype);
        sc[r] = acc * scale;
        if (sc[r] > mx) mx = sc[r];
      }
      double l = 0.0;
      for (int64_t r = 0; r < n; ++r) {
        sc[r] = exp(sc[r] - mx);
        l += sc[r];
      }
      for (int64_t r = 0; r < n; ++r) {
        const double p = sc[r] / l;
        for (int64_t d = 0; d < D; ++d) o[d] += p * elem_to_f64(v, (b + r) * D + d, dtype);
      }
    }
  }
  free(sc);
  return 0;
}

/*
 * Out-of-place append, src/common/kv/kernels.py:7-42 (kernel) and :45-73
 * (launcher): output row j of segment s (cu_new[s] <= j < cu_new[s+1])
 * copies old row cu_old[s] + (j - cu_new[s]) while that index is below the
 * old segment length, else the new token of s.  Returns 0, or -1 if an
 * index leaves the given arrays.
 */
int oracle_interleave_append(const void* old_rows, const void* new_rows,
                             const int32_t* cu_old, const int32_t* cu_new,
                             int64_t n_seg, int64_t total_old, int64_t D,
                             int dtype, void* out) {
  const size_t rb = (size_t)D * esize(dtype);
  const int64_t total_out = total_old + n_seg;
  for (int64_t s = 0; s < n_seg; ++s) {
    const int64_t nlo = cu_new[s], nhi = cu_new[s + 1];
    const int64_t olo = cu_old[s], olen = cu_old[s + 1] - cu_old[s];
    if (nhi < nlo || nlo < 0 || nhi > total_out) return -1;
    for (int64_t j = nlo; j < nhi; ++j) {
      const int64_t i = j - nlo;
      const void* src;
      if (i < olen) {
        if (olo + i < 0 || olo + i >= total_old) return -1;
        src = (const char*)old_rows + (size_t)(olo + i) * rb;
      } else {
        src = (const char*)new_rows + (size_t)s * rb;
      }
      memcpy((char*)out + (size_t)j * rb, src, rb);
    }
  }
  return 0;
}

/*
 * Compaction + load + append, src/algorithms/wnw/code/kernels.py:407-473:
 * for output row j of segment s, row_in_new = j - new_cu[s];
 * kept_len = old_len - sum of the first min(n_evict_s, MAX_EVICT) evict
 * ranges; kept rows map back through the sorted ranges in order
 * (old_rel += ee - es whenever old_rel >= es); then load rows
 * load_starts[s] + (row_in_new - kept_len); then the new token.
 * MAX_EVICT = max(max_evict, 1) as in the launcher (:402).
 */
int oracle_rebuild_append_kv(const void* old_k, const void* old_v,
                             const void* new_k, const void* new_v,
                             const void* load_k, const void* load_v,
                             const int32_t* old_cu, const int32_t* new_cu,
                             const int32_t* load_starts,
                             const int32_t* load_lens,
                             const int32_t* evict_offsets,
                             const int32_t* evict_starts,
                             const int32_t* evict_ends, int64_t n_evict,
                             int64_t n_seg, int64_t total_old,
                             int64_t total_load, int64_t total_out,
                             int64_t max_evict, int64_t D, int dtype,
                             void* out_k, void* out_v) {
  const size_t rb = (size_t)D * esize(dtype);
  const int64_t MAXE = max_evict > 1 ? max_evict : 1;
  for (int64_t s = 0; s < n_seg; ++s) {
    const int64_t nlo = new_cu[s], nhi = new_cu[s + 1];
    const int64_t olo = old_cu[s], olen = old_cu[s + 1] - old_cu[s];
    const int64_t e0 = evict_offsets[s];
    int64_t ne = evict_offsets[s + 1] - e0;
    if (ne > MAXE) ne = MAXE;
    if (ne > 0 && (e0 < 0 || e0 + ne > n_evict)) return -1;
    if (nhi < nlo || nlo < 0 || nhi > total_out) return -1;
    int64_t kept = olen;
    for (int64_t e = 0; e < ne; ++e) kept -= evict_ends[e0 + e] - evict_starts[e0 + e];
    for (int64_t j = nlo; j < nhi; ++j) {
      const int64_t i = j - nlo;
      const void *sk, *sv;
      if (i < kept) {
        int64_t rel = i;
        for (int64_t e = 0; e < ne; ++e)
          if (rel >= evict_starts[e0 + e]) rel += evict_ends[e0 + e] - evict_starts[e0 + e];
        const int64_t src = olo + rel;
        if (src < 0 || src >= total_old) return -1;
        sk = (const char*)old_k + (size_t)src * rb;
        sv = (const char*)old_v + (size_t)src * rb;
      } else if (i < kept + load_lens[s]) {
        const int64_t src = (int64_t)load_starts[s] + (i - kept);
        if (src < 0 || src >= total_load) return -1;
        sk = (const char*)load_k + (size_t)src * rb;
        sv = (const char*)load_v + (size_t)src * rb;
      } else {
        sk = (const char*)new_k + (size_t)s * rb;
        sv = (const char*)new_v + (size_t)s * rb;
      }
      memcpy((char*)out_k + (size_t)j * rb, sk, rb);
      memcpy((char*)out_v + (size_t)j * rb, sv, rb);
    }
  }
  return 0;
}

/*
 * The same result built the way the pure-torch fallback does it
 * (src/algorithms/wnw/code/cache.py:891-1010 with _invert_ranges
 * :1153-1162): per segment, the complement of the sorted evict ranges is
 * turned into keep slices and concatenated, then the loaded parts, then
 * (as decode_before_attn does next, cache.py:497-507) the new token.  An
 * independent restatement used to cross-check oracle_rebuild_append_kv.
 */
int oracle_rebuild_by_slices(const void* old_k, const void* old_v,
                             const void* new_k, const void* new_v,
                             const void* load_k, const void* load_v,
                             const int32_t* old_cu, const int32_t* load_starts,
                             const int32_t* load_lens,
                             const int32_t* evict_offsets,
                             const int32_t* evict_starts,
                             const int32_t* evict_ends, int64_t n_seg,
                             int64_t D, int dtype, void* out_k, void* out_v,
                             int32_t* out_cu) {
  const size_t rb = (size_t)D * esize(dtype);
  int64_t w = 0;
  out_cu[0] = 0;
  for (int64_t s = 0; s < n_seg; ++s) {
    const int64_t olo = old_cu[s], olen = old_cu[s + 1] - old_cu[s];
    int64_t prev = 0;
    for (int64_t e = evict_offsets[s]; e <= evict_offsets[s + 1]; ++e) {
      const int64_t a = prev;
      const int64_t b = (e < evict_offsets[s + 1]) ? evict_starts[e] : olen;
      if (a < b) {
        memcpy((char*)out_k + (size_t)w * rb, (const char*)old_k + (size_t)(olo + a) * rb, (size_t)(b - a) * rb);
        memcpy((char*)out_v + (size_t)w * rb, (const char*)old_v + (size_t)(olo + a) * rb, (size_t)(b - a) * rb);
        w += b - a;
      }
      if (e < evict_offsets[s + 1]) prev = evict_ends[e];
    }
    const int64_t ll = load_lens[s];
    if (ll > 0) {
      memcpy((char*)out_k + (size_t)w * rb, (const char*)load_k + (size_t)load_starts[s] * rb, (size_t)ll * rb);
      memcpy((char*)out_v + (size_t)w * rb, (const char*)load_v + (size_t)load_starts[s] * rb, (size_t)ll * rb);
      w += ll;
    }
    memcpy((char*)out_k + (size_t)w * rb, (const char*)new_k + (size_t)s * rb, rb);
    memcpy((char*)out_v + (size_t)w * rb, (const char*)new_v + (size_t)s * rb, rb);
    w += 1;
    out_cu[s + 1] = (int32_t)w;
  }
  return 0;
}

/*
 * Class-A token scores (float64).  Item i has nh query heads
 * q[i, 0..nh) and the K rows [r0[i], r1[i]); for each head the softmax of
 * scale * q . K over those rows is formed, and for the audio rows
 * [r0 + a0[i], r0 + a1[i]) the weights, summed over the heads, are added to
 * acc[off[i] + j].  This is the arithmetic of both reference scorers:
 * q1_decode_attn_score (src/common/kv/fused_attn.py:68-123, one item per
 * flagged segment, heads = the group) and fused_score_accumulate
 * (src/algorithms/wnw/code/kernels.py:351-370, _fused_score_pytorch).
 * Returns -1 on inconsistent ranges.
 */
int oracle_segment_scores(const void* q, const void* k, const int64_t* r0,
                          const int64_t* r1, const int32_t* a0,
                          const int32_t* a1, const int64_t* off,
                          int64_t n_items, int64_t nh, int64_t D,
                          double scale, int dtype, int64_t k_rows,
                          int64_t acc_len, double* acc) {
  double* w = NULL;
  double* sc = NULL;
  int rc = 0;
  for (int64_t i = 0; i < n_items && rc == 0; ++i) {
    const int64_t n = r1[i] - r0[i];
    const int64_t na = (int64_t)a1[i] - a0[i];
    if (n < 0 || r0[i] < 0 || r1[i] > k_rows || a0[i] < 0 || a1[i] > n || na < 0 || off[i] < 0 ||
        off[i] + na > acc_len) {
      rc = -1;
      break;
    }
    if (na == 0) continue;
    free(w);
    free(sc);
    w = (double*)calloc((size_t)na, sizeof(double));
    sc = (double*)malloc(sizeof(double) * (size_t)n);
    if (!w || !sc) {
      rc = -1;
      break;
    }
    for (int64_t h = 0; h < nh; ++h) {
      const int64_t qoff = (i * nh + h) * D;
      double mx = -INFINITY;
      for (int64_t r = 0; r < n; ++r) {
        double d = 0.0;
        for (int64_t e = 0; e < D; ++e)
          d += elem_to_f64(q, qoff + e, dtype) * elem_to_f64(k, (r0[i] + r) * D + e, dtype);
        sc[r] = d * scale;
        if (sc[r] > mx) mx = sc[r];
      }
      double l = 0.0;
      for (int64_t r = 0; r < n; ++r) l += exp(sc[r] - mx);
      for (int64_t j = 0; j < na; ++j) w[j] += exp(sc[a0[i] + j] - mx) / l;
    }
    for (int64_t j = 0; j < na; ++j) acc[off[i] + j] += w[j];
  }
  free(w);
  free(sc);
  return rc;
}

// Class-A token scores of the decode step (gfx950).
//
// A class-A KV head's query heads rate every audio token of their own
// segment by its softmax weight; the weights, summed over the heads, are
// added to a per-sample accumulator that the chunk planner ranks
// (reference: q1_decode_attn_score, src/common/kv/fused_attn.py:68-156, and
// fused_score_accumulate, src/algorithms/wnw/code/kernels.py:302-370).
//
// Both operators need each head's final softmax normaliser before any
// weight can be formed.  Here it comes from
//   * the attention kernel itself (q1_decode_attn_score): it hands out each
//     segment's final (max, sum) in the log2 domain, so one pass over the
//     audio rows of the flagged segments remains;
//   * or a statistics pass (fused_score_accumulate, which scores a subset of
//     a group's heads with its own scale): the rows of each segment are cut
//     into kStatChunks slices whose partial (max, sum) pairs the scoring
//     pass merges.
// The scoring pass gives one (sample, row range) to one workgroup, which
// sums over heads (and over flagged KV heads) in registers and adds to the
// accumulator once per token: no atomics, deterministic results.
//
// Row dot products: a row of D elements is read by D / EPC lanes, 16 bytes
// each (one 64-byte-aligned run per lane group), and reduced across those
// lanes with a butterfly; q lives in LDS as fp32.
#include <math.h>

#include "wnw_common.h"

namespace wnw {

static constexpr int kScoreThreads = 256;
// Row iterations per scoring workgroup: 16, or 4 when 16 would leave CUs idle
// (few samples or short audio).
static constexpr int kIters = 16;
static constexpr int kItersSmall = 4;
static constexpr int kStatChunks = 32;    // row slices per segment in the statistics pass
static constexpr int kMaxHeads = 16;
static constexpr float kLog2eS = 1.4426950408889634f;
static constexpr float kNegBigS = -1e30f;

template <typename T>
struct RowGeom {
  static constexpr int EPC = 16 / (int)sizeof(T);  // elements per 16-byte chunk
};
// Rows one scoring workgroup covers: `iters` iterations of kScoreThreads / LPR
// rows, LPR = head_dim / EPC lanes per row.
__host__ __device__ constexpr int score_rows_per_wg(int head_dim, int elem_bytes, int iters = kIters) {
  return iters * kScoreThreads / (head_dim / (16 / elem_bytes));
}

// 16-byte chunk -> EPC floats
template <typename T>
__device__ __forceinline__ void chunk_to_f32(const u32x4& w, float* f) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(w[i]);
  } else {
    unpack8(w, f, (T*)nullptr);
  }
}

// Sum over the LPR lanes of a row group (lanes are contiguous, LPR a power of two).
template <int LPR>
__device__ __forceinline__ float group_sum(float x) {
#pragma unroll
  for (int o = LPR / 2; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Loads nh query heads ([nh][D] of T) into LDS as fp32.
template <typename T>
__device__ __forceinline__ void stage_q(float* qf, const T* q, int nh, int D) {
  for (int i = threadIdx.x; i < nh * D; i += blockDim.x) qf[i] = Elem<T>::to_f32(q, i);
}

// ---------------------------------------------------------------------------
// scores from the attention kernel's normalisers (q1_decode_attn_score)
// ---------------------------------------------------------------------------
struct AttnScoreParams {
  const void* q;        // [n_seg, G, D]
  const void* k;        // [kv_rows, D]
  const int32_t* cu;    // [n_seg + 1]
  const int64_t* base;  // [n_seg] or null
  const float* lse;     // [n_seg, G, 2] log2 domain
  const int32_t* mask;  // [Hkv], non-zero = score this KV head
  const int32_t* audio_s;  // [B] audio range relative to the segment start
  const int32_t* audio_e;
  const int32_t* acc_off;  // [B + 1]
  float* acc;
  int32_t* err;
  int64_t kv_rows, acc_len;
  int32_t n_seg, G, Hkv;
  float scale_log2;
};

template <typename T, int D, int IT>
__global__ __launch_bounds__(kScoreThreads) void attn_score_kernel(AttnScoreParams p) {
  constexpr int EPC = RowGeom<T>::EPC;
  constexpr int LPR = D / EPC;            // lanes per row
  constexpr int RPI = kScoreThreads / LPR;  // rows per workgroup iteration
  __shared__ float qf[kMaxHeads * D];
  __shared__ float stat[kMaxHeads][2];    // (max, 1 / sum)
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int sub = tid % LPR;              // this lane's chunk of the row
  const int rl = tid / LPR;               // row slot in an iteration
  const int a0 = p.audio_s[b], a1 = p.audio_e[b];
  const int n_audio = a1 - a0;
  const int j0 = blockIdx.x * RPI * IT;
  if (j0 >= n_audio) return;  // workgroup-uniform
  const int64_t off = p.acc_off[b];
  if (off < 0 || off + n_audio > p.acc_len) {  // the accumulator cannot hold this sample's tokens
    if (tid == 0 && blockIdx.x == 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
    return;  // workgroup-uniform
  }
  float total[IT];
#pragma unroll
  for (int i = 0; i < IT; ++i) total[i] = 0.f;
  const T* kp = (const T*)p.k;
  for (int kv = 0; kv < p.Hkv; ++kv) {
    if (!p.mask[kv]) continue;
    const int s = b * p.Hkv + kv;
    if (s >= p.n_seg) break;
    const int64_t len = (int64_t)p.cu[s + 1] - p.cu[s];
    const int64_t base = p.base ? p.base[s] : (int64_t)p.cu[s];
    if (a0 < 0 || a1 > len || base < 0 || base + len > p.kv_rows) {
      if (tid == 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
      continue;  // uniform
    }
    __syncthreads();  // previous head's q / stat reads are done
    stage_q<T>(qf, (const T*)p.q + (int64_t)s * p.G * D, p.G, D);
    if (tid < p.G) {
      stat[tid][0] = p.lse[((int64_t)s * p.G + tid) * 2];
      stat[tid][1] = 1.f / p.lse[((int64_t)s * p.G + tid) * 2 + 1];
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int j = j0 + it * RPI + rl;
      const bool valid = j < n_audio;
      const int64_t row = base + a0 + (valid ? j : 0);
      u32x4 w = *(const u32x4*)(kp + row * D + sub * EPC);
      float kf[EPC];
      chunk_to_f32<T>(w, kf);
      float sc = 0.f;
      for (int g = 0; g < p.G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < EPC; ++i) d += qf[g * D + sub * EPC + i] * kf[i];
        d = group_sum<LPR>(d);
        sc += exp2f(d * p.scale_log2 - stat[g][0]) * stat[g][1];
      }
      total[it] += valid ? sc : 0.f;
    }
  }
  if (sub == 0) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int j = j0 + it * RPI + rl;
      if (j < n_audio) p.acc[off + j] += total[it];
    }
  }
}

// ---------------------------------------------------------------------------
// scores from the logits the streaming attention kernel kept
// ---------------------------------------------------------------------------
// The attention kernel already computed every scaled logit x = q.k * scale
// (log2 domain) of the scored audio rows; with its final (max, sum) per head
// a weight is exp2(x - max) / sum.  One thread per audio token of a sample
// sums the weights over the flagged KV heads and their query heads, and
// adds the total to the accumulator once (no atomics).  The validity rules
// are those of attn_score_kernel, so both passes score the same rows.
// The fields of the first loads are the kernel's leading scalar arguments
// (see logit_score_kernel); the rest come in this aggregate.
struct LogitScoreParams {
  const float* xlog;       // [n_seg, G, max_audio]
  const int32_t* acc_off;  // [B + 1]
  float* acc;
  int32_t* err;
  int64_t kv_rows, acc_len, max_audio;
};

static constexpr int kLogitThreads = 256;
static constexpr int kLogitKv = 64;  // KV heads per sample this pass takes (a lane of wave 0 each)
static constexpr int kLogitG = 8;    // query heads per KV head (the streaming kernel's limit)

// Latency, not bytes, bounds this pass (a few hundred KB per launch), so
// its loads go out in two batches instead of a chain: wave 0 reads every
// KV head's flag, bounds and normalisers at once (lane = KV head; the
// sample's audio range and offset arrive in the same round trip) and lists
// the flagged, valid segments in LDS; then every thread issues the loads
// of all its logits and of its accumulator entry together.  Loads are
// unconditional (indices clamped into range) and the checks combine with
// bitwise operators, so no load waits behind a branch on another load.
//
// score.hip is built with 16 preloaded argument dwords, of which gfx950
// delivers 14 in SGPRs at dispatch: the six tables of the first round trip
// and the sizes their addresses need (hg = Hkv | G << 16, n_seg), so those
// loads issue before any argument load returns.
__global__ __launch_bounds__(kLogitThreads) void logit_score_kernel(
    const int32_t* audio_s, const int32_t* audio_e, const int32_t* mask, const int32_t* cu, const int64_t* seg_base,
    const float* lse, int32_t hg, int32_t n_seg, LogitScoreParams p) {
  __shared__ int32_t seg_sh[kLogitKv];
  __shared__ float m_sh[kLogitKv * kLogitG], inv_sh[kLogitKv * kLogitG];
  __shared__ int32_t n_sh;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int Hkv = hg & 0xffff, G = hg >> 16;
  const int a0 = audio_s[b], a1 = audio_e[b];
  if (tid < 64) {  // wave 0
    const int kv = min(tid, Hkv - 1);
    const int s = min(b * Hkv + kv, n_seg - 1);
    const int32_t flag = mask[kv];
    const int64_t bv = seg_base ? seg_base[s] : 0;
    const int64_t c0 = cu[s], c1 = cu[s + 1];
    float m[kLogitG], l[kLogitG];
#pragma unroll
    for (int g = 0; g < kLogitG; ++g) {
      const int64_t e = ((int64_t)s * G + min(g, G - 1)) * 2;
      m[g] = lse[e];
      l[g] = lse[e + 1];
    }
    const int64_t len = c1 - c0;
    const int64_t base = seg_base ? bv : c0;
    const bool flagged = (tid < Hkv) & (b * Hkv + tid < n_seg) & (flag != 0);
    const bool oob = (a0 < 0) | (a1 > len) | (base < 0) | (base + len > p.kv_rows);
    const bool use = flagged & !oob;
    if (flagged & oob & (blockIdx.x == 0)) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
    const uint64_t bal = __ballot(use);
    if (use) {
      const int pos = __popcll(bal & ((1ull << tid) - 1ull));
      seg_sh[pos] = s;
#pragma unroll
      for (int g = 0; g < kLogitG; ++g) {
        m_sh[pos * kLogitG + g] = m[g];
        inv_sh[pos * kLogitG + g] = 1.f / l[g];
      }
    }
    if (tid == 0) n_sh = __popcll(bal);
  }
  const int64_t off = p.acc_off[b];
  const int n_audio = a1 - a0;
  if ((int64_t)blockIdx.x * kLogitThreads >= min((int64_t)n_audio, p.max_audio)) return;  // uniform
  if (off < 0 || off + n_audio > p.acc_len) {  // the accumulator cannot hold this sample's tokens
    if (tid == 0 && blockIdx.x == 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
    return;  // uniform
  }
  __syncthreads();
  const int64_t j = (int64_t)blockIdx.x * kLogitThreads + tid;
  const bool valid = j < n_audio && j < p.max_audio;
  const int64_t jc = valid ? j : 0;  // loads stay unconditional; `valid` gates the store
  const float prior = p.acc[off + jc];
  const int nt = n_sh * G;
  float total = 0.f, sc = 0.f;  // a segment's heads are summed first, then added to the total
  // pair t = (segment i, head g), counted rather than divided by G (uniform);
  // loads past the last pair repeat it
  int i = 0, g = 0;
  for (int t0 = 0; t0 < nt; t0 += 8) {
    float x[8];
    int li = i, lg = g;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const bool in = t0 + u < nt;
      const int ii = in ? li : n_sh - 1, gg = in ? lg : G - 1;
      x[u] = p.xlog[((int64_t)seg_sh[ii] * G + gg) * p.max_audio + jc];
      if (++lg == G) {
        lg = 0;
        ++li;
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (t0 + u < nt) {
        // v_exp_f32 directly: arguments are <= 0 (m is the maximum) and
        // weights below 2^-126 (flushed to zero) are negligible
        sc += __builtin_amdgcn_exp2f(x[u] - m_sh[i * kLogitG + g]) * inv_sh[i * kLogitG + g];
        if (g == G - 1) {
          total += sc;
          sc = 0.f;
        }
      }
      if (++g == G) {
        g = 0;
        ++i;
      }
    }
  }
  if (valid) p.acc[off + j] = prior + total;
}

// ---------------------------------------------------------------------------
// fused_score_accumulate: statistics pass + scoring pass
// ---------------------------------------------------------------------------
struct SegScoreParams {
  const void* q;           // [S, nh, D]
  const void* k;           // [k_rows, D]
  const int32_t* seg_s;    // [S] physical first row
  const int32_t* seg_e;    // [S] physical end row
  const int32_t* audio_s;  // [S] relative to seg_s
  const int32_t* audio_e;
  const int32_t* acc_off;  // [S + 1]
  float* acc;
  float* part;             // [S, kStatChunks, nh, 2]
  int32_t* err;
  int64_t k_rows, acc_len;
  int32_t S, nh;
  float scale_log2;
};

__device__ __forceinline__ void merge_ml(float& m, float& l, float m2, float l2) {
  const float mn = fmaxf(m, m2);
  l = l * exp2f(m - mn) + l2 * exp2f(m2 - mn);
  m = mn;
}

template <typename T, int D>
__global__ __launch_bounds__(kScoreThreads) void seg_stats_kernel(SegScoreParams p) {
  constexpr int EPC = RowGeom<T>::EPC;
  constexpr int LPR = D / EPC;
  constexpr int RPI = kScoreThreads / LPR;
  __shared__ float qf[kMaxHeads * D];
  __shared__ float red[kScoreThreads / 64][kMaxHeads][2];
  const int s = blockIdx.y, c = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int sub = tid % LPR, rl = tid / LPR;
  const int64_t r0 = p.seg_s[s], r1 = p.seg_e[s];
  const bool ok = r0 >= 0 && r1 >= r0 && r1 <= p.k_rows;
  if (!ok && tid == 0 && c == 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
  const int64_t len = ok ? r1 - r0 : 0;
  const int64_t c0 = r0 + len * c / kStatChunks, c1 = r0 + len * (c + 1) / kStatChunks;
  stage_q<T>(qf, (const T*)p.q + (int64_t)s * p.nh * D, p.nh, D);
  __syncthreads();
  float m[kMaxHeads], l[kMaxHeads];
#pragma unroll
  for (int h = 0; h < kMaxHeads; ++h) {
    m[h] = kNegBigS;
    l[h] = 0.f;
  }
  const T* kp = (const T*)p.k;
  for (int64_t row0 = c0; row0 < c1; row0 += RPI) {
    const int64_t row = row0 + rl;
    const bool valid = row < c1;
    u32x4 wv = *(const u32x4*)(kp + (valid ? row : c0) * D + sub * EPC);
    float kf[EPC];
    chunk_to_f32<T>(wv, kf);
#pragma unroll
    for (int h = 0; h < kMaxHeads; ++h) {
      if (h < p.nh) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < EPC; ++i) d += qf[h * D + sub * EPC + i] * kf[i];
        d = group_sum<LPR>(d);
        if (valid) merge_ml(m[h], l[h], d * p.scale_log2, 1.f);
      }
    }
  }
  // merge the row groups of the wave (one representative lane per group),
  // then the waves through LDS
#pragma unroll
  for (int h = 0; h < kMaxHeads; ++h) {
    if (h < p.nh) {
      for (int o = LPR; o < 64; o <<= 1) {
        const float m2 = __shfl_xor(m[h], o), l2 = __shfl_xor(l[h], o);
        merge_ml(m[h], l[h], m2, l2);
      }
      if (lane == 0) {
        red[w][h][0] = m[h];
        red[w][h][1] = l[h];
      }
    }
  }
  __syncthreads();
  if (tid < p.nh) {
    float M = kNegBigS, Lsum = 0.f;
    for (int ww = 0; ww < kScoreThreads / 64; ++ww) merge_ml(M, Lsum, red[ww][tid][0], red[ww][tid][1]);
    float* out = p.part + (((int64_t)s * kStatChunks + c) * p.nh + tid) * 2;
    out[0] = M;
    out[1] = Lsum;
  }
}

template <typename T, int D, int IT>
__global__ __launch_bounds__(kScoreThreads) void seg_score_kernel(SegScoreParams p) {
  constexpr int EPC = RowGeom<T>::EPC;
  constexpr int LPR = D / EPC;
  constexpr int RPI = kScoreThreads / LPR;
  __shared__ float qf[kMaxHeads * D];
  __shared__ float stat[kMaxHeads][2];
  const int s = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int sub = tid % LPR, rl = tid / LPR;
  const int64_t r0 = p.seg_s[s], r1 = p.seg_e[s];
  const int a0 = p.audio_s[s], a1 = p.audio_e[s];
  const int n_audio = a1 - a0;
  const int j0 = blockIdx.x * RPI * IT;
  if (j0 >= n_audio) return;
  const int64_t off = p.acc_off[s];
  if (r0 < 0 || r1 < r0 || r1 > p.k_rows || a0 < 0 || r0 + a1 > r1 || off < 0 || off + n_audio > p.acc_len) {
    if (tid == 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
    return;
  }
  stage_q<T>(qf, (const T*)p.q + (int64_t)s * p.nh * D, p.nh, D);
  // merge the statistics slices: wave w takes heads w, w + 4, ...
  for (int h = w; h < p.nh; h += kScoreThreads / 64) {
    const float* pp = p.part + ((int64_t)s * kStatChunks * p.nh + h) * 2;
    const float mq = lane < kStatChunks ? pp[(int64_t)lane * p.nh * 2] : kNegBigS;
    const float lq = lane < kStatChunks ? pp[(int64_t)lane * p.nh * 2 + 1] : 0.f;
    const float M = wave_max(mq);
    const float Lsum = wave_sum(lq * exp2f(mq - M));
    if (lane == 0) {
      stat[h][0] = M;
      stat[h][1] = 1.f / Lsum;
    }
  }
  __syncthreads();
  const T* kp = (const T*)p.k;
  for (int it = 0; it < IT; ++it) {
    const int j = j0 + it * RPI + rl;
    const bool valid = j < n_audio;
    const int64_t row = r0 + a0 + (valid ? j : 0);
    u32x4 wv = *(const u32x4*)(kp + row * D + sub * EPC);
    float kf[EPC];
    chunk_to_f32<T>(wv, kf);
    float sc = 0.f;
    for (int h = 0; h < p.nh; ++h) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < EPC; ++i) d += qf[h * D + sub * EPC + i] * kf[i];
      d = group_sum<LPR>(d);
      sc += exp2f(d * p.scale_log2 - stat[h][0]) * stat[h][1];
    }
    if (valid && sub == 0) p.acc[off + j] += sc;
  }
}

enum ScoreKernel { kAttnScore = 0, kSegStats = 1, kSegScore = 2 };

template <typename T, int D>
static const void* score_fn(int which, int iters) {
  const bool small = iters == kItersSmall;
  switch (which) {
    case kAttnScore:
      return small ? (const void*)&attn_score_kernel<T, D, kItersSmall> : (const void*)&attn_score_kernel<T, D, kIters>;
    case kSegStats: return (const void*)&seg_stats_kernel<T, D>;
    case kSegScore:
      return small ? (const void*)&seg_score_kernel<T, D, kItersSmall> : (const void*)&seg_score_kernel<T, D, kIters>;
  }
  return nullptr;
}

template <typename T>
static const void* score_fn_d(int which, int64_t D, int iters) {
  switch (D) {
    case 64: return score_fn<T, 64>(which, iters);
    case 128: return score_fn<T, 128>(which, iters);
    case 256: return score_fn<T, 256>(which, iters);
  }
  return nullptr;
}

// Rows per iteration count for a scoring grid of `ny` rows of workgroups over
// max_audio rows: 16 iterations when that still gives two workgroups per CU,
// else 4 (more, shorter workgroups).
static int score_iters(int64_t max_audio, int64_t ny, int64_t head_dim, int elem_bytes) {
  const int cus = device_cus();
  const int64_t rows16 = score_rows_per_wg((int)head_dim, elem_bytes, kIters);
  return ((max_audio + rows16 - 1) / rows16) * ny >= 2 * (int64_t)cus ? kIters : kItersSmall;
}

template <typename P>
static hipError_t launch_score(int which, int dtype, int64_t D, int iters, dim3 grid, P prm, hipStream_t st) {
  const void* fn = nullptr;
  switch (dtype) {
    case WNW_BF16: fn = score_fn_d<bf16_t>(which, D, iters); break;
    case WNW_F16: fn = score_fn_d<f16_t>(which, D, iters); break;
    case WNW_F32: fn = score_fn_d<float>(which, D, iters); break;
  }
  if (!fn) return hipErrorInvalidValue;
  void* args[] = {&prm};
  return hipLaunchKernel(fn, grid, dim3(kScoreThreads), args, 0, st);
}

}  // namespace wnw

using namespace wnw;

static int64_t up256(int64_t x) { return (x + 255) / 256 * 256; }

// Workspace of wnw_decode_attn_score: attention workspace, normalisers, then
// (max_audio > 0) the logits of the scored audio rows.
static int64_t score_logits_offset(int64_t attn_ws, int64_t n_seg, int64_t group) {
  return attn_ws + up256(n_seg * group * 2 * 4);
}

extern "C" int64_t wnw_decode_attn_score_workspace_bytes(int64_t n_seg, int64_t group, int64_t head_dim,
                                                         int64_t max_audio) {
  const int64_t a = wnw_decode_attn_workspace_bytes(n_seg, group, head_dim);
  if (a < 0 || max_audio < 0) return -1;
  return score_logits_offset(a, n_seg, group) + up256(n_seg * group * max_audio * 4);
}

// Attention (with the step's append when app is given) + class-A scoring.
static int decode_attn_score_impl(const void* q, const void* k, const void* v, const int32_t* cu_k,
                                  const int64_t* seg_base, int64_t n_seg, int64_t group, int64_t head_dim,
                                  int64_t total_rows, int64_t kv_rows, float scale, int dtype, void* out,
                                  const int32_t* ca_kv_mask, int64_t num_kv_heads, const int32_t* audio_starts,
                                  const int32_t* audio_ends, float* score_acc, const int32_t* score_offsets,
                                  int64_t acc_len, int64_t max_audio, void* workspace, int64_t workspace_bytes,
                                  void* stream, const AttnAppend* app) {
  WNW_CHECK_ARG(num_kv_heads >= 1 && n_seg % num_kv_heads == 0,
                "n_seg (%lld) must be a multiple of num_kv_heads (%lld)", (long long)n_seg,
                (long long)num_kv_heads);
  WNW_CHECK_ARG(ca_kv_mask && audio_starts && audio_ends && score_acc && score_offsets,
                "null pointer argument");
  WNW_CHECK_ARG(max_audio >= 0 && acc_len >= 0, "negative max_audio / acc_len");
  WNW_CHECK_ARG(n_seg / num_kv_heads <= 65535, "at most 65535 samples (the scoring grid's y extent)");
  const int64_t attn_ws = wnw_decode_attn_workspace_bytes(n_seg, group, head_dim);
  WNW_CHECK_ARG(attn_ws >= 0 && workspace_bytes >= attn_ws + up256(n_seg * group * 8),
                "workspace too small for attention + normalisers");
  float* lse = (float*)((char*)workspace + attn_ws);
  // With room for them, the logits of the scored rows are kept by the
  // attention kernel (when the streaming kernel runs) and the scoring pass
  // reads 4 bytes per row and head instead of the K row.
  const int64_t xoff = score_logits_offset(attn_ws, n_seg, group);
  AttnLogits lg;
  lg.xlog = (float*)((char*)workspace + xoff);
  lg.mask = ca_kv_mask;
  lg.audio_s = audio_starts;
  lg.audio_e = audio_ends;
  lg.max_audio = max_audio;
  lg.hkv = (int32_t)num_kv_heads;
  const bool room = max_audio > 0 && num_kv_heads <= kLogitKv && group <= kLogitG &&
                    workspace_bytes >= xoff + n_seg * group * max_audio * 4;
  int kept = 0;
  int rc = decode_attn_impl(q, k, v, cu_k, seg_base, n_seg, group, head_dim, total_rows, kv_rows, scale,
                            dtype, out, workspace, attn_ws, WNW_ATTN_AUTO, 0, lse, room ? &lg : nullptr, &kept,
                            stream, false, app);
  if (rc != WNW_OK || n_seg == 0 || max_audio == 0) return rc;
  const int32_t* cu_scored = app ? app->cu_out : cu_k;  // the segments as the attention saw them
  if (kept) {
    LogitScoreParams lp;
    lp.xlog = lg.xlog;
    lp.acc_off = score_offsets;
    lp.acc = score_acc;
    lp.err = device_error_word();
    lp.kv_rows = kv_rows;
    lp.acc_len = acc_len;
    lp.max_audio = max_audio;
    const int32_t hg = (int32_t)num_kv_heads | ((int32_t)group << 16);  // room: Hkv <= 64, G <= 8
    const dim3 grid((unsigned)((max_audio + kLogitThreads - 1) / kLogitThreads), (unsigned)(n_seg / num_kv_heads));
    hipLaunchKernelGGL(logit_score_kernel, grid, dim3(kLogitThreads), 0, (hipStream_t)stream, audio_starts,
                       audio_ends, ca_kv_mask, cu_scored, seg_base, (const float*)lse, hg, (int32_t)n_seg, lp);
    WNW_CHECK_HIP(hipGetLastError(), "logit score launch");
    return WNW_OK;
  }
  AttnScoreParams sp;
  sp.q = q;
  sp.k = k;
  sp.cu = cu_scored;
  sp.base = seg_base;
  sp.lse = lse;
  sp.mask = ca_kv_mask;
  sp.audio_s = audio_starts;
  sp.audio_e = audio_ends;
  sp.acc_off = score_offsets;
  sp.acc = score_acc;
  sp.err = device_error_word();
  sp.kv_rows = kv_rows;
  sp.acc_len = acc_len;
  sp.n_seg = (int32_t)n_seg;
  sp.G = (int32_t)group;
  sp.Hkv = (int32_t)num_kv_heads;
  sp.scale_log2 = scale * kLog2eS;
  const int iters = score_iters(max_audio, n_seg / num_kv_heads, head_dim, elem_bytes(dtype));
  const int rows_wg = score_rows_per_wg((int)head_dim, elem_bytes(dtype), iters);
  const dim3 grid((unsigned)((max_audio + rows_wg - 1) / rows_wg), (unsigned)(n_seg / num_kv_heads));
  WNW_CHECK_HIP(launch_score(kAttnScore, dtype, head_dim, iters, grid, sp, (hipStream_t)stream),
                "attention score launch");
  return WNW_OK;
}

extern "C" int wnw_decode_attn_score(const void* q, const void* k, const void* v, const int32_t* cu_k,
                                     const int64_t* seg_base, int64_t n_seg, int64_t group, int64_t head_dim,
                                     int64_t total_rows, int64_t kv_rows, float scale, int dtype, void* out,
                                     const int32_t* ca_kv_mask, int64_t num_kv_heads,
                                     const int32_t* audio_starts, const int32_t* audio_ends,
                                     float* score_acc, const int32_t* score_offsets, int64_t acc_len,
                                     int64_t max_audio, void* workspace, int64_t workspace_bytes,
                                     void* stream) {
  return decode_attn_score_impl(q, k, v, cu_k, seg_base, n_seg, group, head_dim, total_rows, kv_rows, scale, dtype,
                                out, ca_kv_mask, num_kv_heads, audio_starts, audio_ends, score_acc, score_offsets,
                                acc_len, max_audio, workspace, workspace_bytes, stream, nullptr);
}

extern "C" int wnw_decode_attn_score_append(
    const void* q, void* k_pool, void* v_pool, const void* new_k, const void* new_v, const int32_t* cu_old,
    int32_t* cu_new, const int64_t* seg_base, const int32_t* seg_cap, int64_t n_seg, int64_t group,
    int64_t head_dim, int64_t total_rows, int64_t pool_rows, float scale, int dtype, void* out,
    const int32_t* ca_kv_mask, int64_t num_kv_heads, const int32_t* audio_starts, const int32_t* audio_ends,
    float* score_acc, const int32_t* score_offsets, int64_t acc_len, int64_t max_audio, void* workspace,
    int64_t workspace_bytes, void* stream) {
  AttnAppend app;
  app.new_k = new_k;
  app.new_v = new_v;
  app.cu_out = cu_new;
  app.cap = seg_cap;
  return decode_attn_score_impl(q, k_pool, v_pool, cu_old, seg_base, n_seg, group, head_dim, total_rows, pool_rows,
                                scale, dtype, out, ca_kv_mask, num_kv_heads, audio_starts, audio_ends, score_acc,
                                score_offsets, acc_len, max_audio, workspace, workspace_bytes, stream, &app);
}

// ---------------------------------------------------------------------------
// deferred scoring: score slots handed from one streaming launch to the next
// ---------------------------------------------------------------------------
// A slot holds one launch's final normalisers [n_seg, G, 2] and its kept
// logits [n_seg, G, max_audio] (fp32, 256-byte aligned parts).
static int64_t slot_logits_offset(int64_t n_seg, int64_t group) { return up256(n_seg * group * 2 * 4); }

extern "C" int64_t wnw_score_slot_bytes(int64_t n_seg, int64_t group, int64_t max_audio) {
  if (n_seg < 0 || group <= 0 || max_audio < 0) return -1;
  return slot_logits_offset(n_seg, group) + up256(n_seg * group * max_audio * 4);
}

// The logit pass over a slot (the scores of a launch that kept them and had
// no later launch to carry them).
extern "C" int wnw_score_kept_logits(const int32_t* kv_mask, const float* slot, const int32_t* cu,
                                     const int64_t* seg_base, int64_t kv_rows, int64_t n_seg, int64_t group,
                                     int64_t num_kv_heads, const int32_t* audio_starts, const int32_t* audio_ends,
                                     int64_t max_audio, float* score_acc, const int32_t* score_offsets,
                                     int64_t acc_len, void* stream) {
  WNW_CHECK_ARG(kv_mask && slot && cu && audio_starts && audio_ends && score_acc && score_offsets,
                "null pointer argument");
  WNW_CHECK_ARG(n_seg >= 0 && group >= 1 && group <= kLogitG && num_kv_heads >= 1 && num_kv_heads <= kLogitKv &&
                    n_seg % num_kv_heads == 0,
                "bad geometry: n_seg %lld, group %lld, num_kv_heads %lld", (long long)n_seg, (long long)group,
                (long long)num_kv_heads);
  WNW_CHECK_ARG(max_audio >= 0 && acc_len >= 0 && kv_rows >= 0, "negative size");
  WNW_CHECK_ARG(n_seg / num_kv_heads <= 65535, "at most 65535 samples (the scoring grid's y extent)");
  if (n_seg == 0 || max_audio == 0) return WNW_OK;
  LogitScoreParams lp;
  lp.xlog = slot + slot_logits_offset(n_seg, group) / 4;
  lp.acc_off = score_offsets;
  lp.acc = score_acc;
  lp.err = device_error_word();
  lp.kv_rows = kv_rows;
  lp.acc_len = acc_len;
  lp.max_audio = max_audio;
  const int32_t hg = (int32_t)num_kv_heads | ((int32_t)group << 16);
  const dim3 grid((unsigned)((max_audio + kLogitThreads - 1) / kLogitThreads), (unsigned)(n_seg / num_kv_heads));
  hipLaunchKernelGGL(logit_score_kernel, grid, dim3(kLogitThreads), 0, (hipStream_t)stream, audio_starts, audio_ends,
                     kv_mask, cu, seg_base, slot, hg, (int32_t)n_seg, lp);
  WNW_CHECK_HIP(hipGetLastError(), "logit score launch");
  return WNW_OK;
}

extern "C" int wnw_decode_attn_append_deferred(
    const void* q, void* k_pool, void* v_pool, const void* new_k, const void* new_v, const int32_t* cu_old,
    int32_t* cu_new, const int64_t* seg_base, const int32_t* seg_cap, int64_t n_seg, int64_t group,
    int64_t head_dim, int64_t total_rows, int64_t pool_rows, float scale, int dtype, void* out,
    int64_t num_kv_heads, const int32_t* audio_starts, const int32_t* audio_ends, int64_t max_audio,
    float* score_acc, const int32_t* score_offsets, int64_t acc_len, const int32_t* keep_mask, float* keep_slot,
    uint64_t prev_kv_bits, const float* prev_slot, const int32_t* prev_cu, const int64_t* prev_base,
    int64_t prev_pool_rows, void* workspace, int64_t workspace_bytes, void* stream) {
  WNW_CHECK_ARG(num_kv_heads >= 1 && num_kv_heads <= kLogitKv && n_seg % num_kv_heads == 0,
                "n_seg (%lld) must be a multiple of num_kv_heads (%lld), at most %d KV heads", (long long)n_seg,
                (long long)num_kv_heads, kLogitKv);
  WNW_CHECK_ARG((keep_mask == nullptr) == (keep_slot == nullptr), "the keep mask and its slot come together");
  WNW_CHECK_ARG(!(keep_slot && prev_slot) || (const float*)keep_slot != prev_slot,
                "this launch's slot must not be the slot it scores");
  WNW_CHECK_ARG(max_audio > 0 || (!keep_mask && !prev_slot), "scoring needs max_audio > 0");
  WNW_CHECK_ARG(!prev_slot || (prev_cu && acc_len > 0), "the scored slot needs its offsets and an accumulator");
  // the kept logits need the streaming kernel (the only one that keeps them)
  if ((keep_mask || prev_slot) &&
      !((dtype == WNW_BF16 || dtype == WNW_F16) && (head_dim == 64 || head_dim == 128) && group <= kLogitG)) {
    set_error("deferred scoring needs the streaming kernel (bf16/f16, head_dim 64 or 128, group <= %d)", kLogitG);
    return WNW_ENOTSUP;
  }
  AttnAppend app;
  app.new_k = new_k;
  app.new_v = new_v;
  app.cu_out = cu_new;
  app.cap = seg_cap;
  AttnLogits lg;
  if (keep_mask) {
    WNW_CHECK_ARG(audio_starts && audio_ends, "null audio range");
    lg.xlog = keep_slot + slot_logits_offset(n_seg, group) / 4;
    lg.mask = keep_mask;
    lg.audio_s = audio_starts;
    lg.audio_e = audio_ends;
    lg.max_audio = max_audio;
    lg.hkv = (int32_t)num_kv_heads;
  }
  AttnPrevScore pv;
  if (prev_slot) {
    pv.lse = prev_slot;
    pv.xlog = prev_slot + slot_logits_offset(n_seg, group) / 4;
    pv.kv_bits = prev_kv_bits;
    pv.cu = prev_cu;
    pv.base = prev_base;
    pv.kv_rows = prev_pool_rows;
    pv.acc = score_acc;
    pv.acc_off = score_offsets;
    pv.acc_len = acc_len;
    pv.audio_s = audio_starts;
    pv.audio_e = audio_ends;
    pv.max_audio = max_audio;
    pv.hkv = (int32_t)num_kv_heads;
  }
  int kept = 0;
  const int rc = decode_attn_impl(q, k_pool, v_pool, cu_old, seg_base, n_seg, group, head_dim, total_rows, pool_rows,
                                  scale, dtype, out, workspace, workspace_bytes, WNW_ATTN_STREAM, 0,
                                  keep_mask ? keep_slot : nullptr, keep_mask ? &lg : nullptr, &kept, stream, false,
                                  &app, prev_slot ? &pv : nullptr);
  if (rc == WNW_OK && keep_mask && !kept) {  // cannot happen with the streaming kernel
    set_error("the logits were not kept");
    return WNW_EHIP;
  }
  return rc;
}

extern "C" int64_t wnw_fused_score_workspace_bytes(int64_t n_samples, int64_t n_heads) {
  if (n_samples < 0 || n_heads <= 0) return -1;
  return up256(n_samples * kStatChunks * n_heads * 2 * 4);
}

extern "C" int wnw_fused_score_accumulate(const void* q, const void* k, const int32_t* seg_starts,
                                          const int32_t* seg_ends, const int32_t* audio_starts,
                                          const int32_t* audio_ends, float* accumulator,
                                          const int32_t* accum_offsets, int64_t n_samples, int64_t n_heads,
                                          int64_t head_dim, int64_t k_rows, int64_t acc_len, int64_t max_audio,
                                          float scale, int dtype, void* workspace, int64_t workspace_bytes,
                                          void* stream) {
  WNW_CHECK_ARG(n_samples >= 0 && n_samples < 65536, "n_samples out of range");
  if (n_samples == 0 || max_audio == 0) return WNW_OK;
  WNW_CHECK_ARG(n_heads >= 1 && n_heads <= kMaxHeads, "n_heads must be in [1, %d]", kMaxHeads);
  WNW_CHECK_ARG(head_dim == 64 || head_dim == 128 || head_dim == 256, "head_dim must be 64, 128 or 256");
  WNW_CHECK_ARG(dtype == WNW_F32 || dtype == WNW_F16 || dtype == WNW_BF16, "bad dtype %d", dtype);
  WNW_CHECK_ARG(q && k && seg_starts && seg_ends && audio_starts && audio_ends && accumulator && accum_offsets &&
                    workspace,
                "null pointer argument");
  WNW_CHECK_ARG(((uintptr_t)k % 16) == 0, "k must be 16-byte aligned");
  WNW_CHECK_ARG(max_audio > 0 && k_rows >= 0 && acc_len >= 0, "bad sizes");
  WNW_CHECK_ARG(workspace_bytes >= wnw_fused_score_workspace_bytes(n_samples, n_heads), "workspace too small");
  SegScoreParams sp;
  sp.q = q;
  sp.k = k;
  sp.seg_s = seg_starts;
  sp.seg_e = seg_ends;
  sp.audio_s = audio_starts;
  sp.audio_e = audio_ends;
  sp.acc_off = accum_offsets;
  sp.acc = accumulator;
  sp.part = (float*)workspace;
  sp.err = device_error_word();
  sp.k_rows = k_rows;
  sp.acc_len = acc_len;
  sp.S = (int32_t)n_samples;
  sp.nh = (int32_t)n_heads;
  sp.scale_log2 = scale * kLog2eS;
  hipStream_t st = (hipStream_t)stream;
  WNW_CHECK_HIP(launch_score(kSegStats, dtype, head_dim, kIters, dim3(kStatChunks, (unsigned)n_samples), sp, st),
                "score statistics launch");
  const int iters = score_iters(max_audio, n_samples, head_dim, elem_bytes(dtype));
  const int rows_wg = score_rows_per_wg((int)head_dim, elem_bytes(dtype), iters);
  const dim3 grid((unsigned)((max_audio + rows_wg - 1) / rows_wg), (unsigned)n_samples);
  WNW_CHECK_HIP(launch_score(kSegScore, dtype, head_dim, iters, grid, sp, st), "score launch");
  return WNW_OK;
}

// First-use set-up of this file's kernels on the current device (the runtime
// resolves a kernel the first time it is used: ~2 ms on MI355X); called by
// wnw_prepare_kernels.
namespace wnw {
void touch_score_kernels() {
  hipFuncAttributes a;
  (void)hipFuncGetAttributes(&a, (const void*)&logit_score_kernel);
}
}  // namespace wnw

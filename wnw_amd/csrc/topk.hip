// Chunk scores and top-k chunk choice of the decode planner (gfx950).
//
// Reference: the chunk selection of WnWCache (src/algorithms/wnw/code/
// cache.py:632-649, per sample: prefix sums of the class-A score
// accumulator, chunk means over each chunk's token bounds, topk) and its
// batched device form in the C++-planner cache (src/algorithms/wnw_cpp/
// code/cache.py:160-171: padded scatter, cumsum, gather, topk per row, -1
// where a sample has fewer chunks than k), which take five or more kernel
// launches.  Here one launch: a workgroup per sample.
//
// Chunk c of sample b covers scores [base_b + s_c, base_b + e_c) of the
// accumulator (base_b = score_offsets[b]); its mean is the difference of
// float64 prefix sums of the sample's scores at e_c and s_c, divided by
// max(1, e_c - s_c) and rounded to float32.  The k largest means are chosen in descending order;
// equal means go to the lower chunk index (the reference's torch.topk leaves
// the order of ties to the device).  Output row b holds the chosen chunk indices, -1 past the
// sample's chunk count.
#include "wnw_common.h"

namespace wnw {

static constexpr int kTopkThreads = 1024;
static constexpr int kTopkMaxChunks = 8192;  // chunks of one sample
static constexpr int kTopkMaxK = 64;
static constexpr int kTopkTok = 4;                           // scores per thread and window
static constexpr int kTopkWindow = kTopkThreads * kTopkTok;  // 4096 scores a window
static constexpr int kTopkPer = kTopkMaxChunks / kTopkThreads;  // chunks per thread
static constexpr int kTopkWaves = kTopkThreads / 64;

struct ChunkTopkParams {
  const float* acc;
  const int32_t* acc_off;    // [B + 1]
  const int32_t* chunk_off;  // [B + 1] CSR of the samples' chunks
  const int32_t* chunk_s;    // [n_chunks] token bounds relative to the sample's scores
  const int32_t* chunk_e;
  int32_t* out;              // [B, k]
  int32_t* err;
  int64_t acc_len, n_chunks;
  int32_t k;
};

// Inclusive prefix sum over the wave's 64 lanes.
__device__ __forceinline__ double wave_inclusive_scan(double v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double u = __shfl_up(v, o);
    if (lane >= o) v += u;
  }
  return v;
}

// A chunk's rank key: larger means rank higher, equal means to the lower
// index (a total order, so every lane agrees on the maximum).  Float bits are
// mapped to an unsigned order (negative values flipped); -inf stays below
// every finite mean.
__device__ __forceinline__ uint64_t rank_key(float v, int i) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)o << 32) | (uint32_t)(0x7fffffff - i);
}
__device__ __forceinline__ int rank_index(uint64_t key) { return 0x7fffffff - (int)(uint32_t)key; }
__device__ __forceinline__ uint64_t key_max(uint64_t a, uint64_t b) { return a > b ? a : b; }
template <int kCtrl>
__device__ __forceinline__ uint64_t key_dpp(uint64_t k) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)k, kCtrl, 0xf, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(k >> 32), kCtrl, 0xf, 0xf, false);
  return ((uint64_t)hi << 32) | lo;
}
// Maximum key over the wave, on the VALU: DPP within rows of 16 lanes (quad
// permutes for lanes ^1 and ^2, then the half-row and row mirrors, which
// pair lanes that already agree on their group's maximum), then the gfx950
// row swaps across rows.  Every lane ends with the wave's maximum.
__device__ __forceinline__ uint64_t wave_key_max(uint64_t k) {
  k = key_max(k, key_dpp<0xB1>(k));   // quad_perm [1, 0, 3, 2]
  k = key_max(k, key_dpp<0x4E>(k));   // quad_perm [2, 3, 0, 1]
  k = key_max(k, key_dpp<0x141>(k));  // row_half_mirror
  k = key_max(k, key_dpp<0x140>(k));  // row_mirror
  {
    const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)k, (uint32_t)k, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(k >> 32), (uint32_t)(k >> 32), false, false);
    k = key_max(((uint64_t)hi[0] << 32) | lo[0], ((uint64_t)hi[1] << 32) | lo[1]);
  }
  {
    const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)k, (uint32_t)k, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(k >> 32), (uint32_t)(k >> 32), false, false);
    k = key_max(((uint64_t)hi[0] << 32) | lo[0], ((uint64_t)hi[1] << 32) | lo[1]);
  }
  return k;
}

// One workgroup per sample.  The sample's scores stream through LDS in
// windows of 4096 (thread t holds scores 4t .. 4t+3 of the window; the next
// window's loads are issued before the current one is scanned) and are
// prefix-summed in float64: P[x] = sum of scores [0, x).  Each thread keeps
// up to eight chunks (t, t + 1024, ...) in registers and picks P at its
// chunks' bounds out of every window, so a chunk's sum P[e] - P[s] costs two
// LDS reads whatever its length and however chunks overlap.  Then wave 0
// takes the k best means (float32, as the reference's means): each lane
// keeps the best key of its chunks (c = lane mod 64), a wave maximum picks
// the round's winner, and only the winner's lane marks it and rescans its own.
// Loads are unconditional (clamped indices, validity applied at use) so that
// they stay in flight together.
__global__ __launch_bounds__(kTopkThreads) void chunk_topk_kernel(ChunkTopkParams p) {
  __shared__ double pre[kTopkWindow];  // P[w0 + i + 1] of the current window
  __shared__ double wave_tot[kTopkWaves];
  float* means = reinterpret_cast<float*>(pre);  // after the last window
  static_assert(sizeof(pre) >= kTopkMaxChunks * sizeof(float), "means alias the prefix window");
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // offsets are int32, so every index below fits 32 bits
  const int32_t c0 = p.chunk_off[b], c1 = p.chunk_off[b + 1];
  const int32_t base = p.acc_off[b], end = p.acc_off[b + 1];
  int32_t n = end - base, nc = c1 - c0;
  if (c0 < 0 || c1 < c0 || c1 > p.n_chunks || nc > kTopkMaxChunks || base < 0 || end < base || end > p.acc_len) {
    if (tid == 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
    nc = 0;  // no chunk chosen for this sample
    n = 0;
  }
  const float* a = p.acc + base;
  int32_t cs[kTopkPer], ce[kTopkPer];
  double sum[kTopkPer];
  if (nc > 0) {
#pragma unroll
    for (int m = 0; m < kTopkPer; ++m) {
      const int32_t c = min(tid + m * kTopkThreads, nc - 1);
      cs[m] = p.chunk_s[c0 + c];
      ce[m] = p.chunk_e[c0 + c];
    }
  }
#pragma unroll
  for (int m = 0; m < kTopkPer; ++m) {
    sum[m] = 0.0;
    const bool mine = tid + m * kTopkThreads < nc;
    if (!mine) {
      cs[m] = ce[m] = 0;
    } else if (!(0 <= cs[m] && cs[m] <= ce[m] && ce[m] <= n)) {
      raise_device_error(p.err, WNW_DEVERR_BOUNDS);
      cs[m] = ce[m] = -1;  // never chosen
    }
  }
  const int n_slots = (nc + kTopkThreads - 1) / kTopkThreads;  // chunk slots in use (uniform)
  float nxt[kTopkTok];
  auto load = [&](int32_t w0) {  // clamped: entries at or past n are zeroed at use
    if (w0 < n) {
#pragma unroll
      for (int i = 0; i < kTopkTok; ++i) nxt[i] = a[min(w0 + tid * kTopkTok + i, n - 1)];
    }
  };
  load(0);
  double carry = 0.0;  // P[w0]
  for (int32_t w0 = 0; w0 < n; w0 += kTopkWindow) {
    double v[kTopkTok];
#pragma unroll
    for (int i = 0; i < kTopkTok; ++i) v[i] = w0 + tid * kTopkTok + i < n ? (double)nxt[i] : 0.0;
    load(w0 + kTopkWindow);
#pragma unroll
    for (int i = 1; i < kTopkTok; ++i) v[i] += v[i - 1];
    const double incl = wave_inclusive_scan(v[kTopkTok - 1], lane);
    if (lane == 63) wave_tot[wave] = incl;
    __syncthreads();
    double before = carry, window_total = 0.0;
#pragma unroll
    for (int w = 0; w < kTopkWaves; ++w) {
      const double t = wave_tot[w];
      if (w < wave) before += t;
      window_total += t;
    }
    before += incl - v[kTopkTok - 1];  // the lanes below this one
#pragma unroll
    for (int i = 0; i < kTopkTok; ++i) pre[tid * kTopkTok + i] = before + v[i];
    __syncthreads();
    // bounds in (w0, w0 + window]: P[x] = pre[x - w0 - 1]
#pragma unroll
    for (int m = 0; m < kTopkPer; ++m) {
      if (m >= n_slots) break;  // uniform
      const int32_t rs = cs[m] - w0 - 1, re = ce[m] - w0 - 1;
      const double ps = pre[min(max(rs, 0), kTopkWindow - 1)];
      const double pe = pre[min(max(re, 0), kTopkWindow - 1)];
      sum[m] += (re >= 0 && re < kTopkWindow ? pe : 0.0) - (rs >= 0 && rs < kTopkWindow ? ps : 0.0);
    }
    carry += window_total;
    __syncthreads();  // the window is read; the next one may overwrite it
  }
#pragma unroll
  for (int m = 0; m < kTopkPer; ++m) {
    const int32_t c = tid + m * kTopkThreads;
    if (c < nc) means[c] = cs[m] < 0 ? -INFINITY : (float)(sum[m] / (double)max(1, ce[m] - cs[m]));
  }
  __syncthreads();
  if (tid >= 64) return;
  // k rounds; a round whose best is -inf (no chunk left) gives -1.  Lane l
  // only ever touches its own chunks l, l + 64, ..., so no barrier is needed
  const uint64_t none = rank_key(-INFINITY, 0x7fffffff);  // below every chunk's key
  auto lane_best = [&]() {
    uint64_t k = none;
#pragma unroll 4
    for (int32_t c = lane; c < nc; c += 64) k = key_max(k, rank_key(means[c], c));
    return k;
  };
  uint64_t mine = lane_best();
  for (int r = 0; r < p.k; ++r) {
    const uint64_t best = wave_key_max(mine);
    // a -inf mean (a chunk outside its sample's scores) is never chosen
    const bool found = (uint32_t)(best >> 32) > (uint32_t)(none >> 32);
    if (lane == 0) p.out[(int64_t)b * p.k + r] = found ? rank_index(best) : -1;
    if (found && mine == best) {  // this lane's chunk won: drop it, find the lane's next best
      means[rank_index(best)] = -INFINITY;
      mine = lane_best();
    }
  }
}

}  // namespace wnw

using namespace wnw;

extern "C" int wnw_chunk_topk(const float* score_acc, int64_t acc_len, const int32_t* score_offsets,
                              int64_t n_samples, const int32_t* chunk_offsets, const int32_t* chunk_starts,
                              const int32_t* chunk_ends, int64_t n_chunks, int64_t k, int32_t* out_idx,
                              void* stream) {
  WNW_CHECK_ARG(n_samples >= 0 && n_samples < (1 << 20), "n_samples out of range");
  WNW_CHECK_ARG(k >= 0 && k <= kTopkMaxK, "k must be in [0, %d]", kTopkMaxK);
  WNW_CHECK_ARG(n_chunks >= 0 && acc_len >= 0, "negative size");
  WNW_CHECK_ARG(acc_len <= INT32_MAX - kTopkWindow && n_chunks <= INT32_MAX, "sizes must fit 32-bit offsets");
  if (n_samples == 0 || k == 0) return WNW_OK;
  WNW_CHECK_ARG(score_acc || acc_len == 0, "null score accumulator");
  WNW_CHECK_ARG(score_offsets && chunk_offsets && out_idx && ((chunk_starts && chunk_ends) || n_chunks == 0),
                "null pointer argument");
  ChunkTopkParams p;
  p.acc = score_acc;
  p.acc_off = score_offsets;
  p.chunk_off = chunk_offsets;
  p.chunk_s = chunk_starts;
  p.chunk_e = chunk_ends;
  p.out = out_idx;
  p.err = device_error_word();
  p.acc_len = acc_len;
  p.n_chunks = n_chunks;
  p.k = (int32_t)k;
  hipLaunchKernelGGL(chunk_topk_kernel, dim3((unsigned)n_samples), dim3(kTopkThreads), 0, (hipStream_t)stream, p);
  WNW_CHECK_HIP(hipGetLastError(), "chunk top-k launch");
  return WNW_OK;
}

namespace wnw {
void touch_topk_kernels() {
  hipFuncAttributes a;
  (void)hipFuncGetAttributes(&a, (const void*)&chunk_topk_kernel);
}
}  // namespace wnw

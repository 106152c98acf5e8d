// Split-K GQA decode attention over the flat varlen KV layout (gfx950).
//
// Mathematics (reference src/common/kv/fused_attn.py:9-44 and the varlen_attn
// call of src/algorithms/wnw/code/session.py:90-106): for every segment s and
// query head g of its GQA group,
//     out[s, g] = sum_r softmax_r(scale * q[s, g] . K[r]) * V[r]
// over the rows r of segment s.
//
// Work split ("stream-K" over the logical row space).  The T = cu[n_seg]
// logical rows are cut into P equal contiguous ranges, one per workgroup, so
// every workgroup streams the same number of K/V bytes however ragged the
// segment lengths are.  A range may cover the tail of one segment, whole
// segments and the head of another; each (workgroup, segment) overlap is a
// "piece".  A piece that is a whole segment writes the output directly.  The
// others write an (m, l, acc) partial to slot (p + s) -- unique because
// ranges and segments are both monotone in the row space -- and bump the
// segment's arrival counter; the last arriver merges the partials by
// log-sum-exp and writes the output (no second kernel launch).
//
// Inside a workgroup the NW waves take 32-row (MFMA) or 64-row (VALU) steps of
// the piece round-robin, each keeping an online-softmax state; the wave states
// are merged through LDS at the end of the piece.
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
  const void* k;        // [kv_rows, D]
  const void* v;        // [kv_rows, D]
  const int32_t* cu;    // [n_seg + 1] logical offsets
  const int64_t* base;  // [n_seg] physical first row, or null (= cu)
  void* out;            // [n_seg, G, D]
  float* part_acc;      // [slots, G, D]
  float* part_ml;       // [slots, G, 2]
  int32_t* counters;    // [n_seg]
  int32_t* err;
  int64_t kv_rows;
  int32_t n_seg;
  int32_t G;
  float scale_log2;  // scale * log2(e)
};

// Per-workgroup schedule, shared through LDS.
struct SchedLds {
  int64_t T;
  int64_t B0, B1;
  int32_t P;  // effective number of workgroups (<= T)
  int32_t s_first, s_last;
  int32_t is_last;  // combine flag broadcast
  int32_t ring_lo[kRing];
  int32_t ring_hi[kRing];
  int64_t ring_base[kRing];
};

__device__ __forceinline__ int64_t range_start(int64_t p, int64_t T, int64_t P) {
  return (p * T) / P;
}
// The workgroup whose row range holds logical row j (P <= T).
__device__ __forceinline__ int64_t owner_of(int64_t j, int64_t T, int64_t P) {
  return ((j + 1) * P - 1) / T;
}

// Workgroup prologue: one pass over cu (all threads, independent loads) finds
// T, this workgroup's row range, the overlapping segments, and writes zero
// outputs for the empty segments this workgroup owns.
template <typename T, int NT>
__device__ void schedule(const AttnParams& p, int D, SchedLds& sl) {
  const int tid = threadIdx.x;
  const int N = p.n_seg;
  if (tid == 0) {
    sl.s_first = 0x7fffffff;
    sl.s_last = -1;
  }
  // All loads of the first chunk are issued before the barrier so the
  // prologue costs one global round trip for n_seg <= 4 * NT.
  const int64_t Ttot = p.cu[N];
  int32_t lo[4], hi[4];
  int64_t bs[4];
  auto load_chunk = [&](int i0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * NT + tid;
      lo[u] = 0;
      hi[u] = 0;
      bs[u] = 0;
      if (i < N) {
        lo[u] = p.cu[i];
        hi[u] = p.cu[i + 1];
        if (p.base) bs[u] = p.base[i];
      }
    }
  };
  load_chunk(0);
  __syncthreads();
  const int64_t P = Ttot > 0 ? min((int64_t)gridDim.x, Ttot) : 0;
  const int64_t pid = blockIdx.x;
  const bool active = pid < P;
  const int64_t B0 = active ? range_start(pid, Ttot, P) : 0;
  const int64_t B1 = active ? range_start(pid + 1, Ttot, P) : 0;
  for (int i0 = 0; i0 < N; i0 += 4 * NT) {
    if (i0 > 0) load_chunk(i0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * NT + tid;
      if (i >= N) continue;
      if (hi[u] < lo[u]) {  // corrupt offsets: treated as an empty segment
        raise_device_error(p.err, WNW_DEVERR_ORDER);
        hi[u] = lo[u];
      }
      if (hi[u] == lo[u]) {
        bool own = false;
        if (Ttot == 0) {
          own = (pid == 0);
        } else if (active) {
          own = (lo[u] >= B0 && lo[u] < B1) || (lo[u] == Ttot && pid == P - 1);
        }
        if (own) {
          T* o = (T*)p.out + (int64_t)i * p.G * D;
          for (int e = 0; e < p.G * D; ++e) Elem<T>::store(o, e, 0.f);
        }
      }
      // Ring membership uses "touching" ranges so every segment between
      // s_first and s_last (including empty ones) has a valid entry.
      if (active && lo[u] <= B1 && hi[u] >= B0) {
        atomicMin(&sl.s_first, i);
        atomicMax(&sl.s_last, i);
        sl.ring_lo[i % kRing] = lo[u];
        sl.ring_hi[i % kRing] = hi[u];
        sl.ring_base[i % kRing] = p.base ? bs[u] : (int64_t)lo[u];
      }
    }
  }
  if (tid == 0) {
    sl.T = Ttot;
    sl.P = (int32_t)P;
    sl.B0 = B0;
    sl.B1 = B1;
  }
  __syncthreads();
}

struct Piece {
  int64_t seg_lo, seg_hi;  // logical segment bounds
  int64_t phys;            // physical row of the piece's first row
  int32_t nrows;           // rows in the piece (-1 if the segment lies outside K/V)
  bool whole;
  bool skip;               // no rows of this segment in the workgroup's range
};

__device__ __forceinline__ Piece make_piece(const AttnParams& p, const SchedLds& sl, int s) {
  Piece pc;
  int64_t lo, hi, b;
  if (sl.s_last - sl.s_first < kRing) {
    lo = sl.ring_lo[s % kRing];
    hi = sl.ring_hi[s % kRing];
    b = sl.ring_base[s % kRing];
  } else {
    lo = p.cu[s];
    hi = p.cu[s + 1];
    b = p.base ? p.base[s] : lo;
  }
  pc.seg_lo = lo;
  pc.seg_hi = hi;
  pc.skip = !(hi > lo && lo < sl.B1 && hi > sl.B0);
  const int64_t a = max(lo, sl.B0), e = min(hi, sl.B1);
  pc.whole = (a == lo) && (e == hi);
  pc.phys = b + (a - lo);
  pc.nrows = (int32_t)(e - a);
  if (b < 0 || b + (hi - lo) > p.kv_rows) pc.nrows = -1;  // caller flags it
  return pc;
}

// Agent-scope coherent accesses (global_{load,store} sc1 on gfx950): they
// bypass the non-coherent per-XCD L2 state, so a partial written by one
// XCD is visible to a reader on another without any L2 write-back or
// invalidation of the whole cache (which a release/acquire fence costs).
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// s_waitcnt vmcnt(0): every vector memory access of this wave has completed.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

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
__device__ void finish_piece(const AttnParams& p, int D, SchedLds& sl, const Piece& pc, int s,
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
      Elem<T>::store(o, idx, A / L);
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
  const int64_t Tt = sl.T, P = sl.P;
  const int64_t p_first = min(max(owner_of(pc.seg_lo, Tt, P), (int64_t)0), P - 1);
  const int64_t p_last = min(max(owner_of(pc.seg_hi - 1, Tt, P), p_first), P - 1);
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(&p.counters[s], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sl.is_last = (old == (int)(p_last - p_first));
  }
  __syncthreads();
  if (!sl.is_last) return;  // workgroup-uniform

  T* o = (T*)p.out + (int64_t)s * GD;
  const int np = (int)(p_last - p_first + 1);
  const int64_t s0 = p_first + s;  // slot of the first piece
  // The merge area is free now; it holds the per-piece (m, l) and then the
  // per-piece weights exp2(m_q - M) / L, so the accumulator pass below has
  // no dependent loads and keeps many of them in flight.
  const int cap = NW * kMaxGroup * D;
  if (2 * np * G + 2 * G <= cap) {
    float* wm = mrg_acc;               // [np][G] m, then weights
    float* wl = mrg_acc + np * G;      // [np][G] l
    float* gm = mrg_acc + 2 * np * G;  // [G] max, [G] 1 / sum
    for (int j = tid; j < np * G; j += NT) {
      const int64_t sq = s0 + j / G;
      const int g = j % G;
      wm[j] = ld_agent(p.part_ml + (sq * G + g) * 2);
      wl[j] = ld_agent(p.part_ml + (sq * G + g) * 2 + 1);
    }
    __syncthreads();
    for (int g = tid; g < G; g += NT) {
      float M = kNegBig;
      for (int q = 0; q < np; ++q) M = fmaxf(M, wm[q * G + g]);
      float L = 0.f;
      for (int q = 0; q < np; ++q) L += wl[q * G + g] * exp2f(wm[q * G + g] - M);
      gm[g] = M;
      gm[G + g] = 1.f / L;
    }
    __syncthreads();
    for (int j = tid; j < np * G; j += NT) {
      const int g = j % G;
      wm[j] = exp2f(wm[j] - gm[g]) * gm[G + g];
    }
    __syncthreads();
    for (int idx = tid; idx < GD; idx += NT) {
      const int g = idx / D;
      float A = 0.f;
#pragma unroll 8
      for (int q = 0; q < np; ++q) A += wm[q * G + g] * ld_agent(p.part_acc + (s0 + q) * GD + idx);
      Elem<T>::store(o, idx, A);
    }
  } else {
    for (int idx = tid; idx < GD; idx += NT) {
      const int g = idx / D;
      float M = kNegBig, L = 0.f, A = 0.f;
      for (int q = 0; q < np; ++q) {
        const int64_t sq = s0 + q;
        const float mq = ld_agent(p.part_ml + (sq * G + g) * 2);
        const float lq = ld_agent(p.part_ml + (sq * G + g) * 2 + 1);
        const float aq = ld_agent(p.part_acc + sq * GD + idx);
        const float mn = fmaxf(M, mq);
        const float so = exp2f(M - mn), sn = exp2f(mq - mn);
        L = L * so + lq * sn;
        A = A * so + aq * sn;
        M = mn;
      }
      Elem<T>::store(o, idx, A / L);
    }
  }
  if (tid == 0) __hip_atomic_store(&p.counters[s], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
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
static constexpr int kVPitch = 288;  // bytes per staged V row
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
  static constexpr int kStage = NW * kStepRows * kVPitch;
  static constexpr int kMerge = NW * kMaxGroup * (D + 2) * 4;
  static constexpr int kBytes = kStage > kMerge ? kStage : kMerge;
};

template <typename T, int D, int NW>
__global__ __launch_bounds__(NW * 64, 2) void attn_mfma_kernel(AttnParams p) {
  constexpr int NT = NW * 64;
  constexpr int NC = D / 32;  // QK k-chunks
  constexpr int NTD = D / 16; // PV output tiles
  __shared__ SchedLds sl;
  __shared__ __attribute__((aligned(16))) uint8_t lds[MfmaLds<D, NW>::kBytes];

  schedule<T, NT>(p, D, sl);
  if (sl.s_first > sl.s_last) return;

  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int lq = lane >> 4;   // lane quarter
  const int lc = lane & 15;   // lane column (g for S/P, m for MFMA A rows)
  const int G = p.G;
  // K row of this lane inside a 16-row tile (rows permuted so that lane
  // quarter q ends up with rows 4i + q of the tile in the S output).
  const int krow = (lc & 3) * 4 + (lc >> 2);
  uint8_t* vst = lds + w * kStepRows * kVPitch;

  for (int s = sl.s_first; s <= sl.s_last; ++s) {
    Piece pc = make_piece(p, sl, s);
    if (pc.skip) continue;  // workgroup-uniform
    if (pc.nrows < 0) {
      if (tid == 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
      pc.nrows = 0;
    }
    // q^T operand: lane (lq, lc) holds q[g = lc][32c + 8lq .. +8].
    u32x4 qb[NC];
    {
      const uint16_t* qs = (const uint16_t*)p.q + (int64_t)s * G * D;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (lc < G)
          qb[c] = *(const u32x4*)(qs + lc * D + 32 * c + 8 * lq);
        else
          qb[c] = u32x4{0, 0, 0, 0};
      }
    }
    float m_run = kNegBig, l_run = 0.f;
    f32x4 acc[NTD];
#pragma unroll
    for (int t = 0; t < NTD; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nsteps = (pc.nrows + kStepRows - 1) / kStepRows;
    const uint16_t* kp = (const uint16_t*)p.k;
    const uint16_t* vp = (const uint16_t*)p.v;

    u32x4 kb[2][NC];
    u32x4 vb[kStepRows * D / 8 / 64];  // 16-byte chunks per lane
    constexpr int VCH = kStepRows * D / 8 / 64;
    constexpr int CPR = D / 8;          // chunks per row
    constexpr int RPI = 64 / CPR;       // rows per wave instruction

    auto issue_loads = [&](int step) {
      const int64_t r0 = pc.phys + (int64_t)step * kStepRows;
      const int valid = min(kStepRows, pc.nrows - step * kStepRows);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        int r = 16 * h + krow;
        r = r < valid ? r : valid - 1;
        const uint16_t* rowp = kp + (r0 + r) * D + 8 * lq;
#pragma unroll
        for (int c = 0; c < NC; ++c) kb[h][c] = __builtin_nontemporal_load((const u32x4*)(rowp + 32 * c));
      }
#pragma unroll
      for (int u = 0; u < VCH; ++u) {
        int r = u * RPI + lane / CPR;
        r = r < valid ? r : valid - 1;
        vb[u] = __builtin_nontemporal_load((const u32x4*)(vp + (r0 + r) * D + 8 * (lane % CPR)));
      }
    };

    int step = w;
    if (step < nsteps) issue_loads(step);
    for (; step < nsteps; step += NW) {
      const int valid = min(kStepRows, pc.nrows - step * kStepRows);
      // stage V rows (row-major, padded pitch) for the transposed reads
#pragma unroll
      for (int u = 0; u < VCH; ++u) {
        const int r = u * RPI + lane / CPR;
        *(u32x4*)(vst + r * kVPitch + (lane % CPR) * 16) = vb[u];
      }
      // S^T = K q^T for the two tiles
      f32x4 sacc[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        sacc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c) sacc[h] = MfmaOps<T>::mma(kb[h][c], qb[c], sacc[h]);
      }
      const int nstep = step + NW;
      if (nstep < nsteps) issue_loads(nstep);

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
      // O^T += V^T P^T, V^T read transposed from the staged rows
#pragma unroll
      for (int t = 0; t < NTD; ++t) {
        const uint8_t* col = vst + (16 * t + lc) * 2;
        uint32_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int r = (j < 4) ? (4 * j + lq) : (16 + 4 * (j - 4) + lq);
          e[j] = *(const uint16_t*)(col + r * kVPitch);
        }
        u32x4 a;
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = e[2 * j] | (e[2 * j + 1] << 16);
        acc[t] = MfmaOps<T>::mma(a, bh, acc[t]);
        acc[t] = MfmaOps<T>::mma(a, bl, acc[t]);
      }
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
    Piece pc = make_piece(p, sl, s);
    if (pc.skip) continue;  // workgroup-uniform
    if (pc.nrows < 0) {
      if (tid == 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
      pc.nrows = 0;
    }
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

static WsLayout ws_layout(int64_t n_seg, int64_t G, int64_t D) {
  const DeviceInfo& di = device_info();
  WsLayout L;
  L.slots = di.max_wg + n_seg;
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  L.counters = 0;
  L.ml = up(n_seg * 4);
  L.acc = L.ml + up(L.slots * G * 2 * 4);
  L.total = L.acc + up(L.slots * G * D * 4);
  return L;
}

__global__ void fill_zero_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

template <typename T, int D>
static hipError_t launch_attn(int kernel, const AttnParams& ap, int64_t n_wg, hipStream_t st) {
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

extern "C" int wnw_decode_attn_ex(const void* q, const void* k, const void* v, const int32_t* cu_k,
                                  const int64_t* seg_base, int64_t n_seg, int64_t group,
                                  int64_t head_dim, int64_t total_rows, int64_t kv_rows, float scale,
                                  int dtype, void* out, void* workspace, int64_t workspace_bytes,
                                  int kernel, int64_t n_wg, void* stream) {
  WNW_CHECK_ARG(n_seg >= 0 && n_seg < (1ll << 30), "n_seg out of range: %lld", (long long)n_seg);
  if (n_seg == 0) return WNW_OK;
  WNW_CHECK_ARG(q && cu_k && out && workspace && ((k && v) || kv_rows == 0), "null pointer argument");
  WNW_CHECK_ARG(group >= 1 && group <= kMaxGroup, "group must be in [1, %d], got %lld", kMaxGroup,
                (long long)group);
  WNW_CHECK_ARG(head_dim == 64 || head_dim == 128 || head_dim == 256,
                "head_dim must be 64, 128 or 256, got %lld", (long long)head_dim);
  WNW_CHECK_ARG(dtype == WNW_F32 || dtype == WNW_F16 || dtype == WNW_BF16, "bad dtype %d", dtype);
  WNW_CHECK_ARG(total_rows >= 0 && kv_rows >= 0, "negative row count");
  WNW_CHECK_ARG(kv_rows < (1ll << 40), "kv_rows too large");
  WNW_CHECK_ARG(((uintptr_t)q % 16) == 0 && ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0,
                "q, k and v must be 16-byte aligned");
  const WsLayout L = ws_layout(n_seg, group, head_dim);
  WNW_CHECK_ARG(workspace_bytes >= L.total, "workspace too small: %lld < %lld bytes",
                (long long)workspace_bytes, (long long)L.total);
  int kern = kernel;
  if (kern == WNW_ATTN_AUTO)
    kern = (dtype != WNW_F32 && (head_dim == 64 || head_dim == 128)) ? WNW_ATTN_MFMA : WNW_ATTN_VALU;
  WNW_CHECK_ARG(kern == WNW_ATTN_MFMA || kern == WNW_ATTN_VALU, "bad kernel id %d", kernel);
  if (kern == WNW_ATTN_MFMA)
    WNW_CHECK_ARG(dtype != WNW_F32 && (head_dim == 64 || head_dim == 128),
                  "the MFMA kernel needs bf16/f16 and head_dim 64 or 128");
  const DeviceInfo& di = device_info();
  int64_t P = n_wg;
  if (P <= 0) {
    // Balanced split of the rows over up to 2 workgroups per CU, never
    // fewer than ~64 rows per workgroup.
    const int64_t by_rows = std::max<int64_t>(1, (total_rows + 63) / 64);
    P = std::min<int64_t>((int64_t)di.cus * 2, by_rows);
  }
  P = std::max<int64_t>(1, std::min<int64_t>(P, di.max_wg));

  AttnParams ap;
  ap.q = q;
  ap.k = k;
  ap.v = v;
  ap.cu = cu_k;
  ap.base = seg_base;
  ap.out = out;
  ap.counters = (int32_t*)((char*)workspace + L.counters);
  ap.part_ml = (float*)((char*)workspace + L.ml);
  ap.part_acc = (float*)((char*)workspace + L.acc);
  ap.err = device_error_word();
  ap.kv_rows = kv_rows;
  ap.n_seg = (int32_t)n_seg;
  ap.G = (int32_t)group;
  ap.scale_log2 = scale * kLog2e;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = hipErrorInvalidValue;
  switch (dtype) {
    case WNW_BF16: e = launch_attn_d<bf16_t>(kern, head_dim, ap, P, st); break;
    case WNW_F16: e = launch_attn_d<f16_t>(kern, head_dim, ap, P, st); break;
    case WNW_F32: e = launch_attn_d<float>(kern, head_dim, ap, P, st); break;
  }
  WNW_CHECK_HIP(e, "decode attention launch");
  return WNW_OK;
}

extern "C" int wnw_decode_attn(const void* q, const void* k, const void* v, const int32_t* cu_k,
                               const int64_t* seg_base, int64_t n_seg, int64_t group,
                               int64_t head_dim, int64_t total_rows, int64_t kv_rows, float scale,
                               int dtype, void* out, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  return wnw_decode_attn_ex(q, k, v, cu_k, seg_base, n_seg, group, head_dim, total_rows, kv_rows,
                            scale, dtype, out, workspace, workspace_bytes, WNW_ATTN_AUTO, 0, stream);
}

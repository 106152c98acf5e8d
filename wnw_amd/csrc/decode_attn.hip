// Split-K GQA decode attention over the flat varlen KV layout (gfx950).
//
// Mathematics (reference src/common/kv/fused_attn.py:9-44 and the varlen_attn
// call of src/algorithms/wnw/code/session.py:90-106): for every segment s and
// query head g of its GQA group,
//     out[s, g] = sum_r softmax_r(scale * q[s, g] . K[r]) * V[r]
// over the rows r of segment s.
//
// Work split ("stream-K" over the physical row space).  The kv_rows physical
// rows of K/V are cut into P equal contiguous ranges, one per workgroup, so
// every workgroup streams the same number of bytes however ragged the
// segment lengths are.  Segments
// must be laid out in index order (base[s] + len[s] <= base[s+1]; the dense
// layout and a per-segment slack layout both are); the kernel checks it.
// A range may cover the tail of one segment, whole segments and the head of
// another; each (workgroup, segment) overlap is a "piece".  A piece that is a
// whole segment writes the output directly.  The others write an (m, l, acc)
// partial to slot (p + s) -- unique because ranges and segments are both
// monotone in the row space -- and bump the segment's arrival counter; the
// last arriver merges the partials by log-sum-exp and writes the output (no
// second kernel launch).
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
  float* lse;           // [n_seg, G, 2] final (max, sum) of each softmax, log2 domain, or null
  int32_t* err;
  int64_t kv_rows;
  int32_t n_seg;
  int32_t G;
  float scale_log2;  // scale * log2(e)
};

// Per-workgroup schedule, shared through LDS.
struct SchedLds {
  int64_t R;       // rows partitioned (kv_rows)
  int64_t B0, B1;  // this workgroup's physical row range
  int32_t P;       // effective number of workgroups (<= R)
  int32_t s_first, s_last;
  int32_t is_last;  // combine flag broadcast
  int64_t ring_base[kRing];
  int32_t ring_len[kRing];
};

__device__ __forceinline__ int64_t range_start(int64_t p, int64_t R, int64_t P) {
  return (p * R) / P;
}
// The workgroup whose row range holds physical row j (P <= R).
__device__ __forceinline__ int64_t owner_of(int64_t j, int64_t R, int64_t P) {
  return ((j + 1) * P - 1) / R;
}
__device__ __forceinline__ int64_t effective_wgs(int64_t R) {
  return R > 0 ? min((int64_t)gridDim.x, R) : 0;
}

// Workgroup prologue: one pass over cu / base (all threads, independent
// loads) finds the segments whose rows overlap this workgroup's range,
// checks the layout, and writes the outputs of empty segments (zeros) and of
// invalid ones (NaN) owned by this workgroup (segment i -> workgroup i % grid).
template <typename T, int NT>
__device__ __forceinline__ void schedule(const AttnParams& p, int D, SchedLds& sl) {
  const int tid = threadIdx.x;
  const int N = p.n_seg;
  if (tid == 0) {
    sl.s_first = 0x7fffffff;
    sl.s_last = -1;
  }
  const int64_t R = p.kv_rows;
  const int64_t P = effective_wgs(R);
  const int64_t pid = blockIdx.x;
  const bool active = pid < P;
  const int64_t B0 = active ? range_start(pid, R, P) : 0;
  const int64_t B1 = active ? range_start(pid + 1, R, P) : 0;
  int32_t lo[4], hi[4], nxt[4];
  int64_t bs[4], bn[4];
  const WNW_GLOBAL int32_t* cu = gptr<int32_t>(p.cu);
  const WNW_GLOBAL int64_t* basep = gptr<int64_t>(p.base);
  auto load_chunk = [&](int i0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * NT + tid;
      lo[u] = hi[u] = nxt[u] = 0;
      bs[u] = bn[u] = 0;
      if (i < N) {
        lo[u] = cu[i];
        hi[u] = cu[i + 1];
        if (p.base) {
          bs[u] = basep[i];
          if (i + 1 < N) bn[u] = basep[i + 1];
        } else if (i + 1 < N) {
          nxt[u] = 1;
        }
      }
    }
  };
  // The loads of the first chunk are issued before the barrier: one global
  // round trip for n_seg <= 4 * NT.
  load_chunk(0);
  __syncthreads();
  for (int i0 = 0; i0 < N; i0 += 4 * NT) {
    if (i0 > 0) load_chunk(i0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * NT + tid;
      if (i >= N) continue;
      int64_t len = (int64_t)hi[u] - lo[u];
      const int64_t b = p.base ? bs[u] : (int64_t)lo[u];
      if (len < 0) {  // corrupt offsets: treated as an empty segment
        raise_device_error(p.err, WNW_DEVERR_ORDER);
        len = 0;
      }
      // layout order: segment i must end before segment i + 1 starts
      if (p.base && i + 1 < N && b + len > bn[u]) raise_device_error(p.err, WNW_DEVERR_ORDER);
      (void)nxt;
      const bool owner = (i % (int)gridDim.x) == (int)pid;
      if (len == 0 || b < 0 || b + len > R) {
        if (len != 0) raise_device_error(p.err, WNW_DEVERR_BOUNDS);
        if (owner) {
          T* o = (T*)p.out + (int64_t)i * p.G * D;
          const float fill = len == 0 ? 0.f : __int_as_float(0x7fc00000);
          for (int e = 0; e < p.G * D; ++e) Elem<T>::store(o, e, fill);
          if (p.lse) {
            for (int g = 0; g < p.G; ++g) {
              p.lse[((int64_t)i * p.G + g) * 2] = len == 0 ? kNegBig : fill;
              p.lse[((int64_t)i * p.G + g) * 2 + 1] = len == 0 ? 0.f : fill;
            }
          }
        }
        continue;
      }
      if (active && b < B1 && b + len > B0) {
        atomicMin(&sl.s_first, i);
        atomicMax(&sl.s_last, i);
        sl.ring_base[i % kRing] = b;
        sl.ring_len[i % kRing] = (int32_t)len;
      }
    }
  }
  if (tid == 0) {
    sl.R = R;
    sl.P = (int32_t)P;
    sl.B0 = B0;
    sl.B1 = B1;
  }
  __syncthreads();
}

struct Piece {
  int64_t seg_base;  // physical first row of the segment
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

__device__ __forceinline__ Piece make_piece(const AttnParams& p, const SchedLds& sl, int s) {
  Piece pc;
  int64_t b, len;
  if (sl.s_last - sl.s_first < kRing) {
    b = sl.ring_base[s % kRing];
    len = sl.ring_len[s % kRing];
  } else {
    const int64_t lo = gptr<int32_t>(p.cu)[s], hi = gptr<int32_t>(p.cu)[s + 1];
    b = p.base ? gptr<int64_t>(p.base)[s] : lo;
    len = hi - lo;
  }
  b = uni(b);
  len = uni(len);
  pc.seg_base = b;
  pc.seg_len = len;
  // Invalid or empty segments inside [s_first, s_last] are skipped here and
  // handled by their owner in schedule(); the condition matches it exactly.
  pc.skip = !(len > 0 && b >= 0 && b + len <= uni(sl.R) && b < uni(sl.B1) && b + len > uni(sl.B0));
  const int64_t B0 = uni(sl.B0), B1 = uni(sl.B1);
  const int64_t a = max(b, B0), e = min(b + len, B1);
  pc.whole = (a == b) && (e == b + len);
  pc.phys = a;
  pc.nrows = pc.skip ? 0 : (int32_t)(e - a);
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
// s_waitcnt vmcnt(n) (expcnt and lgkmcnt not waited on), n < 64.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | ((N & 0x30) << 10));
}

// Last-arriver merge of the np partials of one segment (slots s0 .. s0+np-1)
// into the output.  The partials of consecutive slots are contiguous, so a
// chunk of pieces is one contiguous block of accumulators and one of (m, l)
// pairs: both are copied straight into LDS with agent-coherent (sc1) direct
// global->LDS loads, one memory round trip per chunk and almost no
// registers.  Per head, a wave reduces the chunk's maxima and sums across
// its lanes (one piece per lane); then every thread folds its output
// elements over the chunk.  Summation order is fixed, so results are
// deterministic.  `lds` / `lds_bytes` is the workgroup's LDS, free here.
template <typename T, int NT>
__device__ __forceinline__ void combine_pieces(const AttnParams& p, int D, int64_t s0, int np, T* o,
                                               float* lse, uint8_t* lds, int lds_bytes) {
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int G = p.G;
  const int GD = G * D;
  float* gm = (float*)lds;                    // [3][16]: M, L, rescale per head
  float* wml = gm + 3 * kMaxGroup;            // [pch][G][2]: (m, l), then (weight, l)
  const int head = 3 * kMaxGroup * 4;         // bytes before the (m, l) table
  // pieces per chunk (at most one per lane): (m, l) table (8 * G bytes each)
  // + accumulators (4 * GD bytes each), 1 KB of alignment slack
  const int room = (lds_bytes - head - 2048) / (4 * GD + 8 * G);
  const int pch = max(1, min(min(np, room), 64));
  // 1 KB aligned.  The offset is rounded as an integer so that the pointer
  // keeps its LDS address space (a round trip through uintptr_t would make
  // every access a FLAT one, which forces full memory waits).
  uint8_t* accl = lds + ((head + 8 * pch * G + 1023) & ~1023);  // [pch][GD]
  const int ept = (GD + NT - 1) / NT;
  float accv[kMaxGroup * 256 / 256];          // up to 16 elements per thread (G * D <= 4096)
#pragma unroll
  for (int e = 0; e < kMaxGroup * 256 / 256; ++e) accv[e] = 0.f;
  for (int q0 = 0; q0 < np; q0 += pch) {
    const int nq = min(pch, np - q0);
    // accumulators: nq * GD floats, 1 KB per wave-wide 16-byte load
    const int nvec = nq * GD / 4;
    const WNW_GLOBAL float* src = gptr<float>(p.part_acc + (s0 + q0) * GD);
    for (int k = w; k * 64 < nvec; k += NT / 64) {
      const int v = k * 64 + lane;
      if (v < nvec) __builtin_amdgcn_global_load_lds(src + 4 * v, accl + k * 1024, 16, 0, 16 /* sc1 */);
    }
    // (m, l) pairs: nq * G * 2 floats, 256 B per wave-wide 4-byte load
    const int nml = nq * G * 2;
    const WNW_GLOBAL float* srcm = gptr<float>(p.part_ml + (s0 + q0) * G * 2);
    for (int k = w; k * 64 < nml; k += NT / 64) {
      const int v = k * 64 + lane;
      if (v < nml) __builtin_amdgcn_global_load_lds(srcm + v, (uint8_t*)wml + k * 256, 4, 0, 16 /* sc1 */);
    }
    wait_vmcnt<0>();
    __syncthreads();
    // wave w takes heads w, w + NW, ...; lane q holds piece q of the chunk
    for (int g = w; g < G; g += NT / 64) {
      const float M = q0 == 0 ? kNegBig : gm[g];
      const float mq = lane < nq ? wml[(lane * G + g) * 2] : kNegBig;
      const float Mn = fmaxf(M, wave_max(mq));
      const float wq = lane < nq ? exp2f(mq - Mn) : 0.f;
      const float lsum = wave_sum(lane < nq ? wml[(lane * G + g) * 2 + 1] * wq : 0.f);
      if (lane < nq) wml[(lane * G + g) * 2] = wq;
      if (lane == 0) {
        const float so = exp2f(M - Mn);
        gm[kMaxGroup + g] = (q0 == 0 ? 0.f : gm[kMaxGroup + g]) * so + lsum;
        gm[2 * kMaxGroup + g] = so;
        gm[g] = Mn;
      }
    }
    __syncthreads();
    const float* acl = (const float*)accl;
    for (int e = 0; e < ept; ++e) {
      const int idx = tid + e * NT;
      if (idx < GD) {
        const int g = idx / D;
        float a = accv[e] * gm[2 * kMaxGroup + g];
#pragma unroll 8
        for (int q = 0; q < nq; ++q) a += acl[q * GD + idx] * wml[(q * G + g) * 2];
        accv[e] = a;
      }
    }
    __syncthreads();
  }
  for (int e = 0; e < ept; ++e) {
    const int idx = tid + e * NT;
    if (idx < GD) Elem<T>::store(o, idx, accv[e] / gm[kMaxGroup + idx / D]);
  }
  if (lse && tid < G) {
    lse[tid * 2] = gm[tid];
    lse[tid * 2 + 1] = gm[kMaxGroup + tid];
  }
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
                                             float* mrg_ml, float* mrg_acc, uint8_t* lds, int lds_bytes) {
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
      if (p.lse && idx - g * D == 0) {
        p.lse[((int64_t)s * G + g) * 2] = M;
        p.lse[((int64_t)s * G + g) * 2 + 1] = L;
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
  const int64_t R = sl.R, P = sl.P;
  const int64_t p_first = min(max(owner_of(pc.seg_base, R, P), (int64_t)0), P - 1);
  const int64_t p_last = min(max(owner_of(pc.seg_base + pc.seg_len - 1, R, P), p_first), P - 1);
  if (tid == 0) {
    const int old = __hip_atomic_fetch_add(&p.counters[s], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sl.is_last = (old == (int)(p_last - p_first));
  }
  __syncthreads();
  if (!sl.is_last) return;  // workgroup-uniform

  T* o = (T*)p.out + (int64_t)s * GD;
  const int np = (int)(p_last - p_first + 1);
  const int64_t s0 = p_first + s;  // slot of the first piece
  combine_pieces<T, NT>(p, D, s0, np, o, p.lse ? p.lse + (int64_t)s * G * 2 : nullptr, lds, lds_bytes);
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
    finish_piece<T, NT, NW>(p, D, sl, pc, s, mrg_ml, mrg_acc, lds, MfmaLds<D, NW>::kBytes);
  }
  wait_vmcnt<0>();
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
    finish_piece<T, NT, NW>(p, D, sl, pc, s, mrg_ml, mrg_acc, lds, ValuLds<D, NW>::kBytes);
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

namespace wnw {
// Shared by the public attention entry points; lse (optional) receives each
// segment's final softmax (max, sum) in the log2 domain, [n_seg, G, 2].
int decode_attn_impl(const void* q, const void* k, const void* v, const int32_t* cu_k,
                     const int64_t* seg_base, int64_t n_seg, int64_t group, int64_t head_dim,
                     int64_t total_rows, int64_t kv_rows, float scale, int dtype, void* out,
                     void* workspace, int64_t workspace_bytes, int kernel, int64_t n_wg, float* lse,
                     void* stream) {
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
    const int64_t by_rows = std::max<int64_t>(1, (kv_rows + 63) / 64);
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
  ap.lse = lse;
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

}  // namespace wnw

extern "C" int wnw_decode_attn_ex(const void* q, const void* k, const void* v, const int32_t* cu_k,
                                  const int64_t* seg_base, int64_t n_seg, int64_t group,
                                  int64_t head_dim, int64_t total_rows, int64_t kv_rows, float scale,
                                  int dtype, void* out, void* workspace, int64_t workspace_bytes,
                                  int kernel, int64_t n_wg, void* stream) {
  return decode_attn_impl(q, k, v, cu_k, seg_base, n_seg, group, head_dim, total_rows, kv_rows, scale,
                          dtype, out, workspace, workspace_bytes, kernel, n_wg, nullptr, stream);
}

extern "C" int wnw_decode_attn(const void* q, const void* k, const void* v, const int32_t* cu_k,
                               const int64_t* seg_base, int64_t n_seg, int64_t group,
                               int64_t head_dim, int64_t total_rows, int64_t kv_rows, float scale,
                               int dtype, void* out, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  return wnw_decode_attn_ex(q, k, v, cu_k, seg_base, n_seg, group, head_dim, total_rows, kv_rows,
                            scale, dtype, out, workspace, workspace_bytes, WNW_ATTN_AUTO, 0, stream);
}

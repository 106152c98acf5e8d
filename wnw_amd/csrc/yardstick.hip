// Read-only HBM streaming kernels: the rate a single launch of a given size
// and grid reaches when it only reads, the yardstick beside the decode
// attention launch (which reads the same bytes and adds the softmax, the
// split-K hand-off and the combine).  Measurement code: no counterpart in
// the reference, not on the decode path.
//
// Workgroup i of n_wg reads the i-th contiguous share of the buffer (16-byte
// chunks, rounded to whole chunks), its 256 threads striding through it.
//  * VGPR form: each thread keeps two batches of U 16-byte loads in flight
//    (the next batch is issued before the current one is consumed) and XORs
//    what arrives; U = 4 gives 64 KB in flight per workgroup, as many bytes
//    as the attention kernel's four waves with two 16-row K+V steps each.
//  * LDS form: the attention kernel's own load path -- 1 KB per wave and
//    instruction straight into LDS (global_load_lds_dwordx4), a ring of
//    steps per wave with explicit waits, and one LDS read per lane and step
//    to consume it.
// A workgroup writes to `sink` only if the XOR of everything it read equals
// a fixed constant, so the loads cannot be dropped and (for the buffers the
// bench fills) nothing is written.
#include "wnw_common.h"

namespace wnw {

template <int U>
__global__ __launch_bounds__(256) void read_stream_vgpr_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                               int64_t per_wg, uint32_t* sink) {
  const int64_t lo = (int64_t)blockIdx.x * per_wg;
  const int64_t hi = lo + per_wg < n16 ? lo + per_wg : n16;
  const WNW_GLOBAL u32x4* s = gptr<u32x4>(src);
  u32x4 acc = {0, 0, 0, 0};
  constexpr int64_t kBatch = (int64_t)U * 256;
  int64_t i = lo + threadIdx.x;
  u32x4 a[U], b[U];
  // every load is issued (index clamped to the share's last chunk, which
  // exists: hi >= 1), and the chunks past the share are dropped after
  // arrival, so no load waits behind a branch
  const int64_t last = hi - 1;
  auto load = [&](u32x4 (&r)[U], int64_t at) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = at + (int64_t)u * 256;
      r[u] = s[j < hi ? j : last];
    }
    __builtin_amdgcn_sched_barrier(0);  // the whole batch is issued before anything is consumed
  };
  auto eat = [&](const u32x4 (&r)[U], int64_t at) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool in = at + (int64_t)u * 256 < hi;
      acc ^= in ? r[u] : u32x4{0, 0, 0, 0};
    }
  };
  // batches at i (a) and i + kBatch (b) in flight; the loop eats a, loads
  // the batch after b into a, then eats b
  if (i < hi) {
    load(a, i);
    while (true) {
      const int64_t ib = i + kBatch;
      if (ib >= hi) {
        eat(a, i);
        break;
      }
      load(b, ib);
      eat(a, i);
      const int64_t ia = ib + kBatch;
      if (ia >= hi) {
        eat(b, ib);
        break;
      }
      load(a, ia);
      eat(b, ib);
      i = ia;
    }
  }
  const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (x == 0x9e3779b9u) sink[(int64_t)blockIdx.x * 256 + threadIdx.x] = x;
}

// 16 bytes per lane from gbase + voff into LDS at lds_addr + 16 * lane (M0
// carries the LDS address and is restored after the load).
__device__ __forceinline__ void ys_dma16(const void* gbase, uint32_t voff, uint32_t lds_addr) {
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

template <int N>
__device__ __forceinline__ void ys_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// LDS form: per wave a ring of 2 steps of SB bytes (8 KB: a 16-row K+V step
// of D = 128), issued as SB / 1 KB loads, one step consumed while the next
// is in flight.
__global__ __launch_bounds__(256) void read_stream_lds_kernel(const uint8_t* __restrict__ src, int64_t n_steps,
                                                              int64_t steps_per_wave, uint32_t* sink) {
  constexpr int SB = 8192, NI = SB / 1024;
  __shared__ __attribute__((aligned(16))) uint8_t ring[4][2][SB];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * 4 + w;
  const int64_t s0 = wave * steps_per_wave;
  const int64_t s1 = s0 + steps_per_wave < n_steps ? s0 + steps_per_wave : n_steps;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(
      const __attribute__((address_space(3))) void*)&ring[w][0][0]);
  auto issue = [&](int64_t step, int b) {
    const void* base = src + step * SB;
#pragma unroll
    for (int u = 0; u < NI; ++u) ys_dma16(base, (uint32_t)(u * 1024 + lane * 16), lds0 + b * SB + u * 1024);
  };
  u32x4 acc = {0, 0, 0, 0};
  int64_t st = s0;
  if (st < s1) issue(st, 0);
  int b = 0;
  for (; st < s1; ++st) {
    const bool next = st + 1 < s1;
    if (next) issue(st + 1, b ^ 1);
    if (next)
      ys_wait_vmcnt<NI>();
    else
      ys_wait_vmcnt<0>();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < NI; ++u) acc ^= *(const u32x4*)(&ring[w][b][u * 1024 + lane * 16]);
    __builtin_amdgcn_sched_barrier(0);
    b ^= 1;
  }
  const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (x == 0x9e3779b9u) sink[(int64_t)blockIdx.x * 256 + threadIdx.x] = x;
}

}  // namespace wnw

extern "C" int wnw_read_stream(const void* src, int64_t bytes, int64_t n_wg, int form, void* sink, void* stream) {
  using namespace wnw;
  WNW_CHECK_ARG(src && sink, "read_stream: null pointer");
  WNW_CHECK_ARG(bytes > 0 && bytes % 8192 == 0, "read_stream: bytes must be a positive multiple of 8192");
  WNW_CHECK_ARG(n_wg >= 1 && n_wg <= 65535, "read_stream: n_wg must be in [1, 65535]");
  WNW_CHECK_ARG(form == 0 || form == 2 || form == 4 || form == 8, "read_stream: form must be 0 (LDS) or 2, 4, 8");
  WNW_CHECK_ARG(((uintptr_t)src & 15) == 0, "read_stream: src must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)n_wg), block(256);
  if (form == 0) {
    const int64_t n_steps = bytes / 8192;
    const int64_t waves = n_wg * 4;
    const int64_t per = (n_steps + waves - 1) / waves;
    hipLaunchKernelGGL(read_stream_lds_kernel, grid, block, 0, st, (const uint8_t*)src, n_steps, per,
                       (uint32_t*)sink);
  } else {
    const int64_t n16 = bytes / 16;
    const int64_t per = (n16 + n_wg - 1) / n_wg;
    const u32x4* s = (const u32x4*)src;
    if (form == 2)
      hipLaunchKernelGGL(read_stream_vgpr_kernel<2>, grid, block, 0, st, s, n16, per, (uint32_t*)sink);
    else if (form == 4)
      hipLaunchKernelGGL(read_stream_vgpr_kernel<4>, grid, block, 0, st, s, n16, per, (uint32_t*)sink);
    else
      hipLaunchKernelGGL(read_stream_vgpr_kernel<8>, grid, block, 0, st, s, n16, per, (uint32_t*)sink);
  }
  WNW_CHECK_HIP(hipGetLastError(), "read_stream launch");
  return WNW_OK;
}

// Offload channel: rows of the pinned host restore arrays gathered straight
// into device memory by a kernel (gfx950).
//
// The reference gathers the planned host ranges into a pinned staging buffer
// with memcpy on the host (src/algorithms/wnw_cpp/code/planner.cpp:113-122,
// or torch.cat in src/algorithms/wnw/code/cache.py:868-873) and then copies
// the staging buffer to the device (cache.py:874-881).  Here the device reads
// the pinned host memory itself: a few workgroups stream the ranges
// over the host link into the destination rows, so the host does no copying
// at all and the transfer can be cut per layer (each layer's ranges are
// contiguous in the transfer order) to overlap with the compute of earlier
// layers.
#include <algorithm>

#include "wnw_common.h"

namespace wnw {

// A few workgroups take the ranges r0 .. r1 - 1 in turn (range r0 + i goes
// to workgroup i % gridDim.x) and copy rows [ranges[2r], ranges[2r+1]) of
// host K and V to rows [dst_off[r], dst_off[r+1]) of the outputs.  Reads of
// host memory have a long latency and occupy their CU's memory pipeline
// while in flight, so the gather keeps to a few CUs (with several reads in
// flight per thread) and leaves the others to the compute that overlaps it.
// A range outside either array raises WNW_DEVERR_BOUNDS and is skipped.
static constexpr int kGatherWgs = 8;

__global__ __launch_bounds__(256) void gather_host_rows_kernel(const u32x4* host_k, const u32x4* host_v,
                                                               int64_t host_rows, const int32_t* ranges,
                                                               const int64_t* dst_off, int64_t r0, int64_t r1,
                                                               int64_t row_vec, u32x4* out_k, u32x4* out_v,
                                                               int64_t out_rows, int32_t* err) {
  const WNW_GLOBAL int32_t* rg = gptr<int32_t>(ranges);
  const WNW_GLOBAL int64_t* dof = gptr<int64_t>(dst_off);
  for (int64_t r = r0 + blockIdx.x; r < r1; r += gridDim.x) {
    const int64_t s = rg[2 * r], e = rg[2 * r + 1];
    const int64_t d0 = dof[r], d1 = dof[r + 1];
    if (s < 0 || e < s || e > host_rows || d0 < 0 || d1 > out_rows || d1 - d0 != e - s) {
      if (threadIdx.x == 0) raise_device_error(err, WNW_DEVERR_BOUNDS);
      continue;
    }
    const int64_t n = (e - s) * row_vec;  // 16-byte vectors per tensor
    const u32x4* sk = host_k + s * row_vec;
    const u32x4* sv = host_v + s * row_vec;
    WNW_GLOBAL u32x4* dk = (WNW_GLOBAL u32x4*)out_k + d0 * row_vec;
    WNW_GLOBAL u32x4* dv = (WNW_GLOBAL u32x4*)out_v + d0 * row_vec;
    // two 16-byte reads of each tensor in flight per thread: with 8
    // workgroups that is 128 KB in flight, enough for the host link's
    // bandwidth, and few enough not to hold up other CUs' memory traffic
    constexpr int U = 2;
    int64_t i = threadIdx.x;
    for (; i + (U - 1) * 256 < n; i += U * 256) {
      u32x4 a[U], b[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        a[u] = __builtin_nontemporal_load(sk + i + u * 256);
        b[u] = __builtin_nontemporal_load(sv + i + u * 256);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        dk[i + u * 256] = a[u];
        dv[i + u * 256] = b[u];
      }
    }
    for (; i < n; i += 256) {
      dk[i] = __builtin_nontemporal_load(sk + i);
      dv[i] = __builtin_nontemporal_load(sv + i);
    }
  }
}

// The device address of a host allocation, or null when the device cannot
// read it (not pinned, or not mapped for the current device).
static const void* device_view(const void* host) {
  hipPointerAttribute_t a;
  if (hipPointerGetAttributes(&a, host) != hipSuccess) {
    (void)hipGetLastError();  // clear the sticky error of a failed query
    return nullptr;
  }
  if (a.type != hipMemoryTypeHost || a.devicePointer == nullptr) return nullptr;
  return a.devicePointer;
}

}  // namespace wnw

using namespace wnw;

extern "C" int wnw_host_rows_readable(const void* host_k, const void* host_v) {
  return host_k && host_v && device_view(host_k) && device_view(host_v) ? 1 : 0;
}

extern "C" int wnw_gather_host_rows(const void* host_k, const void* host_v, int64_t host_rows,
                                    const int32_t* ranges, const int64_t* dst_off, int64_t r0, int64_t r1,
                                    int64_t row_bytes, void* out_k, void* out_v, int64_t out_rows, void* stream) {
  WNW_CHECK_ARG(r0 >= 0 && r1 >= r0 && r1 - r0 <= (int64_t)0x7fffffff, "bad range span [%lld, %lld)",
                (long long)r0, (long long)r1);
  if (r1 == r0) return WNW_OK;
  WNW_CHECK_ARG(ranges && dst_off && out_k && out_v, "null pointer argument");
  WNW_CHECK_ARG(row_bytes > 0 && row_bytes % 16 == 0, "row_bytes must be a positive multiple of 16");
  WNW_CHECK_ARG(host_rows >= 0 && out_rows >= 0, "negative row count");
  WNW_CHECK_ARG(((uintptr_t)out_k % 16) == 0 && ((uintptr_t)out_v % 16) == 0, "outputs must be 16-byte aligned");
  const void* dk = device_view(host_k);
  const void* dv = device_view(host_v);
  if (!dk || !dv) {
    set_error("host rows are not pinned memory the device can read");
    return WNW_ENOTSUP;
  }
  WNW_CHECK_ARG(((uintptr_t)dk % 16) == 0 && ((uintptr_t)dv % 16) == 0, "host rows must be 16-byte aligned");
  const unsigned grid = (unsigned)std::min<int64_t>(r1 - r0, kGatherWgs);
  hipLaunchKernelGGL(gather_host_rows_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const u32x4*)dk,
                     (const u32x4*)dv, host_rows, ranges, dst_off, r0, r1, row_bytes / 16, (u32x4*)out_k,
                     (u32x4*)out_v, out_rows, device_error_word());
  WNW_CHECK_HIP(hipGetLastError(), "gather_host_rows launch");
  return WNW_OK;
}

namespace wnw {
void touch_offload_kernels() {
  hipFuncAttributes a;
  (void)hipFuncGetAttributes(&a, (const void*)&gather_host_rows_kernel);
}
}  // namespace wnw

// Shared host/device helpers of the gfx950 kernels: element types, bf16/f16
// conversions, wave-level exchanges, error reporting.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/wnw_amd.h"

namespace wnw {

// ---------------------------------------------------------------------------
// host-side error reporting
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);
// Per-device error word (allocated once per device by the library).
int32_t* device_error_word();
// Compute units of the current device (queried once per device; 256 when
// the query fails).
int device_cus();
// The host planner's layer count and batch size (planner.cpp).
void planner_dims(const wnw_planner* p, int* layers, int* batch);

// Logits of the scored (class-A) audio rows, kept by the streaming attention
// kernel for the scoring pass: xlog[(s * G + g) * max_audio + t].
struct AttnLogits {
  float* xlog;
  const int32_t* mask;     // [hkv] non-zero: KV head scored
  const int32_t* audio_s;  // [n_seg / hkv], relative to the segments' starts
  const int32_t* audio_e;
  int64_t max_audio;
  int32_t hkv;
};

// The step's append of one row per segment, done before the attention reads
// the segments: fused into the streaming kernel, else by the in-place append
// kernel first.  Needs a slack layout (seg_base).
struct AttnAppend {
  const void* new_k;   // [n_seg, D]
  const void* new_v;
  int32_t* cu_out;     // [n_seg + 1] = cu + arange(n_seg + 1); must not alias cu
  const int32_t* cap;  // [n_seg] rows each segment may occupy from its base
};

// Deferred class-A scoring: the logits and normalisers a previous streaming
// launch kept (a score slot), scored by the next streaming launch while its
// first loads are in flight.  Rules as logit_score_kernel's.
struct AttnPrevScore {
  const float* lse;        // [n_seg, G, 2] final (max, sum), log2 domain
  const float* xlog;       // [n_seg, G, max_audio]
  uint64_t kv_bits;        // bit h: KV head h scored by that launch
  const int32_t* cu;       // [n_seg + 1] its offsets after its append
  const int64_t* base;     // [n_seg] its physical first rows (or null: cu)
  int64_t kv_rows;         // its pool rows
  float* acc;              // class-A accumulator, acc_off [B + 1], acc_len entries
  const int32_t* acc_off;
  int64_t acc_len;
  const int32_t* audio_s;  // [B]
  const int32_t* audio_e;
  int64_t max_audio;
  int32_t hkv;
};

// Shared by the public attention entry points; lse (optional) receives each
// segment's final softmax (max, sum) in the log2 domain, [n_seg, G, 2].
// logits (optional) is honoured by the streaming kernel only; *logits_kept
// (optional) tells whether they were written.  total_rows = the logical rows
// the work split covers (after the append, with app).  noalloc: use the
// library's own scratch instead of the workspace argument.
int decode_attn_impl(const void* q, const void* k, const void* v, const int32_t* cu_k,
                     const int64_t* seg_base, int64_t n_seg, int64_t group, int64_t head_dim,
                     int64_t total_rows, int64_t kv_rows, float scale, int dtype, void* out,
                     void* workspace, int64_t workspace_bytes, int kernel, int64_t n_wg, float* lse,
                     const AttnLogits* logits, int* logits_kept, void* stream, bool noalloc,
                     const AttnAppend* app, const AttnPrevScore* prev = nullptr);

#define WNW_CHECK_ARG(cond, ...)       \
  do {                                 \
    if (!(cond)) {                     \
      ::wnw::set_error(__VA_ARGS__);   \
      return WNW_EINVAL;               \
    }                                  \
  } while (0)

#define WNW_CHECK_HIP(expr, what)                         \
  do {                                                    \
    hipError_t e_ = (expr);                               \
    if (e_ != hipSuccess) return ::wnw::hip_fail(e_, what); \
  } while (0)

inline int elem_bytes(int dtype) { return dtype == WNW_F32 ? 4 : 2; }

// ---------------------------------------------------------------------------
// element types
// ---------------------------------------------------------------------------
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t qnan = ((u >> 16) | 0x40u) & 0xffffu;
  return (u & 0x7fffffffu) > 0x7f800000u ? qnan : rne;  // a select, not a branch
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// Element traits: load one element as float / store float as element.
template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kBytes = 4;
  __device__ static float to_f32(const float* p, int64_t i) { return p[i]; }
  __device__ static void store(float* p, int64_t i, float x) { p[i] = x; }
};
template <> struct Elem<bf16_t> {
  static constexpr int kBytes = 2;
  __device__ static float to_f32(const bf16_t* p, int64_t i) {
    return __uint_as_float(((uint32_t)p[i].bits) << 16);
  }
  __device__ static void store(bf16_t* p, int64_t i, float x) {
    p[i].bits = (uint16_t)f32_to_bf16_bits(x);
  }
};
template <> struct Elem<f16_t> {
  static constexpr int kBytes = 2;
  __device__ static float to_f32(const f16_t* p, int64_t i) { return f16_bits_to_f32(p[i].bits); }
  __device__ static void store(f16_t* p, int64_t i, float x) {
    p[i].bits = (uint16_t)f32_to_f16_bits(x);
  }
};

// Unpack 8 packed 16-bit elements (one 16-byte chunk) to fp32.
__device__ __forceinline__ void unpack8(const u32x4& w, float* f, bf16_t*) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(w[i]);
    f[2 * i + 1] = bf16_hi(w[i]);
  }
}
__device__ __forceinline__ void unpack8(const u32x4& w, float* f, f16_t*) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
    f[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
  }
}

// ---------------------------------------------------------------------------
// wave-level exchanges (wave64)
// ---------------------------------------------------------------------------
// x from lane (lane ^ 16), within each 32-lane half.
__device__ __forceinline__ float swap16(float x) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401F));
}
// x from lane (lane ^ 32).
__device__ __forceinline__ float swap32(float x) { return __shfl_xor(x, 32); }

// Max / sum of x over lanes l and l ^ 16 (or l ^ 32) with the gfx950 row
// swaps (v_permlane16_swap / v_permlane32_swap: VALU, no LDS round trip).
// Each returns the pair {x[l], x[l ^ 16]} with the lower row's value first,
// so both lanes of a pair compute the same result.
__device__ __forceinline__ float max_x16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_x32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_x16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_x32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

__device__ __forceinline__ void raise_device_error(int32_t* err, int bits) {
  if (err) atomicOr(err, bits);
}

// Global-memory pointers.  Pointers that reach a kernel inside a struct are
// generic; accessing through them emits FLAT instructions, which are slower
// and count against both vmcnt and lgkmcnt.  Casting to address space 1 gives
// global_* instructions with the scalar-base addressing form.
#define WNW_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ const WNW_GLOBAL T* gptr(const void* p) {
  return (const WNW_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ WNW_GLOBAL T* gptr_w(void* p) {
  return (WNW_GLOBAL T*)p;
}

// Element i of a T array at `base` = x (rounded to nearest even), through a
// global pointer.
template <typename T>
__device__ __forceinline__ void store_elem(void* base, int64_t i, float x);
template <>
__device__ __forceinline__ void store_elem<float>(void* base, int64_t i, float x) {
  gptr_w<float>(base)[i] = x;
}
template <>
__device__ __forceinline__ void store_elem<bf16_t>(void* base, int64_t i, float x) {
  gptr_w<uint16_t>(base)[i] = (uint16_t)f32_to_bf16_bits(x);
}
template <>
__device__ __forceinline__ void store_elem<f16_t>(void* base, int64_t i, float x) {
  gptr_w<uint16_t>(base)[i] = (uint16_t)f32_to_f16_bits(x);
}

__device__ __forceinline__ uint32_t half_bits(float x, bf16_t*) { return f32_to_bf16_bits(x); }
__device__ __forceinline__ uint32_t half_bits(float x, f16_t*) { return f32_to_f16_bits(x); }

// Elements i .. i + 3 (i a multiple of 4) of a T array at `base` = v, in one
// store (rounded to nearest even).
template <typename T>
__device__ __forceinline__ void store_quad(void* base, int64_t i, const float (&v)[4]) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  if constexpr (sizeof(T) == 4) {
    *(WNW_GLOBAL u32x4*)(gptr_w<float>(base) + i) =
        u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
  } else {
    auto cv = [](float x) -> uint32_t { return half_bits(x, (T*)nullptr); };
    *(WNW_GLOBAL u32x2_t*)(gptr_w<uint16_t>(base) + i) =
        u32x2_t{cv(v[0]) | (cv(v[1]) << 16), cv(v[2]) | (cv(v[3]) << 16)};
  }
}

}  // namespace wnw

// Host-side bulk copy for the transfer engine's gather into pinned staging
// (host-only C++, built with the host compiler).
//
// The staging rows are written once by the CPU and then read by the DMA
// engines, never by the CPU again, so they are written with non-temporal
// (streaming) stores: no read-for-ownership of the destination lines and no
// eviction of the caches' useful contents.  SSE2 (part of x86-64).
#include <emmintrin.h>

#include <cstdint>
#include <cstring>

#include "hostcopy.h"

namespace wnw {

void stream_copy(void* dst, const void* src, size_t n) {
  if (((uintptr_t)dst | (uintptr_t)src | n) & 15) {  // unaligned: plain copy
    std::memcpy(dst, src, n);
    return;
  }
  const __m128i* s = static_cast<const __m128i*>(src);
  __m128i* d = static_cast<__m128i*>(dst);
  const size_t k = n / 16;
  size_t i = 0;
  for (; i + 8 <= k; i += 8) {
    const __m128i a0 = _mm_load_si128(s + i), a1 = _mm_load_si128(s + i + 1), a2 = _mm_load_si128(s + i + 2),
                  a3 = _mm_load_si128(s + i + 3), a4 = _mm_load_si128(s + i + 4), a5 = _mm_load_si128(s + i + 5),
                  a6 = _mm_load_si128(s + i + 6), a7 = _mm_load_si128(s + i + 7);
    _mm_stream_si128(d + i, a0);
    _mm_stream_si128(d + i + 1, a1);
    _mm_stream_si128(d + i + 2, a2);
    _mm_stream_si128(d + i + 3, a3);
    _mm_stream_si128(d + i + 4, a4);
    _mm_stream_si128(d + i + 5, a5);
    _mm_stream_si128(d + i + 6, a6);
    _mm_stream_si128(d + i + 7, a7);
  }
  for (; i < k; ++i) _mm_stream_si128(d + i, _mm_load_si128(s + i));
}

void stream_fence() { _mm_sfence(); }

}  // namespace wnw

// Host-side bulk copy with non-temporal stores (hostcopy.cpp).
#pragma once
#include <cstddef>

namespace wnw {
// dst <- src (n bytes); streaming stores when both are 16-byte aligned and
// n is a multiple of 16, else memcpy.  Call stream_fence() before another
// agent (a DMA engine) reads what this thread wrote.
void stream_copy(void* dst, const void* src, size_t n);
void stream_fence();
}  // namespace wnw

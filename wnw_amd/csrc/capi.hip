// Library-wide host glue of the C ABI: thread-local error messages, the
// per-device error word that kernels set instead of reading out of bounds,
// and version queries.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <vector>

#include "wnw_common.h"

namespace wnw {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int hip_fail(hipError_t e, const char* what) {
  set_error("%s: %s (%d)", what, hipGetErrorString(e), (int)e);
  return WNW_EHIP;
}

static std::mutex g_mu;
static std::vector<int32_t*> g_err_words;

// The word kernels record WNW_DEVERR_* bits into: one per device, a
// file-scope device array (zero at load, so nothing is allocated for it).
// Host code reaches it only through the per-device address that
// hipGetSymbolAddress returns with that device current.
static __device__ __align__(256) int32_t g_err_word[64];

// The device address of the current device's error word (resolved once per
// device), or null if the lookup failed, in which case kernels skip the
// recording but still refuse bad offsets.
int32_t* device_error_word() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_mu);
  if ((int)g_err_words.size() <= dev) g_err_words.resize(dev + 1, nullptr);
  if (!g_err_words[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_err_word)) != hipSuccess || !p) return nullptr;
    g_err_words[dev] = (int32_t*)p;
  }
  return g_err_words[dev];
}

int device_cus() {
  static std::vector<int> cus;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(g_mu);
  if ((int)cus.size() <= dev) cus.resize(dev + 1, 0);
  if (cus[dev] == 0) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cus[dev];
}

}  // namespace wnw

extern "C" const char* wnw_last_error(void) { return wnw::g_err; }

extern "C" int wnw_abi_version(void) { return 1; }

extern "C" int wnw_init(void) {
  int32_t* w = wnw::device_error_word();
  if (!w) {
    wnw::set_error("could not resolve the device error word");
    return WNW_EHIP;
  }
  return WNW_OK;
}

// Each source file's kernels of the default decode path (the scoring pass,
// the chunk top-k, the stage permute, the slack compaction, in-place and
// dense appends and rebuild, the host-row gather), resolved on the current
// device: the runtime sets a kernel up the first time it is used.
namespace wnw {
void touch_score_kernels();
void touch_topk_kernels();
void touch_transfer_kernels();
void touch_append_kernels();
void touch_offload_kernels();
}  // namespace wnw
extern "C" int wnw_prepare_kernels(void) {
  wnw::touch_score_kernels();
  wnw::touch_topk_kernels();
  wnw::touch_transfer_kernels();
  wnw::touch_append_kernels();
  wnw::touch_offload_kernels();
  return WNW_OK;
}

extern "C" int wnw_device_error(int clear) {
  int32_t* w = wnw::device_error_word();
  if (!w) return -1;
  if (hipDeviceSynchronize() != hipSuccess) return -1;
  int32_t v = 0;
  if (hipMemcpy(&v, w, 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  if (clear && v != 0) {
    if (hipMemset(w, 0, 4) != hipSuccess) return -1;
  }
  return v;
}

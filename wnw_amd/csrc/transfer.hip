// Host->device transfer of a plan's offloaded rows through the copy engines
// (host code only; no kernels).
//
// Reference: the offload channel of the WnW caches -- the planner gathers
// the plan's host ranges into pinned staging (src/algorithms/wnw_cpp/code/
// planner.cpp:113-122) and the cache copies the staging rows to the device
// on a side stream and makes the rebuild wait for it
// (src/algorithms/wnw/code/cache.py:716-721, :868-881).  There the gather
// runs on one thread and one copy carries every layer's rows, so the first
// layer's rebuild waits for the whole transfer.
//
// Two forms of a job.  Staged (wnw_h2d_start): the ranges (in transfer
// order: layer, sample, head, segment) are split into groups of consecutive
// layers.  A background thread per
// engine walks the groups: a pool of worker threads memcpys the group's
// ranges into the staging rows (ranges split evenly over the workers,
// written with streaming stores: the staging is read by the DMA engines
// only), then
// the thread issues two hipMemcpyAsync (K and V) of the group's staging
// rows into the same rows of the device buffers, and records an event.  A
// layer's rebuild waits for its group's event only, so later groups' host
// gathers and copies overlap earlier layers' compute, and the copies run on
// the DMA engines: unlike a kernel reading pinned host memory, they leave
// the compute kernels' memory traffic alone.
//
// Direct (wnw_h2d_start_direct): no host gather at all.  A group's ranges
// are taken in host-row order, ranges that touch in host memory are merged
// into spans, and each span is copied by the DMA engines straight from the
// pinned host rows into the group's rows of a device stage buffer (in that
// host order; the spans' K and V copies dealt in turn over two copy
// streams, the device's pair);
// once both are done, a kernel on the job's stream moves every range from
// the stage to its transfer-order rows of the outputs, and the group's event
// is recorded.  With a host layout that keeps a segment's rows of consecutive
// layers together, a group is a few large spans, so the host link is the
// only bound (the staged form's host memcpy reads and writes every row once
// more in host memory, which is what kept the DMA engines waiting).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

#include "hostcopy.h"
#include "wnw_common.h"

namespace {

constexpr int kMaxGroups = 64;
// copy streams of the direct form: the spans' copies are dealt over them in
// turn.  On MI355X, 130 copies of ~1.2 MB from pinned rows ran at 39.8 GB/s
// on one stream, 51.5 on two, 55.2 on four and 52.8 on eight.  Four made a
// cfg4 step only ~1.5 % faster (3.34 against 3.38-3.40 ms) and moved the
// compute stream's own small copies onto new DMA engines during the first
// steps (7-10 ms set-ups that no warm-up of these streams removed): two.
constexpr int kCopyStreams = 2;

struct Job {
  const char* host_k = nullptr;
  const char* host_v = nullptr;
  char* stg_k = nullptr;
  char* stg_v = nullptr;
  char* dev_k = nullptr;
  char* dev_v = nullptr;
  std::vector<int32_t> ranges;        // [n, 2] host rows, in staging order
  std::vector<int64_t> dst;           // [n + 1] staging / device row of each range
  std::vector<int64_t> group_ranges;  // [groups + 1] range index bounds
  int64_t row_bytes = 0;
  hipStream_t stream = nullptr;
  int device = 0;
  int parity = 0;
  // direct form: stg_k / stg_v are the device stage rows, and stage_of[r]
  // is range r's first stage row (the group's ranges in host order)
  bool direct = false;
  std::vector<int64_t> stage_of;
  int64_t stage_rows = 0, dev_rows = 0;
};

// Direct form: per range (stage row, output row, rows), int64, read by
// stage_permute_kernel.
constexpr int kDescWords = 3;

// Rows of the device stage moved to their transfer-order rows: ranges
// r = blockIdx.x, blockIdx.x + gridDim.x, ..., tensor blockIdx.y (0: K,
// 1: V).  A range outside either array raises WNW_DEVERR_BOUNDS and is
// skipped.
__global__ __launch_bounds__(256) void stage_permute_kernel(const wnw::u32x4* stage_k, const wnw::u32x4* stage_v,
                                                            int64_t stage_rows, const int64_t* desc, int64_t n,
                                                            int64_t row_vec, wnw::u32x4* out_k, wnw::u32x4* out_v,
                                                            int64_t out_rows, int32_t* err) {
  using wnw::u32x4;
  const u32x4* src = blockIdx.y ? stage_v : stage_k;
  u32x4* dst = blockIdx.y ? out_v : out_k;
  const WNW_GLOBAL int64_t* dsc = wnw::gptr<int64_t>(desc);
  for (int64_t r = blockIdx.x; r < n; r += gridDim.x) {
    const int64_t s = dsc[kDescWords * r], d = dsc[kDescWords * r + 1], len = dsc[kDescWords * r + 2];
    if (s < 0 || d < 0 || len < 0 || s + len > stage_rows || d + len > out_rows) {
      if (threadIdx.x == 0) wnw::raise_device_error(err, WNW_DEVERR_BOUNDS);
      continue;
    }
    const u32x4* sp = src + s * row_vec;
    WNW_GLOBAL u32x4* dp = wnw::gptr_w<u32x4>(dst + d * row_vec);
    const int64_t nv = len * row_vec;
    constexpr int U = 4;  // 16-byte loads in flight per thread
    int64_t i = threadIdx.x;
    for (; i + (U - 1) * 256 < nv; i += U * 256) {
      u32x4 a[U];
#pragma unroll
      for (int u = 0; u < U; ++u) a[u] = __builtin_nontemporal_load(sp + i + u * 256);
#pragma unroll
      for (int u = 0; u < U; ++u) dp[i + u * 256] = a[u];
    }
    for (; i < nv; i += 256) dp[i] = __builtin_nontemporal_load(sp + i);
  }
}

}  // namespace

struct wnw_h2d {
  std::vector<std::thread> workers;
  std::thread lead;
  std::mutex mu;
  std::condition_variable cv_job, cv_task, cv_task_done, cv_issued;
  bool stop = false;
  // the current job: queued by start, walked by the lead thread
  bool job_pending = false, job_running = false;
  Job job;
  int issued = -1;     // groups of the current job whose copies are issued
  int groups = 0;
  int error = WNW_OK;  // first HIP error of the current job
  char error_msg[256] = "";  // its text (error strings are per thread: re-raised by wait / join)
  // the worker task of the lead thread: one group's ranges
  uint64_t task_seq = 0;
  int task_group = -1;
  int task_done = 0;
  hipEvent_t events[2][kMaxGroups] = {};
  // events recorded by the last job of each parity (0: none to wait for);
  // the last of them follows every copy that job issued
  int last_groups[2] = {0, 0};
  int parity = 0;
  int n_workers = 0;
  // direct form, per parity: a job's permute descriptors (pinned host copy
  // and device copy), grown by the lead thread once the parity's previous
  // job is done with them
  int64_t* desc_host[2] = {nullptr, nullptr};
  int64_t* desc_dev[2] = {nullptr, nullptr};
  int64_t desc_cap[2] = {0, 0};  // ranges each pair holds
  // direct form: the spans' K and V copies are dealt in turn over
  // kCopyStreams streams of their own (DMA engines; the device's set, shared
  // by all engines), so each hides the fixed cost of its copies behind the
  // others' transfers, and none waits behind a group's permute on the job's
  // stream; per parity the job-start event they all wait for and per group
  // the ends of their copies, which the job's stream waits for (created at
  // first use)
  hipStream_t aux[kCopyStreams] = {};
  int aux_device = -1;
  hipEvent_t ev_start[2] = {};
  hipEvent_t ev_copy[2][kMaxGroups][kCopyStreams] = {};
};

namespace {

// The direct form's copy streams, one set per device for the whole
// process, shared by every engine: HIP maps each new stream onto one of a
// few hardware queues in turn (GPU_MAX_HW_QUEUES, 4 by default), so streams
// made per engine (per cache) would in time land on the compute stream's
// queue, where copies and kernels wait for each other.
constexpr int kMaxDevices = 64;
std::mutex g_streams_mu;
hipStream_t g_copy[kMaxDevices][kCopyStreams] = {};

hipError_t shared_copy_streams(int dev, hipStream_t* out) {
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_streams_mu);
  hipError_t e = hipSuccess;
  for (int c = 0; c < kCopyStreams && e == hipSuccess; ++c)
    if (!g_copy[dev][c]) e = hipStreamCreateWithFlags(&g_copy[dev][c], hipStreamNonBlocking);  // default priority
  if (e == hipSuccess)
    for (int c = 0; c < kCopyStreams; ++c) out[c] = g_copy[dev][c];
  return e;
}

// The engine's copy streams on `dev` (set up once per device) and the copy
// events of its first n_groups groups (created once).
hipError_t direct_setup(wnw_h2d* x, int dev, int n_groups) {
  hipError_t e = hipSuccess;
  if (x->aux[0] == nullptr || x->aux_device != dev) {
    e = shared_copy_streams(dev, x->aux);
    if (e == hipSuccess) x->aux_device = dev;
  }
  for (int p = 0; p < 2 && e == hipSuccess; ++p)
    for (int g = 0; g < n_groups && e == hipSuccess; ++g)
      for (int c = 0; c < kCopyStreams && e == hipSuccess; ++c)
        if (!x->ev_copy[p][g][c]) e = hipEventCreateWithFlags(&x->ev_copy[p][g][c], hipEventDisableTiming);
  return e;
}

void copy_ranges(const Job& j, int64_t r0, int64_t r1) {
  for (int64_t r = r0; r < r1; ++r) {
    const int64_t s = j.ranges[2 * r], n = (int64_t)j.ranges[2 * r + 1] - s;
    const int64_t d = j.dst[r];
    wnw::stream_copy(j.stg_k + d * j.row_bytes, j.host_k + s * j.row_bytes, n * j.row_bytes);
    wnw::stream_copy(j.stg_v + d * j.row_bytes, j.host_v + s * j.row_bytes, n * j.row_bytes);
  }
  wnw::stream_fence();  // the streaming stores are visible before the copy engine reads the staging
}

// Worker w copies its share of the current task's group.
void worker_loop(wnw_h2d* x, int w) {
  uint64_t seen = 0;
  for (;;) {
    int g;
    {
      std::unique_lock<std::mutex> lk(x->mu);
      x->cv_task.wait(lk, [&] { return x->stop || x->task_seq != seen; });
      if (x->stop) return;
      seen = x->task_seq;
      g = x->task_group;
    }
    const Job& j = x->job;
    const int64_t a = j.group_ranges[g], b = j.group_ranges[g + 1];
    const int64_t n = b - a, W = x->n_workers;
    copy_ranges(j, a + n * w / W, a + n * (w + 1) / W);
    {
      std::lock_guard<std::mutex> lk(x->mu);
      if (++x->task_done == W) x->cv_task_done.notify_one();
    }
  }
}

// Records the first HIP error of the current job (its text is re-raised by
// wait / join) and marks group g issued.
void note_issued(wnw_h2d* x, hipError_t e, int g) {
  std::lock_guard<std::mutex> lk(x->mu);
  if (e != hipSuccess && x->error == WNW_OK) {
    snprintf(x->error_msg, sizeof(x->error_msg), "h2d: %s (%d)", hipGetErrorString(e), (int)e);
    x->error = WNW_EHIP;
  }
  x->issued = g;
  x->cv_issued.notify_all();
}

// The direct form of a job (lead thread, after the wait for the parity's
// previous job): per group the spans' DMA copies into the stage, the
// group's permute descriptors (one small copy), the permute kernel and the
// group's event.  Returns the number of groups whose event is recorded.
int run_direct(wnw_h2d* x, const Job& j, hipError_t e) {
  const int p = j.parity;
  const int64_t n = (int64_t)j.ranges.size() / 2;
  if (e == hipSuccess && n > x->desc_cap[p]) {  // the parity's previous job is done with these
    if (x->desc_host[p]) (void)hipHostFree(x->desc_host[p]);
    if (x->desc_dev[p]) (void)hipFree(x->desc_dev[p]);
    x->desc_host[p] = nullptr;
    x->desc_dev[p] = nullptr;
    x->desc_cap[p] = 0;
    const int64_t cap = std::max<int64_t>(n, 1024);
    e = hipHostMalloc((void**)&x->desc_host[p], (size_t)cap * kDescWords * 8, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMalloc((void**)&x->desc_dev[p], (size_t)cap * kDescWords * 8);
    if (e == hipSuccess) x->desc_cap[p] = cap;
  }
  if (e == hipSuccess) e = direct_setup(x, j.device, x->groups);
  // the copy streams follow everything queued on the job's stream before
  // this job (the previous job's permutes read the stage rows)
  if (e == hipSuccess) e = hipEventRecord(x->ev_start[p], j.stream);
  for (int c = 0; c < kCopyStreams && e == hipSuccess; ++c) e = hipStreamWaitEvent(x->aux[c], x->ev_start[p], 0);
  int recorded = 0;
  const int64_t rb = j.row_bytes;
  std::vector<int64_t> ord;
  int next = 0;  // the copy stream of the next copy (dealt in turn over the job)
  for (int g = 0; g < x->groups; ++g) {
    const int64_t a = j.group_ranges[g], b = j.group_ranges[g + 1];
    if (e == hipSuccess && b > a) {
      // the group's ranges in host order (their stage order), merged into
      // spans where they touch in host memory
      ord.resize(b - a);
      for (int64_t r = a; r < b; ++r) ord[r - a] = r;
      std::sort(ord.begin(), ord.end(), [&](int64_t u, int64_t v) { return j.stage_of[u] < j.stage_of[v]; });
      bool used[kCopyStreams] = {};
      for (size_t i = 0; i < ord.size() && e == hipSuccess;) {
        const int64_t r0 = ord[i];
        const int64_t h0 = j.ranges[2 * r0], st0 = j.stage_of[r0];
        int64_t h1 = j.ranges[2 * r0 + 1];
        size_t k = i + 1;
        while (k < ord.size() && j.ranges[2 * ord[k]] == h1) h1 = j.ranges[2 * ord[k++] + 1];
        if (h1 > h0) {
          const size_t bytes = (size_t)((h1 - h0) * rb);
          e = hipMemcpyAsync(j.stg_k + st0 * rb, j.host_k + h0 * rb, bytes, hipMemcpyHostToDevice, x->aux[next]);
          used[next] = true;
          next = (next + 1) % kCopyStreams;
          if (e == hipSuccess)
            e = hipMemcpyAsync(j.stg_v + st0 * rb, j.host_v + h0 * rb, bytes, hipMemcpyHostToDevice, x->aux[next]);
          used[next] = true;
          next = (next + 1) % kCopyStreams;
        }
        i = k;
      }
      // the end of the group's copies on each stream that took some (the
      // job's stream has waited for every earlier copy on the others)
      for (int c = 0; c < kCopyStreams && e == hipSuccess; ++c)
        if (used[c]) e = hipEventRecord(x->ev_copy[p][g][c], x->aux[c]);
      // the group's permute descriptors go up while its spans are in flight
      int64_t* dh = x->desc_host[p] + a * kDescWords;
      for (int64_t r = a; r < b; ++r) {
        dh[(r - a) * kDescWords] = j.stage_of[r];
        dh[(r - a) * kDescWords + 1] = j.dst[r];
        dh[(r - a) * kDescWords + 2] = (int64_t)j.ranges[2 * r + 1] - j.ranges[2 * r];
      }
      int64_t* dd = x->desc_dev[p] + a * kDescWords;
      if (e == hipSuccess)
        e = hipMemcpyAsync(dd, dh, (size_t)(b - a) * kDescWords * 8, hipMemcpyHostToDevice, j.stream);
      for (int c = 0; c < kCopyStreams && e == hipSuccess; ++c)
        if (used[c]) e = hipStreamWaitEvent(j.stream, x->ev_copy[p][g][c], 0);
      if (e == hipSuccess) {
        const unsigned grid = (unsigned)std::min<int64_t>(b - a, 1024);
        hipLaunchKernelGGL(stage_permute_kernel, dim3(grid, 2), dim3(256), 0, j.stream,
                           (const wnw::u32x4*)j.stg_k, (const wnw::u32x4*)j.stg_v, j.stage_rows, dd, b - a,
                           rb / 16, (wnw::u32x4*)j.dev_k, (wnw::u32x4*)j.dev_v, j.dev_rows,
                           wnw::device_error_word());
        e = hipGetLastError();
      }
    }
    if (e == hipSuccess) e = hipEventRecord(x->events[p][g], j.stream);
    if (e == hipSuccess) recorded = g + 1;
    note_issued(x, e, g);
  }
  return recorded;
}

void lead_loop(wnw_h2d* x) {
  for (;;) {
    {
      std::unique_lock<std::mutex> lk(x->mu);
      x->cv_job.wait(lk, [&] { return x->stop || x->job_pending; });
      if (x->stop) return;
      x->job_pending = false;
      x->job_running = true;
    }
    const Job& j = x->job;
    hipError_t e = hipSetDevice(j.device);
    // the staging pair and events of this parity were last used two jobs
    // ago: its copies must be done before the gather overwrites the staging
    // (the events record in stream order, so the last one covers them all)
    if (e == hipSuccess && x->last_groups[j.parity] > 0)
      e = hipEventSynchronize(x->events[j.parity][x->last_groups[j.parity] - 1]);
    int recorded = 0;
    if (j.direct) recorded = run_direct(x, j, e);
    for (int g = 0; g < x->groups && !j.direct; ++g) {
      if (e == hipSuccess) {  // after an error the staging is left alone (copies may still read it)
        std::unique_lock<std::mutex> lk(x->mu);
        x->task_group = g;
        x->task_done = 0;
        ++x->task_seq;
        x->cv_task.notify_all();
        x->cv_task_done.wait(lk, [&] { return x->task_done == x->n_workers; });
      }
      const int64_t d0 = j.dst[j.group_ranges[g]], d1 = j.dst[j.group_ranges[g + 1]];
      const size_t bytes = (size_t)((d1 - d0) * j.row_bytes);
      if (e == hipSuccess && bytes > 0)
        e = hipMemcpyAsync(j.dev_k + d0 * j.row_bytes, j.stg_k + d0 * j.row_bytes, bytes, hipMemcpyHostToDevice,
                           j.stream);
      if (e == hipSuccess && bytes > 0)
        e = hipMemcpyAsync(j.dev_v + d0 * j.row_bytes, j.stg_v + d0 * j.row_bytes, bytes, hipMemcpyHostToDevice,
                           j.stream);
      if (e == hipSuccess) e = hipEventRecord(x->events[j.parity][g], j.stream);
      if (e == hipSuccess) recorded = g + 1;
      {
        std::lock_guard<std::mutex> lk(x->mu);
        if (e != hipSuccess && x->error == WNW_OK) {
          snprintf(x->error_msg, sizeof(x->error_msg), "h2d: %s (%d)", hipGetErrorString(e), (int)e);
          x->error = WNW_EHIP;
        }
        x->issued = g;
        x->cv_issued.notify_all();
      }
    }
    // after an error some copy may have no event after it: drain the stream,
    // so the next job of this parity has nothing to wait for
    if (recorded < x->groups) {
      (void)hipStreamSynchronize(j.stream);
      for (int c = 0; c < kCopyStreams; ++c)
        if (x->aux[c]) (void)hipStreamSynchronize(x->aux[c]);
      recorded = 0;
    }
    {
      std::lock_guard<std::mutex> lk(x->mu);
      x->last_groups[j.parity] = recorded;
      x->job_running = false;
      x->cv_issued.notify_all();
    }
  }
}

// Blocks until the previous job is fully issued.
void join_locked(wnw_h2d* x, std::unique_lock<std::mutex>& lk) {
  x->cv_issued.wait(lk, [&] { return !x->job_pending && !x->job_running; });
}

}  // namespace

extern "C" wnw_h2d* wnw_h2d_create(int n_workers) {
  if (n_workers < 1 || n_workers > 64) {
    wnw::set_error("h2d: n_workers must be in [1, 64], got %d", n_workers);
    return nullptr;
  }
  wnw_h2d* x = new wnw_h2d();
  for (int p = 0; p < 2; ++p)
    for (int g = 0; g < kMaxGroups; ++g) {
      if (hipEventCreateWithFlags(&x->events[p][g], hipEventDisableTiming) != hipSuccess) {
        wnw::set_error("h2d: event creation failed");
        for (int q = 0; q <= p; ++q)
          for (int h = 0; h < kMaxGroups; ++h)
            if (x->events[q][h]) (void)hipEventDestroy(x->events[q][h]);
        delete x;
        return nullptr;
      }
    }
  bool ok = true;
  for (int p = 0; p < 2; ++p)
    ok = ok && hipEventCreateWithFlags(&x->ev_start[p], hipEventDisableTiming) == hipSuccess;
  if (!ok) {
    wnw::set_error("h2d: event creation failed");
    for (int p = 0; p < 2; ++p) {
      if (x->ev_start[p]) (void)hipEventDestroy(x->ev_start[p]);
      for (int g = 0; g < kMaxGroups; ++g)
        if (x->events[p][g]) (void)hipEventDestroy(x->events[p][g]);
    }
    delete x;
    return nullptr;
  }
  x->n_workers = n_workers;
  for (int w = 0; w < n_workers; ++w) x->workers.emplace_back(worker_loop, x, w);
  x->lead = std::thread(lead_loop, x);
  return x;
}

extern "C" void wnw_h2d_destroy(wnw_h2d* x) {
  if (!x) return;
  {
    std::unique_lock<std::mutex> lk(x->mu);
    join_locked(x, lk);
    x->stop = true;
  }
  x->cv_job.notify_all();
  x->cv_task.notify_all();
  x->lead.join();
  for (auto& t : x->workers) t.join();
  // the caller may free the staging once this returns: the issued copies
  // that read it end first
  for (int p = 0; p < 2; ++p)
    if (x->last_groups[p] > 0) (void)hipEventSynchronize(x->events[p][x->last_groups[p] - 1]);
  for (int p = 0; p < 2; ++p)
    for (int g = 0; g < kMaxGroups; ++g) (void)hipEventDestroy(x->events[p][g]);
  // (the copy streams are the device's, shared: this engine's copies on them
  // end before its last events, waited for above)
  for (int p = 0; p < 2; ++p) {
    if (x->desc_host[p]) (void)hipHostFree(x->desc_host[p]);
    if (x->desc_dev[p]) (void)hipFree(x->desc_dev[p]);
    (void)hipEventDestroy(x->ev_start[p]);
    for (int g = 0; g < kMaxGroups; ++g)
      for (int c = 0; c < kCopyStreams; ++c)
        if (x->ev_copy[p][g][c]) (void)hipEventDestroy(x->ev_copy[p][g][c]);
  }
  delete x;
}

namespace {

// Checks the arguments of a start and fills the job's ranges, rows and
// pointers (both forms).
int make_job(Job& j, const void* host_k, const void* host_v, int64_t host_rows, const int32_t* ranges,
             int64_t n_ranges, const int64_t* group_ranges, int n_groups, void* stg_k, void* stg_v, int64_t stg_rows,
             void* dev_k, void* dev_v, int64_t dev_rows, int64_t row_bytes, void* stream) {
  WNW_CHECK_ARG(n_groups >= 1 && n_groups <= kMaxGroups, "h2d: n_groups must be in [1, %d]", kMaxGroups);
  WNW_CHECK_ARG(n_ranges >= 0 && row_bytes > 0, "h2d: bad sizes");
  WNW_CHECK_ARG(group_ranges && group_ranges[0] == 0 && group_ranges[n_groups] == n_ranges,
                "h2d: group bounds must run from 0 to n_ranges");
  for (int g = 0; g < n_groups; ++g)
    WNW_CHECK_ARG(group_ranges[g] <= group_ranges[g + 1], "h2d: group bounds decrease");
  WNW_CHECK_ARG(n_ranges == 0 || (ranges && host_k && host_v && stg_k && stg_v && dev_k && dev_v),
                "h2d: null pointer argument");
  j.ranges.assign(ranges, ranges + 2 * n_ranges);
  j.dst.resize(n_ranges + 1);
  j.dst[0] = 0;
  for (int64_t r = 0; r < n_ranges; ++r) {
    const int64_t s = j.ranges[2 * r], e = j.ranges[2 * r + 1];
    WNW_CHECK_ARG(s >= 0 && e >= s && e <= host_rows, "h2d: range %lld = [%lld, %lld) outside %lld host rows",
                  (long long)r, (long long)s, (long long)e, (long long)host_rows);
    j.dst[r + 1] = j.dst[r] + (e - s);
  }
  WNW_CHECK_ARG(j.dst[n_ranges] <= stg_rows && j.dst[n_ranges] <= dev_rows,
                "h2d: %lld rows do not fit staging (%lld) and device (%lld) buffers", (long long)j.dst[n_ranges],
                (long long)stg_rows, (long long)dev_rows);
  j.group_ranges.assign(group_ranges, group_ranges + n_groups + 1);
  j.host_k = (const char*)host_k;
  j.host_v = (const char*)host_v;
  j.stg_k = (char*)stg_k;
  j.stg_v = (char*)stg_v;
  j.dev_k = (char*)dev_k;
  j.dev_v = (char*)dev_v;
  j.row_bytes = row_bytes;
  j.stage_rows = stg_rows;
  j.dev_rows = dev_rows;
  j.stream = (hipStream_t)stream;
  WNW_CHECK_HIP(hipGetDevice(&j.device), "h2d: hipGetDevice");
  return WNW_OK;
}

// Direct form: the stage rows of each range -- each group's rows [dst[a],
// dst[b]) hold its ranges in host order, so that ranges touching in host
// memory are one span.
void set_stage_rows(Job& j, int n_groups) {
  const int64_t n_ranges = (int64_t)j.ranges.size() / 2;
  j.direct = true;
  j.stage_of.assign(n_ranges, 0);
  std::vector<int64_t> ord;
  for (int g = 0; g < n_groups; ++g) {
    const int64_t a = j.group_ranges[g], b = j.group_ranges[g + 1];
    ord.resize(b - a);
    for (int64_t r = a; r < b; ++r) ord[r - a] = r;
    std::stable_sort(ord.begin(), ord.end(),
                     [&](int64_t u, int64_t v) { return j.ranges[2 * u] < j.ranges[2 * v]; });
    int64_t at = j.dst[a];
    for (int64_t r : ord) {
      j.stage_of[r] = at;
      at += (int64_t)j.ranges[2 * r + 1] - j.ranges[2 * r];
    }
  }
}

// Hands a job to the lead thread (after the previous job is fully issued).
void submit(wnw_h2d* x, Job&& j, int n_groups) {
  {
    std::unique_lock<std::mutex> lk(x->mu);
    join_locked(x, lk);  // the previous job's groups are issued; its events stay valid (other parity)
    x->parity ^= 1;
    j.parity = x->parity;
    x->job = std::move(j);
    x->groups = n_groups;
    x->issued = -1;
    x->error = WNW_OK;
    x->error_msg[0] = 0;
    x->job_pending = true;
  }
  x->cv_job.notify_all();
}

}  // namespace

extern "C" int wnw_h2d_start(wnw_h2d* x, const void* host_k, const void* host_v, int64_t host_rows,
                             const int32_t* ranges, int64_t n_ranges, const int64_t* group_ranges, int n_groups,
                             void* stg_k, void* stg_v, int64_t stg_rows, void* dev_k, void* dev_v, int64_t dev_rows,
                             int64_t row_bytes, void* stream) {
  WNW_CHECK_ARG(x, "h2d: null engine");
  Job j;
  const int rc = make_job(j, host_k, host_v, host_rows, ranges, n_ranges, group_ranges, n_groups, stg_k, stg_v,
                          stg_rows, dev_k, dev_v, dev_rows, row_bytes, stream);
  if (rc != WNW_OK) return rc;
  submit(x, std::move(j), n_groups);
  return WNW_OK;
}

extern "C" int wnw_h2d_start_direct(wnw_h2d* x, const void* host_k, const void* host_v, int64_t host_rows,
                                    const int32_t* ranges, int64_t n_ranges, const int64_t* group_ranges,
                                    int n_groups, void* stage_k, void* stage_v, int64_t stage_rows, void* dev_k,
                                    void* dev_v, int64_t dev_rows, int64_t row_bytes, void* stream) {
  WNW_CHECK_ARG(x, "h2d: null engine");
  WNW_CHECK_ARG(row_bytes % 16 == 0, "h2d: row_bytes must be a multiple of 16");
  Job j;
  const int rc = make_job(j, host_k, host_v, host_rows, ranges, n_ranges, group_ranges, n_groups, stage_k,
                          stage_v, stage_rows, dev_k, dev_v, dev_rows, row_bytes, stream);
  if (rc != WNW_OK) return rc;
  WNW_CHECK_ARG(n_ranges == 0 || (((uintptr_t)stage_k | (uintptr_t)stage_v | (uintptr_t)dev_k | (uintptr_t)dev_v) &
                                  15) == 0,
                "h2d: stage and device rows must be 16-byte aligned");
  set_stage_rows(j, n_groups);
  submit(x, std::move(j), n_groups);
  return WNW_OK;
}

extern "C" int wnw_h2d_plan_start_direct(wnw_h2d* x, wnw_planner* p, const int32_t* topk, int64_t batch, int64_t k,
                                         int32_t* load_starts_2d, int32_t* load_lens_2d, int32_t* cu_new_2d,
                                         int32_t* new_lens_2d, int32_t* evict_offsets_2d, int32_t* evict_max,
                                         int32_t* evict_layer_ptr, const int32_t* layer_cuts, int n_groups,
                                         const void* host_k, const void* host_v, int64_t host_rows, void* stage_k,
                                         void* stage_v, int64_t stage_rows, void* dev_k, void* dev_v,
                                         int64_t dev_rows, int64_t row_bytes, void* stream, int32_t* any_change,
                                         int64_t* total_rows, int64_t* n_evict, int64_t* n_ranges,
                                         int32_t* started) {
  WNW_CHECK_ARG(x && p && started && layer_cuts, "h2d: null argument");
  WNW_CHECK_ARG(batch >= 0 && k >= 0 && (batch * k == 0 || topk), "h2d: bad top-k choice");
  WNW_CHECK_ARG(n_groups >= 1 && n_groups <= kMaxGroups && layer_cuts[0] == 0,
                "h2d: n_groups must be in [1, %d] with layer cuts from 0", kMaxGroups);
  WNW_CHECK_ARG(row_bytes > 0 && row_bytes % 16 == 0, "h2d: row_bytes must be a positive multiple of 16");
  int pl_layers = 0, pl_batch = 0;
  wnw::planner_dims(p, &pl_layers, &pl_batch);
  WNW_CHECK_ARG(batch == pl_batch && layer_cuts[n_groups] == pl_layers,
                "h2d: the choice covers %lld samples and the cuts %d layers; the planner has %d and %d",
                (long long)batch, layer_cuts[n_groups], pl_batch, pl_layers);
  *started = 0;
  // the choice as the planner's CSR (-1: no chunk)
  std::vector<int32_t> flat, off(batch + 1, 0);
  flat.reserve((size_t)(batch * k));
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t c = 0; c < k; ++c)
      if (topk[b * k + c] >= 0) flat.push_back(topk[b * k + c]);
    off[b + 1] = (int32_t)flat.size();
  }
  const int rc = wnw_planner_compute_and_prepare(p, flat.data(), off.data(), load_starts_2d, load_lens_2d, cu_new_2d,
                                                 new_lens_2d, evict_offsets_2d, evict_max, evict_layer_ptr,
                                                 any_change, total_rows, n_evict, n_ranges);
  if (rc != WNW_OK) return rc;
  // nothing to load, or more rows than the caller's buffers: the caller
  // takes it from here
  if (!*any_change || *total_rows == 0 || *total_rows > stage_rows || *total_rows > dev_rows) return WNW_OK;
  const int L = layer_cuts[n_groups];
  for (int g = 0; g < n_groups; ++g)
    WNW_CHECK_ARG(layer_cuts[g] <= layer_cuts[g + 1], "h2d: layer cuts decrease");
  std::vector<int32_t> lp(L + 1);
  int rc2 = wnw_planner_get_range_layers(p, lp.data(), L + 1);
  if (rc2 != WNW_OK) return rc2;
  WNW_CHECK_ARG(lp[L] == *n_ranges, "h2d: the layer cuts end at layer %d, not the planner's last", L);
  std::vector<int64_t> gr(n_groups + 1);
  for (int g = 0; g <= n_groups; ++g) gr[g] = lp[layer_cuts[g]];
  std::vector<int32_t> rg((size_t)(2 * *n_ranges));
  rc2 = wnw_planner_get_ranges(p, rg.data(), *n_ranges);
  if (rc2 != WNW_OK) return rc2;
  Job j;
  rc2 = make_job(j, host_k, host_v, host_rows, rg.data(), *n_ranges, gr.data(), n_groups, stage_k, stage_v,
                 stage_rows, dev_k, dev_v, dev_rows, row_bytes, stream);
  if (rc2 != WNW_OK) return rc2;
  WNW_CHECK_ARG((((uintptr_t)stage_k | (uintptr_t)stage_v | (uintptr_t)dev_k | (uintptr_t)dev_v) & 15) == 0,
                "h2d: stage and device rows must be 16-byte aligned");
  set_stage_rows(j, n_groups);
  submit(x, std::move(j), n_groups);
  *started = 1;
  return WNW_OK;
}

extern "C" int wnw_h2d_wait(wnw_h2d* x, int group, void* stream) {
  WNW_CHECK_ARG(x, "h2d: null engine");
  hipEvent_t ev;
  {
    std::unique_lock<std::mutex> lk(x->mu);
    WNW_CHECK_ARG(group >= 0 && group < x->groups, "h2d: group %d outside [0, %d)", group, x->groups);
    x->cv_issued.wait(lk, [&] { return x->issued >= group || (!x->job_pending && !x->job_running); });
    if (x->error != WNW_OK) {
      wnw::set_error("%s", x->error_msg);
      return x->error;
    }
    if (x->issued < group) {
      wnw::set_error("h2d: group %d was never issued", group);
      return WNW_EINVAL;
    }
    ev = x->events[x->job.parity][group];
  }
  WNW_CHECK_HIP(hipStreamWaitEvent((hipStream_t)stream, ev, 0), "h2d: hipStreamWaitEvent");
  return WNW_OK;
}

extern "C" int wnw_h2d_reserve(wnw_h2d* x, int64_t n_ranges, int n_groups, void* stream) {
  using namespace wnw;
  WNW_CHECK_ARG(x, "h2d: null engine");
  WNW_CHECK_ARG(n_ranges >= 0 && n_ranges <= (int64_t)1 << 24, "h2d: n_ranges must be in [0, 2^24]");
  WNW_CHECK_ARG(n_groups >= 1 && n_groups <= kMaxGroups, "h2d: n_groups must be in [1, %d]", kMaxGroups);
  int dev = 0;
  WNW_CHECK_HIP(hipGetDevice(&dev), "h2d: hipGetDevice");
  {
    std::unique_lock<std::mutex> lk(x->mu);
    join_locked(x, lk);  // the lead thread is idle: its streams and buffers are ours until the next start
    hipError_t e = hipSuccess;
    e = direct_setup(x, dev, n_groups);
    for (int p = 0; p < 2 && e == hipSuccess; ++p) {
      if (n_ranges <= x->desc_cap[p] && x->desc_host[p]) continue;
      // the parity's last copies may still read its descriptors
      if (x->last_groups[p] > 0) e = hipEventSynchronize(x->events[p][x->last_groups[p] - 1]);
      if (e != hipSuccess) break;
      if (x->desc_host[p]) (void)hipHostFree(x->desc_host[p]);
      if (x->desc_dev[p]) (void)hipFree(x->desc_dev[p]);
      x->desc_host[p] = nullptr;
      x->desc_dev[p] = nullptr;
      x->desc_cap[p] = 0;
      const int64_t cap = std::max<int64_t>(n_ranges, 1024);
      e = hipHostMalloc((void**)&x->desc_host[p], (size_t)cap * kDescWords * 8, hipHostMallocDefault);
      if (e == hipSuccess) e = hipMalloc((void**)&x->desc_dev[p], (size_t)cap * kDescWords * 8);
      if (e == hipSuccess) x->desc_cap[p] = cap;
    }
    // The copy engines: the runtime puts a stream's copy on another DMA
    // engine when the one it used last is busy, and sets up an engine's
    // queue the first time a copy lands on it (6-11 ms on MI355X, every copy
    // submission of the process held meanwhile; the first job of each
    // staging parity met one otherwise).  Spans issued in turn on the copy
    // streams while the job's stream copies too, as in a job, twice, so that
    // the engines a job's copies land on are set up here.  (Repeating rounds
    // of mixed span sizes until no submission took over 1 ms left the
    // streams on engines that ran cfg4 steps ~0.08 ms slower.)
    const hipStream_t js = (hipStream_t)stream;
    {
      constexpr size_t kSpan = 512u << 10;
      constexpr int kCopies = 48;
      const size_t total = (kCopies + 4) * kSpan;
      char* hb = nullptr;
      char* db = nullptr;
      if (e == hipSuccess) e = hipHostMalloc((void**)&hb, total, hipHostMallocDefault);
      if (e == hipSuccess) e = hipMalloc((void**)&db, total);
      if (e == hipSuccess) memset(hb, 0, total);
      for (int round = 0; round < 2 && e == hipSuccess; ++round) {
        for (int i = 0; i < kCopies && e == hipSuccess; ++i) {
          const size_t o = (size_t)i * kSpan;
          e = hipMemcpyAsync(db + o, hb + o, kSpan, hipMemcpyHostToDevice, x->aux[i % kCopyStreams]);
          if (e == hipSuccess && i % 16 == 9) {
            const size_t q = (size_t)(kCopies + i / 16) * kSpan;
            e = hipMemcpyAsync(db + q, hb + q, kSpan, hipMemcpyHostToDevice, js);
          }
        }
        for (int c = 0; c < kCopyStreams && e == hipSuccess; ++c) e = hipStreamSynchronize(x->aux[c]);
        if (e == hipSuccess) e = hipStreamSynchronize(js);
      }
      if (db) (void)hipFree(db);
      if (hb) (void)hipHostFree(hb);
    }
    // every event of the first n_groups groups recorded once, on the stream
    // a job records it on
    for (int p = 0; p < 2 && e == hipSuccess; ++p) {
      e = hipEventRecord(x->ev_start[p], js);
      for (int g = 0; g < n_groups && e == hipSuccess; ++g) {
        for (int c = 0; c < kCopyStreams && e == hipSuccess; ++c) e = hipEventRecord(x->ev_copy[p][g][c], x->aux[c]);
        if (e == hipSuccess) e = hipEventRecord(x->events[p][g], js);
      }
    }
    for (int c = 0; c < kCopyStreams && e == hipSuccess; ++c) e = hipStreamSynchronize(x->aux[c]);
    if (e == hipSuccess) e = hipStreamSynchronize(js);
    WNW_CHECK_HIP(e, "h2d reserve");
  }
  // an empty job through the lead thread (its device, events and the job's
  // stream set up once)
  Job j;
  const int64_t bounds[2] = {0, 0};
  const int rc = make_job(j, nullptr, nullptr, 0, nullptr, 0, bounds, 1, nullptr, nullptr, 0, nullptr, nullptr, 0, 16,
                          stream);
  if (rc != WNW_OK) return rc;
  j.direct = true;
  submit(x, std::move(j), 1);
  return wnw_h2d_join(x);
}

extern "C" int wnw_h2d_join(wnw_h2d* x) {
  WNW_CHECK_ARG(x, "h2d: null engine");
  std::unique_lock<std::mutex> lk(x->mu);
  join_locked(x, lk);
  if (x->error != WNW_OK) wnw::set_error("%s", x->error_msg);
  return x->error;
}

namespace wnw {
void touch_transfer_kernels() {
  hipFuncAttributes a;
  (void)hipFuncGetAttributes(&a, (const void*)&::stage_permute_kernel);
}
}  // namespace wnw

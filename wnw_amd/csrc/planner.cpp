// Host planner of the WnW decode cache (C ABI, no GPU code).
//
// Same plan as the reference's C++ planner (src/algorithms/wnw_cpp/code/
// planner.cpp:124-306) and its Python original (src/algorithms/wnw/code/
// cache.py:609-630 chunk changes, :756-889 rebuild plan), with the same
// iteration order, so the descriptor arrays it writes are bit-identical:
//   * chunk changes per sample from its top-k chunk list: needed segments,
//     to_load = needed - loaded, eviction after `eviction_lag` misses;
//   * per layer, per changed sample, per class-B KV head: sorted relative
//     evict ranges, shift of the surviving resident segments, loads appended
//     at rel_cursor = len - evicted, new_len = len - evicted + loaded + 1;
//   * host transfer ranges in (layer, sample, head, segment) order.
// It keeps its own copy of the segment lengths: a step without a plan is a
// plain append (+1 everywhere), applied at the next call, as the reference's
// `prev_changed_` rule does (planner.cpp:133-136).
//
// Unlike the reference, every index that comes from the caller is checked
// (chunk ids, segment ids, host row ranges, staging capacity).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <set>
#include <utility>
#include <vector>

#include "../../include/wnw_amd.h"

namespace wnw {
void set_error(const char* fmt, ...);
void planner_dims(const wnw_planner* p, int* layers, int* batch);
}

namespace {

struct Range {
  int32_t start, end;
};

struct SegMeta {  // one offloaded segment of one (layer, flat segment)
  int32_t cpu_s = -1, cpu_e = -1;  // host rows, -1 = none
  int32_t gpu_s = -1, gpu_e = -1;  // rows relative to the flat segment, -1 = not resident
};

}  // namespace

struct wnw_planner {
  int L, H, B, N;
  int top_k = 0, lag = 1;
  bool prev_changed = false;
  std::vector<int32_t> seg_count;                     // [B]
  std::vector<std::vector<std::vector<int32_t>>> c2s;  // [B][chunk] -> segments
  std::vector<std::vector<int32_t>> class_b;           // [L] -> KV heads
  std::vector<int64_t> meta_base;                      // [N + 1] offsets into one layer's metas
  std::vector<SegMeta> meta;                           // [L][flat][seg], flattened
  std::vector<std::set<int32_t>> loaded;               // [B]
  std::vector<std::vector<int32_t>> misses;            // [B][seg]
  std::vector<int32_t> seq_lens;                       // [L][N]
  // results of the last compute_and_prepare
  std::vector<int32_t> ev_starts, ev_ends;
  std::vector<Range> ranges;
  std::vector<int32_t> range_layer_ptr;  // [L + 1] first range of each layer
  // host restore rows and pinned staging (caller-owned)
  const char* cpu_k = nullptr;
  const char* cpu_v = nullptr;
  char* stg_k = nullptr;
  char* stg_v = nullptr;
  int64_t cpu_rows = 0, stg_rows = 0, row_bytes = 0;

  SegMeta* metas(int l, int f) { return meta.data() + (int64_t)l * meta_base[N] + meta_base[f]; }
};

#define P_CHECK(cond, ...)          \
  do {                              \
    if (!(cond)) {                  \
      wnw::set_error(__VA_ARGS__);  \
      return WNW_EINVAL;            \
    }                               \
  } while (0)

extern "C" wnw_planner* wnw_planner_create(int num_layers, int num_kv_heads, int batch_size, int group) {
  (void)group;  // kept for signature parity with the reference constructor
  if (num_layers <= 0 || num_kv_heads <= 0 || batch_size <= 0) {
    wnw::set_error("planner: non-positive dimensions");
    return nullptr;
  }
  wnw_planner* p = new wnw_planner();
  p->L = num_layers;
  p->H = num_kv_heads;
  p->B = batch_size;
  p->N = batch_size * num_kv_heads;
  p->seg_count.assign(batch_size, 0);
  p->c2s.resize(batch_size);
  p->class_b.resize(num_layers);
  p->loaded.resize(batch_size);
  p->misses.resize(batch_size);
  p->seq_lens.assign((size_t)num_layers * p->N, 0);
  p->meta_base.assign(p->N + 1, 0);
  return p;
}

extern "C" void wnw_planner_destroy(wnw_planner* p) { delete p; }

extern "C" int wnw_planner_set_config(wnw_planner* p, int top_k_chunks, int eviction_lag) {
  P_CHECK(p, "planner: null handle");
  P_CHECK(top_k_chunks >= 0, "planner: negative top_k_chunks");
  p->top_k = top_k_chunks;
  p->lag = eviction_lag;
  return WNW_OK;
}

extern "C" int wnw_planner_set_seg_count(wnw_planner* p, const int32_t* seg_count, int64_t n) {
  P_CHECK(p && (seg_count || n == 0), "planner: null argument");
  P_CHECK(n == p->B, "planner: seg_count has %lld entries, batch is %d", (long long)n, p->B);
  for (int b = 0; b < p->B; ++b) P_CHECK(seg_count[b] >= 0, "planner: negative segment count");
  p->seg_count.assign(seg_count, seg_count + n);
  for (int f = 0; f < p->N; ++f) p->meta_base[f + 1] = p->meta_base[f] + p->seg_count[f / p->H];
  p->meta.assign((size_t)p->L * p->meta_base[p->N], SegMeta());
  for (int b = 0; b < p->B; ++b) p->misses[b].assign(p->seg_count[b], 0);
  return WNW_OK;
}

extern "C" int wnw_planner_set_chunk_to_segs(wnw_planner* p, int b, const int32_t* flat_segs,
                                             const int32_t* offsets, int64_t num_chunks) {
  P_CHECK(p && offsets, "planner: null argument");
  P_CHECK(b >= 0 && b < p->B, "planner: sample %d out of range", b);
  P_CHECK(num_chunks >= 0 && offsets[0] == 0, "planner: bad chunk offsets");
  std::vector<std::vector<int32_t>> c(num_chunks);
  for (int64_t i = 0; i < num_chunks; ++i) {
    P_CHECK(offsets[i + 1] >= offsets[i], "planner: chunk offsets decrease");
    for (int32_t j = offsets[i]; j < offsets[i + 1]; ++j) {
      P_CHECK(flat_segs && flat_segs[j] >= 0 && flat_segs[j] < p->seg_count[b],
              "planner: chunk %lld of sample %d names segment %d (count %d)", (long long)i, b,
              flat_segs ? flat_segs[j] : -1, p->seg_count[b]);
      c[i].push_back(flat_segs[j]);
    }
  }
  p->c2s[b] = std::move(c);
  return WNW_OK;
}

extern "C" int wnw_planner_set_class_b(wnw_planner* p, int layer, const int32_t* kv_heads, int64_t n) {
  P_CHECK(p && (kv_heads || n == 0), "planner: null argument");
  P_CHECK(layer >= 0 && layer < p->L, "planner: layer %d out of range", layer);
  for (int64_t i = 0; i < n; ++i)
    P_CHECK(kv_heads[i] >= 0 && kv_heads[i] < p->H, "planner: KV head %d out of range", kv_heads[i]);
  p->class_b[layer].assign(kv_heads, kv_heads + n);
  return WNW_OK;
}

// Flattened in (layer, flat segment, segment) order; -1 marks "no metadata".
extern "C" int wnw_planner_set_restore_meta(wnw_planner* p, const int32_t* cpu_s, const int32_t* cpu_e,
                                            const int32_t* gpu_s, const int32_t* gpu_e, int64_t n) {
  P_CHECK(p, "planner: null handle");
  const int64_t want = (int64_t)p->L * p->meta_base[p->N];
  P_CHECK(n == want, "planner: restore meta has %lld entries, expected %lld", (long long)n, (long long)want);
  P_CHECK(n == 0 || (cpu_s && cpu_e && gpu_s && gpu_e), "planner: null argument");
  for (int64_t i = 0; i < n; ++i) {
    SegMeta& m = p->meta[i];
    m.cpu_s = cpu_s[i];
    m.cpu_e = cpu_e[i];
    m.gpu_s = gpu_s[i];
    m.gpu_e = gpu_e[i];
    P_CHECK(m.cpu_s < 0 || m.cpu_e >= m.cpu_s, "planner: host range %lld decreasing", (long long)i);
  }
  return WNW_OK;
}

extern "C" int wnw_planner_set_loaded(wnw_planner* p, int b, const int32_t* segs, int64_t n) {
  P_CHECK(p && (segs || n == 0), "planner: null argument");
  P_CHECK(b >= 0 && b < p->B, "planner: sample %d out of range", b);
  std::set<int32_t> s;
  for (int64_t i = 0; i < n; ++i) {
    P_CHECK(segs[i] >= 0 && segs[i] < p->seg_count[b], "planner: segment %d out of range", segs[i]);
    s.insert(segs[i]);
  }
  p->loaded[b] = std::move(s);
  return WNW_OK;
}

// Flattened [L][N]; also resets the miss counters and the append rule.
extern "C" int wnw_planner_set_seq_lens(wnw_planner* p, const int32_t* lens, int64_t n) {
  P_CHECK(p && (lens || n == 0), "planner: null argument");
  P_CHECK(n == (int64_t)p->L * p->N, "planner: seq_lens has %lld entries, expected %lld", (long long)n,
          (long long)p->L * p->N);
  p->seq_lens.assign(lens, lens + n);
  for (int b = 0; b < p->B; ++b) p->misses[b].assign(p->seg_count[b], 0);
  p->prev_changed = false;
  return WNW_OK;
}

extern "C" int64_t wnw_planner_get_loaded_segments(wnw_planner* p, int b, int32_t* out, int64_t cap) {
  if (!p || b < 0 || b >= p->B) {
    wnw::set_error("planner: bad handle or sample");
    return -1;
  }
  const int64_t n = (int64_t)p->loaded[b].size();
  if (out) {
    int64_t i = 0;
    for (int32_t s : p->loaded[b]) {
      if (i >= cap) break;
      out[i++] = s;
    }
  }
  return n;
}

extern "C" int wnw_planner_set_restore_buffers(wnw_planner* p, const void* cpu_k, const void* cpu_v, void* stg_k,
                                               void* stg_v, int64_t cpu_rows, int64_t stg_rows, int64_t row_bytes) {
  P_CHECK(p, "planner: null handle");
  P_CHECK(cpu_rows >= 0 && stg_rows >= 0 && row_bytes > 0, "planner: bad buffer sizes");
  P_CHECK((cpu_k && cpu_v) || cpu_rows == 0, "planner: null host rows");
  P_CHECK((stg_k && stg_v) || stg_rows == 0, "planner: null staging");
  p->cpu_k = (const char*)cpu_k;
  p->cpu_v = (const char*)cpu_v;
  p->stg_k = (char*)stg_k;
  p->stg_v = (char*)stg_v;
  p->cpu_rows = cpu_rows;
  p->stg_rows = stg_rows;
  p->row_bytes = row_bytes;
  return WNW_OK;
}

// Copies the host rows of the last plan's transfer ranges, in order, to the
// start of the staging buffers (reference planner.cpp:113-122).
extern "C" int wnw_planner_gather_restore(wnw_planner* p) {
  P_CHECK(p, "planner: null handle");
  int64_t dst = 0;
  for (const Range& r : p->ranges) {
    const int64_t n = (int64_t)r.end - r.start;
    P_CHECK(r.start >= 0 && r.end <= p->cpu_rows, "planner: host range [%d, %d) outside %lld rows", r.start,
            r.end, (long long)p->cpu_rows);
    P_CHECK(dst + n <= p->stg_rows, "planner: staging holds %lld rows, plan needs more", (long long)p->stg_rows);
    memcpy(p->stg_k + dst * p->row_bytes, p->cpu_k + (int64_t)r.start * p->row_bytes, n * p->row_bytes);
    memcpy(p->stg_v + dst * p->row_bytes, p->cpu_v + (int64_t)r.start * p->row_bytes, n * p->row_bytes);
    dst += n;
  }
  return WNW_OK;
}

extern "C" int wnw_planner_compute_and_prepare(wnw_planner* p, const int32_t* topk_idx, const int32_t* topk_off,
                                               int32_t* load_starts_2d, int32_t* load_lens_2d, int32_t* cu_new_2d,
                                               int32_t* new_lens_2d, int32_t* evict_offsets_2d, int32_t* evict_max,
                                               int32_t* evict_layer_ptr, int32_t* any_change, int64_t* total_rows,
                                               int64_t* n_evict, int64_t* n_ranges) {
  P_CHECK(p && topk_off && load_starts_2d && load_lens_2d && cu_new_2d && new_lens_2d && evict_offsets_2d &&
              evict_max && evict_layer_ptr && any_change && total_rows && n_evict && n_ranges,
          "planner: null argument");
  const int L = p->L, H = p->H, B = p->B, N = p->N;
  // validate the top-k lists before touching any state
  P_CHECK(topk_off[0] == 0, "planner: topk_off[0] must be 0");
  for (int b = 0; b < B; ++b) {
    P_CHECK(topk_off[b + 1] >= topk_off[b], "planner: topk offsets decrease");
    for (int j = topk_off[b]; j < topk_off[b + 1]; ++j)
      P_CHECK(topk_idx && topk_idx[j] >= 0 && topk_idx[j] < (int32_t)p->c2s[b].size(),
              "planner: chunk %d of sample %d out of range", topk_idx ? topk_idx[j] : -1, b);
  }
  if (!p->prev_changed)  // the previous step was a plain append
    for (int32_t& x : p->seq_lens) x += 1;

  std::vector<std::set<int32_t>> to_load(B), to_evict(B);
  bool change = false;
  for (int b = 0; b < B; ++b) {
    if (topk_off[b + 1] == topk_off[b]) continue;
    std::set<int32_t> needed;
    for (int j = topk_off[b]; j < topk_off[b + 1]; ++j)
      for (int32_t s : p->c2s[b][topk_idx[j]]) needed.insert(s);
    std::set<int32_t>& ld = p->loaded[b];
    std::vector<int32_t>& miss = p->misses[b];
    for (int32_t s : needed)
      if (!ld.count(s)) to_load[b].insert(s);
    for (int32_t s : ld) {
      if (needed.count(s)) {
        miss[s] = 0;
      } else if (++miss[s] >= p->lag) {
        to_evict[b].insert(s);
      }
    }
    ld.insert(to_load[b].begin(), to_load[b].end());
    for (int32_t s : to_evict[b]) {
      ld.erase(s);
      miss[s] = 0;
    }
    change = change || !to_load[b].empty() || !to_evict[b].empty();
  }

  p->ev_starts.clear();
  p->ev_ends.clear();
  p->ranges.clear();
  p->range_layer_ptr.assign((size_t)L + 1, 0);
  *any_change = change ? 1 : 0;
  *total_rows = 0;
  *n_evict = 0;
  *n_ranges = 0;
  if (!change) {
    p->prev_changed = false;
    return WNW_OK;
  }

  // the sets as sorted vectors for the layer loop (same order)
  std::vector<std::vector<int32_t>> tl(B), te(B);
  for (int b = 0; b < B; ++b) {
    tl[b].assign(to_load[b].begin(), to_load[b].end());
    te[b].assign(to_evict[b].begin(), to_evict[b].end());
  }
  std::vector<int32_t> new_lens((size_t)L * N);
  int32_t transfer = 0;
  std::vector<std::pair<int32_t, int32_t>> ev;
  for (int l = 0; l < L; ++l) {
    int32_t* lens_l = p->seq_lens.data() + (size_t)l * N;
    int32_t* nl = new_lens.data() + (size_t)l * N;
    int32_t* ls = load_starts_2d + (size_t)l * N;
    int32_t* ll = load_lens_2d + (size_t)l * N;
    int32_t* eo = evict_offsets_2d + (size_t)l * (N + 1);
    p->range_layer_ptr[l] = (int32_t)p->ranges.size();
    for (int f = 0; f < N; ++f) {
      nl[f] = lens_l[f] + 1;
      ls[f] = -1;
      ll[f] = 0;
    }
    // the evict ranges of flat segment f are emitted in f order below
    std::vector<std::vector<std::pair<int32_t, int32_t>>> ev_f(N);
    for (int b = 0; b < B; ++b) {
      if (tl[b].empty() && te[b].empty()) continue;
      const int sc = p->seg_count[b];
      for (int h : p->class_b[l]) {
        const int f = b * H + h;
        SegMeta* m = p->metas(l, f);
        int32_t evicted = 0;
        ev.clear();
        for (int32_t s : te[b]) {
          if (m[s].cpu_s >= 0 && m[s].gpu_s >= 0) {
            ev.emplace_back(m[s].gpu_s, m[s].gpu_e);
            m[s].gpu_s = m[s].gpu_e = -1;
          }
        }
        std::sort(ev.begin(), ev.end());
        for (auto& r : ev) evicted += r.second - r.first;
        if (!ev.empty()) {
          // (an evicted segment's gpu rows were cleared just above, so the
          // resident test alone leaves it out)
          for (int s = 0; s < sc; ++s) {
            if (m[s].cpu_s < 0 || m[s].gpu_s < 0) continue;
            int32_t shift = 0;
            for (auto& r : ev)
              if (r.second <= m[s].gpu_s) shift += r.second - r.first;
            m[s].gpu_s -= shift;
            m[s].gpu_e -= shift;
          }
        }
        ev_f[f] = ev;
        int32_t cursor = lens_l[f] - evicted;
        int32_t loaded_rows = 0;
        for (int32_t s : tl[b]) {  // ascending segment order
          if (m[s].cpu_s < 0) continue;
          const int32_t n = m[s].cpu_e - m[s].cpu_s;
          p->ranges.push_back({m[s].cpu_s, m[s].cpu_e});
          if (ls[f] < 0) ls[f] = transfer;
          ll[f] += n;
          m[s].gpu_s = cursor;
          m[s].gpu_e = cursor + n;
          cursor += n;
          loaded_rows += n;
          transfer += n;
        }
        nl[f] = lens_l[f] - evicted + loaded_rows + 1;
      }
    }
    // per-layer CSR of evict ranges; the layer pointer indexes the global lists
    evict_layer_ptr[l] = (int32_t)p->ev_starts.size();
    eo[0] = 0;
    int32_t emax = 0;
    for (int f = 0; f < N; ++f) {
      for (auto& r : ev_f[f]) {
        p->ev_starts.push_back(r.first);
        p->ev_ends.push_back(r.second);
      }
      eo[f + 1] = (int32_t)p->ev_starts.size() - evict_layer_ptr[l];
      emax = std::max(emax, (int32_t)ev_f[f].size());
    }
    evict_max[l] = emax;
    int32_t* cu = cu_new_2d + (size_t)l * (N + 1);
    cu[0] = 0;
    for (int f = 0; f < N; ++f) {
      new_lens_2d[(size_t)l * N + f] = nl[f];
      cu[f + 1] = cu[f] + nl[f];
    }
  }
  evict_layer_ptr[L] = (int32_t)p->ev_starts.size();
  p->range_layer_ptr[L] = (int32_t)p->ranges.size();
  p->seq_lens = std::move(new_lens);
  p->prev_changed = true;
  *total_rows = transfer;
  *n_evict = (int64_t)p->ev_starts.size();
  *n_ranges = (int64_t)p->ranges.size();
  return WNW_OK;
}

// Copies the last plan's evict ranges (all layers, layer-major) out.
extern "C" int wnw_planner_get_evictions(wnw_planner* p, int32_t* starts, int32_t* ends, int64_t cap) {
  P_CHECK(p, "planner: null handle");
  const int64_t n = (int64_t)p->ev_starts.size();
  P_CHECK(cap >= n && (n == 0 || (starts && ends)), "planner: evict output holds %lld, need %lld",
          (long long)cap, (long long)n);
  if (n) {
    memcpy(starts, p->ev_starts.data(), n * sizeof(int32_t));
    memcpy(ends, p->ev_ends.data(), n * sizeof(int32_t));
  }
  return WNW_OK;
}

// Copies the last plan's host transfer ranges out as [n, 2] (start, end).
extern "C" int wnw_planner_get_ranges(wnw_planner* p, int32_t* ranges, int64_t cap) {
  P_CHECK(p, "planner: null handle");
  const int64_t n = (int64_t)p->ranges.size();
  P_CHECK(cap >= n && (n == 0 || ranges), "planner: range output holds %lld, need %lld", (long long)cap,
          (long long)n);
  for (int64_t i = 0; i < n; ++i) {
    ranges[2 * i] = p->ranges[i].start;
    ranges[2 * i + 1] = p->ranges[i].end;
  }
  return WNW_OK;
}

// The last plan's [L + 1] layer pointer into its host ranges: the ranges of
// layer l are [layer_ptr[l], layer_ptr[l + 1]) (layer-major transfer order).
extern "C" int wnw_planner_get_range_layers(wnw_planner* p, int32_t* layer_ptr, int64_t cap) {
  P_CHECK(p, "planner: null handle");
  P_CHECK(layer_ptr && cap >= (int64_t)p->L + 1, "planner: layer pointer output holds %lld, need %d",
          (long long)cap, p->L + 1);
  if (p->range_layer_ptr.empty())
    memset(layer_ptr, 0, sizeof(int32_t) * (size_t)(p->L + 1));
  else
    memcpy(layer_ptr, p->range_layer_ptr.data(), sizeof(int32_t) * (size_t)(p->L + 1));
  return WNW_OK;
}

// The planner's layer count and batch size, for the library's own callers
// (the transfer engine's plan step checks its arguments against them).
void wnw::planner_dims(const wnw_planner* p, int* layers, int* batch) {
  *layers = p ? p->L : 0;
  *batch = p ? p->B : 0;
}

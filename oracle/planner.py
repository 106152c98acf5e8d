"""Decode chunk planner of WnW restated in pure Python -- TEST INFRASTRUCTURE.

Only tests/ use this module, as the checker of the native planner
(``wnw_amd/csrc/planner.cpp``) and of the cache's host logic.  It follows the
reference's Python planner, the one the C++ planner of the reference
restates a second time:

* ``chunk_means`` / ``topk_chunks``: ``WnWCache._compute_chunk_changes``
  (src/algorithms/wnw/code/cache.py:632-649): mean of the class-A score
  accumulator over each chunk's token bounds (prefix sums), then the top-k
  chunks.  Ties are broken towards the lower chunk index (the reference's
  ``torch.topk`` leaves the tie order to the device; tests use tie-free
  scores).
* ``PlannerOracle.chunk_changes``: ``_compute_chunk_changes_from_topk``
  (cache.py:609-630): needed = union of the chunks' segments, to_load =
  needed - loaded, eviction after ``eviction_lag`` consecutive misses.
* ``PlannerOracle.plan``: ``_prepare_pending_rebuild`` (cache.py:756-889):
  per layer, per changed sample, per class-B KV head: sorted relative evict
  ranges, shifts of the surviving resident segments, loads appended at
  ``rel_cursor = seg_len - evicted``, ``new_len = seg_len - evicted +
  loaded + 1``; global transfer order (layer, sample, head, sorted segment).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field


@dataclass
class SegMeta:
    """cache.py:18-24: rows of one offloaded segment on the host and, when
    resident, its position relative to the start of its flat segment."""
    cpu_start: int
    cpu_end: int
    gpu_rel_start: int = -1
    gpu_rel_end: int = -1


def compute_segments(num_audio: int, stride: int) -> list[tuple[int, int]]:
    """cache.py:1092-1094: stride tiles of the audio range."""
    n = math.ceil(num_audio / stride) if num_audio > 0 else 0
    return [(i * stride, min((i + 1) * stride, num_audio)) for i in range(n)]


def compute_chunks(segments: list[tuple[int, int]], chunk_size: int, stride: int) -> list[list[int]]:
    """cache.py:1097-1101: chunk c covers segments c .. c + ceil(chunk/stride) - 1."""
    per = math.ceil(chunk_size / stride)
    n = len(segments)
    return [list(range(c, min(c + per, n))) for c in range(n)]


def chunk_bounds(segments, chunk_to_segs) -> list[tuple[int, int]]:
    """cache.py:186-195: token bounds of each chunk (first seg start, last seg end)."""
    out = []
    for segs in chunk_to_segs:
        out.append((segments[segs[0]][0], segments[segs[-1]][1]) if segs else (0, 0))
    return out


def cu_from_lens(lens) -> list[int]:
    """cache.py:1110-1111."""
    out = [0]
    for x in lens:
        out.append(out[-1] + int(x))
    return out


def chunk_means(scores, bounds) -> list[float]:
    """Mean score over each chunk's token range, via a float32-free exact sum
    (the reference takes float32 prefix sums; tests compare rankings only)."""
    prefix = [0.0]
    for s in scores:
        prefix.append(prefix[-1] + float(s))
    return [(prefix[e] - prefix[s]) / max(1, e - s) for s, e in bounds]


def topk_chunks(means, k: int) -> list[int]:
    """Indices of the k largest means, ties to the lower index."""
    k = min(k, len(means))
    order = sorted(range(len(means)), key=lambda i: (-means[i], i))
    return order[:k]


@dataclass
class Plan:
    """Output of one planning step (cache.py:823-889)."""
    any_change: bool
    new_lens: list = field(default_factory=list)       # [L][N]
    cu_new: list = field(default_factory=list)         # [L][N+1]
    load_starts: list = field(default_factory=list)    # [L][N], -1 = none
    load_lens: list = field(default_factory=list)      # [L][N]
    evict_offsets: list = field(default_factory=list)  # [L][N+1] (per layer)
    evict_starts: list = field(default_factory=list)   # [L][E_l]
    evict_ends: list = field(default_factory=list)     # [L][E_l]
    evict_max: list = field(default_factory=list)      # [L]
    cpu_ranges: list = field(default_factory=list)     # [(cpu_start, cpu_end)] in transfer order
    total: int = 0                                     # rows to transfer


class PlannerOracle:
    """State of the reference's decode planner for one batch."""

    def __init__(self, num_layers, num_kv_heads, batch, top_k_chunks, eviction_lag, chunk_to_segs, class_b,
                 restore_meta, loaded, seq_lens):
        self.L, self.H, self.B = num_layers, num_kv_heads, batch
        self.N = batch * num_kv_heads
        self.top_k = top_k_chunks
        self.lag = eviction_lag
        self.chunk_to_segs = chunk_to_segs          # [B][chunk] -> [seg]
        self.class_b = class_b                      # [L] -> [kv heads]
        self.meta = restore_meta                    # [L][B][H][seg] -> SegMeta | None
        self.loaded = [set(x) for x in loaded]      # [B]
        self.counters = [dict() for _ in range(batch)]
        self.seq_lens = [list(x) for x in seq_lens]  # [L][N], lengths now (caller keeps them)

    def chunk_changes(self, b: int, topk: list[int]):
        """cache.py:609-630."""
        needed = set()
        for c in topk:
            needed.update(self.chunk_to_segs[b][c])
        loaded = self.loaded[b]
        cnt = self.counters[b]
        to_load = needed - loaded
        to_evict = set()
        for si in loaded:
            if si in needed:
                cnt.pop(si, None)
            else:
                cnt[si] = cnt.get(si, 0) + 1
                if cnt[si] >= self.lag:
                    to_evict.add(si)
        self.loaded[b] = (loaded | to_load) - to_evict
        for si in to_evict:
            cnt.pop(si, None)
        return to_load, to_evict

    def step(self, topk_per_sample: list[list[int]]) -> Plan:
        """One decode_all_layers_done: chunk changes of every sample with a
        non-empty top-k list, then the rebuild plan if anything changed
        (cache.py:568-607)."""
        to_load = [set() for _ in range(self.B)]
        to_evict = [set() for _ in range(self.B)]
        change = False
        for b in range(self.B):
            if not topk_per_sample[b]:
                continue
            to_load[b], to_evict[b] = self.chunk_changes(b, topk_per_sample[b])
            change = change or bool(to_load[b] or to_evict[b])
        if not change:
            return Plan(any_change=False)
        return self.plan(to_load, to_evict)

    def plan(self, to_load, to_evict) -> Plan:
        """cache.py:756-889 (host metadata; the device tensors are its lists)."""
        L, H, N = self.L, self.H, self.N
        changed = [b for b in range(self.B) if to_load[b] or to_evict[b]]
        transfer = 0
        ranges = []
        load_rec = [[] for _ in range(L)]            # (flat, start, n)
        evict = [[[] for _ in range(N)] for _ in range(L)]
        new_lens_all = []
        for l in range(L):
            new_lens = [x + 1 for x in self.seq_lens[l]]
            for b in changed:
                for h in self.class_b[l]:
                    f = b * H + h
                    seg_len = self.seq_lens[l][f]
                    metas = self.meta[l][b][h]
                    evicted = 0
                    if to_evict[b]:
                        ev = []
                        for si in to_evict[b]:
                            m = metas[si]
                            if m is not None and m.gpu_rel_start >= 0:
                                ev.append((m.gpu_rel_start, m.gpu_rel_end))
                                m.gpu_rel_start = m.gpu_rel_end = -1
                        ev.sort()
                        evict[l][f] = ev
                        evicted = sum(e - s for s, e in ev)
                        if ev:
                            for si, m in enumerate(metas):
                                if m is None or m.gpu_rel_start < 0 or si in to_evict[b]:
                                    continue
                                shift = sum(e - s for s, e in ev if e <= m.gpu_rel_start)
                                m.gpu_rel_start -= shift
                                m.gpu_rel_end -= shift
                    cursor = seg_len - evicted
                    loaded = 0
                    for si in sorted(to_load[b]):
                        m = metas[si]
                        if m is None:
                            continue
                        n = m.cpu_end - m.cpu_start
                        ranges.append((m.cpu_start, m.cpu_end))
                        load_rec[l].append((f, transfer, n))
                        m.gpu_rel_start, m.gpu_rel_end = cursor, cursor + n
                        cursor += n
                        loaded += n
                        transfer += n
                    new_lens[f] = seg_len - evicted + loaded + 1
            new_lens_all.append(new_lens)

        p = Plan(any_change=True, cpu_ranges=ranges, total=transfer)
        for l in range(L):
            ls, ll = [-1] * N, [0] * N
            for f, start, n in load_rec[l]:
                if ls[f] < 0:
                    ls[f] = start
                ll[f] += n
            p.load_starts.append(ls)
            p.load_lens.append(ll)
            p.new_lens.append(new_lens_all[l])
            p.cu_new.append(cu_from_lens(new_lens_all[l]))
            off, es, ee = [0], [], []
            for f in range(N):
                for s, e in evict[l][f]:
                    es.append(s)
                    ee.append(e)
                off.append(len(es))
            p.evict_offsets.append(off)
            p.evict_starts.append(es)
            p.evict_ends.append(ee)
            p.evict_max.append(max((len(r) for r in evict[l]), default=0))
        self.seq_lens = [list(x) for x in new_lens_all]
        return p

    def append_step(self):
        """A decode step without a rebuild: every segment grows by one row."""
        self.seq_lens = [[x + 1 for x in row] for row in self.seq_lens]

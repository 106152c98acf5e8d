"""WnW prefill (pruning, flat layout, host offload, initial chunk loads)
restated with numpy -- TEST INFRASTRUCTURE.

Only tests/ use this module, as the checker of ``WnWCache``'s prefill hooks
(``wnw_amd/wnw/cache.py``).  Rows are handled as raw 16-bit patterns (or
any fixed-width dtype), so every comparison is bit-exact.  It follows the
reference's WnWCache:

* ``keep_per_segment`` / ``keep_global``: ``_select_topk_per_segment`` and
  ``_select_topk_global`` (src/algorithms/wnw/code/cache.py:1114-1150):
  max(1, int(len * ratio)) tokens per segment, or the same total over the
  whole audio range.  Ties go to the lower token index (``torch.topk``
  leaves them to the device; tests use distinct scores).
* ``Prefill.after_attn``: ``prefill_after_attn`` (cache.py:257-337): class-A
  KV heads keep every row after the left padding; the others keep the text
  rows (after the padding, outside the audio range) followed by their kept
  audio rows in token order; class-B heads send the pruned audio rows to
  the host, grouped by segment in token order.
* ``Prefill.all_layers_done``: ``prefill_all_layers_done`` (cache.py:339-
  384): host rows are concatenated in (layer, sample, head, segment) order
  and indexed by ``restore_meta``; per sample, the class-A score sums pick
  the top-k chunks (chunk means, cache.py:632-649), whose segments are
  loaded at once (``_load_segments_for_sample``, cache.py:651-714): for
  every class-B head of the sample, the host rows of those segments are
  appended in segment order, and ``gpu_rel_start/end`` record where.
"""
from __future__ import annotations

import numpy as np

from .planner import SegMeta, chunk_bounds, chunk_means, compute_chunks, compute_segments, topk_chunks


def _top_indices(scores: np.ndarray, n: int) -> np.ndarray:
    """Indices of the n largest scores, ties to the lower index."""
    order = np.lexsort((np.arange(len(scores)), -np.asarray(scores, np.float64)))
    return order[:n]


def keep_per_segment(scores: np.ndarray, seg_ranges, ratio: float) -> np.ndarray:
    """cache.py:1114-1139."""
    kept = np.zeros(len(scores), bool)
    for s, e in seg_ranges:
        if e > s:
            kept[s + _top_indices(scores[s:e], max(1, int((e - s) * ratio)))] = True
    return kept


def keep_global(scores: np.ndarray, seg_ranges, ratio: float) -> np.ndarray:
    """cache.py:1142-1150."""
    n = min(sum(max(1, int((e - s) * ratio)) for s, e in seg_ranges), len(scores))
    kept = np.zeros(len(scores), bool)
    kept[_top_indices(scores, n)] = True
    return kept


class Prefill:
    """State of one prefill.

    ``audio``: per sample (raw_start, raw_end) in the padded sequence;
    ``pads``: left padding per sample; ``class_a_kv[l]`` / ``class_b[l]``:
    KV heads of layer l; ``retention[l][h]``; ``stride`` / ``chunk``: tokens
    per segment / chunk; ``top_k``: chunks kept; ``global_topk``: the
    prefill selection rule.
    """

    def __init__(self, num_layers, num_kv_heads, audio, pads, class_a_kv, class_b, retention, stride, chunk,
                 top_k, global_topk=False):
        self.L, self.H = num_layers, num_kv_heads
        self.B = len(audio)
        self.audio, self.pads = list(audio), list(pads)
        self.class_a_kv, self.class_b = class_a_kv, class_b
        self.retention = retention
        self.stride, self.top_k, self.global_topk = stride, top_k, global_topk
        self.num_audio = [e - s for s, e in self.audio]
        self.segments = [compute_segments(n, stride) for n in self.num_audio]
        self.chunks = [compute_chunks(r, chunk, stride) for r in self.segments]
        self.layer_k = [None] * num_layers
        self.layer_v = [None] * num_layers
        self.seq_lens = [None] * num_layers
        self.meta = [[[[None] * len(self.segments[b]) for _ in range(self.H)] for b in range(self.B)]
                     for _ in range(num_layers)]
        self.loaded = [set() for _ in range(self.B)]
        self._score_sums = [None] * self.B
        self._host_k, self._host_v, self._host_meta = [], [], []
        self.cpu_k = self.cpu_v = None

    def after_attn(self, l, class_a_scores, per_head_scores, k, v):
        """k, v: [B, H, S, D] arrays of one layer; scores as numpy arrays or None."""
        for b in range(self.B):
            if class_a_scores[b] is not None:
                s = np.asarray(class_a_scores[b], np.float64)
                self._score_sums[b] = s if self._score_sums[b] is None else self._score_sums[b] + s
        rows_k, rows_v, lens = [], [], []
        for b in range(self.B):
            (ra, re), pad = self.audio[b], self.pads[b]
            for h in range(self.H):
                kf, vf = k[b, h], v[b, h]
                if h in self.class_a_kv[l]:
                    rows_k.append(kf[pad:])
                    rows_v.append(vf[pad:])
                    lens.append(kf.shape[0] - pad)
                    continue
                rule = keep_global if self.global_topk else keep_per_segment
                kept = rule(np.asarray(per_head_scores[b][h]), self.segments[b], self.retention[l][h])
                text = np.r_[pad:ra, re:kf.shape[0]]
                audio_kept = ra + np.nonzero(kept)[0]
                rows_k.append(kf[np.r_[text, audio_kept]])
                rows_v.append(vf[np.r_[text, audio_kept]])
                lens.append(len(text) + len(audio_kept))
                if h in self.class_b[l]:
                    pruned = np.nonzero(~kept)[0]
                    for si, (s, e) in enumerate(self.segments[b]):
                        idx = pruned[(pruned >= s) & (pruned < e)]
                        if len(idx):
                            self._host_k.append(kf[ra + idx])
                            self._host_v.append(vf[ra + idx])
                            self._host_meta.append((l, b, h, si, len(idx)))
        self.layer_k[l] = np.concatenate(rows_k)
        self.layer_v[l] = np.concatenate(rows_v)
        self.seq_lens[l] = lens

    def all_layers_done(self, row_shape, dtype):
        if self._host_k:
            self.cpu_k = np.concatenate(self._host_k)
            self.cpu_v = np.concatenate(self._host_v)
        else:
            self.cpu_k = np.zeros((0,) + tuple(row_shape), dtype)
            self.cpu_v = np.zeros((0,) + tuple(row_shape), dtype)
        o = 0
        for l, b, h, si, n in self._host_meta:
            self.meta[l][b][h][si] = SegMeta(o, o + n)
            o += n
        for b in range(self.B):
            scores = self._score_sums[b] if self._score_sums[b] is not None else np.ones(self.num_audio[b])
            bounds = chunk_bounds(self.segments[b], self.chunks[b])
            chosen = topk_chunks(chunk_means(scores, bounds), self.top_k)
            needed = {si for c in chosen for si in self.chunks[b][c]}
            if needed:
                self._load(b, sorted(needed))
            self.loaded[b] = needed

    def _load(self, b, segs):
        """cache.py:651-714."""
        for l in range(self.L):
            cu = np.concatenate([[0], np.cumsum(self.seq_lens[l])]).astype(np.int64)
            rows_k, rows_v, lens = [], [], []
            for f in range(self.B * self.H):
                fb, h = divmod(f, self.H)
                s, e = int(cu[f]), int(cu[f + 1])
                rows_k.append(self.layer_k[l][s:e])
                rows_v.append(self.layer_v[l][s:e])
                cursor = e - s
                if fb == b and h in self.class_b[l]:
                    for si in segs:
                        m = self.meta[l][fb][h][si]
                        if m is None:
                            continue
                        rows_k.append(self.cpu_k[m.cpu_start:m.cpu_end])
                        rows_v.append(self.cpu_v[m.cpu_start:m.cpu_end])
                        m.gpu_rel_start, m.gpu_rel_end = cursor, cursor + (m.cpu_end - m.cpu_start)
                        cursor = m.gpu_rel_end
                lens.append(cursor)
            self.layer_k[l] = np.concatenate(rows_k)
            self.layer_v[l] = np.concatenate(rows_v)
            self.seq_lens[l] = lens

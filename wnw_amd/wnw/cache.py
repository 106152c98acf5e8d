"""WnW KV cache on MI355X: flat varlen layout, class-A/B heads, chunk offload.

Mirrors ``WnWCache`` (src/algorithms/wnw/code/cache.py:27-1010) hook for
hook; every device operation is a kernel of ``libwnw_amd.so`` and every
planning decision the native planner (``wnw_amd.wnw_cpp.planner``):

decode step, per layer (cache.py:487-566)
    ``decode_step_attention``   the decode branch of the patched forward in
                                one call: a pending plan's compaction of the
                                changed segments, then the step's append
                                fused into the attention launch (with the
                                class-A scores of a foldable layer);
    ``decode_before_attn``      the reference's hook: the pending compaction,
                                then the append alone (in place; or
                                ``interleave_append`` / ``rebuild_append_kv``
                                on the dense layout);
    ``fused_decode_attention``  foldable class-A layer: attention + scores in
                                one operator (``q1_decode_attn_score``), else
                                attention then ``decode_after_attn``;
    ``decode_after_attn``       class-A scores per KV group
                                (``fused_score_accumulate``);
after the last layer (cache.py:568-607)
    ``decode_all_layers_done``  chunk means and top-k per sample (one
                                launch, read back through pinned memory) ->
                                native plan -> the host rows to the device
                                in groups of layers (``WNW_OFFLOAD``:
                                "copy", the default, the transfer engine's
                                gather threads and DMA copies; "device", a
                                gather kernel reading pinned memory), each
                                group with an event its layers' rebuilds
                                wait for.

Prefill (cache.py:236-390) builds the flat layout: class-A KV heads keep
every token, other heads keep their per-segment top-k audio tokens plus all
text; the pruned audio rows of class-B heads go to pinned host memory,
grouped per (layer, sample, head, segment) (``restore_meta``), and the
initial top-k chunks are loaded back.

Layout.  With ``slack_rows`` > 0 (the default, 256) each layer is a pool
in which segment s owns ``seg_cap[s]`` rows from physical row
``seg_base[s]``: its ``len`` rows, then room for the next appends.  The
logical view is the reference's (``cu_seqlens_k``, ``seq_lens``, row order
within a segment); only the physical placement differs, so every attention
launch takes ``seg_base``, and ``dense_kv(layer)`` gathers the reference's
dense rows for a caller that needs them.  Appends are in place (one row per
segment, no copy of the layer).  A pool with host rows ends in a flip region
of two halves; a plan compacts the layer's class-B segments with their loads
into the half they do not occupy (every class-B segment, so the other half
is wholly free again), and only a plan that does not fit a half, or an
append beyond a segment's room, copies the layer into a fresh pool.
``slack_rows=0`` keeps the reference's dense layout, where every append
copies the layer out of place (``interleave_append``) and every plan
rebuilds it (``rebuild_append_kv``).

One deliberate difference: before the host refills a pinned staging buffer
it waits for the copies that last read it (the reference overwrites staging
that an in-flight copy may still read).
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass
from itertools import accumulate

import numpy as np
import torch
from torch import Tensor

from .. import _lib
from ..kv.flat_cache import FlatVarlenCache
from ..kv.fused_attn import (decode_attn, decode_attn_append_deferred, q1_decode_attn, q1_decode_attn_score,
                             score_kept_logits, score_slot_bytes, workspace_for)
from ..kv.kernels import append_inplace, interleave_append_kv
from ..wnw_cpp.planner import Planner
from .config import WnWConfig
from .transfer import HostToDevice

_TRANSFER_STREAMS: dict[int, torch.cuda.Stream] = {}  # device index -> the offload's side stream
from .kernels import (chunk_topk, compact_segments, fused_score_accumulate, gather_host_rows, host_rows_readable,
                      rebuild_append_kv)


@dataclass
class SegmentMeta:
    """cache.py:18-24: host rows of one offloaded segment and, when
    resident, its rows relative to the start of its flat segment."""
    cpu_start: int
    cpu_end: int
    gpu_rel_start: int = -1
    gpu_rel_end: int = -1


# ---------------------------------------------------------------------------
# offsets and geometry (cache.py:1092-1111)
# ---------------------------------------------------------------------------
def _compute_segments(num_audio: int, stride: int) -> list[tuple[int, int]]:
    return [(i * stride, min(i * stride + stride, num_audio)) for i in range(math.ceil(num_audio / stride))]


def _compute_chunks(segments: list[tuple[int, int]], chunk_size: int, stride: int) -> list[list[int]]:
    per = math.ceil(chunk_size / stride)
    n = len(segments)
    return [list(range(i, min(i + per, n))) for i in range(n)]


def _to_device(data, dtype: torch.dtype, device: torch.device) -> Tensor:
    """A host list or CPU tensor on the device without waiting for the
    device: staged in a fresh pinned block and copied asynchronously on the
    current stream (the host allocator reuses the block only after the copy
    is done, and the caller's CPU tensor may be overwritten at once).  A
    pageable host->device copy would wait for the stream's earlier work."""
    t = data if isinstance(data, Tensor) else torch.tensor(data, dtype=dtype)
    if torch.device(device).type == "cpu":
        return t.to(dtype, copy=True)
    staged = torch.empty(t.shape, dtype=dtype, pin_memory=True)
    staged.copy_(t)
    return staged.to(device, non_blocking=True)


def _to_device_many(arrays: list[Tensor], device: torch.device) -> list[Tensor]:
    """Several host tensors on the device in one asynchronous copy: packed
    (16-byte aligned) into one fresh pinned block, copied on the current
    stream, returned as typed views of the device copy (shapes kept).  Same
    lifetime rules as ``_to_device``."""
    if torch.device(device).type == "cpu":
        return [a.clone() for a in arrays]
    sizes = [a.numel() * a.element_size() for a in arrays]
    offs, o = [], 0
    for n in sizes:
        offs.append(o)
        o += (n + 15) // 16 * 16
    staged = torch.empty(max(o, 16), dtype=torch.uint8, pin_memory=True)
    for a, off, n in zip(arrays, offs, sizes):
        if n:
            staged[off:off + n].view(a.dtype).copy_(a.reshape(-1))
    dev = staged.to(device, non_blocking=True)
    return [dev[off:off + n].view(a.dtype).view(a.shape) for a, off, n in zip(arrays, offs, sizes)]


def _build_cu_seqlens(seq_lens: list[int], device: torch.device) -> Tensor:
    return _to_device(_build_cu_seqlens_list(seq_lens), torch.int32, device)


def _build_cu_seqlens_list(seq_lens: list[int]) -> list[int]:
    return [0] + list(accumulate(seq_lens))


def _round8(n: int) -> int:
    return (n + 7) // 8 * 8


def _select_topk_per_segment(scores: Tensor, seg_ranges: list[tuple[int, int]], ratio: float) -> Tensor:
    """cache.py:1114-1139: keep max(1, int(len * ratio)) top tokens per segment."""
    kept = torch.zeros(scores.shape[0], dtype=torch.bool, device=scores.device)
    for s, e in seg_ranges:
        if e > s:
            kept[scores[s:e].topk(max(1, int((e - s) * ratio))).indices + s] = True
    return kept


def _select_topk_global(scores: Tensor, seg_ranges: list[tuple[int, int]], ratio: float) -> Tensor:
    """cache.py:1142-1150: the same budget, chosen over the whole audio range."""
    n_keep = min(sum(max(1, int((e - s) * ratio)) for s, e in seg_ranges), scores.shape[0])
    kept = torch.zeros(scores.shape[0], dtype=torch.bool, device=scores.device)
    kept[scores.topk(n_keep).indices] = True
    return kept


def _invert_ranges(ranges: list[tuple[int, int]], total_len: int) -> list[tuple[int, int]]:
    """cache.py:1153-1162: complement of sorted disjoint ranges in [0, total_len)."""
    out, prev = [], 0
    for s, e in ranges:
        if prev < s:
            out.append((prev, s))
        prev = e
    if prev < total_len:
        out.append((prev, total_len))
    return out


class WnWCache(FlatVarlenCache):
    """WnW KV cache manager (see the module docstring for the step flow)."""

    def __init__(self, config: WnWConfig, num_layers: int, num_kv_heads: int, num_q_heads: int, head_dim: int,
                 device: torch.device, adapter=None, slack_rows: int | None = None):
        super().__init__(num_layers, num_kv_heads, num_q_heads, head_dim, device, adapter)
        # spare rows per segment for in-place appends (WNW_SLACK_ROWS, default
        # 256); 0 keeps the reference's dense layout
        if slack_rows is None:
            slack_rows = int(os.environ.get("WNW_SLACK_ROWS", "256"))
        if slack_rows < 0:
            raise ValueError("slack_rows must be >= 0")
        self.slack_rows = int(slack_rows)
        # flip region of a pool with host rows: two halves (sized by _half_rows:
        # the plan's bound on the class-B rows, at least tail_rows_min and
        # tail_factor x their present room); a plan moves the layer's class-B
        # segments into the half they do not occupy
        self.tail_rows_min = 1024
        self.tail_factor = 2
        # layout changes so far: (fresh pools, fresh pools applying a plan,
        # plans applied by moving the class-B segments to the other half)
        self.layout_counts = {"relayout": 0, "relayout_plan": 0, "relocate": 0}
        if config.num_layers == 0:
            config.set_model_dims(num_layers, num_kv_heads, num_q_heads)
        self.config = config
        self.batch_size = 0
        self.layer_k: list[Tensor | None] = [None] * num_layers
        self.layer_v: list[Tensor | None] = [None] * num_layers
        self.cu_seqlens_k: list[Tensor | None] = [None] * num_layers
        self.cu_seqlens_list: list[list[int] | None] = [None] * num_layers
        self.seq_lens: list[list[int] | None] = [None] * num_layers
        self._reset_layout_state()
        self.cpu_restore_k: Tensor | None = None
        self.cpu_restore_v: Tensor | None = None
        self.restore_meta: list = []
        self.loaded_segments: list[set[int]] = []
        self.score_accumulator: Tensor | None = None
        self.score_offsets: Tensor | None = None
        # a5: the out-of-place compaction fallback (cache.py:891-1010)
        self.use_triton_rebuild = os.environ.get("WNW_DISABLE_TRITON_REBUILD", "0") != "1"
        self._class_b_heads_by_layer = [config.get_layer_class_b(l) for l in range(num_layers)]
        self._transfer_stream: torch.cuda.Stream | None = None
        self._planner: Planner | None = None
        self._decode_step = 0
        self._clear_pending_rebuild_state()

    # The reference's Python-planner cache counts the host rows each plan
    # loads (cache.py:816-820); its C++-planner variant does not.
    _record_plan_transfers = True

    # ------------------------------------------------------------------ setup
    def setup_audio(self, audio_starts: Tensor, audio_ends: Tensor, attention_mask: Tensor | None = None) -> None:
        """cache.py:144-166."""
        super().setup_audio(audio_starts, audio_ends, attention_mask)
        starts, ends, pads = audio_starts.tolist(), audio_ends.tolist(), self.pad_lens.tolist()
        self.batch_size = len(starts)
        self._setup_segments(starts, ends, pads)
        self._setup_score_buffers(starts, ends, pads)
        self._setup_chunk_state()

    def _setup_segments(self, starts, ends, pads) -> None:
        """cache.py:168-210: segments, chunks and chunk token bounds per sample."""
        self._raw_audio_starts, self._raw_audio_ends = list(starts), list(ends)
        self.pad_lens_list = list(pads)
        self._audio_starts_list = [s - p for s, p in zip(starts, pads)]
        self._audio_ends_list = [e - p for e, p in zip(ends, pads)]
        stride, chunk = self.config.stride_tokens, self.config.chunk_size_tokens
        self.segment_ranges = [_compute_segments(e - s, stride)
                               for s, e in zip(self._audio_starts_list, self._audio_ends_list)]
        self.chunk_to_segs = [_compute_chunks(r, chunk, stride) for r in self.segment_ranges]
        self._chunk_token_bounds = [
            [(r[c[0]][0], r[c[-1]][1]) if c else (0, 0) for c in c2s]
            for r, c2s in zip(self.segment_ranges, self.chunk_to_segs)
        ]

    def _setup_score_buffers(self, starts, ends, pads) -> None:
        """cache.py:212-221: one float32 accumulator over every sample's audio."""
        self._prefill_scores = [[] for _ in range(self.batch_size)]
        lens = [e - s for s, e in zip(starts, ends)]
        self._score_offsets_list = [0] + list(accumulate(lens))
        self.score_offsets = torch.tensor(self._score_offsets_list, dtype=torch.int32, device=self.device)
        self.score_accumulator = torch.zeros(self._score_offsets_list[-1], dtype=torch.float32, device=self.device)
        self._max_audio = max(lens) if lens else 0

    def _setup_chunk_state(self) -> None:
        """cache.py:223-248."""
        L, B, H = self.num_layers, self.batch_size, self.num_kv_heads
        self.loaded_segments = [set() for _ in range(B)]
        self.layer_k = [None] * L
        self.layer_v = [None] * L
        self.cu_seqlens_k = [None] * L
        self.cu_seqlens_list = [None] * L
        self.seq_lens = [None] * L
        self._reset_layout_state()
        self.restore_meta = [[[[None] * len(self.segment_ranges[b]) for _ in range(H)] for b in range(B)]
                             for _ in range(L)]
        self._cpu_buffers_k, self._cpu_buffers_v, self._cpu_buffer_metas = [], [], []
        self._pending_chunk_update = False
        self._decode_step = 0
        self._planner = None
        self._clear_pending_rebuild_state()

    @property
    def slack_layout(self) -> bool:
        return self.slack_rows > 0

    def _reset_layout_state(self) -> None:
        L = self.num_layers
        self.seg_base: list[Tensor | None] = [None] * L   # int64 [N] physical first row (slack layout)
        self.seg_cap: list[Tensor | None] = [None] * L    # int32 [N] rows each segment may occupy
        self._base_list: list[list[int] | None] = [None] * L
        self._cap_list: list[list[int] | None] = [None] * L
        self._cu_spare: list[Tensor | None] = [None] * L  # the offsets buffer the next append writes
        self._headroom = [0] * L                          # min over segments of cap - len
        self._half_start = [0] * L                        # first row of the flip region
        self._half_size = [0] * L                         # rows of each of its two halves
        self._flip = [0] * L                              # the half the next plan moves into
        self._moves: list = [None] * L                    # a pending plan's layout per layer
        self._move_dev = None                             # ... and its device arrays
        self._max_len = [0] * L
        self._rows = [0] * L                              # sum of the segment lengths

    def _clear_pending_rebuild_state(self) -> None:
        L = self.num_layers
        self._pending_layer_events: list = [None] * L  # per layer: the copy of its loaded rows
        self._waited_groups: set = set()  # transfer-engine groups the compute stream already waits for
        self._waited_events: set = set()  # (device-gather group event, stream) pairs already waited for
        self._pending_gpu_k: Tensor | None = None
        self._pending_gpu_v: Tensor | None = None
        self._pending_load_starts: list = [None] * L
        self._pending_load_lens: list = [None] * L
        self._pending_evict_offsets: list = [None] * L
        self._pending_evict_starts: list = [None] * L
        self._pending_evict_ends: list = [None] * L
        self._pending_evict_max = [0] * L
        self._pending_new_lens: list = [None] * L
        self._pending_cu_new: list = [None] * L
        self._pending_layers_applied = 0

    def _get_transfer_stream(self) -> torch.cuda.Stream:
        """The device's transfer stream, one per device for the process and
        shared by every cache: HIP maps each new stream onto one of a few
        hardware queues in turn (GPU_MAX_HW_QUEUES, 4 by default), so a
        stream made per cache would in time share the compute stream's queue,
        where the offload's work and the decode kernels wait for each other."""
        if self._transfer_stream is None:
            idx = self.device.index if self.device.index is not None else torch.cuda.current_device()
            st = _TRANSFER_STREAMS.get(idx)
            if st is None:
                st = _TRANSFER_STREAMS[idx] = torch.cuda.Stream(device=self.device)  # default priority
            self._transfer_stream = st
        return self._transfer_stream

    # ---------------------------------------------------------------- prefill
    def prefill_before_attn(self, layer_idx: int) -> None:
        self.stats.record_prefill_before(self._snapshot_cache_stats)

    def prefill_after_attn(self, layer_idx: int, class_a_scores: list, per_head_scores: list, key_states: Tensor,
                           value_states: Tensor) -> None:
        """cache.py:254-337: build this layer's flat K/V; offload the pruned
        audio rows of class-B heads to the host, grouped per segment."""
        for b in range(self.batch_size):
            if class_a_scores[b] is not None:
                self._prefill_scores[b].append(class_a_scores[b])
        pieces_k, pieces_v, lens = [], [], []
        stride = self.config.stride_tokens
        for b in range(self.batch_size):
            ra, re, pad = self._raw_audio_starts[b], self._raw_audio_ends[b], self.pad_lens_list[b]
            for h in range(self.num_kv_heads):
                k_full, v_full = key_states[b, h], value_states[b, h]
                if self.config.is_class_a_kv_head(layer_idx, h):
                    pieces_k.append(k_full[pad:])
                    pieces_v.append(v_full[pad:])
                    lens.append(k_full.shape[0] - pad)
                    continue
                ratio = self.config.get_retention(layer_idx, h)
                select = _select_topk_global if self.config.prefill_global_topk else _select_topk_per_segment
                kept = select(per_head_scores[b][h], self.segment_ranges[b], ratio)
                text_k = torch.cat([k_full[pad:ra], k_full[re:]])
                text_v = torch.cat([v_full[pad:ra], v_full[re:]])
                audio_k, audio_v = k_full[ra:re], v_full[ra:re]
                pieces_k.append(torch.cat([text_k, audio_k[kept]]))
                pieces_v.append(torch.cat([text_v, audio_v[kept]]))
                lens.append(text_k.shape[0] + int(kept.sum().item()))
                if self.config.is_class_b(layer_idx, h):
                    idx = (~kept).nonzero(as_tuple=True)[0]
                    if idx.numel() == 0:
                        continue
                    rk, rv = audio_k.index_select(0, idx).cpu(), audio_v.index_select(0, idx).cpu()
                    self.stats.record_cpu_gpu_transfer(b, g2c_tokens=int(idx.numel()),
                                                       g2c_bytes=int((rk.numel() + rv.numel()) * rk.element_size()))
                    counts = torch.bincount(idx // stride, minlength=len(self.segment_ranges[b])).tolist()
                    o = 0
                    for si, n in enumerate(counts):
                        if n > 0:
                            self._cpu_buffers_k.append(rk[o:o + n])
                            self._cpu_buffers_v.append(rv[o:o + n])
                            self._cpu_buffer_metas.append((layer_idx, b, h, si, n))
                            o += n
        self.layer_k[layer_idx] = torch.cat(pieces_k)
        self.layer_v[layer_idx] = torch.cat(pieces_v)
        self.seq_lens[layer_idx] = lens
        self.cu_seqlens_k[layer_idx] = _build_cu_seqlens(lens, self.device)
        self.cu_seqlens_list[layer_idx] = _build_cu_seqlens_list(lens)

    def prefill_all_layers_done(self) -> None:
        """cache.py:339-390: pin the host rows, index them, load the initial
        top-k chunks, hand the state to the native planner."""
        if self._cpu_buffers_k:
            # host order (sample, segment, layer, head): a segment's rows of
            # consecutive layers are adjacent, so a plan's loads of a group of
            # layers are one span per (sample, segment) for the DMA engines;
            # restore_meta indexes the rows as in the reference
            metas = self._cpu_buffer_metas
            order = sorted(range(len(metas)), key=lambda i: (metas[i][1], metas[i][3], metas[i][0], metas[i][2]))
            self.cpu_restore_k = torch.cat([self._cpu_buffers_k[i] for i in order]).pin_memory()
            self.cpu_restore_v = torch.cat([self._cpu_buffers_v[i] for i in order]).pin_memory()
            o = 0
            for i in order:
                l, b, h, si, n = metas[i]
                self.restore_meta[l][b][h][si] = SegmentMeta(o, o + n)
                o += n
        else:
            dt = self.layer_k[0].dtype if self.layer_k[0] is not None else torch.bfloat16
            self.cpu_restore_k = torch.empty(0, self.head_dim, dtype=dt)
            self.cpu_restore_v = torch.empty(0, self.head_dim, dtype=dt)
        self._cpu_buffers_k, self._cpu_buffers_v, self._cpu_buffer_metas = [], [], []
        for b in range(self.batch_size):
            if self._prefill_scores[b]:
                avg = torch.stack(self._prefill_scores[b]).sum(dim=0)
            else:
                avg = torch.ones(self._audio_ends_list[b] - self._audio_starts_list[b], device=self.device)
            self._select_and_apply_chunks(b, avg)
            self._prefill_scores[b].clear()
        self.prefilled = True
        self._to_slack_layout()
        self._init_planner()
        self._precompute_decode_constants()
        self._warm_decode_path()
        self.stats.record_prefill(self._snapshot_cache_stats)

    def load_prefilled_state(self, layer_k: list[Tensor], layer_v: list[Tensor], seq_lens: list[list[int]],
                             cpu_restore_k: Tensor, cpu_restore_v: Tensor, restore_meta: list,
                             loaded_segments: list[set[int]]) -> None:
        """Install the state ``prefill_all_layers_done`` leaves (flat layers,
        pinned host rows, ``restore_meta`` [L][B][H][seg] of SegmentMeta or
        None, loaded segments) without running a model prefill; call after
        ``setup_audio``."""
        for l in range(self.num_layers):
            self.layer_k[l], self.layer_v[l] = layer_k[l], layer_v[l]
            self.seq_lens[l] = list(seq_lens[l])
            self.cu_seqlens_k[l] = _build_cu_seqlens(self.seq_lens[l], self.device)
            self.cu_seqlens_list[l] = _build_cu_seqlens_list(self.seq_lens[l])
        self.cpu_restore_k = cpu_restore_k if cpu_restore_k.is_pinned() else cpu_restore_k.pin_memory()
        self.cpu_restore_v = cpu_restore_v if cpu_restore_v.is_pinned() else cpu_restore_v.pin_memory()
        self.restore_meta = restore_meta
        self.loaded_segments = [set(s) for s in loaded_segments]
        self.prefilled = True
        self._to_slack_layout()
        self._init_planner()
        self._precompute_decode_constants()
        self._warm_decode_path()

    def _select_and_apply_chunks(self, b: int, scores: Tensor) -> None:
        """cache.py:603-607: initial chunk choice of a sample, loaded at once."""
        to_load = self._initial_chunk_changes(b, self._topk_of(b, scores))
        if to_load:
            self._load_segments_for_sample(b, to_load)
        self.loaded_segments[b] = to_load

    def _initial_chunk_changes(self, b: int, topk_chunks: list[int]) -> set[int]:
        """cache.py:609-630 at prefill time: nothing is loaded yet, so the
        chunks' segments are loaded and nothing is evicted (the decode-time
        rule with eviction lag is the native planner's)."""
        return {si for c in topk_chunks for si in self.chunk_to_segs[b][c]} - self.loaded_segments[b]

    def _topk_of(self, b: int, scores: Tensor) -> list[int]:
        """cache.py:632-649: mean score per chunk, top-k (``wnw_chunk_topk``
        over one sample)."""
        bounds = self._chunk_token_bounds[b]
        k = min(self.config.top_k_chunks, len(bounds))
        if k == 0:
            return []
        dev = scores.device
        i32 = dict(dtype=torch.int32, device=dev)
        out = torch.empty(1, k, **i32)
        chunk_topk(scores.float().contiguous(), torch.tensor([0, scores.shape[0]], **i32),
                   torch.tensor([0, len(bounds)], **i32), torch.tensor([s for s, _ in bounds], **i32),
                   torch.tensor([e for _, e in bounds], **i32), k, out)
        return [c for c in out[0].tolist() if c >= 0]

    def _load_segments_for_sample(self, b: int, segs: set[int]) -> None:
        """cache.py:651-714: append the host rows of `segs` to every class-B
        segment of sample b, in segment order (prefill only)."""
        order = sorted(segs)
        for l in range(self.num_layers):
            cu = self.cu_seqlens_list[l]
            pieces_k, pieces_v, lens = [], [], []
            for f in range(self.batch_size * self.num_kv_heads):
                fb, h = divmod(f, self.num_kv_heads)
                s, e = cu[f], cu[f + 1]
                pieces_k.append(self.layer_k[l][s:e])
                pieces_v.append(self.layer_v[l][s:e])
                cursor, extra = e - s, 0
                if fb == b and self.config.is_class_b(l, h):
                    for si in order:
                        m = self.restore_meta[l][fb][h][si]
                        if m is None:
                            continue
                        n = m.cpu_end - m.cpu_start
                        pieces_k.append(self.cpu_restore_k[m.cpu_start:m.cpu_end].to(self.device))
                        pieces_v.append(self.cpu_restore_v[m.cpu_start:m.cpu_end].to(self.device))
                        m.gpu_rel_start, m.gpu_rel_end = cursor, cursor + n
                        cursor += n
                        extra += n
                        self.stats.record_cpu_gpu_transfer(b, c2g_tokens=n, c2g_bytes=2 * n * self.head_dim *
                                                           self.cpu_restore_k.element_size())
                lens.append(e - s + extra)
            self.layer_k[l] = torch.cat(pieces_k)
            self.layer_v[l] = torch.cat(pieces_v)
            self.seq_lens[l] = lens
            self.cu_seqlens_k[l] = _build_cu_seqlens(lens, self.device)
            self.cu_seqlens_list[l] = _build_cu_seqlens_list(lens)

    # ----------------------------------------------------------------- layout
    def _to_slack_layout(self) -> None:
        """After prefill: every layer's dense rows into a pool with slack."""
        N = self.batch_size * self.num_kv_heads
        self._all_segs = torch.arange(N, dtype=torch.int32, device=self.device)
        self._no_loads = torch.full((N,), -1, dtype=torch.int32, device=self.device)
        self._zeros_n = torch.zeros(N, dtype=torch.int32, device=self.device)
        self._zeros_n1 = torch.zeros(N + 1, dtype=torch.int32, device=self.device)
        self._empty_i32 = torch.empty(0, dtype=torch.int32, device=self.device)
        H = self.num_kv_heads
        self._classb_segs = [[f for f in range(N) if f % H in set(self._class_b_heads_by_layer[l])]
                             for l in range(self.num_layers)]
        self._classb_segs_dev = [torch.tensor(x, dtype=torch.int32, device=self.device) for x in self._classb_segs]
        for l in range(self.num_layers):
            self._rows[l] = sum(self.seq_lens[l])
            self._max_len[l] = max(self.seq_lens[l], default=0)
            if self.slack_layout:
                self._relayout(l)

    def _half_rows(self, layer_idx: int, lens: list[int]) -> int:
        """Rows of each half of the flip region after the segments, where
        plans put the class-B segments (with their slack): room for every
        class-B segment at its length plus the most host rows it can have
        loaded at once (``top_k_chunks`` x (1 + ``eviction_lag``) of its
        sample's widest chunks of its largest offloaded segment, capped by
        its offloaded rows), and at least ``tail_factor`` times their present
        room and ``tail_rows_min``; none without host rows (no plan changes a
        layout then) or with ``tail_factor`` and ``tail_rows_min`` both 0 (a
        pool without a flip region: every plan rebuilds the layer)."""
        if self.cpu_restore_k is None or self.cpu_restore_k.shape[0] == 0:
            return 0
        if self.tail_factor == 0 and self.tail_rows_min == 0:
            return 0
        H = self.num_kv_heads
        heads = set(self._class_b_heads_by_layer[layer_idx])
        k, lag = self.config.top_k_chunks, self.config.eviction_lag
        room = grown = 0
        for f, n in enumerate(lens):
            if f % H not in heads:
                continue
            b, h = divmod(f, H)
            rows = [m.cpu_end - m.cpu_start for m in self.restore_meta[layer_idx][b][h] if m is not None]
            width = max((len(c) for c in self.chunk_to_segs[b]), default=0)
            extra = min(sum(rows), k * (1 + lag) * width * max(rows)) if rows else 0
            room += _round8(n + self.slack_rows)
            grown += _round8(n + extra + self.slack_rows)
        return _round8(max(self.tail_rows_min, self.tail_factor * room, grown))

    def _relayout(self, layer_idx: int, plan: dict | None = None) -> None:
        """Copy layer ``layer_idx`` into a fresh pool: every segment's rows in
        index order with ``slack_rows`` of room after each, then a free tail.
        The source is the current pool (or the dense layer right after
        prefill).  With ``plan`` (the layer's compaction descriptors) the
        evictions and loads are applied on the way, to the plan's lengths
        without the step's append."""
        l, dev, D = layer_idx, self.device, self.head_dim
        N = self.batch_size * self.num_kv_heads
        new_lens = list(self.seq_lens[l]) if plan is None else list(plan["lens"])
        caps = [_round8(n + self.slack_rows) for n in new_lens]
        bases = [0] + list(accumulate(caps))[:-1]
        used = sum(caps)
        half = self._half_rows(l, new_lens)
        pool = used + 2 * half
        cu = self.cu_seqlens_k[l]
        src_base = self.seg_base[l] if self.seg_base[l] is not None else cu[:-1].to(torch.int64)
        src_len = cu[1:] - cu[:-1]
        dst_base = _to_device(bases, torch.int64, dev)
        new_len_t = _to_device(new_lens, torch.int32, dev)
        old_k, old_v = self.layer_k[l], self.layer_v[l]
        k = torch.empty(pool, D, dtype=old_k.dtype, device=dev)
        v = torch.empty_like(k)
        if max(new_lens, default=0) > 0:
            if plan is None:
                compact_segments(old_k, old_v, k, v, self._all_segs, src_base, src_len, dst_base, new_len_t,
                                 old_k[:0], old_v[:0], self._no_loads, self._zeros_n, self._zeros_n1,
                                 self._empty_i32, self._empty_i32, max(new_lens))
            else:
                compact_segments(old_k, old_v, k, v, self._all_segs, src_base, src_len, dst_base, new_len_t,
                                 plan["load_k"], plan["load_v"], plan["load_starts"], plan["load_lens"],
                                 plan["evict_offsets"], plan["evict_starts"], plan["evict_ends"], max(new_lens))
        self.layer_k[l], self.layer_v[l] = k, v
        self.seg_base[l] = dst_base
        self.seg_cap[l] = _to_device(caps, torch.int32, dev)
        self._base_list[l], self._cap_list[l] = bases, caps
        self._half_start[l], self._half_size[l], self._flip[l] = used, half, 0
        self._set_lens(l, new_lens)
        self.layout_counts["relayout" if plan is None else "relayout_plan"] += 1

    def _set_lens(self, layer_idx: int, lens: list[int], cu_dev: Tensor | None = None) -> None:
        """Host lengths and device offsets of a layer after a layout change
        (``cu_dev``: the offsets already on the device)."""
        l = layer_idx
        self.seq_lens[l] = list(lens)
        self.cu_seqlens_list[l] = _build_cu_seqlens_list(self.seq_lens[l])
        self.cu_seqlens_k[l] = cu_dev if cu_dev is not None else \
            _to_device(self.cu_seqlens_list[l], torch.int32, self.device)
        if self._cu_spare[l] is None or self._cu_spare[l].shape != self.cu_seqlens_k[l].shape:
            self._cu_spare[l] = torch.empty_like(self.cu_seqlens_k[l])
        self._rows[l] = self.cu_seqlens_list[l][-1]
        self._max_len[l] = max(lens, default=0)
        self._headroom[l] = min((c - n for c, n in zip(self._cap_list[l], lens)), default=0)

    def dense_kv(self, layer_idx: int) -> tuple[Tensor, Tensor]:
        """The layer's rows in the reference's dense layout (segment s at
        rows [cu[s], cu[s+1]) of [total, head_dim]); a gather on the slack
        layout, the layer itself on the dense one."""
        l = layer_idx
        if self.seg_base[l] is None:
            return self.layer_k[l], self.layer_v[l]
        idx = torch.cat([torch.arange(b, b + n, device=self.device)
                         for b, n in zip(self._base_list[l], self.seq_lens[l])]) if self._rows[l] else \
            torch.empty(0, dtype=torch.int64, device=self.device)
        return self.layer_k[l].index_select(0, idx), self.layer_v[l].index_select(0, idx)

    def _init_planner(self) -> None:
        """Hand segments, chunks, class-B heads, restore metadata, loaded sets
        and lengths to the native planner (src/algorithms/wnw_cpp/code/
        cache.py:40-120 does the same for the reference's C++ planner)."""
        L, H, B = self.num_layers, self.num_kv_heads, self.batch_size
        p = Planner(L, H, B, self.num_kv_groups)
        p.set_config(self.config.top_k_chunks, self.config.eviction_lag)
        p.set_seg_count([len(self.segment_ranges[b]) for b in range(B)])
        for b in range(B):
            flat, off = [], [0]
            for segs in self.chunk_to_segs[b]:
                flat += segs
                off.append(len(flat))
            p.set_chunk_to_segs(b, flat, off)
        for l in range(L):
            p.set_class_b(l, self._class_b_heads_by_layer[l])
        cs, ce, gs, ge = [], [], [], []
        for l in range(L):
            for f in range(B * H):
                b, h = divmod(f, H)
                for m in self.restore_meta[l][b][h]:
                    if m is None:
                        cs.append(-1), ce.append(-1), gs.append(-1), ge.append(-1)
                    else:
                        cs.append(m.cpu_start), ce.append(m.cpu_end)
                        gs.append(m.gpu_rel_start), ge.append(m.gpu_rel_end)
        p.set_restore_meta(cs, ce, gs, ge)
        for b in range(B):
            p.set_loaded(b, sorted(self.loaded_segments[b]))
        p.set_seq_lens([x for l in range(L) for x in self.seq_lens[l]])
        # two pinned staging pairs, used in turn and grown on demand: a plan's
        # gather waits only for the copy that used its pair two plans ago
        self._staging = [None, None]
        self._staging_turn = 0
        # the offload channel (WNW_OFFLOAD), per group of layers on a side
        # stream, a layer waiting for its own group only:
        # "copy" (default), the transfer engine's direct form -- the DMA
        #   engines copy the plan's rows straight from the pinned restore
        #   rows (merged spans) into a device stage, a kernel puts them in
        #   transfer order; the host copies nothing;
        # "staged", the transfer engine's staged form -- host threads gather
        #   the rows into pinned staging, the DMA engines copy that;
        # "device", a gather kernel reading the pinned restore rows itself
        #   (its reads of host memory outrun the copy engine, but the compute
        #   kernels that run meanwhile slow down by more than that)
        # groups (copies + events) per plan: copy/compute overlap against
        # per-copy cost.  Six: at 30 layers groups of 3, 6, 6, 6, 6 and 3
        # layers.  One layer's spans are too short for the copy engines
        # (each copy takes about as long to submit as to move), so a
        # one-layer first group left the link partly idle at the start of
        # every plan; the short last group shortens what runs after the
        # plan's last copy
        self._load_groups = 6
        mode = os.environ.get("WNW_OFFLOAD", "copy")
        if mode not in ("copy", "staged", "device"):
            raise ValueError(f"WNW_OFFLOAD must be 'copy', 'staged' or 'device', got {mode!r}")
        if mode == "device" and self.cpu_restore_k.shape[0] > 0 and \
                not host_rows_readable(self.cpu_restore_k, self.cpu_restore_v):
            mode = "copy"  # the device cannot read these host rows: through the copy engines
        self._offload = mode
        self._h2d = None
        self._stage = None
        self._started_loads = None  # (K rows, V rows, group of each layer) of a transfer started with its plan
        self._staging_rows_hint = self._plan_rows_bound()
        dt = self.cpu_restore_k.dtype
        if mode == "staged" and self._staging_rows_hint > 0:
            # both pairs now, touched once: a first write into fresh pinned
            # pages is several times slower than the gathers that follow
            self._staging = [tuple(torch.zeros(self._staging_rows_hint, self.head_dim, dtype=dt, pin_memory=True)
                                   for _ in range(2)) for _ in range(2)]
        elif mode == "copy" and self._staging_rows_hint > 0:
            self._device_stage(self._staging_rows_hint)
        N = B * H
        self._plan_out = dict(
            load_starts_2d=torch.empty(L, N, dtype=torch.int32), load_lens_2d=torch.empty(L, N, dtype=torch.int32),
            cu_new_2d=torch.empty(L, N + 1, dtype=torch.int32), new_lens_2d=torch.empty(L, N, dtype=torch.int32),
            evict_offsets_2d=torch.empty(L, N + 1, dtype=torch.int32), evict_max=torch.empty(L, dtype=torch.int32),
            evict_layer_ptr=torch.empty(L + 1, dtype=torch.int32))
        self._planner = p

    def _precompute_decode_constants(self) -> None:
        """cache.py:392-484: per-layer class-A groups by KV head, foldable
        layers (whole GQA groups class A) and their KV masks, audio ranges."""
        N = self.batch_size * self.num_kv_heads
        _lib.ensure_init(self.device)  # module load and device error word (replaces the Triton warm-up)
        self._cu_step_increment = torch.arange(N + 1, dtype=torch.int32, device=self.device)
        self._empty_i32 = torch.empty(0, dtype=torch.int32, device=self.device)
        G = self.num_kv_groups
        self._decode_after_groups = [[] for _ in range(self.num_layers)]
        self._layer_foldable, self._ca_kv_mask_by_layer, self._ca_kv_bits_by_layer = [], [], []
        self._decode_class_a_local = None
        for l in range(self.num_layers):
            ca = self.config.get_layer_class_a(l)
            if ca and self._decode_class_a_local is None:
                self._decode_class_a_local = ca
            by_kv: dict[int, list[int]] = {}
            for qh in ca:
                by_kv.setdefault(qh // G, []).append(qh)
            for kv, qheads in sorted(by_kv.items()):
                seg_idx = torch.tensor([b * self.num_kv_heads + kv for b in range(self.batch_size)],
                                       dtype=torch.int64, device=self.device)
                self._decode_after_groups[l].append((qheads, seg_idx))
            foldable = bool(ca) and all(set(range(kv * G, (kv + 1) * G)) <= set(ca) for kv in by_kv)
            self._layer_foldable.append(foldable)
            if foldable:
                mask = torch.zeros(self.num_kv_heads, dtype=torch.int32)
                mask[list(by_kv)] = 1
                self._ca_kv_mask_by_layer.append(mask.to(self.device))
            else:
                self._ca_kv_mask_by_layer.append(None)
            self._ca_kv_bits_by_layer.append(sum(1 << kv for kv in by_kv) if foldable else 0)
        self._decode_audio_starts_b = torch.tensor(self._audio_starts_list, dtype=torch.int32, device=self.device)
        self._decode_audio_ends_b = torch.tensor(self._audio_ends_list, dtype=torch.int32, device=self.device)
        # deferred class-A scoring (slack layout, fused scoring): a foldable
        # layer's launch keeps its logits in a score slot and the next
        # launch scores them after its own stream, so no scoring launch of
        # its own runs except at the step's end (WNW_DEFER_SCORES=0 turns it
        # off; a geometry the library does not take turns it off by itself)
        self._defer_scores = os.environ.get("WNW_DEFER_SCORES", "1") != "0"
        self._score_slots: list | None = None
        self._slot_turn = 0
        # (mask, slot, cu, seg_base, pool_rows, KV-head bits) of a launch not scored yet
        self._pending_score = None
        # chunk scoring on the device (one launch of wnw_chunk_topk): every
        # sample's chunks as a CSR of token bounds relative to its scores
        B = self.batch_size
        dev = self.device
        self._max_chunks = max((len(c) for c in self.chunk_to_segs), default=0)
        if self._max_chunks > _lib.TOPK_MAX_CHUNKS:
            raise ValueError(f"{self._max_chunks} chunks in one sample; the device top-k takes at most "
                             f"{_lib.TOPK_MAX_CHUNKS}")
        self._tk_k = min(self.config.top_k_chunks, self._max_chunks)
        if self._tk_k > _lib.TOPK_MAX_K:
            raise ValueError(f"top_k_chunks {self._tk_k} above the device top-k's {_lib.TOPK_MAX_K}")
        bounds = [se for b in range(B) for se in self._chunk_token_bounds[b]]
        self._tk_chunk_off = torch.tensor([0] + list(accumulate(len(self._chunk_token_bounds[b]) for b in range(B))),
                                          dtype=torch.int32, device=dev)
        self._tk_s = torch.tensor([s for s, _ in bounds], dtype=torch.int32, device=dev)
        self._tk_e = torch.tensor([e for _, e in bounds], dtype=torch.int32, device=dev)
        k = max(1, self._tk_k)
        self._tk_out = torch.empty(B, k, dtype=torch.int32, device=dev)
        # the choice comes back through pinned memory and an event: the host
        # waits for the top-k launch only, not for the device to go idle
        self._tk_host = torch.empty(B, k, dtype=torch.int32, pin_memory=True)
        self._tk_event = torch.cuda.Event()

    # ----------------------------------------------------------------- decode
    def _before_decode_layer(self, layer_idx: int) -> None:
        """Work due before a layer's decode step (the deferred-plan variant
        finalises its plan at layer 0)."""

    def decode_before_attn(self, layer_idx: int, new_k: Tensor, new_v: Tensor):
        """cache.py:487-515: returns (K, V, cu_seqlens_k, max_seqlen_k).

        Slack layout: K and V are the layer's pools and segment s's rows
        start at physical row ``seg_base[layer_idx][s]``; the append is in
        place.  Dense layout: the reference's arrays, rebuilt out of place."""
        self._before_decode_layer(layer_idx)
        if self.slack_layout:
            l = layer_idx
            self._apply_pending_slack(l)
            self._ensure_headroom(l)
            nk = new_k.squeeze(2).reshape(-1, self.head_dim)
            nv = new_v.squeeze(2).reshape(-1, self.head_dim)
            append_inplace(self.layer_k[l], self.layer_v[l], nk, nv, self.cu_seqlens_k[l], self._cu_spare[l],
                           self.seg_base[l], self.seg_cap[l])
            self._commit_append(l)
            return self.layer_k[l], self.layer_v[l], self.cu_seqlens_k[l], self._max_len[l]
        if self._pending_chunk_update:
            if self.use_triton_rebuild and self._pending_cu_new[layer_idx] is not None:
                return self._rebuild_append_layer(layer_idx, new_k, new_v)
            self._apply_chunk_update_to_layer(layer_idx)
        nk = new_k.squeeze(2).reshape(-1, self.head_dim)
        nv = new_v.squeeze(2).reshape(-1, self.head_dim)
        cu_old = self.cu_seqlens_k[layer_idx]
        new_lens = [x + 1 for x in self.seq_lens[layer_idx]]
        cu_new = cu_old + self._cu_step_increment
        k, v = interleave_append_kv(self.layer_k[layer_idx], self.layer_v[layer_idx], nk, nv, cu_old, cu_new)
        self.layer_k[layer_idx], self.layer_v[layer_idx] = k, v
        self.seq_lens[layer_idx] = new_lens
        self.cu_seqlens_k[layer_idx] = cu_new
        self.cu_seqlens_list[layer_idx] = _build_cu_seqlens_list(new_lens)
        self._rows[layer_idx] += len(new_lens)
        self._max_len[layer_idx] = max(new_lens)
        return k, v, cu_new, max(new_lens)

    def decode_step_attention(self, layer_idx: int, q_flat: Tensor, q: Tensor, new_k: Tensor, new_v: Tensor,
                              scale: float, fused: bool) -> Tensor:
        """The decode branch of the patched forward (session.py:78-116) from
        the append on: ``decode_before_attn`` + the attention (+ scores), in
        as few launches as the layout allows.  Slack layout: a pending plan's
        compaction of the changed segments, then one launch that appends the
        step's row to every segment and attends (with the class-A scores of a
        foldable layer when ``fused``, as ``fused_decode_attention`` does);
        other class-A layers score afterwards (``decode_after_attn``).
        Returns the attention output [N, G, D]."""
        l = layer_idx
        if not self.slack_layout:
            k, v, cu, _ = self.decode_before_attn(l, new_k, new_v)
            if fused:
                return self.fused_decode_attention(l, q_flat, q, k, v, cu, scale)
            out = q1_decode_attn(q_flat, k, v, cu, scale)
            self.decode_after_attn(l, q)
            return out
        self._before_decode_layer(l)
        self._apply_pending_slack(l)
        self._ensure_headroom(l)
        nk = new_k.reshape(-1, self.head_dim)  # [B, Hkv, 1, D] -> [N, D]
        nv = new_v.reshape(-1, self.head_dim)
        rows = self._rows[l] + self.batch_size * self.num_kv_heads
        score_here = fused and self._layer_foldable[l]
        # the cache's own tensors, checked when made: the launches skip the
        # wrappers' argument checks (q and the new rows are the caller's and
        # are checked here)
        q_flat, nk, nv = q_flat.contiguous(), nk.contiguous(), nv.contiguous()
        if not (q_flat.is_cuda and nk.is_cuda and nv.is_cuda and q_flat.dtype == nk.dtype == nv.dtype ==
                self.layer_k[l].dtype and q_flat.shape[0] == nk.shape[0] == len(self.seq_lens[l])
                and q_flat.shape[1:] == (self.num_q_heads // self.num_kv_heads, self.head_dim)):
            raise _lib.WnwError("q and the new K/V rows must be GPU tensors of the cache's dtype, one per segment")
        app = (nk, nv, self._cu_spare[l], self.seg_cap[l])
        if fused and self._defer_scores and (score_here or self._pending_score is not None):
            out = self._deferred_launch(l, q_flat, rows, app, scale, score_here)
            if out is not None:
                self._commit_append(l)
                if not score_here:
                    self.decode_after_attn(l, q)
                return out
        if score_here:
            out = q1_decode_attn_score(q_flat, self.layer_k[l], self.layer_v[l], self.cu_seqlens_k[l], scale,
                                       self._ca_kv_mask_by_layer[l], self.num_kv_heads, self._decode_audio_starts_b,
                                       self._decode_audio_ends_b, self.score_accumulator, self.score_offsets,
                                       seg_base=self.seg_base[l], total_rows=rows, max_audio=self._max_audio,
                                       append=app, validate=False)
        else:
            out = decode_attn(q_flat, self.layer_k[l], self.layer_v[l], self.cu_seqlens_k[l], scale,
                              seg_base=self.seg_base[l], total_rows=rows, append=app, validate=False)
        self._commit_append(l)
        if not score_here:
            self.decode_after_attn(l, q)
        return out

    def _deferred_launch(self, l: int, q_flat: Tensor, rows: int, app: tuple, scale: float, score_here: bool):
        """Layer l's fused append + attention through the deferred-scoring
        form: its class-A logits kept in a score slot when the layer scores
        here, the pending slot of an earlier launch scored by this launch.
        Returns the output, or None (nothing launched, deferral turned off
        and the pending slot scored in its own launch) where the library does
        not take the geometry."""
        self._ensure_score_slots()
        keep = self._ca_kv_mask_by_layer[l] if score_here else None
        slot = self._score_slots[self._slot_turn] if score_here else None
        out = decode_attn_append_deferred(
            q_flat, self.layer_k[l], self.layer_v[l], self.cu_seqlens_k[l], scale, seg_base=self.seg_base[l],
            total_rows=rows, append=app, num_kv_heads=self.num_kv_heads, audio_starts=self._decode_audio_starts_b,
            audio_ends=self._decode_audio_ends_b, max_audio=self._max_audio,
            score_accumulator=self.score_accumulator, score_offsets=self.score_offsets, keep_mask=keep,
            keep_slot=slot, prev=self._pending_score)
        if out is None:
            self._defer_scores = False
            self._flush_pending_scores()
            return None
        # the segments as this launch saw them: its post-append offsets (the
        # buffer _commit_append makes current), its pool
        self._pending_score = (keep, slot, app[2], self.seg_base[l], self.layer_k[l].shape[0],
                               self._ca_kv_bits_by_layer[l]) if score_here else None
        if score_here:
            self._slot_turn ^= 1
        return out

    def _ensure_score_slots(self) -> None:
        """The two score slots of deferred scoring (a launch writes one and
        scores the other)."""
        if self._score_slots is None:
            n = score_slot_bytes(self.batch_size * self.num_kv_heads, self.num_kv_groups, self._max_audio)
            self._score_slots = [torch.empty((n + 3) // 4, dtype=torch.float32, device=self.device) for _ in range(2)]

    def _warm_decode_path(self) -> None:
        """First-use costs of the decode path paid here, at the end of the
        prefill, instead of inside the first decode steps (tens of ms on
        MI355X; cache.py:392-484 warms the reference's Triton kernels for the
        same reason): the attention workspace of the current stream (with the
        scoring room when a layer folds its scoring into the attention), the
        score slots of deferred scoring, one chunk top-k with its copy back,
        and the transfer engine's copy streams, DMA engines, events,
        descriptor room and thread; and the kernels launched outside the
        attention, set up on the device (``wnw_prepare_kernels``)."""
        N, G, D = self.batch_size * self.num_kv_heads, self.num_kv_groups, self.head_dim
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().wnw_prepare_kernels(), "wnw_prepare_kernels")
        ws = workspace_for(self.device)
        if any(self._layer_foldable):
            ws.get(N, G, D, score=True, max_audio=self._max_audio)
            if self._defer_scores and self.slack_layout:
                self._ensure_score_slots()
        else:
            ws.get(N, G, D)
        if self._tk_k > 0:
            self._topk_scores_async()
            self._tk_event.synchronize()
        if self._offload in ("copy", "staged") and self.cpu_restore_k.shape[0] > 0:
            if self._h2d is None:
                self._h2d = HostToDevice()
            self._h2d.reserve(self._plan_ranges_bound(), self._get_transfer_stream(), len(self._group_layers()))

    def _plan_ranges_bound(self) -> int:
        """An upper bound on the host ranges one plan loads: per (layer,
        sample, class-B head), its offloaded segments, at most
        ``top_k_chunks`` chunks of the sample's widest chunk."""
        k = self.config.top_k_chunks
        total = 0
        for b in range(self.batch_size):
            width = max((len(c) for c in self.chunk_to_segs[b]), default=0)
            for l in range(self.num_layers):
                for h in range(self.num_kv_heads):
                    n = sum(1 for m in self.restore_meta[l][b][h] if m is not None)
                    total += min(n, k * width)
        return total

    def _flush_pending_scores(self) -> None:
        """Scores the pending slot in a launch of its own (the last foldable
        layer of a step has no later launch to carry it)."""
        if self._pending_score is not None:
            score_kept_logits(self._pending_score, self.batch_size * self.num_kv_heads, self.num_kv_groups,
                              self.num_kv_heads, self._decode_audio_starts_b, self._decode_audio_ends_b,
                              self._max_audio, self.score_accumulator, self.score_offsets)
            self._pending_score = None
        self._slot_turn = 0

    def _commit_append(self, layer_idx: int) -> None:
        """Host bookkeeping of an in-place append: the offsets the append
        wrote become current, every segment is one row longer."""
        l = layer_idx
        self.cu_seqlens_k[l], self._cu_spare[l] = self._cu_spare[l], self.cu_seqlens_k[l]
        self.seq_lens[l] = [x + 1 for x in self.seq_lens[l]]
        self.cu_seqlens_list[l] = None  # rebuilt on demand (cu_list)
        self._headroom[l] -= 1
        self._max_len[l] += 1
        self._rows[l] += len(self.seq_lens[l])

    def decode_headroom(self) -> int:
        """Decode steps every layer can still append in place (slack layout)
        before a pool is rebuilt: the most steps a captured graph of plain
        decode steps may be replayed for."""
        return min(self._headroom) if self.slack_layout else 0

    def advance_replayed_steps(self, n: int) -> None:
        """Host bookkeeping of ``n`` decode steps that ran as replays of
        captured graphs.  A capture runs the hooks' host side once and a
        replay only the device work (the appends and the offsets they write),
        so after replaying captured plain decode steps the host's lengths
        (and the native planner's) are advanced here.

        Rules, each refused with ``ValueError``:
        * slack layout, with room in every segment for the ``n`` appends;
        * ``n`` even: a step's append reads one offsets buffer and writes the
          other, so a replayable pair of captures alternates them, and the
          host's current buffer is the device's again only after an even
          number of replays;
        * no chunk selection (``top_k_chunks`` 0): a replay skips the
          end-of-step planning the reference runs every step, so a replayed
          step with selection on would not be the reference's step;
        * no plan pending (its compaction would have run in a replay)."""
        if n == 0:
            return
        if n < 0 or n % 2:
            raise ValueError(f"replayed steps come in pairs of alternating captures (got {n})")
        if not self.slack_layout or n > self.decode_headroom():
            raise ValueError("replayed steps need the slack layout and room for every append")
        if self._tk_k > 0:
            raise ValueError("replayed steps skip the per-step chunk selection: top_k_chunks must be 0")
        if self._pending_chunk_update:
            raise ValueError("a plan is pending: its compaction is not part of a replayed plain step")
        for l in range(self.num_layers):
            self.seq_lens[l] = [x + n for x in self.seq_lens[l]]
            self.cu_seqlens_list[l] = None
            self._headroom[l] -= n
            self._max_len[l] += n
            self._rows[l] += n * len(self.seq_lens[l])
        self._decode_step += n
        self._seq_lengths = [x + n for x in self._seq_lengths]
        # a capture of the fused launches alone leaves its last scored
        # layer's slot pending; its replays' scores are read by nobody
        self._pending_score = None
        self._slot_turn = 0
        if self._planner is not None:
            # the planner counts a plain step when it plans the next one; its
            # lengths are the host's after the last plain step
            self._planner.set_seq_lens([x for l in range(self.num_layers) for x in self.seq_lens[l]])

    def cu_list(self, layer_idx: int) -> list[int]:
        """Host copy of a layer's offsets (cu_seqlens_k)."""
        if self.cu_seqlens_list[layer_idx] is None:
            self.cu_seqlens_list[layer_idx] = _build_cu_seqlens_list(self.seq_lens[layer_idx])
        return self.cu_seqlens_list[layer_idx]

    def _ensure_headroom(self, layer_idx: int) -> None:
        """Room for one more row in every segment, else a fresh pool."""
        if self._headroom[layer_idx] < 1:
            self._relayout(layer_idx)

    def _apply_pending_slack(self, layer_idx: int) -> None:
        """A pending plan's compaction + loads for this layer (slack layout),
        as decided when the plan was made (``_plan_slack_moves``): the
        class-B segments move into the free half of the flip region, or the
        whole layer into a fresh pool.  Lengths and offsets become the
        plan's, without the step's append (the append follows)."""
        l = layer_idx
        if not self._pending_chunk_update or self._pending_cu_new[l] is None:
            return
        self._wait_loads(l)
        kind, bases, caps, lens = self._moves[l]
        if kind == "relayout":
            self._relayout(l, dict(lens=lens, load_k=self._pending_gpu_k, load_v=self._pending_gpu_v,
                                   load_starts=self._pending_load_starts[l], load_lens=self._pending_load_lens[l],
                                   evict_offsets=self._pending_evict_offsets[l],
                                   evict_starts=self._pending_evict_starts[l], evict_ends=self._pending_evict_ends[l]))
        elif kind == "move":
            self._move_class_b(l, bases, caps, lens)
        self._moves[l] = None
        self._pending_layers_applied += 1
        if self._pending_layers_applied == self.num_layers:
            self._pending_chunk_update = False
            self._clear_pending_rebuild_state()
            self._move_dev = None

    def _plan_slack_moves(self, new_lens_all: list[list[int]]) -> list[Tensor]:
        """Where a plan puts every layer's rows (slack layout), decided on the
        host when the plan is made; returns the host arrays of every layer's
        move (bases, capacities, lengths, source lengths, offsets), which go
        to the device with the plan's other descriptors.  In a layer the plan changes, every class-B
        segment (changed or not) is compacted with its loads into the half
        of the flip region the class-B segments do not occupy, packed with
        their slack; so the half they leave is wholly free for the next plan
        and no search for room is needed.  A layer whose block does not fit
        a half gets a fresh pool instead (``_relayout`` with the plan)."""
        o = self._plan_out
        eo = o["evict_offsets_2d"]
        changed = ((o["load_lens_2d"] > 0) | (eo[:, 1:] > eo[:, :-1])).any(dim=1).tolist()
        bases_all, caps_all, lens_all, src_all, cu_all = [], [], [], [], []
        for l in range(self.num_layers):
            lens = [x - 1 for x in new_lens_all[l]]  # the step's append comes after the move
            bases, caps = list(self._base_list[l]), list(self._cap_list[l])
            kind = "none"
            if changed[l]:
                t0 = t = self._half_start[l] + self._flip[l] * self._half_size[l]
                for f in self._classb_segs[l]:
                    bases[f], caps[f] = t, _round8(lens[f] + self.slack_rows)
                    t += caps[f]
                kind = "move" if t - t0 <= self._half_size[l] else "relayout"
            self._moves[l] = (kind, bases, caps, lens)
            bases_all.append(bases)
            caps_all.append(caps)
            lens_all.append(lens)
            src_all.append(self.seq_lens[l])
            cu_all.append(_build_cu_seqlens_list(lens))
        return [torch.tensor(bases_all, dtype=torch.int64), torch.tensor(caps_all, dtype=torch.int32),
                torch.tensor(lens_all, dtype=torch.int32), torch.tensor(src_all, dtype=torch.int32),
                torch.tensor(cu_all, dtype=torch.int32)]

    def _move_class_b(self, layer_idx: int, bases: list[int], caps: list[int], lens: list[int]) -> None:
        """The layer's class-B segments, compacted with their loads, into the
        free half of the flip region (disjoint from every segment's rows)."""
        l = layer_idx
        bdev, cdev, ldev, sdev, cudev = self._move_dev
        k, v = self.layer_k[l], self.layer_v[l]
        segs = self._classb_segs[l]
        compact_segments(k, v, k, v, self._classb_segs_dev[l], self.seg_base[l], sdev[l], bdev[l], ldev[l],
                         self._pending_gpu_k, self._pending_gpu_v, self._pending_load_starts[l],
                         self._pending_load_lens[l], self._pending_evict_offsets[l], self._pending_evict_starts[l],
                         self._pending_evict_ends[l], max(lens[f] for f in segs), check=False)
        self.seg_base[l], self.seg_cap[l] = bdev[l], cdev[l]
        self._base_list[l], self._cap_list[l] = bases, caps
        self._flip[l] ^= 1
        self._set_lens(l, lens, cu_dev=cudev[l])
        self.layout_counts["relocate"] += 1

    def decode_after_attn(self, layer_idx: int, q: Tensor) -> None:
        """cache.py:517-544: class-A scores, each KV group against its own
        segment (softmax over the whole segment, summed over its heads)."""
        if self._decode_class_a_local is None or not self._decode_after_groups[layer_idx]:
            return
        cu = self.cu_seqlens_k[layer_idx]
        K = self.layer_k[layer_idx]
        base = self.seg_base[layer_idx]
        for qheads, seg_idx in self._decode_after_groups[layer_idx]:
            Q = q[:, qheads, 0, :]
            lo, hi = cu[seg_idx], cu[seg_idx + 1]
            if base is None:
                starts, ends = lo.to(torch.int32), hi.to(torch.int32)
            else:  # physical rows of the slack layout
                b = base[seg_idx]
                starts, ends = b.to(torch.int32), (b + (hi - lo)).to(torch.int32)
            fused_score_accumulate(Q, K, starts, ends, self._decode_audio_starts_b, self._decode_audio_ends_b,
                                   self.score_accumulator, self.score_offsets, max_audio=self._max_audio)

    def fused_decode_attention(self, layer_idx, q_flat, q, k_flat, v_flat, cu_k, scale):
        """cache.py:546-566: foldable class-A layers score inside the
        attention operator; other class-A layers score afterwards."""
        base = self.seg_base[layer_idx]
        rows = self._rows[layer_idx] if base is not None else None
        if self._layer_foldable[layer_idx]:
            return q1_decode_attn_score(q_flat, k_flat, v_flat, cu_k, scale, self._ca_kv_mask_by_layer[layer_idx],
                                        self.num_kv_heads, self._decode_audio_starts_b, self._decode_audio_ends_b,
                                        self.score_accumulator, self.score_offsets, seg_base=base, total_rows=rows,
                                        max_audio=self._max_audio)
        out = decode_attn(q_flat, k_flat, v_flat, cu_k, scale, seg_base=base, total_rows=rows)
        self.decode_after_attn(layer_idx, q)
        return out

    def decode_all_layers_done(self) -> None:
        """cache.py:568-576 (after the last deferred class-A scores)."""
        self._flush_pending_scores()
        self._decode_step += 1
        self.stats.flush_decode_step(self._decode_step)
        if self.stats.enabled and self._decode_step % self.stats.interval == 0:
            self.stats.record_decode(self._decode_step, self._snapshot_cache_stats)
        any_change = self._compute_decode_chunk_update()
        self._prepare_decode_rebuild_if_needed(any_change)
        self.score_accumulator.zero_()

    # ---------------------------------------------------------------- planning
    def _topk_scores_async(self):
        """Top-k chunks of every sample from the accumulator, on the device
        (src/algorithms/wnw_cpp/code/cache.py:160-171): one launch of
        ``wnw_chunk_topk`` (chunk means, k best per sample, -1 where a sample
        has fewer chunks than k), then a copy of the [B, k] choice into pinned
        memory and an event behind it.  Nothing waits here; the handle goes
        to ``_topk_finalize``."""
        if self._tk_k == 0:
            return None
        chunk_topk(self.score_accumulator, self.score_offsets, self._tk_chunk_off, self._tk_s, self._tk_e,
                   self._tk_k, self._tk_out)
        self._tk_host.copy_(self._tk_out, non_blocking=True)
        self._tk_event.record()
        return self._tk_host

    def _topk_finalize(self, pending) -> tuple[Tensor, Tensor]:
        """CSR of the chosen chunks per sample (wnw_cpp/code/cache.py:173-189),
        after waiting for the top-k's event (the launch and its copy only)."""
        if pending is None:
            return torch.empty(0, dtype=torch.int32), torch.zeros(self.batch_size + 1, dtype=torch.int32)
        self._tk_event.synchronize()
        a = pending.numpy()
        keep = a >= 0
        off = np.zeros(a.shape[0] + 1, dtype=np.int32)
        np.cumsum(keep.sum(axis=1), out=off[1:])
        return torch.from_numpy(a[keep].astype(np.int32)), torch.from_numpy(off)

    def _compute_decode_chunk_update(self) -> bool:
        """cache.py:578-593 + the chunk changes (:609-649): top-k per sample
        from this step's scores, then the native plan of every layer (with
        the direct transfer, the plan and the start of its loads in one
        native call)."""
        self._pending_chunk_update = False
        pending = self._topk_scores_async()
        if pending is not None and self._offload == "copy" and self._staging_rows_hint > 0:
            return self._plan_and_start(pending)
        topk, off = self._topk_finalize(pending)
        return self._plan(topk, off)

    def _plan_and_start(self, pending: Tensor) -> bool:
        """``_topk_finalize`` + ``_plan`` + the start of ``_copy_loads``'s
        direct transfer, with the planner and the transfer engine in one
        native call (``wnw_h2d_plan_start_direct``): the time from the top-k
        to the first copy is on every offload step's critical path.  The
        loaded rows' buffers are taken at the plan bound before the wait,
        while the device still runs the step's last layers."""
        dev = self.device
        stream = self._get_transfer_stream()
        if self._h2d is None:
            self._h2d = HostToDevice()
        bound = self._staging_rows_hint
        with torch.cuda.stream(stream):  # the copies into them follow on this stream
            stg_k, stg_v = self._device_stage(bound)
            kv = torch.empty(2, bound, self.head_dim, dtype=self.cpu_restore_k.dtype, device=dev)
        kv.record_stream(torch.cuda.current_stream(dev))
        cuts = [a for a, _ in self._group_layers()] + [self.num_layers]
        self._tk_event.synchronize()
        flag, total, n_ev, n_rg, started = self._h2d.plan_start_direct(
            self._planner, pending, self._plan_out, cuts, self.cpu_restore_k, self.cpu_restore_v, stg_k, stg_v,
            kv[0], kv[1], stream)
        ev_s, ev_e, ranges = self._planner.plan_lists(n_ev, n_rg)
        range_layers = self._planner.range_layers() if total > 0 else None
        self._plan_result = (total, ev_s, ev_e, ranges, range_layers)
        if started:
            self._started_loads = (kv[0, :total], kv[1, :total], self._layer_groups(range_layers)[1])
        return bool(flag)

    def _plan(self, topk: Tensor, off: Tensor) -> bool:
        flag, total, ev_s, ev_e, ranges = self._planner.compute_and_prepare(topk, off, check=False, **self._plan_out)
        self._plan_result = (total, ev_s, ev_e, ranges, self._planner.range_layers() if total > 0 else None)
        return bool(flag)

    def _prepare_decode_rebuild_if_needed(self, any_change: bool, activate: bool = True) -> None:
        """cache.py:595-600."""
        if any_change:
            if activate:
                self._pending_chunk_update = True
            self._prepare_pending_rebuild()

    def _prepare_pending_rebuild(self) -> None:
        """cache.py:756-889 with the native plan: the host rows' transfer
        started first (its gather threads run while the rest is prepared),
        then the per-layer descriptors on the device."""
        total, ev_s, ev_e, ranges, range_layers = self._plan_result
        started, self._started_loads = self._started_loads, None
        self._clear_pending_rebuild_state()
        o = self._plan_out
        dev = self.device
        dt = self.layer_k[0].dtype
        if total > 0 and self._offload == "device":
            self._gather_loads_on_device(total, ranges, o["load_lens_2d"])
        elif total > 0 and started is not None:  # started with the plan (_plan_and_start)
            self._pending_gpu_k, self._pending_gpu_v, group_of = started
            self._pending_layer_events = [("h2d", g) for g in group_of]
        elif total > 0:
            self._copy_loads(total, ranges, range_layers)
        else:
            self._pending_gpu_k = torch.empty(0, self.head_dim, dtype=dt, device=dev)
            self._pending_gpu_v = torch.empty(0, self.head_dim, dtype=dt, device=dev)
        elp, emax, new_lens = o["evict_layer_ptr"].tolist(), o["evict_max"].tolist(), o["new_lens_2d"].tolist()
        # every descriptor of the plan (and of the slack layout's moves) in
        # one host->device copy
        host = [o["load_starts_2d"], o["load_lens_2d"], o["cu_new_2d"], o["evict_offsets_2d"], ev_s, ev_e]
        moves = self._plan_slack_moves(new_lens) if self.slack_layout else []
        devs = _to_device_many(host + moves, dev)
        ls, ll, cun, eoff = (t.unbind(0) for t in devs[:4])
        evs, eve = devs[4], devs[5]
        for l in range(self.num_layers):
            self._pending_load_starts[l], self._pending_load_lens[l], self._pending_cu_new[l] = ls[l], ll[l], cun[l]
            self._pending_evict_offsets[l] = eoff[l]
            self._pending_evict_max[l] = emax[l]
            self._pending_new_lens[l] = new_lens[l]
            lo, hi = elp[l], elp[l + 1]
            self._pending_evict_starts[l] = evs[lo:hi] if hi > lo else self._empty_i32
            self._pending_evict_ends[l] = eve[lo:hi] if hi > lo else self._empty_i32
        if moves:
            self._move_dev = tuple(t.unbind(0) for t in devs[6:])
        self._segments_changed_ranges = ranges
        if total > 0 and self._record_plan_transfers and self.stats.enabled:
            # cache.py:816-820: host rows loaded per sample (K and V)
            per_row = self.head_dim * 2 * self.cpu_restore_k.element_size()
            lens = o["load_lens_2d"].view(self.num_layers, self.batch_size, self.num_kv_heads).sum(dim=(0, 2))
            for b, n in enumerate(lens.tolist()):
                if n > 0:
                    self.stats.record_cpu_gpu_transfer(b, c2g_tokens=int(n), c2g_bytes=int(n) * per_row)

    def _gather_loads_on_device(self, total: int, ranges: Tensor, load_lens_2d: Tensor) -> None:
        """The plan's host ranges read by the device straight from the pinned
        restore arrays (no host gather, no staging), on the transfer stream in
        a few launches of consecutive layers with an event each: a layer's
        rebuild waits only for its own launch, so later layers' copies overlap
        earlier layers' compute.  Ranges are in transfer order (layer, sample,
        head, segment), so each layer's rows and ranges are contiguous."""
        dev = self.device
        lens = (ranges[:, 1] - ranges[:, 0]).to(torch.int64)
        dst = torch.zeros(ranges.shape[0] + 1, dtype=torch.int64)
        torch.cumsum(lens, 0, out=dst[1:])
        layer_rows = load_lens_2d.to(torch.int64).sum(dim=1)
        bounds = torch.searchsorted(dst, torch.cumsum(layer_rows, 0)).tolist()
        compute = torch.cuda.current_stream(dev)
        stream = self._get_transfer_stream()
        events = [None] * self.num_layers
        with torch.cuda.stream(stream):
            rg, do = _to_device_many([ranges, dst], dev)
            pk = torch.empty(total, self.head_dim, dtype=self.cpu_restore_k.dtype, device=dev)
            pv = torch.empty(total, self.head_dim, dtype=self.cpu_restore_v.dtype, device=dev)
            r0 = 0
            for l0, l1 in self._group_layers():
                r1 = bounds[l1 - 1]
                if r1 > r0:
                    gather_host_rows(self.cpu_restore_k, self.cpu_restore_v, rg, do, r0, r1, pk, pv)
                    ev = torch.cuda.Event()
                    ev.record(stream)
                    events[l0:l1] = [ev] * (l1 - l0)
                r0 = r1
        for t in (pk, pv, rg, do):
            t.record_stream(compute)
        self._pending_gpu_k, self._pending_gpu_v = pk, pv
        self._pending_layer_events = events
        self._waited_events = set()  # these events are new (an id could repeat a dropped one's)

    def _layer_groups(self, range_layers: list[int]) -> tuple[list[int], list[int]]:
        """Groups of consecutive layers for a plan's loads: the range index
        bounds of each group and each layer's group, from the planner's layer
        pointer into its ranges (transfer order (layer, sample, head,
        segment): each layer's ranges are contiguous)."""
        bounds, group_of = [0], []
        for l0, l1 in self._group_layers():
            bounds.append(range_layers[l1])
            group_of += [len(bounds) - 2] * (l1 - l0)
        return bounds, group_of

    def _group_layers(self) -> list[tuple[int, int]]:
        """Layer spans of the load groups: a short first group (its rows
        arrive early), a short last group (its layers are what runs after
        the plan's last copy) and the other layers split evenly over the
        groups between; the short groups hold a tenth of the layers (at
        least one)."""
        L, n = self.num_layers, max(1, min(self._load_groups, self.num_layers))
        if n == 1:
            return [(0, L)]
        edge = max(1, L // 10)
        if n == 2:
            return [(0, edge), (edge, L)]
        lo, hi, m = edge, L - edge, n - 2
        cuts = [0] + [lo + (hi - lo) * g // m for g in range(m + 1)] + [L]
        return [(a, b) for a, b in zip(cuts[:-1], cuts[1:]) if b > a]

    def _copy_loads(self, total: int, ranges: Tensor, range_layers: list[int]) -> None:
        """The plan's host ranges to the device through the transfer engine,
        group of layers by group on the transfer stream, a layer's rebuild
        waiting for its own group only: copied by the DMA engines straight
        from the pinned restore rows into a device stage and put in transfer
        order by a kernel ("copy"), or gathered by host threads into a pinned
        staging pair that the DMA engines copy ("staged").  Returns without
        waiting."""
        dev = self.device
        bounds, group_of = self._layer_groups(range_layers)
        stream = self._get_transfer_stream()
        if self._h2d is None:
            self._h2d = HostToDevice()
        direct = self._offload == "copy"
        with torch.cuda.stream(stream):  # the copies into them follow on this stream
            if direct:
                stg_k, stg_v = self._device_stage(total)
            kv = torch.empty(2, total, self.head_dim, dtype=self.cpu_restore_k.dtype, device=dev)
        kv.record_stream(torch.cuda.current_stream(dev))
        pk, pv = kv[0], kv[1]
        if direct:
            self._h2d.start_direct(self.cpu_restore_k, self.cpu_restore_v, ranges, bounds, stg_k, stg_v, pk, pv,
                                   stream, check=False)
        else:
            stg_k, stg_v = self._engine_staging(total)
            self._h2d.start(self.cpu_restore_k, self.cpu_restore_v, ranges.to(torch.int32), bounds, stg_k, stg_v,
                            pk, pv, stream)
        self._pending_gpu_k, self._pending_gpu_v = pk, pv
        self._pending_layer_events = [("h2d", g) for g in group_of]

    def _device_stage(self, rows: int) -> tuple[Tensor, Tensor]:
        """The direct transfer's device stage (K and V rows, used on the
        transfer stream only, where it is allocated): sized once by the bound
        on a plan's rows, grown past it on demand (a new allocation on the
        transfer stream, so the old rows stay untouched until the copies
        queued before it are done)."""
        if self._stage is None or self._stage[0].shape[0] < rows:
            cap = max(rows, self._staging_rows_hint)
            if self._stage is not None:
                cap = max(cap, 2 * self._stage[0].shape[0])
            dt = self.cpu_restore_k.dtype
            with torch.cuda.stream(self._get_transfer_stream()):
                self._stage = tuple(torch.empty(cap, self.head_dim, dtype=dt, device=self.device) for _ in range(2))
        return self._stage

    def _plan_rows_bound(self) -> int:
        """An upper bound on the host rows one plan loads: per (layer, sample,
        class-B head), at most ``top_k_chunks`` chunks of the sample's widest
        chunk, each segment with that head's most offloaded rows (capped by
        the head's offloaded rows).  Sizes the staging pairs once."""
        k = self.config.top_k_chunks
        total = 0
        for l in range(self.num_layers):
            for b in range(self.batch_size):
                width = max((len(c) for c in self.chunk_to_segs[b]), default=0)
                for h in range(self.num_kv_heads):
                    rows = [m.cpu_end - m.cpu_start for m in self.restore_meta[l][b][h] if m is not None]
                    if rows:
                        total += min(sum(rows), k * width * max(rows))
        return total

    def _engine_staging(self, rows: int) -> tuple[Tensor, Tensor]:
        """The next of two pinned staging pairs (used in turn, one per plan,
        as the engine alternates: a plan's gather waits inside the engine for
        the copies that used its pair two plans ago), holding at least
        ``rows`` rows: first sized by the bound on a plan's rows, grown to the
        next power of two past it (cache.py:128-134 grows its one staging
        buffer the same way)."""
        i = self._staging_turn
        self._staging_turn ^= 1
        pair = self._staging[i]
        if pair is None or pair[0].shape[0] < rows:
            if pair is not None:  # the engine's copies may still read the old pair: drain them before it goes
                self._h2d.join()
                self._get_transfer_stream().synchronize()
            cap = max(rows, self._staging_rows_hint) if pair is None else \
                min(1 << max(0, rows - 1).bit_length(), max(rows, self.cpu_restore_k.shape[0]))
            dt = self.cpu_restore_k.dtype
            pair = (torch.empty(cap, self.head_dim, dtype=dt, pin_memory=True),
                    torch.empty(cap, self.head_dim, dtype=dt, pin_memory=True))
            self._staging[i] = pair
        return pair

    def _rebuild_append_layer(self, layer_idx: int, new_k: Tensor, new_v: Tensor):
        """cache.py:716-754: compaction + load + append in one launch."""
        self._wait_loads(layer_idx)
        nk = new_k.squeeze(2).reshape(-1, self.head_dim)
        nv = new_v.squeeze(2).reshape(-1, self.head_dim)
        cu_new = self._pending_cu_new[layer_idx]
        new_lens = self._pending_new_lens[layer_idx]
        k, v = rebuild_append_kv(
            self.layer_k[layer_idx], self.layer_v[layer_idx], nk, nv, self._pending_gpu_k, self._pending_gpu_v,
            self.cu_seqlens_k[layer_idx], cu_new, self._pending_load_starts[layer_idx],
            self._pending_load_lens[layer_idx], self._pending_evict_offsets[layer_idx],
            self._pending_evict_starts[layer_idx], self._pending_evict_ends[layer_idx],
            self._pending_evict_max[layer_idx], total_out=sum(new_lens))
        self._finish_layer(layer_idx, k, v, cu_new, new_lens)
        return k, v, cu_new, max(new_lens)

    def _apply_chunk_update_to_layer(self, layer_idx: int) -> None:
        """cache.py:891-1010 (the fallback without the fused append): the
        same compaction and load, then the ordinary append follows."""
        self._wait_loads(layer_idx)
        lens_after = [x - 1 for x in self._pending_new_lens[layer_idx]]  # the append comes next
        cu_mid = _build_cu_seqlens(lens_after, self.device)
        k, v = _compact_no_append(self, layer_idx, cu_mid, lens_after)
        self._finish_layer(layer_idx, k, v, cu_mid, lens_after)

    def _wait_loads(self, layer_idx: int) -> None:
        """The compute stream waits for the copy of this layer's loaded rows
        (cache.py:719-721 waits once for the whole transfer)."""
        ev = self._pending_layer_events[layer_idx]
        if ev is None:
            return
        if isinstance(ev, tuple):  # a group of the transfer engine: one wait per group
            if ev[1] not in self._waited_groups:
                self._h2d.wait(ev[1], torch.cuda.current_stream(self.device))
                self._waited_groups.add(ev[1])
        else:  # a group's event: the stream waits once per group (its later work is ordered after)
            key = (id(ev), _lib.stream_of(self.device).value)
            if key not in self._waited_events:
                torch.cuda.current_stream(self.device).wait_event(ev)
                self._waited_events.add(key)
        self._pending_layer_events[layer_idx] = None

    def _finish_layer(self, layer_idx, k, v, cu_new, new_lens) -> None:
        self.layer_k[layer_idx], self.layer_v[layer_idx] = k, v
        self.seq_lens[layer_idx] = list(new_lens)
        self.cu_seqlens_k[layer_idx] = cu_new
        self.cu_seqlens_list[layer_idx] = _build_cu_seqlens_list(new_lens)
        self._rows[layer_idx] = self.cu_seqlens_list[layer_idx][-1]
        self._max_len[layer_idx] = max(new_lens, default=0)
        self._pending_layers_applied += 1
        if self._pending_layers_applied == self.num_layers:
            self._pending_chunk_update = False
            self._clear_pending_rebuild_state()

    # ------------------------------------------------------------------ stats
    def _snapshot_cache_stats(self, step: int = -1) -> list[dict]:
        """cache.py:1013-1081: per-sample token accounting.  Audio rows on the
        GPU are a segment's rows minus its text rows (text before the audio,
        text after it in the prompt, one row per decode step); retention is
        relative to L * H * num_audio."""
        if self._planner is not None:
            self.loaded_segments = [set(self._planner.get_loaded_segments(b)) for b in range(self.batch_size)]
        L, H = self.num_layers, self.num_kv_heads
        cpu_total = self.cpu_restore_k.shape[0] if self.cpu_restore_k is not None else 0
        text_per_seg = self._decode_step if self.prefilled else 0
        prefill_len = (self._seq_lengths[0] - self._decode_step) if self._seq_lengths else 0
        out = []
        for b in range(self.batch_size):
            a0, a1 = self._audio_starts_list[b], self._audio_ends_list[b]
            num_audio = a1 - a0
            full_audio = L * H * num_audio
            non_audio = a0 + max(0, max(0, prefill_len - self.pad_lens_list[b]) - a1)
            gpu_audio = gpu_total = 0
            per_layer = []
            for l in range(L):
                if self.seq_lens[l] is None:
                    per_layer.append(0)
                    continue
                layer_audio = 0
                for h in range(H):
                    n = self.seq_lens[l][b * H + h]
                    gpu_total += n
                    layer_audio += max(0, n - non_audio - text_per_seg)
                gpu_audio += layer_audio
                per_layer.append(layer_audio)
            metas = [(l, h) for l in range(L) for h in range(H) if self.config.is_class_b(l, h)]
            cpu_restore = sum(m.cpu_end - m.cpu_start for l, h in metas for m in self.restore_meta[l][b][h]
                              if m is not None) if self.restore_meta else 0
            cpu_loaded = 0
            if self.prefilled:
                for si in self.loaded_segments[b]:
                    for l, h in metas:
                        m = self.restore_meta[l][b][h][si]
                        if m is not None:
                            cpu_loaded += m.cpu_end - m.cpu_start
            out.append({
                "step": step,
                "num_audio": num_audio,
                "gpu_audio_tokens": gpu_audio,
                "gpu_total_tokens": gpu_total,
                "audio_retention": gpu_audio / full_audio if full_audio > 0 else 1.0,
                "per_layer_audio_tokens": per_layer,
                "cpu_total_tokens": cpu_total,
                "cpu_loaded_tokens": cpu_loaded,
                "cpu_restore_tokens": cpu_restore,
                "gpu_plus_cpu_retention": (gpu_audio + cpu_restore) / full_audio if full_audio > 0 else 1.0,
            })
        return out

    def get_snapshot_stats(self, step: int = -1) -> list[dict]:
        """cache.py:1082-1084."""
        return self._snapshot_cache_stats(step=step)

    def get_compression_stats(self) -> list[dict]:
        """cache.py:1086-1088."""
        return self._snapshot_cache_stats(step=-1)

    def get_all_stats(self) -> list[dict]:
        return self.stats.get_all_stats()

    def collect_stats(self, interval: int = 20) -> None:
        self.stats.set_interval(interval)


def _compact_no_append(cache: WnWCache, layer_idx: int, cu_mid: Tensor, lens_after: list[int]):
    """Compaction + load of one layer without the new row (dense source and
    destination, every segment listed): the kernel of wnw_compact_segments."""
    from .kernels import compact_segments
    N = cache.batch_size * cache.num_kv_heads
    dev = cache.device
    old = cache.layer_k[layer_idx]
    k = torch.empty(sum(lens_after), cache.head_dim, dtype=old.dtype, device=dev)
    v = torch.empty_like(k)
    cu_old = cache.cu_seqlens_k[layer_idx]
    compact_segments(
        cache.layer_k[layer_idx], cache.layer_v[layer_idx], k, v, torch.arange(N, dtype=torch.int32, device=dev),
        cu_old[:-1].to(torch.int64), (cu_old[1:] - cu_old[:-1]).to(torch.int32), cu_mid[:-1].to(torch.int64),
        _to_device(lens_after, torch.int32, dev), cache._pending_gpu_k, cache._pending_gpu_v,
        cache._pending_load_starts[layer_idx], cache._pending_load_lens[layer_idx],
        cache._pending_evict_offsets[layer_idx], cache._pending_evict_starts[layer_idx],
        cache._pending_evict_ends[layer_idx], max(lens_after) if lens_after else 0)
    return k, v

"""Compaction and scoring kernels of the WnW cache.

Mirrors ``rebuild_append_kv`` and ``fused_score_accumulate`` of
``src/algorithms/wnw/code/kernels.py``: same arguments and results, computed
by the gfx950 kernels ``wnw_rebuild_append_kv`` and
``wnw_fused_score_accumulate`` of ``libwnw_amd.so``.
"""
from __future__ import annotations

import torch

from .. import _lib


def rebuild_append_kv(
    old_k: torch.Tensor,
    old_v: torch.Tensor,
    new_k: torch.Tensor,
    new_v: torch.Tensor,
    load_k: torch.Tensor,
    load_v: torch.Tensor,
    old_cu: torch.Tensor,
    new_cu: torch.Tensor,
    load_starts: torch.Tensor,
    load_lens: torch.Tensor,
    evict_offsets: torch.Tensor,
    evict_starts: torch.Tensor,
    evict_ends: torch.Tensor,
    max_evict: int,
    *,
    total_out: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Compaction + load + append of one layer's K and V in one launch.

    Reference: ``rebuild_append_kv`` (src/algorithms/wnw/code/kernels.py:375-404).
    ``total_out`` (= new_cu[-1]) may be given by a caller that knows it; the
    reference always reads it back from the device (kernels.py:393).
    """
    _lib.require_gpu(old_k, old_v, new_k, new_v, old_cu, new_cu, load_starts, load_lens, evict_offsets)
    n = new_k.shape[0]
    d = old_k.shape[1]
    for name, t in (("old_cu", old_cu), ("new_cu", new_cu), ("evict_offsets", evict_offsets)):
        if t.dtype != torch.int32 or t.numel() != n + 1:
            raise _lib.WnwError(f"{name} must be int32 [N+1]")
    for name, t in (("load_starts", load_starts), ("load_lens", load_lens)):
        if t.dtype != torch.int32 or t.numel() != n:
            raise _lib.WnwError(f"{name} must be int32 [N]")
    if evict_starts.numel() != evict_ends.numel():
        raise _lib.WnwError("evict_starts / evict_ends size mismatch")
    if total_out is None:
        total_out = int(new_cu[-1].item())
    out_k = torch.empty(total_out, d, dtype=old_k.dtype, device=old_k.device)
    out_v = torch.empty(total_out, d, dtype=old_v.dtype, device=old_v.device)
    n_ev = evict_starts.numel()
    # contiguous copies are bound to names so they outlive the launch
    old_k, old_v, new_k, new_v = (t.contiguous() for t in (old_k, old_v, new_k, new_v))
    load_k = load_k.contiguous() if load_k.numel() else None
    load_v = load_v.contiguous() if load_v.numel() else None
    old_cu, new_cu, load_starts, load_lens, evict_offsets = (
        t.contiguous() for t in (old_cu, new_cu, load_starts, load_lens, evict_offsets))
    evict_starts = evict_starts.contiguous() if n_ev else None
    evict_ends = evict_ends.contiguous() if n_ev else None
    _lib.ensure_init(old_k.device)
    _lib.check(_lib.lib().wnw_rebuild_append_kv(
        _lib.ptr(old_k), _lib.ptr(old_v), _lib.ptr(new_k), _lib.ptr(new_v), _lib.ptr(load_k), _lib.ptr(load_v),
        _lib.ptr(old_cu), _lib.ptr(new_cu), _lib.ptr(load_starts), _lib.ptr(load_lens), _lib.ptr(evict_offsets),
        _lib.ptr(evict_starts), _lib.ptr(evict_ends), n_ev, n,
        old_k.shape[0], 0 if load_k is None else load_k.shape[0], total_out, int(max_evict), d,
        _lib.dtype_code(old_k.dtype), _lib.ptr(out_k), _lib.ptr(out_v), _lib.stream_of(old_k.device)),
        "rebuild_append_kv")
    return out_k, out_v


_score_ws: dict[tuple[int, int], torch.Tensor] = {}


def fused_score_accumulate(
    Q: torch.Tensor,
    K: torch.Tensor,
    seg_starts: torch.Tensor,
    seg_ends: torch.Tensor,
    audio_starts: torch.Tensor,
    audio_ends: torch.Tensor,
    accumulator: torch.Tensor,
    accum_offsets: torch.Tensor,
    *,
    max_audio: int | None = None,
    scale: float | None = None,
) -> None:
    """Full-segment softmax of each item's query heads, summed over the
    heads, added to the accumulator at the audio rows.

    Reference: ``fused_score_accumulate`` (src/algorithms/wnw/code/
    kernels.py:302-348; ``_fused_score_pytorch`` :351-370 for any head
    count).  Q: [S, nh, d]; K: [rows, d]; seg_starts/seg_ends [S] (rows of
    K); audio_starts/audio_ends [S] relative to seg_starts; accumulator
    float32, updated in place at ``accum_offsets[i] + j``.  ``scale``
    defaults to d^-0.5 like the reference; ``max_audio`` (largest audio
    range) is read back from the device when not given.
    """
    _lib.require_gpu(Q, K, seg_starts, seg_ends, audio_starts, audio_ends, accumulator, accum_offsets)
    S, nh, d = Q.shape
    for name, t, n in (("seg_starts", seg_starts, S), ("seg_ends", seg_ends, S), ("audio_starts", audio_starts, S),
                       ("audio_ends", audio_ends, S), ("accum_offsets", accum_offsets, None)):
        if t.dtype != torch.int32 or (n is not None and t.numel() != n):
            raise _lib.WnwError(f"{name} must be int32 [{n if n is not None else 'S + 1'}]")
    if accum_offsets.numel() < S + 1:
        raise _lib.WnwError("accum_offsets must have at least S + 1 entries")
    if accumulator.dtype != torch.float32 or not accumulator.is_contiguous():
        raise _lib.WnwError("accumulator must be a contiguous float32 tensor")
    if K.dim() != 2 or K.shape[1] != d or K.dtype != Q.dtype:
        raise _lib.WnwError("K must be [rows, d] with the dtype of Q")
    if K.shape[0] > 0 and (K.stride(1) != 1 or K.stride(0) != d):
        raise _lib.WnwError("K rows must be contiguous")
    if S == 0:
        return
    if max_audio is None:
        max_audio = int((audio_ends - audio_starts).max().item())
    if max_audio <= 0:
        return
    scale = d ** -0.5 if scale is None else float(scale)
    Q = Q.contiguous()
    seg_starts, seg_ends, audio_starts, audio_ends, accum_offsets = (
        t.contiguous() for t in (seg_starts, seg_ends, audio_starts, audio_ends, accum_offsets))
    need = int(_lib.lib().wnw_fused_score_workspace_bytes(S, nh))
    dev = Q.device
    key = (dev.index if dev.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(dev).cuda_stream)
    ws = _score_ws.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty(max(need, 1 << 16), dtype=torch.uint8, device=dev)
        _score_ws[key] = ws
    _lib.ensure_init(dev)
    _lib.check(_lib.lib().wnw_fused_score_accumulate(
        _lib.ptr(Q), _lib.ptr(K), _lib.ptr(seg_starts), _lib.ptr(seg_ends), _lib.ptr(audio_starts),
        _lib.ptr(audio_ends), _lib.ptr(accumulator), _lib.ptr(accum_offsets), S, nh, d, K.shape[0],
        accumulator.numel(), int(max_audio), scale, _lib.dtype_code(Q.dtype), _lib.ptr(ws), ws.numel(),
        _lib.stream_of(dev)), "fused_score_accumulate")


def compact_segments(
    src_k: torch.Tensor,
    src_v: torch.Tensor,
    dst_k: torch.Tensor,
    dst_v: torch.Tensor,
    seg_list: torch.Tensor,
    src_base: torch.Tensor,
    src_len: torch.Tensor,
    dst_base: torch.Tensor,
    new_len: torch.Tensor,
    load_k: torch.Tensor,
    load_v: torch.Tensor,
    load_starts: torch.Tensor,
    load_lens: torch.Tensor,
    evict_offsets: torch.Tensor,
    evict_starts: torch.Tensor,
    evict_ends: torch.Tensor,
    max_new_len: int,
    *,
    new_k: torch.Tensor | None = None,
    new_v: torch.Tensor | None = None,
    check: bool = True,
) -> None:
    """Compaction + load (+ optional append) of the listed segments between
    physically addressed layouts (``wnw_compact_segments``).  With
    ``new_k=None`` no row is appended: the compaction step of the reference's
    out-of-place fallback (src/algorithms/wnw/code/cache.py:891-1010).
    ``check=False`` skips the Python-side dtype / device / shape checks (the
    library still checks every bound): for callers whose arguments are
    contiguous tensors of the right dtypes by construction, per layer and
    step."""
    n = src_base.numel()
    if check:
        _lib.require_gpu(src_k, src_v, dst_k, dst_v, seg_list, src_base, src_len, dst_base, new_len, load_starts,
                         load_lens, evict_offsets)
        for name, t, dt in (("seg_list", seg_list, torch.int32), ("src_base", src_base, torch.int64),
                            ("src_len", src_len, torch.int32), ("dst_base", dst_base, torch.int64),
                            ("new_len", new_len, torch.int32), ("load_starts", load_starts, torch.int32),
                            ("load_lens", load_lens, torch.int32), ("evict_offsets", evict_offsets, torch.int32)):
            if t.dtype != dt:
                raise _lib.WnwError(f"{name} must be {dt}")
        if evict_offsets.numel() != n + 1:
            raise _lib.WnwError("evict_offsets must be int32 [N+1]")
        keep = [t.contiguous() if t is not None and t.numel() else None for t in
                (new_k, new_v, load_k, load_v, seg_list, src_base, src_len, dst_base, new_len, load_starts,
                 load_lens, evict_offsets, evict_starts, evict_ends)]
        _lib.ensure_init(src_k.device)
    else:
        keep = [t if t is not None and t.numel() else None for t in
                (new_k, new_v, load_k, load_v, seg_list, src_base, src_len, dst_base, new_len, load_starts,
                 load_lens, evict_offsets, evict_starts, evict_ends)]
    with_new = new_k is not None
    nk, nv, lk, lv, sl, sb, sn, db, nl, ls, ll, eo, es, ee = keep
    n_ev = 0 if es is None else es.numel()
    P = _lib.ptr
    _lib.check(_lib.lib().wnw_compact_segments(
        P(src_k), P(src_v), P(dst_k), P(dst_v), P(nk), P(nv), P(lk), P(lv), P(sl), seg_list.numel(), n,
        int(max_new_len), P(sb), P(sn), P(db), P(nl), P(ls), P(ll), P(eo), P(es), P(ee), n_ev, 1 if with_new else 0,
        src_k.shape[0], dst_k.shape[0], 0 if lk is None else lk.shape[0], src_k.shape[1],
        _lib.dtype_code(src_k.dtype), _lib.stream_of(src_k.device)), "compact_segments")


def chunk_topk(score_acc: torch.Tensor, score_offsets: torch.Tensor, chunk_offsets: torch.Tensor,
               chunk_starts: torch.Tensor, chunk_ends: torch.Tensor, k: int, out: torch.Tensor) -> torch.Tensor:
    """Each sample's k best chunks by mean score, into ``out`` (int32
    [B, k], -1 past the sample's chunk count), in one launch (``wnw_chunk_topk``).

    The chunk selection of the reference (src/algorithms/wnw/code/
    cache.py:632-649; batched, src/algorithms/wnw_cpp/code/cache.py:160-171).
    ``score_offsets`` [B + 1] bounds each sample's scores in ``score_acc``;
    ``chunk_offsets`` [B + 1] each sample's chunks in ``chunk_starts`` /
    ``chunk_ends`` (token bounds relative to the sample's first score).
    Equal means go to the lower chunk index."""
    _lib.require_gpu(score_acc, score_offsets, chunk_offsets, chunk_starts, chunk_ends, out)
    B = score_offsets.numel() - 1
    for name, t in (("score_offsets", score_offsets), ("chunk_offsets", chunk_offsets),
                    ("chunk_starts", chunk_starts), ("chunk_ends", chunk_ends), ("out", out)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise _lib.WnwError(f"{name} must be a contiguous int32 tensor")
    if score_acc.dtype != torch.float32 or not score_acc.is_contiguous():
        raise _lib.WnwError("score_acc must be a contiguous float32 tensor")
    if chunk_offsets.numel() != B + 1 or out.shape != (B, k) or chunk_starts.numel() != chunk_ends.numel():
        raise _lib.WnwError("chunk_offsets must be [B + 1], out [B, k], chunk_starts / chunk_ends equal")
    _lib.ensure_init(score_acc.device)
    _lib.check(_lib.lib().wnw_chunk_topk(
        _lib.ptr(score_acc), score_acc.numel(), _lib.ptr(score_offsets), B, _lib.ptr(chunk_offsets),
        _lib.ptr(chunk_starts), _lib.ptr(chunk_ends), chunk_starts.numel(), int(k), _lib.ptr(out),
        _lib.stream_of(score_acc.device)), "chunk_topk")
    return out


def host_rows_readable(host_k: torch.Tensor, host_v: torch.Tensor) -> bool:
    """Whether the device can read the two host arrays directly (pinned)."""
    return bool(_lib.lib().wnw_host_rows_readable(_lib.ptr(host_k), _lib.ptr(host_v)))


def gather_host_rows(host_k: torch.Tensor, host_v: torch.Tensor, ranges: torch.Tensor, dst_off: torch.Tensor,
                     r0: int, r1: int, out_k: torch.Tensor, out_v: torch.Tensor) -> None:
    """Rows [ranges[r, 0], ranges[r, 1]) of the pinned host arrays, for r in
    [r0, r1), into rows [dst_off[r], dst_off[r + 1]) of out_k / out_v, on the
    current stream (the device reads host memory itself; it replaces the
    host gather into staging + staging copy of the reference's offload,
    src/algorithms/wnw_cpp/code/planner.cpp:113-122 and cache.py:287-295).
    ``ranges`` int32 [n, 2] and ``dst_off`` int64 [n + 1] live on the device."""
    for t in (host_k, host_v):
        if t.device.type != "cpu" or not t.is_pinned() or not t.is_contiguous() or t.dim() != 2:
            raise _lib.WnwError("host rows must be contiguous 2-D pinned tensors")
    if host_k.shape != host_v.shape or out_k.shape != out_v.shape or out_k.shape[1:] != host_k.shape[1:] \
            or out_k.dtype != host_k.dtype or out_v.dtype != host_v.dtype:
        raise _lib.WnwError("host / output shapes or dtypes differ")
    if ranges.dtype != torch.int32 or dst_off.dtype != torch.int64 or ranges.device != out_k.device \
            or dst_off.device != out_k.device:
        raise _lib.WnwError("ranges must be int32 and dst_off int64, on the outputs' device")
    row_bytes = host_k.shape[1] * host_k.element_size()
    _lib.check(_lib.lib().wnw_gather_host_rows(
        _lib.ptr(host_k), _lib.ptr(host_v), host_k.shape[0], _lib.ptr(ranges), _lib.ptr(dst_off), r0, r1, row_bytes,
        _lib.ptr(out_k), _lib.ptr(out_v), out_k.shape[0], _lib.stream_of(out_k.device)), "gather_host_rows")

"""Compaction kernels of the WnW cache.

Mirrors ``rebuild_append_kv`` of ``src/algorithms/wnw/code/kernels.py``:
same arguments and result, computed by the gfx950 kernel
``wnw_rebuild_append_kv`` of ``libwnw_amd.so``.
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

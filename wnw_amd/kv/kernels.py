"""Append kernels of the flat varlen KV layout.

Mirrors ``src/common/kv/kernels.py`` of the reference: same function name,
arguments and result, computed by the gfx950 kernel ``wnw_interleave_append``
of ``libwnw_amd.so`` instead of Triton.
"""
from __future__ import annotations

import torch

from .. import _lib


def interleave_append(
    old: torch.Tensor,
    new_tokens: torch.Tensor,
    cu_old: torch.Tensor,
    cu_new: torch.Tensor,
) -> torch.Tensor:
    """Append one new token per segment into the flat cache (out of place).

    Reference: ``interleave_append`` (src/common/kv/kernels.py:45-73).

    Args:
        old: [total_old, D] existing flat cache.
        new_tokens: [N, D] one token per segment.
        cu_old: [N+1] int32 cumulative lengths of old segments.
        cu_new: [N+1] int32 cumulative lengths of new segments (each = old + 1).

    Returns: [total_old + N, D], bit-identical to the reference.
    """
    _lib.require_gpu(old, new_tokens, cu_old, cu_new)
    if old.dim() != 2 or new_tokens.dim() != 2 or old.shape[1] != new_tokens.shape[1]:
        raise _lib.WnwError(f"shape mismatch: old {tuple(old.shape)}, new {tuple(new_tokens.shape)}")
    if old.dtype != new_tokens.dtype:
        raise _lib.WnwError("old and new_tokens must share a dtype")
    n = new_tokens.shape[0]
    if cu_old.dtype != torch.int32 or cu_new.dtype != torch.int32 or cu_old.numel() != n + 1 or \
            cu_new.numel() != n + 1:
        raise _lib.WnwError("cu_old / cu_new must be int32 [N+1]")
    old = old.contiguous()  # bound to names: must outlive the launch
    new_tokens = new_tokens.contiguous()
    cu_old = cu_old.contiguous()
    cu_new = cu_new.contiguous()
    d = old.shape[1]
    out = torch.empty(old.shape[0] + n, d, dtype=old.dtype, device=old.device)
    _lib.ensure_init(old.device)
    _lib.check(_lib.lib().wnw_interleave_append(
        _lib.ptr(old), _lib.ptr(new_tokens), _lib.ptr(cu_old), _lib.ptr(cu_new),
        n, old.shape[0], d, _lib.dtype_code(old.dtype), _lib.ptr(out), _lib.stream_of(old.device)),
        "interleave_append")
    return out



def interleave_append_kv(
    old_k: torch.Tensor,
    old_v: torch.Tensor,
    new_k: torch.Tensor,
    new_v: torch.Tensor,
    cu_old: torch.Tensor,
    cu_new: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``interleave_append`` of K and V in one launch (the two calls of
    decode_before_attn, src/algorithms/wnw/code/cache.py:506-507); each
    result is bit-identical to ``interleave_append`` of that tensor."""
    _lib.require_gpu(old_k, old_v, new_k, new_v, cu_old, cu_new)
    if old_k.shape != old_v.shape or new_k.shape != new_v.shape or old_k.dim() != 2 or new_k.dim() != 2 or \
            old_k.shape[1] != new_k.shape[1]:
        raise _lib.WnwError(f"shape mismatch: old {tuple(old_k.shape)}/{tuple(old_v.shape)}, "
                            f"new {tuple(new_k.shape)}/{tuple(new_v.shape)}")
    if not (old_k.dtype == old_v.dtype == new_k.dtype == new_v.dtype):
        raise _lib.WnwError("K and V, old and new, must share a dtype")
    n = new_k.shape[0]
    if cu_old.dtype != torch.int32 or cu_new.dtype != torch.int32 or cu_old.numel() != n + 1 or \
            cu_new.numel() != n + 1:
        raise _lib.WnwError("cu_old / cu_new must be int32 [N+1]")
    old_k, old_v = old_k.contiguous(), old_v.contiguous()  # bound to names: must outlive the launch
    new_k, new_v = new_k.contiguous(), new_v.contiguous()
    cu_old, cu_new = cu_old.contiguous(), cu_new.contiguous()
    d = old_k.shape[1]
    out_k = torch.empty(old_k.shape[0] + n, d, dtype=old_k.dtype, device=old_k.device)
    out_v = torch.empty_like(out_k)
    _lib.ensure_init(old_k.device)
    _lib.check(_lib.lib().wnw_interleave_append_kv(
        _lib.ptr(old_k), _lib.ptr(old_v), _lib.ptr(new_k), _lib.ptr(new_v), _lib.ptr(cu_old), _lib.ptr(cu_new),
        n, old_k.shape[0], d, _lib.dtype_code(old_k.dtype), _lib.ptr(out_k), _lib.ptr(out_v),
        _lib.stream_of(old_k.device)), "interleave_append_kv")
    return out_k, out_v

def append_inplace(
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    new_k: torch.Tensor,
    new_v: torch.Tensor,
    cu_old: torch.Tensor,
    cu_new: torch.Tensor,
    seg_base: torch.Tensor,
    seg_cap: torch.Tensor,
) -> None:
    """Write one new row per segment into its slack and set cu_new = cu_old + arange.

    No reference counterpart: replaces the two full-layer copies of
    ``decode_before_attn`` (src/algorithms/wnw/code/cache.py:497-515) for a
    cache that keeps per-segment slack.
    """
    _lib.require_gpu(k_pool, v_pool, new_k, new_v, cu_old, cu_new, seg_base, seg_cap)
    n = new_k.shape[0]
    d = k_pool.shape[1]
    if seg_base.dtype != torch.int64 or seg_cap.dtype != torch.int32 or cu_new.dtype != torch.int32:
        raise _lib.WnwError("seg_base must be int64, seg_cap/cu int32")
    new_k = new_k.contiguous()  # bound to names: must outlive the launch
    new_v = new_v.contiguous()
    _lib.ensure_init(k_pool.device)
    _lib.check(_lib.lib().wnw_append_inplace(
        _lib.ptr(k_pool), _lib.ptr(v_pool), _lib.ptr(new_k), _lib.ptr(new_v),
        _lib.ptr(cu_old), _lib.ptr(cu_new), _lib.ptr(seg_base), _lib.ptr(seg_cap), n, k_pool.shape[0], d,
        _lib.dtype_code(k_pool.dtype), _lib.stream_of(k_pool.device)), "append_inplace")

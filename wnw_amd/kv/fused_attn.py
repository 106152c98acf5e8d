"""q = 1 GQA decode attention over the flat varlen KV layout.

Mirrors ``src/common/kv/fused_attn.py`` of the reference (``q1_decode_attn``)
and stands in for its default ``varlen_attn`` call
(src/algorithms/wnw/code/session.py:90-106).  The computation is the gfx950
split-K kernel ``wnw_decode_attn`` of ``libwnw_amd.so``: the rows of all
segments are divided evenly over the workgroups, partial softmax states are
merged by the last workgroup to finish a segment, so ragged segment lengths
never leave CUs idle (the reference runs one program per segment).
"""
from __future__ import annotations

import torch

from .. import _lib


class AttnWorkspace:
    """Split-K workspace of one (device, stream): partials + arrival counters.

    The kernel leaves the counters at zero after every launch, so a
    workspace is cleared once at allocation and then reused; two streams
    must not share one (launches on one stream are ordered).
    """

    def __init__(self, device: torch.device):
        self.device = device
        self.buf: torch.Tensor | None = None
        self.cleared_for = -1  # n_seg of the layout whose counters are known to be zero
        self._need: dict[tuple, int] = {}  # bytes the library asks for, per layout

    def get(self, n_seg: int, group: int, head_dim: int, score: bool = False,
            max_audio: int = 0) -> tuple[torch.Tensor, int]:
        """Buffer and its size; ``score`` adds room for the softmax
        normalisers of ``wnw_decode_attn_score`` and, with ``max_audio`` > 0,
        for the logits of the scored audio rows."""
        key = (n_seg, group, head_dim, score, max_audio)
        need = self._need.get(key)
        if need is None:
            if score:
                need = int(_lib.lib().wnw_decode_attn_score_workspace_bytes(n_seg, group, head_dim, max_audio))
            else:
                need = int(_lib.lib().wnw_decode_attn_workspace_bytes(n_seg, group, head_dim))
            if need < 0:
                raise _lib.WnwError("bad workspace query")
            self._need[key] = need
        if self.buf is None or self.buf.numel() < need:
            size = max(need, 1 << 20)
            self.buf = torch.empty(size, dtype=torch.uint8, device=self.device)
            self.cleared_for = -1
        if n_seg != self.cleared_for:
            # counters sit at the front, sized by n_seg, and partials follow
            # them: under another n_seg, bytes that held partials become
            # counters (and the reverse), so the buffer is cleared again.
            _lib.check(_lib.lib().wnw_workspace_init(_lib.ptr(self.buf), self.buf.numel(),
                                                     _lib.stream_of(self.device)), "workspace init")
            self.cleared_for = n_seg
        return self.buf, self.buf.numel()


_workspaces: dict[tuple[int, int], AttnWorkspace] = {}


def workspace_for(device: torch.device) -> AttnWorkspace:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, _lib.raw_stream(device))
    ws = _workspaces.get(key)
    if ws is None:
        ws = AttnWorkspace(torch.device("cuda", idx))
        _workspaces[key] = ws
    return ws


_KERNELS = {"auto": _lib.ATTN_AUTO, "mfma": _lib.ATTN_MFMA, "valu": _lib.ATTN_VALU,
            "stream": _lib.ATTN_STREAM}


def decode_attn(
    q_flat: torch.Tensor,
    k_flat: torch.Tensor,
    v_flat: torch.Tensor,
    cu_k: torch.Tensor,
    scale: float,
    *,
    seg_base: torch.Tensor | None = None,
    total_rows: int | None = None,
    out: torch.Tensor | None = None,
    workspace: AttnWorkspace | None = None,
    kernel: str = "auto",
    n_wg: int = 0,
    append: tuple | None = None,
    validate: bool = True,
) -> torch.Tensor:
    """Decode attention with the layout extensions of this package.

    ``seg_base`` (int64 [N]) gives each segment's physical first row in
    ``k_flat``/``v_flat`` (slack layout: segments anywhere, in any order).
    The kernel splits the logical rows ``[0, cu_k[-1])`` over its
    workgroups, reading ``cu_k[-1]`` on the device; ``total_rows``, an
    estimate of it, only sizes the grid (required with ``seg_base``; without
    it the dense layout's ``k_flat.shape[0]``).

    ``append=(new_k [N, D], new_v, cu_new int32 [N+1], seg_cap int32 [N])``
    first appends one row per segment in place (``k_flat``/``v_flat`` are the
    pools, ``cu_k`` the offsets before the append, ``total_rows`` an estimate
    of the rows after it) and attends over the appended segments; the
    streaming kernel does both in one launch.  ``cu_new`` receives
    ``cu_k + arange(N + 1)``.
    """
    if validate:
        q_flat, cu_k = _check_attn(q_flat, k_flat, v_flat, cu_k, seg_base, total_rows)
    nseg, g, d = q_flat.shape
    if out is None:
        out = torch.empty(nseg, g, d, device=q_flat.device, dtype=q_flat.dtype)
    rows = k_flat.shape[0] if total_rows is None else int(total_rows)
    _lib.ensure_init(q_flat.device)
    ws = workspace if workspace is not None else workspace_for(q_flat.device)
    buf, nbytes = ws.get(nseg, g, d)
    if append is not None:
        if kernel != "auto" or n_wg:
            raise _lib.WnwError("the fused append runs the AUTO kernel choice and grid")
        new_k, new_v, cu_new, seg_cap = (_check_append(append, nseg, d, k_flat.dtype, cu_k, seg_base) if validate
                                         else append)
        _lib.check(_lib.lib().wnw_decode_attn_append(
            _lib.ptr(q_flat), _lib.ptr(k_flat), _lib.ptr(v_flat), _lib.ptr(new_k), _lib.ptr(new_v), _lib.ptr(cu_k),
            _lib.ptr(cu_new), _lib.ptr(seg_base), _lib.ptr(seg_cap), nseg, g, d, rows, k_flat.shape[0], float(scale),
            _lib.dtype_code(q_flat.dtype), _lib.ptr(out), _lib.ptr(buf), nbytes, _lib.stream_of(q_flat.device)),
            "decode_attn_append")
        return out
    _lib.check(_lib.lib().wnw_decode_attn_ex(
        _lib.ptr(q_flat), _lib.ptr(k_flat), _lib.ptr(v_flat), _lib.ptr(cu_k), _lib.ptr(seg_base),
        nseg, g, d, rows, k_flat.shape[0], float(scale), _lib.dtype_code(q_flat.dtype), _lib.ptr(out),
        _lib.ptr(buf), nbytes, _KERNELS[kernel], int(n_wg), _lib.stream_of(q_flat.device)), "decode_attn")
    return out


def _check_attn(q_flat, k_flat, v_flat, cu_k, seg_base, total_rows):
    """Validate decode_attn's tensors; returns q_flat and cu_k contiguous."""
    _lib.require_gpu(q_flat, k_flat, v_flat, cu_k, seg_base)
    if q_flat.dim() != 3:
        raise _lib.WnwError(f"q_flat must be [N, G, D], got {tuple(q_flat.shape)}")
    nseg, g, d = q_flat.shape
    if k_flat.dim() != 2 or k_flat.shape[1] != d or v_flat.shape != k_flat.shape:
        raise _lib.WnwError(f"k/v must be [rows, {d}] and equal: {tuple(k_flat.shape)} {tuple(v_flat.shape)}")
    if q_flat.dtype != k_flat.dtype or v_flat.dtype != k_flat.dtype:
        raise _lib.WnwError("q, k and v must share a dtype")
    if cu_k.dtype != torch.int32 or cu_k.numel() != nseg + 1:
        raise _lib.WnwError("cu_k must be int32 [N+1]")
    if seg_base is not None and (seg_base.dtype != torch.int64 or seg_base.numel() != nseg):
        raise _lib.WnwError("seg_base must be int64 [N]")
    if seg_base is not None and total_rows is None:
        raise _lib.WnwError("total_rows (cu_k[-1]) is required with seg_base")
    if k_flat.shape[0] > 0 and (k_flat.stride(1) != 1 or k_flat.stride(0) != d or v_flat.stride(1) != 1
                                or v_flat.stride(0) != d):
        raise _lib.WnwError("k_flat / v_flat rows must be contiguous [rows, D]")
    return q_flat.contiguous(), cu_k.contiguous()


def _check_append(append, nseg: int, d: int, dtype, cu_k, seg_base):
    """Validate the (new_k, new_v, cu_new, seg_cap) of a fused append."""
    if seg_base is None:
        raise _lib.WnwError("the fused append needs a slack layout (seg_base)")
    new_k, new_v, cu_new, seg_cap = append
    _lib.require_gpu(new_k, new_v, cu_new, seg_cap)
    if new_k.shape != (nseg, d) or new_v.shape != (nseg, d) or new_k.dtype != dtype or new_v.dtype != dtype:
        raise _lib.WnwError(f"new_k / new_v must be [{nseg}, {d}] of the pools' dtype")
    if cu_new.dtype != torch.int32 or cu_new.numel() != nseg + 1 or not cu_new.is_contiguous():
        raise _lib.WnwError("cu_new must be a contiguous int32 [N+1]")
    if cu_new.data_ptr() == cu_k.data_ptr():
        raise _lib.WnwError("cu_new must not alias cu_k")
    if seg_cap.dtype != torch.int32 or seg_cap.numel() != nseg:
        raise _lib.WnwError("seg_cap must be int32 [N]")
    return new_k.contiguous(), new_v.contiguous(), cu_new, seg_cap.contiguous()


def q1_decode_attn(
    q_flat: torch.Tensor,
    k_flat: torch.Tensor,
    v_flat: torch.Tensor,
    cu_k: torch.Tensor,
    scale: float,
    block_n: int = 64,
) -> torch.Tensor:
    """Return attention output [nseg, G, D] (same dtype as q_flat).

    Reference: ``q1_decode_attn`` (src/common/kv/fused_attn.py:47-65).
    ``block_n`` is accepted for signature compatibility; the tile shape of
    the gfx950 kernel is fixed (32-row MFMA steps).
    """
    del block_n
    return decode_attn(q_flat, k_flat, v_flat, cu_k, scale)


def q1_decode_attn_score(
    q_flat: torch.Tensor,
    k_flat: torch.Tensor,
    v_flat: torch.Tensor,
    cu_k: torch.Tensor,
    scale: float,
    ca_kv_mask: torch.Tensor,
    num_kv_heads: int,
    audio_starts: torch.Tensor,
    audio_ends: torch.Tensor,
    score_accumulator: torch.Tensor,
    score_offsets: torch.Tensor,
    block_n: int = 64,
    *,
    seg_base: torch.Tensor | None = None,
    total_rows: int | None = None,
    max_audio: int | None = None,
    out: torch.Tensor | None = None,
    workspace: AttnWorkspace | None = None,
    keep_logits: bool = True,
    append: tuple | None = None,
    validate: bool = True,
) -> torch.Tensor:
    """Attention output [nseg, G, D] plus class-A score accumulation.

    Reference: ``q1_decode_attn_score`` (src/common/kv/fused_attn.py:
    124-156): for every segment whose KV head is flagged in ``ca_kv_mask``,
    each audio token's softmax weight summed over the group's query heads is
    added to ``score_accumulator[score_offsets[b] + token]``.  The weights
    use the attention's own final softmax statistics.  ``max_audio`` (the
    largest ``audio_ends - audio_starts``) sizes the scoring grid; when it is
    not given it is read back from the device (one synchronisation).
    ``keep_logits`` lets the attention kernel keep the logits of the scored
    rows for the scoring pass (workspace of n_seg * G * max_audio floats);
    without it the scoring pass reads the K rows again.  ``append`` as for
    ``decode_attn``: the step's rows are appended in place first (scores
    then cover the appended segments).  ``validate=False`` skips the argument
    checks for a caller whose tensors are known to satisfy them (the cache's
    own, per layer and step).
    """
    del block_n
    if validate:
        q_flat, cu_k, ca_kv_mask, audio_starts, audio_ends, score_offsets = _check_score(
            q_flat, k_flat, v_flat, cu_k, ca_kv_mask, num_kv_heads, audio_starts, audio_ends, score_accumulator,
            score_offsets, seg_base, total_rows)
    nseg, g, d = q_flat.shape
    if max_audio is None:
        max_audio = int((audio_ends - audio_starts).max().item()) if audio_ends.numel() else 0
    if out is None:
        out = torch.empty(nseg, g, d, device=q_flat.device, dtype=q_flat.dtype)
    rows = k_flat.shape[0] if total_rows is None else int(total_rows)
    _lib.ensure_init(q_flat.device)
    ws = workspace if workspace is not None else workspace_for(q_flat.device)
    buf, nbytes = ws.get(nseg, g, d, score=True, max_audio=int(max_audio) if keep_logits else 0)
    if append is not None:
        new_k, new_v, cu_new, seg_cap = (_check_append(append, nseg, d, k_flat.dtype, cu_k, seg_base) if validate
                                         else append)
        _lib.check(_lib.lib().wnw_decode_attn_score_append(
            _lib.ptr(q_flat), _lib.ptr(k_flat), _lib.ptr(v_flat), _lib.ptr(new_k), _lib.ptr(new_v), _lib.ptr(cu_k),
            _lib.ptr(cu_new), _lib.ptr(seg_base), _lib.ptr(seg_cap), nseg, g, d, rows, k_flat.shape[0], float(scale),
            _lib.dtype_code(q_flat.dtype), _lib.ptr(out), _lib.ptr(ca_kv_mask), int(num_kv_heads),
            _lib.ptr(audio_starts), _lib.ptr(audio_ends), _lib.ptr(score_accumulator), _lib.ptr(score_offsets),
            score_accumulator.numel(), int(max_audio), _lib.ptr(buf), nbytes, _lib.stream_of(q_flat.device)),
            "q1_decode_attn_score (append)")
        return out
    _lib.check(_lib.lib().wnw_decode_attn_score(
        _lib.ptr(q_flat), _lib.ptr(k_flat), _lib.ptr(v_flat), _lib.ptr(cu_k), _lib.ptr(seg_base), nseg, g, d, rows,
        k_flat.shape[0], float(scale), _lib.dtype_code(q_flat.dtype), _lib.ptr(out), _lib.ptr(ca_kv_mask),
        int(num_kv_heads), _lib.ptr(audio_starts), _lib.ptr(audio_ends), _lib.ptr(score_accumulator),
        _lib.ptr(score_offsets), score_accumulator.numel(), int(max_audio), _lib.ptr(buf), nbytes,
        _lib.stream_of(q_flat.device)), "q1_decode_attn_score")
    return out


def score_slot_bytes(nseg: int, group: int, max_audio: int) -> int:
    """Bytes of one score slot (``wnw_score_slot_bytes``): a launch's final
    softmax normalisers and the logits of its scored audio rows."""
    n = int(_lib.lib().wnw_score_slot_bytes(nseg, group, max_audio))
    if n < 0:
        raise _lib.WnwError("bad score slot geometry")
    return n


def decode_attn_append_deferred(q_flat, k_pool, v_pool, cu_k, scale, *, seg_base, total_rows, append, num_kv_heads,
                                audio_starts, audio_ends, max_audio, score_accumulator, score_offsets,
                                keep_mask=None, keep_slot=None, prev=None, out=None, workspace=None):
    """The step's in-place append + attention in one launch
    (``wnw_decode_attn_append_deferred``) that keeps this launch's class-A
    logits and normalisers in ``keep_slot`` (KV heads ``keep_mask``; not
    scored yet) and scores an earlier launch's slot ``prev`` = (mask, slot,
    cu, seg_base, pool_rows, kv_bits) into the accumulator (``kv_bits``: bit h
    set when KV head h was scored, the host's copy of ``mask``), as the second half of the
    reference's ``q1_decode_attn_score`` (src/common/kv/fused_attn.py:
    68-156) split over two launches.  Returns the output [nseg, G, D], or
    None, launching nothing, where this form does not apply (the caller then
    scores another way).  The caller's tensors are trusted (the cache's own:
    dtypes, devices and shapes checked where they are made); the library
    checks sizes and every offset it follows."""
    nseg, g, d = q_flat.shape
    if out is None:
        out = torch.empty(nseg, g, d, device=q_flat.device, dtype=q_flat.dtype)
    ws = workspace if workspace is not None else workspace_for(q_flat.device)
    buf, nbytes = ws.get(nseg, g, d)
    new_k, new_v, cu_new, seg_cap = append
    _pm, ps, pcu, pbase, prows, pbits = prev if prev is not None else (None, None, None, None, 0, 0)
    rc = _lib.lib().wnw_decode_attn_append_deferred(
        _lib.ptr(q_flat), _lib.ptr(k_pool), _lib.ptr(v_pool), _lib.ptr(new_k), _lib.ptr(new_v), _lib.ptr(cu_k),
        _lib.ptr(cu_new), _lib.ptr(seg_base), _lib.ptr(seg_cap), nseg, g, d, int(total_rows), k_pool.shape[0],
        float(scale), _lib.dtype_code(q_flat.dtype), _lib.ptr(out), int(num_kv_heads), _lib.ptr(audio_starts),
        _lib.ptr(audio_ends), int(max_audio), _lib.ptr(score_accumulator), _lib.ptr(score_offsets),
        score_accumulator.numel(), _lib.ptr(keep_mask), _lib.ptr(keep_slot), int(pbits), _lib.ptr(ps),
        _lib.ptr(pcu), _lib.ptr(pbase), int(prows), _lib.ptr(buf), nbytes, _lib.stream_of(q_flat.device))
    if rc == _lib.WNW_ENOTSUP:
        return None
    _lib.check(rc, "decode_attn_append_deferred")
    return out


def score_kept_logits(prev, nseg: int, group: int, num_kv_heads: int, audio_starts, audio_ends, max_audio: int,
                      score_accumulator, score_offsets) -> None:
    """The scoring pass over a slot ``prev`` = (mask, slot, cu, seg_base,
    pool_rows, kv_bits) in a launch of its own (``wnw_score_kept_logits``)."""
    pm, ps, pcu, pbase, prows, _bits = prev
    _lib.check(_lib.lib().wnw_score_kept_logits(
        _lib.ptr(pm), _lib.ptr(ps), _lib.ptr(pcu), _lib.ptr(pbase), int(prows), nseg, group, int(num_kv_heads),
        _lib.ptr(audio_starts), _lib.ptr(audio_ends), int(max_audio), _lib.ptr(score_accumulator),
        _lib.ptr(score_offsets), score_accumulator.numel(), _lib.stream_of(score_accumulator.device)),
        "score_kept_logits")


def _check_score(q_flat, k_flat, v_flat, cu_k, ca_kv_mask, num_kv_heads, audio_starts, audio_ends,
                 score_accumulator, score_offsets, seg_base, total_rows):
    """Validate q1_decode_attn_score's tensors; returns the ones the launch
    needs contiguous."""
    _lib.require_gpu(q_flat, k_flat, v_flat, cu_k, ca_kv_mask, audio_starts, audio_ends, score_accumulator,
                     score_offsets, seg_base)
    if q_flat.dim() != 3:
        raise _lib.WnwError(f"q_flat must be [N, G, D], got {tuple(q_flat.shape)}")
    nseg, g, d = q_flat.shape
    for name, t, n in (("ca_kv_mask", ca_kv_mask, num_kv_heads), ("audio_starts", audio_starts, nseg // num_kv_heads),
                       ("audio_ends", audio_ends, nseg // num_kv_heads),
                       ("score_offsets", score_offsets, nseg // num_kv_heads + 1)):
        if t.dtype != torch.int32 or t.numel() != n:
            raise _lib.WnwError(f"{name} must be int32 [{n}]")
    if score_accumulator.dtype != torch.float32 or not score_accumulator.is_contiguous():
        raise _lib.WnwError("score_accumulator must be a contiguous float32 tensor")
    if k_flat.dim() != 2 or k_flat.shape[1] != d or v_flat.shape != k_flat.shape:
        raise _lib.WnwError("k/v must be [rows, D] and equal")
    if q_flat.dtype != k_flat.dtype or v_flat.dtype != k_flat.dtype:
        raise _lib.WnwError("q, k and v must share a dtype")
    if cu_k.dtype != torch.int32 or cu_k.numel() != nseg + 1:
        raise _lib.WnwError("cu_k must be int32 [N+1]")
    if seg_base is not None and total_rows is None:
        raise _lib.WnwError("total_rows (cu_k[-1]) is required with seg_base")
    return (q_flat.contiguous(), cu_k.contiguous(), ca_kv_mask.contiguous(), audio_starts.contiguous(),
            audio_ends.contiguous(), score_offsets.contiguous())

"""PyTorch CPU restatement of one decode layer-step -- TEST INFRASTRUCTURE.

Only ``bench.py``'s ``cpu_baseline`` leg (the reported CPU baseline) and
``tests/`` use this module.  It is the reference's decode step on a CPU, in
plain PyTorch, because the reference's own GPU kernels (Triton, and the
flash-only ``varlen_attn``) cannot run on one:

* ``append_by_cat``: the out-of-place append of one row per segment
  (``interleave_append``, src/common/kv/kernels.py:45-73), written as the
  ``torch.cat`` of the segments' old rows and the new rows, the way the
  reference's ``torch.cat`` compaction fallback builds a layer
  (src/algorithms/wnw/code/cache.py:891-1010, ``pieces_k`` / ``torch.cat``);
* ``decode_attn``: per segment ``softmax(K_s q * scale) V_s`` in float32 from
  bf16/f16 storage, the formulation of the reference's PyTorch scoring
  fallback (src/algorithms/wnw/code/kernels.py:351-370: ``K_seg @ q``,
  ``torch.softmax(logits.float())``), extended by the ``@ V`` of the
  attention it scores (src/common/kv/fused_attn.py:9-44).

The segments' GQA heads are handled together (``q_s [G, D] @ K_s^T``), as
the 0-stride K/V of the reference's ``varlen_attn`` call share one K/V row
set per group (src/algorithms/wnw/code/session.py:90-106).
"""
from __future__ import annotations

import torch


def append_by_cat(old: torch.Tensor, new_rows: torch.Tensor, cu_old: list[int]) -> torch.Tensor:
    """[total_old, D] + [N, D] -> [total_old + N, D]: segment s's old rows then new_rows[s]."""
    pieces = []
    for s in range(new_rows.shape[0]):
        pieces.append(old[cu_old[s]:cu_old[s + 1]])
        pieces.append(new_rows[s:s + 1])
    return torch.cat(pieces)


def decode_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu: list[int], scale: float) -> torch.Tensor:
    """q [N, G, D], k/v [T, D] (dense layout, offsets cu) -> [N, G, D] in q's dtype."""
    n, g, d = q.shape
    out = torch.zeros(n, g, d, dtype=torch.float32)
    for s in range(n):
        lo, hi = cu[s], cu[s + 1]
        if hi == lo:
            continue
        ks = k[lo:hi].float()
        vs = v[lo:hi].float()
        logits = (q[s].float() @ ks.T) * scale  # [G, len]
        p = torch.softmax(logits, dim=-1)
        out[s] = p @ vs
    return out.to(q.dtype)

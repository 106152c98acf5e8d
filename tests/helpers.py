"""Shared generators for the parity tests (seeded, numpy)."""
from __future__ import annotations

import numpy as np

from oracle import DT_BF16, DT_F16, DT_F32, f32_to_bf16_bits

DTYPE_CODES = {"float32": DT_F32, "float16": DT_F16, "bfloat16": DT_BF16}


def rand_rows(rng, n: int, d: int, dtype: str, scale: float = 1.0) -> np.ndarray:
    """Random rows in the storage format the oracle takes (uint16 bits for 16-bit)."""
    x = (rng.standard_normal((n, d)) * scale).astype(np.float32)
    if dtype == "float32":
        return x
    if dtype == "bfloat16":
        return f32_to_bf16_bits(x)
    return x.astype(np.float16).view(np.uint16)


def cu_from_lens(lens) -> np.ndarray:
    cu = np.zeros(len(lens) + 1, dtype=np.int32)
    cu[1:] = np.cumsum(np.asarray(lens, dtype=np.int64))
    return cu


def to_torch(a: np.ndarray, dtype: str, device):
    """numpy storage array -> torch tensor of `dtype` on `device`."""
    import torch

    if dtype == "float32" or a.dtype != np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a)).to(device)
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16))
    return t.view(torch.bfloat16 if dtype == "bfloat16" else torch.float16).to(device)


def from_torch(t, dtype: str) -> np.ndarray:
    """torch tensor -> numpy storage array (uint16 bits for 16-bit)."""
    import torch

    t = t.detach().cpu().contiguous()
    if dtype == "float32":
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def rand_rebuild_descriptors(rng, old_lens, load_pool: int, max_ranges: int = 4, p_change: float = 0.6):
    """Random sorted, disjoint evict ranges and contiguous load ranges per segment.

    Returns (load_starts, load_lens, evict_offsets, evict_starts, evict_ends,
    new_lens) as numpy int32 arrays, new_len = old - evicted + loaded + 1.
    """
    n = len(old_lens)
    load_starts = np.full(n, -1, dtype=np.int32)
    load_lens = np.zeros(n, dtype=np.int32)
    ev_off = [0]
    ev_s, ev_e = [], []
    new_lens = np.zeros(n, dtype=np.int32)
    cursor = 0
    for s in range(n):
        L = int(old_lens[s])
        evicted = 0
        if L > 0 and rng.random() < p_change:
            k = int(rng.integers(0, max_ranges + 1))
            cuts = np.sort(rng.choice(L + 1, size=min(2 * k, L + 1), replace=False))
            for a, b in zip(cuts[0::2], cuts[1::2]):
                if b > a:
                    ev_s.append(int(a))
                    ev_e.append(int(b))
                    evicted += int(b - a)
        ev_off.append(len(ev_s))
        loaded = 0
        if rng.random() < p_change and load_pool > 0:
            loaded = int(rng.integers(0, min(64, load_pool) + 1))
            if loaded:
                start = int(rng.integers(0, load_pool - loaded + 1))
                load_starts[s] = start
                load_lens[s] = loaded
        cursor += loaded
        new_lens[s] = L - evicted + loaded + 1
    return (load_starts, load_lens, np.array(ev_off, dtype=np.int32), np.array(ev_s, dtype=np.int32),
            np.array(ev_e, dtype=np.int32), new_lens)


def allclose_report(got: np.ndarray, ref: np.ndarray, atol: float, rtol: float) -> tuple[bool, str]:
    err = np.abs(got.astype(np.float64) - ref)
    bound = atol + rtol * np.abs(ref)
    ok = bool(np.all(err <= bound)) and bool(np.all(np.isfinite(got)))
    worst = float(np.max(err - bound)) if err.size else 0.0
    return ok, f"max_abs={float(err.max()) if err.size else 0:.3e} worst_excess={worst:.3e}"

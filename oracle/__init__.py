"""CPU oracle of WnW's decode-step attention path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline).  The product (``wnw_amd``) never imports it and has no CPU
fallback.

Contents
--------
* ``libwnw_oracle.so`` (built from ``wnw_oracle.c`` by ``oracle/Makefile``):
  float64 decode attention and the byte-exact append / compaction gathers,
  each function citing the reference file:line it restates.
* numpy restatements written independently of the C code (``np_*``) so each
  C function is cross-checked by a second formulation.
* ``planner``: the decode chunk planner of the reference, restated in pure
  Python.

How each function is pinned (a check that a plausible mistake would fail)
is listed in the module docstrings of ``tests/test_oracle.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libwnw_oracle.so")
_lib = None

DT_F32, DT_F16, DT_BF16 = 0, 1, 2


def build() -> None:
    """Compile libwnw_oracle.so with the host C compiler."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        l = ctypes.CDLL(_LIB_PATH)
        vp, i64, i32, dbl = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
        l.oracle_decode_attn.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, dbl, i32, i64, vp]
        l.oracle_interleave_append.argtypes = [vp, vp, vp, vp, i64, i64, i64, i32, vp]
        l.oracle_rebuild_append_kv.argtypes = [vp] * 13 + [i64] * 7 + [i32, vp, vp]
        l.oracle_rebuild_by_slices.argtypes = [vp] * 12 + [i64, i64, i32, vp, vp, vp]
        l.oracle_segment_scores.argtypes = [vp] * 7 + [i64, i64, i64, dbl, i32, i64, i64, vp]
        for f in (l.oracle_decode_attn, l.oracle_interleave_append, l.oracle_rebuild_append_kv,
                  l.oracle_rebuild_by_slices, l.oracle_segment_scores):
            f.restype = ctypes.c_int
        _lib = l
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _dtype_code(a: np.ndarray, dtype: int | None) -> int:
    if dtype is not None:
        return dtype
    if a.dtype == np.float32:
        return DT_F32
    raise ValueError("16-bit arrays must pass dtype= (DT_F16 or DT_BF16) explicitly")


# ---------------------------------------------------------------------------
# bf16 helpers (numpy has no bfloat16): bf16 values travel as uint16 bits
# ---------------------------------------------------------------------------
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_f64(a: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == DT_F32:
        return a.astype(np.float64)
    if dtype == DT_BF16:
        return bf16_bits_to_f32(a).astype(np.float64)
    return a.view(np.float16).astype(np.float64)


# ---------------------------------------------------------------------------
# C oracle wrappers
# ---------------------------------------------------------------------------
def decode_attn(q, k, v, cu, scale, base=None, dtype=None):
    """float64 attention; q [N, G, D], k/v [rows, D] (uint16 bits if 16-bit)."""
    dt = _dtype_code(q, dtype)
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    cu = np.ascontiguousarray(cu, dtype=np.int32)
    n, g, d = q.shape
    out = np.zeros((n, g, d), dtype=np.float64)
    b = None if base is None else np.ascontiguousarray(base, dtype=np.int64)
    rc = lib().oracle_decode_attn(_p(q), _p(k), _p(v), _p(cu), _p(b), n, g, d, float(scale), dt,
                                  k.shape[0], _p(out))
    if rc != 0:
        raise ValueError("oracle_decode_attn: inconsistent offsets")
    return out


def segment_scores(q, k, r0, r1, a0, a1, off, scale, acc, dtype=None):
    """float64 class-A scores added into ``acc`` (float64, updated in place).

    q [items, nh, D]; per item: K rows [r0, r1), audio rows [a0, a1) relative
    to r0, accumulator offset ``off``."""
    dt = _dtype_code(q, dtype)
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    n, nh, d = q.shape
    i64 = lambda a: np.ascontiguousarray(a, dtype=np.int64)  # noqa: E731
    i32 = lambda a: np.ascontiguousarray(a, dtype=np.int32)  # noqa: E731
    assert acc.dtype == np.float64 and acc.flags.c_contiguous
    rc = lib().oracle_segment_scores(_p(q), _p(k), _p(i64(r0)), _p(i64(r1)), _p(i32(a0)), _p(i32(a1)),
                                     _p(i64(off)), n, nh, d, float(scale), dt, k.shape[0], acc.size, _p(acc))
    if rc != 0:
        raise ValueError("oracle_segment_scores: inconsistent ranges")
    return acc


def attn_scores(q, k, cu, scale, ca_kv_mask, num_kv_heads, audio_s, audio_e, offsets, acc, base=None, dtype=None):
    """q1_decode_attn_score's scoring part (fused_attn.py:112-123) mapped onto
    ``segment_scores``: one item per segment whose KV head is flagged."""
    n_seg = q.shape[0]
    items = [s for s in range(n_seg) if ca_kv_mask[s % num_kv_heads]]
    if not items:
        return acc
    bs = [s // num_kv_heads for s in items]
    start = [int(base[s]) if base is not None else int(cu[s]) for s in items]
    r1 = [st + int(cu[s + 1]) - int(cu[s]) for st, s in zip(start, items)]
    return segment_scores(q[items], k, start, r1, [audio_s[b] for b in bs], [audio_e[b] for b in bs],
                          [offsets[b] for b in bs], scale, acc, dtype=dtype)


def interleave_append(old, new, cu_old, cu_new, dtype=None):
    dt = _dtype_code(old, dtype)
    old = np.ascontiguousarray(old)
    new = np.ascontiguousarray(new)
    n, d = new.shape
    out = np.zeros((old.shape[0] + n, d), dtype=old.dtype)
    rc = lib().oracle_interleave_append(_p(old), _p(new), _p(np.ascontiguousarray(cu_old, np.int32)),
                                        _p(np.ascontiguousarray(cu_new, np.int32)), n, old.shape[0], d, dt,
                                        _p(out))
    if rc != 0:
        raise ValueError("oracle_interleave_append: inconsistent offsets")
    return out


def rebuild_append_kv(old_k, old_v, new_k, new_v, load_k, load_v, old_cu, new_cu, load_starts, load_lens,
                      evict_offsets, evict_starts, evict_ends, max_evict, dtype=None):
    dt = _dtype_code(old_k, dtype)
    arrs = [np.ascontiguousarray(a) for a in (old_k, old_v, new_k, new_v, load_k, load_v)]
    ints = [np.ascontiguousarray(a, dtype=np.int32) for a in
            (old_cu, new_cu, load_starts, load_lens, evict_offsets, evict_starts, evict_ends)]
    n, d = arrs[2].shape
    total_out = int(ints[1][-1])
    out_k = np.zeros((total_out, d), dtype=arrs[0].dtype)
    out_v = np.zeros((total_out, d), dtype=arrs[0].dtype)
    rc = lib().oracle_rebuild_append_kv(*[_p(a) for a in arrs], *[_p(a) for a in ints], ints[5].size, n,
                                        arrs[0].shape[0], arrs[4].shape[0], total_out, int(max_evict), d, dt,
                                        _p(out_k), _p(out_v))
    if rc != 0:
        raise ValueError("oracle_rebuild_append_kv: inconsistent descriptors")
    return out_k, out_v


def rebuild_by_slices(old_k, old_v, new_k, new_v, load_k, load_v, old_cu, load_starts, load_lens,
                      evict_offsets, evict_starts, evict_ends, dtype=None):
    dt = _dtype_code(old_k, dtype)
    arrs = [np.ascontiguousarray(a) for a in (old_k, old_v, new_k, new_v, load_k, load_v)]
    ints = [np.ascontiguousarray(a, dtype=np.int32) for a in
            (old_cu, load_starts, load_lens, evict_offsets, evict_starts, evict_ends)]
    n, d = arrs[2].shape
    cap = arrs[0].shape[0] + int(np.sum(ints[2], dtype=np.int64)) + n
    out_k = np.zeros((cap, d), dtype=arrs[0].dtype)
    out_v = np.zeros((cap, d), dtype=arrs[0].dtype)
    out_cu = np.zeros(n + 1, dtype=np.int32)
    lib().oracle_rebuild_by_slices(*[_p(a) for a in arrs], *[_p(a) for a in ints], n, d, dt, _p(out_k),
                                   _p(out_v), _p(out_cu))
    t = int(out_cu[-1])
    return out_k[:t], out_v[:t], out_cu


# ---------------------------------------------------------------------------
# independent numpy restatements (cross-checks of the C code)
# ---------------------------------------------------------------------------
def np_decode_attn(q64, k64, v64, cu, scale, base=None):
    """Vectorised float64 softmax attention per segment (numpy)."""
    n, g, d = q64.shape
    out = np.zeros((n, g, d))
    for s in range(n):
        lo, hi = int(cu[s]), int(cu[s + 1])
        if hi == lo:
            continue
        b = lo if base is None else int(base[s])
        ks = k64[b:b + hi - lo]
        vs = v64[b:b + hi - lo]
        logits = (q64[s] @ ks.T) * scale  # [G, n]
        logits -= logits.max(axis=1, keepdims=True)
        p = np.exp(logits)
        p /= p.sum(axis=1, keepdims=True)
        out[s] = p @ vs
    return out


def np_interleave_append(old, new, cu_old):
    parts = []
    for s in range(new.shape[0]):
        parts.append(old[int(cu_old[s]):int(cu_old[s + 1])])
        parts.append(new[s:s + 1])
    return np.concatenate(parts, axis=0)

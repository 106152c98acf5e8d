"""wnw_decode_attn_noalloc, the attention entry point that allocates
nothing (its split-K scratch is a file-scope device array of the library),
against wnw_decode_attn with a caller-owned workspace, through the C ABI.

Both run the same kernel with the same grid, so the outputs must be
identical bit for bit; each is also held to the oracle's tolerance
(2e-3 + 1e-2 |ref|).  Two calls in a row on the shared scratch, the second
with a smaller input (fewer segments, another layout), then calls beyond the
scratch's limits, which must be refused without a launch.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import allclose_report, cu_from_lens, from_torch, rand_rows, to_torch
from wnw_amd import _lib

pytestmark = pytest.mark.gpu

G, D = 4, 128


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _case(rng, lens, slack):
    n = len(lens)
    base = None
    rows = int(sum(lens))
    if slack:
        base = np.zeros(n, np.int64)
        pos = 5
        for s in range(n):
            base[s] = pos
            pos += lens[s] + int(rng.integers(0, 9))
        rows = pos + 3
    q = rand_rows(rng, n * G, D, "bfloat16").reshape(n, G, D)
    k = rand_rows(rng, rows, D, "bfloat16")
    v = rand_rows(rng, rows, D, "bfloat16")
    return q, k, v, cu_from_lens(lens), base, rows


def _run_both(dev, q, k, v, cu, base, rows):
    n = q.shape[0]
    tq, tk, tv = (to_torch(a, "bfloat16", dev) for a in (q, k, v))
    tcu = torch.from_numpy(cu).to(dev)
    tb = None if base is None else torch.from_numpy(base).to(dev)
    out_na = torch.full((n, G, D), float("nan"), dtype=torch.bfloat16, device=dev)
    out_ws = torch.full((n, G, D), float("nan"), dtype=torch.bfloat16, device=dev)
    lib = _lib.lib()
    _lib.ensure_init(dev)
    stream = _lib.stream_of(dev)
    scale = D ** -0.5
    _lib.check(lib.wnw_decode_attn_noalloc(_ptr(tq), _ptr(tk), _ptr(tv), _ptr(tcu), _ptr(tb), n, G, D, int(cu[-1]),
                                           rows, scale, _lib.DT_BF16, _ptr(out_na), stream), "noalloc")
    nbytes = int(lib.wnw_decode_attn_workspace_bytes(n, G, D))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    _lib.check(lib.wnw_decode_attn(_ptr(tq), _ptr(tk), _ptr(tv), _ptr(tcu), _ptr(tb), n, G, D, int(cu[-1]), rows,
                                   scale, _lib.DT_BF16, _ptr(out_ws), _ptr(ws), nbytes, stream), "workspace")
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    ref = oracle.decode_attn(q, k, v, cu, scale, base=base, dtype=oracle.DT_BF16)
    return from_torch(out_na, "bfloat16"), from_torch(out_ws, "bfloat16"), ref


def test_noalloc_matches_workspace_entry_point(gpu):
    rng = np.random.default_rng(11)
    # a cfg2-like layer (class-A segments beside short class-B ones), then a
    # smaller slack-layout input with an empty segment
    big = [7565 if h in (1, 6) else 513 for _ in range(8) for h in range(8)]
    small = [int(x) for x in rng.integers(1, 900, 13)] + [0, 40]
    for i, (lens, slack) in enumerate(((big, False), (small, True))):
        print(f"noalloc call {i}: n_seg={len(lens)} rows={sum(lens)} slack={slack}", flush=True)
        q, k, v, cu, base, rows = _case(rng, lens, slack)
        na, ws, ref = _run_both(gpu, q, k, v, cu, base, rows)
        np.testing.assert_array_equal(na, ws, err_msg=f"call {i}: no-alloc and workspace outputs differ")
        ok, msg = allclose_report(oracle.to_f64(na, oracle.DT_BF16), ref, 2e-3, 1e-2)
        assert ok, f"call {i}: {msg}"


def test_noalloc_refuses_calls_beyond_its_scratch(gpu):
    lib = _lib.lib()
    dev = gpu
    n = 4097  # WNW_NOALLOC_MAX_SEG + 1
    q = torch.zeros(n, G, D, dtype=torch.bfloat16, device=dev)
    kv = torch.zeros(n, D, dtype=torch.bfloat16, device=dev)
    cu = torch.arange(n + 1, dtype=torch.int32, device=dev)
    out = torch.zeros_like(q)
    rc = lib.wnw_decode_attn_noalloc(_ptr(q), _ptr(kv), _ptr(kv), _ptr(cu), None, n, G, D, n, n, 0.1,
                                     _lib.DT_BF16, _ptr(out), _lib.stream_of(dev))
    assert rc == _lib.WNW_EINVAL and b"at most 4096 segments" in lib.wnw_last_error()
    # within the segment limit, but 16 heads of 256 over 4096 segments need more than 16 MiB of partials
    n, g, d = 4096, 16, 256
    q = torch.zeros(n, g, d, dtype=torch.float32, device=dev)
    kv = torch.zeros(n, d, dtype=torch.float32, device=dev)
    cu = torch.arange(n + 1, dtype=torch.int32, device=dev)
    out = torch.zeros_like(q)
    rc = lib.wnw_decode_attn_noalloc(_ptr(q), _ptr(kv), _ptr(kv), _ptr(cu), None, n, g, d, n, n, 0.1,
                                     _lib.DT_F32, _ptr(out), _lib.stream_of(dev))
    assert rc == _lib.WNW_EINVAL and b"bytes of split-K scratch" in lib.wnw_last_error()
    torch.cuda.synchronize()
    assert _lib.device_error() == 0

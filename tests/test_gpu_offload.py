"""Device-side gather of host rows (the offload channel) against numpy."""
import numpy as np
import pytest
import torch

from wnw_amd import _lib
from wnw_amd.wnw.kernels import gather_host_rows, host_rows_readable

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def _pinned(rng, rows, d):
    a = rng.integers(0, 1 << 16, size=(rows, d), dtype=np.uint16)
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).pin_memory(), a


@pytest.mark.parametrize("d", [64, 128])
def test_gather_matches_numpy(gpu, d):
    rng = np.random.default_rng(d)
    big_k, ak = _pinned(rng, 5000, d)
    big_v, av = _pinned(rng, 5000, d)
    # an interior view of a pinned block
    hk, hv = big_k[300:4300], big_v[300:4300]
    ak, av = ak[300:4300], av[300:4300]
    assert host_rows_readable(hk, hv)
    starts = rng.integers(0, 3900, size=40)
    lens = rng.integers(0, 100, size=40)
    ranges = np.stack([starts, np.minimum(starts + lens, 4000)], axis=1).astype(np.int32)
    n = ranges[:, 1] - ranges[:, 0]
    dst = np.concatenate([[0], np.cumsum(n)]).astype(np.int64)
    total = int(dst[-1])
    out_k = torch.zeros(total + 7, d, dtype=torch.bfloat16, device=gpu)
    out_v = torch.zeros(total + 7, d, dtype=torch.bfloat16, device=gpu)
    rg, do = torch.from_numpy(ranges).to(gpu), torch.from_numpy(dst).to(gpu)
    # in three spans, as the cache launches it per layer
    for r0, r1 in ((0, 13), (13, 13), (13, 40)):
        gather_host_rows(hk, hv, rg, do, r0, r1, out_k, out_v)
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    want_k = np.concatenate([ak[s:e] for s, e in ranges])
    want_v = np.concatenate([av[s:e] for s, e in ranges])
    np.testing.assert_array_equal(_bits(out_k)[:total], want_k)
    np.testing.assert_array_equal(_bits(out_v)[:total], want_v)
    assert not _bits(out_k)[total:].any()  # nothing past the last range


def test_out_of_bounds_range_is_refused(gpu):
    rng = np.random.default_rng(1)
    hk, _ = _pinned(rng, 100, 128)
    hv, _ = _pinned(rng, 100, 128)
    ranges = torch.tensor([[90, 110]], dtype=torch.int32, device=gpu)  # past the 100 host rows
    dst = torch.tensor([0, 20], dtype=torch.int64, device=gpu)
    out_k = torch.zeros(20, 128, dtype=torch.bfloat16, device=gpu)
    out_v = torch.zeros(20, 128, dtype=torch.bfloat16, device=gpu)
    gather_host_rows(hk, hv, ranges, dst, 0, 1, out_k, out_v)
    torch.cuda.synchronize()
    assert _lib.device_error() == _lib.DEVERR_BOUNDS
    assert not _bits(out_k).any() and not _bits(out_v).any()


def test_pageable_memory_is_refused(gpu):
    hk = torch.zeros(10, 128, dtype=torch.bfloat16)
    assert not host_rows_readable(hk, hk)
    rg = torch.tensor([[0, 1]], dtype=torch.int32, device=gpu)
    do = torch.tensor([0, 1], dtype=torch.int64, device=gpu)
    out = torch.zeros(1, 128, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(_lib.WnwError):
        gather_host_rows(hk, hk, rg, do, 0, 1, out, out)

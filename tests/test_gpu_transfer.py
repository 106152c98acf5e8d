"""The host->device transfer engine (``wnw_h2d_*``): the planned host ranges
land bit-exact in the device rows of their transfer order, group by group,
over several consecutive starts (the two staging pairs in turn, the second
reuse of a pair after its copies finish), with empty ranges and groups, and
argument errors are refused without starting anything.  The reference's
counterpart is the planner's gather into staging plus one side-stream copy
(src/algorithms/wnw_cpp/code/planner.cpp:113-122,
src/algorithms/wnw/code/cache.py:868-881); the expected rows here are the
host rows themselves, indexed in numpy."""
import numpy as np
import pytest
import torch

from wnw_amd import _lib
from wnw_amd.wnw.transfer import HostToDevice

pytestmark = pytest.mark.gpu

D = 128


def _host_rows(rng, n):
    a = rng.integers(0, 1 << 16, (n, D), dtype=np.uint16)
    t = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)
    return a, t.pin_memory()


def _case(rng, host_rows, n_ranges, n_groups):
    starts = rng.integers(0, host_rows - 300, n_ranges)
    lens = rng.integers(0, 300, n_ranges)
    lens[rng.random(n_ranges) < 0.1] = 0  # some empty ranges
    ranges = np.stack([starts, starts + lens], 1).astype(np.int32)
    cuts = np.sort(rng.integers(0, n_ranges + 1, n_groups - 1))
    bounds = [0] + cuts.tolist() + [n_ranges]
    return ranges, bounds


def test_ranges_land_in_transfer_order_over_several_starts():
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(5)
    hk_np, hk = _host_rows(rng, 20000)
    hv_np, hv = _host_rows(rng, 20000)
    eng = HostToDevice(workers=4)
    stream = torch.cuda.Stream(device=dev)
    stg = [(torch.empty(60000, D, dtype=torch.bfloat16, pin_memory=True),
            torch.empty(60000, D, dtype=torch.bfloat16, pin_memory=True)) for _ in range(2)]
    outs = []
    for job in range(5):
        ranges, bounds = _case(rng, 20000, int(rng.integers(1, 200)), int(rng.integers(1, 9)))
        total = int((ranges[:, 1] - ranges[:, 0]).sum())
        with torch.cuda.stream(stream):
            dk = torch.empty(max(total, 1), D, dtype=torch.bfloat16, device=dev)
            dv = torch.empty_like(dk)
        sk, sv = stg[job % 2]
        print(f"job {job}: {len(ranges)} ranges, {len(bounds) - 1} groups, {total} rows", flush=True)
        eng.start(hk, hv, torch.from_numpy(ranges), bounds, sk, sv, dk, dv, stream)
        compute = torch.cuda.current_stream(dev)
        for g in range(len(bounds) - 1):
            eng.wait(g, compute)
        got_k = dk[:total].clone()  # on the compute stream, after every group's copy
        got_v = dv[:total].clone()
        outs.append((ranges, got_k, got_v))
    eng.join()
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    for ranges, got_k, got_v in outs:
        idx = np.concatenate([np.arange(s, e) for s, e in ranges]) if len(ranges) else np.zeros(0, np.int64)
        np.testing.assert_array_equal(got_k.cpu().view(torch.int16).numpy().view(np.uint16), hk_np[idx])
        np.testing.assert_array_equal(got_v.cpu().view(torch.int16).numpy().view(np.uint16), hv_np[idx])
    eng.close()


def _chunky_case(rng, host_rows, n_groups):
    """Ranges as a plan over a (sample, segment, layer, head) host layout
    makes them: runs of ranges that touch in host memory (one run per
    segment and group), listed in another order (transfer order), with some
    empty, repeated and overlapping ranges."""
    runs, at = [], 0
    while at < host_rows - 2000:
        n = int(rng.integers(1, 12))
        lens = rng.integers(0, 150, n)
        run = []
        for x in lens:
            run.append((at, at + int(x)))
            at += int(x)
        runs.append(run)
        at += int(rng.integers(0, 500))
    picks = [runs[i] for i in rng.choice(len(runs), size=min(len(runs), 24), replace=False)]
    ranges = [r for run in picks for r in run]
    ranges += [ranges[int(i)] for i in rng.integers(0, len(ranges), 5)]  # repeats
    s0 = int(rng.integers(0, host_rows - 400))
    ranges += [(s0, s0 + 300), (s0 + 100, s0 + 200)]  # overlapping
    order = rng.permutation(len(ranges))
    ranges = np.array([ranges[i] for i in order], dtype=np.int32)
    cuts = np.sort(rng.integers(0, len(ranges) + 1, n_groups - 1))
    return ranges, [0] + cuts.tolist() + [len(ranges)]


def test_direct_form_lands_in_transfer_order():
    """wnw_h2d_start_direct (DMA of merged spans into a device stage, then a
    permute kernel) fills the same rows as the staged form, over several
    starts that alternate the two forms on one engine."""
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(15)
    hk_np, hk = _host_rows(rng, 30000)
    hv_np, hv = _host_rows(rng, 30000)
    eng = HostToDevice(workers=4)
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        stage = (torch.empty(40000, D, dtype=torch.bfloat16, device=dev),
                 torch.empty(40000, D, dtype=torch.bfloat16, device=dev))
    stg = [(torch.empty(40000, D, dtype=torch.bfloat16, pin_memory=True),
            torch.empty(40000, D, dtype=torch.bfloat16, pin_memory=True)) for _ in range(2)]
    outs = []
    for job in range(6):
        ranges, bounds = _chunky_case(rng, 30000, int(rng.integers(1, 9)))
        total = int((ranges[:, 1] - ranges[:, 0]).sum())
        assert total <= 40000
        with torch.cuda.stream(stream):
            dk = torch.empty(max(total, 1), D, dtype=torch.bfloat16, device=dev)
            dv = torch.empty_like(dk)
        direct = job % 3 != 2
        print(f"job {job}: {'direct' if direct else 'staged'}, {len(ranges)} ranges, {len(bounds) - 1} groups, "
              f"{total} rows", flush=True)
        if direct:
            eng.start_direct(hk, hv, torch.from_numpy(ranges), bounds, stage[0], stage[1], dk, dv, stream)
        else:
            eng.start(hk, hv, torch.from_numpy(ranges), bounds, *stg[job % 2], dk, dv, stream)
        compute = torch.cuda.current_stream(dev)
        for g in range(len(bounds) - 1):
            eng.wait(g, compute)
        outs.append((ranges, dk[:total].clone(), dv[:total].clone()))
    eng.join()
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    for ranges, got_k, got_v in outs:
        idx = np.concatenate([np.arange(s, e) for s, e in ranges])
        np.testing.assert_array_equal(got_k.cpu().view(torch.int16).numpy().view(np.uint16), hk_np[idx])
        np.testing.assert_array_equal(got_v.cpu().view(torch.int16).numpy().view(np.uint16), hv_np[idx])
    with pytest.raises(_lib.WnwError):  # more rows than the stage holds
        eng.start_direct(hk, hv, torch.tensor([[0, 20000]], dtype=torch.int32), [0, 1], stage[0][:100],
                         stage[1][:100], dk, dv, stream)
    eng.close()


def test_reserve_then_jobs_land_in_transfer_order():
    """wnw_h2d_reserve (copy streams, descriptor room, an empty job through
    the engine's thread) before and between direct jobs: room below a job's
    range count grows on demand, and the rows land as without it."""
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(21)
    hk_np, hk = _host_rows(rng, 20000)
    hv_np, hv = _host_rows(rng, 20000)
    eng = HostToDevice(workers=2)
    stream = torch.cuda.Stream(device=dev)
    eng.reserve(16, stream)  # less room than the jobs below need
    with torch.cuda.stream(stream):
        stage = (torch.empty(30000, D, dtype=torch.bfloat16, device=dev),
                 torch.empty(30000, D, dtype=torch.bfloat16, device=dev))
    outs = []
    for job in range(4):
        if job == 2:
            eng.reserve(4096, stream)  # between jobs: waits for the engine, then grows both parities
        ranges, bounds = _case(rng, 20000, int(rng.integers(40, 200)), int(rng.integers(1, 9)))
        total = int((ranges[:, 1] - ranges[:, 0]).sum())
        assert total <= 30000
        with torch.cuda.stream(stream):
            dk = torch.empty(max(total, 1), D, dtype=torch.bfloat16, device=dev)
            dv = torch.empty_like(dk)
        print(f"job {job}: {len(ranges)} ranges, {len(bounds) - 1} groups, {total} rows", flush=True)
        eng.start_direct(hk, hv, torch.from_numpy(ranges), bounds, stage[0], stage[1], dk, dv, stream)
        compute = torch.cuda.current_stream(dev)
        for g in range(len(bounds) - 1):
            eng.wait(g, compute)
        outs.append((ranges, dk[:total].clone(), dv[:total].clone()))
    eng.join()
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    for ranges, got_k, got_v in outs:
        idx = np.concatenate([np.arange(s, e) for s, e in ranges])
        np.testing.assert_array_equal(got_k.cpu().view(torch.int16).numpy().view(np.uint16), hk_np[idx])
        np.testing.assert_array_equal(got_v.cpu().view(torch.int16).numpy().view(np.uint16), hv_np[idx])
    with pytest.raises(_lib.WnwError):
        eng.reserve(-1, stream)
    with pytest.raises(_lib.WnwError):
        eng.reserve(16, stream, groups=0)
    eng.close()


def test_arguments_are_checked():
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(6)
    _, hk = _host_rows(rng, 1000)
    _, hv = _host_rows(rng, 1000)
    sk = torch.empty(100, D, dtype=torch.bfloat16, pin_memory=True)
    sv = torch.empty(100, D, dtype=torch.bfloat16, pin_memory=True)
    dk = torch.empty(100, D, dtype=torch.bfloat16, device=dev)
    dv = torch.empty_like(dk)
    s = torch.cuda.current_stream(dev)
    eng = HostToDevice(workers=2)
    ok = torch.tensor([[0, 10], [20, 30]], dtype=torch.int32)
    with pytest.raises(_lib.WnwError):  # groups do not end at n_ranges
        eng.start(hk, hv, ok, [0, 1], sk, sv, dk, dv, s)
    with pytest.raises(_lib.WnwError):  # a range past the host rows
        eng.start(hk, hv, torch.tensor([[990, 1010]], dtype=torch.int32), [0, 1], sk, sv, dk, dv, s)
    with pytest.raises(_lib.WnwError):  # more rows than staging holds
        eng.start(hk, hv, torch.tensor([[0, 200]], dtype=torch.int32), [0, 1], sk, sv, dk, dv, s)
    with pytest.raises(_lib.WnwError):  # pageable staging
        eng.start(hk, hv, ok, [0, 2], torch.empty(100, D, dtype=torch.bfloat16), sv, dk, dv, s)
    eng.start(hk, hv, ok, [0, 1, 2], sk, sv, dk, dv, s)
    with pytest.raises(_lib.WnwError):  # a group the job does not have
        eng.wait(2, s)
    eng.wait(0, s)
    eng.wait(1, s)
    eng.join()
    torch.cuda.synchronize()
    eng.close()


def test_plan_start_direct_checks_the_planner_geometry():
    """The fused plan step refuses a choice for another batch size, or layer
    cuts that do not end at the planner's layer count, before planning."""
    from wnw_amd.wnw_cpp.planner import Planner
    dev = torch.device("cuda", 0)
    L, H, B = 3, 4, 2
    planner = Planner(L, H, B, 2)
    x = HostToDevice(workers=1)
    hk = torch.zeros(64, 64, dtype=torch.bfloat16, pin_memory=True)
    hv = torch.zeros_like(hk).pin_memory()
    st = [torch.zeros(64, 64, dtype=torch.bfloat16, device=dev) for _ in range(4)]
    N = B * H
    outs = dict(load_starts_2d=torch.empty(L, N, dtype=torch.int32), load_lens_2d=torch.empty(L, N, dtype=torch.int32),
                cu_new_2d=torch.empty(L, N + 1, dtype=torch.int32), new_lens_2d=torch.empty(L, N, dtype=torch.int32),
                evict_offsets_2d=torch.empty(L, N + 1, dtype=torch.int32), evict_max=torch.empty(L, dtype=torch.int32),
                evict_layer_ptr=torch.empty(L + 1, dtype=torch.int32))
    stream = torch.cuda.current_stream(dev)
    with pytest.raises(_lib.WnwError, match="samples"):
        x.plan_start_direct(planner, torch.full((B + 1, 2), -1, dtype=torch.int32), outs, [0, 1, L], hk, hv,
                            st[0], st[1], st[2], st[3], stream)
    with pytest.raises(_lib.WnwError, match="samples"):
        x.plan_start_direct(planner, torch.full((B, 2), -1, dtype=torch.int32), outs, [0, 1, L + 1], hk, hv,
                            st[0], st[1], st[2], st[3], stream)
    x.close()

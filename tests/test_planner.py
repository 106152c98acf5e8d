"""Decode chunk planner: native C++ planner vs the Python restatement.

Pinning of the restatement (oracle/planner.py):
* a hand-computed plan (``test_oracle_hand_example``) fixes the evict-range
  shift rule (``end <= start``), the load cursor (after the evicted rows),
  the ``+ 1`` of the step's append and the CSR layouts;
* invariants every plan must satisfy (``test_plan_invariants``): new_len
  arithmetic, sorted disjoint in-range evict ranges, resident segments
  disjoint and inside the new segment;
* end to end through the compaction oracle (``test_plan_drives_compaction``):
  rows tagged with their (segment, row) origin land exactly where the
  updated metadata says.
The native planner (wnw_amd/csrc/planner.cpp) is then held bit-exact to the
restatement over multi-step random scenarios.  All CPU, no GPU.
"""
from __future__ import annotations

import copy
import random

import numpy as np
import pytest
import torch

import oracle
from oracle import planner as op
from wnw_amd.wnw_cpp.planner import Planner


# ---------------------------------------------------------------------------
# scenario builder (the state prefill_all_layers_done leaves, cache.py:339-390)
# ---------------------------------------------------------------------------
def make_scenario(seed: int, L=3, H=3, B=2, max_segs=7, lag=2):
    rng = random.Random(seed)
    N = B * H
    seg_count, c2s = [], []
    for b in range(B):
        n_audio = rng.randint(1, 40)
        stride = rng.choice([4, 5, 8])
        segs = op.compute_segments(n_audio, stride)[:max_segs]
        per = rng.choice([1, 2, 3])
        seg_count.append(len(segs))
        c2s.append(op.compute_chunks(segs, per * stride, stride))
    class_b = [sorted(rng.sample(range(H), rng.randint(0, H))) for _ in range(L)]
    meta = [[[[None] * seg_count[b] for _ in range(H)] for b in range(B)] for _ in range(L)]
    loaded = [set(rng.sample(range(seg_count[b]), rng.randint(0, seg_count[b]))) for b in range(B)]
    seq_lens = [[0] * N for _ in range(L)]
    cpu = 0
    for l in range(L):
        for b in range(B):
            for h in range(H):
                base = rng.randint(0, 12)
                length = base
                if h in class_b[l]:
                    for s in range(seg_count[b]):
                        if rng.random() < 0.2:
                            continue  # no pruned rows in this segment
                        n = rng.randint(1, 4)  # the reference records only n > 0 (cache.py:333-340)
                        meta[l][b][h][s] = op.SegMeta(cpu, cpu + n)
                        cpu += n
                    for s in sorted(loaded[b]):  # initially loaded: appended after the kept rows
                        m = meta[l][b][h][s]
                        if m is not None:
                            n = m.cpu_end - m.cpu_start
                            m.gpu_rel_start, m.gpu_rel_end = length, length + n
                            length += n
                seq_lens[l][b * H + h] = length
    return dict(L=L, H=H, B=B, N=N, lag=lag, seg_count=seg_count, c2s=c2s, class_b=class_b, meta=meta,
                loaded=loaded, seq_lens=seq_lens, cpu_rows=cpu, rng=rng)


def make_oracle(sc, top_k):
    return op.PlannerOracle(sc["L"], sc["H"], sc["B"], top_k, sc["lag"], sc["c2s"], sc["class_b"],
                            copy.deepcopy(sc["meta"]), sc["loaded"], sc["seq_lens"])


def make_native(sc, top_k):
    L, H, B = sc["L"], sc["H"], sc["B"]
    p = Planner(L, H, B, 4)
    p.set_config(top_k, sc["lag"])
    p.set_seg_count(sc["seg_count"])
    for b in range(B):
        flat, off = [], [0]
        for segs in sc["c2s"][b]:
            flat += segs
            off.append(len(flat))
        p.set_chunk_to_segs(b, torch.tensor(flat, dtype=torch.int32), torch.tensor(off, dtype=torch.int32))
    for l in range(L):
        p.set_class_b(l, torch.tensor(sc["class_b"][l], dtype=torch.int32))
    cs, ce, gs, ge = [], [], [], []
    for l in range(L):
        for f in range(sc["N"]):
            b, h = divmod(f, H)
            for m in sc["meta"][l][b][h]:
                if m is None:
                    cs.append(-1); ce.append(-1); gs.append(-1); ge.append(-1)  # noqa: E702
                else:
                    cs.append(m.cpu_start); ce.append(m.cpu_end)  # noqa: E702
                    gs.append(m.gpu_rel_start); ge.append(m.gpu_rel_end)  # noqa: E702
    p.set_restore_meta(*(torch.tensor(x, dtype=torch.int32) for x in (cs, ce, gs, ge)))
    for b in range(B):
        p.set_loaded(b, torch.tensor(sorted(sc["loaded"][b]), dtype=torch.int32))
    p.set_seq_lens(torch.tensor([x for row in sc["seq_lens"] for x in row], dtype=torch.int32))
    return p


def native_outputs(L, N):
    return dict(load_starts_2d=torch.empty(L, N, dtype=torch.int32), load_lens_2d=torch.empty(L, N, dtype=torch.int32),
                cu_new_2d=torch.empty(L, N + 1, dtype=torch.int32), new_lens_2d=torch.empty(L, N, dtype=torch.int32),
                evict_offsets_2d=torch.empty(L, N + 1, dtype=torch.int32), evict_max=torch.empty(L, dtype=torch.int32),
                evict_layer_ptr=torch.empty(L + 1, dtype=torch.int32))


def random_topk(rng, sc, top_k):
    out = []
    for b in range(sc["B"]):
        n = len(sc["c2s"][b])
        k = min(top_k, n)
        out.append(rng.sample(range(n), k) if k else [])
    return out


def compare_plan(plan, flag, total, ev_s, ev_e, ranges, outs, L):
    assert flag == int(plan.any_change)
    if not plan.any_change:
        return
    assert total == plan.total
    assert ranges.tolist() == [list(r) for r in plan.cpu_ranges]
    assert outs["load_starts_2d"].tolist() == plan.load_starts
    assert outs["load_lens_2d"].tolist() == plan.load_lens
    assert outs["new_lens_2d"].tolist() == plan.new_lens
    assert outs["cu_new_2d"].tolist() == plan.cu_new
    assert outs["evict_offsets_2d"].tolist() == plan.evict_offsets
    assert outs["evict_max"].tolist() == plan.evict_max
    ptr = [0]
    for l in range(L):
        ptr.append(ptr[-1] + len(plan.evict_starts[l]))
    assert outs["evict_layer_ptr"].tolist() == ptr
    assert ev_s.tolist() == [x for l in range(L) for x in plan.evict_starts[l]]
    assert ev_e.tolist() == [x for l in range(L) for x in plan.evict_ends[l]]


def check_range_layers(ptr, plan, L):
    """The native layer pointer into the ranges: from 0 to the number of
    ranges, non-decreasing, and layer l's ranges hold exactly the rows the
    oracle loads into layer l (sum of its load_lens)."""
    assert len(ptr) == L + 1
    if not plan.any_change:
        assert ptr == [0] * (L + 1)
        return
    assert ptr[0] == 0 and ptr[L] == len(plan.cpu_ranges)
    for l in range(L):
        assert ptr[l] <= ptr[l + 1]
        rows = sum(e - s for s, e in plan.cpu_ranges[ptr[l]:ptr[l + 1]])
        assert rows == sum(plan.load_lens[l]), f"layer {l}"


# ---------------------------------------------------------------------------
def test_oracle_hand_example():
    """1 layer, 1 sample, KV heads 0 (class A) and 1 (class B), 3 segments."""
    meta = [[[[None] * 3, [op.SegMeta(0, 2, 6, 8), op.SegMeta(2, 5), op.SegMeta(5, 7, 8, 10)]]]]
    o = op.PlannerOracle(1, 2, 1, 2, 1, [[[0], [1], [2]]], [[1]], meta, [{0, 2}], [[20, 10]])
    plan = o.step([[1, 2]])  # needs segments {1, 2}: load 1, evict 0 (lag 1)
    assert plan.any_change
    assert plan.evict_starts == [[6]] and plan.evict_ends == [[8]]
    assert plan.evict_offsets == [[0, 0, 1]] and plan.evict_max == [1]
    assert plan.load_starts == [[-1, 0]] and plan.load_lens == [[0, 3]]
    assert plan.new_lens == [[21, 10 - 2 + 3 + 1]]
    assert plan.cu_new == [[0, 21, 33]]
    assert plan.cpu_ranges == [(2, 5)] and plan.total == 3
    m = o.meta[0][0][1]
    assert (m[0].gpu_rel_start, m[0].gpu_rel_end) == (-1, -1)
    assert (m[2].gpu_rel_start, m[2].gpu_rel_end) == (6, 8)    # shifted down by the 2 evicted rows
    assert (m[1].gpu_rel_start, m[1].gpu_rel_end) == (8, 11)   # loaded after the survivors
    assert o.loaded == [{1, 2}]


def test_oracle_eviction_lag():
    """A segment leaves only after `lag` consecutive steps outside the top-k."""
    meta = [[[[op.SegMeta(0, 1, 0, 1), op.SegMeta(1, 2)]]]]
    o = op.PlannerOracle(1, 1, 1, 1, 3, [[[0], [1]]], [[0]], meta, [{0}], [[1]])
    assert o.step([[1]]).any_change  # load 1 (0 misses once)
    o.append_step()
    for _ in range(1):
        assert not o.step([[1]]).any_change  # 0 misses twice
    plan = o.step([[1]])  # third miss: evicted
    assert plan.any_change and plan.evict_starts == [[0]]
    assert o.loaded == [{1}]


_CHANGES: dict[int, int] = {}


@pytest.mark.parametrize("seed", range(12))
def test_native_matches_oracle_multistep(seed):
    sc = make_scenario(seed)
    rng = random.Random(1000 + seed)
    top_k = rng.randint(1, 3)
    o, p = make_oracle(sc, top_k), make_native(sc, top_k)
    L, N = sc["L"], sc["N"]
    o.append_step()  # first decode step: plain append on both sides
    changes = 0
    for step in range(10):
        topk = random_topk(rng, sc, top_k)
        plan = o.step(topk)
        flat = [c for row in topk for c in row]
        off = [0]
        for row in topk:
            off.append(off[-1] + len(row))
        outs = native_outputs(L, N)
        flag, total, ev_s, ev_e, ranges = p.compute_and_prepare(
            torch.tensor(flat, dtype=torch.int32), torch.tensor(off, dtype=torch.int32), **outs)
        compare_plan(plan, flag, total, ev_s, ev_e, ranges, outs, L)
        check_range_layers(p.range_layers(), plan, L)
        for b in range(sc["B"]):
            assert p.get_loaded_segments(b) == sorted(o.loaded[b])
        if not plan.any_change:
            o.append_step()
        changes += int(plan.any_change)
    _CHANGES[seed] = changes


def test_multistep_scenarios_exercise_rebuilds():
    """The random scenarios above are not vacuous: most seeds rebuild."""
    if len(_CHANGES) < 12:
        pytest.skip("run with the multistep cases")
    assert sum(1 for c in _CHANGES.values() if c > 0) >= 8


@pytest.mark.parametrize("seed", range(6))
def test_plan_invariants(seed):
    sc = make_scenario(100 + seed, max_segs=9, lag=1)
    rng = random.Random(seed)
    o = make_oracle(sc, 2)
    for _ in range(6):
        before = copy.deepcopy(o.seq_lens)
        plan = o.step(random_topk(rng, sc, 2))
        if not plan.any_change:
            o.append_step()
            continue
        for l in range(sc["L"]):
            for f in range(sc["N"]):
                e0, e1 = plan.evict_offsets[l][f], plan.evict_offsets[l][f + 1]
                ev = list(zip(plan.evict_starts[l][e0:e1], plan.evict_ends[l][e0:e1]))
                assert ev == sorted(ev)
                for (s, e), nxt in zip(ev, ev[1:] + [(None, None)]):
                    assert 0 <= s < e <= before[l][f]
                    assert nxt[0] is None or e <= nxt[0]
                evicted = sum(e - s for s, e in ev)
                assert plan.new_lens[l][f] == before[l][f] - evicted + plan.load_lens[l][f] + 1
                b, h = divmod(f, sc["H"])
                spans = sorted((m.gpu_rel_start, m.gpu_rel_end) for m in o.meta[l][b][h]
                               if m is not None and m.gpu_rel_start >= 0)
                for (s, e), nxt in zip(spans, spans[1:] + [(None, None)]):
                    assert 0 <= s <= e <= plan.new_lens[l][f] - 1
                    assert nxt[0] is None or e <= nxt[0]


@pytest.mark.parametrize("seed", range(4))
def test_plan_drives_compaction(seed):
    """Plan -> compaction oracle: every resident segment's rows sit at its
    metadata position afterwards (rows carry their host index as payload)."""
    sc = make_scenario(200 + seed, L=2, lag=1)
    rng = random.Random(seed)
    o = make_oracle(sc, 2)
    D = 8
    # layer rows: a row of a resident offloaded segment holds its host row id
    # (+1, so 0 means "not an offloaded row"); other rows are 0.
    layers = []
    for l in range(sc["L"]):
        rows = []
        for f in range(sc["N"]):
            b, h = divmod(f, sc["H"])
            seg = np.zeros((o.seq_lens[l][f], D), np.float32)
            for m in o.meta[l][b][h]:
                if m is not None and m.gpu_rel_start >= 0:
                    seg[m.gpu_rel_start:m.gpu_rel_end, 0] = np.arange(m.cpu_start, m.cpu_end) + 1
            rows.append(seg)
        layers.append(rows)
    host = (np.arange(max(sc["cpu_rows"], 1), dtype=np.float32) + 1)[:, None] * np.eye(1, D, 0, np.float32)
    for _ in range(4):
        plan = o.step(random_topk(rng, sc, 2))
        if not plan.any_change:
            for l in range(sc["L"]):
                layers[l] = [np.vstack([s, np.zeros((1, D), np.float32)]) for s in layers[l]]
            o.append_step()
            continue
        load = np.vstack([host[s:e] for s, e in plan.cpu_ranges]) if plan.cpu_ranges else np.zeros((0, D), np.float32)
        for l in range(sc["L"]):
            old = np.vstack(layers[l]) if layers[l] else np.zeros((0, D), np.float32)
            old_cu = np.array(op.cu_from_lens([len(s) for s in layers[l]]), np.int32)
            new_cu = np.array(plan.cu_new[l], np.int32)
            new_rows = np.zeros((sc["N"], D), np.float32)
            ok, _ = oracle.rebuild_append_kv(
                old, old, new_rows, new_rows, load, load, old_cu, new_cu,
                np.array(plan.load_starts[l], np.int32), np.array(plan.load_lens[l], np.int32),
                np.array(plan.evict_offsets[l], np.int32), np.array(plan.evict_starts[l], np.int32),
                np.array(plan.evict_ends[l], np.int32), plan.evict_max[l], dtype=oracle.DT_F32)
            layers[l] = [ok[new_cu[f]:new_cu[f + 1]] for f in range(sc["N"])]
            for f in range(sc["N"]):
                b, h = divmod(f, sc["H"])
                for m in o.meta[l][b][h]:
                    if m is not None and m.gpu_rel_start >= 0:
                        got = layers[l][f][m.gpu_rel_start:m.gpu_rel_end, 0]
                        np.testing.assert_array_equal(got, np.arange(m.cpu_start, m.cpu_end) + 1)


def test_gather_restore_copies_ranges_in_order():
    sc = make_scenario(7, lag=1)
    p = make_native(sc, 2)
    rows = max(sc["cpu_rows"], 1)
    cpu_k = torch.arange(rows * 4, dtype=torch.float32).view(rows, 4)
    cpu_v = -cpu_k
    stg_k, stg_v = torch.zeros(rows, 4), torch.zeros(rows, 4)
    p.set_restore_buffers(cpu_k, cpu_v, stg_k, stg_v)
    o = make_oracle(sc, 2)
    o.append_step()
    rng = random.Random(3)
    for _ in range(8):
        topk = random_topk(rng, sc, 2)
        plan = o.step(topk)
        off = [0]
        for row in topk:
            off.append(off[-1] + len(row))
        flag, total, _, _, ranges = p.compute_and_prepare(
            torch.tensor([c for r in topk for c in r], dtype=torch.int32), torch.tensor(off, dtype=torch.int32),
            **native_outputs(sc["L"], sc["N"]))
        if not flag:
            o.append_step()
            continue
        p.gather_restore()
        want = torch.cat([cpu_k[s:e] for s, e in ranges.tolist()]) if total else torch.zeros(0, 4)
        assert torch.equal(stg_k[:total], want) and torch.equal(stg_v[:total], -want)


def test_native_rejects_bad_indices():
    from wnw_amd import _lib
    sc = make_scenario(9)
    p = make_native(sc, 2)
    with pytest.raises(_lib.WnwError):
        p.compute_and_prepare(torch.tensor([999], dtype=torch.int32),
                              torch.tensor([0, 1] + [1] * (sc["B"] - 1), dtype=torch.int32),
                              **native_outputs(sc["L"], sc["N"]))
    with pytest.raises(_lib.WnwError):
        p.set_loaded(0, torch.tensor([sc["seg_count"][0] + 5], dtype=torch.int32))
    with pytest.raises(_lib.WnwError):
        p.set_class_b(0, torch.tensor([sc["H"]], dtype=torch.int32))


def test_range_layers_before_any_plan_and_short_output():
    """Before any plan the layer pointer is all zeros; an output shorter than
    L + 1 entries is refused (no write past it)."""
    import ctypes

    from wnw_amd import _lib
    sc = make_scenario(11)
    p = make_native(sc, 2)
    assert p.range_layers() == [0] * (sc["L"] + 1)
    short = (ctypes.c_int32 * sc["L"])()
    assert _lib.lib().wnw_planner_get_range_layers(p._h, short, sc["L"]) != 0

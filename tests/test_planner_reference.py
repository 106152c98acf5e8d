"""Decode chunk planner against the reference's own C++ planner.

The reference planner (src/algorithms/wnw_cpp/code/planner.cpp:18-341, a
single-file PyTorch extension) is compiled from its source by ``make -C
oracle ref`` into ``oracle/_ref/`` (a checker only; built by
``__graft_entry__.build()`` where the reference tree is present).  Every
scenario below is driven through three planners with the same calls: the
reference, the native planner of this package (wnw_amd/csrc/planner.cpp
through the C ABI) and the Python restatement (oracle/planner.py); every
plan output, the loaded-chunk sets and the staging gather must agree bit
for bit.  CPU only; skipped where the reference module is not built.
"""
from __future__ import annotations

import os
import random
import sys

import pytest
import torch

from tests.test_planner import (compare_plan, make_native, make_oracle, make_scenario, native_outputs,
                                random_topk)

_REF_DIR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref")


def _ref_module():
    if _REF_DIR not in sys.path:
        sys.path.insert(0, _REF_DIR)
    try:
        import wnw_ref_planner  # noqa: PLC0415
    except ImportError:
        pytest.skip("the reference planner is not built (make -C oracle ref, needs the reference tree)")
    return wnw_ref_planner


def make_reference(sc, top_k):
    """The reference planner set up with make_native's calls (the same method
    names and arguments: wnw_cpp/code/cache.py:60-116)."""
    mod = _ref_module()
    L, H, B = sc["L"], sc["H"], sc["B"]
    p = mod.Planner(L, H, B, 4)
    p.set_config(top_k, sc["lag"])
    p.set_seg_count(list(sc["seg_count"]))
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
                cs.append(-1 if m is None else m.cpu_start)
                ce.append(-1 if m is None else m.cpu_end)
                gs.append(-1 if m is None else m.gpu_rel_start)
                ge.append(-1 if m is None else m.gpu_rel_end)
    p.set_restore_meta(*(torch.tensor(x, dtype=torch.int32) for x in (cs, ce, gs, ge)))
    for b in range(B):
        p.set_loaded(b, torch.tensor(sorted(sc["loaded"][b]), dtype=torch.int32))
    p.set_seq_lens(torch.tensor([x for row in sc["seq_lens"] for x in row], dtype=torch.int32))
    return p


def _outs_equal(a, b):
    return all(torch.equal(a[k], b[k]) for k in a)


_SHAPES = [dict(), dict(L=4, H=4, B=3, max_segs=9), dict(L=2, H=8, B=1, max_segs=12, lag=1),
           dict(L=5, H=2, B=4, max_segs=6, lag=3)]


@pytest.mark.parametrize("shape", range(len(_SHAPES)))
@pytest.mark.parametrize("seed", range(10))
def test_reference_native_oracle_agree(seed, shape):
    sc = make_scenario(500 + 37 * seed + shape, **_SHAPES[shape])
    rng = random.Random(7000 + seed)
    top_k = rng.randint(1, 4)
    ref, nat, orc = make_reference(sc, top_k), make_native(sc, top_k), make_oracle(sc, top_k)
    L, N = sc["L"], sc["N"]
    rows = max(sc["cpu_rows"], 1)
    cpu_k = torch.arange(rows * 8, dtype=torch.float32).view(rows, 8)
    cpu_v = 0.5 - cpu_k
    stg = [torch.zeros(rows, 8) for _ in range(4)]
    ref.set_restore_buffers(cpu_k, cpu_v, stg[0], stg[1])
    nat.set_restore_buffers(cpu_k, cpu_v, stg[2], stg[3])
    orc.append_step()  # the first decode step appends on every side (the planners' lengths include it)
    changed = 0
    for step in range(12):
        topk = random_topk(rng, sc, top_k)
        flat = torch.tensor([c for row in topk for c in row], dtype=torch.int32)
        off = [0]
        for row in topk:
            off.append(off[-1] + len(row))
        off = torch.tensor(off, dtype=torch.int32)
        o_ref, o_nat = native_outputs(L, N), native_outputs(L, N)
        r = ref.compute_and_prepare(flat, off, o_ref["load_starts_2d"], o_ref["load_lens_2d"], o_ref["cu_new_2d"],
                                    o_ref["new_lens_2d"], o_ref["evict_offsets_2d"], o_ref["evict_max"],
                                    o_ref["evict_layer_ptr"])
        n = nat.compute_and_prepare(flat, off, **o_nat)
        plan = orc.step(topk)
        assert int(r[0]) == int(n[0]) and int(r[1]) == int(n[1]), f"step {step}: flag/total differ"
        if r[0]:
            assert _outs_equal(o_ref, o_nat), f"step {step}: descriptor arrays differ"
            for a, b in zip(r[2:], n[2:]):
                assert torch.equal(a, b), f"step {step}: eviction ranges or host ranges differ"
            compare_plan(plan, *r, o_ref, L)  # and the restatement
            ref.gather_restore()
            nat.gather_restore()
            t = int(r[1])
            assert torch.equal(stg[0][:t], stg[2][:t]) and torch.equal(stg[1][:t], stg[3][:t])
            changed += 1
        else:
            assert not plan.any_change
            orc.append_step()
        for b in range(sc["B"]):
            assert sorted(ref.get_loaded_segments(b)) == nat.get_loaded_segments(b) == sorted(orc.loaded[b])
    _CHANGED[(seed, shape)] = changed


_CHANGED: dict = {}


def test_reference_scenarios_are_not_vacuous():
    """Most of the scenarios above change the layout at least once."""
    if len(_CHANGED) < 10 * len(_SHAPES):
        pytest.skip("run with the agreement cases")
    assert sum(1 for c in _CHANGED.values() if c > 0) >= 0.75 * len(_CHANGED)

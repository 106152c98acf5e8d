"""Native planner and restatement against golden plan vectors of the
reference's own C++ planner (tests/golden/planner_ref_vectors.json.gz,
written by tests/golden/make_planner_vectors.py from
src/algorithms/wnw_cpp/code/planner.cpp compiled into oracle/_ref).

The fixture holds each scenario's inputs in full and the reference's
outputs at every step, so this check runs wherever the tests run, with or
without the reference tree: the native planner (wnw_amd/csrc/planner.cpp
through the C ABI) and oracle/planner.py are driven with the stored inputs
and must reproduce every output bit for bit.  CPU only.
"""
from __future__ import annotations

import gzip
import json
import os

import pytest
import torch

import oracle.planner as op
from tests.test_planner import compare_plan, make_native, make_oracle, native_outputs

_FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "planner_ref_vectors.json.gz")


def _load():
    with gzip.open(_FIXTURE, "rt") as f:
        return json.load(f)["scenarios"]


_SCENARIOS = _load()


def _scenario(inp):
    """The scenario dict of tests/test_planner.py rebuilt from the stored
    set-up (restore metadata in (layer, segment row, segment) order)."""
    L, H, B = inp["L"], inp["H"], inp["B"]
    N = B * H
    meta = [[[[None] * inp["seg_count"][b] for _ in range(H)] for b in range(B)] for _ in range(L)]
    cs, ce, gs, ge = inp["restore"]
    i = 0
    for l in range(L):
        for f in range(N):
            b, h = divmod(f, H)
            for s in range(inp["seg_count"][b]):
                if cs[i] >= 0:
                    meta[l][b][h][s] = op.SegMeta(cs[i], ce[i], gs[i], ge[i])
                i += 1
    assert i == len(cs), "restore metadata length"
    return dict(L=L, H=H, B=B, N=N, lag=inp["lag"], seg_count=inp["seg_count"],
                c2s=[[list(c) for c in row] for row in inp["c2s"]], class_b=inp["class_b"], meta=meta,
                loaded=[set(x) for x in inp["loaded"]], seq_lens=[list(x) for x in inp["seq_lens"]],
                cpu_rows=inp["cpu_rows"])


class _Stored:
    """A reference plan as compare_plan reads it."""

    def __init__(self, st, L):
        self.any_change = bool(st["flag"])
        self.total = st["total"]
        self.cpu_ranges = [tuple(r) for r in st["ranges"]]
        self.load_starts, self.load_lens = st["load_starts_2d"], st["load_lens_2d"]
        self.new_lens, self.cu_new, self.evict_offsets = st["new_lens_2d"], st["cu_new_2d"], st["evict_offsets_2d"]
        self.evict_max = st["evict_max"]
        ptr = st["evict_layer_ptr"]
        self.evict_starts = [st["ev_s"][ptr[l]:ptr[l + 1]] for l in range(L)]
        self.evict_ends = [st["ev_e"][ptr[l]:ptr[l + 1]] for l in range(L)]


def test_fixture_is_not_vacuous():
    assert len(_SCENARIOS) >= 12
    changed = sum(1 for sc in _SCENARIOS if any(st["flag"] for st in sc["steps"]))
    assert changed >= 0.75 * len(_SCENARIOS)
    assert any(st.get("ev_s") for sc in _SCENARIOS for st in sc["steps"])  # evictions occur
    assert any(st.get("ranges") for sc in _SCENARIOS for st in sc["steps"])  # loads occur


@pytest.mark.parametrize("i", range(len(_SCENARIOS)))
def test_native_and_oracle_match_reference_vectors(i):
    rec = _SCENARIOS[i]
    inp = rec["inputs"]
    sc = _scenario(inp)
    L, N, B = sc["L"], sc["N"], sc["B"]
    nat, orc = make_native(sc, inp["top_k"]), make_oracle(sc, inp["top_k"])
    rows = max(sc["cpu_rows"], 1)
    cpu_k = torch.arange(rows * 8, dtype=torch.float32).view(rows, 8)
    stg_k, stg_v = torch.zeros(rows, 8), torch.zeros(rows, 8)
    nat.set_restore_buffers(cpu_k, 0.5 - cpu_k, stg_k, stg_v)
    orc.append_step()  # the first decode step appends on every side (the planners' lengths include it)
    for t, st in enumerate(rec["steps"]):
        topk = st["topk"]
        flat = torch.tensor([c for row in topk for c in row], dtype=torch.int32)
        off = [0]
        for row in topk:
            off.append(off[-1] + len(row))
        o = native_outputs(L, N)
        n = nat.compute_and_prepare(flat, torch.tensor(off, dtype=torch.int32), **o)
        plan = orc.step(topk)
        assert (int(n[0]), int(n[1])) == (st["flag"], st["total"]), f"step {t}: flag/total"
        if st["flag"]:
            stored = _Stored(st, L)
            compare_plan(stored, *n, o, L)  # native outputs = the reference's
            compare_plan(plan, *n, o, L)    # and the restatement's
            nat.gather_restore()
            tot = st["total"]
            assert [int(x) for x in stg_k[:tot, 0].tolist()] == st["stg_k_col0"], f"step {t}: staging gather"
            assert torch.equal(stg_v[:tot], 0.5 - stg_k[:tot])
        else:
            assert not plan.any_change
            orc.append_step()
        for b in range(B):
            assert nat.get_loaded_segments(b) == st["loaded"][b] == sorted(orc.loaded[b]), f"step {t}: loaded"

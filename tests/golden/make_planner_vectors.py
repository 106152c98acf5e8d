"""Writes tests/golden/planner_ref_vectors.json.gz: decode-plan vectors from
the reference's own C++ planner (src/algorithms/wnw_cpp/code/planner.cpp,
compiled from its source into oracle/_ref by ``make -C oracle ref``).

Each scenario stores its inputs in full (planner configuration, chunk map,
class-B heads, restore metadata, loaded sets, lengths, and the top-k chunks
fed at every step) and the reference planner's outputs at every step: the
change flag and row total, every descriptor array, the eviction and host
ranges, the staging gather (first column of the gathered K rows: host K row
r holds 8r .. 8r + 7, so it names the source row) and the loaded sets.
``tests/test_planner_golden.py`` replays the inputs through the native
planner and the restatement and compares.  Run from the repository root:

    make -C oracle ref && python tests/golden/make_planner_vectors.py
"""
from __future__ import annotations

import gzip
import json
import os
import random
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

from tests.test_planner import make_scenario, native_outputs, random_topk  # noqa: E402
from tests.test_planner_reference import _SHAPES, make_reference  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden", "planner_ref_vectors.json.gz")
STEPS = 12


def scenario_inputs(sc, top_k):
    """The scenario as the planner's set-up calls see it (make_reference)."""
    L, H, B, N = sc["L"], sc["H"], sc["B"], sc["N"]
    restore = [[], [], [], []]
    for l in range(L):
        for f in range(N):
            b, h = divmod(f, H)
            for m in sc["meta"][l][b][h]:
                restore[0].append(-1 if m is None else m.cpu_start)
                restore[1].append(-1 if m is None else m.cpu_end)
                restore[2].append(-1 if m is None else m.gpu_rel_start)
                restore[3].append(-1 if m is None else m.gpu_rel_end)
    return dict(L=L, H=H, B=B, lag=sc["lag"], top_k=top_k, seg_count=list(sc["seg_count"]),
                c2s=[[list(c) for c in sc["c2s"][b]] for b in range(B)], class_b=[list(x) for x in sc["class_b"]],
                restore=restore, loaded=[sorted(sc["loaded"][b]) for b in range(B)],
                seq_lens=[list(x) for x in sc["seq_lens"]], cpu_rows=sc["cpu_rows"])


def main():
    from tests.test_planner_reference import _ref_module
    _ref_module()  # raises (skip) when the reference planner is not built
    scenarios = []
    for shape in range(len(_SHAPES)):
        for seed in range(3):
            sc = make_scenario(900 + 41 * seed + shape, **_SHAPES[shape])
            rng = random.Random(9100 + 7 * seed + shape)
            top_k = rng.randint(1, 4)
            ref = make_reference(sc, top_k)
            L, N = sc["L"], sc["N"]
            rows = max(sc["cpu_rows"], 1)
            cpu_k = torch.arange(rows * 8, dtype=torch.float32).view(rows, 8)
            cpu_v = 0.5 - cpu_k
            stg_k, stg_v = torch.zeros(rows, 8), torch.zeros(rows, 8)
            ref.set_restore_buffers(cpu_k, cpu_v, stg_k, stg_v)
            steps = []
            for _ in range(STEPS):
                topk = random_topk(rng, sc, top_k)
                flat = torch.tensor([c for row in topk for c in row], dtype=torch.int32)
                off = [0]
                for row in topk:
                    off.append(off[-1] + len(row))
                o = native_outputs(L, N)
                r = ref.compute_and_prepare(flat, torch.tensor(off, dtype=torch.int32), o["load_starts_2d"],
                                            o["load_lens_2d"], o["cu_new_2d"], o["new_lens_2d"],
                                            o["evict_offsets_2d"], o["evict_max"], o["evict_layer_ptr"])
                st = dict(topk=topk, flag=int(r[0]), total=int(r[1]))
                if r[0]:
                    st.update({k: v.tolist() for k, v in o.items()})
                    st["ev_s"], st["ev_e"], st["ranges"] = r[2].tolist(), r[3].tolist(), r[4].tolist()
                    ref.gather_restore()
                    t = int(r[1])
                    st["stg_k_col0"] = [int(x) for x in stg_k[:t, 0].tolist()]
                st["loaded"] = [sorted(ref.get_loaded_segments(b)) for b in range(sc["B"])]
                steps.append(st)
            scenarios.append(dict(inputs=scenario_inputs(sc, top_k), steps=steps))
    with gzip.open(OUT, "wt") as f:
        json.dump({"source": "src/algorithms/wnw_cpp/code/planner.cpp (compiled from the reference)",
                   "scenarios": scenarios}, f, separators=(",", ":"))
    print(f"wrote {OUT}: {len(scenarios)} scenarios x {STEPS} steps "
          f"({sum(s['flag'] for sc in scenarios for s in sc['steps'])} plans with changes)")


if __name__ == "__main__":
    main()

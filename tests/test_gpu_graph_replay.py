"""The benchmark's timed path under parity: whole decode steps through
WnWCache captured as HIP graphs and replayed, as bench.py times them.

Workload: the first 3 layers of the cfg2 state at full size (bench.py's
``build_cache``: 64 segments per layer, 7,564-row class-A and 512-row
class-B segments, slack pools) and bench.py's fixed step inputs.  The test

1. runs two eager decode steps, each checked by ``DecodeSimulation``;
2. captures two whole steps (``decode_attention`` over every layer, the
   end-of-step hook included) on a side stream, as bench.py does, replays
   them alternately 6 times and calls ``advance_replayed_steps(4)`` (the
   captures ran the host side of 2 steps);
3. captures the fused launches alone twice (bench.py's roofline graphs),
   replays them 4 times and advances the host by 2;
4. after each replay phase compares every layer's logical K/V rows and
   device offsets with the oracle's appends of the replayed rows
   (bit-exact), the host lengths and row counts, and the last replay's
   attention outputs with ``oracle.decode_attn`` (2e-3 + 1e-2 |ref|);
5. runs two more eager steps against the simulation (the host bookkeeping
   after the replays drives the next launches).

With ``score`` the class-A heads are scored (foldable layers score inside
the attention launch); the eager steps check the scores (1e-6 + 1e-3 |ref|).
"""
import os
import sys

import pytest
import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import bench  # noqa: E402
from tests.cache_sim import DecodeSimulation, recording  # noqa: E402
from wnw_amd import _lib, workloads  # noqa: E402
from wnw_amd.kv import fused_attn  # noqa: E402
from wnw_amd.wnw.cache import WnWCache  # noqa: E402
from wnw_amd.wnw.session import decode_attention  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("score", [False, True])
def test_replayed_cfg2_steps_match_oracle(score):
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cfg = workloads.config2(layers=3)
    L, N, G, D = cfg.layers, cfg.n_seg, cfg.group, cfg.head_dim
    print(f"graph replay: cfg2 first {L} layers, score={score}", flush=True)
    cache = bench.build_cache(cfg, dev, slack_rows=32, score=score, cls=recording(WnWCache))
    cache.rec_acc, cache.rec_topk = [], []
    sim = DecodeSimulation(cache, [(0, int(a)) for a in cfg.audio])
    inputs = bench.step_inputs(cfg, dev)
    qs, ks, vs = ([x[i] for x in inputs] for i in range(3))
    scale = D ** -0.5

    def step():
        return [decode_attention(cache, l, q, k, v, scale, fused=True) for l, (q, k, v) in enumerate(inputs)]

    t = 0
    for _ in range(2):
        outs = step()
        torch.cuda.synchronize()
        assert _lib.device_error() == 0, f"eager step {t}"
        sim.step(t, qs, ks, vs, outs)
        t += 1

    stream = torch.cuda.Stream(device=dev)  # default priority
    with torch.cuda.stream(stream):  # the capture stream's workspace, made before capture
        fused_attn.workspace_for(dev).get(N, G, D)
        if score:
            fused_attn.workspace_for(dev).get(N, G, D, score=True, max_audio=cache._max_audio)
    torch.cuda.synchronize()

    # whole steps, two captures alternating the offset buffers
    graphs, graph_outs = [], []
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            graph_outs.append(step())
        graphs.append(g)
    n = 6
    with torch.cuda.stream(stream):
        for i in range(n):
            graphs[i % 2].replay()
    stream.synchronize()
    assert _lib.device_error() == 0, "step graph replays"
    cache.advance_replayed_steps(n - 2)
    for _ in range(n):
        sim.advance_plain(ks, vs)
    for l in range(L):
        sim.check_layer(f"after {n} step replays", l, qs[l], graph_outs[(n - 1) % 2][l])

    # the fused launches alone (bench.py's roofline graphs): no end-of-step hook
    fgraphs, fouts = [], []
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fouts.append([cache.decode_step_attention(l, q.view(N, G, D), q, k, v, scale, True)
                          for l, (q, k, v) in enumerate(inputs)])
        fgraphs.append(g)
    n = 4
    with torch.cuda.stream(stream):
        for i in range(n):
            fgraphs[i % 2].replay()
    stream.synchronize()
    assert _lib.device_error() == 0, "fused graph replays"
    cache.advance_replayed_steps(n - 2)
    for _ in range(n):
        sim.advance_plain(ks, vs)
    for l in range(L):
        sim.check_layer(f"after {n} fused replays", l, qs[l], fouts[(n - 1) % 2][l].view(N, G, D))
    if score:
        # the fused-launch replays scored into the accumulator without the
        # end-of-step hook that clears it: start the eager steps from zero
        cache.score_accumulator.zero_()

    # eager steps again, driven by the advanced host state
    for _ in range(2):
        outs = step()
        torch.cuda.synchronize()
        assert _lib.device_error() == 0, f"eager step {t}"
        sim.step(t, qs, ks, vs, outs)
        t += 1
    assert len(cache.rec_acc) == t, "captured steps must record nothing"


def test_replay_bookkeeping_refuses_unsound_counts():
    """advance_replayed_steps refuses an odd count (the offsets buffers
    would be swapped), more steps than the slack holds, and chunk selection
    (a replay skips the per-step plan)."""
    dev = torch.device("cuda", 0)
    cfg = workloads.config2(layers=1)
    cfg.lengths = [x[:] // 64 + 1 for x in cfg.lengths]  # small segments: the rule checks need no size
    cache = bench.build_cache(cfg, dev, slack_rows=8, score=False)
    rows = list(cache._rows)
    with pytest.raises(ValueError):
        cache.advance_replayed_steps(3)
    with pytest.raises(ValueError):
        cache.advance_replayed_steps(-2)
    with pytest.raises(ValueError):
        cache.advance_replayed_steps(cache.decode_headroom() // 2 * 2 + 2)
    cache._tk_k = 1
    with pytest.raises(ValueError):
        cache.advance_replayed_steps(2)
    cache._tk_k = 0
    assert cache._rows == rows
    cache.advance_replayed_steps(2)
    assert cache._rows == [r + 2 * cfg.n_seg for r in rows]

#!/usr/bin/env python3
"""Decode-step attention benchmark on one MI355X (BASELINE.json metric).

Workload (default ``--config cfg2``): Voxtral-Mini-3B decode shape, 30 layers,
32 query / 8 KV heads, head_dim 128, bf16, batch 8, 7,500 audio + 64 text
tokens per sequence; per layer 2 of 8 KV heads are class A (full KV, 7,564
rows), the others class B (512 rows).  Synthetic data: K, V ~ N(0, 1) times
a per-(layer, KV head) scale from U(0.5, 2), q ~ N(0, 1).

The step runs through the drop-in: a ``WnWCache`` (slack layout) holding
that state, driven per layer by ``wnw_amd.wnw.session.decode_attention``
(the decode branch of the patched attention forward), which appends the
step's K/V row to every segment and attends in one kernel launch, then
``decode_all_layers_done`` after the last layer.  The configuration offloads
nothing (class-B rows are the prefill's survivors), so no step changes the
layout.  Every layer has its own pool (~2.3 GB in all), far beyond the
256 MB Infinity Cache.  The step is captured as HIP graphs (two, for the
alternating offset buffers) and replayed, so the timed region measures the
GPU, not Python; the eager step is timed as well.

Reported:
* value / ms_per_step -- whole decode step through the cache, replayed from
                    graphs: algorithmic bytes (K/V rows attended + q/o + the
                    appended rows) of the timed steps / wall time.
* ms_per_step_eager -- the same step launched from Python.
* us_per_layer_step -- the fused append + attention launch, per layer-step
                    (HIP events around graph replays of the 30 launches);
                    roofline.achieved = its algorithmic bytes / that time.
* attn_only_us_per_layer_step -- attention without the append, same state.
* compaction    -- the rebuild (compaction + append, ``rebuild_append_kv``)
                    kernel on the reference's dense layout, per layer:
                    class-B segments drop their oldest window row, every
                    segment gets a new row; µs per layer and TB/s moved.
* compaction_slack -- the same eviction as the cache's slack layout runs it
                    (``compact_segments``: only the class-B segments move,
                    into a free region; the append is fused into the
                    attention launch).
* cpu_baseline  -- the reference's decode layer-step restated in PyTorch
                    (torch.cat append + per-segment float32 attention) on the
                    host's cores, on a bounded sample of the same layers.
* extras        -- (default cfg2 run only; ``--no-extras`` skips them) child
                    runs of this script before this process touches the GPU:
                    cfg2 with class-A scoring (deferred, then the separate
                    scoring pass) and the cfg4 offload step, so that the
                    default run reports them too.

``--copy-calibration`` only runs a plain 256 MiB device-to-device copy three
times (for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes).
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "decode-attn µs/layer-step + achieved HBM TB/s (% of MI355X peak), 1 GPU"


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="cfg2", choices=["cfg2", "cfg3", "cfg4", "cfg5"],
                    help="cfg4 runs whole decode steps through the cache with host->device chunk fetches")
    ap.add_argument("--attn-reps", type=int, default=20, help="graph replays of the 30 launches for the roofline")
    ap.add_argument("--score", action="store_true",
                    help="configure the class-A heads as scored (foldable layers score inside the launch)")
    ap.add_argument("--cpu-sample-layers", type=int, default=0,
                    help="layers timed for the CPU baseline (0 = choose ~15 s of work)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-compaction", action="store_true", help="skip the compaction and append timings")
    ap.add_argument("--no-graph", action="store_true", help="time eager steps only")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the child runs (scoring, cfg4) that the default cfg2 run adds to its line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy three times (PMC byte calibration)")
    ap.add_argument("--yardstick", action="store_true",
                    help="only time the read-only streaming kernel (wnw_read_stream) at the attention launches' "
                         "sizes, forms and grids")
    ap.add_argument("--yardstick-grids", default="256,512,1024,2048")
    ap.add_argument("--yardstick-forms", default="0,2,4,8")
    return ap.parse_args()


COPY_CAL_BYTES = 256 << 20


def copy_calibration():
    """A plain copy kernel of known size: reads and writes COPY_CAL_BYTES each."""
    import torch

    dev = torch.device("cuda", 0)
    a = torch.ones(COPY_CAL_BYTES // 4, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": COPY_CAL_BYTES, "launches": 3}), flush=True)


# bytes per fused attention launch of the timed steps (the bench lines'
# bytes_per_launch), rounded down to the yardstick's 8 KB granule
YARDSTICK_SIZES = {"cfg2": 80265216, "cfg3": 118449152, "cfg5": 447935948}


def yardstick(grids: list[int], forms: list[int], reps: int = 10) -> None:
    """Read-only streaming kernel (``wnw_read_stream``) at each attention
    launch size: a graph of launches over buffers cycled past the 256 MB
    Infinity Cache (at least 2.4 GB in all, so every launch reads cold
    data), replayed ``reps`` times, HIP events on the replay stream.  One
    JSON line per (size, form, grid): µs per launch and TB/s."""
    import torch

    from wnw_amd import _lib

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _lib.ensure_init(dev)
    stream = torch.cuda.Stream(device=dev)  # default priority
    sink = torch.zeros(max(grids) * 256, dtype=torch.int32, device=dev)
    best = {}
    for name, size in YARDSTICK_SIZES.items():
        size = size // 8192 * 8192
        n_buf = max(4, -(-(2400 << 20) // size))
        bufs = [torch.randint(-(2 ** 31), 2 ** 31 - 1, (size // 4,), dtype=torch.int32, device=dev)
                for _ in range(n_buf)]
        torch.cuda.synchronize()
        for form in forms:
            for grid in grids:
                def launches():
                    for b in bufs:
                        _lib.check(_lib.lib().wnw_read_stream(_lib.ptr(b), size, grid, form, _lib.ptr(sink),
                                                              _lib.stream_of(dev)), "read_stream")

                with torch.cuda.stream(stream):
                    launches()
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g, stream=stream):
                        launches()
                    g.replay()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    for _ in range(reps):
                        g.replay()
                    e1.record(stream)
                    e1.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / (reps * n_buf)
                tbs = size / (us * 1e-6) / 1e12
                print(json.dumps({"yardstick": name, "bytes_per_launch": size, "form": form, "grid": grid,
                                  "us_per_launch": round(us, 3), "TBs": round(tbs, 3),
                                  "frac_of_peak": round(tbs * 1e3 / HBM_PEAK_GBS, 4)}), flush=True)
                if name not in best or us < best[name]["us_per_launch"]:
                    best[name] = {"form": form, "grid": grid, "us_per_launch": round(us, 3), "TBs": round(tbs, 3)}
                del g
        del bufs
        torch.cuda.synchronize()
    print(json.dumps({"yardstick_best": best}), flush=True)


def build_cache(cfg, dev, slack_rows: int, score: bool, cls=None):
    """A WnWCache (or ``cls``, a subclass) holding the workload's state, as a
    prefill would leave it: every layer's segments of cfg.lengths rows, no
    host rows, nothing offloaded.  With ``score`` the class-A KV heads' query
    heads are configured class A (scored every step)."""
    import numpy as np
    import torch

    from wnw_amd.wnw.cache import WnWCache
    from wnw_amd.wnw.config import WnWConfig

    L, B, Hq, Hkv, D = cfg.layers, cfg.batch, cfg.hq, cfg.hkv, cfg.head_dim
    G = Hq // Hkv
    class_a = [l * Hq + kv * G + g for l in range(L) for kv in range(Hkv) if cfg.class_a[l][kv]
               for g in range(G)] if score else []
    conf = WnWConfig(chunk_size_s=256, overlap_s=0, token_rate=1.0, class_a=class_a, class_b=[],
                     retention_ratios=[None] * (L * Hkv), top_k_chunks=0, eviction_lag=2, prefill_score_mode="last",
                     num_layers=L, num_kv_heads=Hkv, num_q_heads=Hq)
    cache = (cls or WnWCache)(conf, L, Hkv, Hq, D, dev, slack_rows=slack_rows)
    cache.collect_stats(0)  # no memory snapshots: a captured step runs the host side once
    audio = cfg.audio.astype(np.int64)
    cache.setup_audio(torch.zeros(B, dtype=torch.int64, device=dev), torch.from_numpy(audio).to(dev), None)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    layer_k, layer_v, seq_lens = [], [], []
    for l in range(L):
        lens = cfg.lengths[l].astype(np.int64)
        scale_seg = np.tile(cfg.kv_scale[l], B).astype(np.float32)  # segment s = b * Hkv + h
        row_scale = torch.from_numpy(np.repeat(scale_seg, lens)).to(dev).unsqueeze(1)
        rows = int(lens.sum())
        layer_k.append((torch.randn(rows, D, device=dev, generator=gen) * row_scale).to(torch.bfloat16))
        layer_v.append((torch.randn(rows, D, device=dev, generator=gen) * row_scale).to(torch.bfloat16))
        seq_lens.append([int(x) for x in lens])
        del row_scale
    empty = torch.empty(0, D, dtype=torch.bfloat16).pin_memory()
    cache.load_prefilled_state(layer_k, layer_v, seq_lens, empty, empty, cache.restore_meta,
                               [set() for _ in range(B)])
    del layer_k, layer_v
    torch.cuda.synchronize()
    return cache


def step_inputs(cfg, dev, seed: int = 1):
    """The step's q and new K/V row of every layer (fixed tensors: a captured
    graph replays the same addresses)."""
    import torch

    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    B, Hq, Hkv, D = cfg.batch, cfg.hq, cfg.hkv, cfg.head_dim
    out = []
    for _ in range(cfg.layers):
        q = torch.randn(B, Hq, 1, D, device=dev, generator=gen).to(torch.bfloat16)
        k = torch.randn(B, Hkv, 1, D, device=dev, generator=gen).to(torch.bfloat16)
        v = torch.randn(B, Hkv, 1, D, device=dev, generator=gen).to(torch.bfloat16)
        out.append((q, k, v))
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the decode path is single-GPU "
              "per process and multi-GPU runs are not part of this build", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.yardstick:
        yardstick([int(x) for x in args.yardstick_grids.split(",")], [int(x) for x in args.yardstick_forms.split(",")])
        return
    if args.config == "cfg4":
        from wnw_amd import offload_bench

        print(json.dumps({**offload_bench.run(args.steps, args.warmup), "n_gpus": 1}), flush=True)
        return
    extras = None
    if args.config == "cfg2" and not args.score and not args.no_extras:
        extras = extra_legs()

    import numpy as np
    import torch

    from wnw_amd import _lib, workloads
    from wnw_amd.kv import fused_attn
    from wnw_amd.wnw.session import decode_attention

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _lib.lib()
    _lib.ensure_init(dev)
    cfg = workloads.CONFIGS[args.config]()
    L, N, G, D = cfg.layers, cfg.n_seg, cfg.group, cfg.head_dim
    graph = not args.no_graph
    warm_even = args.warmup + args.warmup % 2
    steps_even = args.steps + args.steps % 2
    # appends of the run: the eager steps, and with graphs two captured steps,
    # their replays, two captured sets of fused launches and their replays;
    # the slack covers them all, so no pool is rebuilt on the way
    appends = args.warmup + args.steps
    if graph:
        appends += 2 + 2 + warm_even + steps_even + 2 + 2 + 2 * args.attn_reps
    cache = build_cache(cfg, dev, slack_rows=appends + 16, score=args.score)
    inputs = step_inputs(cfg, dev)
    scale = D ** -0.5
    print(f"# config {cfg.name}: layers={L} n_seg={N} G={G} D={D} steps={args.steps} warmup={args.warmup} "
          f"score={args.score}", flush=True)

    def step():
        for l, (q, k, v) in enumerate(inputs):
            decode_attention(cache, l, q, k, v, scale, fused=True)

    def launch_bytes(rows_before: int) -> int:
        """Algorithmic bytes of one fused launch: K/V of every row after the
        append, q in, o out, and the appended rows (read and written)."""
        return (rows_before + N) * D * 2 * 2 + 2 * N * G * D * 2 + N * D * 2 * 2 * 2

    def steps_bytes(rows_before: list[int], n: int) -> int:
        return sum(launch_bytes(r + i * N) for i in range(n) for r in rows_before)

    # ---- eager steps (Python per layer) -----------------------------------
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    rows_eager = list(cache._rows)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    eager_s = (time.perf_counter() - t0) / args.steps
    assert _lib.device_error() == 0, "device error during the eager steps"
    value = steps_bytes(rows_eager, args.steps) / (eager_s * args.steps) / 1e12

    fused_us = attn_us = step_s = achieved = attn_gbs = fused_bytes = None
    rows_attn = list(cache._rows)
    if graph:
        stream = torch.cuda.Stream(device=dev)  # default priority
        with torch.cuda.stream(stream):  # workspaces of the capture stream, made before capture
            fused_attn.workspace_for(dev).get(N, G, D)
            if args.score:
                fused_attn.workspace_for(dev).get(N, G, D, score=True, max_audio=cache._max_audio)
        torch.cuda.synchronize()
        rows_dev = list(cache._rows)  # the device state before any capture
        # whole decode steps through the cache: two captures (alternating offsets)
        step_graphs = []
        for _ in range(2):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                step()
            step_graphs.append(g)
        # the fused launches alone (no end-of-step hook)
        fused_graphs = []
        for _ in range(2):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for l, (q, k, v) in enumerate(inputs):
                    q_flat = q.squeeze(2).reshape(N, G, D)
                    cache.decode_step_attention(l, q_flat, q, k, v, scale, True)
            fused_graphs.append(g)
        # the captures ran the host side of 4 steps, the device none: the
        # host mirrors are 4 steps ahead until 4 replays have run

        def replay(graphs, n):
            for i in range(n):
                graphs[i % 2].replay()

        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            replay(step_graphs, 2 + warm_even)
            stream.synchronize()
            done = 2 + warm_even
            t0 = time.perf_counter()
            replay(step_graphs, steps_even)
            stream.synchronize()
            step_s = (time.perf_counter() - t0) / steps_even
            bytes_timed = steps_bytes([r + done * N for r in rows_dev], steps_even)
            done += steps_even
            # the fused launches: HIP events on the replay stream
            replay(fused_graphs, 2)
            done += 2
            rows_fused = [r + done * N for r in rows_dev]
            e0.record(stream)
            replay(fused_graphs, 2 * args.attn_reps)
            e1.record(stream)
            e1.synchronize()
            done += 2 * args.attn_reps
        fused_us = e0.elapsed_time(e1) * 1e3 / (2 * args.attn_reps * L)
        cache.advance_replayed_steps(done - 4)
        assert _lib.device_error() == 0, "device error during the graph replays"
        assert list(cache._rows) == [r + done * N for r in rows_dev]
        value = bytes_timed / (step_s * steps_even) / 1e12
        # average over the timed launches: rows grow by N per launch
        fused_bytes = float(np.mean([launch_bytes(r + i * N) for r in rows_fused
                                     for i in range(2 * args.attn_reps)]))
        achieved = fused_bytes / (fused_us * 1e-6) / 1e9
        # attention alone (no append) on the final state
        rows_attn = list(cache._rows)
        outs = [torch.empty(N, G, D, dtype=torch.bfloat16, device=dev) for _ in range(L)]

        def attn_launches():
            for l, (q, _, _) in enumerate(inputs):
                q_flat = q.squeeze(2).reshape(N, G, D)
                fused_attn.decode_attn(q_flat, cache.layer_k[l], cache.layer_v[l], cache.cu_seqlens_k[l], scale,
                                       seg_base=cache.seg_base[l], total_rows=cache._rows[l], out=outs[l])

        with torch.cuda.stream(stream):
            ga = torch.cuda.CUDAGraph()
            with torch.cuda.graph(ga, stream=stream):
                attn_launches()
            ga.replay()
            e0.record(stream)
            for _ in range(args.attn_reps):
                ga.replay()
            e1.record(stream)
            e1.synchronize()
        attn_us = e0.elapsed_time(e1) * 1e3 / (args.attn_reps * L)
        assert _lib.device_error() == 0, "device error during attention timing"
        attn_bytes = float(np.mean([r * D * 2 * 2 + 2 * N * G * D * 2 for r in rows_attn]))
        attn_gbs = attn_bytes / (attn_us * 1e-6) / 1e9

    compact = None if args.no_compaction else compaction_timing(cfg, cache, inputs, dev)
    compact_slack = None if args.no_compaction else slack_compaction_timing(cfg, cache, dev)
    append_t = None if args.no_compaction else append_timing(cfg, cache, inputs, dev)
    cpu = None if args.no_cpu else cpu_baseline(cfg, cache, inputs, scale, args.cpu_sample_layers)
    line = {
        "metric": METRIC, "value": round(value, 4), "unit": "TB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round((step_s if step_s is not None else eager_s) * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": cfg.name, "layers": L, "batch": cfg.batch, "hq": cfg.hq, "hkv": cfg.hkv,
                   "head_dim": D, "n_seg": N, "rows_per_layer_step": int(np.mean(rows_attn)),
                   "path": "WnWCache (slack layout) + session.decode_attention: fused append + attention",
                   "graph": graph, "score": args.score, "notes": cfg.notes},
        "ms_per_step_eager": round(eager_s * 1e3, 4),
        "us_per_layer_step": None if fused_us is None else round(fused_us, 3),
        "attn_only_us_per_layer_step": None if attn_us is None else round(attn_us, 3),
        "attn_only_TBs": None if attn_gbs is None else round(attn_gbs / 1e3, 4),
        "compaction": compact,
        "compaction_slack": compact_slack,
        "append": append_t,
        "roofline": None if achieved is None else {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "attn_stream_kernel, fused append + attention", "bytes_per_launch": int(fused_bytes)},
        "cpu_baseline": cpu,
    }
    if extras is not None:
        line["extras"] = extras
    rl = line["roofline"]
    ratio = traffic_ratio_from_profiles(cfg.name)
    if rl is not None and ratio is not None:
        # the profile's measured HBM bytes per launch over its algorithmic
        # bytes, applied to this run's launches (rows grow with the steps run,
        # so the profiled launches and these differ in size, not in ratio)
        rl["traffic"] = int(round(ratio * fused_bytes))
        rl["traffic_ratio"] = round(ratio, 4)
        rl["traffic_source"] = (f"profile-derived: rocprofv3 FETCH_SIZE + WRITE_SIZE per launch, copy-calibrated, "
                                f"over algorithmic bytes (profiles/decode_attn_{cfg.name}_traffic.json) x this "
                                f"run's bytes_per_launch")
        # the counter-based rate beside the algorithmic one
        rl["traffic_GBs"] = round(rl["traffic"] / (fused_us * 1e-6) / 1e9, 1)
    print(json.dumps(line), flush=True)


# child runs of the default cfg2 bench: (key, arguments, environment, fields kept)
EXTRA_LEGS = [
    ("score_deferred", ["--score", "--no-cpu", "--no-compaction"], {},
     ["us_per_layer_step", "ms_per_step", "attn_only_us_per_layer_step"]),
    ("score_separate_pass", ["--score", "--no-cpu", "--no-compaction"], {"WNW_DEFER_SCORES": "0"},
     ["us_per_layer_step", "ms_per_step", "attn_only_us_per_layer_step"]),
    ("offload_cfg4", ["--config", "cfg4"], {},
     ["value", "unit", "steps", "ms_per_step_staged_path", "ms_per_step_device_path", "ms_per_step_no_offload",
      "h2d_MB_per_step", "h2d_copy_ms_per_step"]),
]


def extra_legs(timeout_s: int = 600) -> dict:
    """The extra figures of the default run, each from a child run of this
    script (one after another, before this process touches the GPU): cfg2
    with the class-A heads scored every step (deferred scoring, then the
    separate scoring pass) and the cfg4 offload step.  A leg that fails is
    reported as such; the headline measurement does not depend on it."""
    out = {}
    for key, argv, env, keep in EXTRA_LEGS:
        cmd = [sys.executable, "-u", os.path.abspath(__file__), "--no-extras", *argv]
        print(f"# extra leg {key}: {' '.join(argv)} {env or ''}", flush=True)
        try:
            r = subprocess.run(cmd, env={**os.environ, **env}, capture_output=True, text=True, timeout=timeout_s)
        except subprocess.TimeoutExpired:
            out[key] = {"error": f"timed out after {timeout_s} s"}
            continue
        lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
        if r.returncode != 0 or not lines:
            out[key] = {"error": f"exit {r.returncode}: {(r.stderr or r.stdout).strip()[-300:]}"}
            continue
        d = json.loads(lines[-1])
        out[key] = {"args": " ".join(argv), **({"env": env} if env else {}), **{k: d.get(k) for k in keep}}
    return out


def compaction_timing(cfg, cache, inputs, dev, reps: int = 5) -> dict:
    """One ``rebuild_append_kv`` per layer on the reference's dense layout
    (the cache's rows gathered densely): every class-B segment drops row 4
    (sink + window: the oldest window row, one relative evict range [4, 5)),
    every segment gets the step's new row, nothing is loaded.  Bytes = rows
    moved: the kept and new rows read, every output row written, K and V."""
    import numpy as np
    import torch

    from wnw_amd.wnw.kernels import rebuild_append_kv

    D, N = cfg.head_dim, cfg.n_seg
    i32 = dict(dtype=torch.int32, device=dev)
    calls, moved = [], 0
    for li in range(cfg.layers):
        dk, dv = cache.dense_kv(li)
        lens = np.asarray(cache.seq_lens[li], np.int64)
        class_b = ~np.tile(cfg.class_a[li].astype(bool), cfg.batch)
        n_ev = (class_b & (lens > 4)).astype(np.int64)
        old_cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        new_lens = lens - n_ev + 1
        new_cu = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.int32)
        ev_off = np.concatenate([[0], np.cumsum(n_ev)]).astype(np.int32)
        n_b = int(n_ev.sum())
        nk = inputs[li][1].reshape(N, D)
        nv = inputs[li][2].reshape(N, D)
        args = (dk, dv, nk, nv, dk[:0], dv[:0], torch.from_numpy(old_cu).to(dev), torch.from_numpy(new_cu).to(dev),
                torch.full((N,), -1, **i32), torch.zeros(N, **i32), torch.from_numpy(ev_off).to(dev),
                torch.full((n_b,), 4, **i32), torch.full((n_b,), 5, **i32), 1)
        calls.append((args, int(new_cu[-1])))
        moved += int(new_cu[-1]) * D * 2 * 2 * 2
    torch.cuda.synchronize()

    def launches():
        for args, tot in calls:
            rebuild_append_kv(*args, total_out=tot)

    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        launches()  # allocates the outputs before capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            launches()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        graph.replay()
        e0.record(stream)
        for _ in range(reps):
            graph.replay()
        e1.record(stream)
        e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * cfg.layers)
    bytes_per_launch = moved / cfg.layers
    return {"kernel": "rebuild_append_kernel", "us_per_layer_step": round(us, 3),
            "bytes_per_launch": int(bytes_per_launch),
            "TBs": round(bytes_per_launch / (us * 1e-6) / 1e12, 3),
            "frac_of_peak": round(bytes_per_launch / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "workload": "dense layout, class-B segments drop row 4 (evict [4, 5)), one new row per segment"}


def slack_move_call(cfg, cache, li: int, dev) -> tuple[dict, dict]:
    """The slack layout's compaction of layer ``li`` as a plan runs it
    (``wnw_compact_segments``, the cache's move of its class-B segments into
    the free half of the flip region): every class-B segment drops row 4
    (sink + window: the oldest window row, relative evict range [4, 5)),
    nothing is loaded, and the segments are packed with their slack into a
    free region (here a region of its own, sized like that half); class-A
    segments do not move.  Returns the keyword arguments of
    ``kernels.compact_segments`` and the move's host-side description
    (listed segments, their new lengths and destination bases, rows moved)."""
    import numpy as np
    import torch

    from wnw_amd.wnw.cache import _round8

    D, N = cfg.head_dim, cfg.n_seg
    i32 = dict(dtype=torch.int32, device=dev)
    lens = np.asarray(cache.seq_lens[li], np.int64)
    class_b = ~np.tile(cfg.class_a[li].astype(bool), cfg.batch)
    segs = np.nonzero(class_b)[0].astype(np.int32)
    n_ev = (class_b & (lens > 4)).astype(np.int64)
    new_len = lens - n_ev
    caps = np.array([_round8(int(new_len[f]) + cache.slack_rows) for f in segs], np.int64)
    dst_base = np.zeros(N, np.int64)
    dst_base[segs] = np.concatenate([[0], np.cumsum(caps)[:-1]]).astype(np.int64)
    region = int(caps.sum())
    k, v = cache.layer_k[li], cache.layer_v[li]
    ev_off = np.concatenate([[0], np.cumsum(n_ev)]).astype(np.int32)
    n_b = int(n_ev.sum())
    kwargs = dict(src_k=k, src_v=v, dst_k=torch.empty(region, D, dtype=k.dtype, device=dev),
                  dst_v=torch.empty(region, D, dtype=v.dtype, device=dev),
                  seg_list=torch.from_numpy(segs).to(dev), src_base=cache.seg_base[li],
                  src_len=torch.from_numpy(lens.astype(np.int32)).to(dev),
                  dst_base=torch.from_numpy(dst_base).to(dev),
                  new_len=torch.from_numpy(new_len.astype(np.int32)).to(dev), load_k=k[:0], load_v=v[:0],
                  load_starts=torch.full((N,), -1, **i32), load_lens=torch.zeros(N, **i32),
                  evict_offsets=torch.from_numpy(ev_off).to(dev), evict_starts=torch.full((n_b,), 4, **i32),
                  evict_ends=torch.full((n_b,), 5, **i32), max_new_len=int(new_len[segs].max()) if len(segs) else 0)
    moved = int(new_len[segs].sum())
    return kwargs, {"segs": segs, "new_len": new_len, "dst_base": dst_base, "rows_moved": moved}


def slack_compaction_timing(cfg, cache, dev, reps: int = 5) -> dict:
    """The product layout's compaction (``slack_move_call``), one
    ``compact_segments`` launch per layer, graph-replayed.  Bytes = the
    class-B rows kept, read and written, K and V (class-A rows stay put)."""
    import torch

    from wnw_amd.wnw.kernels import compact_segments

    D = cfg.head_dim
    calls = [slack_move_call(cfg, cache, li, dev) for li in range(cfg.layers)]
    moved = sum(info["rows_moved"] for _, info in calls) * D * 2 * 2 * 2
    torch.cuda.synchronize()

    def launches():
        for kw, _ in calls:
            compact_segments(**kw, check=False)

    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        launches()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            launches()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        graph.replay()
        e0.record(stream)
        for _ in range(reps):
            graph.replay()
        e1.record(stream)
        e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * cfg.layers)
    bytes_per_launch = moved / cfg.layers
    return {"kernel": "compact_segments_kernel", "us_per_layer_step": round(us, 3),
            "bytes_per_launch": int(bytes_per_launch),
            "TBs": round(bytes_per_launch / (us * 1e-6) / 1e12, 3),
            "frac_of_peak": round(bytes_per_launch / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "workload": "slack layout (the cache's plan path): every class-B segment moved into a free region "
                        "with sink + window eviction (drop row 4), no loads; class-A segments stay"}


def append_timing(cfg, cache, inputs, dev, reps: int = 5) -> dict:
    """The out-of-place append of the dense layout (the reference's
    ``interleave_append`` of K and V, here one launch for both tensors,
    ``interleave_append_kv``, as the cache's dense path calls it): every row
    read and written once more, plus the step's new rows.  Bytes = (T + N
    rows read + T + N rows written) x 2 tensors.  (The cache's default slack
    layout fuses its append into the attention launch instead.)"""
    import numpy as np
    import torch

    from wnw_amd.kv.kernels import interleave_append_kv

    D, N = cfg.head_dim, cfg.n_seg
    calls, moved = [], 0
    for li in range(cfg.layers):
        dk, dv = cache.dense_kv(li)
        lens = np.asarray(cache.seq_lens[li], np.int64)
        cu_old = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        cu_new = cu_old + np.arange(N + 1, dtype=np.int32)
        nk = inputs[li][1].reshape(N, D)
        nv = inputs[li][2].reshape(N, D)
        calls.append((dk, dv, nk, nv, torch.from_numpy(cu_old).to(dev), torch.from_numpy(cu_new).to(dev)))
        T = int(cu_old[-1])
        moved += (T + N) * D * 2 * 2 * 2  # read and written, K and V
    torch.cuda.synchronize()

    def launches():
        for dk, dv, nk, nv, co, cn in calls:
            interleave_append_kv(dk, dv, nk, nv, co, cn)

    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        launches()  # allocates the outputs before capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            launches()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        graph.replay()
        e0.record(stream)
        for _ in range(reps):
            graph.replay()
        e1.record(stream)
        e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * cfg.layers)
    bytes_per_layer = moved / cfg.layers
    return {"kernel": "interleave_append_kernel<true> (K and V, one launch)", "us_per_layer_step": round(us, 3),
            "bytes_per_layer_step": int(bytes_per_layer),
            "TBs": round(bytes_per_layer / (us * 1e-6) / 1e12, 3),
            "frac_of_peak": round(bytes_per_layer / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "workload": "dense layout, one new row per segment, out of place (the reference operator's semantics)"}


def traffic_ratio_from_profiles(workload: str):
    """Measured HBM bytes per launch of the dominant kernel (the committed
    rocprofv3 PMC summary: FETCH_SIZE + WRITE_SIZE, copy-calibrated) over
    the algorithmic bytes of the profiled launches, if present."""
    path = os.path.join(ROOT, "profiles", f"decode_attn_{workload}_traffic.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            d = json.load(f)
        return d["traffic_bytes_per_launch"] / d["algorithmic_bytes_per_launch"]
    except (OSError, ValueError, KeyError, ZeroDivisionError):
        return None


def cpu_threads() -> int:
    """Host threads for the CPU baseline: os.cpu_count(), capped by the
    process's CPU affinity and by OMP_NUM_THREADS when that is set (the GPU
    box gives one GPU's job a share of its cores)."""
    n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except (AttributeError, OSError):
        pass
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_baseline(cfg, cache, inputs, scale, sample_layers: int, budget_s: float = 15.0):
    """The reference's decode layer-step in PyTorch on the host's cores
    (``oracle/torch_cpu.py``): the append of the step's row to every segment
    (``torch.cat``, out of place) and per-segment float32 attention, on a
    bounded sample of the workload's layers (the cache's rows in the dense
    layout, copied to the host before timing)."""
    import torch

    from oracle import torch_cpu

    threads = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    D, G, N = cfg.head_dim, cfg.group, cfg.n_seg
    elapsed, done, bytes_done = 0.0, 0, 0
    limit = sample_layers if sample_layers > 0 else cfg.layers
    try:
        for li in range(limit):
            dk, dv = cache.dense_kv(li)
            k, v = dk.cpu(), dv.cpu()
            cu_old = cache.cu_list(li)
            q, nk, nv = (t.cpu() for t in inputs[li])
            q = q.reshape(N, G, D)
            nk, nv = nk.reshape(N, D), nv.reshape(N, D)
            cu_new = [c + i for i, c in enumerate(cu_old)]
            t0 = time.perf_counter()
            k2 = torch_cpu.append_by_cat(k, nk, cu_old)
            v2 = torch_cpu.append_by_cat(v, nv, cu_old)
            torch_cpu.decode_attn(q, k2, v2, cu_new, scale)
            elapsed += time.perf_counter() - t0
            done += 1
            bytes_done += cu_new[-1] * D * 2 * 2 + 2 * N * G * D * 2
            if sample_layers <= 0 and elapsed > budget_s:
                break
    finally:
        torch.set_num_threads(prev)
    us = elapsed / done * 1e6
    return {"value": round(bytes_done / elapsed / 1e9, 4), "unit": "GB/s", "us_per_layer_step": round(us, 1),
            "cores": threads, "os_cpu_count": os.cpu_count(), "kind": "port",
            "sample": f"{done} of {cfg.layers} layers of one decode step ({cfg.name}): torch.cat append + "
                      f"per-segment float32 softmax attention (PyTorch, {threads} threads)"}


if __name__ == "__main__":
    main()

#!/usr/bin/env python3
"""Decode-step attention benchmark on one MI355X (BASELINE.json metric).

Workload (default ``--config cfg2``): Voxtral-Mini-3B decode shape, 30 layers,
32 query / 8 KV heads, head_dim 128, bf16, batch 8, 7,500 audio + 64 text
tokens per sequence; per layer 2 of 8 KV heads are class A (full KV), the
others class B (512 rows).  Synthetic data: K, V ~ N(0, 1) times a
per-(layer, KV head) scale from U(0.5, 2), q ~ N(0, 1).

One step = for each of the 30 layers: in-place append of the step's K/V row
to every segment (slack layout) + split-K decode attention.  All 30 layers
have distinct buffers (~2.2 GB), far beyond the 256 MB Infinity Cache.  Each
step is captured once as a HIP graph (two graphs: even/odd step, for the
ping-ponged offsets) so the timed region measures the GPU, not Python.

Reported:
* value          -- whole-step throughput: algorithmic bytes (attention K/V
                    rows + q/o + appended rows) of the K timed steps / wall time.
* us_per_layer_step -- decode-attention kernel time per layer-step, from HIP
                    events around back-to-back attention-only graph replays.
* roofline       -- the attention kernel: algorithmic bytes per launch /
                    average launch time vs 8 TB/s.
* append_us_per_layer_step -- the in-place append kernel alone, per layer-step.
* compaction     -- the rebuild (compaction + append) kernel on the dense
                    layout, per layer: class-B segments drop their oldest
                    window row, every segment gets a new row; µs per layer
                    and TB/s of rows moved.
* cpu_baseline   -- the reference's decode layer-step restated in PyTorch
                    (torch.cat append + per-segment float32 attention) on the
                    host's cores, on a bounded sample of the same layers.

``--copy-calibration`` only runs a plain 256 MiB device-to-device copy three
times (for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes).
"""
from __future__ import annotations

import argparse
import json
import os
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
    ap.add_argument("--kernel", default="auto", choices=["auto", "stream", "mfma", "valu"])
    ap.add_argument("--attn-reps", type=int, default=20, help="attention-only graph replays for the roofline")
    ap.add_argument("--cpu-sample-layers", type=int, default=0,
                    help="layers timed for the CPU baseline (0 = choose ~15 s of work)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying HIP graphs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy three times (PMC byte calibration)")
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


class LayerState:
    """Slack layout of one layer: each segment owns len + slack rows."""

    def __init__(self, cfg, layer: int, slack: int, device, gen):
        import numpy as np
        import torch

        self.n = cfg.n_seg
        d = cfg.head_dim
        lens = cfg.lengths[layer].astype(np.int64)
        cap = lens + slack
        cap = (cap + 7) // 8 * 8
        base = np.zeros(self.n, np.int64)
        base[1:] = np.cumsum(cap)[:-1]
        self.pool_rows = int(cap.sum())
        self.lens0 = lens
        self.rows_est = int(lens.sum())  # sizes the grid; the kernel reads the exact rows from cu
        self.base = torch.from_numpy(base).to(device)
        self.cap = torch.from_numpy(cap.astype(np.int32)).to(device)
        cu = np.zeros(self.n + 1, np.int32)
        cu[1:] = np.cumsum(lens)
        self.cu = [torch.from_numpy(cu).to(device), torch.zeros(self.n + 1, dtype=torch.int32, device=device)]
        self.cu_init = torch.from_numpy(cu).to(device)
        scale_seg = np.tile(cfg.kv_scale[layer], cfg.batch).astype(np.float32)  # segment s = b * Hkv + h
        row_scale = torch.from_numpy(np.repeat(scale_seg, cap)).to(device).unsqueeze(1)
        self.k = (torch.randn(self.pool_rows, d, device=device, generator=gen) * row_scale).to(torch.bfloat16)
        self.v = (torch.randn(self.pool_rows, d, device=device, generator=gen) * row_scale).to(torch.bfloat16)
        self.q = torch.randn(self.n, cfg.group, d, device=device, generator=gen).to(torch.bfloat16)
        self.new_k = torch.randn(self.n, d, device=device, generator=gen).to(torch.bfloat16)
        self.new_v = torch.randn(self.n, d, device=device, generator=gen).to(torch.bfloat16)
        self.out = torch.empty(self.n, cfg.group, d, dtype=torch.bfloat16, device=device)

    def reset(self):
        self.cu[0].copy_(self.cu_init)

    def dense_host(self):
        """The logical rows of every segment under cu[0], gathered into the
        reference's dense layout on the host: (k, v, cu)."""
        import torch

        cu = self.cu[0].cpu()
        lens = (cu[1:] - cu[:-1]).to(torch.int64)
        idx = torch.cat([self.base[s].cpu() + torch.arange(int(lens[s])) for s in range(self.n)])
        return self.k.cpu()[idx], self.v.cpu()[idx], cu


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the decode path is single-GPU "
              "per process and multi-GPU runs are not part of this build", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.config == "cfg4":
        from wnw_amd import offload_bench

        print(json.dumps({**offload_bench.run(args.steps, args.warmup), "n_gpus": 1}), flush=True)
        return

    import numpy as np
    import torch

    from wnw_amd import _lib, workloads
    from wnw_amd.kv import fused_attn
    from wnw_amd.kv.kernels import append_inplace

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _lib.lib()
    _lib.ensure_init(dev)
    cfg = workloads.CONFIGS[args.config]()
    L, N, G, D = cfg.layers, cfg.n_seg, cfg.group, cfg.head_dim
    total_steps = args.warmup + args.steps
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    print(f"# config {cfg.name}: layers={L} n_seg={N} G={G} D={D} steps={args.steps} warmup={args.warmup}",
          flush=True)
    # slack: one row per step, plus the four appends of the append-only timing
    layers = [LayerState(cfg, l, total_steps + 6, dev, gen) for l in range(L)]
    torch.cuda.synchronize()
    ws = fused_attn.AttnWorkspace(dev)
    ws.get(N, G, D)
    scale = D ** -0.5

    def step_launches(parity: int):
        for st in layers:
            cu_old, cu_new = st.cu[parity], st.cu[1 - parity]
            append_inplace(st.k, st.v, st.new_k, st.new_v, cu_old, cu_new, st.base, st.cap)
            fused_attn.decode_attn(st.q, st.k, st.v, cu_new, scale, seg_base=st.base, total_rows=st.rows_est,
                                   out=st.out, workspace=ws, kernel=args.kernel)

    def append_launches(parity: int):
        for st in layers:
            append_inplace(st.k, st.v, st.new_k, st.new_v, st.cu[parity], st.cu[1 - parity], st.base, st.cap)

    def attn_launches():
        for st in layers:
            fused_attn.decode_attn(st.q, st.k, st.v, st.cu[0], scale, seg_base=st.base, total_rows=st.rows_est,
                                   out=st.out, workspace=ws, kernel=args.kernel)

    stream = torch.cuda.Stream(device=dev)
    graphs = None
    attn_graph = None
    append_graphs = None
    if not args.no_graph:
        # capture on a side stream (default priority), then replay
        with torch.cuda.stream(stream):
            ws.get(N, G, D)
        torch.cuda.synchronize()
        graphs = []
        for parity in (0, 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                step_launches(parity)
            graphs.append(g)
        attn_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(attn_graph, stream=stream):
            attn_launches()
        append_graphs = []
        for parity in (0, 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                append_launches(parity)
            append_graphs.append(g)
        torch.cuda.synchronize()
        for st in layers:  # capture does not execute; start from the initial offsets
            st.reset()
        torch.cuda.synchronize()

    def run_step(t: int):
        if graphs is not None:
            graphs[t % 2].replay()
        else:
            step_launches(t % 2)

    # ---- warmup + timed decode steps --------------------------------------
    ctx = torch.cuda.stream(stream) if graphs is not None else torch.cuda.stream(torch.cuda.current_stream())
    with ctx:
        for t in range(args.warmup):
            run_step(t)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for t in range(args.warmup, total_steps):
            run_step(t)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    assert _lib.device_error() == 0, "device error during the timed steps"
    step_s = (t1 - t0) / args.steps

    # bytes of the timed steps: rows attended at step t are lens0 + t + 1 per segment
    attn_bytes_total = 0
    append_bytes_total = 0
    for t in range(args.warmup, total_steps):
        for st in layers:
            rows = int(st.lens0.sum()) + N * (t + 1)
            attn_bytes_total += rows * D * 2 * 2 + 2 * N * G * D * 2
            append_bytes_total += 2 * N * D * 2 * 2  # read new row + write it, K and V
    value_tbs = (attn_bytes_total + append_bytes_total) / (t1 - t0) / 1e12

    # ---- attention-only kernel timing (state after the timed steps) -------
    # cu[0] now holds the offsets after an even number of steps, or cu[1]:
    final_parity = total_steps % 2
    for st in layers:
        if final_parity == 1:
            st.cu[0].copy_(st.cu[1])
    torch.cuda.synchronize()
    rows_attn = [int(st.cu[0][-1].item()) for st in layers]
    bytes_per_launch = [r * D * 2 * 2 + 2 * N * G * D * 2 for r in rows_attn]
    with torch.cuda.stream(stream):
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        if attn_graph is not None:
            attn_graph.replay()
        else:
            attn_launches()
        ev0.record(stream)
        for _ in range(args.attn_reps):
            if attn_graph is not None:
                attn_graph.replay()
            else:
                attn_launches()
        ev1.record(stream)
        ev1.synchronize()
    attn_ms = ev0.elapsed_time(ev1)
    launches = args.attn_reps * L
    us_per_launch = attn_ms * 1e3 / launches
    avg_bytes = float(np.mean(bytes_per_launch))
    achieved_gbs = avg_bytes / (us_per_launch * 1e-6) / 1e9
    assert _lib.device_error() == 0, "device error during attention timing"

    # ---- append-only kernel timing: two appends (there and back) per rep --
    # The slack leaves room for them: rows stay within each segment's capacity.
    app_reps = 2
    with torch.cuda.stream(stream):
        ev2 = torch.cuda.Event(enable_timing=True)
        ev3 = torch.cuda.Event(enable_timing=True)
        ev2.record(stream)
        for r in range(app_reps):
            for parity in (0, 1):
                if append_graphs is not None:
                    append_graphs[parity].replay()
                else:
                    append_launches(parity)
        ev3.record(stream)
        ev3.synchronize()
    append_us = ev2.elapsed_time(ev3) * 1e3 / (2 * app_reps * L)
    assert _lib.device_error() == 0, "device error during append timing"

    # ---- compaction timing: one rebuild (a4) per layer ---------------------
    compact = compaction_timing(cfg, layers, dev, stream, graphs is not None)
    assert _lib.device_error() == 0, "device error during compaction timing"

    # ---- CPU baseline: float64 C oracle on a bounded sample ---------------
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cfg, layers, scale, args.cpu_sample_layers)

    line = {
        "metric": METRIC,
        "value": round(value_tbs, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": cfg.name, "layers": L, "batch": cfg.batch, "hq": cfg.hq, "hkv": cfg.hkv,
                   "head_dim": D, "n_seg": N, "rows_per_layer_step": int(np.mean(rows_attn)),
                   "kernel": args.kernel, "graph": graphs is not None, "notes": cfg.notes},
        "us_per_layer_step": round(us_per_launch, 3),
        "append_us_per_layer_step": round(append_us, 3),
        "compaction": compact,
        "attn_TBs": round(achieved_gbs / 1e3, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved_gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(cfg.name)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def compaction_timing(cfg, layers, dev, stream, use_graph: bool, reps: int = 5) -> dict:
    """One ``rebuild_append_kv`` per layer on the dense layout (the reference's
    layout): every class-B segment drops row 4 (sink + window: the oldest
    window row, one relative evict range [4, 5)), every segment gets the
    step's new row, nothing is loaded.  Bytes = rows moved: the kept and new
    rows read, every output row written, K and V."""
    import numpy as np
    import torch

    from wnw_amd.wnw.kernels import rebuild_append_kv

    D = cfg.head_dim
    i32 = dict(dtype=torch.int32, device=dev)
    calls, moved = [], 0
    for li, st in enumerate(layers):
        lens = st.lens0.astype(np.int64)
        base = st.base.cpu().numpy()
        idx = torch.from_numpy(np.concatenate([b + np.arange(n) for b, n in zip(base, lens)])).to(dev)
        dk, dv = st.k.index_select(0, idx), st.v.index_select(0, idx)
        class_b = ~np.tile(cfg.class_a[li].astype(bool), cfg.batch)
        n_ev = class_b.astype(np.int64)
        old_cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        new_lens = lens - n_ev + 1
        new_cu = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.int32)
        ev_off = np.concatenate([[0], np.cumsum(n_ev)]).astype(np.int32)
        n_b = int(n_ev.sum())
        args = (dk, dv, st.new_k, st.new_v, dk[:0], dv[:0], torch.from_numpy(old_cu).to(dev),
                torch.from_numpy(new_cu).to(dev), torch.full((st.n,), -1, **i32), torch.zeros(st.n, **i32),
                torch.from_numpy(ev_off).to(dev), torch.full((n_b,), 4, **i32), torch.full((n_b,), 5, **i32), 1)
        calls.append((args, int(new_cu[-1])))
        moved += int(new_cu[-1]) * D * 2 * 2 * 2
    torch.cuda.synchronize()

    def launches():
        for args, tot in calls:
            rebuild_append_kv(*args, total_out=tot)

    with torch.cuda.stream(stream):
        launches()  # allocates the outputs before capture
        graph = None
        if use_graph:
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                launches()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        (graph.replay if graph is not None else launches)()
        e0.record(stream)
        for _ in range(reps):
            (graph.replay if graph is not None else launches)()
        e1.record(stream)
        e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * len(layers))
    bytes_per_launch = moved / len(layers)
    return {"kernel": "rebuild_append_kernel", "us_per_layer_step": round(us, 3),
            "bytes_per_launch": int(bytes_per_launch),
            "TBs": round(bytes_per_launch / (us * 1e-6) / 1e12, 3),
            "frac_of_peak": round(bytes_per_launch / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "workload": "dense layout, class-B segments drop row 4 (evict [4, 5)), one new row per segment"}


def traffic_from_profiles(workload: str):
    """HBM bytes per attention launch from the committed rocprofv3 PMC summary, if present."""
    path = os.path.join(ROOT, "profiles", f"decode_attn_{workload}_traffic.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
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


def cpu_baseline(cfg, layers, scale, sample_layers: int, budget_s: float = 15.0):
    """The reference's decode layer-step in PyTorch on the host's cores
    (``oracle/torch_cpu.py``): the append of the step's row to every segment
    (``torch.cat``, out of place) and per-segment float32 attention, on a
    bounded sample of the workload's layers (the dense logical rows of each
    layer, copied to the host before timing)."""
    import numpy as np
    import torch

    from oracle import torch_cpu

    threads = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    D, G = cfg.head_dim, cfg.group
    elapsed, done, bytes_done = 0.0, 0, 0
    limit = sample_layers if sample_layers > 0 else len(layers)
    try:
        for li, st in enumerate(layers[:limit]):
            k, v, cu = st.dense_host()
            nk, nv, q = st.new_k.cpu(), st.new_v.cpu(), st.q.cpu()
            cu_old = cu.tolist()
            cu_new = [c + i for i, c in enumerate(cu_old)]
            t0 = time.perf_counter()
            k2 = torch_cpu.append_by_cat(k, nk, cu_old)
            v2 = torch_cpu.append_by_cat(v, nv, cu_old)
            torch_cpu.decode_attn(q, k2, v2, cu_new, scale)
            elapsed += time.perf_counter() - t0
            done += 1
            bytes_done += cu_new[-1] * D * 2 * 2 + 2 * cfg.n_seg * G * D * 2
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

"""Config 4 (long-audio offload) through the whole cache path, on one GPU.

Voxtral shape (30 layers, 32 / 8 heads, head_dim 128, bf16), batch 1,
22,500 audio tokens (+ 64 text tokens before and after).  Two KV heads per
layer are class A (full KV, scored); the other six are class B: they keep
5 rows of each 256-token segment plus the text, and the rest of the audio
lives in pinned host memory as 256-token chunks.  After every decode step
the planner picks the top-8 chunks from the class-A scores of that step and
the cache fetches the newly chosen ones on a side stream in groups of
layers, overlapped with the next step's compute: through the path
``WNW_OFFLOAD`` names ("copy", the default: DMA copies straight from the
pinned host rows into a device stage and a kernel that puts them in
transfer order; "staged": host gather threads into pinned staging, then DMA
copies; "device": a gather kernel reading pinned host memory); the other
paths are timed too.  As in the
reference (src/algorithms/wnw/code/cache.py:609-630) the choice is per
sample, shared by every class-B head and layer.

One decode step = for each layer: ``decode_attention`` (append or
rebuild-with-loads, attention with fused class-A scoring), then the
planning of ``decode_all_layers_done``.  Synthetic data: K, V, q ~ N(0, 1),
prefill scores U(0, 1), seed 0; the step inputs (q and the new K/V row of
every layer) are made before the timed region.

Reported: wall time per decode step (the host is part of the step: the
cache runs its Python and planner logic per layer) through the default path
and through the other one, host->device bytes per step (the cache's own
transfer events), the time a plain pinned copy of those bytes takes on the
copy engine, the step time of the same run without offload (top-k 0:
nothing is ever fetched) and the difference of the default and no-offload
step times (what offload adds per step: planning, fetch and rebuilds, net of
overlap).
"""
from __future__ import annotations

import time

L, HKV, HQ, D = 30, 8, 32, 128
B = 1
AUDIO = 22500
TEXT_BEFORE = TEXT_AFTER = 64
CHUNK = 256
KEEP_PER_SEG = 5
TOP_K = 8


def _config(top_k: int, seed: int = 0):
    import numpy as np

    from .wnw.config import WnWConfig

    rng = np.random.default_rng(seed)
    G = HQ // HKV
    class_a, class_b = [], []
    for layer in range(L):
        a = set(rng.choice(HKV, 2, replace=False).tolist())
        class_a += [layer * HQ + kv * G + g for kv in sorted(a) for g in range(G)]
        class_b += [layer * HKV + h for h in range(HKV) if h not in a]
    return WnWConfig(chunk_size_s=CHUNK, overlap_s=0, token_rate=1.0, class_a=class_a, class_b=class_b,
                     retention_ratios=[KEEP_PER_SEG / CHUNK] * (L * HKV), top_k_chunks=top_k, eviction_lag=2,
                     prefill_score_mode="last", num_layers=L, num_kv_heads=HKV, num_q_heads=HQ)


def _prefilled_cache(top_k: int, dev):
    import torch

    from .wnw.cache import WnWCache

    cfg = _config(top_k)
    cache = WnWCache(cfg, L, HKV, HQ, D, dev)
    cache.collect_stats(1 << 30)  # transfer events every step, no snapshots
    S = TEXT_BEFORE + AUDIO + TEXT_AFTER
    a0, a1 = TEXT_BEFORE, TEXT_BEFORE + AUDIO
    cache.setup_audio(torch.tensor([a0], device=dev), torch.tensor([a1], device=dev), None)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    for layer in range(L):
        k = torch.randn(B, HKV, S, D, device=dev, generator=gen).to(torch.bfloat16)
        v = torch.randn(B, HKV, S, D, device=dev, generator=gen).to(torch.bfloat16)
        ca = [torch.rand(AUDIO, device=dev, generator=gen) if cfg.get_layer_class_a(layer) else None]
        per = [[None if cfg.is_class_a_kv_head(layer, h) else torch.rand(AUDIO, device=dev, generator=gen)
                for h in range(HKV)]]
        cache.prefill_after_attn(layer, ca, per, k, v)
    cache.prefill_all_layers_done()
    torch.cuda.synchronize()
    return cache


def _inputs(steps: int, dev, seed: int):
    """q, k, v of every (step, layer), made before the timed region so that
    it holds the cache path only."""
    import torch

    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    out = []
    for _ in range(steps):
        row = []
        for _layer in range(L):
            q = torch.randn(B, HQ, 1, D, device=dev, generator=gen).to(torch.bfloat16)
            k = torch.randn(B, HKV, 1, D, device=dev, generator=gen).to(torch.bfloat16)
            v = torch.randn(B, HKV, 1, D, device=dev, generator=gen).to(torch.bfloat16)
            row.append((q, k, v))
        out.append(row)
    return out


def _run_steps(cache, inputs):
    from .wnw.session import decode_attention

    scale = D ** -0.5
    for row in inputs:
        for layer, (q, k, v) in enumerate(row):
            decode_attention(cache, layer, q, k, v, scale, fused=True)


def _timed(cache, steps: int, warmup: int, dev):
    import torch

    warm, timed = _inputs(warmup, dev, 1), _inputs(steps, dev, 2)
    _run_steps(cache, warm)
    torch.cuda.synchronize()
    n_events = len(cache.stats.get_all_stats()[0]["cpu_gpu_events"])
    t0 = time.perf_counter()
    _run_steps(cache, timed)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    events = cache.stats.get_all_stats()[0]["cpu_gpu_events"][n_events:]
    c2g = sum(e[3] for e in events)
    return dt / steps, c2g / steps, len(events)


def _copy_time(nbytes: int, dev) -> float:
    """Seconds to copy nbytes (K and V halves) from pinned host memory on a
    side stream, as the cache does."""
    import torch

    if nbytes <= 0:
        return 0.0
    rows = nbytes // (2 * D * 2)
    hk = torch.empty(rows, D, dtype=torch.bfloat16, pin_memory=True)
    hv = torch.empty(rows, D, dtype=torch.bfloat16, pin_memory=True)
    s = torch.cuda.Stream(device=dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        for _ in range(2):
            hk.to(dev, non_blocking=True)
        e0.record(s)
        for _ in range(5):
            hk.to(dev, non_blocking=True)
            hv.to(dev, non_blocking=True)
        e1.record(s)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / 5


def _offload_step(mode: str, steps: int, warmup: int, dev):
    """Step time with the host rows loaded through ``mode`` (WNW_OFFLOAD)."""
    import os

    import torch

    old = os.environ.get("WNW_OFFLOAD")
    os.environ["WNW_OFFLOAD"] = mode
    try:
        cache = _prefilled_cache(TOP_K, dev)
    finally:
        if old is None:
            del os.environ["WNW_OFFLOAD"]
        else:
            os.environ["WNW_OFFLOAD"] = old
    assert cache._offload == mode
    host_rows = int(cache.cpu_restore_k.shape[0])
    t_step, c2g_per_step, n_load_steps = _timed(cache, steps, warmup, dev)
    del cache
    torch.cuda.empty_cache()
    return t_step, c2g_per_step, n_load_steps, host_rows


def run(steps: int, warmup: int) -> dict:
    import os

    import torch

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    default = os.environ.get("WNW_OFFLOAD", "copy")
    others = [m for m in ("copy", "staged", "device") if m != default]
    t_step, c2g_per_step, n_load_steps, host_rows = _offload_step(default, steps, warmup, dev)
    t_others = {m: _offload_step(m, steps, warmup, dev)[0] for m in others}
    base = _prefilled_cache(0, dev)
    t_base, _, _ = _timed(base, steps, warmup, dev)
    del base
    t_copy = _copy_time(int(c2g_per_step), dev)
    exposed = max(0.0, t_step - t_base)
    return {
        "metric": "cfg4 decode step through the cache with host->device chunk fetches, 1 GPU",
        "value": round(t_step * 1e3, 3), "unit": "ms/step", "higher_is_better": False,
        "steps": steps, "warmup": warmup, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "cfg4-offload-22500tok-b1", "layers": L, "batch": B, "hq": HQ, "hkv": HKV,
                   "head_dim": D, "audio": AUDIO, "chunk": CHUNK, "top_k_chunks": TOP_K,
                   "class_b_keep_per_chunk": KEEP_PER_SEG, "host_rows": host_rows},
        "offload_path": default,
        **{f"ms_per_step_{m}_path": round(t * 1e3, 3) for m, t in t_others.items()},
        "ms_per_step_no_offload": round(t_base * 1e3, 3),
        "h2d_MB_per_step": round(c2g_per_step / 1e6, 2),
        "steps_with_loads": n_load_steps,
        "h2d_copy_ms_per_step": round(t_copy * 1e3, 3),
        "h2d_GBs": round(c2g_per_step / t_copy / 1e9, 1) if t_copy > 0 else None,
        "offload_ms_per_step": round(exposed * 1e3, 3),
    }

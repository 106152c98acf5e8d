"""End-to-end decode steps through WnWCache / WnWCppCache vs a CPU simulation.

The cache is prefilled through its own hooks (random K/V and tie-free
scores), then driven through ``decode_attention`` for several steps, and
every step is checked by ``tests.cache_sim.DecodeSimulation``: appends and
compactions (bit-exact K/V, offsets), attention (2e-3 + 1e-2 |ref|), class-A
scores (1e-6 + 1e-3 |ref|), the device's chunk top-k against the oracle's
``topk_chunks(chunk_means(...))`` and the planner's loaded segments; here
also the stats record.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import planner as op
from tests.cache_sim import DecodeSimulation, bits as _bits, recording as _recording
from tests.helpers import allclose_report
from wnw_amd import _lib
from wnw_amd.wnw.cache import WnWCache
from wnw_amd.wnw.config import WnWConfig
from wnw_amd.wnw.session import decode_attention
from wnw_amd.wnw_cpp.cache import WnWCppCache

pytestmark = pytest.mark.gpu

L, H, G, D, B = 2, 4, 4, 128, 2
HQ = H * G
S = 64
AUDIO = [(8, 48), (4, 52)]
STEPS = 8


def _config():
    return WnWConfig(chunk_size_s=8, overlap_s=4, token_rate=1.0,
                     class_a=[0, 1, 2, 3, HQ + 4, HQ + 5],        # layer 0: whole group of KV 0; layer 1: half of KV 1
                     class_b=[2, 3, H + 2, H + 3], retention_ratios=[0.5] * (L * H),
                     top_k_chunks=2, eviction_lag=2, prefill_score_mode="last",
                     num_layers=L, num_kv_heads=H, num_q_heads=HQ)


def _prefill(cache, dev, gen):
    starts = torch.tensor([a for a, _ in AUDIO], dtype=torch.int64, device=dev)
    ends = torch.tensor([e for _, e in AUDIO], dtype=torch.int64, device=dev)
    cache.setup_audio(starts, ends, None)
    for l in range(L):
        k = torch.randn(B, H, S, D, generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn(B, H, S, D, generator=gen, device=dev).to(torch.bfloat16)
        ca = [torch.rand(e - a, generator=gen, device=dev) if cache.config.get_layer_class_a(l) else None
              for a, e in AUDIO]
        per = [[None if cache.config.is_class_a_kv_head(l, h) else torch.rand(e - a, generator=gen, device=dev)
                for h in range(H)] for a, e in AUDIO]
        cache.prefill_after_attn(l, ca, per, k, v)
    cache.prefill_all_layers_done()


# layouts: the default slack layout (plans relocate changed segments into
# the pool's tail), 3 rows of slack and no tail (a relayout every few
# appends, and every plan rebuilds the whole layer), and the reference's
# dense layout
LAYOUTS = {"slack": dict(slack_rows=256), "tight": dict(slack_rows=3, tail=0), "dense": dict(slack_rows=0)}


@pytest.mark.parametrize("layout", ["slack", "tight", "dense"])
@pytest.mark.parametrize("variant,fused,offload", [("wnw", True, "copy"), ("wnw", False, "copy"),
                                                   ("wnw_fallback", True, "copy"), ("wnw_cpp", True, "copy"),
                                                   ("wnw", True, "staged"), ("wnw_cpp", True, "staged"),
                                                   ("wnw_nodefer", True, "copy"),
                                                   ("wnw", True, "device"), ("wnw_cpp", True, "device")])
def test_decode_steps_match_simulation(variant, fused, offload, layout, monkeypatch):
    dev = torch.device("cuda", 0)
    # loads through the transfer engine (DMA copies straight from the host
    # rows into a device stage, or host gather threads into pinned staging
    # + DMA copies) or the device gather kernel reading pinned memory
    monkeypatch.setenv("WNW_OFFLOAD", offload)
    # fused class-A scoring deferred to the next launch (default) or in a
    # scoring pass of its own per layer
    monkeypatch.setenv("WNW_DEFER_SCORES", "0" if variant == "wnw_nodefer" else "1")
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    cls = _recording(WnWCppCache if variant == "wnw_cpp" else WnWCache)
    lay = LAYOUTS[layout]
    cache = cls(_config(), L, H, HQ, D, dev, slack_rows=lay["slack_rows"])
    if "tail" in lay:
        cache.tail_rows_min = cache.tail_factor = lay["tail"]
    cache.rec_acc, cache.rec_topk = [], []
    if variant == "wnw_fallback":
        cache.use_triton_rebuild = False
    cache.collect_stats(1)  # a snapshot every decode step
    print(f"cache variant={variant} fused={fused} offload={offload} layout={layout}", flush=True)
    _prefill(cache, dev, gen)
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    assert cache._offload == offload

    sim = DecodeSimulation(cache, AUDIO)  # no left padding: audio relative to the segments' starts
    scale = D ** -0.5
    for t in range(STEPS):
        qs = [torch.randn(B, HQ, 1, D, generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
        ks = [torch.randn(B, H, 1, D, generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
        vs = [torch.randn(B, H, 1, D, generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
        outs = [decode_attention(cache, l, qs[l], ks[l], vs[l], scale, fused=fused) for l in range(L)]
        torch.cuda.synchronize()
        assert _lib.device_error() == 0, f"step {t}"
        sim.step(t, qs, ks, vs, outs)
    lens, meta, host_k = sim.lens, sim.meta, sim.host_k
    loaded_at_snapshot, want_events, loaded_after_prefill = sim.loaded_at_snapshot, sim.want_events, \
        sim.loaded_after_prefill
    # the stats record (reference cache.py:1013-1081 and inference_stats.py):
    # the last snapshot is taken before the last step's plan
    stats = cache.get_all_stats()
    row = D * 2 * 2  # K and V, bf16
    host = [{(l, h, si): m.cpu_end - m.cpu_start for l in range(L) for h in cache.config.get_layer_class_b(l)
             for si, m in enumerate(meta[l][b][h]) if m is not None} for b in range(B)]
    for b in range(B):
        fin = stats[b]["decode_final"]
        assert len(stats[b]["decode_snapshots"]) == STEPS and fin["step"] == STEPS
        assert fin["gpu_total_tokens"] == sum(lens[l][b * H + h] for l in range(L) for h in range(H))
        assert fin["cpu_total_tokens"] == sum(sum(x.values()) for x in host) == host_k.shape[0]
        assert fin["cpu_restore_tokens"] == sum(host[b].values())
        assert fin["cpu_loaded_tokens"] == sum(n for (l, h, si), n in host[b].items() if si in loaded_at_snapshot[b])
        assert fin["memory_used_bytes"] > 0
        events = stats[b]["cpu_gpu_events"]
        offloaded = sum(host[b].values())
        first_loads = sum(n for (l, h, si), n in host[b].items() if si in loaded_after_prefill[b])
        assert events[0] == (-1, first_loads, offloaded, first_loads * row, offloaded * row), "prefill event"
        got = [(e[0], e[1]) for e in events[1:]]
        if variant == "wnw_cpp":
            assert got == [], "the deferred-plan variant counts no decode loads (as the reference's)"
        else:
            assert got == want_events[b]
            assert all(e[3] == e[1] * row and e[2] == 0 for e in events[1:])
    if variant != "wnw_cpp":  # the deferred variant plans at the next step's start
        sim.final_plan(STEPS - 1)
    for b in range(B):
        assert set(cache._planner.get_loaded_segments(b)) == sim.planner.loaded[b]
    assert sim.n_plans > 0, "no compaction happened: the test would be vacuous"
    counts = cache.layout_counts
    if layout == "slack":  # plans relocate changed segments until the tail is used up
        assert counts["relocate"] > 0 and counts["relayout"] == L, counts
    elif layout == "tight":  # no tail: every plan rebuilds whole layers
        assert counts["relocate"] == 0 and counts["relayout_plan"] > 0, counts
    else:
        assert counts == {"relayout": 0, "relayout_plan": 0, "relocate": 0}, counts
    assert any(want_events), "no decode-time load happened: the stats check would be vacuous"


def test_appends_beyond_the_slack_rebuild_the_pool():
    """Slack of one row and no plans (nothing offloaded): appends run out of
    room every few steps and the layer moves to a fresh pool; its logical
    rows and offsets stay those of the reference's appends (bit-exact), and
    attention over them matches the oracle."""
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(12)
    Hq, Hkv, Bn, Ln = 8, 2, 3, 2
    conf = WnWConfig(chunk_size_s=8, overlap_s=0, token_rate=1.0, class_a=[], class_b=[],
                     retention_ratios=[None] * (Ln * Hkv), top_k_chunks=0, eviction_lag=2,
                     prefill_score_mode="last", num_layers=Ln, num_kv_heads=Hkv, num_q_heads=Hq)
    cache = WnWCache(conf, Ln, Hkv, Hq, D, dev, slack_rows=1)
    cache.collect_stats(0)
    cache.setup_audio(torch.zeros(Bn, dtype=torch.int64, device=dev), torch.full((Bn,), 16, device=dev), None)
    N = Bn * Hkv
    lens = [[int(x) for x in rng.integers(0, 40, N)] for _ in range(Ln)]
    K = [oracle.f32_to_bf16_bits(rng.standard_normal((sum(x), D)).astype(np.float32)) for x in lens]
    V = [oracle.f32_to_bf16_bits(rng.standard_normal((sum(x), D)).astype(np.float32)) for x in lens]
    tb = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)  # noqa: E731
    empty = torch.empty(0, D, dtype=torch.bfloat16).pin_memory()
    cache.load_prefilled_state([tb(k) for k in K], [tb(v) for v in V], lens, empty, empty, cache.restore_meta,
                               [set() for _ in range(Bn)])
    scale = D ** -0.5
    for t in range(20):
        for l in range(Ln):
            q = oracle.f32_to_bf16_bits(rng.standard_normal((Bn, Hq, 1, D)).astype(np.float32))
            nk = oracle.f32_to_bf16_bits(rng.standard_normal((Bn, Hkv, 1, D)).astype(np.float32))
            nv = oracle.f32_to_bf16_bits(rng.standard_normal((Bn, Hkv, 1, D)).astype(np.float32))
            out = decode_attention(cache, l, tb(q), tb(nk), tb(nv), scale, fused=True)
            cu_old = np.array(op.cu_from_lens(lens[l]), np.int32)
            cu_new = cu_old + np.arange(N + 1, dtype=np.int32)
            K[l] = oracle.interleave_append(K[l], nk.reshape(N, D), cu_old, cu_new, dtype=oracle.DT_BF16)
            V[l] = oracle.interleave_append(V[l], nv.reshape(N, D), cu_old, cu_new, dtype=oracle.DT_BF16)
            lens[l] = [x + 1 for x in lens[l]]
            torch.cuda.synchronize()
            assert _lib.device_error() == 0, f"step {t} layer {l}"
            dk, dv = cache.dense_kv(l)
            np.testing.assert_array_equal(_bits(dk), K[l], err_msg=f"K step {t} layer {l}")
            np.testing.assert_array_equal(_bits(dv), V[l], err_msg=f"V step {t} layer {l}")
            np.testing.assert_array_equal(cache.cu_seqlens_k[l].cpu().numpy(), cu_new)
            ref = oracle.decode_attn(q.reshape(N, Hq // Hkv, D), K[l], V[l], cu_new, scale, dtype=oracle.DT_BF16)
            got = oracle.to_f64(_bits(out.reshape(N, Hq // Hkv, D)), oracle.DT_BF16)
            ok, msg = allclose_report(got, ref, 2e-3, 1e-2)
            assert ok, f"attention step {t} layer {l}: {msg}"
    assert cache.layout_counts["relayout"] > 2 * Ln, cache.layout_counts

"""Config 4 (long-audio offload) through WnWCache at full length, every
decode step checked by the oracle simulation (``tests.cache_sim``).

Voxtral shape (32 query / 8 KV heads, head_dim 128, bf16), batch 1, a
22,628-token prompt: 64 text tokens, 22,500 audio tokens, 64 text tokens.
Per layer two KV heads are class A (full KV, 22,628 rows, scored every
step); the other six are class B: they keep 5 rows of each 256-token
segment plus the text, and the rest of their audio sits in pinned host
memory as 256-token chunks (88 segments, one chunk each).  After every step
the planner picks the top-8 chunks from the class-A scores, so with random
scores each step loads new chunks and evicts old ones; the cache relocates
the changed segments in its pools and fetches the rows from host memory.
Three layers stand in for the model's 30 (every layer's path is the same).

Checked at every step: K/V rows and offsets of every layer bit-exact
(including right after each rebuild), attention within 2e-3 + 1e-2 |ref|,
class-A scores within 1e-6 + 1e-3 |ref|, and the device's chunk top-k equal
to the oracle's ``topk_chunks(chunk_means(scores))``.  The chunk choice is
per sample, shared by every class-B head and layer, as in the reference
(src/algorithms/wnw/code/cache.py:609-630).
"""
import pytest
import torch

from tests.cache_sim import DecodeSimulation, recording
from wnw_amd import _lib
from wnw_amd.wnw.cache import WnWCache
from wnw_amd.wnw.config import WnWConfig
from wnw_amd.wnw.session import decode_attention

pytestmark = pytest.mark.gpu

L, HKV, HQ, D, B = 3, 8, 32, 128, 1
G = HQ // HKV
AUDIO, TEXT = 22500, 64
CHUNK, KEEP, TOP_K = 256, 5, 8
STEPS = 5


def _config():
    import numpy as np

    rng = np.random.default_rng(4)
    class_a, class_b = [], []
    for layer in range(L):
        a = set(rng.choice(HKV, 2, replace=False).tolist())
        class_a += [layer * HQ + kv * G + g for kv in sorted(a) for g in range(G)]
        class_b += [layer * HKV + h for h in range(HKV) if h not in a]
    return WnWConfig(chunk_size_s=CHUNK, overlap_s=0, token_rate=1.0, class_a=class_a, class_b=class_b,
                     retention_ratios=[KEEP / CHUNK] * (L * HKV), top_k_chunks=TOP_K, eviction_lag=2,
                     prefill_score_mode="last", num_layers=L, num_kv_heads=HKV, num_q_heads=HQ)


@pytest.mark.parametrize("fused,offload,small", [(True, "copy", False), (False, "copy", False), (True, "staged", False),
                                                 (True, "device", False), (True, "copy", True)])
def test_cfg4_decode_steps_match_simulation(fused, offload, small, monkeypatch):
    """``small``: the copy path's plan step (the planner and the transfer's
    start in one native call) is given loaded-row buffers too small for the
    plans, so it leaves every transfer to the Python start (``_copy_loads``);
    otherwise the copy path never falls back to it."""
    dev = torch.device("cuda", 0)
    n_py_starts = [0]
    py_start = WnWCache._copy_loads

    def counted(self, *a, **k):
        n_py_starts[0] += 1
        return py_start(self, *a, **k)
    monkeypatch.setattr(WnWCache, "_copy_loads", counted)
    # the transfer engine (DMA copies straight from the host rows, or host
    # gather threads + DMA copies, per group of layers) or the device gather
    # kernel reading pinned memory
    monkeypatch.setenv("WNW_OFFLOAD", offload)
    cfg = _config()
    cache = recording(WnWCache)(cfg, L, HKV, HQ, D, dev)
    cache.rec_acc, cache.rec_topk = [], []
    cache.collect_stats(1 << 30)  # transfer events every step, no snapshots
    S = TEXT + AUDIO + TEXT
    cache.setup_audio(torch.tensor([TEXT], device=dev), torch.tensor([TEXT + AUDIO], device=dev), None)
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    print(f"cfg4 cache test fused={fused} offload={offload} small={small}: prefill of {L} layers x {S} tokens",
          flush=True)
    for layer in range(L):
        k = torch.randn(B, HKV, S, D, device=dev, generator=gen).to(torch.bfloat16)
        v = torch.randn(B, HKV, S, D, device=dev, generator=gen).to(torch.bfloat16)
        ca = [torch.rand(AUDIO, device=dev, generator=gen)]
        per = [[None if cfg.is_class_a_kv_head(layer, h) else torch.rand(AUDIO, device=dev, generator=gen)
                for h in range(HKV)]]
        cache.prefill_after_attn(layer, ca, per, k, v)
    cache.prefill_all_layers_done()
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    assert cache._offload == offload
    if small:
        cache._staging_rows_hint = 16  # the plan step's buffers (the stage made at set-up stays)
    assert cache.cpu_restore_k.shape[0] > 6 * L * (AUDIO - AUDIO // CHUNK * KEEP) // 2  # most class-B audio on host
    sim = DecodeSimulation(cache, [(TEXT, TEXT + AUDIO)])
    scale = D ** -0.5
    for t in range(STEPS):
        qs = [torch.randn(B, HQ, 1, D, generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
        ks = [torch.randn(B, HKV, 1, D, generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
        vs = [torch.randn(B, HKV, 1, D, generator=gen, device=dev).to(torch.bfloat16) for _ in range(L)]
        print(f"step {t}", flush=True)
        outs = [decode_attention(cache, l, qs[l], ks[l], vs[l], scale, fused=fused) for l in range(L)]
        torch.cuda.synchronize()
        assert _lib.device_error() == 0, f"step {t}"
        sim.step(t, qs, ks, vs, outs)
    sim.final_plan(STEPS - 1)
    assert set(cache._planner.get_loaded_segments(0)) == sim.planner.loaded[0]
    assert sim.n_plans >= STEPS - 2, "random scores change the chunk choice nearly every step"
    assert sim.n_loaded_rows > 0
    assert cache.layout_counts["relocate"] > 0, cache.layout_counts
    if offload == "copy":
        # with room, every transfer starts with its plan; without, none does
        assert (n_py_starts[0] > 0) == small, n_py_starts[0]

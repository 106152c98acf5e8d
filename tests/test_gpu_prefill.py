"""WnWCache's prefill hooks against the prefill restatement (bit-exact).

Random bf16 K/V of two layers and three left-padded samples go through
``setup_audio`` (with an attention mask), ``prefill_after_attn`` per layer
and ``prefill_all_layers_done``.  The flat layers, their offsets, the
pinned host rows, ``restore_meta``, the loaded segments and the native
planner's view of them must equal ``oracle.prefill``'s (the host rows
through ``restore_meta``: the cache keeps them in another order).  Per-head scores
are distinct values and the class-A sums give well separated chunk means,
so no selection depends on a tie order.
"""
import numpy as np
import pytest
import torch

from oracle import prefill as opf
from wnw_amd import _lib
from wnw_amd.wnw.cache import WnWCache
from wnw_amd.wnw.config import WnWConfig

pytestmark = pytest.mark.gpu

L, H, G, D, S = 2, 4, 4, 64, 72
HQ = H * G
AUDIO = [(8, 56), (6, 62), (9, 30)]  # raw positions in the padded sequence
PADS = [0, 3, 5]
B = len(AUDIO)
CLASS_A_Q = [[0, 1, 2, 3], [5]]      # layer 0: all of KV 0's group; layer 1: one head of KV 1
CLASS_B = [[1, 2], [2, 3]]
RET = [[1.0, 0.5, 0.25, 0.75], [0.5, 1.0, 0.25, 0.5]]


def _bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("global_topk", [False, True])
def test_prefill_matches_restatement(gpu, global_topk):
    dev = gpu
    rng = np.random.default_rng(11 + global_topk)
    cfg = WnWConfig(chunk_size_s=8, overlap_s=4, token_rate=1.0,
                    class_a=[l * HQ + q for l in range(L) for q in CLASS_A_Q[l]],
                    class_b=[l * H + h for l in range(L) for h in CLASS_B[l]],
                    retention_ratios=[r for row in RET for r in row], top_k_chunks=2, eviction_lag=2,
                    prefill_score_mode="last", prefill_global_topk=global_topk,
                    num_layers=L, num_kv_heads=H, num_q_heads=HQ)
    cache = WnWCache(cfg, L, H, HQ, D, dev)
    mask = torch.ones(B, S, dtype=torch.int64)
    for b, p in enumerate(PADS):
        mask[b, :p] = 0
    cache.setup_audio(torch.tensor([s for s, _ in AUDIO], device=dev), torch.tensor([e for _, e in AUDIO], device=dev),
                      mask.to(dev))
    class_a_kv = [{q // G for q in CLASS_A_Q[l]} for l in range(L)]  # config.py:52-59
    pf = opf.Prefill(L, H, AUDIO, PADS, class_a_kv, [set(x) for x in CLASS_B], RET, stride=4, chunk=8, top_k=2,
                     global_topk=global_topk)
    for l in range(L):
        k = torch.from_numpy(rng.standard_normal((B, H, S, D), dtype=np.float32)).to(torch.bfloat16)
        v = torch.from_numpy(rng.standard_normal((B, H, S, D), dtype=np.float32)).to(torch.bfloat16)
        per = [[None if h in class_a_kv[l] else rng.permutation(e - s).astype(np.float32) / (e - s)
                for h in range(H)] for s, e in AUDIO]
        ca = []
        for s, e in AUDIO:
            n = e - s
            bonus = rng.uniform(0, 100, size=(n + 3) // 4)  # per 4-token segment
            ca.append((bonus[np.arange(n) // 4] + rng.uniform(0, 0.01, n)).astype(np.float32))
        cache.prefill_after_attn(l, [torch.from_numpy(x).to(dev) for x in ca],
                                 [[None if x is None else torch.from_numpy(x).to(dev) for x in row] for row in per],
                                 k.to(dev), v.to(dev))
        pf.after_attn(l, ca, per, _bits(k).reshape(B, H, S, D), _bits(v).reshape(B, H, S, D))
    cache.prefill_all_layers_done()
    torch.cuda.synchronize()
    pf.all_layers_done((D,), np.uint16)
    assert _lib.device_error() == 0
    for l in range(L):
        dk, dv = cache.dense_kv(l)  # the logical rows, whatever the physical layout
        np.testing.assert_array_equal(_bits(dk), pf.layer_k[l], err_msg=f"K layer {l}")
        np.testing.assert_array_equal(_bits(dv), pf.layer_v[l], err_msg=f"V layer {l}")
        assert list(cache.seq_lens[l]) == list(pf.seq_lens[l])
        cu = np.concatenate([[0], np.cumsum(pf.seq_lens[l])]).astype(np.int32)
        np.testing.assert_array_equal(cache.cu_seqlens_k[l].cpu().numpy(), cu)
    # the host rows: the same rows per (layer, sample, head, segment) through
    # restore_meta (bit-exact), the same residency offsets; the cache keeps
    # them in (sample, segment, layer, head) order, the restatement in the
    # reference's (layer, sample, head, segment) order
    hk, hv = _bits(cache.cpu_restore_k), _bits(cache.cpu_restore_v)
    assert hk.shape == pf.cpu_k.shape and hv.shape == pf.cpu_v.shape
    placed = []
    for l in range(L):
        for b in range(B):
            for h in range(H):
                for si, (m, w) in enumerate(zip(cache.restore_meta[l][b][h], pf.meta[l][b][h])):
                    assert (m is None) == (w is None), f"restore_meta layer {l} sample {b} head {h} seg {si}"
                    if m is None:
                        continue
                    assert (m.gpu_rel_start, m.gpu_rel_end) == (w.gpu_rel_start, w.gpu_rel_end)
                    assert m.cpu_end - m.cpu_start == w.cpu_end - w.cpu_start
                    np.testing.assert_array_equal(hk[m.cpu_start:m.cpu_end], pf.cpu_k[w.cpu_start:w.cpu_end])
                    np.testing.assert_array_equal(hv[m.cpu_start:m.cpu_end], pf.cpu_v[w.cpu_start:w.cpu_end])
                    placed.append(((b, si, l, h), m.cpu_start, m.cpu_end))
    placed.sort()
    assert [p[1] for p in placed] == [0] + [p[2] for p in placed[:-1]] and placed[-1][2] == hk.shape[0], \
        "host rows in (sample, segment, layer, head) order, back to back"
    assert cache.cpu_restore_k.is_pinned()
    for b in range(B):
        assert set(cache.loaded_segments[b]) == pf.loaded[b]
        assert set(cache._planner.get_loaded_segments(b)) == pf.loaded[b]
    assert any(pf.loaded) and pf.cpu_k.shape[0] > 0, "the case must offload and load rows"

"""WnWConfig and the cache's offset / geometry helpers (CPU only).

Hand-computed expectations (reference src/algorithms/wnw/code/config.py and
cache.py:1092-1162); the geometry helpers are also held to the independent
restatements in oracle/planner.py.
"""
import json

import pytest
import torch

from oracle import planner as op
from wnw_amd.wnw import cache as wc
from wnw_amd.wnw.config import WnWConfig


def _cfg(**kw):
    base = dict(chunk_size_s=4.0, overlap_s=2.0, token_rate=10.0, class_a=[0, 1, 2, 3, 32 + 9], class_b=[1, 2, 8 + 5],
                retention_ratios=[0.5] * 16, top_k_chunks=4, eviction_lag=3, prefill_score_mode="mean_text",
                num_layers=2, num_kv_heads=8, num_q_heads=32)
    base.update(kw)
    return WnWConfig(**base)


def test_chunk_geometry_truncates_like_the_reference():
    # 2.4 s * 12.5 = 30 tokens; 1.25 s * 12.5 = 15.625 -> 15; stride 15 tiles the chunk
    c = _cfg(chunk_size_s=2.4, overlap_s=1.25, token_rate=12.5)
    assert (c.chunk_size_tokens, c.overlap_tokens, c.stride_tokens) == (30, 15, 15)


def test_bad_geometry_is_rejected():
    with pytest.raises(AssertionError):  # 25 tokens, overlap 6 -> stride 19 does not tile 25
        _cfg(chunk_size_s=2.0, overlap_s=0.5, token_rate=12.5)
    with pytest.raises(AssertionError):  # overlap >= chunk
        _cfg(chunk_size_s=1.0, overlap_s=1.0)


def test_class_sets_map_query_heads_to_kv_heads():
    c = _cfg(chunk_size_s=4.0, overlap_s=2.0, token_rate=10.0)  # 40, 20, stride 20
    assert (c.chunk_size_tokens, c.overlap_tokens, c.stride_tokens) == (40, 20, 20)
    assert c.get_layer_class_a(0) == [0, 1, 2, 3] and c.get_layer_class_a(1) == [9]
    assert c.get_layer_class_b(0) == [1, 2] and c.get_layer_class_b(1) == [5]
    assert c.is_class_a_kv_head(0, 0) and not c.is_class_a_kv_head(0, 1)
    assert c.is_class_a_kv_head(1, 2)  # q head 9 of layer 1 -> kv 9 // 4 = 2
    assert c.is_class_a(1, 9) and not c.is_class_a(1, 8)
    assert c.is_class_b(1, 5) and not c.is_class_b(0, 5)
    assert c.get_retention(1, 3) == 0.5


def test_from_json(tmp_path):
    raw = {"chunk": {"size_s": 4.0, "overlap_s": 2.0, "token_rate": 10.0},
           "heads": {"class_a": [1], "class_b": [0, 3], "retention_ratios": [0.25, None, None, 0.5]},
           "selection": {"top_k_chunks": 8, "eviction_lag": 2}, "score": {"prefill_mode": "last"}}
    p = tmp_path / "c.json"
    p.write_text(json.dumps(raw))
    c = WnWConfig.from_json(str(p), num_layers=1, num_kv_heads=4, num_q_heads=8)
    assert c.top_k_chunks == 8 and c.eviction_lag == 2 and c.prefill_score_mode == "last"
    assert not c.prefill_global_topk and c.is_class_a_kv_head(0, 0) and c.get_retention(0, 3) == 0.5
    raw["score"]["prefill_mode"] = "bogus"
    p.write_text(json.dumps(raw))
    with pytest.raises(AssertionError):
        WnWConfig.from_json(str(p), 1, 4, 8)


@pytest.mark.parametrize("n,stride,chunk", [(0, 4, 8), (1, 4, 8), (7500, 19, 38), (41, 5, 15), (40, 4, 4)])
def test_segments_and_chunks(n, stride, chunk):
    segs = wc._compute_segments(n, stride)
    assert segs == op.compute_segments(n, stride)
    if n:
        assert segs[0][0] == 0 and segs[-1][1] == n
        assert all(b - a == stride for a, b in segs[:-1]) and 0 < segs[-1][1] - segs[-1][0] <= stride
    chunks = wc._compute_chunks(segs, chunk, stride)
    assert chunks == op.compute_chunks(segs, chunk, stride)
    per = -(-chunk // stride)
    assert all(c == list(range(i, min(i + per, len(segs)))) for i, c in enumerate(chunks))


def test_cu_seqlens_and_invert_ranges():
    lens = [3, 0, 5, 1]
    assert wc._build_cu_seqlens_list(lens) == [0, 3, 3, 8, 9] == op.cu_from_lens(lens)
    t = wc._build_cu_seqlens(lens, torch.device("cpu"))
    assert t.dtype == torch.int32 and t.tolist() == [0, 3, 3, 8, 9]
    assert wc._invert_ranges([(2, 4), (6, 7)], 10) == [(0, 2), (4, 6), (7, 10)]
    assert wc._invert_ranges([(0, 10)], 10) == []
    assert wc._invert_ranges([], 3) == [(0, 3)]


def test_topk_selection_keeps_per_segment_budget():
    scores = torch.tensor([0.1, 0.9, 0.5, 0.2, 0.8, 0.3, 0.7])
    kept = wc._select_topk_per_segment(scores, [(0, 3), (3, 6), (6, 7)], 0.5)
    # budgets max(1, int(3 * 0.5)) = 1, 1, 1
    assert kept.tolist() == [False, True, False, False, True, False, True]
    kept = wc._select_topk_global(scores, [(0, 3), (3, 6), (6, 7)], 0.5)
    assert kept.tolist() == [False, True, False, False, True, False, True]

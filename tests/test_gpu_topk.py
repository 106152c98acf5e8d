"""Device chunk top-k (``wnw_chunk_topk``) against the oracle planner's
``topk_chunks(chunk_means(...))`` (oracle/planner.py), which restates the
reference's chunk selection (src/algorithms/wnw/code/cache.py:632-649;
batched with -1 padding in src/algorithms/wnw_cpp/code/cache.py:160-171).

Indices are compared exactly.  Random scores are checked with
``assert_topk_matches_oracle``, which accepts a different choice only among
chunks within float32 rounding of the k-th mean; the exact cases use scores
whose chunk sums and means are exact in float32, so there the device must
give the oracle's list itself, in the oracle's order.
"""
import numpy as np
import pytest
import torch

from oracle import planner as op
from tests.cache_sim import assert_topk_matches_oracle
from wnw_amd import _lib
from wnw_amd.wnw.cache import _compute_chunks, _compute_segments
from wnw_amd.wnw.kernels import chunk_topk

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _chunk_bounds(n_audio, stride, chunk):
    """The cache's chunk token bounds of one sample (cache.py:168-210)."""
    segs = _compute_segments(n_audio, stride)
    return [(segs[c[0]][0], segs[c[-1]][1]) for c in _compute_chunks(segs, chunk, stride)]


def _run(scores_per_sample, bounds_per_sample, k):
    lens = [len(s) for s in scores_per_sample]
    acc = np.concatenate([np.asarray(s, np.float32) for s in scores_per_sample]) if lens else np.zeros(0, np.float32)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    coff = np.concatenate([[0], np.cumsum([len(b) for b in bounds_per_sample])]).astype(np.int32)
    flat = [se for b in bounds_per_sample for se in b]
    i32 = dict(dtype=torch.int32, device=DEV)
    out = torch.full((len(lens), k), -7, **i32)
    chunk_topk(torch.from_numpy(acc).to(DEV), torch.tensor(offs, **i32), torch.tensor(coff, **i32),
               torch.tensor([s for s, _ in flat], **i32), torch.tensor([e for _, e in flat], **i32), k, out)
    got = out.cpu().numpy()
    assert _lib.device_error() == 0
    return acc.astype(np.float64), offs, got


def _want(scores, bounds, k):
    w = op.topk_chunks(op.chunk_means(np.asarray(scores, np.float64), bounds), k)
    return w + [-1] * (k - len(w))


@pytest.mark.parametrize("seed", [0, 1])
def test_random_scores_overlapping_chunks(seed):
    rng = np.random.default_rng(seed)
    # three samples: long audio, short audio (fewer chunks than k), one chunk
    lens = [22500, 700, 90]
    bounds = [_chunk_bounds(n, 25, 256) for n in lens]  # 11 segments per chunk: overlapping bounds
    scores = [rng.random(n, dtype=np.float32) * 1e-2 for n in lens]
    k = 8
    acc, offs, got = _run(scores, bounds, k)
    rows = [[int(c) for c in r if c >= 0] for r in got]
    for b in range(3):
        n = min(k, len(bounds[b]))
        assert list(got[b, n:]) == [-1] * (k - n), f"sample {b}: {got[b]}"
        means = op.chunk_means(acc[offs[b]:offs[b + 1]], bounds[b])
        m = [means[c] for c in rows[b]]
        tol = 1e-5 * max(abs(x) for x in means) + 1e-7
        assert all(m[i] >= m[i + 1] - tol for i in range(len(m) - 1)), f"sample {b}: not in descending order"
    assert_topk_matches_oracle(rows, acc, offs, bounds, k, f"seed {seed}")


def test_exact_means_give_the_oracle_list():
    """Dyadic scores and power-of-two chunk lengths: every sum and mean is
    exact in float32, so the device list equals the oracle's, order included."""
    rng = np.random.default_rng(3)
    n = 4096
    bounds = [(i * 64, i * 64 + 64) for i in range(n // 64)] + [(i * 128, i * 128 + 128) for i in range(n // 128)]
    scores = rng.integers(0, 64, n).astype(np.float32) / 64
    for k in (1, 5, 17, 64):
        _, _, got = _run([scores], [bounds], k)
        assert list(got[0]) == _want(scores, bounds, k), f"k={k}"


def test_ties_go_to_the_lower_chunk():
    n = 1000
    bounds = _chunk_bounds(n, 10, 40)
    const = np.full(n, 0.25, np.float32)
    _, _, got = _run([const], [bounds], 6)
    assert list(got[0]) == [0, 1, 2, 3, 4, 5]
    # two separated peaks of equal height, all other chunks lower
    s = np.zeros(n, np.float32)
    s[300:310] = 1.0
    s[700:710] = 1.0
    bounds = [(i * 10, i * 10 + 10) for i in range(n // 10)]
    _, _, got = _run([s], [bounds], 4)
    assert list(got[0]) == [30, 70, 0, 1]
    assert list(got[0]) == _want(s, bounds, 4)


def test_short_samples_pad_with_minus_one():
    """k above a sample's chunk count (and a sample with no chunks at all),
    as the reference's masked topk (wnw_cpp/code/cache.py:167-171)."""
    scores = [np.array([0.5, 0.25, 1.0, 0.0], np.float32), np.zeros(3, np.float32), np.array([], np.float32)]
    bounds = [[(0, 2), (2, 4), (1, 3)], [], []]
    _, _, got = _run(scores, bounds, 5)
    assert list(got[0]) == _want(scores[0], bounds[0], 5) == [2, 1, 0, -1, -1]
    assert list(got[1]) == [-1] * 5
    assert list(got[2]) == [-1] * 5


def test_empty_chunk_has_mean_zero():
    """A chunk with no tokens scores 0 (sum 0 over max(1, 0) tokens)."""
    scores = np.array([-1.0, -2.0, -3.0], np.float32)
    bounds = [(0, 1), (1, 1), (1, 3)]
    _, _, got = _run([scores], [bounds], 3)
    assert list(got[0]) == _want(scores, bounds, 3) == [1, 0, 2]


def test_most_chunks_per_sample():
    rng = np.random.default_rng(9)
    nc = _lib.TOPK_MAX_CHUNKS
    bounds = [(i * 4, i * 4 + 4) for i in range(nc)]
    scores = rng.integers(0, 1 << 12, nc * 4).astype(np.float32) / 4096  # sums of 4 exact, means exact
    got_all = []
    for _ in range(2):
        _, _, got = _run([scores, scores[::-1].copy()], [bounds, bounds], _lib.TOPK_MAX_K)
        got_all.append(got)
        assert list(got[0]) == _want(scores, bounds, _lib.TOPK_MAX_K)
        assert list(got[1]) == _want(scores[::-1], bounds, _lib.TOPK_MAX_K)
    np.testing.assert_array_equal(got_all[0], got_all[1])


def test_out_of_range_bounds_are_flagged_and_never_chosen():
    scores = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    bounds = [(0, 2), (2, 9), (1, 3)]  # chunk 1 ends past the sample's scores
    i32 = dict(dtype=torch.int32, device=DEV)
    out = torch.empty(1, 3, **i32)
    chunk_topk(torch.tensor(scores, device=DEV), torch.tensor([0, 4], **i32), torch.tensor([0, 3], **i32),
               torch.tensor([s for s, _ in bounds], **i32), torch.tensor([e for _, e in bounds], **i32), 3, out)
    assert _lib.device_error() == _lib.DEVERR_BOUNDS
    assert out.cpu().tolist() == [[2, 0, -1]]
    assert _lib.device_error() == 0


def test_argument_errors():
    i32 = dict(dtype=torch.int32, device=DEV)
    z = torch.zeros(2, **i32)
    acc = torch.zeros(4, device=DEV)
    with pytest.raises(_lib.WnwError):
        chunk_topk(acc, z, z, z, z, _lib.TOPK_MAX_K + 1, torch.empty(1, _lib.TOPK_MAX_K + 1, **i32))
    with pytest.raises(_lib.WnwError):
        chunk_topk(acc.double(), z, z, z, z, 1, torch.empty(1, 1, **i32))
    with pytest.raises(_lib.WnwError):
        chunk_topk(acc, z, z, z, z, 2, torch.empty(1, 3, **i32))

"""The slack layout's compaction as bench.py times it (``compaction_slack``):
cfg5's first layer at full size (512 segments, lognormal lengths), every
class-B segment moved into a free region with sink + window eviction (drop
relative row 4), no loads.  The moved rows are bit-exact against the
oracle's rebuild of the same descriptors (``oracle.rebuild_append_kv``, the
reference's index rules of src/algorithms/wnw/code/kernels.py:407-473,
whose appended row is ignored here), and the class-A segments' rows are left
untouched."""
import os
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import bench  # noqa: E402
import oracle  # noqa: E402
from oracle import planner as op  # noqa: E402
from tests.cache_sim import bits  # noqa: E402
from wnw_amd import _lib, workloads  # noqa: E402
from wnw_amd.wnw.kernels import compact_segments  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["cfg5", "cfg2"])
def test_slack_move_matches_oracle(name):
    dev = torch.device("cuda", 0)
    cfg = workloads.CONFIGS[name](layers=1)
    D, N = cfg.head_dim, cfg.n_seg
    print(f"slack compaction: {cfg.name} layer 0, {N} segments", flush=True)
    cache = bench.build_cache(cfg, dev, slack_rows=16, score=False)
    pool_k_before = bits(cache.layer_k[0])
    kw, info = bench.slack_move_call(cfg, cache, 0, dev)
    compact_segments(**kw)
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    segs, new_len, dst_base = info["segs"], info["new_len"], info["dst_base"]
    assert len(segs) > 0 and info["rows_moved"] == int(new_len[segs].sum())

    # the oracle: the dense layer rebuilt with the same evictions (and a
    # dummy appended row per segment, which the move does not write)
    dk, dv = (bits(t) for t in cache.dense_kv(0))
    lens = np.asarray(cache.seq_lens[0], np.int64)
    ev_off = kw["evict_offsets"].cpu().numpy()
    n_b = int(ev_off[-1])
    zero = np.zeros((N, D), np.uint16)
    empty = np.zeros((0, D), np.uint16)
    cu_old = np.array(op.cu_from_lens(lens), np.int32)
    cu_ref = np.array(op.cu_from_lens(new_len + 1), np.int32)
    rk, rv = oracle.rebuild_append_kv(dk, dv, zero, zero, empty, empty, cu_old, cu_ref, np.full(N, -1, np.int32),
                                      np.zeros(N, np.int32), ev_off, np.full(n_b, 4, np.int32),
                                      np.full(n_b, 5, np.int32), 1, dtype=oracle.DT_BF16)
    got_k, got_v = bits(kw["dst_k"]), bits(kw["dst_v"])
    for f in segs:
        n, b, r = int(new_len[f]), int(dst_base[f]), int(cu_ref[f])
        np.testing.assert_array_equal(got_k[b:b + n], rk[r:r + n], err_msg=f"K segment {f}")
        np.testing.assert_array_equal(got_v[b:b + n], rv[r:r + n], err_msg=f"V segment {f}")
    # the source pool is read only
    np.testing.assert_array_equal(bits(cache.layer_k[0]), pool_k_before)

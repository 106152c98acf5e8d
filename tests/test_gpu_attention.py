"""GPU parity of the split-K decode attention against the float64 oracle.

Tolerance: max-abs 2e-3 / max-rel 1e-2, applied as
|got - ref| <= 2e-3 + 1e-2 * |ref| elementwise (bf16/f16 in, fp32 softmax
and accumulation, output in the input dtype).  fp32 inputs are held to
1e-4 / 1e-3.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.helpers import DTYPE_CODES, allclose_report, cu_from_lens, from_torch, rand_rows, to_torch
from wnw_amd import _lib
from wnw_amd import workloads
from wnw_amd.kv import fused_attn

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _tol(dtype):
    return (1e-4, 1e-3) if dtype == "float32" else (ATOL, RTOL)


def _run_case(dev, lens, G, D, dtype, kernel="auto", n_wg=0, scale=None, seed=0, kv_scale=1.0, base=None,
              pool_rows=None):
    rng = np.random.default_rng(seed)
    n = len(lens)
    cu = cu_from_lens(lens)
    T = int(cu[-1])
    scale = D ** -0.5 if scale is None else scale
    q = rand_rows(rng, n * G, D, dtype).reshape(n, G, D)
    rows = T if pool_rows is None else pool_rows
    k = rand_rows(rng, rows, D, dtype, kv_scale)
    v = rand_rows(rng, rows, D, dtype, kv_scale)
    code = DTYPE_CODES[dtype]
    ref = oracle.decode_attn(q, k, v, cu, scale, base=base, dtype=code)
    tq = to_torch(q, dtype, dev)
    tk = to_torch(k, dtype, dev)
    tv = to_torch(v, dtype, dev)
    tcu = torch.from_numpy(cu).to(dev)
    tb = None if base is None else torch.from_numpy(np.asarray(base, np.int64)).to(dev)
    print(f"case n_seg={n} T={T} G={G} D={D} {dtype} kernel={kernel} n_wg={n_wg} seed={seed}", flush=True)
    out = fused_attn.decode_attn(tq, tk, tv, tcu, scale, seg_base=tb, total_rows=T, kernel=kernel, n_wg=n_wg)
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    got = oracle.to_f64(from_torch(out, dtype), code)
    return got, ref


@pytest.mark.parametrize("kernel", ["stream", "mfma", "valu"])
@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("G", [1, 4, 7, 8, 16])
def test_small_ragged(gpu, kernel, dtype, G):
    if kernel == "stream" and G > 8:
        pytest.skip("the streaming kernel takes groups of up to 8 heads")
    lens = [1, 2, 31, 32, 33, 64, 100, 257, 0, 5, 1000, 3]
    got, ref = _run_case(gpu, lens, G, 128, dtype, kernel=kernel, seed=G)
    ok, msg = allclose_report(got, ref, *_tol(dtype))
    assert ok, msg
    assert np.all(got[8] == 0)  # empty segment


@pytest.mark.parametrize("kernel", ["stream", "mfma"])
@pytest.mark.parametrize("D", [64, 128])
def test_head_dims(gpu, D, kernel):
    got, ref = _run_case(gpu, [70, 1, 300, 129], 4, D, "bfloat16", seed=11, kernel=kernel)
    ok, msg = allclose_report(got, ref, ATOL, RTOL)
    assert ok, msg


def test_valu_head_dim_256(gpu):
    got, ref = _run_case(gpu, [70, 1, 300, 129], 4, 256, "bfloat16", kernel="valu", seed=12)
    ok, msg = allclose_report(got, ref, ATOL, RTOL)
    assert ok, msg


@pytest.mark.parametrize("kernel", ["stream", "mfma"])
@pytest.mark.parametrize("n_wg", [1, 2, 3, 7, 64, 333, 2048])
def test_split_counts_agree(gpu, n_wg, kernel):
    """Any stream-K split must give the no-split result (log-sum-exp merge identity)."""
    lens = [513, 7565, 1, 90, 2048, 4]
    got, ref = _run_case(gpu, lens, 4, 128, "bfloat16", n_wg=n_wg, seed=5, kernel=kernel)
    ok, msg = allclose_report(got, ref, ATOL, RTOL)
    assert ok, msg


def test_more_workgroups_than_rows(gpu):
    got, ref = _run_case(gpu, [1, 0, 2, 1], 4, 128, "bfloat16", n_wg=50, seed=6)
    ok, msg = allclose_report(got, ref, ATOL, RTOL)
    assert ok, msg


def test_all_segments_empty(gpu):
    """Segments with no rows return zeros, as flash-style varlen kernels (the
    reference's default `varlen_attn`, session.py:101-106) do for an empty
    key range.  This departs from the reference's Triton q1_decode_attn,
    which divides 0 by 0 there (src/common/kv/fused_attn.py:42, o = acc / l
    with l = 0) and returns NaN; the cache never makes an empty segment
    (every segment holds at least the step's own row)."""
    got, ref = _run_case(gpu, [0, 0, 0], 4, 128, "bfloat16", seed=7)
    assert np.all(got == 0)
    np.testing.assert_array_equal(ref, 0.0)  # the oracle keeps the same rule


def test_single_row_returns_v_exactly(gpu):
    """One key: softmax weight is exactly 1, so the output equals the V row bit for bit."""
    rng = np.random.default_rng(8)
    n, G, D = 40, 4, 128
    q = rand_rows(rng, n * G, D, "bfloat16").reshape(n, G, D)
    k = rand_rows(rng, n, D, "bfloat16")
    v = rand_rows(rng, n, D, "bfloat16")
    cu = np.arange(n + 1, dtype=np.int32)
    out = fused_attn.decode_attn(to_torch(q, "bfloat16", gpu), to_torch(k, "bfloat16", gpu),
                                 to_torch(v, "bfloat16", gpu), torch.from_numpy(cu).to(gpu), 0.088)
    got = from_torch(out, "bfloat16")
    for g in range(G):
        np.testing.assert_array_equal(got[:, g, :], v)


def test_slack_layout_with_seg_base(gpu):
    """Per-segment slack: segments in index order with gaps (garbage rows between)."""
    lens = [40, 0, 700, 33, 1, 129]
    caps = [64, 8, 800, 40, 9, 200]
    base = np.zeros(len(lens), np.int64)
    pos = 3
    for s in range(len(lens)):
        base[s] = pos
        pos += caps[s] + 5
    got, ref = _run_case(gpu, lens, 7, 128, "bfloat16", seed=9, base=base, pool_rows=pos + 10)
    ok, msg = allclose_report(got, ref, ATOL, RTOL)
    assert ok, msg


def test_slack_layout_many_workgroups(gpu):
    """Slack layout where workgroup ranges start inside gaps (speculative loads discarded)."""
    rng = np.random.default_rng(19)
    lens = rng.integers(1, 400, size=40)
    base = np.zeros(40, np.int64)
    pos = 0
    for s in range(40):
        pos += int(rng.integers(0, 70))  # gap
        base[s] = pos
        pos += int(lens[s])
    for n_wg in (0, 17, 333):
        got, ref = _run_case(gpu, lens, 4, 128, "bfloat16", seed=19, base=base, pool_rows=pos + 3, n_wg=n_wg)
        ok, msg = allclose_report(got, ref, ATOL, RTOL)
        assert ok, msg


@pytest.mark.parametrize("kernel", ["stream", "mfma", "valu"])
@pytest.mark.parametrize("n_seg", [5, 90])
def test_segments_in_any_physical_order(gpu, kernel, n_seg):
    """The work split runs over logical rows, so segments may sit anywhere in
    the K/V arrays, in any order and with gaps (n_seg 5: the streaming
    kernel's direct prologue; 90: its table pass)."""
    rng = np.random.default_rng(n_seg)
    lens = [int(x) for x in rng.integers(0, 700, n_seg)]
    order = rng.permutation(n_seg)
    base = np.zeros(n_seg, np.int64)
    pos = 7
    for s in order:
        base[s] = pos
        pos += lens[s] + int(rng.integers(0, 5))
    for n_wg in (0, 13):
        got, ref = _run_case(gpu, lens, 4, 128, "bfloat16", kernel=kernel, seed=n_seg + n_wg, base=base,
                             pool_rows=pos + 2, n_wg=n_wg)
        ok, msg = allclose_report(got, ref, ATOL, RTOL)
        assert ok, msg


@pytest.mark.parametrize("kernel", ["stream", "mfma", "valu"])
@pytest.mark.parametrize("n_seg", [3, 80])
def test_decreasing_offsets_leave_workspace_valid(gpu, kernel, n_seg):
    """Decreasing offsets (a corrupt table: segments overlap in the logical
    row space) are flagged, and every workgroup then skips the split-K
    hand-off: the arrival counters stay at zero, so a valid launch that
    follows on the same workspace (same n_seg, so it is not cleared in
    between) is exact.  n_seg 3 takes the streaming kernel's direct
    prologue, 80 its table pass; every segment crosses a boundary of the
    four workgroup ranges."""
    G, D, n_wg = 4, 128, 4
    rng = np.random.default_rng(5)
    cu_bad = np.array([30 * s for s in range(n_seg + 1)], np.int32)
    # segment 0 = rows [0, 45); segment 1's offsets decrease (45 -> 40);
    # segment 2 = [40, 90) overlaps segment 0 in the logical row space
    cu_bad[1] = 45
    cu_bad[2] = 40
    rows = int(cu_bad[-1]) + 10
    q = torch.zeros(n_seg, G, D, dtype=torch.bfloat16, device=gpu)
    kv = torch.zeros(rows, D, dtype=torch.bfloat16, device=gpu)
    ws = fused_attn.AttnWorkspace(gpu)
    print(f"decreasing offsets kernel={kernel} n_seg={n_seg}", flush=True)
    fused_attn.decode_attn(q, kv, kv, torch.from_numpy(cu_bad).to(gpu), 0.1, kernel=kernel, n_wg=n_wg,
                           workspace=ws)
    torch.cuda.synchronize()
    assert _lib.device_error() & _lib.DEVERR_ORDER
    counters = ws.buf[:4 * n_seg].view(torch.int32)
    assert int(counters.abs().sum().item()) == 0, "an arrival counter was left non-zero"
    # a valid launch on the same workspace: slack layout, ragged lengths
    lens2 = [int(x) for x in rng.integers(1, 90, n_seg)]
    base2 = np.zeros(n_seg, np.int64)
    pos = 3
    for s in range(n_seg):
        base2[s] = pos
        pos += lens2[s] + 2
    qn = rand_rows(rng, n_seg * G, D, "bfloat16").reshape(n_seg, G, D)
    kn, vn = rand_rows(rng, pos, D, "bfloat16"), rand_rows(rng, pos, D, "bfloat16")
    cu2 = cu_from_lens(lens2)
    ref = oracle.decode_attn(qn, kn, vn, cu2, D ** -0.5, base=base2, dtype=oracle.DT_BF16)
    out = fused_attn.decode_attn(to_torch(qn, "bfloat16", gpu), to_torch(kn, "bfloat16", gpu),
                                 to_torch(vn, "bfloat16", gpu), torch.from_numpy(cu2).to(gpu), D ** -0.5,
                                 seg_base=torch.from_numpy(base2).to(gpu), total_rows=int(cu2[-1]), kernel=kernel,
                                 n_wg=n_wg, workspace=ws)
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    ok, msg = allclose_report(oracle.to_f64(from_torch(out, "bfloat16"), oracle.DT_BF16), ref, ATOL, RTOL)
    assert ok, msg


def test_repeated_launches_reuse_workspace(gpu):
    """Counters are left at zero: many launches with different shapes stay correct."""
    for i, lens in enumerate([[300, 5000, 12], [7, 7, 7, 7, 7000], [1, 2, 3], [6000, 6000]]):
        got, ref = _run_case(gpu, lens, 4, 128, "bfloat16", seed=20 + i)
        ok, msg = allclose_report(got, ref, ATOL, RTOL)
        assert ok, msg


def test_cfg1_fp32_and_bf16(gpu):
    """Config 1 (fp32 plumbing) through the VALU kernel, and its bf16 cast through MFMA."""
    cfg = workloads.config1()
    lens = cfg.lengths[0] + 1
    got, ref = _run_case(gpu, lens, cfg.group, cfg.head_dim, "float32", seed=0)
    ok, msg = allclose_report(got, ref, 1e-4, 1e-3)
    assert ok, msg
    got, ref = _run_case(gpu, lens, cfg.group, cfg.head_dim, "bfloat16", seed=0)
    ok, msg = allclose_report(got, ref, ATOL, RTOL)
    assert ok, msg


@pytest.mark.parametrize("name,layer", [("cfg2", 0), ("cfg3", 0), ("cfg5", 0)])
def test_config_layer_full_size(gpu, name, layer):
    """One full-size layer of configs 2, 3 and 5 against the float64 oracle."""
    cfg = workloads.CONFIGS[name]()
    lens = cfg.lengths[layer] + 1
    kvs = float(cfg.kv_scale[layer].mean())
    got, ref = _run_case(gpu, lens, cfg.group, cfg.head_dim, "bfloat16", seed=layer, kv_scale=kvs)
    ok, msg = allclose_report(got, ref, ATOL, RTOL)
    print(name, msg)
    assert ok, msg


def test_large_scores_are_stable(gpu):
    """Keys scaled x8: scores up to ~+-100 must not overflow the online softmax."""
    got, ref = _run_case(gpu, [2000, 33, 517], 4, 128, "bfloat16", seed=30, kv_scale=8.0)
    ok, msg = allclose_report(got, ref, ATOL, RTOL)
    assert ok, msg


def test_q1_decode_attn_reference_signature(gpu):
    rng = np.random.default_rng(31)
    lens = [100, 3000, 7]
    cu = cu_from_lens(lens)
    q = rand_rows(rng, 3 * 4, 128, "bfloat16").reshape(3, 4, 128)
    k = rand_rows(rng, int(cu[-1]), 128, "bfloat16")
    v = rand_rows(rng, int(cu[-1]), 128, "bfloat16")
    ref = oracle.decode_attn(q, k, v, cu, 0.1, dtype=oracle.DT_BF16)
    out = fused_attn.q1_decode_attn(to_torch(q, "bfloat16", gpu), to_torch(k, "bfloat16", gpu),
                                    to_torch(v, "bfloat16", gpu), torch.from_numpy(cu).to(gpu), 0.1)
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (3, 4, 128)
    ok, msg = allclose_report(oracle.to_f64(from_torch(out, "bfloat16"), oracle.DT_BF16), ref, ATOL, RTOL)
    assert ok, msg


def test_bad_offsets_are_refused_not_read(gpu):
    """A segment pointing past the K/V rows sets the device error word instead of faulting."""
    n, G, D = 2, 4, 128
    q = torch.zeros(n, G, D, dtype=torch.bfloat16, device=gpu)
    k = torch.zeros(64, D, dtype=torch.bfloat16, device=gpu)
    cu = torch.tensor([0, 10, 20], dtype=torch.int32, device=gpu)
    base = torch.tensor([0, 60], dtype=torch.int64, device=gpu)  # 60 + 10 > 64
    fused_attn.decode_attn(q, k, k, cu, 0.1, seg_base=base, total_rows=20)
    torch.cuda.synchronize()
    assert _lib.device_error() & _lib.DEVERR_BOUNDS
    # the workspace is still usable afterwards
    got, ref = _run_case(gpu, [50, 60], 4, 128, "bfloat16", seed=40)
    ok, msg = allclose_report(got, ref, ATOL, RTOL)
    assert ok, msg


@pytest.mark.parametrize("kernel", ["stream", "mfma"])
def test_many_tiny_segments(gpu, kernel):
    """More than 64 segments in one workgroup's range (segment bounds read
    from global memory instead of the LDS ring), lengths 0..3."""
    rng = np.random.default_rng(41)
    lens = rng.integers(0, 4, size=900)
    got, ref = _run_case(gpu, lens, 4, 128, "bfloat16", kernel=kernel, seed=41, n_wg=3)
    ok, msg = allclose_report(got, ref, ATOL, RTOL)
    assert ok, msg


@pytest.mark.parametrize("kernel", ["stream", "mfma", "valu"])
@pytest.mark.parametrize("n_wg", [1, 3, 64])
def test_nonfinite_rows_stay_in_their_segment(gpu, kernel, n_wg):
    """A NaN in one segment's K and an Inf in its V leave every other segment
    exact: with few workgroups, several segments share one workgroup's merge
    slots and combine, so any leak across segments would show here."""
    lens = [40, 300, 17, 129, 64, 5, 700, 33]
    bad = 3
    G, D, dtype = 4, 128, "bfloat16"
    rng = np.random.default_rng(5)
    cu = cu_from_lens(lens)
    T = int(cu[-1])
    q = rand_rows(rng, len(lens) * G, D, dtype).reshape(len(lens), G, D)
    k = rand_rows(rng, T, D, dtype)
    v = rand_rows(rng, T, D, dtype)
    k[cu[bad] + 7, 0] = 0x7FC0  # NaN
    v[cu[bad] + 2, 5] = 0x7F80  # +Inf
    ref = oracle.decode_attn(q, k, v, cu, D ** -0.5, dtype=DTYPE_CODES[dtype])
    print(f"case nonfinite kernel={kernel} n_wg={n_wg}", flush=True)
    out = fused_attn.decode_attn(to_torch(q, dtype, gpu), to_torch(k, dtype, gpu), to_torch(v, dtype, gpu),
                                 torch.from_numpy(cu).to(gpu), D ** -0.5, total_rows=T, kernel=kernel, n_wg=n_wg)
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    got = oracle.to_f64(from_torch(out, dtype), DTYPE_CODES[dtype])
    keep = [s for s in range(len(lens)) if s != bad]
    ok, msg = allclose_report(got[keep], ref[keep], ATOL, RTOL)
    assert ok, msg
    assert not np.all(np.isfinite(got[bad]))


@pytest.mark.parametrize("lens", [[17], [16, 16, 16, 16], [15, 1, 33, 64, 5], [1000, 1, 1, 1000]])
def test_stream_step_boundaries(gpu, lens):
    """Pieces ending mid-step, single-row pieces and exact multiples of the 16-row step."""
    for n_wg in (1, 2, 5):
        got, ref = _run_case(gpu, lens, 7, 128, "bfloat16", kernel="stream", seed=len(lens) + n_wg, n_wg=n_wg)
        ok, msg = allclose_report(got, ref, ATOL, RTOL)
        assert ok, msg


@pytest.mark.parametrize("n_seg", [63, 64, 65, 511, 512, 513])
def test_segment_table_sizes(gpu, n_seg):
    """Segment counts around the 64-entry blocks of the segment walk and of
    the workgroup ring, with and without per-segment bases."""
    rng = np.random.default_rng(n_seg)
    lens = rng.integers(0, 40, size=n_seg)
    base = np.zeros(n_seg, np.int64)
    pos = 0
    for s in range(n_seg):
        pos += int(rng.integers(0, 5))
        base[s] = pos
        pos += int(lens[s])
    for b in (None, base):
        for n_wg in (0, 7):
            got, ref = _run_case(gpu, lens, 4, 64, "bfloat16", kernel="stream", seed=n_seg + n_wg, base=b,
                                 pool_rows=pos + 1 if b is not None else None, n_wg=n_wg)
            ok, msg = allclose_report(got, ref, ATOL, RTOL)
            assert ok, msg


def test_workspace_reuse_across_segment_counts(gpu):
    """One cached workspace used with a large, a small, then a middle n_seg:
    bytes that held partials under one layout are counters under the next,
    so the workspace is cleared whenever n_seg changes."""
    rng = np.random.default_rng(77)
    for n_seg in (900, 65, 511, 65, 900):
        lens = rng.integers(0, 40, size=n_seg)
        for kernel in ("stream", "mfma"):
            got, ref = _run_case(gpu, lens, 4, 64, "bfloat16", kernel=kernel, seed=n_seg, n_wg=0)
            ok, msg = allclose_report(got, ref, ATOL, RTOL)
            assert ok, f"n_seg={n_seg} {kernel}: {msg}"


def _random_case(rng):
    """One seeded random configuration: kernel, dtype, shape, ragged lengths
    (empty, short, medium and long segments), dense or slack layout, split."""
    kernel = rng.choice(["stream", "stream", "stream", "mfma", "valu"])
    if kernel == "valu":
        dtype = str(rng.choice(["bfloat16", "float16", "float32"]))
        D = int(rng.choice([64, 128, 256]))
        G = int(rng.integers(1, 17))
    else:
        dtype = str(rng.choice(["bfloat16", "float16"]))
        D = int(rng.choice([64, 128]))
        G = int(rng.integers(1, 9 if kernel == "stream" else 17))
    n = int(rng.integers(1, 300))
    kind = rng.random(n)
    lens = np.where(kind < 0.1, 0, np.where(kind < 0.4, rng.integers(1, 20, n),
                                            np.where(kind < 0.8, rng.integers(20, 600, n), rng.integers(600, 5000, n))))
    lens = [int(x) for x in lens]
    base = pool = None
    if rng.random() < 0.5:  # slack layout: gaps of garbage rows between the segments
        gaps = rng.integers(0, 40, n)
        base = np.zeros(n, np.int64)
        pos = int(rng.integers(0, 16))
        for s in range(n):
            base[s] = pos
            pos += lens[s] + int(gaps[s])
        pool = pos + int(rng.integers(0, 16))
    n_wg = 0 if rng.random() < 0.5 else int(rng.integers(1, 600))
    return dict(lens=lens, G=G, D=D, dtype=dtype, kernel=str(kernel), n_wg=n_wg, base=base, pool_rows=pool)


@pytest.mark.parametrize("seed", range(40))
def test_random_configurations(gpu, seed):
    """A seeded sweep over kernels, dtypes, head sizes, groups, ragged
    segment lengths, layouts and workgroup counts, each against the oracle."""
    c = _random_case(np.random.default_rng(1000 + seed))
    if sum(c["lens"]) == 0 and c["base"] is None:
        c["lens"][0] = 1
    got, ref = _run_case(gpu, c["lens"], c["G"], c["D"], c["dtype"], kernel=c["kernel"], n_wg=c["n_wg"],
                         seed=seed, base=c["base"], pool_rows=c["pool_rows"])
    atol, rtol = _tol(c["dtype"])
    ok, msg = allclose_report(got, ref, atol, rtol)
    assert ok, f"{c['kernel']} {c['dtype']} D={c['D']} G={c['G']} n_seg={len(c['lens'])} n_wg={c['n_wg']}: {msg}"


# ---------------------------------------------------------------------------
# fused append (wnw_decode_attn_append): the step's row of every segment is
# written into its slack, and attention covers it
# ---------------------------------------------------------------------------
def _append_case(dev, lens, G, D, dtype, seed, shuffle=True, short_cap=None, score=None, tight=False,
                 rows_hint=None):
    """Random slack layout (segments in a shuffled physical order with gaps),
    one fused append + attention; returns what to compare.  ``tight``: every
    capacity exactly the length + 1; ``rows_hint``: the row estimate that
    sizes the grid (default: the rows after the append)."""
    rng = np.random.default_rng(seed)
    n = len(lens)
    lens = np.asarray(lens, np.int64)
    cap = lens + 1 + (0 if tight else rng.integers(0, 6, n))
    if short_cap is not None:
        cap[short_cap] = lens[short_cap]  # no room for the new row
    order = rng.permutation(n) if shuffle else np.arange(n)
    base = np.zeros(n, np.int64)
    pos = int(rng.integers(0, 9))
    for s in order:
        base[s] = pos
        # a segment without room gets a gap row after it, so the reference's
        # copy of its (unstored) new row never lands in a neighbour
        pos += int(cap[s]) + int(rng.integers(0, 3)) + (1 if s == short_cap else 0)
    pool = pos + 4
    k = rand_rows(rng, pool, D, dtype)
    v = rand_rows(rng, pool, D, dtype)
    nk, nv = rand_rows(rng, n, D, dtype), rand_rows(rng, n, D, dtype)
    q = rand_rows(rng, n * G, D, dtype).reshape(n, G, D)
    cu_old = cu_from_lens(lens)
    cu_new = cu_old + np.arange(n + 1, dtype=np.int32)
    want_k, want_v = k.copy(), v.copy()
    ok_rows = [s for s in range(n) if lens[s] + 1 <= cap[s]]
    want_k[base[ok_rows] + lens[ok_rows]] = nk[ok_rows]
    want_v[base[ok_rows] + lens[ok_rows]] = nv[ok_rows]
    # the attention sees every new row (read from new_k / new_v)
    att_k, att_v = k.copy(), v.copy()
    att_k[base + lens] = nk
    att_v[base + lens] = nv
    code = DTYPE_CODES[dtype]
    scale = D ** -0.5
    ref = oracle.decode_attn(q, att_k, att_v, cu_new, scale, base=base, dtype=code)
    tk, tv = to_torch(k, dtype, dev), to_torch(v, dtype, dev)
    t32 = lambda a: torch.from_numpy(np.asarray(a, np.int32)).to(dev)  # noqa: E731
    tcu_new = torch.full((n + 1,), -7, dtype=torch.int32, device=dev)
    print(f"append case n_seg={n} G={G} D={D} {dtype} seed={seed} short_cap={short_cap}", flush=True)
    app = (to_torch(nk, dtype, dev), to_torch(nv, dtype, dev), tcu_new, t32(cap))
    tb = torch.from_numpy(base).to(dev)
    if score is None:
        out = fused_attn.decode_attn(to_torch(q, dtype, dev), tk, tv, t32(cu_old), scale, seg_base=tb,
                                     total_rows=int(cu_new[-1]) if rows_hint is None else rows_hint, append=app)
        extra = None
    else:
        H, mask, a_s, a_e = score
        offs = np.concatenate([[0], np.cumsum(np.array(a_e) - np.array(a_s))]).astype(np.int32)
        acc0 = rng.random(int(offs[-1])).astype(np.float32)
        ref_acc = oracle.attn_scores(q, att_k, cu_new, scale, mask, H, a_s, a_e, offs, acc0.astype(np.float64),
                                     base=base, dtype=code)
        acc = torch.from_numpy(acc0).to(dev)
        out = fused_attn.q1_decode_attn_score(
            to_torch(q, dtype, dev), tk, tv, t32(cu_old), scale, t32(mask), H, t32(a_s), t32(a_e), acc, t32(offs),
            seg_base=tb, total_rows=int(cu_new[-1]), max_audio=int(max(np.array(a_e) - np.array(a_s))),
            append=app)
        extra = (acc, ref_acc)
    torch.cuda.synchronize()
    err = _lib.device_error()
    got = oracle.to_f64(from_torch(out, dtype), code)
    return dict(got=got, ref=ref, err=err, k=from_torch(tk, dtype), v=from_torch(tv, dtype), want_k=want_k,
                want_v=want_v, cu_new=tcu_new.cpu().numpy(), want_cu=cu_new, extra=extra)


def _check_append(r, dtype, err=0):
    assert r["err"] == err
    np.testing.assert_array_equal(r["cu_new"], r["want_cu"])
    np.testing.assert_array_equal(r["k"], r["want_k"], err_msg="K pool after the append")
    np.testing.assert_array_equal(r["v"], r["want_v"], err_msg="V pool after the append")
    ok, msg = allclose_report(r["got"], r["ref"], *_tol(dtype))
    assert ok, msg


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("G,D", [(1, 128), (4, 128), (7, 128), (8, 128), (4, 64), (8, 64)])
def test_fused_append_direct(gpu, dtype, G, D):
    """Up to 64 segments (the direct prologue), empty-before-append and
    one-row segments included, segments in a shuffled physical order."""
    lens = [0, 1, 15, 16, 17, 31, 7565, 513, 1000, 2, 300, 0, 64, 65]
    _check_append(_append_case(gpu, lens, G, D, dtype, seed=G * 10 + D), dtype)


@pytest.mark.parametrize("n_seg", [65, 300, 1100])
def test_fused_append_table_pass(gpu, n_seg):
    """More than 64 segments: the workgroup table pass (with its LDS ring, or
    the direct table reads beyond it)."""
    rng = np.random.default_rng(n_seg)
    lens = [int(x) for x in rng.integers(0, 900 if n_seg < 1000 else 90, n_seg)]
    _check_append(_append_case(gpu, lens, 4, 128, "bfloat16", seed=n_seg), "bfloat16")


def test_fused_append_walks_across_segment_windows(gpu):
    """A workgroup whose waves walk more than 64 segments (one workgroup, by
    a small row estimate, over 300 segments): a wave reads its segments in
    windows of 64, and the walk moves to the next window right after the
    last step of a window's last segment.  That segment's new row must be
    kept by its own capacity, not by the next window's: the window-last
    segments (63, 127, 191, 255) are longer than every segment of the next
    window, with every capacity exactly the length + 1."""
    n = 300
    lens = [2] * n
    for s, ln in ((63, 40), (127, 30), (191, 20), (255, 10)):
        lens[s] = ln
    r = _append_case(gpu, lens, 4, 128, "bfloat16", seed=63, shuffle=True, tight=True, rows_hint=64)
    _check_append(r, "bfloat16")


@pytest.mark.parametrize("case", ["direct", "table_pass"])
def test_fused_append_pieces_of_whole_steps(gpu, case):
    """Pieces that end their segment with a multiple of 16 old rows (the
    kernel then cuts their first step to 15 rows, so the step that ends the
    segment has room for the new row).  direct: 64 segments of 256 rows,
    R = 16384 = 1024 * 16, so with the usual grid of 256 workgroups (4 waves
    each) every wave's range is 16 rows and every segment ends a full 16-row
    piece.  table_pass: 2000 segments of 16, 32 or 48 rows, most of them
    whole inside a wave's range."""
    if case == "direct":
        lens = [256] * 64
    else:
        lens = [int(x) for x in np.random.default_rng(5).choice([16, 32, 48], 2000)]
    for dtype in ("bfloat16", "float16"):
        print(f"pieces of whole steps: {case} {dtype}", flush=True)
        _check_append(_append_case(gpu, lens, 4, 128, dtype, seed=len(lens)), dtype)


@pytest.mark.parametrize("dtype,G,D", [("float32", 4, 128), ("bfloat16", 16, 128), ("bfloat16", 4, 256)])
def test_fused_append_other_kernels(gpu, dtype, G, D):
    """Where the streaming kernel does not apply (fp32, group > 8, head_dim
    256) the entry point runs the in-place append, then the attention."""
    lens = [0, 3, 700, 129, 1, 2000, 45]
    _check_append(_append_case(gpu, lens, G, D, dtype, seed=3), dtype)


def test_fused_append_capacity_is_refused(gpu):
    """A segment without room for its new row: WNW_DEVERR_CAPACITY, and the
    row is not stored (the neighbouring rows keep their bytes)."""
    lens = [40, 300, 5, 77]
    r = _append_case(gpu, lens, 4, 128, "bfloat16", seed=9, short_cap=1)
    _check_append(r, "bfloat16", err=_lib.DEVERR_CAPACITY)


@pytest.mark.parametrize("keep_logits", [True])
def test_fused_append_with_scores(gpu, keep_logits):
    """Append + attention + class-A scores of the appended segments."""
    H = 4
    lens = [40, 300, 17, 1000, 64, 2, 513, 90]  # B = 2
    r = _append_case(gpu, lens, 4, 128, "bfloat16", seed=4, score=(H, [0, 1, 0, 1], [3, 0], [17, 2]))
    _check_append(r, "bfloat16")
    acc, ref_acc = r["extra"]
    ok, msg = allclose_report(acc.cpu().numpy().astype(np.float64), ref_acc, 1e-6, 1e-3)
    assert ok, msg


@pytest.mark.parametrize("n_seg", [6, 100])
def test_total_rows_only_sizes_the_grid(gpu, n_seg):
    """The kernel reads cu[-1] itself: a stale total_rows (as a captured
    graph keeps while the segments grow) changes the grid size at most,
    never the result."""
    rng = np.random.default_rng(31 + n_seg)
    lens = [int(x) for x in rng.integers(1, 2000, n_seg)]
    G, D = 4, 128
    cu = cu_from_lens(lens)
    T = int(cu[-1])
    q = rand_rows(rng, n_seg * G, D, "bfloat16").reshape(n_seg, G, D)
    k, v = rand_rows(rng, T, D, "bfloat16"), rand_rows(rng, T, D, "bfloat16")
    ref = oracle.decode_attn(q, k, v, cu, D ** -0.5, dtype=oracle.DT_BF16)
    base = torch.from_numpy(cu[:-1].astype(np.int64)).to(gpu)
    for total in (T // 3, T, 5 * T):
        print(f"total_rows={total} actual={T} n_seg={n_seg}", flush=True)
        out = fused_attn.decode_attn(to_torch(q, "bfloat16", gpu), to_torch(k, "bfloat16", gpu),
                                     to_torch(v, "bfloat16", gpu), torch.from_numpy(cu).to(gpu), D ** -0.5,
                                     seg_base=base, total_rows=total)
        torch.cuda.synchronize()
        assert _lib.device_error() == 0
        ok, msg = allclose_report(oracle.to_f64(from_torch(out, "bfloat16"), oracle.DT_BF16), ref, ATOL, RTOL)
        assert ok, f"total_rows={total}: {msg}"


def test_fused_append_many_tiny_segments(gpu):
    """Segments of 1-3 rows after the append: each wave ends many segments,
    more than it can save for the end of its stream, so the surplus new
    rows are stored during the stream."""
    rng = np.random.default_rng(77)
    lens = [int(x) for x in rng.integers(0, 3, 2000)]
    _check_append(_append_case(gpu, lens, 4, 128, "bfloat16", seed=77), "bfloat16")

"""Pins the CPU oracle before it is trusted as the parity checker.

The reference ships no golden vectors for this path (its only tests are
end-to-end runs that need a checkpoint and a GPU), so each oracle function
is pinned by closed forms, special cases that reduce to textbook results,
hand-worked known answers, and a second, independently written restatement:

* oracle.decode_attn (reference src/common/kv/fused_attn.py:9-44,
  src/algorithms/wnw/code/session.py:81-106):
  - two-row closed form p0 = 1 / (1 + exp(scale * (s1 - s0)))  -> catches a
    dropped or misplaced scale, a sign error, V/K swaps;
  - one row -> V exactly; equal keys or scale 0 -> mean(V);
  - per-head closed form with distinct q per GQA head -> catches a wrong
    q-head -> KV-head mapping;
  - numpy restatement (matrix form) on random ragged inputs, dense and with
    permuted physical bases;
  - bf16 / f16 bit decoding against known patterns.
* oracle.interleave_append (src/common/kv/kernels.py:7-73): hand example,
  numpy concatenation restatement, empty segments.
* oracle.rebuild_append_kv (src/algorithms/wnw/code/kernels.py:407-473):
  hand example, the reference's own second formulation (torch.cat of keep
  slices, src/algorithms/wnw/code/cache.py:891-1010 + :1153-1162) restated
  as oracle.rebuild_by_slices, length invariant
  new_len = old_len - evicted + loaded + 1, degenerate case == append, and
  the MAX_EVICT truncation rule.
"""
import numpy as np
import pytest

import oracle
from oracle import DT_BF16, DT_F16, DT_F32
from tests.helpers import cu_from_lens, rand_rebuild_descriptors, rand_rows


# --------------------------------------------------------------------------
# decode attention
# --------------------------------------------------------------------------
def test_attn_two_row_closed_form():
    a, b, c = 0.7, -1.3, 0.37
    q = np.array([[[1.0, 0.0]]], dtype=np.float32)
    k = np.array([[a, 0.0], [b, 0.0]], dtype=np.float32)
    v = np.array([[2.0, -1.0], [-3.0, 5.0]], dtype=np.float32)
    out = oracle.decode_attn(q, k, v, np.array([0, 2]), c)
    a64, b64 = float(np.float32(a)), float(np.float32(b))
    p0 = 1.0 / (1.0 + np.exp(c * (b64 - a64)))
    want = p0 * v[0].astype(np.float64) + (1 - p0) * v[1].astype(np.float64)
    np.testing.assert_allclose(out[0, 0], want, rtol=1e-13, atol=1e-13)


def test_attn_single_row_returns_v():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((3, 4, 16)).astype(np.float32)
    k = rng.standard_normal((3, 16)).astype(np.float32)
    v = rng.standard_normal((3, 16)).astype(np.float32)
    out = oracle.decode_attn(q, k, v, np.array([0, 1, 2, 3]), 0.25)
    for s in range(3):
        for g in range(4):
            np.testing.assert_array_equal(out[s, g], v[s].astype(np.float64))


def test_attn_equal_keys_and_zero_scale_give_mean():
    rng = np.random.default_rng(2)
    n, d = 37, 8
    q = rng.standard_normal((1, 2, d)).astype(np.float32)
    v = rng.standard_normal((n, d)).astype(np.float32)
    k_eq = np.tile(rng.standard_normal((1, d)).astype(np.float32), (n, 1))
    k_rand = rng.standard_normal((n, d)).astype(np.float32)
    mean = v.astype(np.float64).mean(axis=0)
    np.testing.assert_allclose(oracle.decode_attn(q, k_eq, v, np.array([0, n]), 0.3)[0, 1], mean, rtol=1e-12,
                               atol=1e-12)
    np.testing.assert_allclose(oracle.decode_attn(q, k_rand, v, np.array([0, n]), 0.0)[0, 0], mean, rtol=1e-12,
                               atol=1e-12)


def test_attn_gqa_head_mapping_closed_form():
    # Two segments, G = 3, D = 1: q[s, g] = g + 1 + 10 s, two keys per segment.
    G = 3
    q = np.array([[[g + 1 + 10 * s] for g in range(G)] for s in range(2)], dtype=np.float32)
    k = np.array([[0.5], [-0.25], [0.125], [1.0]], dtype=np.float32)
    v = np.array([[1.0], [-1.0], [4.0], [2.0]], dtype=np.float32)
    scale = 0.5
    out = oracle.decode_attn(q, k, v, np.array([0, 2, 4]), scale)
    for s in range(2):
        k0, k1 = float(k[2 * s, 0]), float(k[2 * s + 1, 0])
        v0, v1 = float(v[2 * s, 0]), float(v[2 * s + 1, 0])
        for g in range(G):
            qq = float(q[s, g, 0])
            p0 = 1.0 / (1.0 + np.exp(scale * qq * (k1 - k0)))
            assert out[s, g, 0] == pytest.approx(p0 * v0 + (1 - p0) * v1, rel=1e-13, abs=1e-13)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_attn_matches_numpy_restatement(dtype):
    rng = np.random.default_rng(3)
    lens = [0, 1, 5, 64, 65, 200, 3, 0, 129]
    n, G, D = len(lens), 4, 32
    cu = cu_from_lens(lens)
    T = int(cu[-1])
    code = {"float32": DT_F32, "bfloat16": DT_BF16, "float16": DT_F16}[dtype]
    q = rand_rows(rng, n * G, D, dtype).reshape(n, G, D)
    k = rand_rows(rng, T, D, dtype)
    v = rand_rows(rng, T, D, dtype)
    got = oracle.decode_attn(q, k, v, cu, 0.17, dtype=code)
    ref = oracle.np_decode_attn(oracle.to_f64(q, code), oracle.to_f64(k, code), oracle.to_f64(v, code), cu, 0.17)
    np.testing.assert_allclose(got, ref, rtol=1e-11, atol=1e-12)
    assert np.all(got[0] == 0) and np.all(got[7] == 0)  # empty segments -> zeros


def test_attn_physical_base_matches_dense():
    rng = np.random.default_rng(4)
    lens = [7, 0, 33, 12]
    cu = cu_from_lens(lens)
    T = int(cu[-1])
    q = rng.standard_normal((4, 2, 16)).astype(np.float32)
    k = rng.standard_normal((T, 16)).astype(np.float32)
    v = rng.standard_normal((T, 16)).astype(np.float32)
    dense = oracle.decode_attn(q, k, v, cu, 0.3)
    # scatter segments in reverse order with gaps
    base = np.zeros(4, dtype=np.int64)
    pk = np.full((T + 40, 16), np.nan, dtype=np.float32)
    pv = np.full((T + 40, 16), np.nan, dtype=np.float32)
    pos = 5
    for s in reversed(range(4)):
        base[s] = pos
        pk[pos:pos + lens[s]] = k[cu[s]:cu[s + 1]]
        pv[pos:pos + lens[s]] = v[cu[s]:cu[s + 1]]
        pos += lens[s] + 3
    np.testing.assert_array_equal(oracle.decode_attn(q, pk, pv, cu, 0.3, base=base), dense)


def test_attn_rejects_out_of_range_base():
    q = np.zeros((1, 1, 8), np.float32)
    k = np.zeros((4, 8), np.float32)
    with pytest.raises(ValueError):
        oracle.decode_attn(q, k, k, np.array([0, 4]), 1.0, base=np.array([1]))


def test_half_and_bfloat_decoding():
    bf = np.array([0x3F80, 0xC000, 0x0000, 0x4049], dtype=np.uint16)
    np.testing.assert_array_equal(oracle.to_f64(bf, DT_BF16), [1.0, -2.0, 0.0, 3.140625])
    hf = np.array([0x3C00, 0xC000, 0x0001, 0x7BFF], dtype=np.uint16)
    np.testing.assert_array_equal(oracle.to_f64(hf, DT_F16), [1.0, -2.0, 2.0 ** -24, 65504.0])
    # the C oracle decodes the same bits (single-row attention returns V)
    v = np.array([[0x3F80, 0xC000]], dtype=np.uint16)
    out = oracle.decode_attn(np.zeros((1, 1, 2), np.uint16), np.zeros((1, 2), np.uint16), v, np.array([0, 1]),
                             1.0, dtype=DT_BF16)
    np.testing.assert_array_equal(out[0, 0], [1.0, -2.0])
    vh = np.array([[0x0001, 0x7BFF]], dtype=np.uint16)
    outh = oracle.decode_attn(np.zeros((1, 1, 2), np.uint16), np.zeros((1, 2), np.uint16), vh, np.array([0, 1]),
                              1.0, dtype=DT_F16)
    np.testing.assert_array_equal(outh[0, 0], [2.0 ** -24, 65504.0])


def test_bf16_rounding_is_nearest_even():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.5, 3.0e38], dtype=np.float32)
    bits = oracle.f32_to_bf16_bits(x)
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 3*2^-8 is a tie -> even (1 + 2^-6)
    np.testing.assert_array_equal(oracle.bf16_bits_to_f32(bits), [1.0, 1.0, 1.0 + 2 ** -6, -1.5,
                                                                  oracle.bf16_bits_to_f32(np.array([0x7F62],
                                                                                                   np.uint16))[0]])


# --------------------------------------------------------------------------
# append
# --------------------------------------------------------------------------
def test_interleave_append_hand_example():
    old = np.array([[1], [2], [3], [4], [5]], dtype=np.float32)  # segs [1,2] [] [3,4,5]
    new = np.array([[10], [20], [30]], dtype=np.float32)
    cu_old = np.array([0, 2, 2, 5])
    cu_new = np.array([0, 3, 4, 8])
    out = oracle.interleave_append(old, new, cu_old, cu_new)
    np.testing.assert_array_equal(out[:, 0], [1, 2, 10, 20, 3, 4, 5, 30])


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_interleave_append_matches_concat(dtype):
    rng = np.random.default_rng(5)
    lens = rng.integers(0, 50, size=40)
    cu_old = cu_from_lens(lens)
    cu_new = cu_old + np.arange(41, dtype=np.int32)
    old = rand_rows(rng, int(cu_old[-1]), 24, dtype)
    new = rand_rows(rng, 40, 24, dtype)
    code = {"float32": DT_F32, "bfloat16": DT_BF16}[dtype]
    got = oracle.interleave_append(old, new, cu_old, cu_new, dtype=code)
    np.testing.assert_array_equal(got, oracle.np_interleave_append(old, new, cu_old))


# --------------------------------------------------------------------------
# compaction
# --------------------------------------------------------------------------
def _rebuild_case(rng, n=24, d=16, dtype="float32", pool=100):
    lens = rng.integers(0, 80, size=n)
    old_cu = cu_from_lens(lens)
    T = int(old_cu[-1])
    ok = rand_rows(rng, T, d, dtype)
    ov = rand_rows(rng, T, d, dtype)
    nk = rand_rows(rng, n, d, dtype)
    nv = rand_rows(rng, n, d, dtype)
    lk = rand_rows(rng, pool, d, dtype)
    lv = rand_rows(rng, pool, d, dtype)
    ls, ll, eo, es, ee, nl = rand_rebuild_descriptors(rng, lens, pool)
    return lens, old_cu, ok, ov, nk, nv, lk, lv, ls, ll, eo, es, ee, nl


def test_rebuild_hand_example():
    # one segment [a b c d e], evict rel [1,3) -> a d e, load 2 rows, new token
    old = np.arange(5, dtype=np.float32).reshape(5, 1)
    load = np.array([[100], [101], [102]], dtype=np.float32)
    new = np.array([[-1]], dtype=np.float32)
    ok, ov = oracle.rebuild_append_kv(old, old + 50, new, new - 50, load, load + 50, [0, 5], [0, 6], [1], [2],
                                      [0, 1], [1], [3], 1)
    np.testing.assert_array_equal(ok[:, 0], [0, 3, 4, 101, 102, -1])
    np.testing.assert_array_equal(ov[:, 0], [50, 53, 54, 151, 152, -51])


@pytest.mark.parametrize("seed", range(5))
def test_rebuild_two_formulations_agree(seed):
    rng = np.random.default_rng(100 + seed)
    lens, old_cu, ok, ov, nk, nv, lk, lv, ls, ll, eo, es, ee, nl = _rebuild_case(rng)
    new_cu = cu_from_lens(nl)
    max_evict = int(np.max(np.diff(eo))) if len(es) else 0
    a_k, a_v = oracle.rebuild_append_kv(ok, ov, nk, nv, lk, lv, old_cu, new_cu, ls, ll, eo, es, ee, max_evict)
    b_k, b_v, b_cu = oracle.rebuild_by_slices(ok, ov, nk, nv, lk, lv, old_cu, ls, ll, eo, es, ee)
    np.testing.assert_array_equal(b_cu, new_cu)
    np.testing.assert_array_equal(a_k, b_k)
    np.testing.assert_array_equal(a_v, b_v)
    # length invariant
    evicted = np.array([int(np.sum(ee[eo[s]:eo[s + 1]] - es[eo[s]:eo[s + 1]])) for s in range(len(lens))])
    np.testing.assert_array_equal(nl, lens - evicted + ll + 1)


def test_rebuild_without_changes_is_append():
    rng = np.random.default_rng(7)
    lens = rng.integers(0, 30, size=12)
    old_cu = cu_from_lens(lens)
    new_cu = old_cu + np.arange(13, dtype=np.int32)
    ok = rand_rows(rng, int(old_cu[-1]), 8, "float32")
    nk = rand_rows(rng, 12, 8, "float32")
    empty = np.zeros((0, 8), np.float32)
    zeros = np.zeros(12, np.int32)
    a_k, _ = oracle.rebuild_append_kv(ok, ok, nk, nk, empty, empty, old_cu, new_cu, zeros - 1, zeros,
                                      np.zeros(13, np.int32), np.zeros(0, np.int32), np.zeros(0, np.int32), 0)
    np.testing.assert_array_equal(a_k, oracle.interleave_append(ok, nk, old_cu, new_cu))


def test_rebuild_max_evict_truncation():
    # two ranges but MAX_EVICT = 1: only [0,1) is removed, [3,4) is kept
    old = np.arange(6, dtype=np.float32).reshape(6, 1)
    new = np.array([[9]], dtype=np.float32)
    empty = np.zeros((0, 1), np.float32)
    ok, _ = oracle.rebuild_append_kv(old, old, new, new, empty, empty, [0, 6], [0, 6], [-1], [0], [0, 2], [0, 3],
                                     [1, 4], 1)
    np.testing.assert_array_equal(ok[:, 0], [1, 2, 3, 4, 5, 9])


# ---------------------------------------------------------------------------
# class-A token scores (oracle_segment_scores)
# ---------------------------------------------------------------------------
def _np_scores(q, k, r0, r1, a0, a1, off, scale, acc_len):
    """Independent formulation: numpy softmax per (item, head)."""
    acc = np.zeros(acc_len)
    for i in range(q.shape[0]):
        seg = k[r0[i]:r1[i]].astype(np.float64)
        logits = seg @ q[i].astype(np.float64).T * scale          # [rows, nh]
        w = np.exp(logits - logits.max(axis=0))
        w /= w.sum(axis=0)
        acc[off[i]:off[i] + a1[i] - a0[i]] += w[a0[i]:a1[i]].sum(axis=1)
    return acc


def test_scores_whole_segment_sum_to_head_count():
    """With the audio range = the whole segment, the weights of each head sum to 1."""
    rng = np.random.default_rng(50)
    nh, d = 3, 16
    lens = [5, 40, 1]
    k = rng.standard_normal((sum(lens), d)).astype(np.float32)
    q = rng.standard_normal((3, nh, d)).astype(np.float32)
    r0 = np.cumsum([0] + lens[:-1])
    r1 = r0 + lens
    acc = np.zeros(sum(lens))
    oracle.segment_scores(q, k, r0, r1, [0] * 3, lens, r0, 0.3, acc, dtype=oracle.DT_F32)
    for i in range(3):
        assert abs(acc[r0[i]:r1[i]].sum() - nh) < 1e-12


def test_scores_closed_forms():
    d = 8
    k = np.tile(np.arange(d, dtype=np.float32), (10, 1))  # equal keys: uniform weights
    q = np.ones((1, 2, d), np.float32)
    acc = np.zeros(4)
    oracle.segment_scores(q, k, [0], [10], [3], [7], [0], 0.5, acc, dtype=oracle.DT_F32)
    np.testing.assert_allclose(acc, [2 / 10] * 4, rtol=0, atol=1e-15)
    acc = np.zeros(1)  # one row: weight exactly 1 per head
    oracle.segment_scores(q, k[:1], [0], [1], [0], [1], [0], 0.5, acc, dtype=oracle.DT_F32)
    assert acc[0] == 2.0


def test_scores_match_numpy_and_accumulate():
    rng = np.random.default_rng(51)
    nh, d = 4, 32
    lens = [30, 7, 64]
    k = rng.standard_normal((120, d)).astype(np.float32)
    q = rng.standard_normal((3, nh, d)).astype(np.float32)
    r0 = np.array([2, 40, 50])  # arbitrary placement inside K (ranges may overlap)
    r1 = r0 + lens
    a0, a1 = np.array([3, 0, 10]), np.array([20, 7, 64])
    off = np.array([0, 17, 24])
    acc = np.full(24 + 54, 0.25)
    want = _np_scores(q, k, r0, r1, a0, a1, off, 0.2, acc.size) + 0.25
    oracle.segment_scores(q, k, r0, r1, a0, a1, off, 0.2, acc, dtype=oracle.DT_F32)
    np.testing.assert_allclose(acc, want, rtol=1e-12, atol=1e-14)


def test_attn_scores_maps_flagged_segments():
    """Only segments of flagged KV heads contribute; audio offsets are per sample."""
    rng = np.random.default_rng(52)
    H, G, d = 3, 2, 16
    lens = [12, 9, 15, 11, 8, 20]  # B = 2
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    k = rng.standard_normal((cu[-1], d)).astype(np.float32)
    q = rng.standard_normal((6, G, d)).astype(np.float32)
    mask = [0, 1, 1]
    a_s, a_e, offs = [2, 1], [7, 6], [0, 5, 10]
    acc = np.zeros(10)
    oracle.attn_scores(q, k, cu, 0.25, mask, H, a_s, a_e, offs, acc, dtype=oracle.DT_F32)
    want = np.zeros(10)
    for s in range(6):
        if mask[s % H]:
            b = s // H
            want += _np_scores(q[s:s + 1], k, [cu[s]], [cu[s + 1]], [a_s[b]], [a_e[b]], [offs[b]], 0.25, 10)
    np.testing.assert_allclose(acc, want, rtol=1e-12, atol=1e-14)

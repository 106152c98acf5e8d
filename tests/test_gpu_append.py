"""GPU parity of the append / compaction gathers: bit-exact against the oracle."""
import numpy as np
import pytest
import torch

import oracle
from tests.helpers import DTYPE_CODES, cu_from_lens, from_torch, rand_rebuild_descriptors, rand_rows, to_torch
from wnw_amd import _lib
from wnw_amd.kv import kernels as kv_kernels
from wnw_amd.wnw import kernels as wnw_kernels

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("dtype,D", [("bfloat16", 128), ("float32", 128), ("float16", 64), ("bfloat16", 256)])
@pytest.mark.parametrize("n_seg", [1, 16, 64, 1500])
def test_interleave_append_bit_exact(gpu, dtype, D, n_seg):
    rng = np.random.default_rng(n_seg + D)
    lens = rng.integers(0, 300, size=n_seg)
    lens[rng.random(n_seg) < 0.1] = 0
    cu_old = cu_from_lens(lens)
    cu_new = cu_old + np.arange(n_seg + 1, dtype=np.int32)
    old = rand_rows(rng, int(cu_old[-1]), D, dtype)
    new = rand_rows(rng, n_seg, D, dtype)
    print(f"interleave_append n_seg={n_seg} rows={cu_old[-1]} {dtype} D={D}", flush=True)
    ref = oracle.interleave_append(old, new, cu_old, cu_new, dtype=DTYPE_CODES[dtype])
    out = kv_kernels.interleave_append(to_torch(old, dtype, gpu), to_torch(new, dtype, gpu), _t(cu_old, gpu),
                                       _t(cu_new, gpu))
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    np.testing.assert_array_equal(from_torch(out, dtype), ref)


@pytest.mark.parametrize("dtype,D", [("bfloat16", 128), ("float32", 128), ("float16", 64)])
@pytest.mark.parametrize("n_seg", [1, 64, 1500])
def test_interleave_append_kv_bit_exact(gpu, dtype, D, n_seg):
    """K and V appended in one launch: each bit-exact against the oracle's
    interleave_append of that tensor (the reference's two calls)."""
    rng = np.random.default_rng(7 * n_seg + D)
    lens = rng.integers(0, 300, size=n_seg)
    lens[rng.random(n_seg) < 0.1] = 0
    cu_old = cu_from_lens(lens)
    cu_new = cu_old + np.arange(n_seg + 1, dtype=np.int32)
    ok_, ov_ = rand_rows(rng, int(cu_old[-1]), D, dtype), rand_rows(rng, int(cu_old[-1]), D, dtype)
    nk, nv = rand_rows(rng, n_seg, D, dtype), rand_rows(rng, n_seg, D, dtype)
    print(f"interleave_append_kv n_seg={n_seg} rows={cu_old[-1]} {dtype} D={D}", flush=True)
    code = DTYPE_CODES[dtype]
    rk = oracle.interleave_append(ok_, nk, cu_old, cu_new, dtype=code)
    rv = oracle.interleave_append(ov_, nv, cu_old, cu_new, dtype=code)
    gk, gv = kv_kernels.interleave_append_kv(to_torch(ok_, dtype, gpu), to_torch(ov_, dtype, gpu),
                                             to_torch(nk, dtype, gpu), to_torch(nv, dtype, gpu), _t(cu_old, gpu),
                                             _t(cu_new, gpu))
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    np.testing.assert_array_equal(from_torch(gk, dtype), rk)
    np.testing.assert_array_equal(from_torch(gv, dtype), rv)


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_rebuild_append_kv_bit_exact(gpu, seed, dtype):
    rng = np.random.default_rng(200 + seed)
    n, D, pool = 96, 128, 700
    lens = rng.integers(0, 600, size=n)
    old_cu = cu_from_lens(lens)
    T = int(old_cu[-1])
    ok, ov = rand_rows(rng, T, D, dtype), rand_rows(rng, T, D, dtype)
    nk, nv = rand_rows(rng, n, D, dtype), rand_rows(rng, n, D, dtype)
    lk, lv = rand_rows(rng, pool, D, dtype), rand_rows(rng, pool, D, dtype)
    ls, ll, eo, es, ee, nl = rand_rebuild_descriptors(rng, lens, pool, max_ranges=5)
    new_cu = cu_from_lens(nl)
    max_evict = int(np.max(np.diff(eo)))
    code = DTYPE_CODES[dtype]
    rk, rv = oracle.rebuild_append_kv(ok, ov, nk, nv, lk, lv, old_cu, new_cu, ls, ll, eo, es, ee, max_evict,
                                      dtype=code)
    print(f"rebuild seed={seed} rows={T} -> {new_cu[-1]} evict_ranges={len(es)}", flush=True)
    T_ = lambda a: to_torch(a, dtype, gpu)  # noqa: E731
    gk, gv = wnw_kernels.rebuild_append_kv(T_(ok), T_(ov), T_(nk), T_(nv), T_(lk), T_(lv), _t(old_cu, gpu),
                                           _t(new_cu, gpu), _t(ls, gpu), _t(ll, gpu), _t(eo, gpu), _t(es, gpu),
                                           _t(ee, gpu), max_evict)
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    np.testing.assert_array_equal(from_torch(gk, dtype), rk)
    np.testing.assert_array_equal(from_torch(gv, dtype), rv)


def test_rebuild_max_evict_truncation_matches_reference_rule(gpu):
    old = np.arange(6, dtype=np.float32).reshape(6, 1).repeat(4, axis=1)
    new = np.full((1, 4), 9, dtype=np.float32)
    empty = np.zeros((0, 4), np.float32)
    args = dict(old_cu=[0, 6], new_cu=[0, 6], load_starts=[-1], load_lens=[0], evict_offsets=[0, 2],
                evict_starts=[0, 3], evict_ends=[1, 4])
    rk, _ = oracle.rebuild_append_kv(old, old, new, new, empty, empty, max_evict=1, **args)
    ti = {k: _t(np.asarray(v, np.int32), gpu) for k, v in args.items()}
    tf = lambda a: _t(a, gpu)  # noqa: E731
    gk, _ = wnw_kernels.rebuild_append_kv(tf(old), tf(old), tf(new), tf(new), tf(empty), tf(empty),
                                          max_evict=1, **ti)
    np.testing.assert_array_equal(gk.cpu().numpy(), rk)


def test_append_inplace_and_compact_segments(gpu):
    """Slack layout: in-place append, then compaction of listed segments into fresh
    regions; the logical view must equal the oracle's dense rebuild."""
    rng = np.random.default_rng(300)
    n, D, dtype = 48, 128, "bfloat16"
    lens = rng.integers(1, 400, size=n)
    cap = lens + 8
    base = np.zeros(n, np.int64)
    base[1:] = np.cumsum(cap)[:-1]
    pool_rows = int(cap.sum()) + 20000
    k = rand_rows(rng, pool_rows, D, dtype)
    v = rand_rows(rng, pool_rows, D, dtype)
    cu_old = cu_from_lens(lens)
    nk, nv = rand_rows(rng, n, D, dtype), rand_rows(rng, n, D, dtype)
    tk, tv = to_torch(k, dtype, gpu), to_torch(v, dtype, gpu)
    cu_new_t = torch.zeros(n + 1, dtype=torch.int32, device=gpu)
    kv_kernels.append_inplace(tk, tv, to_torch(nk, dtype, gpu), to_torch(nv, dtype, gpu), _t(cu_old, gpu),
                              cu_new_t, _t(base, gpu), _t(cap.astype(np.int32), gpu))
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    np.testing.assert_array_equal(cu_new_t.cpu().numpy(), cu_old + np.arange(n + 1))
    k_after = from_torch(tk, dtype)
    # expected: dense append of the logical view
    dense_old = np.concatenate([k[base[s]:base[s] + lens[s]] for s in range(n)])
    ref_append = oracle.interleave_append(dense_old, nk, cu_old, cu_old + np.arange(n + 1), dtype=oracle.DT_BF16)
    lens1 = lens + 1
    view = np.concatenate([k_after[base[s]:base[s] + lens1[s]] for s in range(n)])
    np.testing.assert_array_equal(view, ref_append)

    # compaction of a subset of segments (evictions + loads + a second new row)
    pool = 500
    lk, lv = rand_rows(rng, pool, D, dtype), rand_rows(rng, pool, D, dtype)
    ls, ll, eo, es, ee, nl = rand_rebuild_descriptors(rng, lens1, pool, max_ranges=3, p_change=0.7)
    nk2, nv2 = rand_rows(rng, n, D, dtype), rand_rows(rng, n, D, dtype)
    listed = np.array(sorted(rng.choice(n, size=20, replace=False)), dtype=np.int32)
    dst_base = base.copy()
    cursor = int(cap.sum()) + 100
    for s in listed:
        dst_base[s] = cursor
        cursor += int(nl[s]) + 4
    assert cursor < pool_rows
    v_after = from_torch(tv, dtype)
    print(f"compact_segments listed={len(listed)} max_new={nl[listed].max()}", flush=True)
    # every device array is kept in `dev` until after the launch (a temporary
    # freed early would hand its block to the next argument's allocation)
    dev = dict(nk=to_torch(nk2, dtype, gpu), nv=to_torch(nv2, dtype, gpu), lk=to_torch(lk, dtype, gpu),
               lv=to_torch(lv, dtype, gpu), listed=_t(listed, gpu), base=_t(base, gpu),
               src_len=_t(lens1.astype(np.int32), gpu), dst_base=_t(dst_base, gpu), nl=_t(nl, gpu),
               ls=_t(ls, gpu), ll=_t(ll, gpu), eo=_t(eo, gpu), es=_t(es, gpu), ee=_t(ee, gpu))
    P = {k: _lib.ptr(t) for k, t in dev.items()}
    _lib.check(_lib.lib().wnw_compact_segments(
        _lib.ptr(tk), _lib.ptr(tv), _lib.ptr(tk), _lib.ptr(tv), P["nk"], P["nv"], P["lk"], P["lv"], P["listed"],
        len(listed), n, int(nl[listed].max()), P["base"], P["src_len"], P["dst_base"], P["nl"], P["ls"], P["ll"],
        P["eo"], P["es"], P["ee"], len(es), 1, pool_rows, pool_rows, pool, D, _lib.DT_BF16,
        _lib.stream_of(gpu)), "compact_segments")
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    k_new, v_new = from_torch(tk, dtype), from_torch(tv, dtype)
    # oracle: dense rebuild of every segment, compare only the listed ones
    dense_k = np.concatenate([k_after[base[s]:base[s] + lens1[s]] for s in range(n)])
    dense_v = np.concatenate([v_after[base[s]:base[s] + lens1[s]] for s in range(n)])
    rk, rv = oracle.rebuild_append_kv(dense_k, dense_v, nk2, nv2, lk, lv, cu_from_lens(lens1), cu_from_lens(nl),
                                      ls, ll, eo, es, ee, int(np.max(np.diff(eo))), dtype=oracle.DT_BF16)
    ncu = cu_from_lens(nl)
    for s in range(n):
        if s in listed:
            np.testing.assert_array_equal(k_new[dst_base[s]:dst_base[s] + nl[s]], rk[ncu[s]:ncu[s + 1]])
            np.testing.assert_array_equal(v_new[dst_base[s]:dst_base[s] + nl[s]], rv[ncu[s]:ncu[s + 1]])
        else:  # untouched
            np.testing.assert_array_equal(k_new[base[s]:base[s] + lens1[s]], k_after[base[s]:base[s] + lens1[s]])


def test_append_inplace_capacity_is_enforced(gpu):
    D = 128
    k = torch.zeros(16, D, dtype=torch.bfloat16, device=gpu)
    new = torch.ones(2, D, dtype=torch.bfloat16, device=gpu)
    cu_old = torch.tensor([0, 4, 8], dtype=torch.int32, device=gpu)
    cu_new = torch.zeros(3, dtype=torch.int32, device=gpu)
    base = torch.tensor([0, 8], dtype=torch.int64, device=gpu)
    cap = torch.tensor([4, 8], dtype=torch.int32, device=gpu)  # segment 0 is full
    kv_kernels.append_inplace(k, k, new, new, cu_old, cu_new, base, cap)
    torch.cuda.synchronize()
    assert _lib.device_error() & _lib.DEVERR_CAPACITY
    assert torch.all(k[4] == 0)  # not written past capacity
    assert torch.all(k[12] == 1)  # segment 1 appended


def test_rebuild_beyond_infinity_cache_bit_exact(gpu):
    """A layer whose K and V output exceeds 256 MB (~600 K rows of bf16,
    d 128) takes the non-temporal copies: still bit-exact."""
    rng = np.random.default_rng(77)
    n, D, dtype = 512, 128, "bfloat16"
    lens = rng.integers(1200, 1600, size=n)
    pool = 3000
    ls, ll, eo, es, ee, nl = rand_rebuild_descriptors(rng, lens, pool, max_ranges=3)
    old_cu, new_cu = cu_from_lens(lens), cu_from_lens(nl)
    T = int(old_cu[-1])
    assert int(new_cu[-1]) * D * 2 * 2 > (256 << 20)
    bits = lambda rows: rng.integers(0, 1 << 16, size=(rows, D), dtype=np.uint16)  # noqa: E731
    ok, ov, nk, nv, lk, lv = bits(T), bits(T), bits(n), bits(n), bits(pool), bits(pool)
    max_evict = int(np.max(np.diff(eo)))
    rk, rv = oracle.rebuild_append_kv(ok, ov, nk, nv, lk, lv, old_cu, new_cu, ls, ll, eo, es, ee, max_evict,
                                      dtype=DTYPE_CODES[dtype])
    print(f"rebuild large rows={T}->{new_cu[-1]} ranges={len(es)}", flush=True)
    T_ = lambda a: to_torch(a, dtype, gpu)  # noqa: E731
    gk, gv = wnw_kernels.rebuild_append_kv(T_(ok), T_(ov), T_(nk), T_(nv), T_(lk), T_(lv), _t(old_cu, gpu),
                                           _t(new_cu, gpu), _t(ls, gpu), _t(ll, gpu), _t(eo, gpu), _t(es, gpu),
                                           _t(ee, gpu), max_evict)
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    np.testing.assert_array_equal(from_torch(gk, dtype), rk)
    np.testing.assert_array_equal(from_torch(gv, dtype), rv)


@pytest.mark.parametrize("seed", range(12))
def test_rebuild_random_sweep(gpu, seed):
    """Seeded sweep: up to 30 evict ranges per segment (several batches of
    the kernel's range reads), MAX_EVICT truncation, head sizes, dtypes."""
    rng = np.random.default_rng(500 + seed)
    dtype = str(rng.choice(["bfloat16", "float16", "float32"]))
    D = int(rng.choice([64, 128, 256]))
    n = int(rng.integers(1, 200))
    pool = int(rng.integers(0, 900))
    lens = rng.integers(0, 800, size=n)
    ls, ll, eo, es, ee, nl = rand_rebuild_descriptors(rng, lens, pool, max_ranges=int(rng.choice([3, 12, 30])),
                                                      p_change=0.8)
    widest = int(np.max(np.diff(eo))) if n else 0
    # the reference's MAX_EVICT: the widest segment's count, or fewer (later ranges ignored)
    max_evict = max(1, widest if rng.random() < 0.5 else int(rng.integers(1, max(2, widest + 1))))
    if max_evict < widest:
        # with ranges ignored, a segment keeps more rows: the reference's new length follows kept_len
        kept = []
        for s in range(n):
            k = min(int(eo[s + 1] - eo[s]), max_evict)
            kept.append(int(lens[s]) - int(np.sum(ee[eo[s]:eo[s] + k] - es[eo[s]:eo[s] + k])))
        nl = np.array([kept[s] + int(ll[s]) + 1 for s in range(n)], np.int32)
    old_cu, new_cu = cu_from_lens(lens), cu_from_lens(nl)
    T = int(old_cu[-1])
    ok, ov = rand_rows(rng, T, D, dtype), rand_rows(rng, T, D, dtype)
    nk, nv = rand_rows(rng, n, D, dtype), rand_rows(rng, n, D, dtype)
    lk, lv = rand_rows(rng, pool, D, dtype), rand_rows(rng, pool, D, dtype)
    code = DTYPE_CODES[dtype]
    rk, rv = oracle.rebuild_append_kv(ok, ov, nk, nv, lk, lv, old_cu, new_cu, ls, ll, eo, es, ee, max_evict,
                                      dtype=code)
    print(f"rebuild sweep seed={seed} {dtype} D={D} n={n} rows={T}->{new_cu[-1]} ranges={len(es)} "
          f"widest={widest} max_evict={max_evict}", flush=True)
    T_ = lambda a: to_torch(a, dtype, gpu)  # noqa: E731
    gk, gv = wnw_kernels.rebuild_append_kv(T_(ok), T_(ov), T_(nk), T_(nv), T_(lk), T_(lv), _t(old_cu, gpu),
                                           _t(new_cu, gpu), _t(ls, gpu), _t(ll, gpu), _t(eo, gpu), _t(es, gpu),
                                           _t(ee, gpu), max_evict)
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    np.testing.assert_array_equal(from_torch(gk, dtype), rk)
    np.testing.assert_array_equal(from_torch(gv, dtype), rv)

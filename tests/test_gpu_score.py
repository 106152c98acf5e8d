"""GPU parity of the class-A scorers against the float64 oracle.

Scores are sums of softmax weights (fp32 on the GPU); they are held to
|got - ref| <= 1e-6 + 1e-3 * |ref|.  The attention output of
q1_decode_attn_score is held to the attention tolerance (2e-3 + 1e-2 |ref|).
"""
import numpy as np
import pytest
import torch

import oracle
from tests.helpers import allclose_report, cu_from_lens, from_torch, rand_rows, to_torch
from wnw_amd import _lib
from wnw_amd import workloads
from wnw_amd.kv import fused_attn
from wnw_amd.wnw import kernels as wk

pytestmark = pytest.mark.gpu

S_ATOL, S_RTOL = 1e-6, 1e-3


def _attn_score_case(dev, lens, H, G, D, mask, a_s, a_e, seed, base=None, pool_rows=None, kv_scale=1.0,
                     keep_logits=True, dtype="bfloat16"):
    rng = np.random.default_rng(seed)
    odt = oracle.DT_BF16 if dtype == "bfloat16" else oracle.DT_F16
    n = len(lens)
    B = n // H
    cu = cu_from_lens(lens)
    rows = int(cu[-1]) if pool_rows is None else pool_rows
    q = rand_rows(rng, n * G, D, dtype).reshape(n, G, D)
    k = rand_rows(rng, rows, D, dtype, kv_scale)
    v = rand_rows(rng, rows, D, dtype, kv_scale)
    offs = np.concatenate([[0], np.cumsum(np.array(a_e) - np.array(a_s))]).astype(np.int32)
    acc0 = rng.random(int(offs[-1])).astype(np.float32)
    scale = D ** -0.5
    ref_out = oracle.decode_attn(q, k, v, cu, scale, base=base, dtype=odt)
    ref_acc = oracle.attn_scores(q, k, cu, scale, mask, H, a_s, a_e, offs, acc0.astype(np.float64),
                                 base=base, dtype=odt)
    t = lambda a, dt=torch.int32: torch.from_numpy(np.asarray(a)).to(dt).to(dev)  # noqa: E731
    acc = torch.from_numpy(acc0).to(dev)
    print(f"attn_score n_seg={n} H={H} G={G} D={D} mask={mask} seed={seed} keep_logits={keep_logits}", flush=True)
    out = fused_attn.q1_decode_attn_score(
        to_torch(q, dtype, dev), to_torch(k, dtype, dev), to_torch(v, dtype, dev), t(cu), scale,
        t(mask), H, t(a_s), t(a_e), acc, t(offs),
        seg_base=None if base is None else t(base, torch.int64), total_rows=int(cu[-1]),
        max_audio=int(max(np.array(a_e) - np.array(a_s))),
        keep_logits=keep_logits)
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    got_out = oracle.to_f64(from_torch(out, dtype), odt)
    return got_out, ref_out, acc.cpu().numpy().astype(np.float64), ref_acc


# keep_logits: the attention kernel keeps the scored rows' logits (streaming
# kernel) or the scoring pass reads K again; both must match the oracle.
@pytest.mark.parametrize("keep_logits", [True, False])
def test_attn_score_small(keep_logits):
    lens = [40, 300, 17, 1000, 64, 2, 513, 90]  # B = 2, H = 4
    got, ref, gacc, racc = _attn_score_case(torch.device("cuda", 0), lens, 4, 4, 128, [0, 1, 0, 1],
                                            [3, 0], [17, 2], seed=1, keep_logits=keep_logits)
    ok, msg = allclose_report(got, ref, 2e-3, 1e-2)
    assert ok, msg
    ok, msg = allclose_report(gacc, racc, S_ATOL, S_RTOL)
    assert ok, msg


@pytest.mark.parametrize("keep_logits", [True, False])
def test_attn_score_f16_head_dim_64(keep_logits):
    lens = [700, 30, 129, 64, 1, 333]  # B = 3, H = 2
    got, ref, gacc, racc = _attn_score_case(torch.device("cuda", 0), lens, 2, 4, 64, [1, 0], [0, 5, 0],
                                            [650, 100, 1], seed=5, keep_logits=keep_logits, dtype="float16")
    ok, msg = allclose_report(got, ref, 2e-3, 1e-2)
    assert ok, msg
    ok, msg = allclose_report(gacc, racc, S_ATOL, S_RTOL)
    assert ok, msg


@pytest.mark.parametrize("keep_logits", [True, False])
def test_attn_score_slack_layout_and_group7(keep_logits):
    lens = [500, 33, 260, 70]  # B = 2, H = 2
    caps = [520, 40, 300, 80]
    base = np.zeros(4, np.int64)
    pos = 5
    for s in range(4):
        base[s] = pos
        pos += caps[s] + 3
    got, ref, gacc, racc = _attn_score_case(torch.device("cuda", 0), lens, 2, 7, 128, [1, 0], [10, 5],
                                            [480, 250], seed=2, base=base, pool_rows=pos + 4,
                                            keep_logits=keep_logits)
    ok, msg = allclose_report(got, ref, 2e-3, 1e-2)
    assert ok, msg
    ok, msg = allclose_report(gacc, racc, S_ATOL, S_RTOL)
    assert ok, msg


@pytest.mark.parametrize("keep_logits", [True, False])
def test_attn_score_cfg2_layer(keep_logits):
    """One cfg2 layer at full size: class-A segments hold 7,500 audio rows."""
    cfg = workloads.config2()
    lens = cfg.lengths[0] + 1
    H = cfg.hkv
    mask = cfg.class_a[0].astype(np.int32).tolist()
    a_s, a_e = [0] * cfg.batch, [7500] * cfg.batch
    got, ref, gacc, racc = _attn_score_case(torch.device("cuda", 0), lens, H, cfg.group, cfg.head_dim, mask,
                                            a_s, a_e, seed=3, kv_scale=float(cfg.kv_scale[0].mean()),
                                            keep_logits=keep_logits)
    ok, msg = allclose_report(got, ref, 2e-3, 1e-2)
    assert ok, msg
    ok, msg = allclose_report(gacc, racc, S_ATOL, S_RTOL)
    print(msg)
    assert ok, msg


@pytest.mark.parametrize("nh,D", [(1, 128), (4, 128), (3, 64), (2, 256)])
def test_fused_score_accumulate(nh, D):
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(10 + nh)
    lens = [900, 33, 5000, 1]
    S = len(lens)
    starts = np.concatenate([[7], 7 + np.cumsum(lens)[:-1] + 11])  # gaps between items
    ends = starts + lens
    rows = int(ends[-1]) + 9
    k = rand_rows(rng, rows, D, "bfloat16")
    q = rand_rows(rng, S * nh, D, "bfloat16").reshape(S, nh, D)
    a_s = np.array([100, 0, 2500, 0], np.int32)
    a_e = np.array([800, 33, 5000, 1], np.int32)
    offs = np.concatenate([[0], np.cumsum(a_e - a_s)]).astype(np.int32)
    acc0 = rng.random(int(offs[-1])).astype(np.float32)
    ref = oracle.segment_scores(q, k, starts, ends, a_s, a_e, offs[:-1], D ** -0.5, acc0.astype(np.float64),
                                dtype=oracle.DT_BF16)
    t = lambda a: torch.from_numpy(np.asarray(a, np.int32)).to(dev)  # noqa: E731
    acc = torch.from_numpy(acc0).to(dev)
    print(f"fused_score nh={nh} D={D}", flush=True)
    wk.fused_score_accumulate(to_torch(q, "bfloat16", dev), to_torch(k, "bfloat16", dev), t(starts), t(ends),
                              t(a_s), t(a_e), acc, t(offs))
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    ok, msg = allclose_report(acc.cpu().numpy().astype(np.float64), ref, S_ATOL, S_RTOL)
    assert ok, msg


def test_score_bad_audio_range_is_flagged():
    """An audio range past its segment sets the device error word and is skipped."""
    dev = torch.device("cuda", 0)
    q = torch.zeros(2, 1, 128, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(64, 128, dtype=torch.bfloat16, device=dev)
    acc = torch.zeros(100, device=dev)
    t = lambda a: torch.tensor(a, dtype=torch.int32, device=dev)  # noqa: E731
    wk.fused_score_accumulate(q, k, t([0, 10]), t([10, 20]), t([0, 0]), t([50, 5]), acc, t([0, 50, 55]))
    torch.cuda.synchronize()
    assert _lib.device_error() & _lib.DEVERR_BOUNDS
    assert float(acc[:50].abs().sum()) == 0.0  # the bad item wrote nothing
    assert _lib.device_error() == 0


@pytest.mark.parametrize("keep_logits", [True, False])
def test_attn_score_many_tiny_segments(keep_logits):
    """8,192 segments alternating 1 and 0 rows: each workgroup's range spans
    more than 64 segment indices, so the kernels read the offsets, flags and
    audio ranges from memory instead of their LDS window."""
    B, H = 4096, 2
    lens = [1, 0] * B
    got, ref, gacc, racc = _attn_score_case(torch.device("cuda", 0), lens, H, 4, 128, [1, 0], [0] * B, [1] * B,
                                            seed=21, keep_logits=keep_logits)
    ok, msg = allclose_report(got, ref, 2e-3, 1e-2)
    assert ok, msg
    ok, msg = allclose_report(gacc, racc, S_ATOL, S_RTOL)
    assert ok, msg


@pytest.mark.parametrize("keep_logits", [True, False])
def test_attn_score_bad_audio_range_is_flagged(keep_logits):
    """A flagged segment whose audio range ends past the segment sets the
    device error word; that sample's tokens are left untouched, the other
    sample is scored."""
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(14)
    lens = [100, 50, 80, 60]  # B = 2, H = 2; KV head 0 is flagged
    cu = cu_from_lens(lens)
    q = to_torch(rand_rows(rng, 4 * 4, 64, "bfloat16").reshape(4, 4, 64), "bfloat16", dev)
    k = to_torch(rand_rows(rng, int(cu[-1]), 64, "bfloat16"), "bfloat16", dev)
    t = lambda a: torch.tensor(a, dtype=torch.int32, device=dev)  # noqa: E731
    acc = torch.zeros(170, device=dev)
    print(f"attn_score bad audio range keep_logits={keep_logits}", flush=True)
    fused_attn.q1_decode_attn_score(q, k, k, t(cu), 0.125, t([1, 0]), 2, t([0, 10]), t([120, 60]), acc,
                                    t([0, 120, 170]), max_audio=120, keep_logits=keep_logits)
    torch.cuda.synchronize()
    assert _lib.device_error() & _lib.DEVERR_BOUNDS
    assert float(acc[:120].abs().sum()) == 0.0  # sample 0: 120 audio rows in a 100-row segment
    assert float(acc[120:170].min()) > 0.0      # sample 1: scored
    assert _lib.device_error() == 0


@pytest.mark.parametrize("keep_logits", [True, False])
def test_attn_score_short_accumulator_is_flagged(keep_logits):
    """Offsets that put a sample's tokens past the accumulator's end set the
    device error word; that sample writes nothing (not even past the end:
    the accumulator is a view into a larger buffer whose tail must stay
    untouched), the other sample is scored."""
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(15)
    lens = [100, 50, 80, 60]  # B = 2, H = 2; KV head 0 is flagged
    cu = cu_from_lens(lens)
    q = to_torch(rand_rows(rng, 4 * 4, 64, "bfloat16").reshape(4, 4, 64), "bfloat16", dev)
    k = to_torch(rand_rows(rng, int(cu[-1]), 64, "bfloat16"), "bfloat16", dev)
    t = lambda a: torch.tensor(a, dtype=torch.int32, device=dev)  # noqa: E731
    big = torch.full((200,), 7.0, device=dev)
    acc = big[:150]  # sample 1's 50 tokens would need [120, 170)
    print(f"attn_score short accumulator keep_logits={keep_logits}", flush=True)
    fused_attn.q1_decode_attn_score(q, k, k, t(cu), 0.125, t([1, 0]), 2, t([0, 0]), t([60, 50]), acc,
                                    t([0, 120, 170]), max_audio=60, keep_logits=keep_logits)
    torch.cuda.synchronize()
    assert _lib.device_error() & _lib.DEVERR_BOUNDS
    host = big.cpu()
    assert float(host[:60].min()) > 7.0            # sample 0: scored
    assert bool((host[60:] == 7.0).all())          # sample 1 refused; nothing past the end written
    assert _lib.device_error() == 0


def test_fused_score_negative_offset_is_flagged():
    """A negative accumulator offset sets the device error word and writes nothing."""
    dev = torch.device("cuda", 0)
    q = torch.ones(2, 1, 128, dtype=torch.bfloat16, device=dev)
    k = torch.ones(64, 128, dtype=torch.bfloat16, device=dev)
    big = torch.zeros(100, device=dev)
    acc = big[10:]
    t = lambda a: torch.tensor(a, dtype=torch.int32, device=dev)  # noqa: E731
    wk.fused_score_accumulate(q, k, t([0, 10]), t([10, 20]), t([0, 0]), t([5, 5]), acc, t([-5, 0, 5]))
    torch.cuda.synchronize()
    assert _lib.device_error() & _lib.DEVERR_BOUNDS
    host = big.cpu()
    assert float(host[:10].abs().sum()) == 0.0   # nothing before the accumulator
    assert float(host[10:15].min()) > 0.0        # the valid item is scored
    assert _lib.device_error() == 0


@pytest.mark.parametrize("keep_logits", [True, False])
def test_attn_score_many_samples(keep_logits):
    """Enough samples x audio rows for the long (16-iteration) scoring workgroups."""
    rng = np.random.default_rng(12)
    B, H = 24, 2
    lens = [int(x) for x in rng.integers(6000, 6100, size=B * H)]
    a_s, a_e = [0] * B, [6000] * B
    got, ref, gacc, racc = _attn_score_case(torch.device("cuda", 0), lens, H, 4, 128, [1, 0], a_s, a_e, seed=12,
                                            keep_logits=keep_logits)
    ok, msg = allclose_report(got, ref, 2e-3, 1e-2)
    assert ok, msg
    ok, msg = allclose_report(gacc, racc, S_ATOL, S_RTOL)
    assert ok, msg


def test_fused_score_accumulate_many_samples():
    """fused_score_accumulate with the long (16-iteration) scoring workgroups."""
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(13)
    S, nh, D = 24, 2, 128
    lens = rng.integers(6000, 6100, size=S)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    ends = starts + lens
    k = rand_rows(rng, int(ends[-1]), D, "bfloat16")
    q = rand_rows(rng, S * nh, D, "bfloat16").reshape(S, nh, D)
    a_s = np.zeros(S, np.int32)
    a_e = np.full(S, 6000, np.int32)
    offs = np.concatenate([[0], np.cumsum(a_e - a_s)]).astype(np.int32)
    acc0 = rng.random(int(offs[-1])).astype(np.float32)
    ref = oracle.segment_scores(q, k, starts, ends, a_s, a_e, offs[:-1], D ** -0.5, acc0.astype(np.float64),
                                dtype=oracle.DT_BF16)
    t = lambda a: torch.from_numpy(np.asarray(a, np.int32)).to(dev)  # noqa: E731
    acc = torch.from_numpy(acc0).to(dev)
    wk.fused_score_accumulate(to_torch(q, "bfloat16", dev), to_torch(k, "bfloat16", dev), t(starts), t(ends),
                              t(a_s), t(a_e), acc, t(offs))
    torch.cuda.synchronize()
    assert _lib.device_error() == 0
    ok, msg = allclose_report(acc.cpu().numpy().astype(np.float64), ref, S_ATOL, S_RTOL)
    assert ok, msg


def _slack_layer(rng, lens, D, dtype, dev, slack=8):
    """A pool with `slack` spare rows after each segment (slack layout):
    (k pool, v pool, cu, seg_base, seg_cap) on the device and the host bits."""
    n = len(lens)
    cap = np.asarray(lens) + slack
    base = np.concatenate([[0], np.cumsum(cap)[:-1]]).astype(np.int64)
    rows = int(cap.sum()) + 64
    k = rand_rows(rng, rows, D, dtype)
    v = rand_rows(rng, rows, D, dtype)
    t = lambda a, dt=torch.int32: torch.from_numpy(np.asarray(a)).to(dt).to(dev)  # noqa: E731
    return dict(k=to_torch(k, dtype, dev), v=to_torch(v, dtype, dev), cu=t(cu_from_lens(lens)),
                cu_out=torch.empty(n + 1, dtype=torch.int32, device=dev), base=t(base, torch.int64),
                cap=t(cap.astype(np.int32)), rows=rows)


# (KV heads, group, samples, the layers' scored-head masks: None = a layer
# that keeps nothing), within the deferred form's 16 scored (KV head, query
# head) pairs
_DEFERRED_CASES = [
    (4, 4, 4, [[1, 0, 1, 0], [0, 1, 1, 0], None, [1, 1, 0, 1]]),
    (2, 8, 3, [[1, 1], [0, 1], [1, 0], None, [1, 1]]),
    (4, 7, 2, [[1, 0, 0, 1], None, [0, 1, 0, 0], [0, 0, 1, 1]]),
]


@pytest.mark.parametrize("H,G,B,masks", _DEFERRED_CASES)
def test_deferred_scoring_matches_the_scoring_pass(H, G, B, masks):
    """wnw_decode_attn_append_deferred over a sequence of layers (scored and
    not scored, then the last slot scored on its own) gives the same
    outputs, pools, offsets and accumulator bits as q1_decode_attn_score's
    append form (attention + its own scoring pass) layer by layer, and the
    accumulator matches the oracle."""
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(77 + G)
    D = 128
    n = B * H
    dtype = "bfloat16"
    a_s = [3, 0, 5, 1][:B]
    a_e = [900, 700, 1000, 650][:B]
    max_audio = max(e - s for s, e in zip(a_s, a_e))
    offs = np.concatenate([[0], np.cumsum(np.array(a_e) - np.array(a_s))]).astype(np.int32)
    t = lambda a, dt=torch.int32: torch.from_numpy(np.asarray(a)).to(dt).to(dev)  # noqa: E731
    layers = []
    for li in range(len(masks)):
        lens = [int(x) for x in rng.integers(1000, 1400, n)]
        layers.append(dict(lens=lens, q=rand_rows(rng, n * G, D, dtype).reshape(n, G, D),
                           nk=rand_rows(rng, n, D, dtype), nv=rand_rows(rng, n, D, dtype), seed=int(rng.integers(1 << 30))))
    acc0 = rng.random(int(offs[-1])).astype(np.float32)
    scale = D ** -0.5

    def run(deferred):
        acc = torch.from_numpy(acc0.copy()).to(dev)
        slots = [torch.empty(fused_attn.score_slot_bytes(n, G, max_audio) // 4, dtype=torch.float32, device=dev)
                 for _ in range(2)]
        outs, states, pending, turn = [], [], None, 0
        for li, lay in enumerate(layers):
            st = _slack_layer(np.random.default_rng(lay["seed"]), lay["lens"], D, dtype, dev)
            q = to_torch(lay["q"], dtype, dev)
            app = (to_torch(lay["nk"], dtype, dev), to_torch(lay["nv"], dtype, dev), st["cu_out"], st["cap"])
            rows = sum(lay["lens"]) + n
            mask = None if masks[li] is None else t(masks[li])
            if not deferred:
                if mask is None:
                    out = fused_attn.decode_attn(q, st["k"], st["v"], st["cu"], scale, seg_base=st["base"],
                                                 total_rows=rows, append=app)
                else:
                    out = fused_attn.q1_decode_attn_score(q, st["k"], st["v"], st["cu"], scale, mask, H, t(a_s),
                                                          t(a_e), acc, t(offs), seg_base=st["base"], total_rows=rows,
                                                          max_audio=max_audio, append=app)
            else:
                slot = slots[turn] if mask is not None else None
                print(f"deferred layer {li}: keep={mask is not None} prev={pending is not None}", flush=True)
                out = fused_attn.decode_attn_append_deferred(
                    q, st["k"], st["v"], st["cu"], scale, seg_base=st["base"], total_rows=rows, append=app,
                    num_kv_heads=H, audio_starts=t(a_s), audio_ends=t(a_e), max_audio=max_audio,
                    score_accumulator=acc, score_offsets=t(offs), keep_mask=mask, keep_slot=slot, prev=pending)
                assert out is not None, "the geometry is one the deferred form takes"
                pending = (mask, slot, st["cu_out"], st["base"], st["rows"],
                           sum(1 << h for h, f in enumerate(masks[li]) if f)) if mask is not None else None
                if mask is not None:
                    turn ^= 1
            outs.append(out)
            states.append(st)
        if deferred and pending is not None:
            fused_attn.score_kept_logits(pending, n, G, H, t(a_s), t(a_e), max_audio, acc, t(offs))
        torch.cuda.synchronize()
        assert _lib.device_error() == 0
        return outs, states, acc

    o1, s1, acc1 = run(False)
    o2, s2, acc2 = run(True)
    for li in range(len(layers)):
        assert torch.equal(o1[li], o2[li]), f"output layer {li}"
        for key in ("k", "v", "cu_out"):
            assert torch.equal(s1[li][key], s2[li][key]), f"{key} layer {li}"
    assert torch.equal(acc1, acc2), "accumulator bits"
    # and the accumulator against the oracle (the appended segments)
    ref = acc0.astype(np.float64)
    for li, lay in enumerate(layers):
        if masks[li] is None:
            continue
        st = s2[li]
        kb = from_torch(st["k"], dtype)
        cu2 = st["cu_out"].cpu().numpy()
        ref = oracle.attn_scores(lay["q"], kb, cu2, scale, masks[li], H, a_s, a_e, offs, ref,
                                 base=st["base"].cpu().numpy(), dtype=oracle.DT_BF16)
    ok, msg = allclose_report(acc2.cpu().numpy().astype(np.float64), ref, S_ATOL, S_RTOL)
    assert ok, msg


def test_deferred_scoring_refuses_what_it_cannot_take():
    """More than 64 segments: the deferred form launches nothing and says so
    (None), leaving the output and the accumulator untouched."""
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(78)
    H, G, D, B = 8, 4, 128, 9  # 72 segments
    n = B * H
    dtype = "bfloat16"
    lens = [int(x) for x in rng.integers(200, 300, n)]
    st = _slack_layer(rng, lens, D, dtype, dev)
    t = lambda a, dt=torch.int32: torch.from_numpy(np.asarray(a)).to(dt).to(dev)  # noqa: E731
    q = to_torch(rand_rows(rng, n * G, D, dtype).reshape(n, G, D), dtype, dev)
    app = (to_torch(rand_rows(rng, n, D, dtype), dtype, dev), to_torch(rand_rows(rng, n, D, dtype), dtype, dev),
           st["cu_out"], st["cap"])
    acc = torch.zeros(B * 100, dtype=torch.float32, device=dev)
    offs = t(np.arange(B + 1) * 100)
    slots = [torch.empty(fused_attn.score_slot_bytes(n, G, 100) // 4, dtype=torch.float32, device=dev)
             for _ in range(2)]
    mask = t([1] + [0] * (H - 1))
    out = torch.full((n, G, D), 7.0, dtype=torch.bfloat16, device=dev)
    prev = (mask, slots[0], st["cu"], st["base"], st["rows"], 1)
    got = fused_attn.decode_attn_append_deferred(
        q, st["k"], st["v"], st["cu"], D ** -0.5, seg_base=st["base"], total_rows=sum(lens) + n, append=app,
        num_kv_heads=H, audio_starts=t([0] * B), audio_ends=t([100] * B), max_audio=100, score_accumulator=acc,
        score_offsets=offs, keep_mask=mask, keep_slot=slots[1], prev=prev, out=out)
    torch.cuda.synchronize()
    assert got is None
    assert bool((out == 7.0).all()) and bool((acc == 0).all())
    assert _lib.device_error() == 0

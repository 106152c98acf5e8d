"""The prefill restatement (oracle/prefill.py) against hand-computed results
and invariants of the reference's rules (CPU only)."""
import numpy as np

from oracle import prefill as opf


def test_keep_rules_hand_values():
    s = np.array([0.9, 0.8, 0.1, 0.2, 0.3])
    segs = [(0, 2), (2, 4), (4, 5)]
    # per segment: max(1, int(len * 0.5)) = 1, 1, 1 -> the best of each
    assert set(np.nonzero(opf.keep_per_segment(s, segs, 0.5))[0]) == {0, 3, 4}
    # global: the same total (3), taken over the whole range
    assert set(np.nonzero(opf.keep_global(s, segs, 0.5))[0]) == {0, 1, 4}
    # ratio 0 still keeps one token per segment; ratio 1 keeps all
    assert opf.keep_per_segment(s, segs, 0.0).sum() == 3
    assert opf.keep_per_segment(s, segs, 1.0).all()
    # ties go to the lower index
    assert set(np.nonzero(opf.keep_per_segment(np.ones(4), [(0, 4)], 0.5))[0]) == {0, 1}


def test_prefill_hand_example():
    """One layer, two KV heads (0 class A, 1 class B at ratio 0.5), one
    sample with one pad token and audio at raw positions [3, 7)."""
    S = 10
    k = np.zeros((1, 2, S, 1), np.int64)
    for h in range(2):
        k[0, h, :, 0] = h * 100 + np.arange(S)
    pf = opf.Prefill(1, 2, audio=[(3, 7)], pads=[1], class_a_kv=[{0}], class_b=[{1}], retention=[[1.0, 0.5]],
                     stride=2, chunk=2, top_k=1)
    pf.after_attn(0, [np.array([1.0, 1.0, 5.0, 5.0])], [[None, np.array([0.2, 0.7, 0.9, 0.1])]], k, k + 1000)
    # head 0 keeps rows 1..9; head 1 keeps text rows 1, 2, 7, 8, 9 then audio rows 4, 5
    assert pf.seq_lens[0] == [9, 7]
    assert list(pf.layer_k[0][:, 0]) == list(range(1, 10)) + [101, 102, 107, 108, 109, 104, 105]
    pf.all_layers_done((1,), np.int64)
    # pruned rows 3 (segment 0) and 6 (segment 1) went to the host in that order
    assert list(pf.cpu_k[:, 0]) == [103, 106] and list(pf.cpu_v[:, 0]) == [1103, 1106]
    m0, m1 = pf.meta[0][0][1]
    assert (m0.cpu_start, m0.cpu_end, m0.gpu_rel_start) == (0, 1, -1)
    # chunk means 1 and 5: chunk 1 (segment 1) is loaded and appended to head 1
    assert pf.loaded[0] == {1}
    assert (m1.cpu_start, m1.cpu_end, m1.gpu_rel_start, m1.gpu_rel_end) == (1, 2, 7, 8)
    assert pf.seq_lens[0] == [9, 8]
    assert list(pf.layer_k[0][9:, 0]) == [101, 102, 107, 108, 109, 104, 105, 106]
    assert list(pf.layer_v[0][9:, 0]) == [1101, 1102, 1107, 1108, 1109, 1104, 1105, 1106]


def test_prefill_invariants_random():
    rng = np.random.default_rng(3)
    L, H, B, S = 3, 4, 3, 80
    audio = [(10, 70), (5, 77), (20, 21)]
    pads = [0, 4, 2]
    class_a = [{0}, {1, 2}, set()]
    class_b = [{1, 2}, {3}, {0, 2, 3}]
    ret = [[float(rng.choice([0.25, 0.5, 0.75])) for _ in range(H)] for _ in range(L)]
    pf = opf.Prefill(L, H, audio, pads, class_a, class_b, ret, stride=8, chunk=16, top_k=2)
    ks = []
    for l in range(L):
        k = rng.permutation(L * B * H * S).reshape(1, 1, 1, -1)[0, 0, 0][: B * H * S].reshape(B, H, S, 1)
        ks.append(k)
        per = [[rng.permutation(e - s).astype(float) for _ in range(H)] for s, e in audio]
        ca = [rng.random(e - s) if class_a[l] else None for s, e in audio]
        pf.after_attn(l, ca, per, k, k)
    pre_lens = [list(x) for x in pf.seq_lens]
    pf.all_layers_done((1,), np.int64)
    for l in range(L):
        cu = np.concatenate([[0], np.cumsum(pf.seq_lens[l])])
        for b in range(B):
            (ra, re), pad = audio[b], pads[b]
            for h in range(H):
                f = b * H + h
                rows = set(pf.layer_k[l][cu[f]:cu[f + 1], 0])
                audio_rows = set(ks[l][b, h, ra:re, 0])
                text_rows = set(ks[l][b, h, pad:ra, 0]) | set(ks[l][b, h, re:, 0])
                assert text_rows <= rows
                host = set()
                for m in pf.meta[l][b][h]:
                    if m is not None:
                        host |= set(pf.cpu_k[m.cpu_start:m.cpu_end, 0])
                if h in class_a[l]:
                    assert rows == audio_rows | text_rows and not host
                    continue
                kept = rows - text_rows
                nseg = len(pf.segments[b])
                want = sum(max(1, int((e - s) * ret[l][h])) for s, e in pf.segments[b])
                resident = {si for si in range(nseg) if pf.meta[l][b][h][si] is not None
                            and pf.meta[l][b][h][si].gpu_rel_start >= 0}
                loaded_rows = sum(pf.meta[l][b][h][si].cpu_end - pf.meta[l][b][h][si].cpu_start for si in resident)
                assert len(kept) == want + loaded_rows
                assert pf.seq_lens[l][f] == pre_lens[l][f] + loaded_rows
                if h in class_b[l]:
                    # kept and offloaded rows partition the audio rows
                    assert (kept - host) | host == audio_rows
                    assert resident == {si for si in pf.loaded[b] if pf.meta[l][b][h][si] is not None}
                else:
                    assert not host

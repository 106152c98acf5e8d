"""Step-by-step CPU simulation of the WnW decode path, the checker of the
end-to-end cache tests (``test_gpu_cache.py``, ``test_gpu_cache_cfg4.py``).

From a prefilled cache's state, each decode step is replayed with the
oracle: appends and plan-driven compactions (bit-exact K/V and offsets,
``oracle.interleave_append`` / ``oracle.rebuild_append_kv``), attention
(2e-3 + 1e-2 |ref|, ``oracle.decode_attn``), class-A scores (1e-6 + 1e-3
|ref|, ``oracle.segment_scores``) and the planner (``oracle.planner``).  The
chunk top-k the device computes from its own float32 scores is checked
against the oracle's ``topk_chunks(chunk_means(...))`` of the same recorded
scores, then fed to the oracle planner, so both sides plan from the same
chunks.
"""
from __future__ import annotations

import copy

import numpy as np
import torch

import oracle
from oracle import planner as op
from tests.helpers import allclose_report


def bits(t: torch.Tensor) -> np.ndarray:
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def recording(cls):
    """A cache class that records each step's score accumulator (before it is
    cleared) and the chunk top-k handed to the planner.  A step captured into
    a HIP graph records nothing (a capture runs the host side once and may
    not read device memory back)."""
    class Rec(cls):
        def decode_all_layers_done(self):
            if not torch.cuda.is_current_stream_capturing():
                self._flush_pending_scores()  # the last deferred class-A scores of the step
                self.rec_acc.append(self.score_accumulator.double().cpu().numpy().copy())
            return super().decode_all_layers_done()

        def _plan(self, topk, off):
            if not torch.cuda.is_current_stream_capturing():
                o = off.tolist()
                self.rec_topk.append([topk.tolist()[o[b]:o[b + 1]] for b in range(self.batch_size)])
            return super()._plan(topk, off)

        def _plan_and_start(self, pending):
            # the fused plan step reads the pinned [B, k] choice (-1: none)
            # itself; the planner takes each row's chosen chunks in order
            if not torch.cuda.is_current_stream_capturing():
                self._tk_event.synchronize()
                self.rec_topk.append([[c for c in row if c >= 0] for row in pending.tolist()])
            return super()._plan_and_start(pending)
    return Rec


def assert_topk_matches_oracle(got_per_sample, acc, offs, bounds_per_sample, k, what=""):
    """The device's chosen chunks of every sample equal the oracle's top-k of
    the chunk means of ``acc`` (float64 sums over each chunk's token bounds,
    oracle/planner.py).  A different choice is accepted only where the
    chunks involved are within float32 rounding of the k-th largest mean
    (the device rounds float64 prefix-sum means to float32)."""
    for b, got in enumerate(got_per_sample):
        means = op.chunk_means(acc[offs[b]:offs[b + 1]], bounds_per_sample[b])
        want = op.topk_chunks(means, k)
        assert len(got) == len(want) and len(set(got)) == len(got), f"{what} sample {b}: {got} vs {want}"
        assert all(0 <= c < len(means) for c in got), f"{what} sample {b}: {got}"
        if sorted(got) == sorted(want):
            continue
        kth = sorted(means, reverse=True)[len(want) - 1]
        tol = 1e-5 * max(abs(m) for m in means) + 1e-7
        assert all(means[c] >= kth - tol for c in got), \
            f"{what} sample {b}: device chose {sorted(got)}, oracle {sorted(want)} (means {means})"


class DecodeSimulation:
    """The oracle's view of a prefilled cache, advanced one decode step at a
    time by ``step`` (which checks the cache against it)."""

    def __init__(self, cache, audio: list[tuple[int, int]]):
        self.cache = cache
        L, H, B = cache.num_layers, cache.num_kv_heads, cache.batch_size
        self.L, self.H, self.B, self.G, self.D = L, H, B, cache.num_kv_groups, cache.head_dim
        self.K = [bits(cache.dense_kv(l)[0]) for l in range(L)]
        self.V = [bits(cache.dense_kv(l)[1]) for l in range(L)]
        self.lens = [list(cache.seq_lens[l]) for l in range(L)]
        self.host_k, self.host_v = bits(cache.cpu_restore_k), bits(cache.cpu_restore_v)
        self.meta = [[[[None if m is None else op.SegMeta(m.cpu_start, m.cpu_end, m.gpu_rel_start, m.gpu_rel_end)
                        for m in cache.restore_meta[l][b][h]] for h in range(H)] for b in range(B)]
                     for l in range(L)]
        self.loaded_after_prefill = [set(x) for x in cache.loaded_segments]
        cfg = cache.config
        self.planner = op.PlannerOracle(L, H, B, cfg.top_k_chunks, cfg.eviction_lag, cache.chunk_to_segs,
                                        [cfg.get_layer_class_b(l) for l in range(L)], self.meta,
                                        copy.deepcopy(cache.loaded_segments), self.lens)
        self.groups = []  # per layer: (kv, qheads)
        for l in range(L):
            by_kv = {}
            for qh in cfg.get_layer_class_a(l):
                by_kv.setdefault(qh // self.G, []).append(qh)
            self.groups.append(sorted(by_kv.items(), key=lambda x: x[0]))
        self.audio = audio  # relative to the segments' starts (no left padding)
        self.offs = np.concatenate([[0], np.cumsum([e - a for a, e in audio])])
        self.scale = self.D ** -0.5
        self.plan = None
        self.n_plans = 0
        self.n_loaded_rows = 0
        self.want_events = [[] for _ in range(B)]  # (step, c2g_tokens) of the decode-time loads
        self.loaded_at_snapshot = [set(x) for x in cache.loaded_segments]

    def step(self, t: int, qs, ks, vs, outs) -> None:
        """Check decode step t (inputs qs / ks / vs per layer, outputs outs)."""
        cache, L, H, B, G, D = self.cache, self.L, self.H, self.B, self.G, self.D
        if t > 0:  # the plan made from the previous step's scores applies now
            assert_topk_matches_oracle(cache.rec_topk[t - 1], cache.rec_acc[t - 1], self.offs,
                                       cache._chunk_token_bounds, cache.config.top_k_chunks, f"step {t - 1}")
            self.planner.seq_lens = [list(x) for x in self.lens]
            self.plan = self.planner.step(cache.rec_topk[t - 1])
            self.n_plans += int(self.plan.any_change)
            for b in range(B):
                n = sum(self.plan.load_lens[l][f] for l in range(L) for f in range(b * H, (b + 1) * H)) \
                    if self.plan.any_change else 0
                if n:
                    self.want_events[b].append((t + 1, n))  # planned at step t, flushed with step t + 1
                self.n_loaded_rows += n
            self.loaded_at_snapshot = [set(x) for x in self.planner.loaded]
        acc = np.zeros(int(self.offs[-1]))
        plan = self.plan
        for l in range(L):
            nk = bits(ks[l].reshape(B * H, D))
            nv = bits(vs[l].reshape(B * H, D))
            cu_old = np.array(op.cu_from_lens(self.lens[l]), np.int32)
            if plan is not None and plan.any_change:
                empty = np.zeros((0, D), np.uint16)
                load_k = np.concatenate([self.host_k[s:e] for s, e in plan.cpu_ranges]) if plan.cpu_ranges else empty
                load_v = np.concatenate([self.host_v[s:e] for s, e in plan.cpu_ranges]) if plan.cpu_ranges else empty
                cu_new = np.array(plan.cu_new[l], np.int32)
                self.K[l], self.V[l] = oracle.rebuild_append_kv(
                    self.K[l], self.V[l], nk, nv, load_k, load_v, cu_old, cu_new, plan.load_starts[l],
                    plan.load_lens[l], plan.evict_offsets[l], plan.evict_starts[l], plan.evict_ends[l],
                    plan.evict_max[l], dtype=oracle.DT_BF16)
                self.lens[l] = list(plan.new_lens[l])
            else:
                cu_new = cu_old + np.arange(B * H + 1, dtype=np.int32)
                self.K[l] = oracle.interleave_append(self.K[l], nk, cu_old, cu_new, dtype=oracle.DT_BF16)
                self.V[l] = oracle.interleave_append(self.V[l], nv, cu_old, cu_new, dtype=oracle.DT_BF16)
                self.lens[l] = [x + 1 for x in self.lens[l]]
            cu = self.check_layer(f"step {t}", l, qs[l], outs[l])
            qfull = bits(qs[l].reshape(B, H * G, D))
            for kv, qheads in self.groups[l]:
                segs = [b * H + kv for b in range(B)]
                oracle.segment_scores(qfull[:, qheads], self.K[l], [cu[s] for s in segs], [cu[s + 1] for s in segs],
                                      [a for a, _ in self.audio], [e for _, e in self.audio], self.offs[:-1],
                                      self.scale, acc, dtype=oracle.DT_BF16)
        ok, msg = allclose_report(cache.rec_acc[t], acc, 1e-6, 1e-3)
        assert ok, f"scores step {t}: {msg}"

    def check_layer(self, what: str, l: int, q=None, out=None) -> np.ndarray:
        """The cache's layer ``l`` against the oracle's state: logical K/V rows
        and device offsets bit-exact, host lengths equal, and with ``q`` and
        ``out`` the attention of that step within 2e-3 + 1e-2 |ref|.
        Returns the offsets."""
        cache, B, H, G, D = self.cache, self.B, self.H, self.G, self.D
        dk, dv = cache.dense_kv(l)
        np.testing.assert_array_equal(bits(dk), self.K[l], err_msg=f"K {what} layer {l}")
        np.testing.assert_array_equal(bits(dv), self.V[l], err_msg=f"V {what} layer {l}")
        cu = np.array(op.cu_from_lens(self.lens[l]), np.int32)
        np.testing.assert_array_equal(cache.cu_seqlens_k[l].cpu().numpy(), cu, err_msg=f"cu {what} layer {l}")
        assert list(cache.seq_lens[l]) == list(self.lens[l]), f"host lengths {what} layer {l}"
        assert cache._rows[l] == int(cu[-1]), f"host row count {what} layer {l}"
        if out is not None:
            q_flat = bits(q.reshape(B * H, G, D))
            ref = oracle.decode_attn(q_flat, self.K[l], self.V[l], cu, self.scale, dtype=oracle.DT_BF16)
            got = oracle.to_f64(bits(out.reshape(B * H, G, D)), oracle.DT_BF16)
            ok, msg = allclose_report(got, ref, 2e-3, 1e-2)
            assert ok, f"attention {what} layer {l}: {msg}"
        return cu

    def advance_plain(self, ks, vs) -> None:
        """One plain decode step on the oracle's state (every segment appends
        the step's row, no plan), checking nothing: the device work of a
        replayed captured step."""
        B, H, D = self.B, self.H, self.D
        for l in range(self.L):
            nk = bits(ks[l].reshape(B * H, D))
            nv = bits(vs[l].reshape(B * H, D))
            cu_old = np.array(op.cu_from_lens(self.lens[l]), np.int32)
            cu_new = cu_old + np.arange(B * H + 1, dtype=np.int32)
            self.K[l] = oracle.interleave_append(self.K[l], nk, cu_old, cu_new, dtype=oracle.DT_BF16)
            self.V[l] = oracle.interleave_append(self.V[l], nv, cu_old, cu_new, dtype=oracle.DT_BF16)
            self.lens[l] = [x + 1 for x in self.lens[l]]

    def final_plan(self, last_step: int) -> None:
        """The plan of the last step's scores (made by the immediate-plan cache
        at the end of that step)."""
        self.planner.seq_lens = [list(x) for x in self.lens]
        self.planner.step(self.cache.rec_topk[last_step])

"""Binding of the host->device transfer engine (``wnw_h2d_*``, csrc/transfer.hip).

The offload channel of the reference (src/algorithms/wnw_cpp/code/
planner.cpp:113-122 gathers a plan's host ranges into pinned staging;
src/algorithms/wnw/code/cache.py:716-721, :868-881 copies the staging rows to
the device on a side stream and waits for them before the rebuild), done by
a background engine group by group (groups of consecutive layers), a layer
waiting only for its own group's copy.  Two forms: ``start`` (worker threads
gather the ranges into pinned staging, then the DMA engines copy each
group) and ``start_direct`` (the DMA engines copy merged spans straight from
the pinned host rows into a device stage, and a kernel puts the rows in
transfer order).
"""
from __future__ import annotations

import ctypes
import os

import torch

from .. import _lib


class HostToDevice:
    """One engine (a lead thread and ``workers`` gather threads) per cache."""

    def __init__(self, workers: int | None = None):
        if workers is None:
            # the host's cores less a few for the caller's thread, the engine's
            # lead thread and the runtime
            workers = int(os.environ.get("WNW_H2D_WORKERS", "0")) or max(1, min(12, (os.cpu_count() or 2) - 4))
        self._h = _lib.lib().wnw_h2d_create(int(workers))
        if not self._h:
            raise _lib.WnwError("wnw_h2d_create: " + _lib.lib().wnw_last_error().decode(errors="replace"))
        self.workers = int(workers)
        self._keep = ()

    def start(self, host_k: torch.Tensor, host_v: torch.Tensor, ranges: torch.Tensor, group_ranges: list[int],
              stg_k: torch.Tensor, stg_v: torch.Tensor, dev_k: torch.Tensor, dev_v: torch.Tensor,
              stream: torch.cuda.Stream) -> None:
        """Gathers rows ``ranges[r, 0] .. ranges[r, 1]`` of the pinned host
        arrays into consecutive staging rows and copies them to the same rows
        of ``dev_k`` / ``dev_v`` on ``stream``, group ``g`` being ranges
        ``group_ranges[g] .. group_ranges[g + 1]``.  Returns at once; the
        previous start must be issued (it waits for that)."""
        for t in (host_k, host_v, stg_k, stg_v):
            if t.device.type != "cpu" or not t.is_pinned() or not t.is_contiguous():
                raise _lib.WnwError("host and staging rows must be contiguous pinned tensors")
        if ranges.dtype != torch.int32 or ranges.device.type != "cpu" or ranges.dim() != 2 or ranges.shape[1] != 2:
            raise _lib.WnwError("ranges must be a CPU int32 [n, 2] tensor")
        row_bytes = host_k.shape[1] * host_k.element_size()
        # the engine counts staging and device rows in units of the host's
        # row bytes: every array must have the host's row shape and dtype
        if host_k.shape != host_v.shape or stg_k.shape[1:] != host_k.shape[1:] or dev_k.shape[1:] != host_k.shape[1:] \
                or dev_k.shape != dev_v.shape or stg_k.shape != stg_v.shape or \
                len({host_k.dtype, host_v.dtype, stg_k.dtype, stg_v.dtype, dev_k.dtype, dev_v.dtype}) != 1:
            raise _lib.WnwError("host, staging and device rows must have one row shape and dtype")
        cur = torch.cuda.current_device()
        if not (dev_k.is_cuda and dev_v.is_cuda and dev_k.device.index == cur and dev_v.device.index == cur
                and dev_k.is_contiguous() and dev_v.is_contiguous()):
            raise _lib.WnwError("device rows must be contiguous tensors on the current device")
        rg = ranges.contiguous()
        gr = (ctypes.c_int64 * len(group_ranges))(*group_ranges)
        self._keep = (rg, gr)  # the engine copies both at start; kept for symmetry with the pointers' lifetime
        _lib.check(_lib.lib().wnw_h2d_start(
            self._h, _lib.ptr(host_k), _lib.ptr(host_v), host_k.shape[0], _lib.ptr(rg), rg.shape[0], gr,
            len(group_ranges) - 1, _lib.ptr(stg_k), _lib.ptr(stg_v), stg_k.shape[0], _lib.ptr(dev_k), _lib.ptr(dev_v),
            dev_k.shape[0], row_bytes, ctypes.c_void_p(stream.cuda_stream)), "h2d start")

    def start_direct(self, host_k: torch.Tensor, host_v: torch.Tensor, ranges: torch.Tensor,
                     group_ranges: list[int], stage_k: torch.Tensor, stage_v: torch.Tensor, dev_k: torch.Tensor,
                     dev_v: torch.Tensor, stream: torch.cuda.Stream, check: bool = True) -> None:
        """``start`` without the host gather (``wnw_h2d_start_direct``): the
        ranges are copied by the DMA engines straight from the pinned host
        rows into ``stage_k`` / ``stage_v`` (device rows, in host order per
        group, spans merged where ranges touch) and moved by a kernel on
        ``stream`` into the same transfer-order rows of ``dev_k`` /
        ``dev_v`` that ``start`` fills.  ``check=False`` skips the Python
        checks for callers whose tensors are right by construction (the
        library still checks every range and size)."""
        if check:
            for t in (host_k, host_v):
                if t.device.type != "cpu" or not t.is_pinned() or not t.is_contiguous():
                    raise _lib.WnwError("host rows must be contiguous pinned tensors")
            if ranges.dtype != torch.int32 or ranges.device.type != "cpu" or ranges.dim() != 2 or \
                    ranges.shape[1] != 2:
                raise _lib.WnwError("ranges must be a CPU int32 [n, 2] tensor")
            cur = torch.cuda.current_device()
            for t in (stage_k, stage_v, dev_k, dev_v):
                if not (t.is_cuda and t.device.index == cur and t.is_contiguous()):
                    raise _lib.WnwError("stage and device rows must be contiguous tensors on the current device")
            if host_k.shape != host_v.shape or stage_k.shape != stage_v.shape or dev_k.shape != dev_v.shape or \
                    stage_k.shape[1:] != host_k.shape[1:] or dev_k.shape[1:] != host_k.shape[1:] or \
                    len({host_k.dtype, host_v.dtype, stage_k.dtype, stage_v.dtype, dev_k.dtype, dev_v.dtype}) != 1:
                raise _lib.WnwError("host, stage and device rows must have one row shape and dtype")
        row_bytes = host_k.shape[1] * host_k.element_size()
        rg = ranges.contiguous()
        gr = (ctypes.c_int64 * len(group_ranges))(*group_ranges)
        self._keep = (rg, gr)
        _lib.check(_lib.lib().wnw_h2d_start_direct(
            self._h, _lib.ptr(host_k), _lib.ptr(host_v), host_k.shape[0], _lib.ptr(rg), rg.shape[0], gr,
            len(group_ranges) - 1, _lib.ptr(stage_k), _lib.ptr(stage_v), stage_k.shape[0], _lib.ptr(dev_k),
            _lib.ptr(dev_v), dev_k.shape[0], row_bytes, ctypes.c_void_p(stream.cuda_stream)), "h2d start_direct")

    def plan_start_direct(self, planner, topk: torch.Tensor, outs: dict, layer_cuts: list[int],
                          host_k: torch.Tensor, host_v: torch.Tensor, stage_k: torch.Tensor, stage_v: torch.Tensor,
                          dev_k: torch.Tensor, dev_v: torch.Tensor, stream: torch.cuda.Stream):
        """``wnw_h2d_plan_start_direct``: the planner's compute_and_prepare
        from the device top-k's choice (``topk``, a CPU int32 [B, k] tensor,
        -1 = none; ``outs`` its output tensors, as for compute_and_prepare),
        then, if the plan loads rows that fit the stage and device rows, the
        direct transfer of its ranges in the groups of layers ``layer_cuts``
        describes.  Returns ``(any_change, total, n_evict, n_ranges,
        started)``; with ``started`` False the caller starts the transfer
        itself.  The tensors are the caller's, right by construction (the
        library checks every index and size)."""
        tk = topk.contiguous()
        cuts = (ctypes.c_int32 * len(layer_cuts))(*layer_cuts)
        flag, started = ctypes.c_int32(0), ctypes.c_int32(0)
        total, n_ev, n_rg = ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_int64(0)
        o = outs
        row_bytes = host_k.shape[1] * host_k.element_size()
        _lib.check(_lib.lib().wnw_h2d_plan_start_direct(
            self._h, planner._h, _lib.ptr(tk), tk.shape[0], tk.shape[1] if tk.dim() == 2 else 0,
            _lib.ptr(o["load_starts_2d"]), _lib.ptr(o["load_lens_2d"]), _lib.ptr(o["cu_new_2d"]),
            _lib.ptr(o["new_lens_2d"]), _lib.ptr(o["evict_offsets_2d"]), _lib.ptr(o["evict_max"]),
            _lib.ptr(o["evict_layer_ptr"]), cuts, len(layer_cuts) - 1, _lib.ptr(host_k), _lib.ptr(host_v),
            host_k.shape[0], _lib.ptr(stage_k), _lib.ptr(stage_v), stage_k.shape[0], _lib.ptr(dev_k),
            _lib.ptr(dev_v), dev_k.shape[0], row_bytes, ctypes.c_void_p(stream.cuda_stream), ctypes.byref(flag),
            ctypes.byref(total), ctypes.byref(n_ev), ctypes.byref(n_rg), ctypes.byref(started)),
            "h2d plan_start_direct")
        return int(flag.value), int(total.value), int(n_ev.value), int(n_rg.value), bool(started.value)

    def reserve(self, n_ranges: int, stream: torch.cuda.Stream, groups: int = 8) -> None:
        """Pays the engine's set-up costs now (``wnw_h2d_reserve``): the
        direct form's copy streams on the current device, descriptor room for
        ``n_ranges`` ranges per job, the DMA engines a job's copies land on
        (a job's copy pattern replayed on scratch buffers), the events of the
        first ``groups`` groups, and an empty job through the engine's thread
        on ``stream``.  Blocks until done."""
        _lib.check(_lib.lib().wnw_h2d_reserve(self._h, int(n_ranges), int(groups),
                                              ctypes.c_void_p(stream.cuda_stream)), "h2d reserve")

    def wait(self, group: int, stream: torch.cuda.Stream | None = None) -> None:
        """``stream`` (default: the current one) waits for group ``group``'s
        copy; the host blocks only until that copy is issued."""
        s = stream if stream is not None else torch.cuda.current_stream()
        _lib.check(_lib.lib().wnw_h2d_wait(self._h, int(group), ctypes.c_void_p(s.cuda_stream)), "h2d wait")

    def join(self) -> None:
        """Blocks until every group of the last start is issued."""
        _lib.check(_lib.lib().wnw_h2d_join(self._h), "h2d join")

    def close(self) -> None:
        if self._h:
            _lib.lib().wnw_h2d_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

"""Host planner of the C++ WnW cache variant.

``Planner`` keeps the method names, argument meaning and results of the
reference's pybind module (src/algorithms/wnw_cpp/code/planner.cpp:327-341,
loaded by src/algorithms/wnw_cpp/code/_ext.py:21-46); every method calls the
native planner in ``libwnw_amd.so`` (``wnw_planner_*`` in
``include/wnw_amd.h``).  Index arrays are CPU int32 tensors, as in the
reference.  Unlike the reference, bad indices raise ``WnwError`` instead of
reading out of bounds.
"""
from __future__ import annotations

import ctypes

import torch

from .. import _lib


def _i32(x) -> torch.Tensor:
    t = x if isinstance(x, torch.Tensor) else torch.tensor(list(x), dtype=torch.int32)
    if t.dtype != torch.int32 or t.device.type != "cpu":
        raise _lib.WnwError("planner arrays must be CPU int32 tensors")
    return t.contiguous()


def _p(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr()) if t.numel() else None


class Planner:
    """Planner(num_layers, num_kv_heads, batch_size, group) (planner.cpp:18-25)."""

    def __init__(self, num_layers: int, num_kv_heads: int, batch_size: int, group: int):
        self._lib = _lib.lib()
        h = self._lib.wnw_planner_create(num_layers, num_kv_heads, batch_size, group)
        if not h:
            raise _lib.WnwError(self._lib.wnw_last_error().decode())
        self._h = ctypes.c_void_p(h)
        self.L, self.H, self.B = num_layers, num_kv_heads, batch_size
        self.N = batch_size * num_kv_heads
        self._buffers = None  # restore / staging tensors kept alive

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.wnw_planner_destroy(h)
            self._h = None

    def _check(self, rc: int, what: str) -> None:
        _lib.check(rc, f"planner.{what}")

    def set_config(self, top_k_chunks: int, eviction_lag: int) -> None:
        self._check(self._lib.wnw_planner_set_config(self._h, top_k_chunks, eviction_lag), "set_config")

    def set_seg_count(self, seg_count) -> None:
        t = _i32(seg_count)
        self._check(self._lib.wnw_planner_set_seg_count(self._h, _p(t), t.numel()), "set_seg_count")

    def set_chunk_to_segs(self, b: int, flat_segs, offsets) -> None:
        f, o = _i32(flat_segs), _i32(offsets)
        self._check(self._lib.wnw_planner_set_chunk_to_segs(self._h, b, _p(f), _p(o), o.numel() - 1),
                    "set_chunk_to_segs")

    def set_class_b(self, layer: int, kv_heads) -> None:
        t = _i32(kv_heads)
        self._check(self._lib.wnw_planner_set_class_b(self._h, layer, _p(t), t.numel()), "set_class_b")

    def set_restore_meta(self, cpu_s, cpu_e, gpu_s, gpu_e) -> None:
        a, b, c, d = (_i32(x) for x in (cpu_s, cpu_e, gpu_s, gpu_e))
        if not a.numel() == b.numel() == c.numel() == d.numel():
            raise _lib.WnwError("restore meta arrays differ in length")
        self._check(self._lib.wnw_planner_set_restore_meta(self._h, _p(a), _p(b), _p(c), _p(d), a.numel()),
                    "set_restore_meta")

    def set_loaded(self, b: int, segs) -> None:
        t = _i32(segs)
        self._check(self._lib.wnw_planner_set_loaded(self._h, b, _p(t), t.numel()), "set_loaded")

    def set_seq_lens(self, seq_lens_flat) -> None:
        t = _i32(seq_lens_flat)
        self._check(self._lib.wnw_planner_set_seq_lens(self._h, _p(t), t.numel()), "set_seq_lens")

    def get_loaded_segments(self, b: int) -> list[int]:
        n = self._lib.wnw_planner_get_loaded_segments(self._h, b, None, 0)
        if n < 0:
            raise _lib.WnwError(self._lib.wnw_last_error().decode())
        out = torch.empty(n, dtype=torch.int32)
        self._lib.wnw_planner_get_loaded_segments(self._h, b, _p(out), n)
        return out.tolist()

    def set_restore_buffers(self, cpu_k: torch.Tensor, cpu_v: torch.Tensor, stg_k: torch.Tensor,
                            stg_v: torch.Tensor) -> None:
        for t in (cpu_k, cpu_v, stg_k, stg_v):
            if t.device.type != "cpu" or not t.is_contiguous() or t.dim() != 2:
                raise _lib.WnwError("restore and staging buffers must be contiguous 2-D host tensors")
        if cpu_k.shape != cpu_v.shape or stg_k.shape != stg_v.shape or cpu_k.shape[1] != stg_k.shape[1] \
                or cpu_k.dtype != stg_k.dtype:
            raise _lib.WnwError("restore / staging shapes or dtypes differ")
        row_bytes = cpu_k.shape[1] * cpu_k.element_size()
        self._buffers = (cpu_k, cpu_v, stg_k, stg_v)
        self._check(self._lib.wnw_planner_set_restore_buffers(
            self._h, _p(cpu_k), _p(cpu_v), _p(stg_k), _p(stg_v), cpu_k.shape[0], stg_k.shape[0], row_bytes),
            "set_restore_buffers")

    def gather_restore(self) -> None:
        self._check(self._lib.wnw_planner_gather_restore(self._h), "gather_restore")

    def compute_and_prepare(self, topk_idx, topk_off, load_starts_2d: torch.Tensor, load_lens_2d: torch.Tensor,
                            cu_new_2d: torch.Tensor, new_lens_2d: torch.Tensor, evict_offsets_2d: torch.Tensor,
                            evict_max: torch.Tensor, evict_layer_ptr: torch.Tensor, check: bool = True):
        """Returns ``(any_change, total, ev_s, ev_e, ranges)`` like the
        reference (planner.cpp:124-306): ints, int32 [E], int32 [E],
        int32 [nr, 2]; the 2-D outputs are written in place.
        ``check=False`` skips the Python checks of the output tensors, for a
        caller that made them once with the right shapes (the library still
        checks every index it reads)."""
        L, N = self.L, self.N
        if check:
            shapes = ((load_starts_2d, (L, N)), (load_lens_2d, (L, N)), (cu_new_2d, (L, N + 1)),
                      (new_lens_2d, (L, N)), (evict_offsets_2d, (L, N + 1)), (evict_max, (L,)),
                      (evict_layer_ptr, (L + 1,)))
            for t, shape in shapes:
                if t.dtype != torch.int32 or t.device.type != "cpu" or not t.is_contiguous() or \
                        tuple(t.shape) != shape:
                    raise _lib.WnwError(f"planner output must be a contiguous CPU int32 tensor of shape {shape}")
        tk, to = _i32(topk_idx), _i32(topk_off)
        if to.numel() != self.B + 1:
            raise _lib.WnwError("topk_off must have batch + 1 entries")
        flag = ctypes.c_int32(0)
        total, n_ev, n_rg = ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_int64(0)
        self._check(self._lib.wnw_planner_compute_and_prepare(
            self._h, _p(tk), _p(to), _p(load_starts_2d), _p(load_lens_2d), _p(cu_new_2d), _p(new_lens_2d),
            _p(evict_offsets_2d), _p(evict_max), _p(evict_layer_ptr), ctypes.byref(flag), ctypes.byref(total),
            ctypes.byref(n_ev), ctypes.byref(n_rg)), "compute_and_prepare")
        ev_s, ev_e, ranges = self.plan_lists(n_ev.value, n_rg.value)
        return int(flag.value), int(total.value), ev_s, ev_e, ranges

    def plan_lists(self, n_evict: int, n_ranges: int):
        """The last plan's evict lists and host ranges (``ev_s``, ``ev_e``,
        ``ranges`` of compute_and_prepare's result), ``n_evict`` and
        ``n_ranges`` long."""
        ev_s = torch.empty(n_evict, dtype=torch.int32)
        ev_e = torch.empty(n_evict, dtype=torch.int32)
        ranges = torch.empty(n_ranges, 2, dtype=torch.int32)
        self._check(self._lib.wnw_planner_get_evictions(self._h, _p(ev_s), _p(ev_e), n_evict), "get_evictions")
        self._check(self._lib.wnw_planner_get_ranges(self._h, _p(ranges), n_ranges), "get_ranges")
        return ev_s, ev_e, ranges

    def range_layers(self) -> list[int]:
        """The last plan's layer pointer into its ``ranges`` (L + 1 entries;
        layer l's ranges are rows [ptr[l], ptr[l + 1]) of ``ranges``)."""
        out = (ctypes.c_int32 * (self.L + 1))()
        self._check(self._lib.wnw_planner_get_range_layers(self._h, out, self.L + 1), "get_range_layers")
        return list(out)

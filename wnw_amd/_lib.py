"""Loader of ``libwnw_amd.so``, the C ABI of the gfx950 kernels.

The library is built in-tree by ``__graft_entry__.build()`` (or
``make -C wnw_amd/csrc``).  Everything here fails loudly: there is no CPU or
PyTorch fallback for any operator of this package.
"""
from __future__ import annotations

import ctypes
import os

import torch  # loads torch's HIP runtime first; the library binds to it

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libwnw_amd.so")

WNW_OK, WNW_EINVAL, WNW_EHIP, WNW_ENOTSUP = 0, 1, 2, 3
DT_F32, DT_F16, DT_BF16 = 0, 1, 2
ATTN_AUTO, ATTN_MFMA, ATTN_VALU, ATTN_STREAM = 0, 1, 2, 3
DEVERR_BOUNDS, DEVERR_ORDER, DEVERR_CAPACITY = 1, 2, 4
NOALLOC_SCRATCH_BYTES, NOALLOC_MAX_SEG = 16 << 20, 4096
TOPK_MAX_CHUNKS, TOPK_MAX_K = 8192, 64  # wnw_chunk_topk: chunks of one sample, k

_TORCH_DTYPES = {torch.float32: DT_F32, torch.float16: DT_F16, torch.bfloat16: DT_BF16}

_lib: ctypes.CDLL | None = None

_vp, _i64, _i32, _f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float

# name -> (restype, argtypes); mirrors include/wnw_amd.h
_SIGNATURES = {
    "wnw_last_error": (ctypes.c_char_p, []),
    "wnw_abi_version": (_i32, []),
    "wnw_init": (_i32, []),
    "wnw_prepare_kernels": (_i32, []),
    "wnw_device_error": (_i32, [_i32]),
    "wnw_interleave_append": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp, _vp]),
    "wnw_interleave_append_kv": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp, _vp, _vp]),
    "wnw_append_inplace": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp]),
    "wnw_rebuild_append_kv": (_i32, [_vp] * 13 + [_i64] * 7 + [_i32, _vp, _vp, _vp]),
    "wnw_compact_segments": (_i32, [_vp] * 9 + [_i64, _i64, _i64] + [_vp] * 9 + [_i64, _i32, _i64, _i64, _i64,
                                                                           _i64, _i32, _vp]),
    "wnw_decode_attn_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "wnw_workspace_init": (_i32, [_vp, _i64, _vp]),
    "wnw_decode_attn": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _vp, _vp,
                               _i64, _vp]),
    "wnw_decode_attn_ex": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _vp, _vp,
                                  _i64, _i32, _i64, _vp]),
    "wnw_decode_attn_append": (_i32, [_vp] * 9 + [_i64] * 5 + [_f32, _i32, _vp, _vp, _i64, _vp]),
    "wnw_decode_attn_score_append": (_i32, [_vp] * 9 + [_i64] * 5 + [_f32, _i32, _vp, _vp, _i64, _vp, _vp, _vp,
                                                                 _vp, _i64, _i64, _vp, _i64, _vp]),
    "wnw_decode_attn_noalloc": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _vp,
                                       _vp]),
    "wnw_decode_attn_score_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "wnw_decode_attn_score": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _vp,
                                     _vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _vp]),
    "wnw_fused_score_workspace_bytes": (_i64, [_i64, _i64]),
    "wnw_fused_score_accumulate": (_i32, [_vp] * 8 + [_i64] * 6 + [_f32, _i32, _vp, _i64, _vp]),
    "wnw_chunk_topk": (_i32, [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _vp, _vp]),
    "wnw_score_slot_bytes": (_i64, [_i64, _i64, _i64]),
    "wnw_decode_attn_append_deferred": (_i32, [_vp] * 9 + [_i64] * 5 + [_f32, _i32, _vp, _i64, _vp, _vp, _i64, _vp,
                                                                      _vp, _i64, _vp, _vp, ctypes.c_uint64]
                                        + [_vp] * 3 + [_i64, _vp, _i64, _vp]),
    "wnw_score_kept_logits": (_i32, [_vp, _vp, _vp, _vp] + [_i64] * 4 + [_vp, _vp, _i64, _vp, _vp, _i64, _vp]),
    "wnw_read_stream": (_i32, [_vp, _i64, _i64, _i32, _vp, _vp]),
    # host planner (CPU only)
    "wnw_planner_create": (_vp, [_i32, _i32, _i32, _i32]),
    "wnw_planner_destroy": (None, [_vp]),
    "wnw_planner_set_config": (_i32, [_vp, _i32, _i32]),
    "wnw_planner_set_seg_count": (_i32, [_vp, _vp, _i64]),
    "wnw_planner_set_chunk_to_segs": (_i32, [_vp, _i32, _vp, _vp, _i64]),
    "wnw_planner_set_class_b": (_i32, [_vp, _i32, _vp, _i64]),
    "wnw_planner_set_restore_meta": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64]),
    "wnw_planner_set_loaded": (_i32, [_vp, _i32, _vp, _i64]),
    "wnw_planner_set_seq_lens": (_i32, [_vp, _vp, _i64]),
    "wnw_planner_get_loaded_segments": (_i64, [_vp, _i32, _vp, _i64]),
    "wnw_planner_set_restore_buffers": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64]),
    "wnw_planner_gather_restore": (_i32, [_vp]),
    "wnw_host_rows_readable": (_i32, [_vp, _vp]),
    "wnw_gather_host_rows": (_i32, [_vp, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp]),
    "wnw_planner_compute_and_prepare": (_i32, [_vp] * 14),
    "wnw_planner_get_evictions": (_i32, [_vp, _vp, _vp, _i64]),
    "wnw_planner_get_ranges": (_i32, [_vp, _vp, _i64]),
    "wnw_planner_get_range_layers": (_i32, [_vp, _vp, _i64]),
    "wnw_h2d_create": (_vp, [_i32]),
    "wnw_h2d_destroy": (None, [_vp]),
    "wnw_h2d_start": (_i32, [_vp, _vp, _vp, _i64, _vp, _i64, _vp, _i32, _vp, _vp, _i64, _vp, _vp, _i64, _i64, _vp]),
    "wnw_h2d_start_direct": (_i32, [_vp, _vp, _vp, _i64, _vp, _i64, _vp, _i32, _vp, _vp, _i64, _vp, _vp, _i64, _i64,
                                    _vp]),
    "wnw_h2d_plan_start_direct": (_i32, [_vp, _vp, _vp, _i64, _i64] + [_vp] * 8 + [_i32, _vp, _vp, _i64, _vp, _vp,
                                                                            _i64, _vp, _vp, _i64, _i64, _vp]
                                  + [_vp] * 5),
    "wnw_h2d_wait": (_i32, [_vp, _i32, _vp]),
    "wnw_h2d_join": (_i32, [_vp]),
    "wnw_h2d_reserve": (_i32, [_vp, _i64, _i32, _vp]),
}


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP extension first "
                "(python -c 'import __graft_entry__ as g; g.build()')")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


class WnwError(RuntimeError):
    pass


def check(rc: int, what: str = "") -> None:
    if rc != WNW_OK:
        msg = lib().wnw_last_error().decode(errors="replace")
        raise WnwError(f"{what}: status {rc}: {msg}")


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _TORCH_DTYPES[dt]
    except KeyError:
        raise WnwError(f"unsupported dtype {dt}") from None


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def raw_stream(device: torch.device) -> int:
    """The current HIP stream of ``device`` as an integer handle, without
    building a torch Stream object where torch offers that."""
    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return int(_raw_stream(idx))
    return int(torch.cuda.current_stream(device).cuda_stream)


def stream_of(device: torch.device) -> ctypes.c_void_p:
    """The current HIP stream of ``device`` (the raw handle)."""
    return ctypes.c_void_p(raw_stream(device))


def require_gpu(*tensors: torch.Tensor) -> None:
    """Raise unless every tensor lives on a HIP device (no CPU fallback)."""
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise WnwError(f"wnw_amd kernels need GPU tensors, got a tensor on {t.device}")


def device_error(clear: bool = True) -> int:
    """WNW_DEVERR_* bits recorded by kernels on the current device (syncs)."""
    v = lib().wnw_device_error(1 if clear else 0)
    if v < 0:
        raise WnwError("wnw_device_error failed")
    return v


_init_done: set[int] = set()


def ensure_init(device: torch.device) -> None:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx in _init_done:
        return
    with torch.cuda.device(idx):
        check(lib().wnw_init(), "wnw_init")
    _init_done.add(idx)

"""wnw_amd -- MI355X-native decode-step attention path of WnW.

The package mirrors the reference's operator and cache interfaces for that
path and runs every operator as a hand-written gfx950 HIP kernel behind the C
ABI declared in ``include/wnw_amd.h`` (``libwnw_amd.so``):

* ``wnw_amd.kv.kernels.interleave_append``          (src/common/kv/kernels.py)
* ``wnw_amd.kv.fused_attn.q1_decode_attn``          (src/common/kv/fused_attn.py)
* ``wnw_amd.wnw.kernels.rebuild_append_kv``         (src/algorithms/wnw/code/kernels.py)
* ``wnw_amd.kv.flat_cache.FlatVarlenCache``         (src/common/kv/flat_cache.py)
* ``wnw_amd.wnw.cache.WnWCache``                    (src/algorithms/wnw/code/cache.py)
"""

__all__ = ["kv", "wnw"]

"""Synthetic workloads of the benchmark configurations.

Each configuration is a list of per-layer segment layouts: segment
s = b * Hkv + h of layer l has a length and a class (A keeps its full KV,
B a compressed set).  Only lengths and classes matter to the decode path;
the K/V values are drawn from N(0, 1) times a per-(layer, KV head) scale.

Choices the configuration text leaves open are fixed here and recorded in
``Config.notes`` (printed by bench.py):
* class-A count per layer = round(fraction * Hkv), at least 1 when the
  fraction is positive, heads drawn uniformly without replacement;
* all seeds derive from ``seed`` (default 0) through numpy's PCG64;
* config 5 uses sigma = 1 for the lognormal lengths;
* config 4 (``wnw_amd/offload_bench.py``) selects chunks per sample, one
  choice shared by every class-B head and layer, as the reference's planner
  does (src/algorithms/wnw/code/cache.py:609-630).
"""
from __future__ import annotations

import dataclasses

import numpy as np


@dataclasses.dataclass
class Config:
    name: str
    layers: int
    batch: int
    hq: int
    hkv: int
    head_dim: int
    dtype: str
    steps: int
    # lengths[l] : int64 [batch * hkv] rows per segment BEFORE the step's append
    lengths: list[np.ndarray]
    # class_a[l] : bool [hkv]
    class_a: list[np.ndarray]
    # kv_scale[l] : float32 [hkv]
    kv_scale: list[np.ndarray]
    notes: list[str]
    # audio tokens per sequence (the scored rows of its class-A segments)
    audio: np.ndarray | None = None

    @property
    def group(self) -> int:
        return self.hq // self.hkv

    @property
    def n_seg(self) -> int:
        return self.batch * self.hkv

    def rows_after_append(self, layer: int) -> int:
        return int(self.lengths[layer].sum()) + self.n_seg

    def attn_bytes(self, layer: int, elem: int = 2) -> int:
        """Algorithmic HBM bytes of one layer-step of decode attention.

        K and V of every row once, plus q in and o out:
        sum_s len_s * D * 2 * elem + 2 * B * Hq * D * elem.
        """
        d = self.head_dim
        return self.rows_after_append(layer) * d * 2 * elem + 2 * self.batch * self.hq * d * elem


def _class_a_heads(rng, hkv: int, frac: float) -> np.ndarray:
    n = int(round(frac * hkv))
    if frac > 0:
        n = max(1, n)
    mask = np.zeros(hkv, dtype=bool)
    mask[rng.choice(hkv, size=n, replace=False)] = True
    return mask


def config1(seed: int = 0) -> Config:
    """CPU plumbing: one layer of Voxtral-Mini shape, fp32, batch 2.

    KV heads 0-1 class A with 1024 cached tokens; heads 2-7 class B with
    4 sink + 124 recent tokens.
    """
    hkv, b = 8, 2
    lens = np.array([1024 if h < 2 else 128 for _ in range(b) for h in range(hkv)], dtype=np.int64)
    ca = np.array([h < 2 for h in range(hkv)])
    return Config("cfg1-voxtral-cpu-plumbing", 1, b, 32, hkv, 128, "float32", 1, [lens], [ca],
                  [np.ones(hkv, np.float32)], ["q, K, V ~ N(0,1), seed 0"], np.full(b, 1024 - 64))


def config2(seed: int = 0, layers: int = 30) -> Config:
    """Voxtral-Mini-3B decode: 30 layers, 32/8 heads, d128, bf16, batch 8.

    7,500 audio + 64 text tokens per sequence; per layer round(0.3 * 8) = 2
    class-A KV heads (full 7,564 rows); class B keeps 4 sink + 508 recent.
    """
    rng = np.random.default_rng(seed)
    hkv, b = 8, 8
    full = 7500 + 64
    lengths, cas, scales = [], [], []
    for _ in range(layers):
        ca = _class_a_heads(rng, hkv, 0.3)
        lengths.append(np.array([full if ca[h] else 512 for _ in range(b) for h in range(hkv)], dtype=np.int64))
        cas.append(ca)
        scales.append(rng.uniform(0.5, 2.0, size=hkv).astype(np.float32))
    return Config("cfg2-voxtral-7500tok-b8", layers, b, 32, hkv, 128, "bfloat16", 128, lengths, cas, scales,
                  ["class-A count round(0.3*8)=2 per layer, heads uniform", f"seed {seed}",
                   "class-B segments hold 512 rows at the start and grow by the step's row"], np.full(b, 7500))


def config3(seed: int = 0, layers: int = 28) -> Config:
    """Qwen2.5-Omni-7B thinker: 28 layers, 28/4 heads (G=7), d128, bf16, batch 16."""
    rng = np.random.default_rng(seed + 3)
    hkv, b = 4, 16
    audio = rng.integers(2000, 16000, size=b, endpoint=True)
    lengths, cas, scales = [], [], []
    for _ in range(layers):
        ca = _class_a_heads(rng, hkv, float(rng.uniform(0.25, 0.5)))
        lengths.append(np.array([audio[bi] + 32 if ca[h] else 1024 for bi in range(b) for h in range(hkv)],
                                dtype=np.int64))
        cas.append(ca)
        scales.append(rng.uniform(0.5, 2.0, size=hkv).astype(np.float32))
    return Config("cfg3-qwen-omni-b16", layers, b, 28, hkv, 128, "bfloat16", 64, lengths, cas, scales,
                  ["class-A count round(U[0.25,0.5]*4) >= 1", f"seed {seed}"], audio.astype(np.int64))


def config5(seed: int = 0, layers: int = 30) -> Config:
    """Heavily ragged batch at Voxtral shape: batch 64, lognormal lengths."""
    rng = np.random.default_rng(seed + 5)
    hkv, b = 8, 64
    seq = np.clip(np.round(rng.lognormal(mean=np.log(3000.0), sigma=1.0, size=b)), 256, 32768).astype(np.int64)
    lengths, cas, scales = [], [], []
    for _ in range(layers):
        ca = _class_a_heads(rng, hkv, float(rng.uniform(0.1, 0.6)))
        win = rng.choice([256, 512, 1024], size=(b, hkv))
        lens = np.array([seq[bi] if ca[h] else min(seq[bi], 4 + int(win[bi, h]))
                         for bi in range(b) for h in range(hkv)], dtype=np.int64)
        lengths.append(lens)
        cas.append(ca)
        scales.append(rng.uniform(0.5, 2.0, size=hkv).astype(np.float32))
    return Config("cfg5-ragged-b64", layers, b, 32, hkv, 128, "bfloat16", 32, lengths, cas, scales,
                  ["lognormal sigma=1, median 3000, clip [256, 32768]", "class-A count round(U[0.1,0.6]*8) >= 1",
                   f"seed {seed}"], seq.astype(np.int64))


CONFIGS = {"cfg1": config1, "cfg2": config2, "cfg3": config3, "cfg5": config5}

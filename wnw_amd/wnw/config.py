"""WnW configuration: chunk geometry and head classes.

Same fields, JSON layout and lookups as the reference's ``WnWConfig``
(src/algorithms/wnw/code/config.py:7-121):
* chunks of ``chunk_size_s`` seconds overlapping by ``overlap_s`` at
  ``token_rate`` tokens/s; segments are the stride tiles
  (stride = chunk - overlap tokens), and a chunk must be a whole number of
  strides;
* head classes by global id: class A lists query heads
  (``layer * num_q_heads + q``), class B and the retention ratios list KV
  heads (``layer * num_kv_heads + kv``); a KV head is class A when any of
  its query heads is (config.py:52-59).
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field


class WnWConfigError(ValueError, AssertionError):
    """Invalid configuration (the reference asserts, so AssertionError too)."""


@dataclass
class WnWConfig:
    chunk_size_s: float
    overlap_s: float
    token_rate: float

    class_a: list[int]
    class_b: list[int]
    retention_ratios: list[float | None]

    top_k_chunks: int
    eviction_lag: int

    prefill_score_mode: str

    prefill_global_topk: bool = False

    num_layers: int = 0
    num_kv_heads: int = 0
    num_q_heads: int = 0

    _class_a_set: set[int] = field(default_factory=set, repr=False)
    _class_b_set: set[int] = field(default_factory=set, repr=False)
    _class_a_kv_set: set[int] = field(default_factory=set, repr=False)

    def __post_init__(self):
        self._class_a_set = set(self.class_a)
        self._class_b_set = set(self.class_b)
        if self.stride_tokens <= 0:
            raise WnWConfigError(f"stride must be positive: chunk_size_tokens={self.chunk_size_tokens} "
                             f"<= overlap_tokens={self.overlap_tokens}")
        if self.chunk_size_tokens % self.stride_tokens:
            raise WnWConfigError(f"chunk_size_tokens ({self.chunk_size_tokens}) must be a multiple of "
                             f"stride_tokens ({self.stride_tokens})")
        if self.prefill_score_mode not in ("last", "mean_text"):
            raise WnWConfigError(f"unknown prefill_score_mode {self.prefill_score_mode!r}")
        if self.num_q_heads > 0 and self.num_kv_heads > 0:
            self._rebuild_class_a_kv_set()

    def set_model_dims(self, num_layers: int, num_kv_heads: int, num_q_heads: int) -> None:
        self.num_layers, self.num_kv_heads, self.num_q_heads = num_layers, num_kv_heads, num_q_heads
        self._rebuild_class_a_kv_set()

    def _rebuild_class_a_kv_set(self) -> None:
        group = self.num_q_heads // self.num_kv_heads
        self._class_a_kv_set = {
            (gid // self.num_q_heads) * self.num_kv_heads + (gid % self.num_q_heads) // group
            for gid in self.class_a
        }

    # chunk geometry (config.py:61-71): int() truncation as in the reference
    @property
    def chunk_size_tokens(self) -> int:
        return int(self.chunk_size_s * self.token_rate)

    @property
    def overlap_tokens(self) -> int:
        return int(self.overlap_s * self.token_rate)

    @property
    def stride_tokens(self) -> int:
        return self.chunk_size_tokens - self.overlap_tokens

    # per-layer lookups (config.py:73-92)
    def get_layer_class_a(self, layer_idx: int) -> list[int]:
        lo = layer_idx * self.num_q_heads
        return [gid - lo for gid in self.class_a if lo <= gid < lo + self.num_q_heads]

    def get_layer_class_b(self, layer_idx: int) -> list[int]:
        lo = layer_idx * self.num_kv_heads
        return [gid - lo for gid in self.class_b if lo <= gid < lo + self.num_kv_heads]

    def get_retention(self, layer_idx: int, local_kv_head: int) -> float | None:
        return self.retention_ratios[layer_idx * self.num_kv_heads + local_kv_head]

    def is_class_a(self, layer_idx: int, q_head: int) -> bool:
        return layer_idx * self.num_q_heads + q_head in self._class_a_set

    def is_class_a_kv_head(self, layer_idx: int, kv_head: int) -> bool:
        return layer_idx * self.num_kv_heads + kv_head in self._class_a_kv_set

    def is_class_b(self, layer_idx: int, kv_head: int) -> bool:
        return layer_idx * self.num_kv_heads + kv_head in self._class_b_set

    @classmethod
    def from_json(cls, path: str, num_layers: int = 0, num_kv_heads: int = 0, num_q_heads: int = 0) -> "WnWConfig":
        """config.py:94-121: {"chunk": {size_s, overlap_s, token_rate},
        "heads": {class_a, class_b, retention_ratios}, "selection":
        {top_k_chunks, eviction_lag}, "score": {prefill_mode,
        prefill_global_topk}}."""
        with open(path) as f:
            raw = json.load(f)
        chunk, heads, sel = raw["chunk"], raw["heads"], raw["selection"]
        score = raw.get("score", {})
        return cls(
            chunk_size_s=chunk["size_s"], overlap_s=chunk["overlap_s"], token_rate=chunk["token_rate"],
            class_a=heads["class_a"], class_b=heads["class_b"], retention_ratios=heads["retention_ratios"],
            top_k_chunks=sel["top_k_chunks"], eviction_lag=sel["eviction_lag"],
            prefill_score_mode=score.get("prefill_mode", "mean_text"),
            prefill_global_topk=score.get("prefill_global_topk", False),
            num_layers=num_layers, num_kv_heads=num_kv_heads, num_q_heads=num_q_heads,
        )

"""Flat varlen KV cache contract (HF ``Cache`` subclass).

Same layout, HF methods and hook API as the reference's
``FlatVarlenCache`` (src/common/kv/flat_cache.py:12-186):
* per layer ``layer_k[i]`` / ``layer_v[i]``: [total_rows, head_dim],
  segment s = b * num_kv_heads + h, offsets ``cu_seqlens`` int32 [N + 1];
* HF sees per-layer lengths through ``_SeqLengthStub`` layers
  (``get_seq_length`` / ``get_mask_sizes``, flat_cache.py:12-44, :127-137);
  ``update`` only counts tokens (the patched attention does the storage);
* hooks for the algorithm: ``prefill_before_attn``, ``prefill_after_attn``,
  ``prefill_all_layers_done``, ``decode_before_attn`` (returns
  ``(K_flat, V_flat, cu_seqlens_k, max_seqlen_k)``), ``decode_after_attn``,
  ``decode_all_layers_done`` (flat_cache.py:161-186);
* beam search, assisted-decoding crop and batch reshuffles raise.
"""
from __future__ import annotations

import torch
from torch import Tensor
from transformers.cache_utils import Cache, CacheLayerMixin

from .stats import InferenceStats


class _SeqLengthStub(CacheLayerMixin):
    """Per-layer stand-in HF queries for lengths; storage lives in the cache."""

    is_compileable = False
    is_sliding = False

    def __init__(self, get_len_fn):
        super().__init__()
        self._get_len = get_len_fn
        self.is_initialized = True

    def lazy_initialization(self, *args, **kwargs):
        pass

    def update(self, key_states, value_states, *args, **kwargs):
        raise RuntimeError("FlatVarlenCache: layers[].update should never be called directly")

    def get_seq_length(self) -> int:
        return self._get_len()

    def get_max_cache_shape(self) -> int:
        return -1

    def get_max_length(self) -> int:
        return -1  # grows without bound (newer transformers require it)

    def get_mask_sizes(self, query_length: int):
        n = self._get_len()
        return n + query_length, n

    def reset(self):
        pass

    def reorder_cache(self, beam_idx):
        raise NotImplementedError("Beam search not supported")


class FlatVarlenCache(Cache):
    """Flat K/V rows + cu_seqlens per layer, for varlen decode attention."""

    is_compileable = False

    # HF's Cache derives batch_size from its layers (read-only in newer
    # transformers); this cache owns it, as the reference's subclass expects.
    @property
    def batch_size(self) -> int:
        return getattr(self, "_flat_batch_size", 0)

    @batch_size.setter
    def batch_size(self, value: int) -> None:
        self._flat_batch_size = value

    def __init__(self, num_layers: int, num_kv_heads: int, num_q_heads: int, head_dim: int,
                 device: torch.device, adapter=None):
        stubs = [_SeqLengthStub(lambda i=i: self._seq_lengths[i] if i < len(self._seq_lengths) else 0)
                 for i in range(num_layers)]
        super().__init__(layers=stubs)
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.num_q_heads = num_q_heads
        self.num_kv_groups = num_q_heads // num_kv_heads
        self.head_dim = head_dim
        self.device = device
        self.adapter = adapter
        self._seq_lengths: list[int] = [0] * num_layers
        self.prefilled = False
        self.audio_starts: Tensor | None = None
        self.audio_ends: Tensor | None = None
        self.pad_lens: Tensor | None = None
        self.stats = InferenceStats(device, interval=5)

    def setup_audio(self, audio_starts: Tensor, audio_ends: Tensor, attention_mask: Tensor | None) -> None:
        """flat_cache.py:85-106: per-sample audio ranges and left-padding."""
        self.audio_starts = audio_starts
        self.audio_ends = audio_ends
        self.prefilled = False
        self._seq_lengths = [0] * self.num_layers
        self.stats.reset(audio_starts.shape[0])
        B = audio_starts.shape[0]
        if attention_mask is not None:
            pads = []
            for b in range(attention_mask.shape[0]):
                nz = (attention_mask[b] == 1).nonzero(as_tuple=True)[0]
                pads.append(int(nz[0].item()) if len(nz) > 0 else 0)
            self.pad_lens = torch.tensor(pads, dtype=torch.int64, device=self.device)
        else:
            self.pad_lens = torch.zeros(B, dtype=torch.int64, device=self.device)

    def update(self, key_states: Tensor, value_states: Tensor, layer_idx: int, *args, **kwargs):
        """flat_cache.py:108-121: counts tokens only."""
        self._seq_lengths[layer_idx] += key_states.shape[-2]
        return key_states, value_states

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self._seq_lengths[layer_idx] if layer_idx < self.num_layers else 0

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        return -1

    def get_mask_sizes(self, query_length: int, layer_idx: int) -> tuple[int, int]:
        n = self.get_seq_length(layer_idx)
        return n + query_length, n

    def reset(self):
        self.prefilled = False
        self._seq_lengths = [0] * self.num_layers
        self.audio_starts = self.audio_ends = self.pad_lens = None
        self.stats.reset(0)

    def reorder_cache(self, beam_idx):
        raise NotImplementedError("FlatVarlenCache does not support beam search")

    def crop(self, max_length: int):
        raise NotImplementedError("FlatVarlenCache does not support assisted decoding crop")

    def batch_repeat_interleave(self, repeats: int):
        raise NotImplementedError("FlatVarlenCache does not support batch_repeat_interleave")

    def batch_select_indices(self, indices):
        raise NotImplementedError("FlatVarlenCache does not support batch_select_indices")

    # -- hooks (flat_cache.py:161-186) --------------------------------------
    def prefill_before_attn(self, layer_idx: int) -> None:
        """Before attention during prefill (subclass sets up storage)."""

    def prefill_after_attn(self, layer_idx: int, scores: Tensor, k: Tensor, v: Tensor) -> None:
        """After attention during prefill (subclass compresses)."""

    def prefill_all_layers_done(self) -> None:
        self.prefilled = True

    def decode_before_attn(self, layer_idx: int, k_new: Tensor, v_new: Tensor) -> tuple[Tensor, Tensor, Tensor, int]:
        """Returns (K_flat, V_flat, cu_seqlens_k, max_seqlen_k)."""
        raise NotImplementedError("Subclass must implement decode_before_attn")

    def decode_after_attn(self, layer_idx: int, q: Tensor) -> None:
        """After attention during decode (subclass collects scores)."""

    def decode_all_layers_done(self) -> None:
        """After the last layer of a decode step (subclass plans)."""

    def _snapshot_cache_stats(self, step: int = -1) -> list[dict]:
        raise NotImplementedError("Subclass must implement _snapshot_cache_stats")

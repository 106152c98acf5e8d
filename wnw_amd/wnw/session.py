"""Attention patch that drives the WnW cache (the caller of the decode path).

Mirrors ``WnWSession`` (src/algorithms/wnw/code/session.py:20-116) and the
context manager of ``AlgorithmSession`` (src/common/session.py:15-92):
inside the ``with`` block every decoder layer's attention forward is
replaced by one that
* prefill: runs causal attention, computes the prefill token scores and
  hands K/V to ``cache.prefill_after_attn`` (session.py:53-76);
* decode: appends and attends through the cache (``decode_attention``: one
  fused launch for the WnW cache, else ``cache.decode_before_attn`` and the
  gfx950 decode attention) and feeds the cache's scoring and planning hooks
  (session.py:78-116).
The model-specific parts (q/k/v projections, RoPE, o_proj, locating the
audio tokens, generate) come from the caller's adapter, exactly the methods
the reference's adapters provide (``compute_qkv``, ``apply_rope``,
``attention_meta``, ``get_decoder_layers``, ``locate_audio_tokens``,
``generate``, ``prepare_for_inference``, ``restore_after_inference``,
``assert_compatible``).
"""
from __future__ import annotations

import os
import types

import torch
import torch.nn.functional as F
from torch import Tensor

from ..kv.flat_cache import FlatVarlenCache
from ..kv.fused_attn import q1_decode_attn


def fused_attn_enabled() -> bool:
    """The reference's switch between its fused kernel and varlen_attn
    (session.py:17); here both paths run the gfx950 kernel, the switch only
    selects whether scoring is folded into the attention operator."""
    return os.environ.get("WNW_FUSED_ATTN", "0") == "1"


def decode_attention(cache, layer_idx: int, q: Tensor, k: Tensor, v: Tensor, scaling: float,
                     fused: bool | None = None) -> Tensor:
    """Decode branch of the patched forward (session.py:78-116).

    q: [B, Hq, 1, D], k/v: [B, Hkv, 1, D] (after RoPE).  Returns the
    attention output [B, 1, Hq * D] before o_proj.  The GQA layout of q is
    q head = kv * G + g (session.py:81-83).
    """
    fused = fused_attn_enabled() if fused is None else fused
    B = q.shape[0]
    H, G, D = cache.num_kv_heads, cache.num_kv_groups, cache.head_dim
    cache.update(k, v, layer_idx)
    # [B, H*G, 1, D] -> [B*H, G, D]: one view when q is contiguous
    q_flat = q.view(B * H, G, D) if q.is_contiguous() else q.squeeze(2).reshape(B * H, G, D)
    step = getattr(cache, "decode_step_attention", None)
    if step is not None:
        # the WnW cache appends and attends in one launch (slack layout)
        out = step(layer_idx, q_flat, q, k, v, scaling, fused)
    else:
        k_flat, v_flat, cu_k, _max_k = cache.decode_before_attn(layer_idx, k, v)
        if fused:
            out = cache.fused_decode_attention(layer_idx, q_flat, q, k_flat, v_flat, cu_k, scaling)
        else:
            out = q1_decode_attn(q_flat, k_flat, v_flat, cu_k, scaling)
            cache.decode_after_attn(layer_idx, q)
    out = out.reshape(B, 1, H * G * D)  # [B*H, G, D] -> [B, 1, Hq*D] (q head = kv*G + g)
    if layer_idx == cache.num_layers - 1:
        cache.decode_all_layers_done()
    return out


def prefill_attention(q: Tensor, k: Tensor, v: Tensor, attention_mask: Tensor | None, scaling: float,
                      q_chunk: int = 1024) -> Tensor:
    """Prompt attention of the prefill branch (session.py:53-63: SDPA with
    the model's mask, causal when there is none).  q/k/v: [B, Hq, S, D]
    (K/V already repeated over the group).

    SDPA runs with its fused backends only (flash, memory-efficient); when
    neither takes the inputs, the same attention is computed in float32
    over query chunks with contiguous operands (the products in float32,
    so no batched bf16 product with a transposed operand is issued)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v, attn_mask=attention_mask, scale=scaling,
                                                  is_causal=attention_mask is None)
    except RuntimeError:
        pass
    B, Hq, S, D = q.shape
    Skv = k.shape[2]
    kt = k.float().transpose(-1, -2).contiguous()
    vf = v.float().contiguous()
    if attention_mask is not None and attention_mask.dtype == torch.bool:
        attention_mask = torch.where(attention_mask, 0.0, float("-inf"))
    out = torch.empty(B, Hq, S, D, dtype=q.dtype, device=q.device)
    for i0 in range(0, S, q_chunk):
        i1 = min(S, i0 + q_chunk)
        s = torch.matmul(q[:, :, i0:i1].float().contiguous(), kt) * scaling
        if attention_mask is None:
            rows = torch.arange(i0, i1, device=q.device).unsqueeze(1) + (Skv - S)
            s = s.masked_fill(torch.arange(Skv, device=q.device).unsqueeze(0) > rows, float("-inf"))
        else:
            s = s + attention_mask[..., i0:i1, :].float()
        out[:, :, i0:i1] = torch.matmul(s.softmax(dim=-1), vf).to(q.dtype)
    return out


def compute_prefill_scores(q: Tensor, k: Tensor, attention_mask: Tensor | None, cache, layer_idx: int,
                           num_kv_heads: int, num_kv_groups: int, scaling: float):
    """Prefill token scores (session.py:119-169): class-A scores from the
    last prompt token of the layer's class-A query heads against their KV
    head, and per class-B/other KV head scores by ``prefill_score_mode``
    ("last": last token; "mean_text": mean over the text after the audio)."""
    B, _, S, _ = q.shape
    if attention_mask is not None and attention_mask.dim() == 4 and attention_mask.dtype == torch.bool:
        attention_mask = torch.where(attention_mask, 0.0, float("-inf")).to(q.dtype)
    if attention_mask is None:
        causal = torch.full((S, S), float("-inf"), device=q.device, dtype=q.dtype).triu_(1)
        attention_mask = causal.unsqueeze(0).unsqueeze(0).expand(B, 1, S, S)
    cfg = cache.config
    ca = cfg.get_layer_class_a(layer_idx)
    class_a_scores, per_head = [], []
    for b in range(B):
        ra, re = cache._raw_audio_starts[b], cache._raw_audio_ends[b]
        if ca:
            kv = ca[0] // num_kv_groups
            # transposed operands are made contiguous before batched bf16 products
            s = torch.matmul(q[b, ca, -1:, :], k[b, kv:kv + 1].transpose(-1, -2).contiguous()) * scaling
            s = (s + attention_mask[b, :, -1:, :]).float().softmax(dim=-1)
            class_a_scores.append(s[:, 0, ra:re].sum(dim=0).detach())
        else:
            class_a_scores.append(None)
        heads = []
        for h in range(num_kv_heads):
            if cfg.is_class_a_kv_head(layer_idx, h):
                heads.append(None)
                continue
            qs = q[b, h * num_kv_groups:(h + 1) * num_kv_groups]
            kk_t = k[b, h].unsqueeze(0).transpose(-1, -2).contiguous()
            if cfg.prefill_score_mode == "last":
                s = torch.matmul(qs[:, -1:], kk_t) * scaling + attention_mask[b, :, -1:, :]
                heads.append(s.float().softmax(dim=-1)[:, 0, ra:re].sum(dim=0))
            else:  # mean_text
                if S - re == 0:
                    heads.append(torch.zeros(re - ra, device=q.device, dtype=torch.float32))
                    continue
                s = torch.matmul(qs[:, re:], kk_t) * scaling + attention_mask[b, :, re:, :]
                heads.append(s.float().softmax(dim=-1)[:, :, ra:re].mean(dim=1).sum(dim=0))
        per_head.append(heads)
    return class_a_scores, per_head


class AlgorithmSession:
    """Context manager that swaps every decoder layer's attention forward
    for the cache-driven one and restores it on exit
    (src/common/session.py:15-92)."""

    def __init__(self, model, adapter, cache: FlatVarlenCache, processor=None):
        self.model, self.adapter, self.cache, self.processor = model, adapter, cache, processor
        self._adapter_state = None
        self._orig_forwards: list = []

    def __enter__(self):
        self.cache.reset()
        self.adapter.assert_compatible(self.model)
        self._adapter_state = self.adapter.prepare_for_inference(self.model)
        for layer in self.adapter.get_decoder_layers(self.model):
            attn = layer.self_attn
            self._orig_forwards.append((attn, attn.forward))
            attn.forward = types.MethodType(self._make_patched_forward(attn), attn)
        return self

    def __exit__(self, *exc):
        for attn, fwd in self._orig_forwards:
            attn.forward = fwd
        self._orig_forwards.clear()
        self.adapter.restore_after_inference(self.model, self._adapter_state)
        self._adapter_state = None

    def setup_audio(self, input_ids: Tensor, attention_mask: Tensor | None = None):
        starts, ends = self.adapter.locate_audio_tokens(input_ids, attention_mask, self.processor)
        self.cache.setup_audio(starts, ends, attention_mask)

    def generate(self, inputs: dict, **gen_kwargs) -> Tensor:
        gen_kwargs["past_key_values"] = self.cache
        return self.adapter.generate(self.model, inputs, **gen_kwargs)

    def get_stats(self) -> list[dict]:
        stats = getattr(self.cache, "stats", None)
        return [] if stats is None else stats.get_all_stats()

    def _make_patched_forward(self, attn_module):
        raise NotImplementedError


class WnWSession(AlgorithmSession):
    """session.py:20-116."""

    def _make_patched_forward(self, attn_module):
        cache, adapter = self.cache, self.adapter
        meta = adapter.attention_meta(attn_module)
        H, G = meta["num_kv_heads"], meta["num_kv_groups"]
        scaling, layer_idx = meta["scaling"], meta["layer_idx"]
        last = layer_idx == cache.num_layers - 1

        def patched_forward(self_attn, hidden_states: Tensor, position_embeddings=None,
                            attention_mask: Tensor | None = None, past_key_values=None, **kwargs):
            B, S, _ = hidden_states.shape
            q, k, v = adapter.compute_qkv(self_attn, hidden_states)
            q, k = adapter.apply_rope(q, k, position_embeddings, self_attn)
            if not cache.prefilled:
                cache.prefill_before_attn(layer_idx)
                cache.update(k, v, layer_idx)
                out = prefill_attention(q, k.repeat_interleave(G, dim=1), v.repeat_interleave(G, dim=1),
                                        attention_mask, scaling)
                ca, per_head = compute_prefill_scores(q, k, attention_mask, cache, layer_idx, H, G, scaling)
                cache.prefill_after_attn(layer_idx, ca, per_head, k, v)
                if last:
                    cache.prefill_all_layers_done()
                out = out.transpose(1, 2).reshape(B, S, -1).contiguous()
                return self_attn.o_proj(out), None
            out = decode_attention(cache, layer_idx, q, k, v, scaling)
            return self_attn.o_proj(out.reshape(B, S, -1).contiguous()), None

        return patched_forward

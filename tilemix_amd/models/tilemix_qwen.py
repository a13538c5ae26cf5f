"""TileMix attention for Hugging Face Qwen2 models (reference models/tilemix_qwen.py).

Same routing/bucket logic as the Llama module; differences kept from the
reference: the class name ``TileMixqwenAttention`` (lower-case "qwen"), the
Qwen2 forward signature (with its shim for callers that pass the attention
mask positionally), and the routing-map sanitisation before the kernel call
(:626-636): bits past the last mask group are cleared, and a map whose every
row is exactly the highest valid bit is widened to all-INT8 rows.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor
from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention, apply_rotary_pos_emb

from ..attention.tilemix_varlen import tilemix_varlen_attention
from ._common import MIN_TILEMIX_SEQLEN, TileMixRoutingMixin
from .tilemix_llama import _swap_attention

__all__ = ["TileMixqwenAttention", "inject_tilemix_into_qwen", "configure_tilemix_attention_pattern",
           "sanitize_precision_map"]


def sanitize_precision_map(precision_map: Tensor, seqlen: int, block_n_mask: int) -> Tensor:
    """Reference models/tilemix_qwen.py:626-636 (see the module docstring)."""
    groups = (seqlen + block_n_mask - 1) // block_n_mask
    valid = (1 << groups) - 1
    rows = [int(x) for x in precision_map.reshape(-1).tolist()]
    rows = [r & valid for r in rows]
    top = 1 << (groups - 1) if groups > 0 else 0
    if rows and all(r == top for r in rows):
        rows = [valid] * len(rows)
    out = torch.tensor(rows, dtype=torch.uint64)
    return out.to(precision_map.device)


class TileMixqwenAttention(TileMixRoutingMixin, Qwen2Attention):
    """Reference models/tilemix_qwen.py:46-658."""

    def __init__(self, config, layer_idx: int):
        Qwen2Attention.__init__(self, config, layer_idx=layer_idx)
        self._init_tilemix_state(config.num_attention_heads, config.num_key_value_heads)
        self._sanitized: dict[tuple, Tensor] = {}

    def _prewarm_triton_kernels(self):
        return None

    def _ensure_cuda(self, hidden_states: Tensor) -> Tensor:
        return hidden_states if hidden_states.is_cuda else hidden_states.cuda()

    def set_attention_pattern(self, pattern_type: str, **pattern_params):
        super().set_attention_pattern(pattern_type, **pattern_params)
        self._sanitized.clear()

    def forward(self, hidden_states: Tensor, position_embeddings: Optional[Tuple[Tensor, Tensor]] = None,
                attention_mask=None, past_key_values=None, cache_position=None, **kwargs):
        if past_key_values is None:
            past_key_values = kwargs.pop("past_key_value", None)
        # A caller passing the mask in the second position (reference :519-523).
        if position_embeddings is not None and not (isinstance(position_embeddings, tuple)
                                                    and len(position_embeddings) == 2):
            attention_mask = position_embeddings
            position_embeddings = kwargs.pop("position_embeddings", None)
        bsz, seqlen, _ = hidden_states.size()
        hidden_states = self._ensure_cuda(hidden_states)
        device = hidden_states.device
        if seqlen < MIN_TILEMIX_SEQLEN:
            return Qwen2Attention.forward(self, hidden_states, position_embeddings=position_embeddings,
                                          attention_mask=attention_mask, past_key_values=past_key_values,
                                          cache_position=cache_position, **kwargs)
        head_dim = self.config.hidden_size // self.config.num_attention_heads
        cfg, block_n_mask, pmap = self._routing_for(seqlen, device)
        skey = (seqlen, cfg.block_m, block_n_mask, pmap.data_ptr())
        clean = self._sanitized.get(skey)
        if clean is None:
            clean = sanitize_precision_map(pmap, seqlen, block_n_mask)
            self._sanitized[skey] = clean

        q = self.q_proj(hidden_states).view(bsz, seqlen, self.nh, head_dim).transpose(1, 2)
        k = self.k_proj(hidden_states).view(bsz, seqlen, self.nkv, head_dim).transpose(1, 2)
        v = self.v_proj(hidden_states).view(bsz, seqlen, self.nkv, head_dim).transpose(1, 2)
        if position_embeddings is not None:
            cos, sin = position_embeddings
        else:
            cos, sin = self.rotary_emb(q, kwargs.get("position_ids"))
        cos, sin = cos.to(device), sin.to(device)
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        if past_key_values is not None:
            k, v = past_key_values.update(k, v, self.layer_idx,
                                          cache_kwargs={"sin": sin, "cos": cos, "cache_position": cache_position})
        assert q.shape[1] == self.nh, f"Q heads {q.shape[1]} != nh {self.nh}"
        assert k.shape[1] == self.nkv, f"K heads {k.shape[1]} != nkv {self.nkv}"
        assert v.shape[1] == self.nkv, f"V heads {v.shape[1]} != nkv {self.nkv}"
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()

        out = tilemix_varlen_attention(q, k, v, cfg.block_m, cfg.block_n, block_n_mask=block_n_mask, causal=True,
                                       scale=head_dim ** -0.5, precision_map_all=clean,
                                       candidates=[(cfg.block_m, cfg.block_n)], flat_lengths=[clean.numel()])
        out = out.transpose(1, 2).reshape(bsz, seqlen, -1)
        return self.o_proj(out), None


def inject_tilemix_into_qwen(model):
    """Replace every layer's self-attention with ``TileMixqwenAttention`` (weights copied)."""
    return _swap_attention(model, TileMixqwenAttention)


def configure_tilemix_attention_pattern(model, pattern_type: str = "one", **pattern_params):
    root = model.model if hasattr(model, "model") else model
    for layer in root.layers:
        if isinstance(layer.self_attn, TileMixqwenAttention):
            layer.self_attn.set_attention_pattern(pattern_type, **pattern_params)
    return model

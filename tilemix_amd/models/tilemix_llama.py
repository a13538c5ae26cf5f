"""TileMix attention for Hugging Face Llama models (reference models/tilemix_llama.py).

Public surface, same names and signatures as the reference:

* ``TileMixLlamaAttention`` -- a ``LlamaAttention`` whose prefill runs the
  routed FP16/INT8 kernel through ``tilemix_varlen_attention``;
* ``inject_tilemix_into_llama(model)`` / ``configure_tilemix_attention_pattern``;
* ``PrefillCache`` -- a KV cache whose first update stores the prefill K/V
  without a copy (reference :703-715);
* ``prepare_llama_prefill(model)`` -- prefill helpers: RMSNorm, token-major
  RoPE (so the attention entry needs no transpose copy) and SiLU*mul
  (reference :718-895), restated with torch ops at the reference's rounding
  points: fp16 products and sum for RoPE (identical to ``apply_rotary_pos_emb``
  in fp16), fp16 SiLU then an fp16 product with ``up``.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor, nn
from transformers.cache_utils import Cache, DynamicLayer
from transformers.models.llama.modeling_llama import LlamaAttention, apply_rotary_pos_emb

from .. import _native
from ..attention.tilemix_varlen import tilemix_varlen_attention
from ._common import (MIN_TILEMIX_SEQLEN, BucketConfig, TileMixRoutingMixin, pick_block_n_for_64,  # noqa: F401
                      pick_mask_block_n)

__all__ = ["TileMixLlamaAttention", "inject_tilemix_into_llama", "configure_tilemix_attention_pattern", "rms_norm",
           "PrefillCache", "prepare_llama_prefill", "prepare_llama_norms", "rotary_token_major", "silu_mul",
           "PrefillRMSNorm", "PrefillMLP", "build_block_tables", "BucketConfig", "pick_mask_block_n",
           "pick_block_n_for_64"]


class TileMixLlamaAttention(TileMixRoutingMixin, LlamaAttention):
    """Reference models/tilemix_llama.py:52-646."""

    apply_rotary = staticmethod(apply_rotary_pos_emb)

    def __init__(self, config, layer_idx: int):
        LlamaAttention.__init__(self, config, layer_idx=layer_idx)
        self._init_tilemix_state(config.num_attention_heads, config.num_key_value_heads)

    # The reference warms Triton's JIT here (:177-217); the HIP kernels are
    # compiled ahead of time, so there is nothing to warm.
    def _prewarm_triton_kernels(self):
        return None

    def _ensure_cuda(self, hidden_states: Tensor) -> Tensor:
        return hidden_states if hidden_states.is_cuda else hidden_states.cuda()

    def forward(self, hidden_states: Tensor, attention_mask=None, position_ids=None, past_key_value=None,
                output_attentions: bool = False, use_cache: bool = False, cache_position=None,
                position_embeddings: Optional[Tuple[Tensor, Tensor]] = None, **kwargs):
        past_kv = past_key_value if past_key_value is not None else kwargs.pop("past_key_values", None)
        bsz, seqlen, _ = hidden_states.size()
        hidden_states = self._ensure_cuda(hidden_states)
        device = hidden_states.device
        if seqlen < MIN_TILEMIX_SEQLEN:
            return LlamaAttention.forward(self, hidden_states, position_embeddings=position_embeddings,
                                          attention_mask=attention_mask, past_key_values=past_kv,
                                          cache_position=cache_position, **kwargs)
        head_dim = self.config.hidden_size // self.config.num_attention_heads
        cfg, block_n_mask, pmap = self._routing_for(seqlen, device)

        q = self.q_proj(hidden_states).view(bsz, seqlen, self.nh, head_dim).transpose(1, 2)
        k = self.k_proj(hidden_states).view(bsz, seqlen, self.nkv, head_dim).transpose(1, 2)
        v = self.v_proj(hidden_states).view(bsz, seqlen, self.nkv, head_dim).transpose(1, 2)
        if position_embeddings is None:
            cos, sin = self.rotary_emb(q, position_ids)
        else:
            cos, sin = position_embeddings
        cos, sin = cos.to(device), sin.to(device)
        q, k = self.apply_rotary(q, k, cos, sin)
        if past_kv is not None:
            k, v = past_kv.update(k, v, self.layer_idx,
                                  cache_kwargs={"sin": sin, "cos": cos, "cache_position": cache_position})
        assert q.shape[1] == self.nh, f"Q heads {q.shape[1]} != nh {self.nh}"
        assert k.shape[1] == self.nkv, f"K heads {k.shape[1]} != nkv {self.nkv}"
        assert v.shape[1] == self.nkv, f"V heads {v.shape[1]} != nkv {self.nkv}"

        out = tilemix_varlen_attention(q, k, v, cfg.block_m, cfg.block_n, block_n_mask=block_n_mask, causal=True,
                                       scale=head_dim ** -0.5, precision_map_all=pmap,
                                       candidates=[(cfg.block_m, cfg.block_n)], flat_lengths=[pmap.numel()])
        out = out.transpose(1, 2).reshape(bsz, seqlen, -1)
        return self.o_proj(out), None


def build_block_tables(precision_map_2d: Tensor, num_heads: int) -> Tensor:
    """Reference :649-654: the block map as int32, replicated per head."""
    return precision_map_2d.to(torch.int32).unsqueeze(0).expand(num_heads, -1, -1).contiguous()


def _copy_attention_weights(src: nn.Module, dst: nn.Module) -> None:
    dst_state = dst.state_dict()
    for name, value in src.state_dict().items():
        if name in dst_state and dst_state[name].shape == value.shape:
            dst_state[name].copy_(value)


def _swap_attention(model, cls):
    root = model.model if hasattr(model, "model") else model
    for layer in root.layers:
        old = layer.self_attn
        ref = next(old.parameters())
        new = cls(old.config, old.layer_idx).to(device=ref.device, dtype=ref.dtype)
        with torch.no_grad():
            _copy_attention_weights(old, new)
        layer.self_attn = new
    model.use_tilemix = True
    return model


def inject_tilemix_into_llama(model):
    """Replace every layer's self-attention with ``TileMixLlamaAttention`` (weights copied)."""
    return _swap_attention(model, TileMixLlamaAttention)


def configure_tilemix_attention_pattern(model, pattern_type: str = "one", **pattern_params):
    """Set the routing layout of every TileMix attention module (clears their map caches)."""
    root = model.model if hasattr(model, "model") else model
    for layer in root.layers:
        if isinstance(layer.self_attn, TileMixLlamaAttention):
            layer.self_attn.set_attention_pattern(pattern_type, **pattern_params)
    return model


class _PrefillDynamicLayer(DynamicLayer):
    """First update keeps the given tensors (no concatenation copy)."""

    def update(self, key_states, value_states, cache_kwargs=None, *args, **kwargs):
        if not self.is_initialized:
            self.dtype, self.device = key_states.dtype, key_states.device
            self.keys, self.values = key_states, value_states
            self.is_initialized = True
            return self.keys, self.values
        return super().update(key_states, value_states, cache_kwargs, *args, **kwargs)


class PrefillCache(Cache):
    def __init__(self):
        super().__init__(layer_class_to_replicate=_PrefillDynamicLayer)


# ---- prefill helpers ---------------------------------------------------------
def _require_cuda(what: str, *tensors) -> None:
    if not all(t.is_cuda for t in tensors):
        raise RuntimeError(f"{what} is a GPU-only HIP kernel (reference: CUDA/Triton only)")


def rms_norm(hidden_states, weight, eps: float):
    """HIP RMSNorm over the last dim: weight * fp16(x * rsqrt(mean(x^2) + eps)),
    the mean in fp32 (reference models/tilemix_llama.py:718-797)."""
    if hidden_states.dtype != torch.float16 or weight.dtype != torch.float16:
        raise ValueError("prefill RMSNorm requires FP16 operands")
    cols = hidden_states.shape[-1]
    if weight.shape != (cols,) or not weight.is_contiguous():
        raise ValueError("RMSNorm weight must be a contiguous vector over the last dim")
    _require_cuda("prefill RMSNorm", hidden_states, weight)
    x = hidden_states if hidden_states.stride(-1) == 1 else hidden_states.contiguous()
    x2 = x.reshape(-1, cols)  # a view whenever rows are uniformly strided
    out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    p = _native.RmsNormParams()
    p.x, p.weight, p.out = x2.data_ptr(), weight.data_ptr(), out.data_ptr()
    p.rows, p.stride_x, p.stride_out = x2.shape[0], x2.stride(0) if x2.shape[0] > 1 else cols, cols
    p.cols, p.eps = cols, float(eps)
    _native.rms_norm_f16(p, x.device)
    return out


class PrefillRMSNorm(nn.Module):
    """weight * fp16(x * rsqrt(mean(x^2) + eps)), the mean in fp32 (reference :776-797),
    one HIP kernel."""

    def __init__(self, original):
        super().__init__()
        self.weight = original.weight
        self.variance_epsilon = original.variance_epsilon
        self.train(original.training)

    def forward(self, hidden_states):
        return rms_norm(hidden_states, self.weight, self.variance_epsilon)


def prepare_llama_norms(model):
    for layer in model.model.layers:
        layer.input_layernorm = PrefillRMSNorm(layer.input_layernorm)
        layer.post_attention_layernorm = PrefillRMSNorm(layer.post_attention_layernorm)
    model.model.norm = PrefillRMSNorm(model.model.norm)


def rotary_token_major(q, k, cos, sin):
    """Split-half RoPE whose outputs are token-major ``[b, t, h, d]`` tensors
    returned as ``[b, h, t, d]`` views (reference :808-847): q*cos and
    rotate(q)*sin are each rounded to fp16 and their sum is rounded to fp16.
    One HIP kernel for Q and K."""
    b, hq, t, d = q.shape
    hk = k.shape[1]
    if q.dtype != torch.float16 or any(x.dtype != q.dtype for x in (k, cos, sin)):
        raise ValueError("prefill rotary requires FP16 operands")
    if d % 2 or k.shape != (b, hk, t, d) or cos.shape[-2:] != (t, d) or sin.shape != cos.shape:
        raise ValueError("incompatible split-half rotary shapes")
    if cos.shape[0] not in (1, b):
        raise ValueError("rotary batch must be one or match the input")
    if q.stride(-1) != 1 or k.stride(-1) != 1 or cos.stride(-1) != 1 or sin.stride(-1) != 1:
        raise ValueError("rotary operands must have contiguous head dimensions")
    _require_cuda("prefill rotary", q, k, cos, sin)
    oq = torch.empty((b, t, hq, d), device=q.device, dtype=q.dtype)
    ok = torch.empty((b, t, hk, d), device=k.device, dtype=k.dtype)
    p = _native.RotaryParams()
    p.q, p.k, p.cos, p.sin = q.data_ptr(), k.data_ptr(), cos.data_ptr(), sin.data_ptr()
    p.q_out, p.k_out = oq.data_ptr(), ok.data_ptr()
    p.stride_q_batch, p.stride_q_head, p.stride_q_token = q.stride(0), q.stride(1), q.stride(2)
    p.stride_k_batch, p.stride_k_head, p.stride_k_token = k.stride(0), k.stride(1), k.stride(2)
    p.stride_cos_batch = cos.stride(0) if cos.shape[0] > 1 else 0
    p.stride_cos_token = cos.stride(1)
    p.stride_sin_batch = sin.stride(0) if sin.shape[0] > 1 else 0
    p.stride_sin_token = sin.stride(1)
    p.batch, p.tokens, p.heads_q, p.heads_k, p.head_dim = b, t, hq, hk, d
    _native.rotary_f16(p, q.device)
    return oq.transpose(1, 2), ok.transpose(1, 2)


def silu_mul(gate, up):
    """fp16(silu(gate)) * up in fp32, rounded to fp16 (reference :849-868), one HIP kernel."""
    if gate.dtype != torch.float16 or up.dtype != gate.dtype or gate.shape != up.shape:
        raise ValueError("SiLU requires equally shaped FP16 operands")
    if not gate.is_contiguous() or not up.is_contiguous():
        raise ValueError("SiLU requires contiguous operands")
    _require_cuda("prefill SiLU", gate, up)
    out = torch.empty_like(gate)
    _native.silu_mul_f16(gate, up, out)
    return out


class PrefillMLP(nn.Module):
    def __init__(self, original):
        super().__init__()
        self.gate_proj = original.gate_proj
        self.up_proj = original.up_proj
        self.down_proj = original.down_proj
        self.train(original.training)

    def forward(self, x):
        return self.down_proj(silu_mul(self.gate_proj(x), self.up_proj(x)))


def prepare_llama_prefill(model):
    """Swap in the prefill helpers (reference :883-895); TileMix must be injected first."""
    if model.training or model.config.hidden_act != "silu":
        raise ValueError("prefill requires an eval-mode SiLU LLaMA")
    for layer in model.model.layers:
        if not isinstance(layer.self_attn, TileMixLlamaAttention):
            raise ValueError("inject TileMix attention before preparing prefill")
        if layer.mlp.gate_proj.weight.dtype != torch.float16:
            raise ValueError("prefill requires FP16 model weights")
    prepare_llama_norms(model)
    for layer in model.model.layers:
        layer.self_attn.apply_rotary = rotary_token_major
        layer.mlp = PrefillMLP(layer.mlp)
    return model

"""CPU/torch restatement of the LLaMA prefill helper kernels -- TEST
INFRASTRUCTURE ONLY (the checker of tilemix_amd's HIP helpers; the product
path never imports it).

Each function restates, with torch tensor ops in fp32 and the reference's
fp16 rounding points, one helper of models/tilemix_llama.py:

* ``rms_norm``   <- squared_mean extension (:718-760: fp32 mean of x^2, the
  products rounded separately) and _norm_tail (:763-765):
  weight * fp16(fp32(x) * rsqrt(var + eps)).
* ``rotary_token_major`` <- _rotary (:808-829) and its launch (:832-847):
  fp16(fp16(x c) + fp16(x[d'] sign s)) into token-major [b, t, h, d].
* ``silu_mul``   <- _silu_mul (:850-858) and silu_mul (:861-869):
  fp16(fp16(g / (1 + exp(-g))) * up).

Parity pinning (tests/test_models.py): ``rotary_token_major`` equals
transformers' ``apply_rotary_pos_emb`` on fp16 tensors bit for bit (an
independent implementation of the same split-half RoPE with the same fp16
rounding points); ``silu_mul`` equals fp16(fp16(torch.nn.functional.silu) *
up); ``rms_norm`` matches an fp64 evaluation of the same formula to one fp16
ulp and the transformers LlamaRMSNorm to the same bound.
"""
from __future__ import annotations

import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    var = (xf * xf).mean(dim=-1, keepdim=True)
    return weight * (xf * torch.rsqrt(var + eps)).to(x.dtype)


def rotary_token_major(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    b, hq, t, d = q.shape
    hk = k.shape[1]
    c = cos[:, None].float()
    s = sin[:, None].float()

    def rope(x, heads):
        xf = x.float()
        half = d // 2
        rot = torch.cat((-xf[..., half:], xf[..., :half]), dim=-1)
        y = (xf * c).half().float() + (rot * s).half().float()
        out = torch.empty((b, t, heads, d), device=x.device, dtype=x.dtype)
        out.copy_(y.transpose(1, 2))
        return out.transpose(1, 2)

    return rope(q, hq), rope(k, hk)


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    g = gate.float()
    act = (g / (1.0 + torch.exp(-g))).half()
    return (act.float() * up.float()).half()

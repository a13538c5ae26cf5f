"""GPU parity of the HIP prefill helpers (RMSNorm, token-major rotary, SiLU * up)
against the oracle's torch restatement of the reference formulas
(oracle/prefill_oracle.py, evaluated on the CPU on the same fp16 inputs).

Bars: rotary is bit-exact (products of fp16 values are exact in fp32, one
fp32 add, the same two roundings).  SiLU * up is bit-exact except where the
device exp and the host exp differ by an fp32 ulp at an fp16 rounding
boundary (at most 1 in 1000 elements, each within one fp16 ulp).  RMSNorm
sums squares in a different order than the host reduction: the normalised
fp16 value may move by one ulp, which the weight multiply can carry to two
ulps of the output; at most 1% of the elements differ.
"""
from __future__ import annotations

import pytest
import torch

from oracle import prefill_oracle as PO
from tilemix_amd.models import tilemix_llama as TL

pytestmark = pytest.mark.gpu


def _ulp16(x: torch.Tensor) -> torch.Tensor:
    """One fp16 ulp at |x| (subnormal spacing below 2^-14)."""
    a = x.float().abs().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 10)


def _within_ulps(got: torch.Tensor, want: torch.Tensor, n: int = 1):
    g, w = got.float().cpu(), want.float().cpu()
    diff = (g - w).abs()
    tol = n * torch.maximum(_ulp16(g), _ulp16(w))
    return bool((diff <= tol).all()), (diff > 0).float().mean().item()


def _rope_inputs(b, hq, hk, t, d, cos_batch, seed, device):
    g = torch.Generator().manual_seed(seed)
    # q/k as the model produces them: token-major projections viewed [b, h, t, d]
    qp = (torch.randn(b, t, hq * d, generator=g) * 3).half()
    kp = (torch.randn(b, t, hk * d, generator=g) * 3).half()
    q = qp.view(b, t, hq, d).transpose(1, 2)
    k = kp.view(b, t, hk, d).transpose(1, 2)
    pos = torch.arange(t, dtype=torch.float32)
    inv = 1.0 / (500000.0 ** (torch.arange(0, d, 2).float() / d))
    emb = torch.cat((torch.outer(pos, inv),) * 2, dim=-1)
    cos = emb.cos().half()[None].expand(cos_batch, t, d).contiguous()
    sin = emb.sin().half()[None].expand(cos_batch, t, d).contiguous()
    return q, k, cos, sin


@pytest.mark.parametrize("b,hq,hk,t,d,cos_batch", [
    (2, 24, 8, 333, 128, 1),   # Llama-3.2-3B heads, broadcast cos/sin (vector path)
    (2, 4, 2, 37, 32, 2),      # per-batch cos/sin
    (1, 3, 1, 19, 24, 1),      # head_dim % 16 != 0: element-wise path
])
def test_rotary_bitexact(device, b, hq, hk, t, d, cos_batch):
    q, k, cos, sin = _rope_inputs(b, hq, hk, t, d, cos_batch, seed=d + t, device=device)
    wq, wk = PO.rotary_token_major(q, k, cos, sin)
    gq, gk = TL.rotary_token_major(q.to(device), k.to(device), cos.to(device), sin.to(device))
    torch.cuda.synchronize()
    assert gq.shape == (b, hq, t, d) and gk.shape == (b, hk, t, d)
    assert gq.transpose(1, 2).is_contiguous() and gk.transpose(1, 2).is_contiguous()
    assert torch.equal(gq.cpu(), wq) and torch.equal(gk.cpu(), wk)


@pytest.mark.parametrize("shape", [(4096, 8192), (7, 999), (3, 5)])
def test_silu_mul_matches_oracle(device, shape):
    g = torch.Generator().manual_seed(shape[1])
    gate = (torch.randn(*shape, generator=g) * 6).half()
    up = (torch.randn(*shape, generator=g) * 2).half()
    want = PO.silu_mul(gate, up)
    got = TL.silu_mul(gate.to(device), up.to(device))
    torch.cuda.synchronize()
    ok, frac = _within_ulps(got, want, 1)
    assert ok and frac <= 1e-3, frac
    assert torch.isfinite(got.float()).all()


@pytest.mark.parametrize("rows,cols,scale", [
    (4096, 3072, 1.0),   # Llama-3.2-3B hidden rows (vector path, row in registers)
    (65, 200, 30.0),     # large activations
    (9, 77, 1.0),        # ragged tail (cols % 8 != 0: scalar path)
    (5, 12288, 1.0),     # rows longer than the register-resident limit
])
def test_rms_norm_matches_oracle(device, rows, cols, scale):
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * scale).half()
    w = (torch.randn(cols, generator=g) * 0.3 + 1.0).half()
    want = PO.rms_norm(x, w, 1e-5)
    got = TL.rms_norm(x.to(device), w.to(device), 1e-5)
    torch.cuda.synchronize()
    ok, frac = _within_ulps(got, want, 2)
    assert ok and frac <= 0.01, frac


def test_rms_norm_strided_rows(device):
    """Rows taken from a wider buffer (row stride 3100, not a multiple of 8)."""
    g = torch.Generator().manual_seed(11)
    base = torch.randn(32, 3100, generator=g).half()
    x = base[:, 10:3082]
    w = (torch.randn(3072, generator=g) * 0.3 + 1.0).half()
    want = PO.rms_norm(x, w, 1e-6)
    got = TL.rms_norm(base.to(device)[:, 10:3082], w.to(device), 1e-6)
    torch.cuda.synchronize()
    ok, frac = _within_ulps(got, want, 2)
    assert ok and frac <= 0.01, frac

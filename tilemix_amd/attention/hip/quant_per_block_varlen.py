"""Per-block int8 quantisation of varlen token-major tensors on the HIP library.

Same public functions, arguments and results as the reference module
attention/triton/quant_per_block_varlen.py:

* ``per_block_int8_single(x, cu_seqlens_x, max_seqlen_x, BLK=128, sm_scale=1.0)``
  (reference :48-75) -> ``(x_int8, x_scale fp32 [rows, H], cu_seqlens_x_scale int64 [B+1])``
* ``per_block_int8(q, k, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
  BLKQ=128, BLKK=64, sm_scale=None)`` (reference :78-106).

The device kernel computes the scale-row prefix itself, so the internal
``quantize_blocks`` used by the attention entry needs no device->host copy.
The public ``per_block_int8_single`` still returns a scale tensor with exactly
``cu_seqlens_x_scale[-1]`` rows, which needs the row count on the host: it is
taken from ``cu_seqlens_x`` directly when that lives on the CPU, otherwise read
back once (the reference reads it back too, :62-63).
"""
from __future__ import annotations

import torch

from ... import _native


def _scale_capacity(n_tokens: int, batch: int, blk: int) -> int:
    # sum_b ceil(L_b / blk) <= ceil(sum_b L_b / blk) + batch, with sum_b L_b <= n_tokens
    return (n_tokens + blk - 1) // blk + batch


def _prepare_input(x: torch.Tensor) -> torch.Tensor:
    if x.ndim != 3:
        raise ValueError("expected a flattened [tokens, heads, dim] tensor")
    if x.dtype != torch.float16:
        raise TypeError(f"TileMix HIP quantisation supports float16 input, got {x.dtype}")
    if not x.is_cuda:
        raise RuntimeError("TileMix quantisation runs on the GPU (HIP); got a CPU tensor")
    if x.stride(2) != 1 or x.stride(0) % 8 or x.stride(1) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    return x


def quantize_blocks(x: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int, blk: int,
                    sm_scale: float = 1.0, *, half_scales: bool = False):
    """Quantise without any host synchronisation.

    Returns ``(codes int8 like x, scale fp32 [capacity, H], scale16 fp16 [capacity, H] | None,
    cu_scale int32 [B+1])``; rows of the scale tensors past ``cu_scale[-1]`` are
    unused.
    """
    x = _prepare_input(x)
    device = x.device
    cu = cu_seqlens.to(device=device, dtype=torch.int32).contiguous()
    batch = cu.numel() - 1
    heads, dim = x.shape[1], x.shape[2]
    if dim % 8:
        raise ValueError(f"head_dim must be a multiple of 8, got {dim}")
    cap = _scale_capacity(x.shape[0], batch, blk)
    codes = torch.empty(x.shape, dtype=torch.int8, device=device)
    scale = torch.empty((cap, heads), dtype=torch.float32, device=device)
    scale16 = torch.empty((cap, heads), dtype=torch.float16, device=device) if half_scales else None
    cu_scale = torch.empty(batch + 1, dtype=torch.int32, device=device)
    if batch > 0:
        p = _native.QuantParams()
        p.input = x.data_ptr()
        p.output = codes.data_ptr()
        p.scale = scale.data_ptr()
        p.scale_half = scale16.data_ptr() if scale16 is not None else None
        p.cu_seqlens = cu.data_ptr()
        p.cu_seqlens_scale = cu_scale.data_ptr()
        p.stride_in_token, p.stride_in_head = x.stride(0), x.stride(1)
        p.stride_out_token, p.stride_out_head = codes.stride(0), codes.stride(1)
        p.scale_rows_capacity = cap
        p.sm_scale = float(sm_scale)
        p.heads, p.head_dim, p.blk_tokens = heads, dim, int(blk)
        p.batch, p.max_seqlen = batch, int(max_seqlen)
        _native.quant_per_block_int8(p, device)
    else:
        cu_scale.zero_()
    return codes, scale, scale16, cu_scale


@torch.no_grad()
def per_block_int8_single(x, cu_seqlens_x, max_seqlen_x, BLK=128, sm_scale=1.0):
    """Reference attention/triton/quant_per_block_varlen.py:48-75."""
    if cu_seqlens_x.device.type == "cpu":
        lens = (cu_seqlens_x[1:] - cu_seqlens_x[:-1]).to(torch.int64)
        rows = int(((lens + BLK - 1) // BLK).sum())
    else:
        rows = None
    codes, scale, _, cu_scale = quantize_blocks(x, cu_seqlens_x, max_seqlen_x, BLK, sm_scale)
    if rows is None:
        rows = int(cu_scale[-1].item())
    return codes, scale[:rows], cu_scale.to(torch.int64)


@torch.no_grad()
def per_block_int8(q, k, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                   BLKQ=128, BLKK=64, sm_scale=None):
    """Reference attention/triton/quant_per_block_varlen.py:78-106 (same Q sm_scale rule)."""
    head_dim = q.shape[-1]
    if sm_scale is None:
        sm_scale = head_dim ** -0.5
    if abs(sm_scale - 1.0) < 1e-6:
        q_sm_scale = 1.0
    else:
        q_sm_scale = sm_scale * 1.44269504
    q_int8, q_scale, cu_seqlens_q_scale = per_block_int8_single(
        q, cu_seqlens_q, max_seqlen_q, BLK=BLKQ, sm_scale=q_sm_scale)
    k_int8, k_scale, cu_seqlens_k_scale = per_block_int8_single(
        k, cu_seqlens_k, max_seqlen_k, BLK=BLKK, sm_scale=1.0)
    return q_int8, q_scale, k_int8, k_scale, cu_seqlens_q_scale, cu_seqlens_k_scale

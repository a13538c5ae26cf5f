"""Dense-batch entry of the TileMix prefill attention (drop-in for the reference's
attention/tilemix_varlen.py:17-96).

``[B, H, T, D]`` query/key/value tensors are viewed token-major ``[B*T, H, D]``
with uniform ``cu_seqlens`` and handed to ``tilemix_attention_with_quant`` with
the reference's fixed call parameters (BLKQ=128, BLKK=64, run_length off,
scalar scales iff (block_m, block_n) == (128, 64), routing mode from
``TILEMIX_BITMASK_ROUTING_MODE`` (default ``mixed``), fp16 V for INT8 tiles
unless ``TILEMIX_SCORE_ONLY_PV`` is falsy).  The result is the same
``[B, Hq, T, D]`` permuted view of the token-major output.
"""
from __future__ import annotations

import os
from typing import Optional

import torch
from torch import Tensor

from .hip.tilemix import tilemix_attention_with_quant


def _env_flag(name: str, default: str = "0") -> bool:
    """Reference :8-14: anything but 0/false/no/'' is true."""
    return (os.getenv(name) or default).strip().lower() not in ("0", "false", "no", "")


def tilemix_varlen_attention(
    q: Tensor, k: Tensor, v: Tensor,
    block_m: int, block_n: int,
    *,
    block_n_mask: Optional[int] = None,
    causal: bool,
    scale: float,
    precision_map_all: Tensor,
    candidates: list[tuple[int, int]],
    flat_lengths: list[int],
    bias: Optional[Tensor] = None,
) -> Tensor:
    """Reference attention/tilemix_varlen.py:17-96 (``candidates`` and
    ``flat_lengths`` are accepted and unused, as there)."""
    B, Hq, Tq, D = q.shape
    _, Hk, Tk, Dk = k.shape
    _, Hv, Tv, Dv = v.shape
    if Dk != D or Dv != D:
        raise AssertionError("Q/K/V head dims differ")
    if Hk != Hv:
        raise AssertionError("K and V must have the same number of heads (GQA support)")

    Q = q.permute(0, 2, 1, 3).reshape(B * Tq, Hq, D).contiguous()
    K = k.permute(0, 2, 1, 3).reshape(B * Tk, Hk, D).contiguous()
    V = v.permute(0, 2, 1, 3).reshape(B * Tk, Hv, D).contiguous()

    device = Q.device
    cu_q = torch.arange(0, (B + 1) * Tq, Tq, device=device, dtype=torch.int32)
    cu_k = torch.arange(0, (B + 1) * Tk, Tk, device=device, dtype=torch.int32)

    pm = precision_map_all
    if pm.dtype != torch.uint64:
        raise AssertionError(f"precision_map dtype must be uint64, got {pm.dtype}")
    if block_n_mask is None:
        block_n_mask = block_n
    if block_n_mask % block_n != 0:
        raise ValueError(f"block_n_mask ({block_n_mask}) must be a multiple of block_n ({block_n})")
    if Tq != Tk:
        raise ValueError(
            f"Tq ({Tq}) != Tk ({Tk}). Bitmask was created assuming they're equal. "
            f"This will cause incorrect indexing in the kernel.")

    m_blocks_total = (Tq + block_m - 1) // block_m
    n_mask_blocks_total = (Tk + block_n_mask - 1) // block_n_mask
    if n_mask_blocks_total > 64:
        raise ValueError(
            f"64-bit precision mask requires n_mask_blocks<=64, got n_mask_blocks={n_mask_blocks_total} "
            f"(Tk={Tk}, block_n_mask={block_n_mask})")
    expected_pm_elems = Hk * m_blocks_total
    if pm.numel() != expected_pm_elems:
        raise AssertionError(
            f"precision_map length mismatch: got {pm.numel()}, expected {expected_pm_elems} "
            f"(Hk={Hk} KV heads x m_blocks={m_blocks_total}, n_mask_blocks={n_mask_blocks_total})")

    if bias is not None:
        bias = bias.to(device=device, dtype=q.dtype).contiguous()
        if bias.shape != (B, Hq, Tq, Tk):
            raise ValueError(f"Bias shape mismatch: got {bias.shape}, expected {(B, Hq, Tq, Tk)}")

    routing_mode = (os.getenv("TILEMIX_BITMASK_ROUTING_MODE") or "mixed").strip().lower()
    Out, _ = tilemix_attention_with_quant(
        Q, K, V, cu_q, cu_k,
        max_seqlens_q=Tq, max_seqlens_k=Tk,
        precision_bitmask=pm,
        block_m=block_m, block_n=block_n, block_n_mask=block_n_mask,
        BLKQ=128, BLKK=64,
        causal=causal, sm_scale=scale, bias=bias,
        routing_mode=routing_mode, run_length=False,
        scalar_scales=(block_m == 128 and block_n == 64),
        int8_cache_ca=False,
        int8_use_fp16_v=_env_flag("TILEMIX_SCORE_ONLY_PV", "1"),
    )
    return Out.view(B, Tq, Hq, D).permute(0, 2, 1, 3)

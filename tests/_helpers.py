"""Shared input builders for the parity tests (CPU-side, seeded)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import tilemix_oracle as O

# Parity bar of the attention output against the fp32 emulation.
MAX_ABS_TOL = 2e-3
MEAN_ABS_TOL = 2e-4


def packed_inputs(lengths, hq, hk, d, seed=0, outliers=(), outlier_scale=8.0, scale=1.0):
    """Packed varlen fp16 q [N, hq, d], k/v [N, hk, d] ~ N(0,1)*scale and cu_seqlens."""
    rng = np.random.default_rng(seed)
    n = int(sum(lengths))
    q = rng.standard_normal((n, hq, d), dtype=np.float32) * scale
    k = rng.standard_normal((n, hk, d), dtype=np.float32) * scale
    v = rng.standard_normal((n, hk, d), dtype=np.float32)
    for c in outliers:
        q[:, :, c] *= outlier_scale
        k[:, :, c] *= outlier_scale
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    return q.astype(np.float16), k.astype(np.float16), v.astype(np.float16), cu


def random_bitmask(hk, m_blocks, seed=0, p=0.5):
    rng = np.random.default_rng(seed + 99)
    bits = rng.random((hk * m_blocks, 64)) < p
    rows = [sum(1 << j for j in range(64) if bits[r, j]) for r in range(bits.shape[0])]
    return np.array(rows, dtype=np.uint64)


def to_dev(a, device, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(device)


def bitmask_tensor(rows, device):
    return torch.tensor([int(x) for x in rows], dtype=torch.uint64).to(device)


def oracle_quant(q, k, cu, blkq=128, blkk=64):
    q8, sq, cuq = O.quant_per_block_int8(q, cu, blkq)
    k8, sk, cuk = O.quant_per_block_int8(k, cu, blkk)
    return q8, sq, cuq, k8, sk, cuk


def assert_close_out(out_gpu: np.ndarray, out_ref: np.ndarray, *, max_tol=MAX_ABS_TOL, mean_tol=MEAN_ABS_TOL):
    d = np.abs(out_gpu.astype(np.float64) - out_ref.astype(np.float64))
    assert np.isfinite(out_gpu).all(), "non-finite output"
    assert d.max() <= max_tol and d.mean() <= mean_tol, f"max {d.max():.3e} mean {d.mean():.3e}"
    return d.max(), d.mean()

"""The PyTorch-eager CPU restatement (oracle/tilemix_torch_cpu.py, the CPU
baseline bench.py times) against the pinned numpy oracle on the same inputs:
codes and scales bit for bit, attention outputs within the parity bar."""
from __future__ import annotations

import numpy as np
import torch

from oracle import tilemix_oracle as O
from oracle import tilemix_torch_cpu as T
from tests._helpers import packed_inputs, random_bitmask


def test_quant_blocks_bitexact():
    q, k, v, cu = packed_inputs([200], 3, 1, 64, seed=1, outliers=(5,))
    for blk in (64, 128):
        codes, s = T.quant_blocks(torch.from_numpy(q), blk)
        c_ref, s_ref, _ = O.quant_per_block_int8(q, np.array([0, 200]), blk)
        assert np.array_equal(codes.numpy(), c_ref)
        assert np.array_equal(s.numpy(), s_ref)


def test_attention_matches_numpy_oracle():
    """Varlen causal GQA launch with a random mixed map at block_m 128 and 64,
    mask groups of 1 and 2 tiles, 4 outlier channels (peaked softmax)."""
    for block_m, bnm in ((128, 64), (64, 128)):
        lengths, hq, hk, d = [300, 129, 1], 6, 2, 64
        q, k, v, cu = packed_inputs(lengths, hq, hk, d, seed=block_m, outliers=(3, 17))
        bits = random_bitmask(hk, -(-300 // block_m), seed=block_m)
        got = T.attn_fwd_causal(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), cu, bits,
                                block_m=block_m, block_n_mask=bnm).numpy()
        q8, sq, cuq = O.quant_per_block_int8(q, cu, 128)
        k8, sk, cuk = O.quant_per_block_int8(k, cu, 64)
        ref = O.attn_fwd(q, k, v, cu, cu, bits, block_m=block_m, block_n_mask=bnm, causal=True, q8=q8, k8=k8,
                         sq16=sq.astype(np.float16), sk16=sk.astype(np.float16), cu_q_scale=cuq, cu_k_scale=cuk)
        diff = np.abs(got.astype(np.float64) - ref.astype(np.float64))
        assert diff.max() <= 2e-3 and diff.mean() <= 2e-4, (block_m, diff.max(), diff.mean())
        assert (diff == 0).mean() > 0.99

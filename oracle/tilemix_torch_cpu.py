"""PyTorch-eager CPU restatement of the TileMix prefill attention -- TEST
INFRASTRUCTURE ONLY.

This is the CPU baseline ``bench.py`` times (the reference itself has no CPU
path: it is CUDA-only, attention/triton/tilemix.py:1167-1168), and only
tests/ and ``bench.py``'s ``cpu_baseline`` leg import it.  It is checked
against the numpy oracle (oracle/tilemix_oracle.py, itself pinned by
tests/test_oracle.py) by tests/test_torch_cpu_oracle.py.

Same numerics as the numpy oracle, restricted to the benchmark's launch:
causal, equal Q/K lengths per sequence, block_n = 64, BLKQ = 128, BLKK = 64,
fp16 V for PV (int8_use_fp16_v), no bias.  Per sequence and query block of
block_m rows it forms the FP16-route scores fp16(q16 . k) (exact sum in fp64,
rounded once) and the INT8-route scores fp16(fp32(q8 . k8) * ss) of every key
up to the block's last row, picks each 64-key tile's route from the packed
bitmask, and runs the online softmax tile by tile:

* quantisation  <- attention/triton/quant_per_block_varlen.py:29-45
* scores        <- attention/triton/tilemix.py:254 (FP16), :380-404 (INT8)
* mask          <- :256-262
* online softmax<- :179-207, acc += fp16(p) . V (fp32), out = fp16(acc / l)
                   (:299, :935-951)

Work is vectorised over heads (torch batched matmuls on the host's threads).
"""
from __future__ import annotations

import torch

LOG2E = 1.4426950408889634
BN = 64


def quant_blocks(x: torch.Tensor, blk: int):
    """x fp16 [L, H, D] (one sequence) -> (int8 codes [L, H, D], fp32 scales
    [ceil(L / blk), H]): scale = max|x| / 127 per (block, head), code =
    trunc(x / scale +- 0.5); an all-zero block gets scale 0 and codes 0."""
    L, H, D = x.shape
    nb = -(-L // blk)
    xs = torch.zeros(nb * blk, H, D, dtype=torch.float32)
    xs[:L] = x.float()
    b = xs.view(nb, blk, H, D)
    s = b.abs().amax(dim=(1, 3)) / 127.0
    t = b / s[:, None, :, None]
    t = t + torch.where(t >= 0, 0.5, -0.5)
    t = torch.where(s[:, None, :, None] == 0, torch.zeros_like(t), t)
    codes = t.trunc().to(torch.int64).to(torch.int8).view(nb * blk, H, D)[:L]
    return codes, s


@torch.no_grad()
def attn_fwd_causal(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens, bitmask, *, block_m: int,
                    block_n_mask: int, sm_scale: float | None = None) -> torch.Tensor:
    """Mixed-routing causal prefill over packed fp16 q [N, Hq, D], k/v [N, Hk, D]
    (Lq == Lk per sequence); ``bitmask`` holds the packed routing rows
    (``Hk * ceil(max_len / block_m)`` integers, row hk * ceil(L / block_m) + m
    per sequence).  Returns fp16 [N, Hq, D]."""
    n, hq, d = q.shape
    hk = k.shape[1]
    group = hq // hk
    if sm_scale is None:
        sm_scale = d ** -0.5
    qk_scale = torch.tensor(sm_scale, dtype=torch.float32) * torch.tensor(LOG2E, dtype=torch.float32)
    bits = [int(x) for x in bitmask]
    cu = [int(x) for x in cu_seqlens]
    out = torch.zeros(n, hq, d, dtype=torch.float16)
    tiles_per_group = block_n_mask // BN
    for z in range(len(cu) - 1):
        s0, L = cu[z], cu[z + 1] - cu[z]
        if L == 0:
            continue
        qz, kz, vz = q[s0:s0 + L], k[s0:s0 + L], v[s0:s0 + L]
        q8, sq = quant_blocks(qz, 128)
        k8, sk = quant_blocks(kz, 64)
        sq16, sk16 = sq.half(), sk.half()
        # head-major views, KV heads repeated for their query heads (GQA)
        q16h = (qz.float() * qk_scale).half().permute(1, 0, 2).double()          # [Hq, L, D]
        q8h = q8.permute(1, 0, 2).double()
        kh = kz.permute(1, 0, 2).double().repeat_interleave(group, 0)            # [Hq, L, D]
        k8h = k8.permute(1, 0, 2).double().repeat_interleave(group, 0)
        vh = vz.permute(1, 0, 2).float().repeat_interleave(group, 0)
        mbz = -(-L // block_m)
        for m in range(mbz):
            r0, r1 = m * block_m, min(L, (m + 1) * block_m)
            kend = r1                                                          # causal
            nt = -(-kend // BN)
            rows = torch.arange(r0, r1)
            keys = torch.arange(kend)
            # routes of the block's tiles, [Hq, nt] (True = INT8)
            route_t = torch.tensor([[(bits[(h // group) * mbz + m] >> (t // tiles_per_group)) & 1
                                     for t in range(nt)] for h in range(hq)], dtype=torch.bool)
            route = route_t.repeat_interleave(BN, 1)[:, None, :kend]           # [Hq, 1, kend]
            s16 = (q16h[:, r0:r1] @ kh[:, :kend].transpose(1, 2)).half()       # exact sum, one rounding
            acc_i = q8h[:, r0:r1] @ k8h[:, :kend].transpose(1, 2)              # exact integers
            sqr = sq16[rows // 128].t()                                        # [Hq, R]
            skr = sk16[keys // 64].t().repeat_interleave(group, 0)             # [Hq, kend]
            sqk = sqr[:, :, None] * skr[:, None, :]                            # fp16 product, one rounding
            ss = (sqk.float() * qk_scale).half()
            s8 = (acc_i.float() * ss.float()).half()
            qk = torch.where(route, s8, s16).float()
            valid = keys[None, :] <= rows[:, None]
            qk = torch.where(valid[None], qk, torch.tensor(float("-inf")))
            m_i = torch.full((hq, r1 - r0), float("-inf"))
            l_i = torch.ones(hq, r1 - r0)
            acc = torch.zeros(hq, r1 - r0, d)
            for t in range(nt):
                k0, k1 = t * BN, min(kend, (t + 1) * BN)
                st = qk[:, :, k0:k1]
                mx = st.amax(-1)
                has = mx != float("-inf")
                m_next = torch.where(has, torch.maximum(m_i, mx), m_i)
                shifted = torch.where(has[..., None], st - m_next[..., None], torch.tensor(float("-inf")))
                alpha = torch.where(has, torch.exp2(m_i - m_next), torch.ones_like(m_i))
                p16 = torch.exp2(shifted).half().float()
                acc = acc * alpha[..., None]
                l_i = l_i * alpha + p16.sum(-1)
                m_i = m_next
                acc = acc + p16 @ vh[:, k0:k1]
            out[s0 + r0:s0 + r1] = (acc / l_i[..., None]).half().permute(1, 0, 2)
    return out

"""BASELINE configs[4] on the GPU: the random-init fp16 Llama-3.2-3B (28 layers,
hidden 3072, 24/8 heads, head_dim 128, SwiGLU 8192, vocab 128256, RoPE theta
500000) with TileMix SpTrans50 injected in every layer.

* B8 x 4096 prefill into a ``PrefillCache`` with ``logits_to_keep=1`` (the
  reference harness, examples/benchmark_prefill.py:41-78): finite logits,
  every layer's cache holds the 4096 tokens, and the prefill-helper path gives
  the plain path's last-position top-1 with close logits.
* Teacher-forced parity of every layer on the real B8 x 4096 activations: the
  q/k/v each of the 28 TileMix calls receives (post-RoPE, not N(0,1) data) are
  captured with the kernel's output, and three query blocks per layer (first,
  middle, last) are recomputed by the CPU oracle on exactly that sub-problem.
  This isolates the kernel from the growth of ulp-level differences through
  28 layers.
* Agreement with the same 28-layer model whose attention calls are answered by
  the CPU oracle (everything else identical, on the GPU), at a length the
  oracle can afford: top-1 of the logits at every position of 12 sequences x
  256 tokens (3072 positions, the last of each sequence among them), on the
  positions where two valid oracle models agree, beside the all-position rate.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM

from oracle import tilemix_oracle as O
from tests.test_gpu_models import _oracle_varlen_attention
from tilemix_amd.models import tilemix_llama as TL

pytestmark = pytest.mark.gpu


def _cfg5_config():
    return LlamaConfig(vocab_size=128256, hidden_size=3072, intermediate_size=8192, num_hidden_layers=28,
                       num_attention_heads=24, num_key_value_heads=8, head_dim=128, rope_theta=500000.0,
                       max_position_embeddings=131072, rms_norm_eps=1e-5, hidden_act="silu",
                       tie_word_embeddings=True)


@pytest.fixture(scope="module")
def cfg5_model(device):
    cfg = _cfg5_config()
    torch.manual_seed(0)
    with torch.device(device):
        model = LlamaForCausalLM._from_config(cfg, dtype=torch.float16).eval()
    TL.inject_tilemix_into_llama(model)
    TL.configure_tilemix_attention_pattern(model, "sptrans", percentage=0.5, stride=128, c=32)
    yield model
    del model
    torch.cuda.empty_cache()


@pytest.mark.timeout(600)
def test_cfg5_prefill_b8x4096(device, cfg5_model):
    model = cfg5_model
    vocab = model.config.vocab_size
    ids = torch.randint(100, vocab, (8, 4096), generator=torch.Generator().manual_seed(0)).to(device)
    with torch.no_grad():
        plain = model(ids, use_cache=False, logits_to_keep=1).logits.float()
        TL.prepare_llama_prefill(model)
        cache = TL.PrefillCache()
        out = model(ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
        fast = out.logits.float()
    torch.cuda.synchronize()
    assert fast.shape == (8, 1, vocab)
    assert torch.isfinite(fast).all() and torch.isfinite(plain).all()
    for layer in range(model.config.num_hidden_layers):
        assert cache.get_seq_length(layer) == 4096
        assert cache.layers[layer].keys.shape == (8, 8, 4096, 128)
    diff = (fast - plain).abs()
    print(f"cfg5 B8x4096 helper vs plain path: last-position logits max-abs {diff.max().item():.3e} "
          f"mean-abs {diff.mean().item():.3e}", flush=True)
    assert torch.equal(fast[:, -1].argmax(-1), plain[:, -1].argmax(-1))
    assert diff.max().item() < 5e-2


# (sequence, 128-row query block) pairs checked in every layer: first, middle, last.
CFG5_BLOCKS = ((0, 0), (3, 15), (7, 31))


def _oracle_sub_block(q, k, v, pmap, z, m, block_m, block_n, bnm, scale, accum):
    """Oracle output of rows [m bm, m bm + bm) of sequence z of one dense-entry
    call (q [Hq, rows, D], k/v [Hk, keys, D] already cut to the block's rows and
    to the keys up to its last row): with causal attention those rows depend on
    nothing else, and the Q / K quantisation blocks are the full call's (BLKQ
    128 over the block's rows, BLKK 64 from the sequence's first key)."""
    hq, rows, d = q.shape
    hk, kend, _ = k.shape
    qs = np.ascontiguousarray(q.transpose(1, 0, 2))
    ks = np.ascontiguousarray(k.transpose(1, 0, 2))
    vs = np.ascontiguousarray(v.transpose(1, 0, 2))
    cuq, cuk = np.array([0, rows]), np.array([0, kend])
    mbz = pmap.size // hk
    sub_bits = np.array([int(pmap[h * mbz + m]) for h in range(hk)], dtype=np.uint64)
    q8, sq, cuqs = O.quant_per_block_int8(qs, cuq, 128)
    k8, sk, cuks = O.quant_per_block_int8(ks, cuk, 64)
    out = O.attn_fwd(qs, ks, vs, cuq, cuk, sub_bits, block_m=block_m, block_n_mask=bnm, causal=True,
                     sm_scale=scale, q8=q8, k8=k8, sq16=sq.astype(np.float16), sk16=sk.astype(np.float16),
                     cu_q_scale=cuqs, cu_k_scale=cuks, fp16_accum=accum, block_n=block_n)
    return out.transpose(1, 0, 2)


@pytest.mark.timeout(900)
def test_cfg5_per_layer_attention_parity(device, cfg5_model, monkeypatch):
    """Every one of the 28 TileMix attention calls of the B8 x 4096 SpTrans50
    prefill, on its real inputs: the kernel's rows of three query blocks per
    layer against the oracle on the same sub-problem.  Bar per layer and block:
    max-abs 2e-3 / mean-abs 2e-4 against the oracle with fp32 accumulation per
    16-wide k-step (the MFMA's order), and mean-abs 2e-4 with 99.9% of elements
    within 2e-3 against the exact-sum oracle (the definition; one fp16 ulp of
    an FP16-route score can move a peaked row by more than 2e-3, see
    tests/test_accumulation_models.py)."""
    model = cfg5_model
    vocab = model.config.vocab_size
    ids = torch.randint(100, vocab, (8, 4096), generator=torch.Generator().manual_seed(0)).to(device)
    captured = []
    real = TL.tilemix_varlen_attention

    def spy(q, k, v, block_m, block_n, **kw):
        out = real(q, k, v, block_m, block_n, **kw)
        blocks = []
        for z, m in CFG5_BLOCKS:
            r0, r1 = m * 128, min((m + 1) * 128, q.shape[2])
            blocks.append((z, m, q[z, :, r0:r1].cpu().numpy(), k[z, :, :r1].cpu().numpy(),
                           v[z, :, :r1].cpu().numpy(), out[z, :, r0:r1].cpu().numpy()))
        captured.append(dict(block_m=block_m, block_n=block_n, bnm=kw.get("block_n_mask") or block_n,
                             scale=kw["scale"], causal=kw["causal"], blocks=blocks,
                             pmap=np.array([int(x) for x in kw["precision_map_all"].reshape(-1).tolist()],
                                           dtype=np.uint64)))
        return out

    monkeypatch.setattr(TL, "tilemix_varlen_attention", spy)
    with torch.no_grad():
        model(ids, use_cache=False, logits_to_keep=1)
    torch.cuda.synchronize()
    monkeypatch.undo()
    assert len(captured) == model.config.num_hidden_layers
    worst = {"k16_max": 0.0, "k16_mean": 0.0, "exact_max": 0.0, "exact_mean": 0.0, "exact_within": 1.0}
    for layer, c in enumerate(captured):
        assert c["causal"] and c["block_m"] == 128, (c["block_m"], c["causal"])
        line = []
        for z, m, qb, kb, vb, ob in c["blocks"]:
            got = ob.astype(np.float64)
            assert np.isfinite(got).all()
            args = (qb, kb, vb, c["pmap"], z, m, c["block_m"], c["block_n"], c["bnm"], c["scale"])
            d16 = np.abs(got - _oracle_sub_block(*args, "fp32_k16"))
            dex = np.abs(got - _oracle_sub_block(*args, "exact"))
            within = float((dex <= 2e-3).mean())
            line.append(f"({z},{m}) k16 {d16.max():.2e}/{d16.mean():.1e} exact {dex.max():.2e}/{dex.mean():.1e} "
                        f"{within:.5f}")
            worst["k16_max"] = max(worst["k16_max"], d16.max())
            worst["k16_mean"] = max(worst["k16_mean"], d16.mean())
            worst["exact_max"] = max(worst["exact_max"], dex.max())
            worst["exact_mean"] = max(worst["exact_mean"], dex.mean())
            worst["exact_within"] = min(worst["exact_within"], within)
            assert d16.max() <= 2e-3 and d16.mean() <= 2e-4, (layer, z, m, d16.max(), d16.mean())
            assert dex.mean() <= 2e-4 and within >= 0.999, (layer, z, m, dex.mean(), within)
        print(f"cfg5 layer {layer:2d}: " + "; ".join(line), flush=True)
    print("cfg5 per-layer worst: " + ", ".join(f"{k} {v:.3e}" for k, v in worst.items()), flush=True)


@pytest.mark.timeout(900)
def test_cfg5_top1_agrees_with_oracle_attention(device, cfg5_model, monkeypatch):
    """Top-1 of TileMix vs the oracle-attention model, beside a control: the same
    model on two CPU oracles that differ only in how FP16-route scores
    accumulate (exact sum vs fp32 per 16-wide k-step, the MFMA's order).  The
    random-init model's logits are flat (top-2 gaps down to 0), so any
    ulp-level difference in an attention output flips some argmaxes after 28
    layers; the control measures that rate for two valid evaluations of the
    oracle's semantics."""
    model = cfg5_model
    vocab = model.config.vocab_size
    ids = torch.randint(100, vocab, (12, 256), generator=torch.Generator().manual_seed(1)).to(device)

    def run_with(accum):
        calls = []

        def attn(*args, **kwargs):
            calls.append(1)
            if len(calls) % 7 == 0:
                print(f"  oracle attention ({accum}): layer {len(calls)}", flush=True)
            return _oracle_varlen_attention(*args, fp16_accum=accum, **kwargs)

        monkeypatch.setattr(TL, "tilemix_varlen_attention", attn)
        try:
            return model(ids).logits.float()
        finally:
            monkeypatch.undo()
            assert len(calls) == model.config.num_hidden_layers

    with torch.no_grad():
        got = model(ids).logits.float()
        ref = run_with("exact")
        ref32 = run_with("fp32_k16")
    assert torch.isfinite(got).all()

    def stats(a, b):
        ta, tb = a.argmax(-1), b.argmax(-1)
        d = (a - b).abs()
        return ((ta == tb).float().mean().item(), (ta[:, -1] == tb[:, -1]).float().mean().item(),
                d.max().item(), d.mean().item())

    top2 = ref.topk(2, dim=-1).values
    gap = (top2[..., 0] - top2[..., 1]).flatten().cpu().numpy()
    res = {"tilemix_vs_oracle": stats(got, ref), "tilemix_vs_oracle_fp32k16": stats(got, ref32),
           "control_oracle_vs_oracle_fp32k16": stats(ref32, ref)}
    for name, (agree, last, dmax, dmean) in res.items():
        print(f"cfg5 8x256 {name}: top-1 agreement {agree:.5f} over {got.shape[0] * got.shape[1]} positions "
              f"(last positions {last:.3f}); logits max-abs {dmax:.3e} mean-abs {dmean:.3e}", flush=True)
    print(f"oracle model top-2 logit gap: median {np.median(gap):.3e}, 1% quantile {np.quantile(gap, 0.01):.3e}",
          flush=True)
    agree, last, dmax, dmean = res["tilemix_vs_oracle"]
    c_agree, _, c_dmax, c_dmean = res["control_oracle_vs_oracle_fp32k16"]
    # Oracle-stable positions: the two valid oracle models give the same top-1
    # and the exact oracle's top-2 gap is more than twice the largest logit
    # difference between the two oracles at that position (a position inside
    # that margin is a near-tie that any ulp-level difference can flip).
    t_got, t_ref, t_ref32 = got.argmax(-1), ref.argmax(-1), ref32.argmax(-1)
    both = t_ref == t_ref32
    gap_t = torch.from_numpy(gap).to(device).view(got.shape[:2])
    dc = (ref32 - ref).abs().amax(-1)
    stable = both & (gap_t > 2 * dc)
    n_stable, n_both = int(stable.sum().item()), int(both.sum().item())
    agree_stable = (t_got == t_ref)[stable].float().mean().item()
    agree_both = (t_got == t_ref)[both].float().mean().item()
    print(f"cfg5 top-1 on oracle-stable positions: {agree_stable:.5f} over {n_stable} positions; "
          f"where the two oracles agree: {agree_both:.5f} over {n_both}; all positions {agree:.5f} "
          f"over {t_got.numel()}", flush=True)
    assert n_stable >= 2048, n_stable
    assert agree_stable >= 0.999, (agree_stable, n_stable)
    # Fixed floor on the all-position rate (measured 0.9873 over 2048 positions
    # of this model; the control of two oracle models measured 0.9902).
    assert agree >= 0.98, agree
    assert dmean <= 1.5 * c_dmean, (dmean, c_dmean)
    # every position whose top-2 gap is wider than three times the largest
    # logit difference of the control agrees
    decisive = torch.from_numpy(gap > 3 * c_dmax).to(device).view(got.shape[:2])
    assert (got.argmax(-1) == ref.argmax(-1))[decisive].all()
    assert decisive.float().mean().item() > 0.4

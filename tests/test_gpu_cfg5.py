"""BASELINE configs[4] on the GPU: the random-init fp16 Llama-3.2-3B (28 layers,
hidden 3072, 24/8 heads, head_dim 128, SwiGLU 8192, vocab 128256, RoPE theta
500000) with TileMix SpTrans50 injected in every layer.

* B8 x 4096 prefill into a ``PrefillCache`` with ``logits_to_keep=1`` (the
  reference harness, examples/benchmark_prefill.py:41-78): finite logits,
  every layer's cache holds the 4096 tokens, and the prefill-helper path gives
  the plain path's last-position top-1 with close logits.
* Agreement with the same 28-layer model whose attention calls are answered by
  the CPU oracle (everything else identical, on the GPU), at a length the
  oracle can afford: top-1 of the logits at every position of 8 sequences x 256
  tokens (2048 positions, the last of each sequence among them), beside the
  same comparison between two variants of the oracle (see the test).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM

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
    ids = torch.randint(100, vocab, (8, 256), generator=torch.Generator().manual_seed(1)).to(device)

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
    # Measured on MI355X: agreement 0.9873 vs the control's 0.9902, logits
    # mean-abs 6.2e-3 vs 5.0e-3 (2048 positions; the standard error of either
    # agreement is ~0.0022).
    assert agree >= 0.999 or agree >= c_agree - 0.005, (agree, c_agree)
    assert dmean <= 1.5 * c_dmean, (dmean, c_dmean)
    # every position whose top-2 gap is wider than three times the largest
    # logit difference of the control agrees
    decisive = torch.from_numpy(gap > 3 * c_dmax).to(device).view(got.shape[:2])
    assert (got.argmax(-1) == ref.argmax(-1))[decisive].all()
    assert decisive.float().mean().item() > 0.4

"""GPU tests of the model glue: small random-init Llama / Qwen2 models with
TileMix injected (SpTrans routing), against the same models whose attention
call is answered by the CPU oracle (everything else identical, on the GPU).

Bar: top-1 of the logits agrees on >= 99.9% of
positions; logits stay within a small absolute distance.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM

from oracle import tilemix_oracle as O
from tilemix_amd.models import tilemix_llama as TL
from tilemix_amd.models import tilemix_qwen as TQ

pytestmark = pytest.mark.gpu


def _oracle_varlen_attention(q, k, v, block_m, block_n, *, block_n_mask=None, causal, scale, precision_map_all,
                             candidates=None, flat_lengths=None, bias=None, fp16_accum="exact"):
    """tilemix_varlen_attention computed by the CPU oracle (mixed routing,
    BLKQ 128 / BLKK 64, fp16 V for PV: the defaults of the dense entry);
    ``fp16_accum`` selects the oracle's FP16-route score accumulation model."""
    B, Hq, T, D = q.shape
    Hk = k.shape[1]
    qn = q.permute(0, 2, 1, 3).reshape(B * T, Hq, D).float().cpu().numpy().astype(np.float16)
    kn = k.permute(0, 2, 1, 3).reshape(B * T, Hk, D).float().cpu().numpy().astype(np.float16)
    vn = v.permute(0, 2, 1, 3).reshape(B * T, Hk, D).float().cpu().numpy().astype(np.float16)
    cu = np.arange(0, (B + 1) * T, T)
    q8, sq, cuq = O.quant_per_block_int8(qn, cu, 128)
    k8, sk, cuk = O.quant_per_block_int8(kn, cu, 64)
    bits = np.array([int(x) for x in precision_map_all.reshape(-1).tolist()], dtype=np.uint64)
    out = O.attn_fwd(qn, kn, vn, cu, cu, bits, block_m=block_m, block_n_mask=block_n_mask or block_n,
                     causal=causal, sm_scale=scale, q8=q8, k8=k8, sq16=sq.astype(np.float16),
                     sk16=sk.astype(np.float16), cu_q_scale=cuq, cu_k_scale=cuk, fp16_accum=fp16_accum,
                     block_n=block_n)
    o = torch.from_numpy(out.astype(np.float32)).to(q.device, torch.float16)
    return o.view(B, T, Hq, D).permute(0, 2, 1, 3)


def _compare(model, module, ids, monkeypatch):
    with torch.no_grad():
        got = model(ids).logits.float()
        monkeypatch.setattr(module, "tilemix_varlen_attention", _oracle_varlen_attention)
        ref = model(ids).logits.float()
        monkeypatch.undo()
    assert torch.isfinite(got).all()
    agree = (got.argmax(-1) == ref.argmax(-1)).float().mean().item()
    diff = (got - ref).abs()
    return agree, diff.max().item(), diff.mean().item()


def test_llama_tilemix_matches_oracle_attention(device, monkeypatch):
    cfg = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, rope_theta=500000.0)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).half().to(device).eval()
    TL.inject_tilemix_into_llama(model)
    TL.configure_tilemix_attention_pattern(model, "sptrans", percentage=0.5, stride=128, c=32)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 512, (4, 384), generator=g).to(device)
    agree, dmax, dmean = _compare(model, TL, ids, monkeypatch)
    assert agree >= 0.999, agree
    assert dmax < 0.05 and dmean < 2e-3, (dmax, dmean)


@pytest.mark.parametrize("forced", ["64,128", "64,256"])
def test_llama_forced_block_n(device, monkeypatch, forced):
    """TILEMIX_FORCE_CONFIG picks the reference's (64, 128) / (64, 256) sizes
    (models/tilemix_llama.py:143-153): the model runs the block_n > 64 kernels
    and agrees with the oracle attention of the same block_n."""
    monkeypatch.setenv("TILEMIX_FORCE_CONFIG", forced)
    cfg = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, rope_theta=500000.0)
    torch.manual_seed(7)
    model = LlamaForCausalLM(cfg).half().to(device).eval()
    TL.inject_tilemix_into_llama(model)
    TL.configure_tilemix_attention_pattern(model, "sptrans", percentage=0.5, stride=128, c=32)
    seen = []
    real = TL.tilemix_varlen_attention

    def spy(q, k, v, block_m, block_n, **kw):
        seen.append((block_m, block_n))
        return real(q, k, v, block_m, block_n, **kw)

    ids = torch.randint(0, 512, (2, 640), generator=torch.Generator().manual_seed(8)).to(device)
    with torch.no_grad():
        monkeypatch.setattr(TL, "tilemix_varlen_attention", spy)
        got = model(ids).logits.float()
        monkeypatch.setattr(TL, "tilemix_varlen_attention", _oracle_varlen_attention)
        ref = model(ids).logits.float()
    assert set(seen) == {tuple(int(x) for x in forced.split(","))}
    agree = (got.argmax(-1) == ref.argmax(-1)).float().mean().item()
    diff = (got - ref).abs()
    assert agree >= 0.999, agree
    assert diff.max().item() < 0.05 and diff.mean().item() < 2e-3


@pytest.mark.parametrize("block_m", [256, 512])
@pytest.mark.parametrize("seqlen", [40, 700])
def test_dense_entry_block_m_256_512(device, block_m, seqlen):
    """block_m 256 / 512 through tilemix_varlen_attention (the sizes the
    reference's block-size search falls back to, models/tilemix_llama.py:137-140;
    its model forward then rejects them, :546-555, so the attention entry is
    where they are reachable): against the oracle attention of that block_m."""
    B, Hq, Hk, D = 2, 4, 2, 128
    g = torch.Generator().manual_seed(block_m + seqlen)
    q, k, v = (torch.randn(B, h, seqlen, D, generator=g).half() for h in (Hq, Hk, Hk))
    m_blocks = -(-seqlen // block_m)
    rows = torch.randint(0, 2 ** 62, (Hk * m_blocks,), generator=g).to(torch.uint64)
    args = (q.to(device), k.to(device), v.to(device), block_m, 64)
    kw = dict(block_n_mask=64, causal=True, scale=D ** -0.5, precision_map_all=rows.to(device),
              candidates=[(block_m, 64)], flat_lengths=[rows.numel()])
    got = TL.tilemix_varlen_attention(*args, **kw).float()
    ref = _oracle_varlen_attention(*args, **kw).float()
    torch.cuda.synchronize()
    d = (got - ref).abs()
    assert d.max().item() <= 2e-3 and d.mean().item() <= 2e-4, (d.max().item(), d.mean().item())


def test_llama_head_dim_72(device, monkeypatch):
    """A head_dim that is not a multiple of 16 (72): the host zero-pads Q/K/V
    and the model agrees with the oracle attention at the original width."""
    cfg = LlamaConfig(vocab_size=512, hidden_size=288, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=72)
    torch.manual_seed(9)
    model = LlamaForCausalLM(cfg).half().to(device).eval()
    TL.inject_tilemix_into_llama(model)
    TL.configure_tilemix_attention_pattern(model, "sptrans", percentage=0.5, stride=128, c=32)
    ids = torch.randint(0, 512, (2, 320), generator=torch.Generator().manual_seed(10)).to(device)
    agree, dmax, dmean = _compare(model, TL, ids, monkeypatch)
    assert agree >= 0.999, agree
    assert dmax < 0.05 and dmean < 2e-3, (dmax, dmean)


def test_llama_prefill_helpers_keep_logits(device):
    cfg = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2)
    torch.manual_seed(2)
    model = LlamaForCausalLM(cfg).half().to(device).eval()
    TL.inject_tilemix_into_llama(model)
    TL.configure_tilemix_attention_pattern(model, "sptrans", percentage=0.5, stride=64, c=16)
    ids = torch.randint(0, 512, (2, 256), generator=torch.Generator().manual_seed(3)).to(device)
    with torch.no_grad():
        base = model(ids).logits.float()
        TL.prepare_llama_prefill(model)
        cache = TL.PrefillCache()
        out = model(ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
        fast = out.logits.float()
    assert cache.get_seq_length(0) == 256
    assert (fast[:, -1] - base[:, -1]).abs().max().item() < 2e-2
    assert torch.equal(fast[:, -1].argmax(-1), base[:, -1].argmax(-1))


def test_qwen_tilemix_matches_oracle_attention(device, monkeypatch):
    cfg = Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=1)
    torch.manual_seed(4)
    model = Qwen2ForCausalLM(cfg).half().to(device).eval()
    TQ.inject_tilemix_into_qwen(model)
    TQ.configure_tilemix_attention_pattern(model, "bigbird", percentage=0.5)
    ids = torch.randint(0, 512, (2, 320), generator=torch.Generator().manual_seed(5)).to(device)
    agree, dmax, dmean = _compare(model, TQ, ids, monkeypatch)
    assert agree >= 0.999, agree
    assert dmax < 0.05 and dmean < 2e-3, (dmax, dmean)


def test_short_sequences_use_the_parent_attention(device):
    cfg = LlamaConfig(vocab_size=128, hidden_size=128, intermediate_size=256, num_hidden_layers=1,
                      num_attention_heads=2, num_key_value_heads=1)
    torch.manual_seed(6)
    model = LlamaForCausalLM(cfg).half().to(device).eval()
    ids = torch.randint(0, 128, (1, 9)).to(device)
    with torch.no_grad():
        want = model(ids).logits
        TL.inject_tilemix_into_llama(model)
        got = model(ids).logits
    assert torch.equal(got, want)

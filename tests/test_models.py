"""CPU tests of the model glue (tilemix_amd.models): block-size buckets, routing
maps and their caches, injection, the prefill cache and the prefill helpers.
Kernel launches are covered by the GPU tests (test_gpu_models.py)."""
from __future__ import annotations

import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM
from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

from oracle import prefill_oracle as PO
from tilemix_amd.attention import precision_maps as pm
from tilemix_amd.models import tilemix_llama as TL
from tilemix_amd.models import tilemix_qwen as TQ
from tilemix_amd.models._common import sptrans_token_mask


def _tiny_llama(layers=2):
    cfg = LlamaConfig(vocab_size=96, hidden_size=128, intermediate_size=256, num_hidden_layers=layers,
                      num_attention_heads=4, num_key_value_heads=2)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).eval()


def test_pick_mask_block_n():
    # ceil(L/64) rounded up to a multiple of the compute tile, at least the tile.
    for L, bn, want in [(256, 64, 64), (4096, 64, 64), (4097, 64, 128), (8192, 64, 128), (32768, 64, 512),
                        (100, 128, 128), (20000, 128, 384)]:
        assert TL.pick_mask_block_n(L, bn) == want
        assert (L + want - 1) // want <= 64
    assert TL.pick_block_n_for_64(4096, [64, 128, 256]) == 64
    assert TL.pick_block_n_for_64(8192, [64, 128, 256]) == 128
    assert TL.pick_block_n_for_64(10 ** 6, [64, 128, 256]) == 256


def test_block_config_buckets(monkeypatch):
    attn = _tiny_llama(1)
    TL.inject_tilemix_into_llama(attn)
    a = attn.model.layers[0].self_attn
    monkeypatch.delenv("TILEMIX_FORCE_CONFIG", raising=False)
    assert (a._get_block_config(256).block_m, a._get_block_config(256).block_n) == (64, 64)
    assert (a._get_block_config(4095).block_m, a._get_block_config(4096).block_m) == (64, 128)
    assert a._get_block_config(40000) == TL.BucketConfig(128, 64)
    monkeypatch.setenv("TILEMIX_FORCE_CONFIG", "128,64,8,2")
    assert a._get_block_config(512) == TL.BucketConfig(128, 64)
    monkeypatch.setenv("TILEMIX_FORCE_CONFIG", "60,250,8,2")      # snapped to the nearest available size
    assert a._get_block_config(4096) == TL.BucketConfig(64, 256)
    monkeypatch.setenv("TILEMIX_FORCE_CONFIG", "not,a,config")   # ignored, like the reference
    assert a._get_block_config(256) == TL.BucketConfig(64, 64)


@pytest.mark.parametrize("forced,want", [("256,64", (256, 64)), ("512,64", (512, 64))])
def test_forced_fallback_block_m_is_rejected_by_the_model(monkeypatch, forced, want):
    """Below every available block_n (40 tokens) the forced size falls back to
    the nearest of block_m 64/128/256/512 (reference models/tilemix_llama.py:
    137-140), and the model's forward then rejects a size outside
    available_block_sizes with the reference's ValueError (:546-555); the
    attention entry itself runs block_m 256 / 512 (GPU tests)."""
    model = _tiny_llama(1)
    TL.inject_tilemix_into_llama(model)
    a = model.model.layers[0].self_attn
    monkeypatch.setenv("TILEMIX_FORCE_CONFIG", forced)
    assert (a._get_block_config(40).block_m, a._get_block_config(40).block_n) == want
    with pytest.raises(ValueError, match="is not in available_block_sizes. This should not happen"):
        a._routing_for(40, torch.device("cpu"))


def test_inject_copies_weights_and_configure_clears_caches():
    model = _tiny_llama()
    before = {k: v.clone() for k, v in model.state_dict().items()}
    TL.inject_tilemix_into_llama(model)
    assert model.use_tilemix
    after = model.state_dict()
    for k, v in before.items():
        assert torch.equal(v, after[k]), k
    a = model.model.layers[1].self_attn
    assert isinstance(a, TL.TileMixLlamaAttention)
    assert a.kv_head_mapping.tolist() == [0, 0, 1, 1]
    TL.configure_tilemix_attention_pattern(model, "band", percentage=0.5)
    cfg, bnm, full = a._routing_for(512, torch.device("cpu"))
    assert len(a.precision_map_cache) == 1
    row = pm.make_precision_bitmask(512, cfg.block_m, bnm, None, percentage=0.5, pattern_type="band",
                                    pattern_params={"percentage": 0.5}, COMPUTE_BLOCK_N=cfg.block_n)
    assert full.tolist() == row.tolist() * 2          # one row map per KV head
    again = a._routing_for(512, torch.device("cpu"))[2]
    assert again.tolist() == full.tolist()
    TL.configure_tilemix_attention_pattern(model, "zero")
    assert not a.precision_map_cache
    assert set(a._routing_for(512, torch.device("cpu"))[2].tolist()) == {0}


@pytest.mark.parametrize("ptype,params", [("one", {}), ("causal", {}), ("global", {}), ("row_rand", {}),
                                          ("align_sparse", {}), ("bigbird", {}), ("block", {}),
                                          ("layout_causal", {}), ("sptrans", {"stride": 64, "c": 16})])
def test_token_mask_patterns_route(ptype, params):
    model = _tiny_llama(1)
    TL.inject_tilemix_into_llama(model)
    a = model.model.layers[0].self_attn
    TL.configure_tilemix_attention_pattern(model, ptype, **params)
    torch.manual_seed(3)
    cfg, bnm, full = a._routing_for(320, torch.device("cpu"))
    m_blocks = (320 + cfg.block_m - 1) // cfg.block_m
    assert full.numel() == 2 * m_blocks and full.dtype == torch.uint64


def test_sptrans_token_mask_matches_per_query_construction():
    for L, stride, c in [(256, 64, 16), (300, 64, 16), (200, 50, 60), (17, 4, 9), (100, 128, 32)]:
        want = torch.zeros(L, L, dtype=torch.bool)
        for q in range(L):
            qs = q // stride
            want[q, qs * stride:min((qs + 1) * stride, q + 1)] = True
            for ks in range(qs):
                lo, hi = ks * stride + stride - c, (ks + 1) * stride
                if lo < L and hi <= L:
                    want[q, lo:hi] = True
        assert torch.equal(sptrans_token_mask(L, stride, c)[0, 0], want)


def test_qwen_sanitize_quirk():
    # Bits beyond the last mask group are dropped.
    got = TQ.sanitize_precision_map(torch.tensor([0xFFFF, 0x3], dtype=torch.uint64), 256, 64)
    assert got.tolist() == [0xF, 0x3]
    # Every row exactly the highest valid bit -> all-INT8 rows.
    got = TQ.sanitize_precision_map(torch.tensor([0x8, 0x8, 0x8], dtype=torch.uint64), 256, 64)
    assert got.tolist() == [0xF] * 3
    # Not every row: unchanged.
    got = TQ.sanitize_precision_map(torch.tensor([0x8, 0x4], dtype=torch.uint64), 256, 64)
    assert got.tolist() == [0x8, 0x4]
    got = TQ.sanitize_precision_map(torch.tensor([2 ** 63], dtype=torch.uint64), 64 * 64, 64)
    assert got.tolist() == [2 ** 64 - 1]


def test_inject_qwen():
    cfg = Qwen2Config(vocab_size=96, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2)
    torch.manual_seed(0)
    model = Qwen2ForCausalLM(cfg).eval()
    before = {k: v.clone() for k, v in model.state_dict().items()}
    TQ.inject_tilemix_into_qwen(model)
    assert all(isinstance(l.self_attn, TQ.TileMixqwenAttention) for l in model.model.layers)
    for k, v in before.items():
        assert torch.equal(v, model.state_dict()[k]), k
    TQ.configure_tilemix_attention_pattern(model, "sptrans", percentage=0.25, stride=64, c=16)
    assert model.model.layers[0].self_attn.default_pattern_type == "sptrans"


def test_prefill_cache_keeps_first_update():
    cache = TL.PrefillCache()
    k = torch.randn(2, 2, 40, 16)
    v = torch.randn(2, 2, 40, 16)
    kk, vv = cache.update(k, v, 0)
    assert kk is k and vv is v
    k2 = torch.randn(2, 2, 1, 16)
    kk, vv = cache.update(k2, k2, 0)
    assert kk.shape[-2] == 41 and torch.equal(kk[..., :40, :], k)
    assert cache.get_seq_length(0) == 41


def test_rotary_oracle_matches_hf_fp16():
    """The oracle's split-half RoPE (the checker of the HIP kernel) equals
    transformers' apply_rotary_pos_emb on fp16 tensors bit for bit."""
    torch.manual_seed(1)
    b, hq, hk, t, d = 2, 4, 2, 37, 32
    q = torch.randn(b, hq, t, d).half()
    k = torch.randn(b, hk, t, d).half()
    pos = torch.arange(t, dtype=torch.float32)
    inv = 1.0 / (10000 ** (torch.arange(0, d, 2).float() / d))
    freqs = torch.outer(pos, inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = emb.cos().half()[None].expand(b, t, d).contiguous(), emb.sin().half()[None].expand(b, t, d).contiguous()
    oq, ok = PO.rotary_token_major(q, k, cos, sin)
    rq, rk = apply_rotary_pos_emb(q, k, cos, sin)
    assert torch.equal(oq, rq) and torch.equal(ok, rk)
    # token-major storage: the [b, h, t, d] view is a transpose of a dense [b, t, h, d]
    assert oq.transpose(1, 2).is_contiguous() and ok.transpose(1, 2).is_contiguous()


def test_rotary_product_validates_then_needs_gpu():
    q = torch.randn(1, 2, 8, 16).half()
    k = torch.randn(1, 1, 8, 16).half()
    cos = torch.randn(1, 8, 16).half()
    with pytest.raises(ValueError, match="FP16"):
        TL.rotary_token_major(q.float(), k, cos, cos)
    with pytest.raises(ValueError, match="split-half"):
        TL.rotary_token_major(q, k[..., :8], cos, cos)
    with pytest.raises(RuntimeError, match="GPU-only HIP kernel"):
        TL.rotary_token_major(q, k, cos, cos)


def test_silu_mul_oracle_matches_fp16_reference():
    torch.manual_seed(2)
    g = (torch.randn(64, 96) * 4).half()
    u = torch.randn(64, 96).half()
    want = (torch.nn.functional.silu(g.float()).half().float() * u.float()).half()
    assert torch.equal(PO.silu_mul(g, u), want)
    with pytest.raises(ValueError, match="equally shaped FP16"):
        TL.silu_mul(g, u[:, :10])
    with pytest.raises(RuntimeError, match="GPU-only HIP kernel"):
        TL.silu_mul(g, u)


def test_rms_norm_oracle_matches_llama_rmsnorm():
    """The oracle's RMSNorm equals transformers' LlamaRMSNorm run in fp16 on the
    CPU bit for bit (same formula and rounding points), and an fp64 evaluation
    of the formula to one fp16 ulp."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    torch.manual_seed(3)
    x = (torch.randn(33, 200) * 3).half()
    norm = LlamaRMSNorm(200, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(200) * 0.5 + 1.0)
    norm = norm.half()
    with torch.no_grad():
        want = norm(x)
    got = PO.rms_norm(x, norm.weight.detach(), 1e-5)
    assert torch.equal(got, want)
    xd = x.double()
    exact = norm.weight.double() * (xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-5)).half().double()
    ulp = torch.finfo(torch.float16).eps * exact.abs().clamp_min(2 ** -14)
    assert ((got.double() - exact).abs() <= ulp + 1e-12).all()
    with pytest.raises(ValueError, match="FP16"):
        TL.rms_norm(x.float(), norm.weight, 1e-5)
    with pytest.raises(RuntimeError, match="GPU-only HIP kernel"):
        TL.rms_norm(x, norm.weight.detach(), 1e-5)


def test_prepare_llama_prefill_checks_and_swaps():
    model = _tiny_llama()
    with pytest.raises(ValueError, match="inject TileMix attention before"):
        TL.prepare_llama_prefill(model)
    TL.inject_tilemix_into_llama(model)
    with pytest.raises(ValueError, match="FP16 model weights"):
        TL.prepare_llama_prefill(model)
    model = model.half()
    TL.prepare_llama_prefill(model)
    layer = model.model.layers[0]
    assert isinstance(layer.mlp, TL.PrefillMLP) and isinstance(layer.input_layernorm, TL.PrefillRMSNorm)
    assert layer.self_attn.apply_rotary is TL.rotary_token_major
    with pytest.raises(RuntimeError, match="GPU-only HIP kernel"):
        model.model.norm(torch.randn(3, 128).half())
    model.train()
    with pytest.raises(ValueError, match="eval-mode SiLU"):
        TL.prepare_llama_prefill(model)

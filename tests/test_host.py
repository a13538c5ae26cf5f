"""CPU tests of the host side: the C-ABI library (load, exported symbols,
struct layout, argument validation) and the Python mirror of the reference's
operator interface (routing classification, validation order, env knobs).

No test here launches a kernel: the C-ABI calls below fail argument
validation, which returns before any HIP call.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from tilemix_amd import _native
from tilemix_amd.attention.hip import tilemix as tmx
from tilemix_amd.attention.tilemix_varlen import tilemix_varlen_attention

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "tilemix_hip.h"


@pytest.fixture(scope="module")
def lib():
    if not _native.LIB_PATH.exists():
        from tilemix_amd.csrc import build
        build.build()
    return _native.load_library()


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tilemix_[a-z0-9_]+)\s*\(", text)))


# ------------------------------------------------------------------ C ABI
def test_header_declares_the_entry_points():
    names = _declared_functions()
    assert {"tilemix_quant_per_block_int8", "tilemix_attn_fwd", "tilemix_attn_fwd_debug",
            "tilemix_abi_version", "tilemix_params_size", "tilemix_last_error"} <= set(names)


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    assert sorted(_native.EXPORTED_SYMBOLS) == _declared_functions()


def test_abi_version_and_struct_layout(lib):
    abi = int(re.search(r"#define TILEMIX_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert lib.tilemix_abi_version() == abi == _native.ABI_VERSION
    assert lib.tilemix_params_size(0) == ctypes.sizeof(_native.QuantParams)
    assert lib.tilemix_params_size(1) == ctypes.sizeof(_native.AttnParams)
    assert lib.tilemix_params_size(2) == ctypes.sizeof(_native.RmsNormParams)
    assert lib.tilemix_params_size(3) == ctypes.sizeof(_native.RotaryParams)
    assert lib.tilemix_params_size(7) == -1


def test_ctypes_mirror_matches_header_field_order():
    text = HEADER.read_text()
    for struct, cls in (("tilemix_quant_params", _native.QuantParams), ("tilemix_attn_params", _native.AttnParams),
                        ("tilemix_rmsnorm_params", _native.RmsNormParams),
                        ("tilemix_rotary_params", _native.RotaryParams)):
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (struct, struct), text, re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            names = decl.split(None, 1)[1] if not decl.startswith("const") else decl.split(None, 2)[2]
            for n in names.replace("*", " ").split(","):
                fields.append(n.strip())
        assert [f[0] for f in cls._fields_] == fields


def test_null_params_are_rejected(lib):
    assert lib.tilemix_attn_fwd(None, None) == 1
    assert b"null params" in lib.tilemix_last_error()
    assert lib.tilemix_quant_per_block_int8(None, None) == 1
    assert lib.tilemix_attn_fwd_debug(None, None, None, 0, 0, None) == 1


def test_attn_validation_messages(lib):
    p = _native.AttnParams()
    assert lib.tilemix_attn_fwd(ctypes.byref(p), None) == 1
    assert b"null q/k/v/out" in lib.tilemix_last_error()
    dummy = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    for f in ("q", "k", "v", "out", "cu_seqlens_q", "cu_seqlens_k"):
        setattr(p, f, dummy)
    p.routing_mode, p.heads_q, p.heads_k, p.head_dim = 5, 4, 1, 64
    assert lib.tilemix_attn_fwd(ctypes.byref(p), None) == 1
    assert b"routing_mode" in lib.tilemix_last_error()
    p.routing_mode, p.heads_q, p.heads_k = 1, 3, 2
    assert lib.tilemix_attn_fwd(ctypes.byref(p), None) == 1
    assert b"multiple of KV heads" in lib.tilemix_last_error()
    p.heads_q, p.heads_k, p.head_dim = 4, 1, 72
    assert lib.tilemix_attn_fwd(ctypes.byref(p), None) == 1
    assert b"head_dim" in lib.tilemix_last_error()
    p.head_dim, p.block_m, p.block_n, p.block_n_mask = 64, 32, 64, 64
    assert lib.tilemix_attn_fwd(ctypes.byref(p), None) == 1
    assert b"block_m" in lib.tilemix_last_error()
    p.block_m, p.max_seqlen_q, p.max_seqlen_k = 128, 8192, 8192
    assert lib.tilemix_attn_fwd(ctypes.byref(p), None) == 1
    assert b"exceeds 64 mask blocks" in lib.tilemix_last_error()
    p.max_seqlen_q = p.max_seqlen_k = 256
    p.routing_mode = 0
    assert lib.tilemix_attn_fwd(ctypes.byref(p), None) == 1
    assert b"precision_bitmask" in lib.tilemix_last_error()
    p.precision_bitmask = dummy
    assert lib.tilemix_attn_fwd(ctypes.byref(p), None) == 1
    assert b"int8 routing needs" in lib.tilemix_last_error()
    # A short sequence with a huge token stride: the lane offsets of one
    # 64-key tile (not just max_seqlen_k rows) must fit the 32-bit buffer range.
    p.routing_mode = 1
    p.max_seqlen_q = p.max_seqlen_k = 4
    aligned_dummy = ctypes.c_void_p(1 << 12)
    for f in ("q", "k", "v", "out"):
        setattr(p, f, aligned_dummy)
    p.stride_k_token = p.stride_v_token = 1 << 25  # 64 MiB per token
    assert lib.tilemix_attn_fwd(ctypes.byref(p), None) == 1
    assert b"exceeds 2 GiB" in lib.tilemix_last_error()
    # In-kernel Q quantisation needs 128-row workgroups: block_m 64 with mixed
    # routing on int8 V codes runs 64-row workgroups.
    p.stride_k_token = p.stride_v_token = 128
    p.routing_mode, p.block_m, p.blkq, p.blkk = 0, 64, 128, 64
    p.q_quant_in_kernel, p.int8_use_fp16_v = 1, 0
    assert lib.tilemix_attn_fwd(ctypes.byref(p), None) == 1
    assert b"128-row workgroups" in lib.tilemix_last_error()
    p.blkq = 64
    assert lib.tilemix_attn_fwd(ctypes.byref(p), None) == 1
    assert b"128-row workgroups" in lib.tilemix_last_error()


def test_quant_validation_messages(lib):
    p = _native.QuantParams()
    assert lib.tilemix_quant_per_block_int8(ctypes.byref(p), None) == 1
    assert b"null tensor pointer" in lib.tilemix_last_error()
    dummy = ctypes.c_void_p(16)
    p.input = p.output = p.scale = p.cu_seqlens = dummy
    p.heads, p.batch, p.blk_tokens, p.head_dim = 2, 1, 64, 12
    assert lib.tilemix_quant_per_block_int8(ctypes.byref(p), None) == 1
    assert b"head_dim" in lib.tilemix_last_error()


def test_prefill_helper_validation_messages(lib):
    assert lib.tilemix_rms_norm_f16(None, None) == 1
    assert b"null params" in lib.tilemix_last_error()
    assert lib.tilemix_rotary_f16(None, None) == 1
    assert b"null params" in lib.tilemix_last_error()
    assert lib.tilemix_silu_mul_f16(None, None, None, 4, None) == 1
    assert b"null tensor pointer" in lib.tilemix_last_error()
    dummy = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    assert lib.tilemix_silu_mul_f16(dummy, dummy, dummy, -1, None) == 1
    assert lib.tilemix_silu_mul_f16(dummy, dummy, dummy, 0, None) == 0  # nothing to do
    p = _native.RmsNormParams()
    assert lib.tilemix_rms_norm_f16(ctypes.byref(p), None) == 1
    assert b"null tensor pointer" in lib.tilemix_last_error()
    p.x = p.weight = p.out = dummy
    p.rows, p.cols, p.stride_x, p.stride_out, p.eps = 4, 64, 32, 64, 1e-6
    assert lib.tilemix_rms_norm_f16(ctypes.byref(p), None) == 1
    assert b"invalid shape" in lib.tilemix_last_error()
    r = _native.RotaryParams()
    assert lib.tilemix_rotary_f16(ctypes.byref(r), None) == 1
    assert b"null tensor pointer" in lib.tilemix_last_error()
    r.q = r.k = r.cos = r.sin = r.q_out = r.k_out = dummy
    r.batch, r.tokens, r.heads_q, r.heads_k, r.head_dim = 1, 8, 2, 1, 15
    assert lib.tilemix_rotary_f16(ctypes.byref(r), None) == 1
    assert b"invalid shape" in lib.tilemix_last_error()


# ------------------------------------------------------- host-side logic
def _brute_classify(rows, seqlen_q, seqlen_k, block_m, block_n, block_n_mask, causal):
    m_blocks = -(-seqlen_q // block_m)
    n_tiles = -(-seqlen_k // block_n)
    g = block_n_mask // block_n
    seen = set()
    for r, raw in enumerate(rows):
        m = r % m_blocks
        nb = n_tiles
        if causal:
            nb = max(0, min(n_tiles, -(-((m + 1) * block_m + seqlen_k - seqlen_q) // block_n)))
        for n in range(nb):
            seen.add((int(raw) >> (n // g)) & 1)
    if seen == {1}:
        return "int8"
    if 1 not in seen:
        return "fp16"
    return "mixed"


@pytest.mark.parametrize("seed", range(6))
def test_classify_bitmask_routing_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    L = int(rng.integers(64, 1500))
    bm, bn = (64, 64) if seed % 2 else (128, 64)
    bnm = bn * int(rng.choice([1, 2]))
    hk = int(rng.integers(1, 3))
    m_blocks = -(-L // bm)
    kind = seed % 3
    legal = [(1 << -(-min(-(-L // bn), -(-((m + 1) * bm) // bn)) // (bnm // bn))) - 1 for m in range(m_blocks)]
    if kind == 0:
        rows = [int(rng.integers(0, 2 ** 63)) for _ in range(hk * m_blocks)]
    elif kind == 1:
        rows = [legal[r % m_blocks] | (int(rng.integers(0, 2 ** 20)) << 40) for r in range(hk * m_blocks)]
    else:
        rows = [int(rng.integers(0, 2 ** 20)) << 44 for _ in range(hk * m_blocks)]
    t = torch.tensor(rows, dtype=torch.uint64)
    got = tmx.classify_bitmask_routing(t, seqlen_q=L, seqlen_k=L, block_m=bm, block_n=bn, block_n_mask=bnm,
                                       causal=True)
    assert got == _brute_classify(rows, L, L, bm, bn, bnm, True)


def test_routing_mode_names():
    assert tmx._routing_mode_code(" Mixed ") == 0
    assert tmx._routing_mode_code("FP16") == 1 and tmx._routing_mode_code("int8") == 2
    with pytest.raises(ValueError, match="routing_mode must be one of"):
        tmx._routing_mode_code("bf16")


def test_forced_config(monkeypatch):
    monkeypatch.setenv("TILEMIX_FORCE_CONFIG", "128,64,8,2")
    tmx._forced_config_check(128, 64)
    with pytest.raises(ValueError, match="TILEMIX_FORCE_CONFIG block sizes must match"):
        tmx._forced_config_check(64, 64)


def test_launch_requires_gpu_tensors():
    q = torch.zeros(64, 2, 64, dtype=torch.float16)
    k = torch.zeros(64, 1, 64, dtype=torch.float16)
    cu = torch.tensor([0, 64], dtype=torch.int32)
    bm = torch.zeros(1, dtype=torch.uint64)
    with pytest.raises(RuntimeError, match="GPU-only"):
        tmx.tilemix_attention_with_quant(q, k, k, cu, cu, 64, 64, bm, block_m=64, block_n=64, causal=True,
                                         routing_mode="mixed")


def test_mismatched_head_dims_are_rejected_before_padding(monkeypatch):
    """q with head_dim 72 and k/v with 64 (or K != V): the reference's
    ValueError, raised before the head-dim padding (which would pad all three
    to 80 and let them pass) and before any launch."""
    calls = []
    monkeypatch.setattr(tmx, "launch_prequantized", lambda *a, **kw: calls.append(1))
    cu = torch.tensor([0, 64], dtype=torch.int32)
    bm = torch.zeros(1, dtype=torch.uint64)
    q = torch.zeros(64, 2, 72, dtype=torch.float16)
    k = torch.zeros(64, 1, 64, dtype=torch.float16)
    kw = dict(block_m=64, block_n=64, causal=True, routing_mode="fp16")
    with pytest.raises(ValueError, match="K/V shapes and Q/K/V head dimensions must match"):
        tmx.tilemix_attention_with_quant(q, k, k, cu, cu, 64, 64, bm, **kw)
    with pytest.raises(ValueError, match="K/V shapes and Q/K/V head dimensions must match"):
        tmx.tilemix_attention_with_quant(q, q[:, :1], q[:, :1, :64], cu, cu, 64, 64, bm, **kw)
    with pytest.raises(ValueError, match="expected flattened"):
        tmx.tilemix_attention_with_quant(q[None], k, k, cu, cu, 64, 64, bm, **kw)
    assert not calls


def test_wide_token_strides_get_a_head_major_copy():
    """The kernel reads (max_seqlen_k + 64) K/V token strides (and 128 Q token
    strides) through one 32-bit buffer: a view whose span reaches 2 GiB is
    replaced by a head-major copy of the same values (token stride head_dim),
    any other tensor is passed through as is."""
    small = torch.zeros(10, 2, 16, dtype=torch.float16)
    assert tmx._token_stride_fit(small, 1000) is small
    base = torch.arange(4 * (1 << 20), dtype=torch.float16).view(4, 1 << 20)
    view = base.as_strided((4, 2, 16), (1 << 20, 16, 1), 32)  # 2 MiB token stride
    assert not tmx._span_fits(view, 1024)
    fit = tmx._token_stride_fit(view, 1024)
    assert fit.stride() == (16, 64, 1) and torch.equal(fit, view)
    assert tmx._span_fits(fit, 1024)
    assert tmx._token_stride_fit(view, 1000) is view  # 1000 rows of 2 MiB stay below 2 GiB


def test_varlen_entry_validates_before_launch():
    q = torch.zeros(1, 4, 256, 64, dtype=torch.float16)
    k = torch.zeros(1, 1, 256, 64, dtype=torch.float16)
    pm = torch.zeros(4, dtype=torch.uint64)
    kw = dict(causal=True, scale=0.125, candidates=[(64, 64)], flat_lengths=[4])
    with pytest.raises(AssertionError, match="precision_map dtype must be uint64"):
        tilemix_varlen_attention(q, k, k, 64, 64, precision_map_all=pm.to(torch.int64), **kw)
    with pytest.raises(ValueError, match="must be a multiple of block_n"):
        tilemix_varlen_attention(q, k, k, 64, 64, block_n_mask=96, precision_map_all=pm, **kw)
    with pytest.raises(AssertionError, match="precision_map length mismatch"):
        tilemix_varlen_attention(q, k, k, 64, 64, precision_map_all=pm[:3], **kw)
    with pytest.raises(ValueError, match="Tq .* != Tk"):
        tilemix_varlen_attention(q[:, :, :128], k, k, 64, 64, precision_map_all=pm[:2], **kw)
    with pytest.raises(AssertionError, match="head dims differ"):
        tilemix_varlen_attention(q[..., :32], k, k, 64, 64, precision_map_all=pm, **kw)
    with pytest.raises(ValueError, match="Bias shape mismatch"):
        tilemix_varlen_attention(q, k, k, 64, 64, precision_map_all=pm, bias=torch.zeros(1, 4, 256, 255), **kw)


def test_q_in_kernel_rule():
    """In-kernel Q quantisation needs a 128-row workgroup that is one BLKQ = 128
    block: block_m 128, or block_m 64 unless mixed routing runs on int8 V codes."""
    mixed, int8 = tmx.ROUTING_MODE_MIXED, tmx.ROUTING_MODE_INT8
    assert tmx._q_in_kernel_supported(128, 128, mixed, False)
    assert tmx._q_in_kernel_supported(64, 128, mixed, True)
    assert tmx._q_in_kernel_supported(64, 128, int8, False)
    assert not tmx._q_in_kernel_supported(64, 128, mixed, False)
    assert not tmx._q_in_kernel_supported(128, 64, mixed, True)


def test_int8_views_are_copied_to_16_byte_strides():
    """q8/k8/v8 are streamed as 16-byte vectors: a view whose token or head
    stride is not a multiple of 16 bytes (here 8 mod 16) is replaced by a dense
    copy, an aligned one is passed through (the C layer rejects other strides)."""
    base = torch.zeros(10, 3, 136, dtype=torch.int8)
    view = base[..., :128]
    assert view.stride(1) % 16 == 8
    fixed = tmx._inner_contiguous(view, 16)
    assert fixed.stride(0) % 16 == 0 and fixed.stride(1) % 16 == 0 and fixed.is_contiguous()
    aligned = torch.zeros(10, 3, 144, dtype=torch.int8)[..., :128]
    assert tmx._inner_contiguous(aligned, 16) is aligned
    src = (Path(tmx.__file__)).read_text()
    # every int8 operand goes through the 16-byte rule before the launch
    assert "_inner_contiguous(v8, 16)" in src and "_inner_contiguous(k8, 16)" in src
    assert "_inner_contiguous(q8, 16)" in src


def test_auto_routing_classification_is_cached_per_tensor_version(monkeypatch):
    """routing_mode='auto' reads a bitmask back to the host once per tensor
    and version: the same tensor again is not re-read, an in-place change or
    another tensor with other bits is."""
    calls = []
    real = tmx.classify_bitmask_routing

    def counting(t, **kw):
        calls.append(1)
        return real(t, **kw)

    monkeypatch.setattr(tmx, "classify_bitmask_routing", counting)
    kw = dict(seqlen_q=256, seqlen_k=256, block_m=128, block_n=64, block_n_mask=64, causal=True)
    bm = torch.zeros(4, dtype=torch.uint64)
    assert tmx._classify_cached(bm, **kw) == "fp16"
    assert tmx._classify_cached(bm, **kw) == "fp16"
    assert len(calls) == 1
    bm.fill_(0xF)  # in place: version counter moves
    assert tmx._classify_cached(bm, **kw) == "int8"
    assert len(calls) == 2
    other = torch.tensor([1, 0, 1, 0], dtype=torch.uint64)
    assert tmx._classify_cached(other, **kw) == "mixed"
    assert tmx._classify_cached(bm, **{**kw, "causal": False}) == real(bm, **{**kw, "causal": False})
    assert len(calls) == 4


def test_placeholder_metadata_shapes_and_sharing():
    """The all-FP16 / fp16-V placeholders keep the reference's shapes, dtypes
    and zero scale prefixes (attention/triton/tilemix.py:1087-1129), and are
    created once: a second call returns the same tensors (no fill per call)."""
    q = torch.zeros((300, 6, 128), dtype=torch.float16)
    k = torch.zeros((300, 2, 128), dtype=torch.float16)
    cu = torch.tensor([0, 100, 300], dtype=torch.int32)
    v8, sv, cuv = tmx._dummy_v_quantization_metadata(k, cu)
    assert v8.shape == (1, 2, 128) and v8.dtype == torch.int8
    assert sv.shape == (1, 2) and sv.dtype == torch.float16
    assert cuv.shape == cu.shape and cuv.dtype == torch.int32 and not cuv.any()
    again = tmx._dummy_v_quantization_metadata(k, cu)
    assert all(a is b for a, b in zip((v8, sv, cuv), again))
    q8, sq, cuq, k8, sk, cuk, v8b, svb, cuvb = tmx._dummy_quantization_metadata(q, k, k, cu, cu)
    assert q8.shape == (1, 6, 128) and k8.shape == (1, 2, 128) and v8b.shape == (1, 2, 128)
    assert sq.shape == (1, 6) and sk.shape == (1, 2) and svb.shape == (1, 2)
    assert all(t.dtype == torch.int32 and t.shape == cu.shape and not t.any() for t in (cuq, cuk, cuvb))
    other = tmx._dummy_v_quantization_metadata(k, torch.tensor([0, 300], dtype=torch.int32))
    assert other[2].shape == (2,) and other[2] is not cuv

"""GPU tests of the public drop-in surface around the kernel: the quantisation
functions a caller imports directly, and operands that are strided views.

* ``per_block_int8`` / ``per_block_int8_single`` (reference
  attention/triton/quant_per_block_varlen.py:48-106), ``quantize_qk_for_tilemix``
  and ``quantize_qkv_for_tilemix`` (attention/triton/tilemix.py:45-156):
  codes and scales bit-exact against the oracle, the returned tuple order and
  dtypes of the reference, the ``q_sm_scale = sm_scale * 1.44269504`` rule
  (sm_scale None, 1.0 and another value), ragged / empty / one-token
  sequences, cu_seqlens on the host and on the device.
* head_dim 80 as ``[..., :80]`` views of 128-wide buffers whose other columns
  hold NaN and Inf: the kernels read no column past head_dim (every kernel
  variant and routing), outputs equal the oracle on the dense data.
* int8 V codes passed as a view whose head stride is 8 mod 16 bytes.
"""
import numpy as np
import pytest
import torch

from oracle import tilemix_oracle as O
from tests._helpers import assert_close_out, bitmask_tensor, packed_inputs, random_bitmask, to_dev
from tilemix_amd.attention.hip import tilemix as tmx
from tilemix_amd.attention.hip.quant_per_block_varlen import per_block_int8, per_block_int8_single

pytestmark = pytest.mark.gpu

LENGTHS = [300, 0, 77, 1, 128]


def _q_sm_scale(sm_scale, d):
    """The Q multiplier per_block_int8 applies (reference quant_per_block_varlen.py:84-88)."""
    if sm_scale is None:
        sm_scale = d ** -0.5
    return 1.0 if abs(sm_scale - 1.0) < 1e-6 else sm_scale * 1.44269504


def _same_codes(got, ref, cu):
    g = got.cpu().numpy()
    for b in range(len(cu) - 1):  # tokens outside sequences are not written
        np.testing.assert_array_equal(g[cu[b]:cu[b + 1]], ref[cu[b]:cu[b + 1]])


@pytest.mark.parametrize("host_cu", [False, True], ids=["cu_device", "cu_host"])
@pytest.mark.parametrize("sm_scale", [None, 1.0, 0.3])
def test_per_block_int8(device, sm_scale, host_cu):
    d = 64
    q, k, _, cu = packed_inputs(LENGTHS, 4, 2, d, seed=51, outliers=(3, 17))
    cu_t = torch.from_numpy(cu) if host_cu else to_dev(cu, device)
    out = per_block_int8(to_dev(q, device), to_dev(k, device), cu_t, cu_t, max(LENGTHS), max(LENGTHS),
                         BLKQ=128, BLKK=64, sm_scale=sm_scale)
    q8, qs, k8, ks, cuqs, cuks = out
    rq8, rqs, rcuq = O.quant_per_block_int8(q, cu, 128, sm_scale=_q_sm_scale(sm_scale, d))
    rk8, rks, rcuk = O.quant_per_block_int8(k, cu, 64, sm_scale=1.0)
    torch.cuda.synchronize()
    assert q8.dtype == k8.dtype == torch.int8
    assert qs.dtype == ks.dtype == torch.float32
    assert cuqs.dtype == cuks.dtype == torch.int64
    assert tuple(qs.shape) == rqs.shape and tuple(ks.shape) == rks.shape
    assert cuqs.cpu().tolist() == rcuq.tolist() and cuks.cpu().tolist() == rcuk.tolist()
    _same_codes(q8, rq8, cu)
    _same_codes(k8, rk8, cu)
    np.testing.assert_array_equal(qs.cpu().numpy().view(np.uint32), rqs.view(np.uint32))
    np.testing.assert_array_equal(ks.cpu().numpy().view(np.uint32), rks.view(np.uint32))


def test_per_block_int8_single_blk_and_scale(device):
    x, _, _, cu = packed_inputs([65, 0, 257], 3, 1, 128, seed=52)
    for blk, sm in ((64, 1.0), (128, 0.7), (256, 1.44269504 * 0.125)):
        codes, scale, cus = per_block_int8_single(to_dev(x, device), to_dev(cu, device), 257, BLK=blk, sm_scale=sm)
        rc, rs, rcu = O.quant_per_block_int8(x, cu, blk, sm_scale=sm)
        torch.cuda.synchronize()
        assert cus.dtype == torch.int64 and cus.cpu().tolist() == rcu.tolist()
        _same_codes(codes, rc, cu)
        np.testing.assert_array_equal(scale.cpu().numpy().view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("sm_scale", [None, 0.5])
def test_quantize_qk_for_tilemix(device, sm_scale):
    """Quantised with sm_scale = 1 whatever sm_scale is (reference :126-140);
    scales cast to q.dtype, cu arrays to int32; tuple (q8, sq, cuq, k8, sk, cuk)."""
    d = 128
    q, k, _, cu = packed_inputs(LENGTHS, 4, 2, d, seed=53, outliers=(1, 9))
    res = tmx.quantize_qk_for_tilemix(to_dev(q, device), to_dev(k, device), to_dev(cu, device), to_dev(cu, device),
                                      max(LENGTHS), max(LENGTHS), BLKQ=128, BLKK=64, sm_scale=sm_scale)
    assert len(res) == 6
    q8, sq, cuq, k8, sk, cuk = res
    rq8, rqs, rcuq = O.quant_per_block_int8(q, cu, 128)
    rk8, rks, rcuk = O.quant_per_block_int8(k, cu, 64)
    torch.cuda.synchronize()
    assert (q8.dtype, sq.dtype, cuq.dtype) == (torch.int8, torch.float16, torch.int32)
    assert (k8.dtype, sk.dtype, cuk.dtype) == (torch.int8, torch.float16, torch.int32)
    assert all(t.is_contiguous() for t in res)
    _same_codes(q8, rq8, cu)
    _same_codes(k8, rk8, cu)
    np.testing.assert_array_equal(sq.cpu().numpy().view(np.uint16), rqs.astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(sk.cpu().numpy().view(np.uint16), rks.astype(np.float16).view(np.uint16))
    assert cuq.cpu().tolist() == rcuq.tolist() and cuk.cpu().tolist() == rcuk.tolist()


def test_quantize_qkv_for_tilemix_feeds_launch_prequantized(device):
    """The 9-tuple (q8, sq, cuq, k8, sk, cuk, v8, sv, cuv) with V quantised per
    BLKK keys, bit-exact; passed to launch_prequantized with int8 V codes it
    gives the oracle's output (the caller-side pre-quantised path)."""
    lengths, hq, hk, d = [300, 0, 77, 1, 128], 4, 2, 128
    q, k, v, cu = packed_inputs(lengths, hq, hk, d, seed=54)
    dq, dk, dv, dcu = (to_dev(x, device) for x in (q, k, v, cu))
    res = tmx.quantize_qkv_for_tilemix(dq, dk, dv, dcu, dcu, max(lengths), max(lengths), BLKQ=128, BLKK=64)
    assert len(res) == 9
    q8, sq, cuq, k8, sk, cuk, v8, sv, cuv = res
    rv8, rvs, rcuv = O.quant_per_block_int8(v, cu, 64)
    torch.cuda.synchronize()
    assert (v8.dtype, sv.dtype, cuv.dtype) == (torch.int8, torch.float16, torch.int32)
    _same_codes(v8, rv8, cu)
    np.testing.assert_array_equal(sv.cpu().numpy().view(np.uint16), rvs.astype(np.float16).view(np.uint16))
    assert cuv.cpu().tolist() == rcuv.tolist()
    bits = random_bitmask(hk, -(-max(lengths) // 128), seed=54)
    out, mode = tmx.launch_prequantized(dq, dk, dv, dcu, dcu, max(lengths), max(lengths), bitmask_tensor(bits, device),
                                        q8=q8, k8=k8, v8=v8, sQ_blocks=sq, sK_blocks=sk, sV_blocks=sv,
                                        cu_q_scale=cuq, cu_k_scale=cuk, cu_v_scale=cuv, block_m=128, block_n=64,
                                        causal=True, routing_mode="mixed", int8_use_fp16_v=False)
    assert mode == "mixed"
    rq8, rqs, rcuq = O.quant_per_block_int8(q, cu, 128)
    rk8, rks, rcuk = O.quant_per_block_int8(k, cu, 64)
    ref = O.attn_fwd(q, k, v, cu, cu, bits, block_m=128, block_n_mask=64, causal=True, q8=rq8, k8=rk8,
                     sq16=rqs.astype(np.float16), sk16=rks.astype(np.float16), cu_q_scale=rcuq, cu_k_scale=rcuk,
                     int8_use_fp16_v=False, v8=rv8, sv16=rvs.astype(np.float16), cu_v_scale=rcuv)
    assert_close_out(out.cpu().numpy(), ref)


# --------------------------------------------- head_dim < tile width, padded views
# block_m, routing mode, int8_use_fp16_v: covers the 32-row kernel (block_m 128,
# and 64 in split and plain workgroups) and the 16-row kernel (block_m 64, mixed
# routing on int8 V codes).
PAD_CASES = [(128, "fp16", True), (128, "int8", True), (128, "mixed", True), (128, "mixed", False),
             (64, "mixed", True), (64, "mixed", False), (64, "int8", False)]


def _padded_view(x: np.ndarray, device, width=128):
    """x [N, H, d] as the first d columns of an fp16 [N, H, width] buffer whose
    remaining columns alternate NaN and +Inf."""
    n, h, d = x.shape
    buf = torch.empty((n, h, width), dtype=torch.float16)
    buf[..., d::2] = float("nan")
    buf[..., d + 1::2] = float("inf")
    buf[..., :d] = torch.from_numpy(x)
    return buf.to(device)[..., :d]


@pytest.mark.parametrize("block_m,mode,int8v", PAD_CASES)
def test_head_dim_80_views_with_nan_padding(device, block_m, mode, int8v):
    lengths, hq, hk, d = [130, 63, 1], 6, 3, 80
    q, k, v, cu = packed_inputs(lengths, hq, hk, d, seed=61)
    dq, dk, dv = (_padded_view(x, device) for x in (q, k, v))
    assert dk.stride(1) == 128 and not dk.is_contiguous()
    bits = random_bitmask(hk, -(-max(lengths) // block_m), seed=61)
    print(f"block_m {block_m} mode {mode} int8_use_fp16_v {int8v}", flush=True)
    out, _ = tmx.tilemix_attention_with_quant(
        dq, dk, dv, to_dev(cu, device), to_dev(cu, device), max(lengths), max(lengths), bitmask_tensor(bits, device),
        block_m=block_m, block_n=64, block_n_mask=64, BLKQ=128, BLKK=64, causal=True, routing_mode=mode,
        scalar_scales=(block_m == 128), int8_use_fp16_v=int8v)
    q8, sq, cuq = O.quant_per_block_int8(q, cu, 128)
    k8, sk, cuk = O.quant_per_block_int8(k, cu, 64)
    extra = {}
    if not int8v:
        v8, sv, cuv = O.quant_per_block_int8(v, cu, 64)
        extra = dict(v8=v8, sv16=sv.astype(np.float16), cu_v_scale=cuv)
    ref = O.attn_fwd(q, k, v, cu, cu, bits, block_m=block_m, block_n_mask=64, causal=True,
                     routing_mode={"mixed": 0, "fp16": 1, "int8": 2}[mode], q8=q8, k8=k8,
                     sq16=sq.astype(np.float16), sk16=sk.astype(np.float16), cu_q_scale=cuq, cu_k_scale=cuk,
                     int8_use_fp16_v=int8v, **extra)
    assert_close_out(out.cpu().numpy(), ref)


def test_int8_v_view_with_8_mod_16_head_stride(device):
    """v8 given as [..., :128] of a 136-wide int8 buffer (head stride 8 mod 16):
    the host takes a dense copy before the launch, results equal the dense call."""
    lengths, hq, hk, d = [200, 70], 4, 2, 128
    q, k, v, cu = packed_inputs(lengths, hq, hk, d, seed=62)
    dq, dk, dv, dcu = (to_dev(x, device) for x in (q, k, v, cu))
    q8, sq, cuq, k8, sk, cuk, v8, sv, cuv = tmx.quantize_qkv_for_tilemix(dq, dk, dv, dcu, dcu, 200, 200)
    wide = torch.full((v8.shape[0], hk, 136), 77, dtype=torch.int8, device=device)
    wide[..., :128] = v8
    v8_view = wide[..., :128]
    assert v8_view.stride(1) % 16 == 8
    bits = bitmask_tensor(random_bitmask(hk, 2, seed=62), device)
    kw = dict(q8=q8, k8=k8, sQ_blocks=sq, sK_blocks=sk, sV_blocks=sv, cu_q_scale=cuq, cu_k_scale=cuk,
              cu_v_scale=cuv, block_m=128, block_n=64, causal=True, routing_mode="mixed", int8_use_fp16_v=False)
    o_dense, _ = tmx.launch_prequantized(dq, dk, dv, dcu, dcu, 200, 200, bits, v8=v8, **kw)
    o_view, _ = tmx.launch_prequantized(dq, dk, dv, dcu, dcu, 200, 200, bits, v8=v8_view, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o_dense, o_view)

"""TileMix fused FP16/INT8 prefill attention: host launch layer over libtilemix_hip.so.

Drop-in for the host half of the reference's attention/triton/tilemix.py: the
same public names, arguments, return values and validation errors --

* ``quantize_qkv_for_tilemix`` (reference :45-107)
* ``quantize_qk_for_tilemix`` (:110-156)
* ``classify_bitmask_routing`` (:968-1014)
* ``launch_prequantized`` (:1132-1337)
* ``tilemix_attention_with_quant`` (:1340-1447)
* ``ROUTING_MODE_MIXED / FP16 / INT8`` (:159-161)

-- while the device work is one hand-written gfx950 kernel reached through the
C ABI (include/tilemix_hip.h); there is no Triton and no CPU fallback.

Differences that do not change results:
* a head_dim that is not a multiple of 16 is zero-padded to the next multiple
  of 16 on the host (Q, K, V and their int8 codes) and the output is copied
  back at the original width: zero columns add 0 to every dot product and do
  not change a block's max|x|, where the reference masks the columns past
  head_dim inside the kernel (:252, :364, :639); sm_scale defaults to
  head_dim ** -0.5 of the original width;
* the scale tensors used inside ``tilemix_attention_with_quant`` are sized
  from the token count (no device->host read of the scale-row count);
* Triton's autotune table is replaced by a fixed gfx950 tiling, so
  ``TILEMIX_FORCE_CONFIG`` only keeps its block-size consistency check;
* ``run_length`` and ``int8_cache_ca`` are accepted: run-length merging only
  regroups identical per-tile routes (same tiles, same order) and the cache
  modifier has no numeric effect;
* ``routing_mode="auto"`` classifies a bitmask tensor once and reuses the
  result while the tensor and its version counter are unchanged (the
  reference reads the map back to the host, waiting for the GPU, on every
  call).
"""
from __future__ import annotations

import os
import weakref
from typing import Literal, Optional

import torch

from ... import _native
from .quant_per_block_varlen import per_block_int8 as quant_per_block_int8
from .quant_per_block_varlen import per_block_int8_single, quantize_blocks

LOG2E = 1.4426950408889634

ROUTING_MODE_MIXED = _native.ROUTING_MIXED
ROUTING_MODE_FP16 = _native.ROUTING_FP16
ROUTING_MODE_INT8 = _native.ROUTING_INT8
RoutingMode = Literal["auto", "mixed", "fp16", "int8"]

# Tile sizes the gfx950 kernel is instantiated for (block_n > 64 runs as
# 64-key tiles with the reference's per-block_n softmax step).
SUPPORTED_BLOCK_M = (64, 128, 256, 512)
SUPPORTED_BLOCK_N = (64, 128, 256)
# The kernel's head-dim granularity; other widths are zero-padded to it.
HEAD_DIM_MULTIPLE = 16


def _scale_dtype(dtype: torch.dtype) -> torch.dtype:
    if dtype == torch.float16:
        return torch.float16
    if dtype == torch.bfloat16:
        return torch.bfloat16
    return torch.float32


@torch.no_grad()
def quantize_qkv_for_tilemix(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                             BLKQ: int = 128, BLKK: int = 64, sm_scale: float = None):
    """Reference attention/triton/tilemix.py:45-107 (Q, K and V quantised with sm_scale=1)."""
    q8, sq, k8, sk, cuq, cuk = quant_per_block_int8(
        q, k, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
        BLKQ=BLKQ, BLKK=BLKK, sm_scale=1.0)
    v8, sv, cuv = per_block_int8_single(v, cu_seqlens_k, max_seqlen_k, BLK=BLKK, sm_scale=1.0)
    sdt = _scale_dtype(q.dtype)
    return (
        q8, sq.to(dtype=sdt).contiguous(), cuq.to(dtype=torch.int32).contiguous(),
        k8, sk.to(dtype=sdt).contiguous(), cuk.to(dtype=torch.int32).contiguous(),
        v8, sv.to(dtype=sdt).contiguous(), cuv.to(dtype=torch.int32).contiguous(),
    )


@torch.no_grad()
def quantize_qk_for_tilemix(q, k, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                            BLKQ: int = 128, BLKK: int = 64, sm_scale: float = None):
    """Reference attention/triton/tilemix.py:110-156."""
    q8, sq, k8, sk, cuq, cuk = quant_per_block_int8(
        q, k, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
        BLKQ=BLKQ, BLKK=BLKK, sm_scale=1.0)
    sdt = _scale_dtype(q.dtype)
    return (
        q8.contiguous(), sq.to(dtype=sdt).contiguous(), cuq.to(dtype=torch.int32).contiguous(),
        k8.contiguous(), sk.to(dtype=sdt).contiguous(), cuk.to(dtype=torch.int32).contiguous(),
    )


def _quantize_for_launch(t: torch.Tensor, cu: torch.Tensor, max_seqlen: int, blk: int):
    """No-sync quantisation with fp16 scales written by the kernel itself."""
    codes, _, scale16, cu_scale = quantize_blocks(t, cu, max_seqlen, blk, 1.0, half_scales=True)
    return codes, scale16, cu_scale


def _routing_mode_code(mode: str) -> int:
    normalized = mode.strip().lower()
    codes = {"mixed": ROUTING_MODE_MIXED, "fp16": ROUTING_MODE_FP16, "int8": ROUTING_MODE_INT8}
    if normalized not in codes:
        raise ValueError(f"routing_mode must be one of {tuple(codes)}, got {mode!r}")
    return codes[normalized]


def classify_bitmask_routing(precision_bitmask: torch.Tensor, *, seqlen_q: int, seqlen_k: int,
                             block_m: int, block_n: int, block_n_mask: int,
                             causal: bool) -> Literal["mixed", "fp16", "int8"]:
    """Reference attention/triton/tilemix.py:968-1014.

    A row counts only its causally executed groups; the map is ``fp16`` if no
    such group is routed to INT8, ``int8`` if all of them are, else ``mixed``.
    """
    if block_n_mask % block_n != 0:
        raise ValueError("block_n_mask must be a multiple of block_n")
    m_blocks = (seqlen_q + block_m - 1) // block_m
    compute_blocks = (seqlen_k + block_n - 1) // block_n
    mask_group = block_n_mask // block_n
    host_masks = precision_bitmask.detach().reshape(-1).cpu().tolist()
    if len(host_masks) == 0 or len(host_masks) % m_blocks:
        raise ValueError("precision_bitmask has an invalid row count")
    # Groups executed by query block j (identical for every KV head).
    valid = []
    for query_block in range(m_blocks):
        row_blocks = compute_blocks
        if causal:
            numerator = (query_block + 1) * block_m + seqlen_k - seqlen_q
            row_blocks = max(0, min(compute_blocks, (numerator + block_n - 1) // block_n))
        route_blocks = (row_blocks + mask_group - 1) // mask_group
        valid.append((1 << route_blocks) - 1 if route_blocks else 0)
    any_int8 = any_fp16 = False
    for row, raw in enumerate(host_masks):
        vm = valid[row % m_blocks]
        routed = int(raw) & vm
        any_int8 |= routed != 0
        any_fp16 |= routed != vm
        if any_int8 and any_fp16:
            return "mixed"
    if not any_int8:
        return "fp16"
    if not any_fp16:
        return "int8"
    return "mixed"


# id(bitmask tensor) -> (weak reference, key, classification)
_ROUTE_CACHE: dict[int, tuple] = {}


def _classify_cached(precision_bitmask: torch.Tensor, **kw) -> Literal["mixed", "fp16", "int8"]:
    """``classify_bitmask_routing`` remembered per bitmask tensor: the
    classification reads the map on the host (a device-to-host copy that waits
    for every queued kernel), so a caller that passes the same map on every
    call (a model layer, a benchmark loop) pays that wait once instead of on
    every launch.  An entry holds while the tensor object, its storage, shape
    and version counter (bumped by every in-place torch op) are unchanged."""
    key = (precision_bitmask.data_ptr(), tuple(precision_bitmask.shape), precision_bitmask.device,
           precision_bitmask._version, tuple(sorted(kw.items())))
    hit = _ROUTE_CACHE.get(id(precision_bitmask))
    if hit is not None and hit[0]() is precision_bitmask and hit[1] == key:
        return hit[2]
    mode = classify_bitmask_routing(precision_bitmask, **kw)
    if len(_ROUTE_CACHE) >= 512:
        _ROUTE_CACHE.clear()
    _ROUTE_CACHE[id(precision_bitmask)] = (weakref.ref(precision_bitmask), key, mode)
    return mode


def _forced_config_check(block_m: int, block_n: int) -> None:
    """TILEMIX_FORCE_CONFIG="bm,bn,warps,stages" (reference :1024-1047): the block
    sizes must match the request; warps/stages have no meaning for the HIP kernel."""
    forced = os.environ.get("TILEMIX_FORCE_CONFIG")
    if not forced:
        return
    parts = [part.strip() for part in forced.split(",")]
    forced_m, forced_n = int(parts[0]), int(parts[1])
    if (forced_m, forced_n) != (block_m, block_n):
        raise ValueError(
            "TILEMIX_FORCE_CONFIG block sizes must match the kernel request: "
            f"forced=({forced_m}, {forced_n}), requested=({block_m}, {block_n})")


_PLACEHOLDERS: dict = {}


def _placeholder(kind: str, shape: tuple, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """A placeholder quantisation tensor, created once per (kind, shape, dtype,
    device) and shared by every later call.  The kernel never reads or writes
    the placeholders of an unquantised operand, so sharing them is safe, and
    the zero-filled scale prefixes then cost no fill kernel per call (a
    per-call fill put a ~2-5 us kernel into every step)."""
    key = (kind, tuple(shape), dtype, device)
    t = _PLACEHOLDERS.get(key)
    if t is None:
        if len(_PLACEHOLDERS) >= 256:
            _PLACEHOLDERS.clear()
        t = (torch.zeros if kind == "zeros" else torch.empty)(shape, dtype=dtype, device=device)
        _PLACEHOLDERS[key] = t
    return t


def _dummy_quantization_metadata(q, k, v, cu_seqlens_q, cu_seqlens_k):
    """Reference :1087-1115 -- placeholders for the all-FP16 mode (shared
    between calls: the kernel reads none of them in that mode)."""
    dev = q.device
    q8 = _placeholder("empty", (1, q.shape[1], q.shape[2]), torch.int8, dev)
    k8 = _placeholder("empty", (1, k.shape[1], k.shape[2]), torch.int8, dev)
    v8 = _placeholder("empty", (1, v.shape[1], v.shape[2]), torch.int8, dev)
    sq = _placeholder("empty", (1, q.shape[1]), q.dtype, dev)
    sk = _placeholder("empty", (1, k.shape[1]), k.dtype, dev)
    sv = sk
    cuq = _placeholder("zeros", tuple(cu_seqlens_q.shape), torch.int32, dev)
    cuk = _placeholder("zeros", tuple(cu_seqlens_k.shape), torch.int32, dev)
    cuv = cuk
    return q8, sq, cuq, k8, sk, cuk, v8, sv, cuv


def _dummy_v_quantization_metadata(v, cu_seqlens_k):
    """Reference :1118-1129 (placeholders shared between calls: with fp16 V the
    kernel reads none of them)."""
    v8 = _placeholder("empty", (1, v.shape[1], v.shape[2]), torch.int8, v.device)
    sv = _placeholder("empty", (1, v.shape[1]), v.dtype, v.device)
    cuv = _placeholder("zeros", tuple(cu_seqlens_k.shape), torch.int32, v.device)
    return v8, sv, cuv


def _padded_head_dim(head_dim: int) -> int:
    return -(-head_dim // HEAD_DIM_MULTIPLE) * HEAD_DIM_MULTIPLE


def _pad_head_dim(t: Optional[torch.Tensor], width: int) -> Optional[torch.Tensor]:
    """[tokens, heads, d] -> a dense [tokens, heads, width] copy, zeros past d."""
    if t is None or t.shape[-1] == width:
        return t
    out = torch.zeros((*t.shape[:-1], width), dtype=t.dtype, device=t.device)
    out[..., :t.shape[-1]] = t
    return out


def _inner_contiguous(t: torch.Tensor, align: int) -> torch.Tensor:
    """The kernel reads 16-byte vectors along the head dim: unit dim stride and
    vector-aligned token/head strides; otherwise take a dense copy."""
    if t.stride(2) != 1 or t.stride(0) % align or t.stride(1) % align or t.data_ptr() % 16:
        return t.contiguous()
    return t


# The kernel reads a sequence's K/V tiles through 32-bit buffer offsets:
# (max_seqlen_k + 64) * token stride must stay below 2 GiB, and 128 Q rows
# likewise (include/tilemix_hip.h).
_SPAN_LIMIT = 1 << 31


def _span_fits(t: torch.Tensor, rows: int) -> bool:
    return rows * t.stride(0) * t.element_size() < _SPAN_LIMIT


def _token_stride_fit(t: torch.Tensor, rows: int) -> torch.Tensor:
    """``t`` itself when ``rows`` token strides span less than 2 GiB, else a
    head-major copy: the same [tokens, heads, d] tensor with token stride d,
    so the span becomes rows * d elements (the reference addresses K/V with
    64-bit pointers over any strides, attention/triton/tilemix.py:1259-1275)."""
    if _span_fits(t, rows):
        return t
    return t.transpose(0, 1).contiguous().transpose(0, 1)


@torch.no_grad()
def launch_prequantized(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
    cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
    max_seqlens_q: int, max_seqlens_k: int,
    precision_bitmask: torch.Tensor,
    *,
    q8: torch.Tensor, k8: torch.Tensor, v8: torch.Tensor,
    sQ_blocks: torch.Tensor, sK_blocks: torch.Tensor, sV_blocks: torch.Tensor,
    cu_q_scale: torch.Tensor, cu_k_scale: torch.Tensor, cu_v_scale: torch.Tensor,
    block_m: int = 128, block_n: int = 64, block_n_mask: Optional[int] = None,
    BLKQ: int = 128, BLKK: int = 64,
    causal: bool = False, sm_scale: Optional[float] = None,
    bias: Optional[torch.Tensor] = None, o: Optional[torch.Tensor] = None,
    routing_mode: RoutingMode = "auto", run_length: bool = False,
    scalar_scales: bool = True, int8_cache_ca: bool = False, int8_use_fp16_v: bool = False,
    _q_in_kernel: bool = False,
) -> tuple[torch.Tensor, Literal["mixed", "fp16", "int8"]]:
    """Reference attention/triton/tilemix.py:1132-1337: validate, then one kernel launch.

    ``_q_in_kernel`` (not in the reference): q8 / sQ_blocks / cu_q_scale may be
    None and the kernel quantises Q itself (block_m == BLKQ == 128 only).
    """
    if not q.is_cuda:
        raise RuntimeError("TileMix is a GPU-only HIP kernel")
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("expected flattened [tokens, heads, dim] tensors")
    if k.shape != v.shape or q.shape[-1] != k.shape[-1]:
        raise ValueError("K/V shapes and Q/K/V head dimensions must match")
    if q.shape[1] % k.shape[1] != 0:
        raise ValueError("Q heads must be divisible by KV heads")
    if q.device != k.device or q.device != v.device:
        raise ValueError("q, k, and v must share one CUDA device")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise TypeError("q, k, and v must share one dtype")
    if max_seqlens_q != max_seqlens_k:
        raise ValueError("packed routing currently requires equal Q/K lengths")
    if block_n_mask is None:
        block_n_mask = block_n
    if block_n_mask % block_n:
        raise ValueError("block_n_mask must be a multiple of block_n")
    if (max_seqlens_k + block_n_mask - 1) // block_n_mask > 64:
        raise ValueError("packed routing exceeds 64 mask blocks")
    if scalar_scales and (block_m != BLKQ or block_n != BLKK):
        raise ValueError("scalar_scales requires block_m == BLKQ and block_n == BLKK")

    expected_rows = k.shape[1] * ((max_seqlens_q + block_m - 1) // block_m)
    if precision_bitmask.dtype != torch.uint64:
        raise TypeError("precision_bitmask must be torch.uint64")
    if precision_bitmask.numel() != expected_rows:
        raise ValueError(
            f"precision_bitmask has {precision_bitmask.numel()} rows, expected {expected_rows}")

    normalized_mode = routing_mode.strip().lower()
    if normalized_mode == "auto":
        normalized_mode = _classify_cached(
            precision_bitmask, seqlen_q=max_seqlens_q, seqlen_k=max_seqlens_k,
            block_m=block_m, block_n=block_n, block_n_mask=block_n_mask, causal=causal)
    mode_code = _routing_mode_code(normalized_mode)

    quant_tensors = (q8, k8, v8, sQ_blocks, sK_blocks, sV_blocks, cu_q_scale, cu_k_scale, cu_v_scale)
    if any(t is not None and t.device != q.device for t in quant_tensors):
        raise ValueError("all quantization tensors must share q.device")
    if (q8 is not None and q8.dtype != torch.int8) or k8.dtype != torch.int8:
        raise TypeError("q8 and k8 must be torch.int8")
    q_in_kernel = bool(_q_in_kernel) and mode_code != ROUTING_MODE_FP16
    if q_in_kernel and not _q_in_kernel_supported(block_m, BLKQ, mode_code, int8_use_fp16_v):
        raise ValueError("in-kernel Q quantisation needs BLKQ == 128 and 128-row workgroups "
                         "(block_m 128, 256 or 512, or block_m 64 without mixed routing on int8 V codes)")
    if mode_code != ROUTING_MODE_FP16 and not q_in_kernel and (q8 is None or sQ_blocks is None
                                                                or cu_q_scale is None):
        raise ValueError("q8, sQ_blocks and cu_q_scale are required")
    if v8.dtype != torch.int8:
        raise TypeError("v8 must be torch.int8")

    # ---- limits of this build (checked before any launch) ----------------
    if q.dtype != torch.float16:
        raise TypeError(f"the HIP TileMix kernel computes in float16, got {q.dtype}")
    if block_m not in SUPPORTED_BLOCK_M or block_n not in SUPPORTED_BLOCK_N:
        raise ValueError(
            f"the HIP TileMix kernel supports block_m in {SUPPORTED_BLOCK_M} and block_n in "
            f"{SUPPORTED_BLOCK_N}, got ({block_m}, {block_n})")
    head_dim = q.shape[-1]
    padded_head_dim = max(32, 1 << (head_dim - 1).bit_length())
    padded_head_dim = ((padded_head_dim + 31) // 32) * 32
    if padded_head_dim > 128:
        raise ValueError("head dimension must be <= 128")
    if mode_code != ROUTING_MODE_FP16 and (BLKK <= 0 or BLKK % 4):
        raise ValueError(f"the HIP TileMix kernel needs BLKK to be a positive multiple of 4, got {BLKK}")
    _forced_config_check(block_m, block_n)

    if sm_scale is None:
        sm_scale = head_dim ** -0.5
    out_user = o
    if o is None:
        o = torch.empty_like(q)
    run_dim = _padded_head_dim(head_dim)
    if run_dim != head_dim:
        q, k, v = (_pad_head_dim(t, run_dim) for t in (q, k, v))
        q8, k8, v8 = (_pad_head_dim(t, run_dim) for t in (q8, k8, v8))
    kv_rows = int(max_seqlens_k) + 64
    q = _token_stride_fit(_inner_contiguous(q, 8), 128)
    k = _token_stride_fit(_inner_contiguous(k, 8), kv_rows)
    v = _token_stride_fit(_inner_contiguous(v, 8), kv_rows)
    o_dev = o if (run_dim == head_dim and o.stride(2) == 1 and o.stride(0) % 4 == 0 and o.stride(1) % 4 == 0
                  and o.data_ptr() % 8 == 0) else torch.empty(q.shape, dtype=q.dtype, device=q.device)
    device = q.device
    cu_seqlens_q = cu_seqlens_q.to(device=device, dtype=torch.int32).contiguous()
    cu_seqlens_k = cu_seqlens_k.to(device=device, dtype=torch.int32).contiguous()
    precision_bitmask = precision_bitmask.to(device=device, dtype=torch.uint64).contiguous()
    batch = cu_seqlens_q.numel() - 1
    heads_q, heads_k = q.shape[1], k.shape[1]

    p = _native.AttnParams()
    p.q, p.k, p.v, p.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), o_dev.data_ptr()
    p.precision_bitmask = precision_bitmask.data_ptr()
    p.cu_seqlens_q, p.cu_seqlens_k = cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr()
    p.stride_q_token, p.stride_q_head = q.stride(0), q.stride(1)
    p.stride_k_token, p.stride_k_head = k.stride(0), k.stride(1)
    p.stride_v_token, p.stride_v_head = v.stride(0), v.stride(1)
    p.stride_o_token, p.stride_o_head = o_dev.stride(0), o_dev.stride(1)
    keep = []
    if mode_code != ROUTING_MODE_FP16:
        if q_in_kernel:
            p.q_quant_in_kernel = 1
        else:
            q8c = _inner_contiguous(q8, 16)
            sq = sQ_blocks.to(torch.float16).contiguous()
            cqs = cu_q_scale.to(dtype=torch.int32).contiguous()
            keep += [q8c, sq, cqs]
            p.q8, p.sq, p.cu_q_scale = q8c.data_ptr(), sq.data_ptr(), cqs.data_ptr()
            p.stride_q8_token, p.stride_q8_head = q8c.stride(0), q8c.stride(1)
        k8c = _token_stride_fit(_inner_contiguous(k8, 16), kv_rows)
        sk = sK_blocks.to(torch.float16).contiguous()
        cks = cu_k_scale.to(dtype=torch.int32).contiguous()
        keep += [k8c, sk, cks]
        p.k8, p.sk, p.cu_k_scale = k8c.data_ptr(), sk.data_ptr(), cks.data_ptr()
        p.stride_k8_token, p.stride_k8_head = k8c.stride(0), k8c.stride(1)
        if not int8_use_fp16_v:
            v8c = _token_stride_fit(_inner_contiguous(v8, 16), kv_rows)
            sv = sV_blocks.to(torch.float16).contiguous()
            cvs = cu_v_scale.to(dtype=torch.int32).contiguous()
            keep += [v8c, sv, cvs]
            p.v8, p.sv, p.cu_v_scale = v8c.data_ptr(), sv.data_ptr(), cvs.data_ptr()
            p.stride_v8_token, p.stride_v8_head = v8c.stride(0), v8c.stride(1)
    if bias is not None:
        b = bias.to(device=device, dtype=torch.float16)
        keep.append(b)
        p.bias = b.data_ptr()
        p.stride_bias_head, p.stride_bias_m, p.stride_bias_n = b.stride(1), b.stride(2), b.stride(3)
    p.sm_scale = float(sm_scale)
    p.heads_q, p.heads_k, p.head_dim, p.batch = heads_q, heads_k, run_dim, batch
    p.max_seqlen_q, p.max_seqlen_k = int(max_seqlens_q), int(max_seqlens_k)
    p.block_m, p.block_n, p.block_n_mask = int(block_m), int(block_n), int(block_n_mask)
    p.blkq, p.blkk = int(BLKQ), int(BLKK)
    p.causal = 1 if causal else 0
    p.routing_mode = mode_code
    p.int8_use_fp16_v = 1 if int8_use_fp16_v else 0
    if batch > 0:
        _native.attn_fwd(p, device)
    if o_dev is not o:
        o.copy_(o_dev[..., :head_dim])
    del keep
    if out_user is not None:
        return out_user, normalized_mode
    return o, normalized_mode


@torch.no_grad()
def tilemix_attention_with_quant(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
    cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
    max_seqlens_q: int, max_seqlens_k: int,
    precision_bitmask: torch.Tensor,
    *,
    block_m: int = 128, block_n: int = 64, block_n_mask: Optional[int] = None,
    BLKQ: int = 128, BLKK: int = 64,
    causal: bool = False, sm_scale: Optional[float] = None,
    bias: Optional[torch.Tensor] = None,
    routing_mode: RoutingMode = "auto", run_length: bool = False,
    scalar_scales: bool = True, int8_cache_ca: bool = False, int8_use_fp16_v: bool = False,
) -> tuple[torch.Tensor, Literal["mixed", "fp16", "int8"]]:
    """Reference attention/triton/tilemix.py:1340-1447: quantise (unless all-FP16), then launch.

    Quantisation here uses the no-sync path: fp16 scales are written by the
    quantisation kernel and its scale-row prefix is computed on the device.
    A head_dim that is not a multiple of 16 is zero-padded before quantising
    (codes and scales of the real columns are unchanged).
    """
    if block_n_mask is None:
        block_n_mask = block_n
    # launch_prequantized's shape checks (reference :1169-1172), before any
    # padding or quantisation: padding mismatched head dims to one width would
    # make them pass.
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("expected flattened [tokens, heads, dim] tensors")
    if k.shape != v.shape or q.shape[-1] != k.shape[-1]:
        raise ValueError("K/V shapes and Q/K/V head dimensions must match")
    head_dim = q.shape[-1]
    run_dim = _padded_head_dim(head_dim)
    if run_dim != head_dim and run_dim <= 128:
        if sm_scale is None:
            sm_scale = head_dim ** -0.5
        out, mode = tilemix_attention_with_quant(
            _pad_head_dim(q, run_dim), _pad_head_dim(k, run_dim), _pad_head_dim(v, run_dim),
            cu_seqlens_q, cu_seqlens_k, max_seqlens_q, max_seqlens_k, precision_bitmask,
            block_m=block_m, block_n=block_n, block_n_mask=block_n_mask, BLKQ=BLKQ, BLKK=BLKK,
            causal=causal, sm_scale=sm_scale, bias=bias, routing_mode=routing_mode, run_length=run_length,
            scalar_scales=scalar_scales, int8_cache_ca=int8_cache_ca, int8_use_fp16_v=int8_use_fp16_v)
        return out[..., :head_dim].contiguous(), mode
    normalized_mode = routing_mode.strip().lower()
    if normalized_mode == "auto":
        normalized_mode = _classify_cached(
            precision_bitmask, seqlen_q=max_seqlens_q, seqlen_k=max_seqlens_k,
            block_m=block_m, block_n=block_n, block_n_mask=block_n_mask, causal=causal)

    if normalized_mode == "fp16":
        quantized = _dummy_quantization_metadata(q, k, v, cu_seqlens_q, cu_seqlens_k)
    else:
        if not q.is_cuda:
            raise RuntimeError("TileMix is a GPU-only HIP kernel")
        fused = _q_in_kernel_enabled() and _q_in_kernel_supported(
            block_m, BLKQ, _routing_mode_code(normalized_mode), int8_use_fp16_v)
        if fused:
            q8 = sq = cuq = None
        else:
            q8, sq, cuq = _quantize_for_launch(q, cu_seqlens_q, max_seqlens_q, BLKQ)
        k8, sk, cuk = _quantize_for_launch(k, cu_seqlens_k, max_seqlens_k, BLKK)
        if int8_use_fp16_v:
            v8, sv, cuv = _dummy_v_quantization_metadata(v, cu_seqlens_k)
        else:
            v8, sv, cuv = _quantize_for_launch(v, cu_seqlens_k, max_seqlens_k, BLKK)
        quantized = q8, sq, cuq, k8, sk, cuk, v8, sv, cuv

    q8, sq, cuq, k8, sk, cuk, v8, sv, cuv = quantized
    fused = normalized_mode != "fp16" and q8 is None
    return launch_prequantized(
        q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlens_q, max_seqlens_k, precision_bitmask,
        q8=q8, k8=k8, v8=v8, sQ_blocks=sq, sK_blocks=sk, sV_blocks=sv,
        cu_q_scale=cuq, cu_k_scale=cuk, cu_v_scale=cuv,
        block_m=block_m, block_n=block_n, block_n_mask=block_n_mask, BLKQ=BLKQ, BLKK=BLKK,
        causal=causal, sm_scale=sm_scale, bias=bias, routing_mode=normalized_mode,
        run_length=run_length, scalar_scales=scalar_scales, int8_cache_ca=int8_cache_ca,
        int8_use_fp16_v=int8_use_fp16_v, _q_in_kernel=fused,
    )


def _q_in_kernel_supported(block_m: int, BLKQ: int, mode_code: int, int8_use_fp16_v: bool) -> bool:
    """The kernel quantises Q per 128-row workgroup, which is one BLKQ = 128
    block: block_m 128, 256 and 512, and block_m 64 except with mixed routing
    on int8 V codes (that variant runs 64-row workgroups)."""
    wg128 = block_m >= 128 or bool(int8_use_fp16_v) or mode_code != ROUTING_MODE_MIXED
    return wg128 and BLKQ == 128


def _q_in_kernel_enabled() -> bool:
    """``TILEMIX_HIP_FUSED_Q_QUANT`` (default 1): with BLKQ == 128 and 128-row
    workgroups the attention kernel quantises Q itself instead of a separate
    pre-pass (same codes and scales, bit for bit)."""
    return os.environ.get("TILEMIX_HIP_FUSED_Q_QUANT", "1").strip() not in ("0", "false", "False", "")


def debug_launch(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlens_q, max_seqlens_k, precision_bitmask,
                 *, q8, k8, sQ_blocks, sK_blocks, cu_q_scale, cu_k_scale, block_m, block_n_mask,
                 BLKQ=128, BLKK=64, causal=True, sm_scale=None, routing_mode="mixed", q_in_kernel=False,
                 block_n=64):
    """Run the kernel's DUMP instantiation (C entry ``tilemix_attn_fwd_debug``).

    Returns ``(out, qk_i32 [tokens_q, Hq, max_k] int32, qk16 [tokens_q, Hq, max_k] fp16)``;
    entries the kernel did not compute keep the fill values (INT32_MIN / NaN).
    No reference counterpart: it exposes the int32 Q8.K8 accumulators and the
    fp16 scores for the bit-exact parity tests.  ``q_in_kernel``: the kernel
    quantises Q itself (q8 / sQ_blocks / cu_q_scale are then ignored).
    """
    mode_code = _routing_mode_code(routing_mode)
    device = q.device
    if sm_scale is None:
        sm_scale = q.shape[-1] ** -0.5
    q, k, v = (t.contiguous() for t in (q, k, v))
    o = torch.empty_like(q)
    qk_i32 = torch.full((q.shape[0], q.shape[1], max_seqlens_k), -2 ** 31, dtype=torch.int32, device=device)
    qk16 = torch.full((q.shape[0], q.shape[1], max_seqlens_k), float("nan"), dtype=torch.float16, device=device)
    cu_q = cu_seqlens_q.to(device=device, dtype=torch.int32).contiguous()
    cu_k = cu_seqlens_k.to(device=device, dtype=torch.int32).contiguous()
    bm = precision_bitmask.to(device=device, dtype=torch.uint64).contiguous()
    q8c, k8c = q8.contiguous(), k8.contiguous()
    sq, sk = sQ_blocks.to(torch.float16).contiguous(), sK_blocks.to(torch.float16).contiguous()
    cqs, cks = cu_q_scale.to(device=device, dtype=torch.int32).contiguous(), cu_k_scale.to(
        device=device, dtype=torch.int32).contiguous()
    p = _native.AttnParams()
    p.q, p.k, p.v, p.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    p.precision_bitmask = bm.data_ptr()
    p.q8, p.k8, p.sq, p.sk = q8c.data_ptr(), k8c.data_ptr(), sq.data_ptr(), sk.data_ptr()
    p.cu_seqlens_q, p.cu_seqlens_k = cu_q.data_ptr(), cu_k.data_ptr()
    p.cu_q_scale, p.cu_k_scale = cqs.data_ptr(), cks.data_ptr()
    p.stride_q_token, p.stride_q_head = q.stride(0), q.stride(1)
    p.stride_k_token, p.stride_k_head = k.stride(0), k.stride(1)
    p.stride_v_token, p.stride_v_head = v.stride(0), v.stride(1)
    p.stride_o_token, p.stride_o_head = o.stride(0), o.stride(1)
    p.stride_q8_token, p.stride_q8_head = q8c.stride(0), q8c.stride(1)
    p.stride_k8_token, p.stride_k8_head = k8c.stride(0), k8c.stride(1)
    p.sm_scale = float(sm_scale)
    p.heads_q, p.heads_k, p.head_dim = q.shape[1], k.shape[1], q.shape[2]
    p.batch = cu_q.numel() - 1
    p.max_seqlen_q, p.max_seqlen_k = int(max_seqlens_q), int(max_seqlens_k)
    p.block_m, p.block_n, p.block_n_mask = int(block_m), int(block_n), int(block_n_mask)
    p.blkq, p.blkk = int(BLKQ), int(BLKK)
    p.causal = 1 if causal else 0
    p.routing_mode = mode_code
    p.int8_use_fp16_v = 1
    p.q_quant_in_kernel = 1 if q_in_kernel else 0
    _native.attn_fwd_debug(p, qk_i32, qk16, device)
    return o, qk_i32, qk16

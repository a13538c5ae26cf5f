"""Shared routing / block-size logic of the TileMix attention modules.

Behaviour follows the reference's model glue (models/tilemix_llama.py:34-460,
models/tilemix_qwen.py:28-455): size buckets, the block size each bucket
launches with, the mask-group width, the per-module routing-map cache keyed
by (seqlen, block sizes, pattern), and the token-mask generation of the
non-percentage layouts.  The map itself comes from
``tilemix_amd.attention.precision_maps`` and is repeated once per KV head.
"""
from __future__ import annotations

import hashlib
import math
import os
from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor

from ..attention import precision_maps as pm

# Below this many query tokens the module falls back to its parent's attention
# (reference models/tilemix_llama.py:527-537).
MIN_TILEMIX_SEQLEN = 16

# Layouts whose percentage-driven map needs no token mask (reference
# models/tilemix_llama.py:343-359).
_PERCENTAGE_LAYOUTS = frozenset({"band", "global", "row_rand", "align_sparse", "bigbird", "sptrans"})


@dataclass(frozen=True)
class BucketConfig:
    block_m: int
    block_n: int


def pick_block_n_for_64(seq_len: int, choices: list[int]) -> int:
    """Smallest tile width that keeps a row within 64 tiles (reference :39-43)."""
    for bn in sorted(choices):
        if math.ceil(seq_len / bn) <= 64:
            return bn
    return max(choices)


def pick_mask_block_n(seqlen: int, compute_block_n: int) -> int:
    """Mask-group width: a multiple of the compute tile with <= 64 groups per row
    (reference models/tilemix_llama.py:46-49)."""
    need = max((seqlen + 63) // 64, compute_block_n)
    return -(-need // compute_block_n) * compute_block_n


def _bucket(seqlen: int) -> str:
    for limit, name in ((128, "decode"), (2048, "short"), (8192, "medium"), (16384, "long"), (32768, "xl")):
        if seqlen <= limit:
            return name
    return "xxl"


def sptrans_token_mask(seqlen: int, stride: int, c: int) -> Tensor:
    """Token-level SpTrans mask (reference models/tilemix_llama.py:285-298):
    each query sees its own stride block up to itself and the last ``c`` keys
    of every earlier stride block."""
    q = torch.arange(seqlen)[:, None]
    k = torch.arange(seqlen)[None, :]
    qs = q // stride
    mask = (k >= qs * stride) & (k <= q) & (k < (qs + 1) * stride)
    for ks in range(max(seqlen - 1, 0) // stride):
        start, end = ks * stride + stride - c, (ks + 1) * stride
        if start < seqlen and end <= seqlen:
            lo = start if start >= 0 else max(seqlen + start, 0)  # Python slice semantics
            mask |= (qs > ks) & (k >= lo) & (k < end)
    return mask.view(1, 1, seqlen, seqlen)


class TileMixRoutingMixin:
    """Bucket, pattern and routing-map state of one TileMix attention module.

    Expects ``self.nh`` / ``self.nkv`` to be set by the module's ``__init__``
    before :meth:`_init_tilemix_state` runs.
    """

    def _init_tilemix_state(self, nh: int, nkv: int) -> None:
        if nh % nkv != 0:
            raise ValueError(f"num_attention_heads ({nh}) must be divisible by num_key_value_heads ({nkv})")
        self.nh, self.nkv = nh, nkv
        self.register_buffer("kv_head_mapping", torch.arange(nkv, dtype=torch.long).repeat_interleave(nh // nkv))
        self.decode_precision_cache: dict[tuple, Tensor] = {}
        buckets = ("decode", "short", "medium", "long", "xl", "xxl")
        self._bucket_configs = {b: BucketConfig(64, 64) for b in buckets}
        self._supported_ns = [64, 128, 256]
        sizes = [(c.block_m, c.block_n) for c in self._bucket_configs.values()]
        for extra in ((64, 64), (64, 128), (64, 256), (128, 64)):
            if extra not in sizes:
                sizes.append(extra)
        self.available_block_sizes = sizes
        self._block_to_candidate = {bs: i for i, bs in enumerate(sizes)}
        self.precision_map_cache: dict[tuple, Tensor] = {}
        self.default_pattern_type = "one"
        self.default_pattern_params: dict = {}

    # ---- block sizes --------------------------------------------------------
    def _choose_bucket(self, seqlen: int) -> Optional[str]:
        return _bucket(seqlen)

    def _find_nearest_available_block_size(self, seqlen: int, block_m: int, block_n: int) -> tuple[int, int]:
        """Nearest (block_m, block_n) of ``available_block_sizes`` whose tile fits
        the sequence (distance 0.5 |dm| + 1.5 |dn|, reference :122-141)."""
        fits = [(m, n) for m, n in self.available_block_sizes if n <= seqlen]
        if fits:
            return min(fits, key=lambda s: abs(block_m - s[0]) * 0.5 + abs(block_n - s[1]) * 1.5)
        return (min((64, 128, 256, 512), key=lambda x: abs(x - block_m)),
                min(self._supported_ns, key=lambda x: abs(x - block_n)))

    def _get_block_config(self, seqlen: int) -> BucketConfig:
        """Reference :143-175: ``TILEMIX_FORCE_CONFIG`` wins (snapped to an
        available size), else the bucket's size with block_m >= 128 from 4096 tokens."""
        forced = os.getenv("TILEMIX_FORCE_CONFIG")
        if forced:
            try:
                fm, fn = (int(p.strip()) for p in forced.split(",")[:2])
                return BucketConfig(*self._find_nearest_available_block_size(seqlen, fm, fn))
            except Exception:
                pass
        cfg = self._bucket_configs[self._choose_bucket(seqlen)]
        bn = min(max(cfg.block_n, 64), max(self._supported_ns))
        bm = max(cfg.block_m, 128) if seqlen >= 4096 else cfg.block_m
        return BucketConfig(*self._find_nearest_available_block_size(seqlen, bm, bn))

    # ---- routing patterns ---------------------------------------------------
    def set_attention_pattern(self, pattern_type: str, **pattern_params):
        """Switch the routing layout.  Both map caches are cleared (the
        reference clears only ``precision_map_cache`` and keeps serving a
        (64, 64) map built under the previous layout from
        ``decode_precision_cache``; that stale map is not kept here)."""
        self.default_pattern_type = pattern_type
        self.default_pattern_params = pattern_params
        self.precision_map_cache.clear()
        self.decode_precision_cache.clear()

    def _get_pattern_config(self, seqlen: int):
        return self.default_pattern_type, tuple(sorted(self.default_pattern_params.items()))

    @staticmethod
    def _get_pattern_hash(pattern_type: str, pattern_params: dict) -> str:
        key = f"{pattern_type}_{sorted(pattern_params.items())}"
        return hashlib.md5(key.encode()).hexdigest()[:8]

    def _generate_attention_pattern(self, seqlen: int, pattern_type: str, pattern_params: dict) -> Tensor:
        """Token-level mask of a layout without a percentage (reference :222-310)."""
        base = dict(num_query=seqlen, num_key=seqlen, dtype=torch.bool, num_layer=1, num_head=1)
        p = {**base, **pattern_params}
        if pattern_type == "zero":
            return pm.gen_zero_pattern(**base)
        if pattern_type == "causal":
            return pm.gen_causal_pattern(**base)
        if pattern_type == "band":
            p["percentage"] = pattern_params.get("percentage")
            return pm.gen_band_pattern(**p)
        if pattern_type == "global":
            p.pop("percentage", None)
            p["key_pos"] = [i for i in p.get("key_pos", list(range(min(4, seqlen)))) if 0 <= i < seqlen]
            return pm.gen_global_pattern(**p)
        if pattern_type == "row_rand":
            p.pop("percentage", None)
            p["num_rand_block_per_row"] = min(p.get("num_rand_block_per_row", 3), seqlen)
            return pm.gen_row_rand_pattern(**p)
        if pattern_type == "align_sparse":
            p.pop("percentage", None)
            p.setdefault("alpha", min(32, seqlen // 4))
            p.setdefault("beta", 0.1)
            return pm.gen_align_sparse_pattern(**p)
        if pattern_type == "bigbird":
            p.pop("percentage", None)
            p["num_global_block"] = min(p.get("num_global_block", 2), seqlen)
            p["num_rand_block"] = min(p.get("num_rand_block", 3), seqlen)
            p.setdefault("num_band_block", min(3, seqlen))
            return pm.gen_bigbird_pattern(**p)
        if pattern_type == "block":
            bs = pattern_params.get("block_size", 64)
            layout = pattern_params.get("layout")
            if layout is None:
                # Block diagonal band |i - j| < min(3, nb) (the reference builds it
                # with torch.eye(nb, k=i), which torch does not accept).
                nb = (seqlen + bs - 1) // bs
                idx = torch.arange(nb)
                layout = (idx[:, None] - idx[None, :]).abs() < max(1, min(3, nb))
            return pm.gen_block_pattern(layout, bs, dtype=torch.bool)
        if pattern_type == "layout_causal":
            bs = pattern_params.get("block_size", 64)
            layout = pattern_params.get("layout")
            if layout is None:
                nb = (seqlen + bs - 1) // bs
                layout = torch.ones(1, 1, nb, nb, dtype=torch.bool)
            return pm.layout_to_causal_mask(layout, bs, dtype=torch.bool)
        if pattern_type == "sptrans":
            stride = pattern_params.get("stride", min(128, seqlen // 4))
            c = pattern_params.get("c", min(32, stride // 4))
            return sptrans_token_mask(seqlen, stride, c)
        return pm.gen_one_pattern(**base)

    def _get_or_create_precision_map(self, seqlen: int, block_m: int, block_n: int, block_n_mask: int,
                                     pattern_type: str, pattern_params: tuple, device: torch.device) -> Tensor:
        """Packed routing row of one KV head ``[ceil(seqlen/block_m)]``, cached per module."""
        params = dict(pattern_params)
        percentage = None if pattern_type in ("one", "causal") else params.get("percentage")
        key = (seqlen, block_m, block_n, block_n_mask, self._get_pattern_hash(pattern_type, params), percentage)
        cached = self.precision_map_cache.get(key)
        if cached is not None:
            if cached.device != device:
                cached = cached.to(device)
                self.precision_map_cache[key] = cached
            return cached
        if pattern_type in ("zero", "one") or (percentage is not None and pattern_type in _PERCENTAGE_LAYOUTS):
            token_mask = None
        else:
            token_mask = self._generate_attention_pattern(seqlen, pattern_type, params)
        row = pm.make_precision_bitmask(seq_len=seqlen, BLOCK_M=block_m, BLOCK_N=block_n_mask,
                                        token_mask=token_mask, percentage=percentage, pattern_type=pattern_type,
                                        pattern_params=params, COMPUTE_BLOCK_N=block_n)
        m_blocks = (seqlen + block_m - 1) // block_m
        n_mask = (seqlen + block_n_mask - 1) // block_n_mask
        if n_mask > 64:
            raise ValueError(f"64-bit precision mask requires n_mask_blocks<=64, got n_mask_blocks={n_mask} "
                             f"(seqlen={seqlen}, block_n_mask={block_n_mask})")
        if not isinstance(row, Tensor):
            raise TypeError(f"precision_bitmask must be a tensor, got {type(row)}")
        if row.numel() != m_blocks:
            raise ValueError(f"Precision bitmask length mismatch: got {row.numel()}, expected {m_blocks} "
                             f"(m_blocks={m_blocks}, n_mask_blocks={n_mask})")
        row = row.to(device=device, dtype=torch.uint64)
        self.precision_map_cache[key] = row
        return row

    def _prepare_precision_map(self, seqlen: int, bucket_config: BucketConfig, block_n_mask: int,
                               pattern_type: str, pattern_params: tuple, device: torch.device) -> Tensor:
        """The row map repeated for every KV head ``[nkv * m_blocks]`` (reference :407-460);
        maps of the decode bucket's block size are kept per device and shape."""
        decode = self._bucket_configs["decode"]
        is_decode_size = (bucket_config.block_m, bucket_config.block_n) == (decode.block_m, decode.block_n)
        dkey = (device.type, bucket_config.block_m, bucket_config.block_n, block_n_mask, self.nh, self.nkv, seqlen)
        if is_decode_size:
            hit = self.decode_precision_cache.get(dkey)
            if hit is not None and hit.device == device:
                return hit
        row = self._get_or_create_precision_map(seqlen, bucket_config.block_m, bucket_config.block_n,
                                                block_n_mask, pattern_type, pattern_params, device)
        m_blocks = (seqlen + bucket_config.block_m - 1) // bucket_config.block_m
        n_mask = (seqlen + block_n_mask - 1) // block_n_mask
        if n_mask > 64:
            raise ValueError(f"64-bit precision mask requires n_mask_blocks<=64, got n_mask_blocks={n_mask} "
                             f"(seqlen={seqlen}, block_n_mask={block_n_mask})")
        if row.numel() != m_blocks:
            raise ValueError(f"Precision bitmask length {row.numel()} != expected {m_blocks} "
                             f"(m_blocks={m_blocks}, n_mask_blocks={n_mask})")
        full = row.to(device=device, dtype=torch.uint64).repeat(self.nkv)
        if is_decode_size:
            self.decode_precision_cache[dkey] = full
        return full

    def _routing_for(self, seqlen: int, device: torch.device):
        """(block_m, block_n, block_n_mask, map [nkv * m_blocks]) for one forward."""
        cfg = self._get_block_config(seqlen)
        bnm = pick_mask_block_n(seqlen, cfg.block_n)
        if (cfg.block_m, cfg.block_n) not in self._block_to_candidate:
            raise ValueError(f"Block size {(cfg.block_m, cfg.block_n)} for bucket {self._choose_bucket(seqlen)} "
                             f"is not in available_block_sizes. This should not happen if _get_block_config is "
                             f"working correctly. Available sizes: {self.available_block_sizes}")
        ptype, pparams = self._get_pattern_config(seqlen)
        full = self._prepare_precision_map(seqlen, cfg, bnm, ptype, pparams, device)
        expected = self.nkv * ((seqlen + cfg.block_m - 1) // cfg.block_m)
        if full.numel() != expected:
            raise ValueError(f"precision_map length mismatch after regen: got {full.numel()}, expected {expected} "
                             f"(Hk={self.nkv}, block_m={cfg.block_m}, block_n={cfg.block_n}, "
                             f"block_n_mask={bnm}, seqlen={seqlen})")
        return cfg, bnm, full

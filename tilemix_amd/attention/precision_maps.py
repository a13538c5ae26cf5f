"""Routing-map construction for TileMix: which tile groups go to INT8.

Drop-in for the reference's attention/precision_maps.py (same function names,
arguments and results).  A routing map is a bool matrix ``[num_m, num_n_mask]``
(True = INT8) over (query block of BLOCK_M rows) x (key group of
BLOCK_N(mask) keys), packed LSB-first into one uint64 per query block.

Results must be bit-identical to the reference, including every map that
depends on torch's CPU random generator or Python's ``random``: the functions
below therefore issue exactly the reference's sequence of RNG calls
(``torch.manual_seed`` / ``torch.randperm`` / ``torch.Generator`` /
``random.sample``), with the same arguments and in the same order.  The
deterministic parts (tile weights, band/stride layouts, bit packing) are
computed with array arithmetic instead of the reference's per-element loops.
Caller-visible side effects are kept too: ``row_rand`` and ``bigbird`` reseed
the global torch RNG with 42 (reference :537, :580).
"""
from __future__ import annotations

import random

import numpy as np
import torch


# --------------------------------------------------------------------------
# token-level pattern generators (reference :5-198)
# --------------------------------------------------------------------------
def gen_one_pattern(num_query, num_key, dtype: torch.dtype = torch.bool,
                    num_layer: int = 1, num_head: int = 1) -> torch.Tensor:
    """Reference :5-8."""
    return torch.ones((num_layer, num_head, num_query, num_key), dtype=dtype)


def gen_zero_pattern(num_query, num_key, dtype: torch.dtype = torch.bool,
                     num_layer: int = 1, num_head: int = 1) -> torch.Tensor:
    """Reference :11-14."""
    return torch.zeros((num_layer, num_head, num_query, num_key), dtype=dtype)


def gen_causal_pattern(num_query, num_key, dtype: torch.dtype = torch.bool,
                       num_layer: int = 1, num_head: int = 1) -> torch.Tensor:
    """Reference :17-25: True strictly above the diagonal (future keys)."""
    upper = torch.arange(num_key)[None, :] > torch.arange(num_query)[:, None]
    return upper[None, None].expand(num_layer, num_head, -1, -1).to(dtype)


def calculate_band_width_from_percentage(seq_len: int, percentage: float, block_n: int) -> int:
    """Reference :28-62: odd band width (tokens) leaving ``percentage`` outside the band."""
    if percentage is None or percentage <= 0.0 or percentage >= 1.0:
        return 5
    if block_n is None or block_n <= 0:
        width = int((1.0 - percentage) * seq_len)
        width += width % 2 == 0
        return max(3, min(width, seq_len))
    num_n = (seq_len + block_n - 1) // block_n
    target = (1.0 - percentage) * num_n
    blocks = int(round(target))
    if blocks % 2 == 0:
        blocks = blocks + 1 if target > blocks else max(1, blocks - 1)
    blocks = max(1, min(blocks, num_n))
    width = blocks * block_n
    width += width % 2 == 0
    return max(3, min(width, seq_len))


def gen_band_pattern(num_query, num_key, band_width: int = None, dtype: torch.dtype = torch.bool,
                     num_layer: int = 1, num_head: int = 1, percentage: float = None,
                     block_n: int = None) -> torch.Tensor:
    """Reference :65-85: |key - query| <= band_width // 2 (band width forced odd)."""
    if band_width is None and percentage is not None:
        band_width = calculate_band_width_from_percentage(num_query, percentage, block_n)
    if band_width is None:
        band_width = 5
    if band_width % 2 == 0:
        band_width += 1
    band_width = min(band_width, num_key)
    half = band_width // 2
    offset = torch.arange(num_key)[None, :] - torch.arange(num_query)[:, None]
    band = (offset >= -half) & (offset < half + 1)
    return band[None, None].expand(num_layer, num_head, -1, -1).to(dtype)


def gen_global_pattern(num_query, num_key, key_pos: list, dtype: torch.dtype = torch.bool,
                       num_layer: int = 1, num_head: int = 1) -> torch.Tensor:
    """Reference :88-103: whole key columns ``key_pos`` (those < num_key)."""
    cols = [pos for pos in key_pos if pos < num_key]
    g = torch.zeros((num_layer, num_head, num_query, num_key), dtype=torch.bool)
    if cols:
        g[:, :, :, cols] = True
    return g.to(dtype)


def gen_row_rand_pattern(num_query, num_key, num_rand_block_per_row: int,
                         dtype: torch.dtype = torch.bool, num_layer: int = 1,
                         num_head: int = 1) -> torch.Tensor:
    """Reference :106-120: ``random.sample`` per (layer, head, query) row, in that order."""
    rand = torch.zeros((num_layer, num_head, num_query, num_key), dtype=torch.bool)
    for layer in range(num_layer):
        for head in range(num_head):
            for i in range(num_query):
                rand[layer, head, i, random.sample(range(num_key), num_rand_block_per_row)] = True
    return rand.to(dtype)


def gen_align_sparse_pattern(num_query, num_key, alpha: int, beta: float,
                             dtype: torch.dtype = torch.bool, num_layer: int = 1,
                             num_head: int = 1) -> torch.Tensor:
    """Reference :123-139: row i keeps a right-aligned run of
    nnz = min(alpha + beta (eff - alpha) [eff > alpha], eff) keys, eff = min(i+1, num_key)."""
    rows = []
    for i in range(num_query):
        eff = min(i + 1, num_key)
        nnz = int(min(alpha + beta * (eff - alpha) * (eff > alpha), eff))
        start = max(0, min(i - nnz + 1, num_key - nnz))
        rows.append((start, start + nnz))
    bounds = torch.tensor(rows, dtype=torch.int64).reshape(num_query, 2)
    k = torch.arange(num_key)[None, :]
    row_mask = (k >= bounds[:, :1]) & (k < bounds[:, 1:])
    return row_mask[None, None].expand(num_layer, num_head, -1, -1).clone().to(dtype)


def gen_bigbird_pattern(num_query, num_key, num_band_block: int = 3, num_global_block: int = 2,
                        num_rand_block: int = 3, dtype: torch.dtype = torch.bool,
                        num_layer: int = 1, num_head: int = 1) -> torch.Tensor:
    """Reference :142-176: band | (global rows and columns) | random per row."""
    band = gen_band_pattern(num_query, num_key, num_band_block, dtype, num_layer, num_head)
    glob = gen_global_pattern(num_query, num_key, list(range(min(num_global_block, num_key))),
                              dtype, num_layer, num_head)
    glob = glob | glob.transpose(-2, -1)
    rand = gen_row_rand_pattern(num_query, num_key, min(num_rand_block, num_key), dtype,
                                num_layer, num_head)
    return (band | glob | rand).to(dtype)


def gen_block_pattern(layout: torch.Tensor, block_size: int = 64,
                      dtype: torch.dtype = torch.bool) -> torch.Tensor:
    """Reference :179-190: expand a block layout to tokens."""
    if layout.ndim == 2:
        layout = layout[None, None]
    elif layout.ndim == 3:
        layout = layout[None]
    return layout.repeat_interleave(block_size, dim=-2).repeat_interleave(block_size, dim=-1).to(dtype)


def layout_to_causal_mask(layout: torch.Tensor, block_size: int,
                          dtype: torch.dtype = torch.bool) -> torch.Tensor:
    """Reference :193-198."""
    L, H, QB, KB = layout.shape
    full = gen_block_pattern(layout, block_size, dtype)
    return full & gen_causal_pattern(QB * block_size, KB * block_size, dtype, L, H)


# --------------------------------------------------------------------------
# block-level policy (reference :201-401)
# --------------------------------------------------------------------------
def _apply_percentage_control(block_precision_map: torch.Tensor, percentage: float) -> torch.Tensor:
    """Reference :201-235: flip random FP16 cells to INT8 until int(total * p) are INT8.

    Uses the unseeded global torch RNG (one ``randperm`` call), like the reference.
    """
    if percentage is None or percentage < 0.0 or percentage > 1.0:
        return block_precision_map
    num_m, num_n = block_precision_map.shape
    current = block_precision_map.sum().item()
    target = int(num_m * num_n * percentage)
    if current >= target:
        return block_precision_map
    fp16_cells = torch.nonzero(~block_precision_map, as_tuple=False)
    if len(fp16_cells) == 0:
        return block_precision_map
    n_flip = min(target - current, len(fp16_cells))
    perm = torch.randperm(len(fp16_cells), device=block_precision_map.device)
    chosen = fp16_cells[perm[:n_flip]]
    result = block_precision_map.clone()
    result[chosen[:, 0], chosen[:, 1]] = True
    return result


def _causal_compute_tile_weights(seq_len: int, block_m: int, block_n_mask: int, compute_block_n: int,
                                 *, device: torch.device | None = None) -> torch.Tensor:
    """Reference :238-270: number of causally executed compute tiles in each mask cell.

    Query block r executes min(ceil(L/bn), ceil((r+1) bm / bn)) tiles of bn
    keys; mask group j holds tiles [j G, (j+1) G), G = block_n_mask / bn.
    """
    if block_n_mask % compute_block_n != 0:
        raise ValueError(
            f"block_n_mask ({block_n_mask}) must be a multiple of compute_block_n ({compute_block_n})")
    num_m = (seq_len + block_m - 1) // block_m
    num_mask_n = (seq_len + block_n_mask - 1) // block_n_mask
    num_compute_n = (seq_len + compute_block_n - 1) // compute_block_n
    group = block_n_mask // compute_block_n
    rows = np.arange(num_m, dtype=np.int64)
    executed = np.minimum(num_compute_n, ((rows + 1) * block_m + compute_block_n - 1) // compute_block_n)
    first_tile = np.arange(num_mask_n, dtype=np.int64) * group
    w = np.clip(executed[:, None] - first_tile[None, :], 0, group)
    return torch.from_numpy(np.ascontiguousarray(w)).to(device=device)


def _retarget_weighted_int8_fraction(block_precision_map: torch.Tensor, weights: torch.Tensor,
                                     percentage: float, *, seed: int = 42) -> torch.Tensor:
    """Reference :273-326: make the weighted INT8 fraction round(sum(w) p).

    Illegal cells (weight 0) are cleared; then candidates (cells that can move
    toward the target) are visited in ``randperm(len, Generator(seed))`` order
    and flipped whenever the flip does not move away from the target.
    """
    if percentage < 0.0 or percentage > 1.0:
        raise ValueError(f"percentage must be in [0, 1], got {percentage}")
    if block_precision_map.shape != weights.shape:
        raise ValueError(
            "block_precision_map and weights must have identical shapes, got "
            f"{tuple(block_precision_map.shape)} and {tuple(weights.shape)}")
    original_device = block_precision_map.device
    result = block_precision_map.detach().to(device="cpu", dtype=torch.bool).clone()
    w = weights.detach().to(device="cpu", dtype=torch.int64)
    legal = w > 0
    result &= legal
    total = int(w.sum().item())
    if total == 0:
        return result.to(device=original_device)
    target = int(round(total * percentage))
    current = int((w * result).sum().item())
    if current == target:
        return result.to(device=original_device)
    add_int8 = current < target
    candidates = torch.nonzero(((~result) if add_int8 else result) & legal, as_tuple=False)
    generator = torch.Generator(device="cpu")
    generator.manual_seed(seed)
    order = torch.randperm(len(candidates), generator=generator).tolist()
    cand = candidates.tolist()
    wl = w.tolist()
    res = result.numpy()  # shares memory with `result`
    for position in order:
        row, col = cand[position]
        weight = wl[row][col]
        proposed = current + weight if add_int8 else current - weight
        if abs(target - proposed) <= abs(target - current):
            res[row, col] = add_int8
            current = proposed
        if current == target:
            break
    max_weight = int(w.max().item())
    if abs(current - target) > max_weight:
        raise RuntimeError(
            "unable to retarget executable INT8 fraction within one mask-bit "
            f"weight: target={target}, achieved={current}, max_weight={max_weight}")
    return result.to(device=original_device)


def _make_sptrans_block_precision_map(seq_len: int, block_m: int, block_n_mask: int, compute_block_n: int,
                                      percentage: float, pattern_params: dict, *,
                                      device: torch.device | None = None) -> torch.Tensor:
    """Reference :329-385: strided "SpTrans" layout, then weighted retarget.

    FP16 (False) cells of query block r: the key groups overlapping the local
    stride of each query stride in the block, plus the groups overlapping the
    last ``c`` keys of every earlier stride; everything else starts as INT8.
    """
    num_m = (seq_len + block_m - 1) // block_m
    num_n = (seq_len + block_n_mask - 1) // block_n_mask
    stride = pattern_params.get("stride", min(128, seq_len // 4))
    c = pattern_params.get("c", min(32, stride // 4))
    sparse = np.ones((num_m, num_n), dtype=bool)
    # Key-group range [lo, hi) of the tail of each stride p (last c keys).
    n_strides = (seq_len - 1) // stride + 1 if seq_len > 0 else 0
    p = np.arange(n_strides, dtype=np.int64)
    tail_lo = np.maximum(p * stride, (p + 1) * stride - c) // block_n_mask
    tail_hi = np.minimum(num_n, ((p + 1) * stride + block_n_mask - 1) // block_n_mask)
    tail_cover = np.zeros((n_strides + 1, num_n), dtype=bool)  # tail_cover[s] = union over p < s
    for s in range(1, n_strides + 1):
        tail_cover[s] = tail_cover[s - 1]
        lo, hi = int(tail_lo[s - 1]), int(tail_hi[s - 1])
        if lo < num_n:
            tail_cover[s, lo:hi] = True
    for row in range(num_m):
        q0 = row * block_m
        q1 = min(seq_len, (row + 1) * block_m)
        first, last = q0 // stride, (q1 - 1) // stride
        for qs in range(first, last + 1):
            lo = (qs * stride) // block_n_mask
            hi = min(num_n, (min((qs + 1) * stride, q1) + block_n_mask - 1) // block_n_mask)
            if lo < num_n:
                sparse[row, lo:hi] = False
        sparse[row, tail_cover[last]] = False
    weights = _causal_compute_tile_weights(seq_len, block_m, block_n_mask, compute_block_n, device=device)
    return _retarget_weighted_int8_fraction(torch.from_numpy(sparse).to(device=device), weights,
                                            percentage, seed=42)


def pack_block_precision_map(block_precision_map: torch.Tensor) -> torch.Tensor:
    """Reference :388-401: row r -> uint64 with bit j = column j (LSB first)."""
    if block_precision_map.ndim != 2 or block_precision_map.shape[1] > 64:
        raise ValueError(
            "block_precision_map must be 2D with at most 64 columns, got "
            f"{tuple(block_precision_map.shape)}")
    original_device = block_precision_map.device
    bits = block_precision_map.detach().to(device="cpu", dtype=torch.bool).numpy().astype(np.uint64)
    weights = np.left_shift(np.uint64(1), np.arange(bits.shape[1], dtype=np.uint64))
    packed = (bits * weights[None, :]).sum(axis=1, dtype=np.uint64) if bits.shape[1] else \
        np.zeros(bits.shape[0], dtype=np.uint64)
    return torch.from_numpy(np.ascontiguousarray(packed)).to(device=original_device)


def make_precision_bitmask(seq_len: int, BLOCK_M: int, BLOCK_N: int, token_mask: torch.Tensor | None,
                           percentage: float = None, pattern_type: str = None,
                           pattern_params: dict = None, COMPUTE_BLOCK_N: int = None) -> torch.Tensor:
    """Reference :404-636: packed routing rows ``[ceil(seq_len / BLOCK_M)]`` uint64.

    ``BLOCK_N`` is the mask-group width (block_n_mask) and ``COMPUTE_BLOCK_N``
    the kernel's key tile (defaults to BLOCK_N).
    """
    num_m = (seq_len + BLOCK_M - 1) // BLOCK_M
    num_n = (seq_len + BLOCK_N - 1) // BLOCK_N
    if COMPUTE_BLOCK_N is None:
        COMPUTE_BLOCK_N = BLOCK_N
    if BLOCK_N % COMPUTE_BLOCK_N != 0:
        raise ValueError(
            f"BLOCK_N(mask) ({BLOCK_N}) must be a multiple of COMPUTE_BLOCK_N ({COMPUTE_BLOCK_N})")
    if num_n > 64:
        raise ValueError(
            f"num_n_mask={num_n} > 64; BLOCK_N(mask) too small (seq_len={seq_len}, BLOCK_N(mask)={BLOCK_N})")
    if pattern_type in {"zero", "one"}:
        weights = _causal_compute_tile_weights(seq_len, BLOCK_M, BLOCK_N, COMPUTE_BLOCK_N)
        sparse = torch.zeros_like(weights, dtype=torch.bool) if pattern_type == "zero" else weights > 0
        return pack_block_precision_map(sparse)

    block_patterns = {"band", "global", "row_rand", "align_sparse", "bigbird", "sptrans"}
    if pattern_type == "sptrans" and percentage is not None and pattern_params is not None:
        device = token_mask.device if token_mask is not None else None
        return pack_block_precision_map(_make_sptrans_block_precision_map(
            seq_len, BLOCK_M, BLOCK_N, COMPUTE_BLOCK_N, percentage, pattern_params, device=device))

    direct = percentage is not None and pattern_type in block_patterns and pattern_params is not None
    if token_mask is None and not direct:
        raise ValueError("token_mask may be None only for a percentage-aware block policy")
    if direct:
        device = token_mask.device if token_mask is not None else None
        mask2d = torch.empty(0, dtype=torch.bool, device=device)
        tiles = None
    else:
        mask2d = token_mask[0, 0]
        padded = torch.nn.functional.pad(
            mask2d, (0, num_n * BLOCK_N - seq_len, 0, num_m * BLOCK_M - seq_len), value=True)
        tiles = padded.unfold(0, BLOCK_M, BLOCK_M).unfold(1, BLOCK_N, BLOCK_N)
    device = mask2d.device
    frac_hp = None if percentage is None else 1.0 - percentage

    if pattern_type == "one":
        sparse = torch.ones((num_m, num_n), dtype=torch.bool, device=device)
    elif pattern_type == "band" and percentage is not None:
        # Reference :495-506: an odd number of FP16 groups centred on column i.
        width = int(round(num_n * frac_hp))
        if width % 2 == 0:
            width = max(1, width - 1)
        width = max(1, min(width, num_n))
        col = torch.arange(num_n, device=device)[None, :]
        centre = torch.arange(num_m, device=device)[:, None]
        in_band = (col >= centre - width // 2) & (col < centre + width // 2 + 1)
        sparse = ~in_band
    elif pattern_type == "global" and percentage is not None and pattern_params is not None:
        # Reference :507-531: FP16 columns = key_pos columns, topped up from column 0.
        n_cols = max(1, min(int(round(num_n * frac_hp)), num_n))
        key_pos = pattern_params.get("key_pos", list(range(min(4, seq_len))))
        cols = {pos // BLOCK_N for pos in key_pos if 0 <= pos < seq_len and pos // BLOCK_N < num_n}
        fill = 0
        while len(cols) < n_cols and len(cols) < num_n:
            while fill in cols:
                fill += 1
            cols.add(fill)
        cols = sorted(cols)[:n_cols]
        sparse = torch.ones((num_m, num_n), dtype=torch.bool, device=device)
        if cols:
            sparse[:, cols] = False
    elif pattern_type == "row_rand" and percentage is not None and pattern_params is not None:
        # Reference :532-540: global seed 42, one randperm per row.
        per_row = max(1, min(int(round(num_n * frac_hp)), num_n))
        sparse = torch.ones((num_m, num_n), dtype=torch.bool, device=device)
        torch.manual_seed(42)
        for i in range(num_m):
            sparse[i, torch.randperm(num_n, device=device)[:per_row]] = False
    elif pattern_type == "align_sparse" and percentage is not None and pattern_params is not None:
        # Reference :541-548: the last `per_row` groups of every row are FP16.
        per_row = max(1, min(int(round(num_n * frac_hp)), num_n))
        sparse = torch.ones((num_m, num_n), dtype=torch.bool, device=device)
        sparse[:, max(0, num_n - per_row):] = False
    elif pattern_type == "bigbird" and percentage is not None and pattern_params is not None:
        sparse = _bigbird_block_map(num_m, num_n, frac_hp, pattern_params, device)
    else:
        sparse = tiles.any(dim=(2, 3)) if pattern_type == "causal" else (~tiles).any(dim=(2, 3))
        if percentage is not None and pattern_type not in ["one", "causal"]:
            sparse = _apply_percentage_control(sparse, percentage)

    if percentage is not None and pattern_type in {"band", "global", "row_rand", "align_sparse", "bigbird"}:
        weights = _causal_compute_tile_weights(seq_len, BLOCK_M, BLOCK_N, COMPUTE_BLOCK_N, device=sparse.device)
        sparse = _retarget_weighted_int8_fraction(sparse, weights, percentage, seed=42)
    return pack_block_precision_map(sparse)


def _bigbird_block_map(num_m: int, num_n: int, frac_hp: float, pattern_params: dict,
                       device) -> torch.Tensor:
    """Reference :549-601: band + global rows/columns + seeded random groups, then
    random flips (global RNG, continuing after the seed) to hit round(total (1-p)) FP16."""
    target_hp = max(1, min(int(round(num_m * num_n * frac_hp)), num_m * num_n))
    sparse = torch.ones((num_m, num_n), dtype=torch.bool, device=device)
    num_global_block = pattern_params.get("num_global_block", 2)
    num_rand_block = pattern_params.get("num_rand_block", 3)
    band = max(1, min(int(round(num_n * frac_hp * 0.5)), num_n))
    band += band % 2 == 0
    band = min(band, num_n)
    col = torch.arange(num_n, device=device)[None, :]
    centre = torch.clamp(torch.arange(num_m, device=device), max=num_n - 1)[:, None]
    in_band = (col >= centre - band // 2) & (col < centre + band // 2 + 1)
    sparse &= ~in_band
    n_glob = min(num_global_block, num_n)
    sparse[:, :n_glob] = False
    sparse[: min(n_glob, num_m), :] = False
    per_row = min(num_rand_block, num_n)
    torch.manual_seed(42)
    for i in range(num_m):
        sparse[i, torch.randperm(num_n, device=device)[:per_row]] = False
    current_hp = (~sparse).sum().item()
    if current_hp < target_hp:
        int8_cells = torch.nonzero(sparse, as_tuple=False)
        n_flip = target_hp - current_hp
        if n_flip > 0 and len(int8_cells) > 0:
            pick = torch.randperm(len(int8_cells), device=device)[:n_flip]
            chosen = int8_cells[pick]
            sparse[chosen[:, 0], chosen[:, 1]] = False
    elif current_hp > target_hp:
        fp16_cells = torch.nonzero(~sparse, as_tuple=False)
        n_flip = current_hp - target_hp
        if n_flip > 0 and len(fp16_cells) > 0:
            pick = torch.randperm(len(fp16_cells), device=device)[:n_flip]
            chosen = fp16_cells[pick]
            sparse[chosen[:, 0], chosen[:, 1]] = True
    return sparse

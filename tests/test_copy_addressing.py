"""Host-side model of the attention kernels' HBM->LDS tile copies: which bytes a
launch reads.

The kernels copy every 64-key tile of K (fp16 or int8), V (fp16) and int8 V
codes with ``buffer_load_dwordx4 ... lds``.  Both kernels read through one raw
buffer per stream based at the sequence's first key (sequence start + head
offset) and sized to the sequence, adding the tile's byte offset to the 32-bit
lane offsets.  A 4-byte lane of the load reads memory only below the buffer
size (zeros otherwise).  The lane offsets restated here are those of
``lane_off0`` / ``issue_tile`` in tilemix_amd/csrc/attn_kernel32.h and of
``lane_off`` / ``issue_tile`` in tilemix_amd/csrc/attn_kernel16.h (swizzles:
``swz_k``, ``swz_v``, ``swz_v32`` in attn_common.h; out-of-range offset
``kOffOutside``).

The check: every byte read is a byte of an element (token of the tile's own
sequence, the tile's KV head, column < head_dim) -- nothing past the end of a
tensor, nothing of a neighbouring head, nothing of the padded columns.  With
the head_dim mask taken out (the copies before the fix), the model reads past
the end of the last head of the last token, which the planted case asserts.
"""
from __future__ import annotations

import numpy as np
import pytest

OUTSIDE = 0x80000000  # kOffOutside as a 32-bit lane offset


def swz_k(rowb, r):
    if rowb >= 256:
        return r & 15
    if rowb == 128:
        return (r >> 1) & 7
    return (r >> 2) & 3


def swz_v(rowb, r):
    return 2 * (r & 7) if rowb >= 256 else 2 * ((r >> 1) & 3)


def swz_v32(rowb, r):
    return 4 * (r & 3) if rowb >= 256 else 4 * ((r >> 1) & 1)


def lane_offsets(kernel, rowb, tok_bytes, swz, valid_bytes, nw=4, mask=True):
    """u32 lane offsets of one tile's copies of one stream (all waves, lanes, copies)."""
    rpi, cpr = 1024 // rowb, rowb // 16
    offs = []
    if kernel == 32:
        ins = 64 * rowb // 1024 // nw
        step = nw * rpi * tok_bytes
        for wave in range(nw):
            for lane in range(64):
                r = wave * rpi + lane // cpr
                chunk = (lane % cpr) ^ swz(rowb, r)
                o0 = OUTSIDE if (mask and chunk * 16 >= valid_bytes) else r * tok_bytes + chunk * 16
                for i in range(ins):
                    offs.append((o0 + i * step) & 0xFFFFFFFF)
    else:
        tiles = 64 * rowb // 1024
        n_i = (tiles + nw - 1) // nw
        for i in range(n_i):
            for wave in range(nw):
                L = i * nw + wave
                if L >= tiles:
                    continue
                for lane in range(64):
                    r = L * rpi + lane // cpr
                    chunk = (lane % cpr) ^ swz(rowb, r)
                    o = OUTSIDE if (mask and chunk * 16 >= valid_bytes) else r * tok_bytes + chunk * 16
                    offs.append(o & 0xFFFFFFFF)
    return np.array(offs, dtype=np.int64)


def tile_dwords(kernel, offs, L, t, tok_bytes):
    """Byte offsets from the buffer base that the lanes of tile t read (dword
    starts), and the buffer size: the buffer spans the sequence and the tile
    offset is added in 32 bits (both kernels)."""
    dw = offs[:, None] + 4 * np.arange(4)[None, :]  # every dword of every lane
    return (dw + 64 * t * tok_bytes) & 0xFFFFFFFF, L * tok_bytes


def bytes_read(offs, lens, hk, tok_bytes, head_bytes, kernel=32):
    """Relative byte addresses (from the tensor's data pointer) read by the copies."""
    out = []
    cu = np.concatenate([[0], np.cumsum(lens)])
    for z, L in enumerate(lens):
        for h in range(hk):
            for t in range((L + 63) // 64):
                dw, size = tile_dwords(kernel, offs, L, t, tok_bytes)
                base = cu[z] * tok_bytes + h * head_bytes
                hit = dw[dw < size]
                out.append((base + hit[:, None] + np.arange(4)[None, :]).ravel())
    return np.concatenate(out) if out else np.zeros(0, dtype=np.int64)


def check_elements(addr, lens, hk, tok_bytes, head_bytes, elem, d):
    """Every byte address lies in a valid element: token < total, head < hk, column < d."""
    n = int(sum(lens))
    assert addr.min() >= 0
    tok, within = addr // tok_bytes, addr % tok_bytes
    head, col = within // head_bytes, (within % head_bytes) // elem
    bad = (tok >= n) | (head >= hk) | (col >= d)
    return int(bad.sum())


# kernel, head_dim, padded width DP, Hk, storage width (head stride in elements), lengths
CASES = [
    (32, 80, 128, 3, 80, [1, 63, 64, 65, 130]),
    (32, 80, 128, 3, 128, [200, 7]),  # [..., :80] view of a 128-wide buffer
    (32, 96, 128, 2, 96, [129, 64]),
    (32, 112, 128, 2, 112, [70]),
    (32, 48, 64, 3, 48, [100, 1]),
    (32, 16, 64, 2, 16, [65]),
    (32, 128, 128, 3, 128, [130]),
    (16, 80, 128, 3, 80, [1, 63, 64, 65, 130]),
    (16, 48, 64, 3, 48, [100, 1]),
    (16, 32, 64, 2, 32, [64, 3]),
]


def _streams(kernel, dp, d, hstride, hk):
    """(rowb, tok_bytes, head_bytes, elem bytes, valid bytes, swizzle) per copy stream."""
    row16, row8 = 2 * dp, dp
    tok16, tok8 = 2 * hstride * hk, hstride * hk
    # int8 tensors need 16-byte strides: round the int8 head stride up
    h8 = ((hstride + 15) // 16) * 16
    tok8 = h8 * hk
    vswz = swz_v32 if kernel == 32 else swz_v
    return [
        ("k16", row16, tok16, 2 * hstride, 2, 2 * d, swz_k),
        ("v16", row16, tok16, 2 * hstride, 2, 2 * d, vswz),
        ("k8", row8, tok8, h8, 1, d, swz_k),
        ("v8", row8, tok8, h8, 1, d, swz_k),
    ]


@pytest.mark.parametrize("kernel,d,dp,hk,hstride,lens", CASES)
def test_copies_read_only_valid_elements(kernel, d, dp, hk, hstride, lens):
    for name, rowb, tok, head, elem, valid, swz in _streams(kernel, dp, d, hstride, hk):
        offs = lane_offsets(kernel, rowb, tok, swz, valid)
        addr = bytes_read(offs, lens, hk, tok, head, kernel)
        assert addr.size > 0
        bad = check_elements(addr, lens, hk, tok, head, elem, d)
        assert bad == 0, f"{name}: {bad} bytes outside the valid elements"


@pytest.mark.parametrize("kernel", [32, 16])
def test_planted_unmasked_copy_reads_past_the_end(kernel):
    """Without the head_dim mask, d=80 in a dense [N, 3, 80] K reads past the
    tensor's end (last head, last token) and into the neighbouring head."""
    d, dp, hk, lens = 80, 128, 3, [1, 63, 64, 65, 130]
    name, rowb, tok, head, elem, valid, swz = _streams(kernel, dp, d, d, hk)[0]
    offs = lane_offsets(kernel, rowb, tok, swz, valid, mask=False)
    addr = bytes_read(offs, lens, hk, tok, head, kernel)
    n_bytes = sum(lens) * tok
    assert addr.max() >= n_bytes  # past the end of the allocation
    assert check_elements(addr, lens, hk, tok, head, elem, d) > 0


def _outside_lanes_in_range(kernel, L, tok, d=80, dp=128):
    """Dwords of padded-column lanes (kOffOutside) of a kernel's K copies that
    land inside the sequence's buffer, over all tiles of a sequence of L keys
    (the tile offset added in 32 bits)."""
    rowb = 2 * dp
    offs = lane_offsets(kernel, rowb, tok, swz_k, 2 * d)
    outside = offs[offs >= OUTSIDE]
    assert outside.size > 0
    n_in = 0
    for t in range((L + 63) // 64):
        dw, size = tile_dwords(kernel, outside, L, t, tok)
        n_in += int((dw < size).sum())
    return n_in


@pytest.mark.parametrize("kernel", [32, 16])
def test_span_check_keeps_padded_lanes_out_of_range(kernel):
    """attn.hip rejects (max_seqlen_k + 64) * token stride >= 2^31: at the
    largest accepted length, no padded-column lane's offset (0x80000000 + tile
    offset + copy step) wraps past 2^32 back into the buffer."""
    tok = 3 << 18  # 768 KiB per token: a few thousand keys reach the limit
    L = ((1 << 31) - 1) // tok - 64
    assert (L + 64) * tok < 1 << 31
    assert _outside_lanes_in_range(kernel, L, tok) == 0


def test_planted_span_check_without_slack_wraps():
    """With the check as max(max_seqlen_k, 64) * token stride < 2^31 (no
    64-row slack), the longest accepted sequence lets padded-column offsets
    of its last tiles wrap into the buffer: the slack is needed."""
    tok = 3 << 18
    L = ((1 << 31) - 1) // tok
    assert max(L, 64) * tok < 1 << 31
    assert _outside_lanes_in_range(32, L, tok) > 0


def test_lds_receives_every_valid_chunk_once():
    """The copies of one tile fill each (row, column chunk < head_dim) exactly
    once: the mask removes only padded columns (32-row kernel, K fp16, d=80)."""
    d, dp, hk = 80, 128, 1
    rowb, tok = 2 * dp, 2 * d
    rpi, cpr, nw = 1024 // rowb, rowb // 16, 4
    seen = np.zeros((64, cpr), dtype=np.int64)
    for o in lane_offsets(32, rowb, tok, swz_k, 2 * d):
        if o >= OUTSIDE:
            continue
        seen[o // tok, (o % tok) // 16] += 1
    assert (seen[:, : 2 * d // 16] == 1).all()
    assert (seen[:, 2 * d // 16:] == 0).all()


# ---------------------------------------------------------------- Q block copy
def q_copy_size(lq, row0w, tok, wave_rows=True):
    """Byte size of a wave's Q buffer as the kernel stores it: a 32-bit value
    (make_srsrc takes an int), sized to the rows the wave reads (at most 32);
    ``wave_rows=False`` plants the size of every row left in the sequence."""
    if row0w >= lq:
        return 0
    rows = min(lq - row0w, 32) if wave_rows else lq - row0w
    return (rows * tok) & 0xFFFFFFFF


def q_padded_lanes_inside(lq, tok, d=80, dp=128, wave_rows=True):
    """Dwords of the Q copies' padded-column lanes (kOffOutside) that land
    inside their wave's buffer, over every wave of every query block of a
    sequence of lq rows with token stride tok bytes.  (The swizzle depends on
    the row mod 16, so every wave has the same padded lanes.)"""
    row16 = 2 * dp
    qrpi, qcpr = 1024 // row16, row16 // 16
    offs = []
    for i in range(32 // qrpi):
        for lane in range(64):
            rl = i * qrpi + lane // qcpr
            if ((lane % qcpr) ^ swz_k(row16, rl)) * 16 >= 2 * d:
                offs += [OUTSIDE + 4 * dw for dw in range(4)]
    offs = np.array(offs, dtype=np.int64)
    sizes = np.array([q_copy_size(lq, r, tok, wave_rows) for r in range(0, lq, 32)], dtype=np.int64)
    return int((offs[None, :] < sizes[:, None]).sum())


def test_q_buffer_size_is_the_waves_rows():
    """d = 80 with 32 query heads (5120-byte tokens) and 2^20 query rows: the
    sequence's remaining rows span more than 2^31 bytes, but a wave's buffer is
    sized to its 32 rows, so no padded-column lane reads inside it.  Sized to
    the rest of the sequence (planted), the 32-bit size lets those lanes read
    2 GiB past the wave's rows."""
    lq, tok = 1 << 20, 2 * 80 * 32
    assert 128 * tok < 1 << 31  # the host's Q stride check passes
    assert q_padded_lanes_inside(lq, tok) == 0
    assert q_padded_lanes_inside(lq, tok, wave_rows=False) > 0


def q_block_through_lds(q, cu, h, m, d, dp, read_swz_from_block_row=False, copy_swizzle=True):
    """Model of the 32-row kernel's Q staging for query block m (128 rows) of
    every sequence, head h: each wave w copies rows 32 w .. 32 w + 31 of the
    block into LDS (K-tile layout, raw buffer based at the wave's first row,
    sized to the rows left in the sequence), then lane (l32, hi) reads k-step s
    at (row * ROW16 + ((16 hi) ^ (16 swz_k(l32)))) ^ (32 s).  Returns, per
    sequence, the [128, DP] fp16 block as the lanes see it, and the relative
    byte addresses every copy read.  ``read_swz_from_block_row`` swizzles the
    read with the block row instead of the lane's (equivalent: the swizzle
    depends on the row mod 16); ``copy_swizzle=False`` plants an unswizzled copy."""
    row16 = 2 * dp
    qrpi, qcpr = 1024 // row16, row16 // 16
    qins = 32 // qrpi
    ntok, hq, hstride = q.shape
    tok = 2 * hstride * hq
    raw = q.view(np.uint8).reshape(-1)
    blocks, reads = [], []
    for z in range(len(cu) - 1):
        lq = int(cu[z + 1] - cu[z])
        lds = np.full(128 * row16, 0xEE, dtype=np.uint8)
        for w in range(4):
            row0w = m * 128 + 32 * w
            base = (int(cu[z]) + row0w) * tok + h * 2 * hstride
            size = q_copy_size(lq, row0w, tok)
            for i in range(qins):
                for lane in range(64):
                    rl = i * qrpi + lane // qcpr
                    chunk = (lane % qcpr) ^ (swz_k(row16, w * 32 + rl) if copy_swizzle else 0)
                    off = OUTSIDE if chunk * 16 >= 2 * d else rl * tok + chunk * 16
                    dst = (w * 32 + i * qrpi) * row16 + lane * 16
                    for dw in range(4):
                        o = off + 4 * dw
                        if o < size:
                            reads.append(base + o + np.arange(4))
                            lds[dst + 4 * dw:dst + 4 * dw + 4] = raw[base + o:base + o + 4]
                        else:
                            lds[dst + 4 * dw:dst + 4 * dw + 4] = 0
        got = np.zeros((128, dp), dtype=np.float16)
        for w in range(4):
            for lane in range(64):
                l32, hi = lane & 31, lane >> 5
                r = w * 32 + l32
                sw = swz_k(row16, r if read_swz_from_block_row else l32)
                qbase = r * row16 + ((16 * hi) ^ (16 * sw))
                for s in range(dp // 16):
                    a = qbase ^ (32 * s)
                    got[r, 16 * s + 8 * hi:16 * s + 8 * hi + 8] = lds[a:a + 16].view(np.float16)
        blocks.append(got)
    return blocks, (np.concatenate(reads) if reads else np.zeros(0, dtype=np.int64))


# d, DP, Hq, head stride (elements), lengths, block m
Q_CASES = [
    (128, 128, 3, 128, [300, 129, 1], 0),
    (128, 128, 3, 128, [300, 129, 1], 1),
    (80, 128, 2, 128, [200, 37], 1),     # [..., :80] view of a 128-wide buffer
    (80, 128, 2, 80, [140, 129], 1),
    (48, 64, 3, 48, [100, 130], 0),
    (64, 64, 2, 64, [257], 2),
]


@pytest.mark.parametrize("d,dp,hq,hstride,lens,m", Q_CASES)
def test_q_block_staging(d, dp, hq, hstride, lens, m):
    """Each lane receives exactly Q[row][16 s + 8 hi .. + 7] of its row (zeros
    past the sequence end and past head_dim), and every byte the copies read
    belongs to a valid element of the block's own head."""
    rng = np.random.default_rng(d + m)
    ntok = sum(lens)
    q = np.full((ntok, hq, hstride), np.nan, dtype=np.float16)  # padding and other heads: NaN
    q[:, :, :d] = rng.standard_normal((ntok, hq, d)).astype(np.float16)
    cu = np.concatenate([[0], np.cumsum(lens)])
    for h in range(hq):
        blocks, addr = q_block_through_lds(q, cu, h, m, d, dp)
        tok = 2 * hstride * hq
        if addr.size:
            head, col = (addr % tok) // (2 * hstride), (addr % (2 * hstride)) // 2
            assert addr.max() < ntok * tok and (head == h).all() and (col < d).all()
        for z, got in enumerate(blocks):
            lq = int(cu[z + 1] - cu[z])
            want = np.zeros((128, dp), dtype=np.float16)
            rows = max(0, min(128, lq - m * 128))
            want[:rows, :d] = q[cu[z] + m * 128:cu[z] + m * 128 + rows, h, :d]
            np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


def test_q_block_read_swizzle_uses_the_lane_row():
    """The fragment reads swizzle with the lane's row l32 rather than the block
    row 32 w + l32: the same value for every wave (the swizzle depends on the
    row mod 16), checked at both row widths."""
    for dp in (64, 128):
        q = np.random.default_rng(dp).standard_normal((256, 1, dp)).astype(np.float16)
        cu = np.array([0, 256])
        got, _ = q_block_through_lds(q, cu, 0, 0, dp, dp, read_swz_from_block_row=True)
        ok, _ = q_block_through_lds(q, cu, 0, 0, dp, dp)
        assert np.array_equal(ok[0].view(np.uint16), q[:128, 0].view(np.uint16))
        assert np.array_equal(got[0].view(np.uint16), ok[0].view(np.uint16))


def test_q_block_staging_planted_unswizzled_copy():
    """A copy that skips the K swizzle puts chunks where the reads do not look:
    the model catches it."""
    q = np.random.default_rng(1).standard_normal((256, 1, 128)).astype(np.float16)
    cu = np.array([0, 256])
    got, _ = q_block_through_lds(q, cu, 0, 0, 128, 128, copy_swizzle=False)
    assert not np.array_equal(got[0].view(np.uint16), q[:128, 0].view(np.uint16))

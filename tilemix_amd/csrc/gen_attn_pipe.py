"""Generates attn_pipe_asm.h: the software-pipelined tile loop of the 32-row
attention kernel (attn_kernel32.h, PIPE instantiations) as gfx950 assembly.

build.py runs this script before every build.  The generated header is also
committed, and tests/test_pipe_codegen.py checks it against this script's
output.

Scope: a 128-row workgroup (4 waves x 32 query rows), head_dim 128, 64-key
tiles, fp16 V, and the tiles [0, n_sw) that need no mask for any row of the
workgroup.  The whole loop over those tiles is ONE inline-assembly statement
(pipe_loop_<mode>), so the loop-carried state (the O accumulators, the scores
of the next tile, m / alpha / -m / l) stays in fixed registers: the compiler
moves values only at the statement's boundary.  Modes: f16, i8 and mixed
routing, and split (mixed routing at block_m 64: the workgroup's two 64-row
halves route separately, a 40 KB stage holds K in both formats when their
routes differ, and each wave takes its own half's route).

Iteration n (stage parity P = n & 1; tile t's K sits in K slot t & 1, its V in
V slot t & 1), in the order of the default schedule options (OPTS below):
  1. s_waitcnt vmcnt(0) + s_barrier: this wave's copies of K(n+1) and V(n)
     have landed, every wave's have, and every wave is done with K(n) and
     V(n-1);
  2. the first four LDS operand reads of tile n+1's QK;
  3. copies: K(n+2) into K slot P (with its route and K scale, while
     n+2 <= n_sw and n+2 < n_blocks) and V(n+1) into V slot 1-P;
  4. the last steps of tile n's running maximum: m' = max(m, mx),
     alpha = exp2(min(m - mx, 0)), -m' (computed from the row maximum that
     the previous body left in a temporary);
  5. phase A: QK MFMAs of tile n+1 (fp16: 16 x 32x32x16, int8: 8 x 32x32x32)
     beside tile n's softmax, p = fp16(exp2(fp32(s) - m')), its row sum, and
     the O rescale of d block 0; the first PV operand reads go out beside
     the last four QK MFMAs;
  6. phase B: PV MFMAs of tile n (16 x 32x32x16 f16) beside the rest of the O
     rescale, the l update, the conversion of tile n+1's accumulators to fp16
     scores (INT8 tiles: fma(acc bits, ss, -1.5 2^23 ss), the single
     rounding of acc * ss), the INT8 bias refill when the tile after next is
     an INT8 tile, and tile n+1's packed row maximum.
Before the loop, FILL runs tile 0's QK, conversion and maximum (after the
barrier that also ends the Q block's use of stage 1, and the copy of K(1));
the last iteration (DRAIN) has no next tile.  The C++ tile body continues at
tile n_sw with K(n_sw) and V(n_sw) in flight, the route / scale bookkeeping
and the copy offsets handed back through the statement's outputs.

Numerics: instruction for instruction those of the C++ tile body (the same
conversions and roundings, the row sum over the 16 pairs in the same order,
PV accumulated over the k-steps in the same order, the same scale
arithmetic), so the outputs are bit-identical to it.  Two reformulations, both
exact: alpha = exp2(min(m - mx, 0)) equals exp2(m - max(m, mx)) (1 when the
tile brings nothing new), and -m' is clamped to FLT_MAX so p = exp2(-inf +
FLT_MAX) = 0 while every score so far is -inf.  INT8 chains start from the
QK accumulator registers preloaded with 1.5 * 2^23 as int bits (refilled with
two 64-bit moves per pair after each conversion), the magic bias of the C++
body.

Register map:
  v[0:63]    O accumulators, d blocks 0..3
  v[64:79]   packed fp16 scores of the tile whose softmax is next
  v[80:111]  QK accumulators of the next tile (kb 0, kb 1)
  v[112:127] packed fp16 p of the current tile (the PV B operands)
  v[128:143] four 4-VGPR slots for the LDS operand reads (K in A, V in B)
  v[144:150] softmax / maximum temporaries and the row-sum accumulator
  v151, v152 INT8 dequant scale ss and -1.5 2^23 ss
  v153       copy offset
Everything else is an ordinary operand (Q fragments, int8 Q codes, LDS read
addresses, copy descriptors and offsets, the route bits and counters).

Hazards (gfx950; the compiler does not look inside the statement): an MFMA
result is read by VALU code no sooner than ~18 instructions after the MFMA; a
VALU write to an O block or to the INT8 accumulators precedes the MFMA that
reads it by at least three wait states (pad_valu_mfma inserts the s_nop where
the schedule does not provide them); an exp result is never read by the next
instruction; v_permlane32_swap's operand is written two wait states earlier;
the row sum a v_dot2c chain accumulates (a DOT result) is read or overwritten
by another instruction no sooner than three wait states after the last
v_dot2c (the l update reads it a whole phase later); one wait state
separates an M0 write from the LDS-DMA copy that uses it.  LDS
waits count only the statement's own reads (every compute body starts with
s_waitcnt lgkmcnt(0), and the scale loads are VMEM loads); auto_wait derives
them from the operand registers of each read's first use.
tests/test_pipe_codegen.py replays every body against these rules.
"""
from __future__ import annotations

import re
import sys
from contextlib import contextmanager
from pathlib import Path

ACC = (0, 16, 32, 48)
S16 = 64
QA, QB = 80, 96
P = 112
RING = 128
T = 144
LS = 150
SS, NMS = 151, 152
VO = 153
STAGE = 32768  # bytes per LDS stage (K 16 KB + V 16 KB)
VOFF = 16384   # V slot offset inside a stage
# Split workgroups (block_m 64: the two 64-row halves route separately): a
# stage holds K in both formats, int8 K after V.
SPLIT_STAGE, SPLIT_K8OFF = 40960, 32768
ROW16, ROW8 = 256, 128
NW = 4
K16_INS, K8_INS, V16_INS = 4, 2, 4  # 1 KB copies per wave and tile

# Schedule options (the defaults are the measured production choice):
#   copy_at       the tile copies go out after this phase-A MFMA (None: before
#                 the compute body);
#   skip_refill   the INT8 accumulator refill is skipped when the tile after
#                 next is an FP16 tile;
#   skip_rescale  the O rescale is skipped when alpha = 1 on every row of the
#                 wave (an exact no-op then).
#   qk_il         the two QK chains (kb 0, kb 1) alternate MFMA by MFMA;
#   pv_il         the PV chains of d blocks (0, 1) and then (2, 3) alternate;
#   early         the first four K operand reads go out right after the
#                 barrier, before the tile copies (the drain: its first V
#                 reads), so the copy issue covers their LDS latency;
#   v_ahead       the first four PV operand reads go out beside the last four
#                 QK MFMAs (their ring slots are free by then);
#   tail_first    the last steps of the running maximum (m', alpha, -m') run
#                 at the start of the next iteration, after its reads and
#                 copies, instead of at the end of the body;
#   auto_wait     LDS waits are recomputed from the operand registers (always
#                 on with early / v_ahead);
#   v_spread      in a body with a next tile, the four V copies go out one by
#                 one after QK MFMAs 1, 3, 5 and 7 instead of with the K copy;
#   wait_pairs    one LDS wait per two MFMAs (see auto_wait).
OPTS = {"copy_at": None, "skip_refill": True, "skip_rescale": False, "qk_il": False, "pv_il": False,
        "early": True, "v_ahead": True, "tail_first": True, "auto_wait": False, "v_spread": False,
        "wait_pairs": True}

# The launch the loop is generated for (loop_asm sets it per mode): the stage
# size, the int8 K offset inside a stage, and whether routes are per half
# (split: %[rn] / %[rn2] carry the low half's route in bit 0 and the high
# half's in bit 1, and each wave tests bit %[half]).
LAYOUT = {"stage": STAGE, "k8off": 0, "split": False, "mode": "mixed"}


@contextmanager
def layout(mode: str):
    saved = dict(LAYOUT)
    LAYOUT["mode"] = mode
    if mode == "split":
        LAYOUT.update(stage=SPLIT_STAGE, k8off=SPLIT_K8OFF, split=True)
    try:
        yield
    finally:
        LAYOUT.clear()
        LAYOUT.update(saved)


def qk_step(i: int, nm: int) -> tuple[int, int]:
    """(kb, ks) of the i-th QK MFMA of a tile with nm MFMAs (k-steps in order per chain)."""
    if OPTS["qk_il"]:
        return i % 2, i // 2
    return divmod(i, nm // 2)


def pv_step(i: int) -> tuple[int, int]:
    """(db, ks) of the i-th PV MFMA (k-steps in order per d block)."""
    if OPTS["pv_il"]:
        half, r = divmod(i, 8)
        return 2 * half + r % 2, r // 2
    return divmod(i, 4)


def vr(a: int, n: int) -> str:
    return f"v[{a}:{a + n - 1}]" if n > 1 else f"v{a}"


def slot(i: int) -> str:
    return vr(RING + 4 * (i % 4), 4)


# ---- compute blocks -----------------------------------------------------------

def read_k16(i: int, kslot: int) -> str:
    kb, ks = qk_step(i, 16)
    return f"ds_read_b128 {slot(i)}, %[ka{ks}] offset:{kslot * LAYOUT['stage'] + kb * 32 * ROW16}"


def read_k8(i: int, kslot: int) -> str:
    kb, ks = qk_step(i, 8)
    return f"ds_read_b128 {slot(i)}, %[k8a{ks}] offset:{kslot * LAYOUT['stage'] + kb * 32 * ROW8}"


def mfma_k16(i: int) -> str:
    kb, ks = qk_step(i, 16)
    d = QA if kb == 0 else QB
    c = "0" if ks == 0 else vr(d, 16)
    return f"v_mfma_f32_32x32x16_f16 {vr(d, 16)}, {slot(i)}, %[qf{ks}], {c}"


def mfma_k8(i: int) -> str:
    # The first k-step accumulates on top of the magic bias preloaded in the
    # accumulator registers.
    kb, ks = qk_step(i, 8)
    d = QA if kb == 0 else QB
    return f"v_mfma_i32_32x32x32_i8 {vr(d, 16)}, {slot(i)}, %[q8f{ks}], {vr(d, 16)}"


def reads_v(i: int, vslot: int) -> list[str]:
    db, ks = pv_step(i)
    base = RING + 4 * (i % 4)
    return [f"ds_read_b64_tr_b16 {vr(base + 2 * h2, 2)}, %[va{db}] "
            f"offset:{vslot * LAYOUT['stage'] + (16 * ks + 8 * h2) * ROW16}" for h2 in range(2)]


def mfma_pv(i: int) -> str:
    db, ks = pv_step(i)
    a = vr(ACC[db], 16)
    return f"v_mfma_f32_32x32x16_f16 {a}, {slot(i)}, {vr(P + 4 * ks, 4)}, {a}"


def softmax_steps() -> list[str]:
    """p = fp16(exp2(fp32(s) - m)) per packed score pair, skewed over three
    steps (subtract, exp, pack + row sum) so dependent instructions are apart;
    the row sum accumulates pairs 0..15 in order, from 0."""
    out = [f"v_mov_b32 v{LS}, 0"]
    for c in range(18):
        if c < 16:
            t0 = T + 2 * (c % 3)
            out.append(f"v_fma_mix_f32 v{t0}, v{S16 + c}, 1.0, %[ng] op_sel_hi:[1,0,0]")
            out.append(f"v_fma_mix_f32 v{t0 + 1}, v{S16 + c}, 1.0, %[ng] op_sel:[1,0,0] op_sel_hi:[1,0,0]")
        if 0 <= c - 1 < 16:
            t0 = T + 2 * ((c - 1) % 3)
            out.append(f"v_exp_f32 v{t0}, v{t0}")
            out.append(f"v_exp_f32 v{t0 + 1}, v{t0 + 1}")
        if 0 <= c - 2 < 16:
            j = c - 2
            t0 = T + 2 * (j % 3)
            out.append(f"v_cvt_pk_f16_f32 v{P + j}, v{t0}, v{t0 + 1}")
            out.append(f"v_dot2c_f32_f16 v{LS}, 0x3c003c00, v{P + j}")
    return out


def rescale(db: int) -> list[str]:
    return [f"v_mul_f32 v{ACC[db] + e}, %[al], v{ACC[db] + e}" for e in range(16)]


def l_update() -> list[str]:
    return ["v_mul_f32 %[li], %[li], %[al]", f"v_add_f32 %[li], %[li], v{LS}"]


def conv(pairs: range, int8: bool) -> list[str]:
    """Accumulators of the next tile -> packed fp16 scores (pair j = keys
    2j, 2j+1 of the lane's slots; pairs 0-7 from kb 0, 8-15 from kb 1)."""
    out = []
    for j in pairs:
        src = (QA if j < 8 else QB) + 2 * (j % 8)
        if int8:
            out.append(f"v_fma_f32 v{T + 4}, v{src}, v{SS}, v{NMS}")
            out.append(f"v_fma_f32 v{T + 5}, v{src + 1}, v{SS}, v{NMS}")
            out.append(f"v_cvt_pk_f16_f32 v{S16 + j}, v{T + 4}, v{T + 5}")
        else:
            out.append(f"v_cvt_pk_f16_f32 v{S16 + j}, v{src}, v{src + 1}")
    return out


def refill(base: int) -> list[str]:
    """1.5 * 2^23 as int bits into 16 accumulator registers (the C operand of
    the next INT8 chain's first MFMA)."""
    return [f"v_mov_b64 v[{base + 2 * i}:{base + 2 * i + 1}], %[magic2]" for i in range(8)]


def int8_scale(par_next: int) -> list[str]:
    """ss = fp16(fp32(fp16(sq * sk)) * qk_scale) as fp32, and -1.5 2^23 ss,
    for the tile whose K scale sits in the scale register of parity
    par_next."""
    return [f"v_mul_f16 v{T + 4}, %[sq16], %[sk{par_next}]",
            f"v_cvt_f32_f16 v{T + 4}, v{T + 4}",
            f"v_mul_f32 v{T + 4}, %[qks], v{T + 4}",
            f"v_cvt_f16_f32 v{T + 4}, v{T + 4}",
            f"v_cvt_f32_f16 v{SS}, v{T + 4}",
            f"v_mul_f32 v{NMS}, 0xcb400000, v{SS}"]


def s(j: int) -> str:
    return f"v{S16 + j}"


# Row maximum of the new scores (any tree: the packed IEEE maximum is exact
# and order independent), then the two lanes (l, l+32) of a row, then
# m' = max(m, mx), alpha = exp2(min(m - mx, 0)) and -m' clamped to FLT_MAX.
MAX_A = [f"v_pk_maximum3_f16 v{T + 0}, {s(0)}, {s(1)}, {s(2)}",
         f"v_pk_maximum3_f16 v{T + 1}, {s(3)}, {s(4)}, {s(5)}"]
MAX_B = [f"v_pk_maximum3_f16 v{T + 2}, {s(6)}, {s(7)}, v{T + 0}"]
MAX_C = [f"v_pk_maximum3_f16 v{T + 3}, {s(8)}, {s(9)}, {s(10)}"]
MAX_D = [f"v_pk_maximum3_f16 v{LS}, {s(11)}, {s(12)}, {s(13)}",
         f"v_pk_maximum3_f16 v{T + 4}, {s(14)}, {s(15)}, v{T + 1}",
         f"v_pk_maximum3_f16 v{T + 5}, v{T + 2}, v{T + 3}, v{LS}"]
MAX_E = [f"v_pk_max_f16 v{T + 0}, v{T + 5}, v{T + 4}",
         f"v_pk_max_f16 v{T + 1}, v{T + 0}, v{T + 0} op_sel:[1,0]",
         f"v_cvt_f32_f16 v{T + 2}, v{T + 1}"]
MAX_F = [f"v_mov_b32 v{T + 3}, v{T + 2}",
         "s_nop 1",
         f"v_permlane32_swap_b32 v{T + 2}, v{T + 3}",
         f"v_max_f32 v{T + 2}, v{T + 2}, v{T + 3}"]
MAX_TAIL = [f"v_sub_f32 v{T + 4}, %[mn], v{T + 2}",
            f"v_min_f32 v{T + 4}, 0, v{T + 4}",
            f"v_exp_f32 %[al], v{T + 4}",
            f"v_max_f32 %[mn], %[mn], v{T + 2}",
            "v_min_f32 %[ng], -%[mn], %[fmax]"]


def spread(items: list[str], n: int) -> list[list[str]]:
    """Split items into n consecutive chunks of near-equal size."""
    out, k = [], 0
    for i in range(n):
        m = (len(items) - k) // (n - i)
        out.append(items[k:k + m])
        k += m
    return out


def phase_a(kind: str, kslot: int, valu: list[str], copy: list[str] | None = None,
            tail: list[str] | None = None, pre: list[str] | None = None,
            vslot: int | None = None, vgroups: list[list[str]] | None = None) -> list[str]:
    """kind: 'f16' / 'i8' QK of the next tile, or 'none' (VALU only).  copy:
    the tile copies, placed after MFMA OPTS['copy_at'] (OPTS['early']: after
    the first operand reads); pre: VALU work after the first reads and the
    copies, before the first MFMA; tail: after the last chunk; vslot: the V
    slot whose first PV operand reads go out beside the last four MFMAs."""
    copy, tail, pre = copy or [], tail or [], pre or []
    if kind == "none":
        assert not vgroups
        return copy + pre + list(valu) + tail
    nm = 16 if kind == "f16" else 8
    rd = read_k16 if kind == "f16" else read_k8
    mf = mfma_k16 if kind == "f16" else mfma_k8
    early = OPTS["early"]
    out = [rd(i, kslot) for i in range(4)]
    if early:
        out += copy
    out += pre
    chunks = spread(valu, nm)
    at = min(OPTS["copy_at"] or 0, nm - 1)
    for i in range(nm):
        out += [f"s_waitcnt lgkmcnt({min(3, nm - 1 - i)})", mf(i)]
        if i + 4 < nm:
            out.append(rd(i + 4, kslot))
        elif vslot is not None:
            out += reads_v(i - (nm - 4), vslot)
        if i == at and not early:
            out += copy
        if vgroups and i % 2 == 1 and i // 2 < len(vgroups):
            out += vgroups[i // 2]
        out += chunks[i]
    return out + tail


def phase_b(vslot: int, chunks: list[list[str]], tail: list[str], pre_read: bool = False) -> list[str]:
    """pre_read: the first four MFMAs' operand reads were issued earlier."""
    out: list[str] = []
    if not pre_read:
        for i in range(4):
            out += reads_v(i, vslot)
    for i in range(16):
        out += [f"s_waitcnt lgkmcnt({min(6, 30 - 2 * i)})", mfma_pv(i)]
        if i + 4 < 16:
            out += reads_v(i + 4, vslot)
        out += chunks[i]
    return out + tail


_REG = re.compile(r"v\[(\d+):(\d+)\]|\bv(\d+)\b")


def _regs(tok: str) -> set[int]:
    out: set[int] = set()
    for m in _REG.finditer(tok):
        if m.group(1) is not None:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
        else:
            out.add(int(m.group(3)))
    return out


def _next_mfma(lines: list[str], k: int) -> str | None:
    """The next MFMA after line k in straight-line code (None past a label or
    a branch)."""
    for ln in lines[k + 1:]:
        if ln.endswith(":") or ln.startswith("s_cbranch") or ln.startswith("s_branch"):
            return None
        if ln.startswith("v_mfma"):
            return ln
    return None


def auto_wait(lines: list[str]) -> list[str]:
    """The body's LDS waits, recomputed as the minimal ones: before an
    instruction that reads or overwrites the destination of an outstanding
    LDS read, wait until that read has returned (LDS reads return in order).
    OPTS['wait_pairs']: a wait before an MFMA also covers the outstanding
    reads of the next MFMA, which then needs none (half the waits).  A full
    drain at the body's start is kept.  The only branches inside a body skip
    blocks without LDS reads, so both paths see the same outstanding reads."""
    out: list[str] = []
    pending: list[set[int]] = []
    for k, ln in enumerate(lines):
        if ln.startswith("s_waitcnt lgkmcnt("):
            if k == 0:
                out.append(ln)
            continue
        if ln.endswith(":") or ln.startswith("s_") or ln.startswith("buffer_"):
            out.append(ln)
            continue
        op, _, rest = ln.partition(" ")
        regs = _regs(rest)
        hit = [j for j, d in enumerate(pending) if d & regs]
        if hit:
            j = max(hit)
            nxt = _next_mfma(lines, k) if OPTS["wait_pairs"] and op.startswith("v_mfma") else None
            if nxt is not None:
                regs2 = _regs(nxt.partition(" ")[2])
                j = max([j] + [i for i, d in enumerate(pending) if d & regs2])
            out.append(f"s_waitcnt lgkmcnt({len(pending) - 1 - j})")
            pending = pending[j + 1:]
        out.append(ln)
        if op.startswith("ds_read"):
            pending.append(_regs(rest.split(",")[0]))
    return out


def pad_valu_mfma(lines: list[str]) -> list[str]:
    """An s_nop before an MFMA that reads a register a VALU instruction wrote
    fewer than three wait states earlier (each instruction is one wait
    state, s_nop k is k + 1)."""
    out: list[str] = []
    written: dict[int, int] = {}  # register -> clock of its last VALU write
    clock = 0
    for ln in lines:
        if ln.endswith(":"):
            out.append(ln)
            continue
        op, _, rest = ln.partition(" ")
        if op.startswith("v_mfma"):
            gap = min((clock - written[r] for r in _regs(rest) if r in written), default=3)
            if gap < 3:
                out.append(f"s_nop {2 - gap}")
                clock += 3 - gap
        elif op.startswith("v_"):
            for r in _regs(rest.split(",")[0]):
                written[r] = clock
        out.append(ln)
        clock += int(rest) + 1 if op == "s_nop" else 1
    return out


def guard_rescale(lines: list[str], lbl: str) -> list[str]:
    """Skip an O rescale block when no lane has alpha != 1 (VCC, set at the
    start of the body)."""
    return [f"s_cbranch_vccz {lbl}"] + lines + [f"{lbl}:"]


def guard_refill(lines: list[str], lbl: str, test: bool = True) -> list[str]:
    """Skip an accumulator refill when the tile after next is an FP16 tile
    (split: for this wave's half).  test=False: SCC still holds the test of
    the previous guard (body_iter checks that nothing in between writes SCC).
    With int8 routing every tile is an INT8 tile: always refill."""
    if LAYOUT["mode"] == "i8":
        return list(lines)
    t = ["s_bitcmp0_b32 %[rn2], %[half]" if LAYOUT["split"] else "s_cmp_eq_u32 %[rn2], 0"] if test else []
    return t + [f"s_cbranch_scc1 {lbl}"] + lines + [f"{lbl}:"]


_NO_SCC = ("s_nop", "s_waitcnt", "s_cbranch", "s_branch", "s_barrier", "s_setprio")


def check_scc_kept(lines: list[str], lbl_a: str, lbl_b: str) -> None:
    """No instruction between the end of guard lbl_a and the branch to lbl_b
    writes SCC (so the second guard may reuse the first one's test)."""
    if f"{lbl_a}:" not in lines or f"s_cbranch_scc1 {lbl_b}" not in lines:
        return
    i, j = lines.index(f"{lbl_a}:"), lines.index(f"s_cbranch_scc1 {lbl_b}")
    for ln in lines[i + 1:j]:
        if ln.startswith("s_") and not ln.startswith(_NO_SCC):
            raise AssertionError(f"SCC written between the refill guards: {ln}")


def to_int8_body(lbl: str) -> list[str]:
    """Branch to lbl when the next tile to compute is an INT8 tile (split: for
    this wave's half)."""
    if LAYOUT["split"]:
        return ["s_bitcmp1_b32 %[rn], %[half]", f"s_cbranch_scc1 {lbl}"]
    return ["s_cmp_eq_u32 %[rn], 0", f"s_cbranch_scc0 {lbl}"]


def b_chunks(kind: str, mixed_regs: bool, lbl: str) -> tuple[list[list[str]], list[str]]:
    """VALU of phase B: the l update and the O rescale of d blocks 1..3 (each
    done a chunk before the first MFMA into that block), and, with a next
    tile, its conversion, the accumulator refill and the row maximum."""
    r1, r2, r3 = rescale(1), rescale(2), rescale(3)
    ch: list[list[str]] = [[] for _ in range(16)]
    if OPTS["pv_il"]:
        # d blocks 0 and 1 are rescaled in phase A; 2 and 3 before MFMA 8
        r23 = r2 + r3
        ch[0] = l_update() + r23[:6]
        for c in range(1, 6):
            ch[c] = r23[6 * c:6 * c + 6]
    elif OPTS["skip_rescale"]:
        ch[0] = l_update() + guard_rescale(r1, f"{lbl}_rs1")
        ch[4] = guard_rescale(r2, f"{lbl}_rs2")
        ch[8] = guard_rescale(r3, f"{lbl}_rs3")
    else:
        ch[0] = l_update() + r1[:5]
        ch[1], ch[2] = r1[5:11], r1[11:]
        ch[4], ch[5], ch[6] = r2[:5], r2[5:11], r2[11:]
        ch[8], ch[9], ch[10] = r3[:5], r3[5:11], r3[11:]
    tail: list[str] = []
    if kind != "none":
        i8 = kind == "i8"
        ch[3] += conv(range(0, 4), i8)
        ch[7] += conv(range(4, 8), i8) + MAX_A
        ch[11] += conv(range(8, 12), i8) + MAX_B
        ch[12] += conv(range(12, 16), i8) + MAX_C
        ch[13] += MAX_D
        ch[14] += MAX_E
        ch[15] += MAX_F
        tail = [] if OPTS["tail_first"] else list(MAX_TAIL)
        if mixed_regs:
            fa, fb = refill(QA), refill(QB)
            if OPTS["skip_refill"]:
                ch[9] = ch[9] + guard_refill(fa, f"{lbl}_rfa")
                ch[14] = ch[14] + guard_refill(fb, f"{lbl}_rfb", test=False)
            else:
                ch[8] = ch[8] + fa[:4]
                ch[9] = ch[9] + fa[4:]
                ch[13] = ch[13] + fb[:4]
                ch[14] = ch[14] + fb[4:]
    return ch, tail


def body_iter(kind: str, kslot: int, vslot: int, mixed_regs: bool, par_next: int, lbl: str = ".Lb",
              copy: list[str] | None = None, vgroups: list[list[str]] | None = None) -> list[str]:
    early, v_ahead = OPTS["early"], OPTS["v_ahead"] and kind != "none"
    pre: list[str] = list(MAX_TAIL) if OPTS["tail_first"] else []
    if OPTS["skip_rescale"]:
        pre.append("v_cmp_neq_f32 vcc, 1.0, %[al]")
    if kind == "i8":
        pre += int8_scale(par_next)
    # no LDS read is outstanding when a body starts (the previous body's
    # reads were all consumed by its MFMAs)
    out: list[str] = []
    if not early:
        out, pre = out + pre, []
    elif kind == "none":
        # the drain computes no QK: its first PV operand reads go out first
        for i in range(4):
            out += reads_v(i, vslot)
        out, pre, copy = out + (copy or []) + pre, [], None
    vs = vslot if v_ahead else None
    if OPTS["pv_il"]:
        out += phase_a(kind, kslot, softmax_steps() + rescale(0) + rescale(1), copy, None, pre, vs, vgroups)
    elif OPTS["skip_rescale"]:
        out += phase_a(kind, kslot, softmax_steps(), copy, guard_rescale(rescale(0), f"{lbl}_rs0"), pre, vs,
                       vgroups)
    else:
        out += phase_a(kind, kslot, softmax_steps() + rescale(0), copy, None, pre, vs, vgroups)
    ch, tail = b_chunks(kind, mixed_regs, lbl)
    out += phase_b(vslot, ch, tail, pre_read=v_ahead or (early and kind == "none"))
    if early or v_ahead or OPTS["auto_wait"] or OPTS["wait_pairs"]:
        out = pad_valu_mfma(auto_wait(out))
    check_scc_kept(out, f"{lbl}_rfa", f"{lbl}_rfb")
    return out


def body_fill(kind: str, kslot: int, mixed_regs: bool, lbl: str = ".Lf") -> list[str]:
    out = ["s_waitcnt lgkmcnt(0)"]
    if kind == "i8":
        # tile 0's INT8 chains start from the magic bias as well
        out += refill(QA) + refill(QB) + int8_scale(0)
    out += phase_a(kind, kslot, [])
    # the last QK MFMA's result is read by the conversion below
    out += ["s_nop 15", "s_nop 3"]
    out += conv(range(16), kind == "i8")
    if mixed_regs:
        if OPTS["skip_refill"]:
            out += guard_refill(refill(QA) + refill(QB), f"{lbl}_rf")
        else:
            out += refill(QA) + refill(QB)
    out += MAX_A + MAX_B + MAX_C + MAX_D + MAX_E + MAX_F
    if not OPTS["tail_first"]:
        out += MAX_TAIL
    return out


# ---- copies and bookkeeping (SALU / VMEM) ---------------------------------------
#
# A wave issues at most one instruction per issue slot, and on gfx950 every
# s_waitcnt, s_nop and SALU instruction costs a wave about as much issue time
# as a VALU instruction (probe: ~4 clk each, a taken branch 7-10 clk, also
# with two waves per SIMD).  The bookkeeping below is therefore branch-free
# where it can be, the M0 write of a copy is separated from the copy by the
# copy's own address add instead of an s_nop, and the loop tests the drain
# and the waves without rows once per item instead of once per tile.

def routed(mode: str) -> bool:
    """The route of a tile comes from the route bits (else it is constant)."""
    return mode in ("mixed", "split")


def _copy(dest: int, addr: str, rsrc: str) -> list[str]:
    """One 1 KB copy: M0 (LDS destination), the lane's address (the one wait
    state M0 needs before the copy), the LDS-DMA load."""
    return [f"s_add_u32 m0, %[ldsw], {dest}", addr, f"buffer_load_dwordx4 v{VO}, %[{rsrc}], 0 offen lds"]


def copy_k(mode: str, par: int, lbl: str) -> list[str]:
    """K(t) for t = n + 2 (in %[t]) into K slot par, with its route (->
    %[rn2]), its K scale (-> scale register par) and the bookkeeping advance
    of the C++ issue_next_k: route group, scale block, tile offsets."""
    out: list[str] = []
    if mode == "mixed":
        out += ["s_bitcmp1_b64 %[bits], %[grp]", "s_cselect_b32 %[rn2], 1, 0"]
    elif mode == "split":
        # bit 1: the high half's route; bit 0: the low half's, or the high
        # half's for a tile past the low half's last key
        out += ["s_bitcmp1_b64 %[bitsh], %[grp]", "s_cselect_b32 %[rn2], 3, 0",
                "s_cmp_ge_u32 %[t], %[lolim]", f"s_cbranch_scc1 {lbl}_past",
                "s_and_b32 %[rn2], %[rn2], 2", "s_bitcmp1_b64 %[bits], %[grp]", "s_cselect_b32 %[t], 1, 0",
                "s_or_b32 %[rn2], %[rn2], %[t]", f"{lbl}_past:"]
    if routed(mode):
        # route group: ++gc == mask_tiles -> gc = 0, ++grp
        out += ["s_add_u32 %[gc], %[gc], 1", "s_cmp_eq_u32 %[gc], %[mt]", "s_cselect_b32 %[gc], 0, %[gc]",
                "s_addc_u32 %[grp], %[grp], 0"]

    def k16() -> list[str]:
        o: list[str] = []
        for i in range(K16_INS):
            addr = (f"v_add_u32 v{VO}, %[tok16], %[dk16]" if i == 0 else f"v_add_u32 v{VO}, %[stpk16], v{VO}")
            o += _copy(par * LAYOUT["stage"] + i * NW * 1024, addr, "rsk16")
        return o

    def k8() -> list[str]:
        o: list[str] = []
        for i in range(K8_INS):
            addr = (f"v_add_u32 v{VO}, %[tok8], %[dk8]" if i == 0 else f"v_add_u32 v{VO}, %[stpk8], v{VO}")
            o += _copy(par * LAYOUT["stage"] + LAYOUT["k8off"] + i * NW * 1024, addr, "rsk8")
        # the tile's K scale (clamped lookup: the pointer stops at the last block)
        o += ["s_cmp_eq_u32 %[hask], 0", f"s_cbranch_scc1 {lbl}_nosk",
              f"buffer_load_ushort %[sk{par}], off, %[rssk], %[skoff]", f"s_branch {lbl}_skd",
              f"{lbl}_nosk:", f"v_mov_b32 %[sk{par}], 0x3c00", f"{lbl}_skd:"]
        return o

    if mode == "f16":
        out += k16()
    elif mode == "i8":
        out += k8()
    elif mode == "split":
        # fp16 K unless both halves are INT8, int8 K (and the scale) unless both are FP16
        out += ["s_cmp_eq_u32 %[rn2], 3", f"s_cbranch_scc1 {lbl}_n16"] + k16() + [f"{lbl}_n16:"]
        out += ["s_cmp_eq_u32 %[rn2], 0", f"s_cbranch_scc1 {lbl}_n8"] + k8() + [f"{lbl}_n8:"]
    else:
        out += ["s_cmp_eq_u32 %[rn2], 0", f"s_cbranch_scc0 {lbl}_k8"]
        out += k16()
        out += [f"s_branch {lbl}_kd", f"{lbl}_k8:"]
        out += k8()
        out += [f"{lbl}_kd:"]
    if mode != "i8":
        out += ["s_add_u32 %[tok16], %[tok16], %[tsk16]"]
    if mode != "f16":
        out += ["s_add_u32 %[tok8], %[tok8], %[tsk8]",
                # scale block: ++sc == kb_tiles -> sc = 0 and the offset moves to
                # the next block, clamped at the sequence's last one (offsets of
                # one head's blocks are hk2 apart, so the clamp stops exactly there)
                "s_add_u32 %[sc], %[sc], 1", "s_cmp_eq_u32 %[sc], %[kbt]", "s_cselect_b32 %[sc], 0, %[sc]",
                "s_cselect_b32 %[t], %[hk2], 0", "s_add_u32 %[skoff], %[skoff], %[t]",
                "s_min_u32 %[skoff], %[skoff], %[sklast]"]
    return out


def copy_v(par: int) -> list[str]:
    """V(t) for t = n + 1 into V slot 1 - par."""
    o: list[str] = []
    for i in range(V16_INS):
        addr = (f"v_add_u32 v{VO}, %[tov16], %[dv16]" if i == 0 else f"v_add_u32 v{VO}, %[stpv16], v{VO}")
        o += _copy((1 - par) * LAYOUT["stage"] + VOFF + i * NW * 1024, addr, "rsv16")
    return o + ["s_add_u32 %[tov16], %[tov16], %[tsv16]"]


def copy_v_groups(par: int) -> list[list[str]]:
    """copy_v split into its four copies (the offset advance goes with the last)."""
    lines = copy_v(par)
    groups: list[list[str]] = [[]]
    for ln in lines:
        groups[-1].append(ln)
        if ln.startswith("buffer_load"):
            groups.append([])
    tail = groups.pop()
    groups[-1] += tail
    assert len(groups) == V16_INS
    return groups


def copies(mode: str, par: int, lbl: str, with_v: bool = True, v_always: bool = False) -> list[str]:
    """Iteration n's copies: K(n+2) while n + 2 <= %[klim] = min(n_sw,
    n_blocks - 1) (its route -> %[rn2]), V(n+1) while n + 1 < n_blocks
    (v_always: a body with a next tile, where n + 1 < n_sw <= n_blocks)."""
    out = ["s_add_u32 %[t], %[n], 2", "s_cmp_gt_u32 %[t], %[klim]", f"s_cbranch_scc1 {lbl}_nok"]
    out += copy_k(mode, par, f"{lbl}_ck")
    out += [f"{lbl}_nok:"]
    if not with_v:
        return out
    if v_always:
        return out + copy_v(par)
    out += ["s_add_u32 %[t], %[n], 1", "s_cmp_ge_u32 %[t], %[nblk]", f"s_cbranch_scc1 {lbl}_nov"]
    out += copy_v(par)
    return out + [f"{lbl}_nov:"]


def _tile_start(mode: str) -> list[str]:
    """Every iteration: this wave's copies have landed, then every wave's; the
    route of the tile after next starts as the next tile's (no K copy)."""
    out = ["s_waitcnt vmcnt(0)", "s_barrier"]
    return out + (["s_mov_b32 %[rn2], %[rn]"] if routed(mode) else [])


def _tile_end(mode: str) -> list[str]:
    return ["s_mov_b32 %[rn], %[rn2]"] if routed(mode) else []


def iteration(mode: str, par: int, lbl: str) -> list[str]:
    """Iteration n (n & 1 == par; %[n] holds n) of an active wave, n + 1 < n_sw:
    a body with a next tile (FP16 or INT8 by the next tile's route)."""
    mixed_regs = mode != "f16"
    inner = OPTS["copy_at"] is not None or OPTS["early"]
    out = _tile_start(mode)
    vsp = OPTS["v_spread"] and inner
    vg = copy_v_groups(par) if vsp else None
    cps = copies(mode, par, f"{lbl}_c", not vsp, v_always=True)
    if not inner:
        out += cps

    def body(kind: str, tag: str) -> list[str]:
        cp = copies(mode, par, f"{lbl}_{tag}c", not vsp, v_always=True) if inner else None
        return body_iter(kind, 1 - par, par, mixed_regs, 1 - par, f"{lbl}_{tag}", cp, vg)

    if mode == "f16":
        out += body("f16", "f")
    elif mode == "i8":
        out += body("i8", "i")
    else:
        out += to_int8_body(f"{lbl}_i8")
        out += body("f16", "f")
        out += [f"s_branch {lbl}_end", f"{lbl}_i8:"]
        out += body("i8", "i")
        out += [f"{lbl}_end:"]
    return out + _tile_end(mode)


def drain(mode: str, par: int, lbl: str) -> list[str]:
    """The last iteration (n = n_sw - 1) of an active wave: no next tile."""
    out = _tile_start(mode)
    out += body_iter("none", 0, par, mode != "f16", 0, f"{lbl}_d", copies(mode, par, f"{lbl}_dc"))
    return out + _tile_end(mode)


def inactive(mode: str, par: int, lbl: str) -> list[str]:
    """Iteration n of a wave whose rows all lie past the sequence end: only the
    barrier and the copies."""
    return _tile_start(mode) + copies(mode, par, f"{lbl}_xc") + _tile_end(mode)


def fill_copy(mode: str, lbl: str) -> list[str]:
    """The barrier after the prologue (the Q block's use of stage 1 ends, K(0)
    and V(0) have landed) and the copy of K(1): iteration -1 (parity 1) of
    the copy schedule, for every wave.  %[rn] stays tile 0's route (FILL
    computes tile 0) until the caller moves tile 1's into it."""
    out = _tile_start(mode)
    out += ["s_cmp_le_u32 %[nblk], 1", f"s_cbranch_scc1 {lbl}_nok", "s_mov_b32 %[t], 1"]
    out += copy_k(mode, 1, f"{lbl}_ck")
    return out + [f"{lbl}_nok:"]


def fill(mode: str, lbl: str) -> list[str]:
    """Tile 0's QK, conversion and maximum (active waves)."""
    mixed_regs = mode != "f16"
    f16_body = body_fill("f16", 0, mixed_regs, f"{lbl}_bf") if mode != "i8" else []
    i8_body = body_fill("i8", 0, mixed_regs, f"{lbl}_bi") if mode != "f16" else []
    if mode == "f16":
        return f16_body
    if mode == "i8":
        return i8_body
    return to_int8_body(f"{lbl}_i8") + f16_body + [f"s_branch {lbl}_end", f"{lbl}_i8:"] + i8_body + \
        [f"{lbl}_end:"]


def loop_asm(mode: str) -> list[str]:
    with layout(mode):
        return _loop_asm(mode)


def _loop_asm(mode: str) -> list[str]:
    L = ".Lpipe%="
    # M0 carries the LDS address of every copy; the compiler's value of M0
    # is restored at the end (M0 is a reserved register).
    out = ["s_mov_b32 %[m0s], m0",
           "s_sub_u32 %[klim], %[nblk], 1", "s_min_u32 %[klim], %[klim], %[nsw]",
           "s_sub_u32 %[nsw1], %[nsw], 1", "s_mov_b32 %[n], 0"]
    out += fill_copy(mode, f"{L}_fc")
    out += ["s_cmp_eq_u32 %[act], 0", f"s_cbranch_scc1 {L}_xin"]
    out += fill(mode, f"{L}_f") + _tile_end(mode)
    # iterations 0 .. n_sw - 2 have a next tile; n_sw - 1 is the drain
    out += ["s_cmp_eq_u32 %[nsw1], 0", f"s_cbranch_scc1 {L}_d0", f"{L}_loop:"]
    out += iteration(mode, 0, f"{L}_p0")
    out += ["s_add_u32 %[n], %[n], 1", "s_cmp_ge_u32 %[n], %[nsw1]", f"s_cbranch_scc1 {L}_d1"]
    out += iteration(mode, 1, f"{L}_p1")
    out += ["s_add_u32 %[n], %[n], 1", "s_cmp_lt_u32 %[n], %[nsw1]", f"s_cbranch_scc1 {L}_loop", f"{L}_d0:"]
    out += drain(mode, 0, f"{L}_q0")
    out += [f"s_branch {L}_done", f"{L}_d1:"]
    out += drain(mode, 1, f"{L}_q1")
    out += [f"s_branch {L}_done", f"{L}_xin:"] + _tile_end(mode) + [f"{L}_inact:"]
    out += inactive(mode, 0, f"{L}_x0")
    out += ["s_add_u32 %[n], %[n], 1", "s_cmp_ge_u32 %[n], %[nsw]", f"s_cbranch_scc1 {L}_done"]
    out += inactive(mode, 1, f"{L}_x1")
    out += ["s_add_u32 %[n], %[n], 1", "s_cmp_lt_u32 %[n], %[nsw]", f"s_cbranch_scc1 {L}_inact"]
    out += [f"{L}_done:",
            # the C++ code after the statement reads the O accumulators: the
            # last PV MFMAs' results are read 36 wait states after them
            "s_nop 15", "s_nop 15", "s_nop 3", "s_mov_b32 m0, %[m0s]"]
    return out


def function(mode: str) -> str:
    lines = loop_asm(mode)
    outs = ['"+{v[0:15]}"(st.acc[0])', '"+{v[16:31]}"(st.acc[1])', '"+{v[32:47]}"(st.acc[2])',
            '"+{v[48:63]}"(st.acc[3])', '"+{v[64:79]}"(st.s16)',
            '[mn] "+v"(st.mn)', '[al] "+v"(st.al)', '[ng] "+v"(st.ng)', '[li] "+v"(st.li)',
            '[tok16] "+s"(c.tok16)', '[tov16] "+s"(c.tov16)', '[grp] "+s"(c.grp)', '[gc] "+s"(c.gc)',
            '[rn] "+s"(c.rn)', '[n] "=&s"(n)', '[t] "=&s"(t)', '[rn2] "=&s"(rn2)',
            '[m0s] "=&s"(m0s)', '[klim] "=&s"(klim)', '[nsw1] "=&s"(nsw1)']
    ins = ['[nsw] "s"(c.nsw)', '[nblk] "s"(c.nblk)', '[act] "s"(c.act)', '[mt] "s"(c.mt)',
           '[ldsw] "s"(c.ldsw)', '[rsk16] "s"(c.rsk16)', '[rsv16] "s"(c.rsv16)',
           '[stpk16] "s"(c.stpk16)', '[stpv16] "s"(c.stpv16)', '[tsk16] "s"(c.tsk16)', '[tsv16] "s"(c.tsv16)',
           '[dk16] "v"(c.dk16)', '[dv16] "v"(c.dv16)',
           '[fmax] "s"(o.fmax)']
    ins += [f'[va{i}] "v"(o.va[{i}])' for i in range(4)]
    if mode != "i8":
        ins += [f'[ka{i}] "v"(o.ka[{i}])' for i in range(8)]
        ins += [f'[qf{i}] "v"(o.qf[{i}])' for i in range(8)]
    if mode != "f16":
        outs += ['[tok8] "+s"(c.tok8)', '[sc] "+s"(c.sc)', '[skoff] "+s"(c.skoff)',
                 '[sk0] "+v"(c.sk[0])', '[sk1] "+v"(c.sk[1])']
        ins += ['[kbt] "s"(c.kbt)', '[hask] "s"(c.hask)', '[sklast] "s"(c.sklast)', '[hk2] "s"(c.hk2)',
                '[rssk] "s"(c.rssk)', '[rsk8] "s"(c.rsk8)', '[stpk8] "s"(c.stpk8)', '[tsk8] "s"(c.tsk8)',
                '[dk8] "v"(c.dk8)', '[sq16] "v"(c.sq16)', '[qks] "s"(c.qks)', '[magic2] "s"(c.magic2)']
        ins += [f'[k8a{i}] "v"(o.k8a[{i}])' for i in range(4)]
        ins += [f'[q8f{i}] "v"(o.q8f[{i}])' for i in range(4)]
    if mode in ("mixed", "split"):
        ins += ['[bits] "s"(c.bits)']
    if mode == "split":
        ins += ['[bitsh] "s"(c.bits_hi)', '[lolim] "s"(c.lolim)', '[half] "s"(c.half)']
    text = "\n".join(f'      "{ln}\\n"' for ln in lines)
    clob = ", ".join(f'"v{r}"' for r in range(QA, VO + 1))
    return f'''__device__ __forceinline__ void pipe_loop_{mode}(PipeState& st, const PipeOps& o, PipeCopy& c) {{
  int n, t, rn2, m0s, klim, nsw1;
  asm volatile(
{text}
      : {", ".join(outs)}
      : {", ".join(ins)}
      : {clob}, "vcc", "scc", "memory");
}}
'''


HEADER = '''// GENERATED by gen_attn_pipe.py -- do not edit; edit the generator and rebuild.
//
// The software-pipelined tile loop of attn32_kernel (PIPE instantiations):
// gfx950 assembly with a fixed register map.  gen_attn_pipe.py documents the
// schedule, the register map and the hazard rules it follows.
#pragma once

#include "attn_common.h"

namespace tmx {

typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));

// Loop-carried compute state (fixed registers inside the statement).
struct PipeState {
  f32x16 acc[4];  // O^T accumulators, d blocks 0..3
  u32x16 s16;     // packed fp16 scores of the tile whose softmax is next
  float mn;       // running row maximum including that tile
  float al;       // its alpha = exp2(m_before - mn)
  float ng;       // -mn (clamped to FLT_MAX while mn = -inf)
  float li;       // this lane's share of the row sum before that tile
};

// Loop-invariant compute operands.
struct PipeOps {
  f16x8 qf[8];    // fp16 Q fragments (B operands of the fp16 QK MFMAs)
  i32x4 q8f[4];   // int8 Q codes (B operands of the int8 QK MFMAs)
  int ka[8];      // LDS byte addresses of the fp16 K operand reads, k-step 0..7 (stage 0)
  int k8a[4];     // the same for int8 K, k-step 0..3
  int va[4];      // LDS byte addresses of the V^T reads, d block 0..3 (stage 0's V slot;
                  // the 16-bit read offsets then reach stage 1 of a split stage too)
  float fmax;     // FLT_MAX
};

// Copy schedule and bookkeeping: the state of the C++ issue_next_k / issue_v
// (in and out) and the copy constants.
struct PipeCopy {
  int tok16, tok8, tov16;  // byte offset of the next K16 / K8 / V tile copy
  int grp, gc, sc;         // route group, tiles into it, tiles into the scale block (next K)
  int skoff;               // byte offset of the next K tile's scale (scale buffer rssk)
  int rn;                  // route of the next tile to compute
  uint32_t sk[2];          // K scale (fp16 bits) of the tiles of each parity
  int nsw, nblk, act;      // pipelined tiles, tiles, wave has rows
  uint64_t bits;           // route bits of the workgroup's block (split: of its low half)
  uint64_t bits_hi;        // split: route bits of the high half
  int lolim;               // split: tiles from this one on lie past the low half's last key
  int half;                // split: this wave's half (0 low, 1 high)
  int mt, kbt, hask;       // tiles per route group / per scale block, K scales present
  int sklast;              // byte offset of the sequence's last K scale of the head
  i32x4 rssk;              // buffer descriptor over the K scales
  int hk2;                 // bytes between two scale blocks of a head
  i32x4 rsk16, rsk8, rsv16;   // buffer descriptors of the K16 / K8 / V streams
  int stpk16, stpk8, stpv16;  // bytes between a wave's copies of one tile
  int tsk16, tsk8, tsv16;     // bytes per tile
  int ldsw;                   // LDS byte address of stage 0 + 1 KB * wave
  int dk16, dk8, dv16;        // the lane's copy offsets
  uint32_t sq16;              // Q block scale (fp16 bits)
  float qks;                  // qk_scale
  uint64_t magic2;            // 1.5 * 2^23 as int bits, twice
};

'''


def generate() -> str:
    parts = [HEADER]
    for mode in ("f16", "i8", "mixed", "split"):
        parts.append(function(mode))
    parts.append("}  // namespace tmx\n")
    return "\n".join(parts)


OUT = Path(__file__).resolve().parent / "attn_pipe_asm.h"


def write(path: Path = OUT) -> bool:
    """Write the header if its content changed; returns True when written."""
    text = generate()
    if path.exists() and path.read_text() == text:
        return False
    path.write_text(text)
    return True


if __name__ == "__main__":
    write(Path(sys.argv[1]) if len(sys.argv) > 1 else OUT)

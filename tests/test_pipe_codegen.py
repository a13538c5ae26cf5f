"""CPU checks of the generated assembly tile loop (tilemix_amd/csrc/attn_pipe_asm.h).

* The committed header is exactly what gen_attn_pipe.py generates.
* A static checker replays every straight-line compute body of the loop
  (FILL / ITER for fp16 and int8 next tiles, DRAIN, both stage parities) and
  enforces the gfx950 rules the generator relies on, since the compiler does
  not look inside the asm statement:
    - an LDS read has completed (s_waitcnt lgkmcnt accounting, in-order
      return) before any instruction reads its destination;
    - a VALU instruction reads an MFMA result no sooner than 18 wait states
      after the MFMA (accumulation chains, MFMA -> the same MFMA's SrcC, excepted);
    - an MFMA reads a VALU result no sooner than 3 wait states after it;
    - no instruction reads the result of the v_exp_f32 right before it;
    - v_permlane32_swap's operands were written at least 2 wait states earlier;
    - the result of a DOT instruction (v_dot2c) is read or overwritten by any
      other instruction no sooner than 3 wait states after it (the next
      v_dot2c accumulating into it excepted);
    - a copy (buffer_load ... lds) is at least one wait state after the M0
      write it uses.
  Each rule is shown to catch a planted violation.
* Structure: every body reads each K / V operand once per MFMA in the
  reference's k-step order, and the row sum accumulates 16 pairs in order.
"""
from __future__ import annotations

import re
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
CSRC = REPO / "tilemix_amd" / "csrc"
sys.path.insert(0, str(CSRC))
import gen_attn_pipe as G  # noqa: E402

sys.path.pop(0)


def test_committed_header_is_generated():
    assert (CSRC / "attn_pipe_asm.h").read_text() == G.generate()


_REG = re.compile(r"v\[(\d+):(\d+)\]|\bv(\d+)\b")


def _regs(tok: str) -> set[int]:
    out: set[int] = set()
    for m in _REG.finditer(tok):
        if m.group(1) is not None:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
        else:
            out.add(int(m.group(3)))
    return out


def _parse(line: str):
    op, _, rest = line.partition(" ")
    args = [a.strip() for a in rest.split(",")] if rest else []
    return op, args


def _wait_states(op: str, args) -> int:
    if op == "s_nop":
        return int(args[0]) + 1
    return 1


def check_body(lines: list[str]) -> None:
    """Raises AssertionError on the first violated rule."""
    pending: list[set[int]] = []   # outstanding LDS reads, oldest first
    inflight: set[int] = set()      # registers written by outstanding LDS reads
    mfma_w: dict[int, tuple[int, int]] = {}  # reg -> (wait-state clock of the MFMA write, its dst base)
    valu_w: dict[int, int] = {}     # reg -> clock of the last VALU write
    clock = 0
    prev_exp: set[int] = set()
    dot_w: dict[int, int] = {}      # reg -> clock of the last v_dot2c write
    for line in lines:
        if line.endswith(":") or not line:
            continue
        op, args = _parse(line)
        ws = _wait_states(op, args)
        if op == "s_waitcnt":
            m = re.match(r"lgkmcnt\((\d+)\)", args[0])
            if m:
                keep = int(m.group(1))
                while len(pending) > keep:
                    pending.pop(0)
                inflight = set().union(*pending) if pending else set()
            clock += ws
            prev_exp = set()
            continue
        if op.startswith("s_") or op.startswith("buffer_"):
            clock += ws
            prev_exp = set()
            continue
        dst = _regs(args[0]) if args else set()
        srcs = set().union(*(_regs(a) for a in args[1:])) if len(args) > 1 else set()
        if op == "v_dot2c_f32_f16":
            srcs |= dst
        if op == "v_permlane32_swap_b32":
            srcs |= dst
        assert not (srcs & inflight), f"reads an LDS destination before its wait: {line}"
        assert not (srcs & prev_exp), f"reads the exp result of the previous instruction: {line}"
        if op != "v_dot2c_f32_f16":
            for r in (srcs | dst) & set(dot_w):
                assert clock - dot_w[r] >= 4, f"uses a DOT result within 3 wait states: {line}"
        if op.startswith("v_mfma"):
            c_regs = _regs(args[3]) if len(args) > 3 else set()
            for r in srcs:
                if r in valu_w:
                    assert clock - valu_w[r] >= 3, f"MFMA reads a VALU result too early: {line}"
                if r in mfma_w and not (r in c_regs and r in dst):
                    assert clock - mfma_w[r][0] >= 18, f"MFMA reads another MFMA's result too early: {line}"
            for r in dst:
                mfma_w[r] = (clock, min(dst))
                valu_w.pop(r, None)
        elif op.startswith("ds_read"):
            assert not (dst & inflight), f"LDS destination reused before its wait: {line}"
            pending.append(dst)
            inflight |= dst
        else:  # VALU
            for r in srcs:
                if r in mfma_w:
                    assert clock - mfma_w[r][0] >= 18, f"VALU reads an MFMA result too early: {line}"
                if op == "v_permlane32_swap_b32" and r in valu_w:
                    assert clock - valu_w[r] >= 2, f"permlane operand written too late: {line}"
            for r in dst:
                valu_w[r] = clock
                mfma_w.pop(r, None)
        prev_exp = dst if op == "v_exp_f32" else set()
        for r in dst:
            if op == "v_dot2c_f32_f16":
                dot_w[r] = clock
            else:
                dot_w.pop(r, None)
        clock += ws


def check_m0(lines: list[str]) -> None:
    last_m0 = None
    clock = 0
    for line in lines:
        if line.endswith(":"):
            continue
        op, args = _parse(line)
        if op.startswith("s_") and args and args[0] == "m0":
            last_m0 = clock
        if op.startswith("buffer_load") and line.endswith("lds"):
            assert last_m0 is not None and clock - last_m0 >= 2, f"copy right after its M0 write: {line}"
        clock += _wait_states(op, args)


def _bodies():
    out = {}
    for mixed_regs in (False, True):
        for kind in ("f16", "i8"):
            if kind == "i8" and not mixed_regs:
                continue
            for par in (0, 1):
                out[f"iter_{kind}_p{par}_{mixed_regs}"] = G.body_iter(kind, 1 - par, par, mixed_regs, 1 - par)
            out[f"fill_{kind}_{mixed_regs}"] = G.body_fill(kind, 0, mixed_regs)
        for par in (0, 1):
            out[f"drain_p{par}_{mixed_regs}"] = G.body_iter("none", 0, par, mixed_regs, 0)
    return out


BODIES = _bodies()


@pytest.mark.parametrize("name", sorted(BODIES))
def test_body_hazards(name):
    check_body(BODIES[name])


@pytest.mark.parametrize("mode", ["f16", "i8", "mixed", "split"])
def test_loop_m0_rule(mode):
    check_m0(G.loop_asm(mode))


@pytest.mark.parametrize("mode", ["f16", "i8", "mixed", "split"])
def test_lds_offsets_fit_and_stay_in_the_stages(mode):
    """Every LDS read offset fits the 16-bit field; every copy destination
    (M0 offset + this wave's 1 KB) lies inside the two stages, in the slot of
    its stream."""
    stage = G.SPLIT_STAGE if mode == "split" else G.STAGE
    k8off = G.SPLIT_K8OFF if mode == "split" else 0
    loop = G.loop_asm(mode)
    for ln in loop:
        m = re.search(r"offset:(\d+)$", ln)
        if ln.startswith("ds_read") and m:
            assert int(m.group(1)) < 1 << 16, ln
    dest = None
    for ln in loop:
        m = re.match(r"s_add_u32 m0, %\[ldsw\], (\d+)$", ln)
        if m:
            dest = int(m.group(1))
        elif ln.startswith("buffer_load_dwordx4") and ln.endswith("lds"):
            stream = re.search(r"%\[(rs\w+)\]", ln).group(1)
            par, off = divmod(dest, stage)
            assert par in (0, 1) and off + G.NW * 1024 <= stage, ln
            lo, size = {"rsk16": (0, 64 * G.ROW16), "rsk8": (k8off, 64 * G.ROW8),
                        "rsv16": (G.VOFF, 64 * G.ROW16)}[stream]
            assert lo <= off and off + G.NW * 1024 <= lo + size, (ln, dest)


def _salu_route(lines, regs):
    """Runs the SALU route computation of a K copy (the lines up to the route
    group advance) and returns %[rn2]."""
    scc, i = 0, 0
    labels = {ln[:-1]: j for j, ln in enumerate(lines) if ln.endswith(":")}
    val = lambda a: regs[a[2:-1]] if a.startswith("%[") else int(a)
    while i < len(lines):
        ln = lines[i]
        i += 1
        if ln.endswith(":"):
            continue
        op, args = _parse(ln)
        if op == "s_add_u32" and args[0] == "%[gc]":
            break
        if op in ("s_bitcmp1_b64", "s_bitcmp1_b32"):
            scc = (val(args[0]) >> val(args[1])) & 1
        elif op == "s_cselect_b32":
            regs[args[0][2:-1]] = val(args[1]) if scc else val(args[2])
        elif op == "s_cmp_ge_u32":
            scc = int(val(args[0]) >= val(args[1]))
        elif op == "s_cbranch_scc1":
            if scc:
                i = labels[args[0]]
        elif op == "s_and_b32":
            regs[args[0][2:-1]] = val(args[1]) & val(args[2])
        elif op == "s_or_b32":
            regs[args[0][2:-1]] = val(args[1]) | val(args[2])
        elif op == "s_mov_b32":
            regs[args[0][2:-1]] = val(args[1])
        else:
            raise AssertionError(f"unexpected instruction in the route block: {ln}")
    return regs["rn2"]


def test_split_route_matches_the_kernels_tile_route():
    """The split loop's route of a copied tile, run instruction by
    instruction, equals attn_kernel32.h's tile_route for SPLIT: bit 1 the high
    half's bit of the route group, bit 0 the low half's unless the tile starts
    past the low half's last key (t * 64 > lo_last_key, i.e. t >= lolim)."""
    import random
    with G.layout("split"):
        lines = G.copy_k("split", 0, ".Lt")

    def mismatches(route_lines, lolim_of=lambda lk: 0 if lk < 0 else lk // 64 + 1):
        rnd = random.Random(7)
        bad = 0
        for _ in range(3000):
            bits, bitsh = rnd.getrandbits(64), rnd.getrandbits(64)
            t, grp = rnd.randrange(64), rnd.randrange(64)
            lo_last_key = rnd.randrange(-200, 64 * 64)
            rhi = (bitsh >> grp) & 1
            rlo = rhi if t * 64 > lo_last_key else (bits >> grp) & 1
            regs = {"bits": bits, "bitsh": bitsh, "grp": grp, "t": t, "lolim": lolim_of(lo_last_key)}
            bad += _salu_route(route_lines, regs) != rlo | (rhi << 1)
        return bad

    assert mismatches(lines) == 0
    # planted mistakes: the halves' words swapped, the limit off by one tile
    swapped = [ln.replace("%[bitsh]", "%[X]").replace("%[bits]", "%[bitsh]").replace("%[X]", "%[bits]")
               for ln in lines]
    assert mismatches(swapped) > 0
    assert mismatches(lines, lambda lk: 0 if lk < 0 else lk // 64) > 0


def _guard_tests(loop, tag):
    """The test instruction of every refill guard (the line before its first
    branch; a second guard reuses the first one's SCC)."""
    return [loop[i - 1] for i, ln in enumerate(loop) if ln.startswith("s_cbranch_scc1") and ln.endswith(tag)]


def test_split_loop_formats_and_wave_bits():
    """split: fp16 K is copied unless both halves are INT8 and int8 K unless
    both are FP16; each compute branch and refill guard tests this wave's bit
    of the two-bit route, never the whole route."""
    loop, mixed = G.loop_asm("split"), G.loop_asm("mixed")
    assert "s_cmp_eq_u32 %[rn], 0" not in "\n".join(loop)
    assert sum(ln == "s_bitcmp1_b32 %[rn], %[half]" for ln in loop) == \
        sum(ln == "s_cmp_eq_u32 %[rn], 0" for ln in mixed) > 0
    assert set(_guard_tests(loop, "_rfa")) == {"s_bitcmp0_b32 %[rn2], %[half]"}
    assert set(_guard_tests(mixed, "_rfa")) == {"s_cmp_eq_u32 %[rn2], 0"}
    assert len(_guard_tests(loop, "_rfa")) == len(_guard_tests(mixed, "_rfa")) > 0
    # int8 routing: every tile after next is an INT8 tile, the refill is unconditional
    assert not _guard_tests(G.loop_asm("i8"), "_rfa")
    with G.layout("split"):
        ck = G.copy_k("split", 1, ".Lt")
    i16 = ck.index("s_cmp_eq_u32 %[rn2], 3")
    i8 = ck.index("s_cmp_eq_u32 %[rn2], 0")
    assert i16 < i8
    assert all("rsk16" not in ln for ln in ck[i8:]) and any("rsk8" in ln for ln in ck[i8:])
    assert any("buffer_load_ushort" in ln for ln in ck[i8:])
    # the generated header carries the split loop and restores the default layout
    assert "pipe_loop_split" in G.generate() and G.LAYOUT["stage"] == G.STAGE


def _planted(lines, pred, repl):
    out = list(lines)
    for i, ln in enumerate(out):
        if pred(ln):
            out[i:i + 1] = repl(ln)
            return out
    raise AssertionError("no line to plant in")


@pytest.mark.parametrize("plant", ["drop_lds_wait", "early_conversion", "rescale_late", "exp_then_use",
                                   "permlane_no_nop", "m0_no_nop", "dot_then_use"])
def test_checker_catches_planted_violations(plant):
    body = BODIES["iter_f16_p0_True"]
    if plant == "drop_lds_wait":
        bad = _planted(body, lambda ln: ln.startswith("s_waitcnt lgkmcnt("), lambda ln: [])
    elif plant == "early_conversion":
        # read the first QK accumulator pair right after the last QK MFMA
        idx = max(i for i, ln in enumerate(body) if ln.startswith("v_mfma_f32_32x32x16_f16 v[96:111]"))
        bad = body[:idx + 1] + [f"v_cvt_pk_f16_f32 v{G.T}, v96, v97"] + body[idx + 1:]
    elif plant == "rescale_late":
        idx = next(i for i, ln in enumerate(body) if ln.startswith("v_mfma_f32_32x32x16_f16 v[16:31]"))
        bad = body[:idx] + [f"v_mul_f32 v16, %[al], v16"] + body[idx:]
    elif plant == "exp_then_use":
        idx = next(i for i, ln in enumerate(body) if ln.startswith("v_exp_f32 v"))
        r = _parse(body[idx])[1][0]
        bad = body[:idx + 1] + [f"v_mov_b32 v{G.T + 5}, {r}"] + body[idx + 1:]
    elif plant == "dot_then_use":
        # the l update right behind the last row-sum step
        idx = max(i for i, ln in enumerate(body) if ln.startswith("v_dot2c_f32_f16"))
        bad = body[:idx + 1] + [f"v_add_f32 %[li], %[li], v{G.LS}"] + body[idx + 1:]
    elif plant == "permlane_no_nop":
        bad = _planted(body, lambda ln: ln == "s_nop 1", lambda ln: [])
    else:
        # the copy's address add moved before its M0 write: the copy follows M0 at once
        loop = G.loop_asm("mixed")
        i = next(i for i, ln in enumerate(loop) if ln.startswith("s_add_u32 m0"))
        assert loop[i + 1].startswith("v_add_u32") and loop[i + 2].startswith("buffer_load")
        bad = loop[:i] + [loop[i + 1], loop[i]] + loop[i + 2:]
        with pytest.raises(AssertionError):
            check_m0(bad)
        return
    with pytest.raises(AssertionError):
        check_body(bad)


_LEGACY = {"early": False, "v_ahead": False, "tail_first": False, "skip_refill": False, "wait_pairs": False}
OPTION_SETS = [{}, _LEGACY, {**_LEGACY, "copy_at": 1}, {**_LEGACY, "skip_rescale": True},
               {**_LEGACY, "qk_il": True}, {**_LEGACY, "pv_il": True}, {**_LEGACY, "early": True},
               {**_LEGACY, "v_ahead": True}, {**_LEGACY, "tail_first": True}, {"skip_rescale": True},
               {"qk_il": True, "pv_il": True}, {"auto_wait": True}, {"v_spread": True},
               {"copy_at": 3, "skip_refill": True, "skip_rescale": True, "qk_il": True, "pv_il": True,
                "early": False}]


@pytest.fixture
def opts():
    saved = dict(G.OPTS)
    yield G.OPTS
    G.OPTS.clear()
    G.OPTS.update(saved)


@pytest.mark.parametrize("option_set", OPTION_SETS, ids=lambda o: "-".join(sorted(o)) or "default")
def test_every_schedule_option_keeps_the_work(opts, option_set):
    """Under every schedule option each body still passes the hazard rules,
    rescales every O register exactly once (ITER / DRAIN), writes every score
    register exactly once (FILL / ITER), packs every p register once and
    accumulates the 16 pairs of the row sum."""
    opts.update(option_set)
    for name, body in _bodies().items():
        check_body(body)
        muls = [ln for ln in body if ln.startswith("v_mul_f32 v") and "%[al]" in ln]
        targets = sorted(int(ln.split()[1].rstrip(",")[1:]) for ln in muls)
        conv = [ln for ln in body if ln.startswith("v_cvt_pk_f16_f32 v") and
                G.S16 <= int(ln.split()[1].rstrip(",")[1:]) < G.S16 + 16]
        packs = [ln for ln in body if ln.startswith("v_cvt_pk_f16_f32 v") and
                 G.P <= int(ln.split()[1].rstrip(",")[1:]) < G.P + 16]
        dots = [ln for ln in body if ln.startswith("v_dot2c_f32_f16")]
        if name.startswith("fill"):
            assert not muls and not packs and not dots, name
            assert sorted(int(ln.split()[1].rstrip(",")[1:]) for ln in conv) == list(range(G.S16, G.S16 + 16))
        else:
            assert targets == list(range(64)), (name, len(targets))
            assert sorted(int(ln.split()[1].rstrip(",")[1:]) for ln in packs) == list(range(G.P, G.P + 16))
            assert len(dots) == 16
            if not name.startswith("drain"):
                assert sorted(int(ln.split()[1].rstrip(",")[1:]) for ln in conv) == \
                    list(range(G.S16, G.S16 + 16)), name
    for mode in ("f16", "i8", "mixed", "split"):
        loop = G.loop_asm(mode)
        check_m0(loop)
        # every wave's share of a V tile is copied on each path of an iteration
        if opts.get("v_spread"):
            assert sum(ln.startswith("buffer_load_dwordx4 v153, %[rsv16]") for ln in loop) >= 4 * G.V16_INS


def test_auto_wait_reproduces_the_hand_counted_waits(opts):
    """With every read in its original place, the recomputed LDS waits equal
    the counts the phase code writes by hand."""
    opts.update(_LEGACY)
    hand = G.generate()
    opts["auto_wait"] = True
    assert G.generate() == hand


def test_bodies_read_operands_in_kstep_order():
    body = BODIES["iter_f16_p0_True"]
    qk = [ln for ln in body if ln.startswith("v_mfma_f32_32x32x16_f16 v[80:95]") or
          ln.startswith("v_mfma_f32_32x32x16_f16 v[96:111]")]
    assert [int(re.search(r"%\[qf(\d)\]", ln).group(1)) for ln in qk] == list(range(8)) * 2
    assert qk[0].endswith(", 0") and qk[8].endswith(", 0")
    pv = [ln for ln in body if re.match(r"v_mfma_f32_32x32x16_f16 v\[(0|16|32|48):", ln)]
    assert len(pv) == 16
    for db in range(4):
        chain = [ln for ln in pv if ln.startswith(f"v_mfma_f32_32x32x16_f16 v[{16 * db}:")]
        assert [re.search(r"v\[(\d+):\d+\], v\[\d+:\d+\]$", ln).group(1) for ln in chain] == \
            [str(G.P + 4 * ks) for ks in range(4)]
    dots = [ln for ln in body if ln.startswith("v_dot2c_f32_f16")]
    assert [int(ln.split("v")[-1]) - G.P for ln in dots] == list(range(16))
    i8 = [ln for ln in BODIES["iter_i8_p0_True"] if ln.startswith("v_mfma_i32_32x32x32_i8")]
    assert [int(re.search(r"%\[q8f(\d)\]", ln).group(1)) for ln in i8] == list(range(4)) * 2


@pytest.mark.parametrize("mode", ["mixed", "split"])
def test_fill_computes_tile0_with_its_own_route(mode):
    """%[rn] holds tile 0's route until FILL has chosen tile 0's body: the K(1)
    copy before FILL leaves tile 1's route in %[rn2], and %[rn] takes it only
    after FILL (else tile 0 would be computed with tile 1's route)."""
    loop = G.loop_asm(mode)
    test = "s_cmp_eq_u32 %[rn], 0" if mode == "mixed" else "s_bitcmp1_b32 %[rn], %[half]"
    first_test = loop.index(test)
    first_write = next(i for i, ln in enumerate(loop) if ln.startswith("s_mov_b32 %[rn],"))
    assert first_test < first_write
    assert any(ln.startswith("s_cselect_b32 %[rn2]") for ln in loop[:first_test])


def _walk(lines, take):
    """Instruction classes executed along one path through straight-line code
    with forward branches (take(label) decides each conditional branch)."""
    labels = {ln[:-1]: i for i, ln in enumerate(lines) if ln.endswith(":")}
    counts = {}
    i = 0
    while i < len(lines):
        ln = lines[i]
        i += 1
        if ln.endswith(":"):
            continue
        op = ln.split()[0]
        if op.startswith("s_cbranch") or op == "s_branch":
            counts["branch"] = counts.get("branch", 0) + 1
            tgt = ln.split()[1]
            if op == "s_branch" or take(tgt):
                i = labels[tgt]
            continue
        k = ("mfma" if op.startswith("v_mfma") else "lds" if op.startswith("ds_") else
             "vmem" if op.startswith("buffer_") else "wait" if op == "s_waitcnt" else
             "nop" if op == "s_nop" else "salu" if op.startswith("s_") else "valu")
        counts[k] = counts.get(k, 0) + 1
    return counts


def test_iteration_instruction_budget():
    """The mixed loop's iteration on an FP16 tile (K of an FP16 tile copied,
    refill skipped) keeps its lean shape: one LDS wait per two MFMAs, no
    s_nop per copy, the drain / row-less checks outside the iteration.  Every
    such instruction costs a wave an issue slot."""
    with G.layout("mixed"):
        lines = G.iteration("mixed", 0, ".L0")

    def take(t):
        return t.endswith("_rfa") or t.endswith("_rfb") or t.endswith("_end")

    c = _walk(lines, take)
    assert c["mfma"] == 32 and c["lds"] == 48 and c["vmem"] == 8
    assert c["wait"] <= 18 and c.get("nop", 0) <= 2
    assert c["salu"] + c["branch"] <= 38, c

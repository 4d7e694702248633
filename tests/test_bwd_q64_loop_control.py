"""Control flow of the generated sweep of the first backward's dQ kernel
(flash-hog_amd/csrc/gen_bwd_q64_loop.py).

The sweep is inline assembly, so nothing but this test looks at its scalar
side before it runs. The test executes the scalar instructions and branches
of every generated variant, for both kinds of wave (a key-side tensor,
nothing streamed), over ranges of key tiles, masked steps and ragged key
tails, treating vector, LDS and matrix instructions as no-ops, and checks:
  - the sweep ends after exactly one LDS DMA sequence per tile the kernel's
    own prologue did not issue, in order: four 16-byte loads from the tile's
    pointer (waves 0-1) or none (waves 2-3), the pointer advancing one key
    tile per DMA from the kernel's own cursor, into ring stage (tile mod 8),
    with the ragged offsets exactly for the ragged last key tile;
  - at each DMA the stage it overwrites (tile - 8) was last read in a step
    every wave has finished, and every step's tile has been waited for;
  - step t takes the masked element-wise step iff t >= nfull, and then with
    the key offset of its own tile;
  - on executed traces: no matrix instruction reads an LDS fragment, and no
    vector instruction an LDS result, before the s_waitcnt that retires it;
    distances between matrix results and vector reads (12), vector results
    and matrix reads (2), transcendental results and vector reads (2); a
    score tile is read only once its chain of four products is complete, and
    no vector instruction writes a register a chain still accumulates into;
  - the committed fhog_bwd_q64_loop.inc is the generator's output.
CPU only.
"""

from __future__ import annotations

import importlib.util
import pathlib
import re
import sys

import pytest

CSRC = pathlib.Path(__file__).resolve().parent.parent / "flash-hog_amd" / "csrc"
sys.path.insert(0, str(CSRC))


def _gen():
    spec = importlib.util.spec_from_file_location("gen_bwd_q64_loop", CSRC / "gen_bwd_q64_loop.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


G = _gen()
M32, M64 = (1 << 32) - 1, (1 << 64) - 1


def _val(tok, s):
    m = re.fullmatch(r"s(\d+)", tok)
    if m:
        return s[int(m.group(1))]
    if tok == "m0":
        return s["m0"]
    return int(tok, 0)


def _pair(tok, s):
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        lo = int(m.group(1))
        return s[lo] | (s[lo + 1] << 32)
    return int(tok, 0) & M64


def run(prog, ops, max_steps=400000, trace=None):
    """Executes the scalar side of prog, with the kernel's bound registers
    (gen_bwd_q64_loop.BOUND) preset from ops[name + '_init']. Returns events:
    ('dma', kind, ptr, m0, voff operand), ('barrier',), ('wait', n),
    ('label', name, state)."""
    labels = {ins[:-1]: i for i, ins in enumerate(prog) if ins.endswith(":")}
    s = {"m0": 0}
    for i in range(106):
        s[i] = 0
    for n in G.BOUND:
        val, r = ops[f"{n}_init"], G.SG[n]
        s[r] = val & M32
        if n.startswith("p"):
            s[r + 1] = val >> 32
    scc = 0
    events = []
    pc = 0
    steps = 0
    sub = lambda t: re.sub(r"%\[(\w+)\]", lambda m: str(ops[m.group(1)]), t)
    while pc < len(prog):
        steps += 1
        assert steps < max_steps, "the sweep does not end"
        ins = prog[pc]
        pc += 1
        if ins.endswith(":"):
            events.append(("label", ins[:-1], dict(s)))
            continue
        if trace is not None:
            trace.append(ins)
        op, *args = ins.replace(",", " ").split()
        if op.startswith("global_load_lds"):
            events.append(("dma", op, _pair(args[1], s), s["m0"], args[0]))
            continue
        if not op.startswith("s_"):
            continue
        a = [sub(x) for x in args]
        dst = lambda d: int(d[1:]) if d != "m0" else "m0"
        if op == "s_mov_b32":
            s[dst(a[0])] = _val(a[1], s) & M32
        elif op == "s_mov_b64":
            lo = int(re.fullmatch(r"s\[(\d+):\d+\]", a[0]).group(1))
            val = _pair(a[1], s)
            s[lo], s[lo + 1] = val & M32, val >> 32
        elif op in ("s_add_u32", "s_sub_u32", "s_and_b32", "s_lshl_b32", "s_addc_u32"):
            x, y = _val(a[1], s) & M32, _val(a[2], s) & M32
            if op == "s_add_u32":
                r = x + y
                scc = int(r > M32)
            elif op == "s_addc_u32":
                r = x + y + scc
                scc = int(r > M32)
            elif op == "s_sub_u32":
                r = x - y
                scc = int(r < 0)
            elif op == "s_and_b32":
                r = x & y
                scc = int((r & M32) != 0)
            else:
                r = x << y
                scc = int((r & M32) != 0)
            s[dst(a[0])] = r & M32
        elif op == "s_cselect_b32":
            s[dst(a[0])] = (_val(a[1], s) if scc else _val(a[2], s)) & M32
        elif op == "s_cselect_b64":
            lo = int(re.fullmatch(r"s\[(\d+):\d+\]", a[0]).group(1))
            val = _pair(a[1], s) if scc else _pair(a[2], s)
            s[lo], s[lo + 1] = val & M32, val >> 32
        elif op.startswith("s_cmp_"):
            x, y = _val(a[0], s) & M32, _val(a[1], s) & M32
            kind = op.split("_")[2]
            scc = int({"eq": x == y, "lt": x < y, "ge": x >= y, "gt": x > y, "lg": x != y}[kind])
        elif op == "s_cbranch_scc1":
            if scc:
                pc = labels[a[0]]
        elif op == "s_cbranch_scc0":
            if not scc:
                pc = labels[a[0]]
        elif op == "s_branch":
            pc = labels[a[0]]
        elif op == "s_barrier":
            events.append(("barrier",))
        elif op == "s_waitcnt":
            m = re.search(r"vmcnt\((\d+)\)", ins)
            if m:
                events.append(("wait", int(m.group(1))))
        elif op == "s_nop":
            pass
        else:
            raise AssertionError(f"unmodelled scalar instruction {ins}")
    return events


def program(dtype):
    return [ins.replace("%=", "0") for ins in G.BQ64(dtype).generate()]


LDSK, STAGE, GSTEP = 0x4000, 8192, 32 * 2048
KINDS = {"tiles": 4096, "none": G.WAVE_NONE}


def _case(kind, ntot, nfull, ragged):
    """Operands as the kernel computes them for a synthetic block of ntot key
    tiles (ragged: the last one is the sequence's ragged key tile)."""
    hi = min(4, ntot - 1)          # the kernel's prologue: tiles 0 .. min(4, ntot - 1)
    base = 1 << 40
    ops = dict(ntot=ntot, nfull=nfull, nsd=ntot - (1 if ragged else 0),
               ragk0=(ntot - 1) * 32 if ragged else M32, ldsk=LDSK, ldsw=KINDS[kind],
               gstep_lo=GSTEP & M32, gstep_hi=GSTEP >> 32, hi_init=hi, dgi_init=0,
               dq0_init=32 * (hi + 1), eq0_init=0, p0_init=base + GSTEP * (hi + 1))
    return ops, base


CASES = [(nt, nf, rag)
         for nt in (1, 2, 3, 5, 6, 7, 8, 9, 12, 17)
         for rag in (False, True)
         for nf in sorted({0, nt - 4 if nt > 4 else 0, nt - 1 if rag else nt, nt - (1 if rag else 0)})
         if nf >= 0]


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("kind", sorted(KINDS))
def test_sweep_control_flow(dtype, kind):
    prog = program(dtype)
    for ntot, nfull, ragged in CASES:
        ops, base = _case(kind, ntot, nfull, ragged)
        ev = run(prog, ops)
        where = (ntot, nfull, ragged)
        dmas = [e for e in ev if e[0] == "dma"]
        tiles = list(range(ops["hi_init"] + 1, ntot)) if kind == "tiles" else []
        assert len(dmas) == 4 * len(tiles), where
        for i, kt in enumerate(tiles):
            rag_tile = ragged and kt == ntot - 1
            for j in range(4):
                _, op, ptr_j, m0, which = dmas[4 * i + j]
                assert op == "global_load_lds_dwordx4", where
                assert ptr_j == base + GSTEP * kt, (where, kt, j)
                assert m0 == LDSK + (kt % 8) * STAGE + 4096 + 1024 * j, (where, kt, j)
                assert which == f"%[{'vp' if rag_tile else 'vo'}{j}]", (where, kt, which)
        # barriers: the prologue waits for tile 0, steps 0 .. ntot - 2 for tiles 1 .. ntot - 1
        bars = 0
        hi = ops["hi_init"]
        waited = -1
        waited_now = -1
        for e in ev:
            if e[0] == "wait":
                waited_now = hi - e[1] // 4
            elif e[0] == "barrier":
                waited = waited_now
                assert kind == "none" or waited >= bars, (where, bars, waited)
                bars += 1
            elif e[0] == "dma" and e[4].endswith("0]"):
                hi += 1
                # the stage of tile hi was last read by step hi - 7 at the latest
                # (step t reads tiles t - 1 .. t + 1), which every wave finished
                # before the barrier of the step that waited for tile waited
                assert hi - 8 <= waited - 3, (where, hi, waited)
        assert bars == ntot, (where, bars)
        # masked element-wise steps and their key offsets
        steps = []
        for e in ev:
            if e[0] == "label":
                m = re.fullmatch(r"Lbq64_(first|mid|last|single)(_m|_s)?_0", e[1])
                if m and m.group(2) == "_m":
                    steps.append(e[2])
        want = [t for t in range(ntot) if t >= nfull]
        assert len(steps) == len(want), (where, len(steps), want)
        for state, t in zip(steps, want):
            assert state[G.SG["eq0"]] == 32 * t, (where, t, state[G.SG["eq0"]])


def test_committed_inc_is_current():
    assert G.render() == (CSRC / "fhog_bwd_q64_loop.inc").read_text(), \
        "fhog_bwd_q64_loop.inc is out of date: run flash-hog_amd/csrc/gen_bwd_q64_loop.py"


def _regs(tok):
    m = re.fullmatch(r"-?([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.fullmatch(r"-?([va])(\d+)", tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _ws(ins):
    op = ins.split()[0]
    return int(ins.split()[1]) + 1 if op == "s_nop" else 1


CHAIN = 4


# bf16 operands of the output products (dS): each value written is read by
# exactly two matrix instructions (column blocks dt = 0, 1) before the next
# write, so no conversion overwrites a tile's values before its output
# products have taken them
OUT_OPERANDS = {("v", r) for r in [G.EDS[h] + i for h in range(2) for i in range(8)]}


def check_hazards(trace):
    last_mfma_write, last_valu_write, last_trans_write = {}, {}, {}
    chain = {}  # register -> matrix products in its current chain
    reads = {}  # output operand register -> matrix reads of its current value
    lds_pending = []
    clock = 0
    for ins in trace:
        op, *args = ins.replace(",", " ").split()
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", ins)
            if m:
                n = int(m.group(1))
                while len(lds_pending) > n:
                    lds_pending.pop(0)
        elif op.startswith("ds_read"):
            lds_pending.append(_regs(args[0]))
        elif op.startswith("v_mfma"):
            dst, a, b, c = args[:4]
            srcs = _regs(a) | _regs(b) | _regs(c)
            for regs in lds_pending:
                assert not (regs & srcs), f"matrix operand read before its LDS read completed: {ins}"
            for r in srcs:
                if r in last_valu_write:
                    assert clock - last_valu_write[r] >= 2, f"vector result read by {ins} too early"
            # an accumulator input that is the destination continues a chain:
            # nothing but the chain's previous matrix instruction has written
            # it since (a chain may start from a tuple a vector instruction
            # wrote, the -D start of dP)
            for r in (_regs(c) if _regs(c) == _regs(dst) else set()):
                if r in last_valu_write:
                    assert last_valu_write[r] < last_mfma_write.get(r, -1), f"accumulator overwritten before {ins}"
            for r in (_regs(a) | _regs(b)) & OUT_OPERANDS:
                reads[r] = reads.get(r, 0) + 1
                assert reads[r] <= 2, f"{ins} reads an output operand a third time"
            for r in _regs(dst):
                last_mfma_write[r] = clock
                chain[r] = chain.get(r, 0) + 1 if _regs(c) == _regs(dst) else 1
        elif op.startswith("v_"):
            dst = args[0]
            srcs = set()
            for x in args[1:]:
                srcs |= _regs(x)
            for r in srcs | _regs(dst):
                if r in last_mfma_write:
                    assert clock - last_mfma_write[r] >= 12, f"matrix result used by {ins} after {clock - last_mfma_write[r]}"
                # a score tile is read whole: its chain of four 16-deep
                # products is complete
                assert chain.get(r, CHAIN) == CHAIN, f"{ins} reads a score chain of {chain.get(r)} products"
            for r in srcs:
                if r in last_trans_write:
                    assert clock - last_trans_write[r] >= 2, f"transcendental result read by {ins} too early"
            for regs in lds_pending:
                assert not (regs & (srcs | _regs(dst))), f"vector instruction touches a pending LDS read: {ins}"
            for r in _regs(dst) & OUT_OPERANDS:
                assert reads.get(r, 2) == 2, f"{ins} overwrites an output operand read {reads.get(r)} times"
                reads[r] = 0
            for r in _regs(dst):
                last_valu_write[r] = clock
                if op == "v_exp_f32":
                    last_trans_write[r] = clock
                else:
                    last_trans_write.pop(r, None)
        clock += _ws(ins)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_sweep_hazards(dtype):
    prog = program(dtype)
    for ntot, nfull, ragged in [(1, 1, False), (1, 0, False), (2, 2, False), (2, 0, False), (3, 1, False),
                                (7, 3, True), (12, 12, False), (12, 8, True), (20, 12, False), (16, 0, False)]:
        ops = _case("tiles", ntot, nfull, ragged)[0]
        trace = []
        run(prog, ops, trace=trace)
        check_hazards(trace)

"""Control flow of the generated sweep of the first backward's dK/dV kernel
(flash-hog_amd/csrc/gen_bwd_k64_loop.py).

The sweep is inline assembly, so nothing but this test looks at its scalar
side before it runs. The test executes the scalar instructions and branches
of every generated variant, for the three kinds of wave (a query-side tensor,
the row statistics, nothing streamed), over small combinations of steps,
grouped heads, masked steps and ragged tails, treating vector, LDS and matrix
instructions as no-ops, and checks:
  - the sweep ends after exactly one LDS DMA sequence per tile the kernel's
    own prologue did not issue, in order: four 16-byte loads from the tile's
    pointer (waves 0-1), four 4-byte loads from the four statistics pointers
    (wave 2) or none (wave 3), with the (query tile, head) cursor of the
    kernel's own prologue (tests the pointer steps of the grouped-head
    order), into ring stage (tile mod 8), with the ragged offsets exactly for
    tiles of the ragged query tile;
  - at each DMA the stage it overwrites (tile - 8) was last read in a step
    every wave has finished, and every step's tile has been waited for;
  - step t takes the masked element-wise step iff t < mlo or t >= mhi, and
    then with the query offset of its own tile;
  - on executed traces: no matrix instruction reads an LDS fragment, and no
    vector instruction an LDS result, before the s_waitcnt that retires it;
    distances between matrix results and vector reads (12), vector results
    and matrix reads (2), transcendental results and vector reads (2); no
    vector instruction writes a register a matrix instruction of the same
    step still reads as its accumulator;
  - the committed fhog_bwd_k64_loop.inc is the generator's output.
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
    spec = importlib.util.spec_from_file_location("gen_bwd_k64_loop", CSRC / "gen_bwd_k64_loop.py")
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
    (gen_bwd_k64_loop.BOUND) preset from ops[name + '_init']. Returns events:
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
    return [ins.replace("%=", "0") for ins in G.BK64(dtype).generate()]


LDSQ, NQ_ROW = 0x4000, 1 << 20


KINDS = {"tiles": 4096, "stats": G.ST_OFF, "none": G.WAVE_NONE}
STAGE = 16384


def _case(kind, ntot, grp, mlo, mhi, ragged):
    """Operands as the kernel computes them for a synthetic problem with
    qt_begin = 3 and query tiles of 32 rows (ragged: the last query tile)."""
    w3 = kind == "stats"
    nqt = 3 + ntot // grp
    nq = 32 * nqt - (5 if ragged else 0)
    stepa = 4 * nq if w3 else 128
    stepb = (4 * (32 - (grp - 1) * nq) if w3 else (32 * NQ_ROW - (grp - 1) * 64) * 2) & M64
    base = [(1 << 40) + (j << 34) for j in range(4)] if w3 else [1 << 40] * 4
    # the kernel's prologue: tiles 0 .. min(4, ntot - 1)
    hi = min(4, ntot - 1)
    ptr, dgi, dq0 = list(base), 0, 3 * 32
    for _ in range(hi + 1):
        dgi += 1
        wrap = dgi == grp
        if wrap:
            dgi, dq0 = 0, dq0 + 32
        ptr = [(x + (stepb if wrap else stepa)) & M64 for x in ptr]
    ops = dict(ntot=ntot, grp=grp, mlo=mlo, mhi=mhi, nsd=ntot - (grp if ragged else 0),
               ragq0=(nqt - 1) * 32 if ragged else M32, ldsq=LDSQ, ldsw=KINDS[kind],
               stepa=stepa, stepb=stepb, hi_init=hi, dgi_init=dgi, dq0_init=dq0, eq0_init=3 * 32,
               **{f"p{j}_init": ptr[j] for j in range(4)})
    return ops, base, stepa, stepb, nq


CASES = [(nt, grp, ml, mh, rag)
         for grp in (1, 2, 3)
         for nt in sorted({grp, 2 * grp, 3 * grp, 5 * grp, 9 * grp, 12 * grp})
         for rag in (False, True)
         for ml, mh in sorted({(0, nt - (grp if rag else 0)), (min(nt, 2 * grp), nt - (grp if rag else 0)),
                               (nt, nt)})]


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("kind", sorted(KINDS))
def test_sweep_control_flow(dtype, kind):
    prog = program(dtype)
    w3 = kind == "stats"
    for ntot, grp, mlo, mhi, ragged in CASES:
        ops, base, stepa, stepb, nq = _case(kind, ntot, grp, mlo, mhi, ragged)
        ev = run(prog, ops)
        where = (ntot, grp, mlo, mhi, ragged)
        # DMAs: tiles hi + 1 .. ntot - 1 in order, with the cursor of the kernel
        dmas = [e for e in ev if e[0] == "dma"]
        tiles = list(range(ops["hi_init"] + 1, ntot))
        if kind == "none":
            tiles = []
        assert len(dmas) == 4 * len(tiles), where
        ptr, dgi, dq0 = list(base), 0, 3 * 32
        cursor = []
        for i in range(ntot):
            cursor.append((list(ptr), dq0))
            dgi += 1
            wrap = dgi == grp
            if wrap:
                dgi, dq0 = 0, dq0 + 32
            ptr = [(x + (stepb if wrap else stepa)) & M64 for x in ptr]
        for i, kt in enumerate(tiles):
            p_kt, q0 = cursor[kt]
            rag_tile = ragged and q0 == ops["ragq0"]
            for j in range(4):
                _, op, ptr_j, m0, which = dmas[4 * i + j]
                stage = LDSQ + (kt % 8) * STAGE
                if w3:
                    assert op == "global_load_lds_dword", where
                    assert ptr_j == p_kt[j], (where, kt, j)
                    assert m0 == stage + G.ST_OFF + 256 * j, (where, kt, j)
                else:
                    assert op == "global_load_lds_dwordx4", where
                    assert ptr_j == p_kt[0], (where, kt, j)
                    assert m0 == stage + 4096 + 1024 * j, (where, kt, j)
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
                # a wave that streams nothing has nothing of its own to wait for
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
        # masked element-wise steps and their tile offsets
        steps = []
        for e in ev:
            if e[0] == "label":
                m = re.fullmatch(r"Lbk64_(first|mid|last|single)(_m|_s)?_0", e[1])
                if m and m.group(2) != "_s":
                    steps.append((m.group(1), m.group(2) == "_m", e[2]))
        # a step is entered through its selection labels; the unmasked paths
        # fall through without a label, so count masked entries only
        masked_steps = [st for st in steps if st[1]]
        want = [t for t in range(ntot) if t < mlo or t >= mhi]
        assert len(masked_steps) == len(want), (where, len(masked_steps), want)
        for (_, _, state), t in zip(masked_steps, want):
            q0 = cursor[t][1]
            assert state[G.SG["eq0"]] == q0, (where, t, state[G.SG["eq0"]], q0)


def test_committed_inc_is_current():
    assert G.render() == (CSRC / "fhog_bwd_k64_loop.inc").read_text(), \
        "fhog_bwd_k64_loop.inc is out of date: run flash-hog_amd/csrc/gen_bwd_k64_loop.py"


def _regs(tok):
    m = re.fullmatch(r"-?([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.fullmatch(r"-?([va])(\d+)", tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _ws(ins):
    op = ins.split()[0]
    return int(ins.split()[1]) + 1 if op == "s_nop" else 1


CHAIN = 5


# bf16 operands of the output products (P, dS): each value written is read by
# exactly two matrix instructions (column blocks dt = 0, 1) before the next
# write, so no conversion overwrites a tile's values before its output
# products have taken them
OUT_OPERANDS = {("v", r) for r in [b[h] + i for b in (G.EDS, G.EP) for h in range(2) for i in range(8)]}


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
            # an accumulator input continues a chain: nothing but the chain's
            # previous matrix instruction has written it since
            for r in _regs(c):
                if r in last_valu_write:
                    assert last_valu_write[r] < last_mfma_write.get(r, -1), f"accumulator overwritten before {ins}"
            for r in (_regs(a) | _regs(b)) & OUT_OPERANDS:
                reads[r] = reads.get(r, 0) + 1
                assert reads[r] <= 2, f"{ins} reads an output operand a third time"
            for r in _regs(dst):
                last_mfma_write[r] = clock
                chain[r] = 1 if c == "0" else chain.get(r, 0) + 1
        elif op.startswith("v_"):
            dst = args[0]
            srcs = set()
            for x in args[1:]:
                srcs |= _regs(x)
            for r in srcs | _regs(dst):
                if r in last_mfma_write:
                    assert clock - last_mfma_write[r] >= 12, f"matrix result used by {ins} after {clock - last_mfma_write[r]}"
                # a score tile is read whole: its chain (the constants product
                # and four 16-deep products) is complete
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
    for ntot, grp, mlo, mhi, ragged in [(1, 1, 0, 1, False), (1, 1, 1, 1, False), (2, 1, 0, 2, False),
                                         (2, 2, 2, 2, False), (3, 1, 1, 3, False), (7, 1, 2, 6, True),
                                         (12, 2, 0, 12, False), (12, 3, 6, 9, True), (20, 1, 10, 19, True),
                                         (16, 2, 16, 16, False)]:
        ops = _case("tiles", ntot, grp, mlo, mhi, ragged)[0]
        trace = []
        run(prog, ops, trace=trace)
        check_hazards(trace)

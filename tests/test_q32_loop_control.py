"""Control flow of the generated stage-1 sweep (flash-hog_amd/csrc/gen_q32_loop.py).

The sweep is inline assembly, so nothing but this test looks at its scalar
side before it runs. The test executes the scalar instructions and branches
of every generated variant for each small (tiles, full tiles, ragged tail)
combination, treating vector, LDS and matrix instructions as no-ops, and
checks:
  - the sweep ends, after exactly one LDS DMA of every tile the kernel's own
    prologue did not issue, in order, from that tile's global address and
    into ring stage ((t0 + tile) mod 8) for the block's first ring tile t0,
    with the ragged tail's offsets only for the ragged tile;
  - at each DMA the tile it overwrites (tile - 8) was last read in a step
    that every wave has finished (its step index is at least two less than
    the current one), and every tile a step reads has been waited for;
  - on executed traces: no matrix instruction reads a fragment before the
    s_waitcnt that retires its LDS read, a matrix result is read by a vector
    instruction at least 12 wait states later, a vector result by a matrix
    instruction at least 2 later, a transcendental result by the next
    vector instruction at least 2 later;
  - the committed fhog_q32_loop.inc is the generator's output.
CPU only.
"""

from __future__ import annotations

import importlib.util
import pathlib
import re

import pytest

CSRC = pathlib.Path(__file__).resolve().parent.parent / "flash-hog_amd" / "csrc"


def _gen():
    spec = importlib.util.spec_from_file_location("gen_q32_loop", CSRC / "gen_q32_loop.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


G = _gen()


def _sreg(tok, s):
    m = re.fullmatch(r"s(\d+)", tok)
    if m:
        return s[int(m.group(1))]
    if tok == "m0":
        return s["m0"]
    return int(tok, 0)


def run(prog, ops, max_steps=200000, trace=None):
    """Executes the scalar side of prog with operand values ops. Returns the
    list of events: ('dma', gptr, m0, which), ('barrier',), ('wait', n). If
    trace is a list, every executed instruction is appended to it."""
    labels = {}
    for i, ins in enumerate(prog):
        if ins.endswith(":"):
            labels[ins[:-1]] = i
    s = {"m0": 0}
    scc = 0
    events = []
    pc = 0
    M = 0xFFFFFFFF
    steps = 0
    sub = lambda t: re.sub(r"%\[(\w+)\]", lambda m: str(ops[m.group(1)]), t)
    while pc < len(prog):
        steps += 1
        assert steps < max_steps, "the sweep does not end"
        ins = prog[pc]
        pc += 1
        if ins.endswith(":"):
            continue
        if trace is not None:
            trace.append(ins)
        op, *args = ins.replace(",", " ").split()
        if not op.startswith("s_") and not op.startswith("global_load_lds"):
            continue
        if op.startswith("global_load_lds"):
            base = args[1]
            m = re.fullmatch(r"s\[(\d+):(\d+)\]", base)
            lo = int(m.group(1))
            gptr = s[lo] | (s[lo + 1] << 32)
            events.append(("dma", gptr, s["m0"], args[0]))
            continue
        a = [sub(x) for x in args]
        if op == "s_mov_b32":
            s[int(a[0][1:]) if a[0] != "m0" else "m0"] = _sreg(a[1], s) & M
        elif op == "s_mov_b64":
            lo = int(re.fullmatch(r"s\[(\d+):\d+\]", a[0]).group(1))
            val = int(a[1], 0) if not a[1].startswith("s") else (s[int(a[1][2:].split(":")[0])] | (s[int(a[1][2:].split(":")[0]) + 1] << 32))
            s[lo], s[lo + 1] = val & M, val >> 32
        elif op in ("s_add_u32", "s_sub_u32", "s_and_b32", "s_lshl_b32", "s_addc_u32"):
            d = a[0]
            x, y = _sreg(a[1], s), _sreg(a[2], s)
            if op == "s_add_u32":
                r = x + y
                scc = int(r > M)
            elif op == "s_addc_u32":
                r = x + y + scc
                scc = int(r > M)
            elif op == "s_sub_u32":
                r = x - y
                scc = int(r < 0)
            elif op == "s_and_b32":
                r = x & y
                scc = int((r & M) != 0)
            else:
                r = x << y
                scc = int((r & M) != 0)
            s[int(d[1:]) if d != "m0" else "m0"] = r & M
        elif op.startswith("s_cmp_"):
            x, y = _sreg(a[0], s), _sreg(a[1], s)
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
        elif op in ("s_nop",):
            pass
        else:
            raise AssertionError(f"unmodelled scalar instruction {ins}")
    return events


def program(dtype, pre):
    prog = G.Gen(dtype, pre).generate()
    return [ins.replace("%=", "0") for ins in prog]


LDS_KV, LDS_W, GBASE, GSTEP = 0x10000, 0x10000 + 3 * 4096, 1 << 40, 32 * 2048


@pytest.mark.parametrize("variant", G.VARIANTS, ids=[v[0] for v in G.VARIANTS])
def test_sweep_control_flow(variant):
    _, dtype, pre = variant
    prog = program(dtype, pre)
    for nkt, t0 in [(k, 0) for k in range(1, 24)] + [(k, t) for k in (1, 2, 5, 6, 7, 9, 14) for t in (3, 7)]:
        for nfull in sorted({0, 1, nkt // 2, nkt - 1, nkt}):
            for ragged in (False, True):
                hi0 = min(4, nkt - 1)
                rag = t0 + nkt - 1 if ragged else 0xFFFFFFFF
                # operands in ring-tile numbers: the block's tile j is ring tile t0 + j
                ops = dict(nkt=t0 + nkt, nfull=t0 + nfull, rag=rag, hi0=t0 + hi0, t0=t0, ldskv=LDS_KV, ldsw=LDS_W,
                           gptr=GBASE + (hi0 + 1) * GSTEP, gstep=GSTEP)
                # the 64-bit operands are moved with s_mov_b64 from these values
                ev = run(prog, ops)
                dmas = [e for e in ev if e[0] == "dma"]
                # 4 loads per tile, tiles hi0 + 1 .. nkt - 1 in order
                tiles = list(range(hi0 + 1, nkt))
                assert len(dmas) == 4 * len(tiles), (nkt, nfull, len(dmas))
                for i, kt in enumerate(tiles):
                    for j in range(4):
                        _, gptr, m0, which = dmas[4 * i + j]
                        assert gptr == GBASE + kt * GSTEP, (nkt, kt, gptr)
                        assert m0 == LDS_W + ((t0 + kt) % 8) * 4 * 4096 + 1024 * j, (nkt, t0, kt, m0)
                        want = "%[vp{}]".format(j) if (ragged and kt == nkt - 1) else "%[vo{}]".format(j)
                        assert which == want.replace("%", "%"), (nkt, kt, which)
                # Ring discipline: number the barriers; the DMA of tile kt may
                # only follow the barrier that starts step kt - 6 + 1 ... i.e.
                # each DMA is issued after a barrier and at most 5 tiles ahead
                # of the newest tile any step has waited for.
                bars = 0
                waited = hi0 - 4  # tile waited for (by vmcnt) at the last barrier
                hi = hi0
                for e in ev:
                    if e[0] == "wait":
                        waited_now = hi - e[1] // 4
                    elif e[0] == "barrier":
                        waited = waited_now
                        # barrier k starts the step that reads tile k (the prologue
                        # tile 0, step t tile t + 1): it must have landed
                        assert waited >= bars, (nkt, nfull, bars, waited)
                        bars += 1
                    elif e[0] == "dma" and e[3].endswith("0]"):
                        hi += 1
                        # the stage of tile hi was last used by tile hi - 8,
                        # which is at least two steps behind the tile waited for
                        # (step t waits for tile t + 1 and reads tiles t - 1 .. t + 1)
                        assert hi - 8 <= waited - 3, (nkt, nfull, hi, waited)
                # steps: the prologue waits for tile 0, the first and middle steps
                # for tiles 1 .. nkt - 1
                assert bars == nkt, (nkt, nfull, bars)


def test_committed_inc_is_current():
    assert G.render() == (CSRC / "fhog_q32_loop.inc").read_text(), \
        "fhog_q32_loop.inc is out of date: run flash-hog_amd/csrc/gen_q32_loop.py"


def _regs(tok):
    """Registers named by an operand token: ('v', i) / ('a', i) tuples."""
    m = re.fullmatch(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.fullmatch(r"([va])(\d+)", tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _ws(ins):
    """Wait states an instruction provides."""
    op = ins.split()[0]
    return int(ins.split()[1]) + 1 if op == "s_nop" else 1


def check_hazards(trace):
    """Hazard rules of the generated code on an executed trace (pinned
    registers only; operands %[...] are the compiler's and are not written by
    vector instructions inside the sweep except the row sums)."""
    last_mfma_write = {}   # reg -> wait-state clock of the writing matrix instruction
    last_valu_write = {}   # reg -> clock
    last_trans_write = {}  # reg -> clock
    lds_pending = []       # registers of LDS reads not yet known complete, oldest first
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
            for r in _regs(dst):
                last_mfma_write[r] = clock
        elif op.startswith("v_"):
            dst = args[0]
            srcs = set()
            for x in args[1:]:
                srcs |= _regs(x)
            for r in srcs | _regs(dst):
                if r in last_mfma_write:
                    assert clock - last_mfma_write[r] >= 12, f"matrix result used by {ins} after {clock - last_mfma_write[r]}"
            for r in srcs:
                if r in last_trans_write:
                    assert clock - last_trans_write[r] >= 2, f"transcendental result read by {ins} too early"
            for regs in lds_pending:
                assert not (regs & (srcs | _regs(dst))), f"vector instruction touches a pending LDS read: {ins}"
            for r in _regs(dst):
                last_valu_write[r] = clock
                if op == "v_exp_f32":
                    last_trans_write[r] = clock
                else:
                    last_trans_write.pop(r, None)
        clock += _ws(ins)


@pytest.mark.parametrize("variant", G.VARIANTS, ids=[v[0] for v in G.VARIANTS])
def test_sweep_hazards(variant):
    _, dtype, pre = variant
    prog = program(dtype, pre)
    for nkt, nfull in ((1, 0), (1, 1), (2, 0), (2, 2), (3, 1), (7, 4), (12, 12), (12, 8)):
        hi0 = min(4, nkt - 1)
        t0 = nkt % 8
        ops = dict(nkt=t0 + nkt, nfull=t0 + nfull, rag=0xFFFFFFFF, hi0=t0 + hi0, t0=t0, ldskv=LDS_KV, ldsw=LDS_W,
                   gptr=GBASE + (hi0 + 1) * GSTEP, gstep=GSTEP)
        trace = []
        run(prog, ops, trace=trace)
        check_hazards(trace)

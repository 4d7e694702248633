#!/usr/bin/env python3
"""Writes fhog_bwd_k64_loop.inc: the query sweep of bwd_k64_kernel
(fhog_bwd_k64.hip, the dK/dV kernel of the first backward) as one
inline-assembly statement per input type (bf16, fp16).

A workgroup owns 256 keys (64 per wave, one wave per SIMD) and streams
32-query tiles of Q and dO and the tiles' row statistics L and D through an
8-stage LDS ring. Wave 0 streams Q, wave 1 dO (four global_load_lds_dwordx4
per tile each), wave 2 the statistics (four global_load_lds_dword: L, D and
the same two again, so that every streaming wave issues four loads per tile
and one wait count serves all), wave 3 nothing. Score tiles are S = Q K^T
(queries x keys): a lane holds one key column and sixteen query rows. The
wave's keys are two halves of 32 (h = 0, 1), each with its own resident K
and V, score tiles and accumulators; the query-side fragments a step reads
from LDS serve both halves, which halves the LDS bytes per pair against 32
keys per wave.

Per-query constants. The score accumulators start at -L k1 (S; k1 = 1 /
scale, so that S' = S - L / scale) and -D (dP), sixteen values per lane
each. Each wave turns the tile's raw statistics into one bf16 matrix operand:
lane (query m, half 0) holds the parts hi, mid, lo of a = -L k1 and b = -D at
k = 0, 2, 4 (a) and 1, 3, 5 (b); the other lanes hold zeros. Each chain of
score products starts with one bf16 matrix product of that operand and a
0/1 selector whose ones pick the three parts of its constant, so the
accumulator starts at hi + mid + lo, the fp32 constant to within an ulp
(the parts are successive roundings, see gen_k32_loop.py). For fp16 inputs
this product is still the bf16 instruction: it only initialises the fp32
accumulator. A row that sees no key (L = +inf) takes L = 1e30 (P = 0).

Step t (tile t's element-wise step):
  phase A: the 16 output products of tile t - 1 (dK += Q^T dS, dV += dO^T P
           for both halves; Q and dO fragments read transposed) beside the
           part of the element-wise step that reads S (P = exp2(S c2),
           masked) and the constants of tile t + 1;
  phase B: the 20 score products of tile t + 1, in chains S (h = 0), S
           (h = 1), dP (h = 0), dP (h = 1), each register set overwritten
           only after the element-wise step has read it, beside
           dS = P u (u = dP - D) and the conversions to the input type.
The DMA wait, barrier and DMA of tile t + 6 sit after phase A's third
matrix instruction in the steady step. Hazard distances follow
gen_q32_loop.py.

Usage: python gen_bwd_k64_loop.py [--check]   (--check: compare with the file on disk)
"""

from __future__ import annotations

import argparse
import pathlib
import sys

import gen_q32_loop as q

HERE = pathlib.Path(__file__).resolve().parent
OUT = HERE / "fhog_bwd_k64_loop.inc"

Frag, Sched, v, vr, frag = q.Frag, q.Sched, q.v, q.vr, q.frag

QTILE = 4096                  # bytes of one 32 x 64 tile of a 2-byte type
NST = 8
TOFF = {"Q": 0, "dO": QTILE}
ST_OFF = 2 * QTILE            # statistics: L at ST_OFF + 4 lane, D at + 256 (copies at + 512, + 768)
ADV_POS = 2                   # steady step: DMA wait, barrier, DMA after this matrix instruction
NH = 2                        # key halves per wave

# pinned registers
SC = (0, 32)                                 # S of half h (fp32, 16)
DPC = (16, 48)                               # dP of half h
EP = (64, 80)                                # bf16 P of half h (2 query halves x 4 regs)
EDS = (72, 88)                               # bf16 dS of half h
TP = (96, 128)                               # element-wise temporaries: P of half h (16)
TX = (112, 144)                              # dS of half h (16)
ADDR_R = 160                                 # 4: row fragments of tile t + 1, per 16-deep step
ADDR_TC = 164                                # 4: transposed fragments (a0, a1, b0, b1)
ADDR_TN = 168                                # 4: transposed fragments of tile t (last step)
MLO = (172, 173)                             # masked steps: first kept row offset of half h
STATA = 174                                  # 4: constants operand (hi, mid, lo, zero pairs; even)
STR = 178                                    # 2: raw statistics L, D
STT = 180                                    # 4: temporaries of the constants
ADDR_SA = 184                                # statistics reads of tile t + 1
NVGPR_PINNED = 185
FRAG0 = q.FRAG0
# s100 and s101 are outside the compiler's allocatable set and are not
# touched; m0 is saved in m0s and restored at the end. k2 is even (a pair).
SG = {"m0s": 80, "t": 81, "hi": 82, "dgi": 83, "dq0": 84, "egi": 85, "eq0": 86, "k0": 87,
      "k2": 88, "k3": 89, "k1": 90, "p0": 92, "p1": 94, "p2": 96, "p3": 98}
# Registers the kernel binds as in/out operands ("+{sN}") with their start
# values (the DMA cursor after the kernel's own first tiles): not clobbered.
BOUND = ("hi", "dgi", "dq0", "eq0", "p0", "p1", "p2", "p3")
WAVE_NONE = 0xFFFF            # ldsw of a wave that streams nothing


class BK64:
    def __init__(self, dtype: str):
        self.dtype = dtype
        self.mfma_op = f"v_mfma_f32_32x32x16_{'bf16' if dtype == 'bf16' else 'f16'}"
        self.const_op = "v_mfma_f32_32x32x16_bf16"   # the constants operand is bf16 for both types
        self.cvt = f"v_cvt_pk_{'bf16' if dtype == 'bf16' else 'f16'}_f32"
        self.out: list[str] = []

    def lbl(self, name):
        return f"Lbk64_{name}_%="

    def emit(self, s):
        self.out.append(s)

    # ----- fragments -----
    def row_frags(self):
        """Score-product A operands of one tile: per 16-deep step ks the Q
        and dO row fragments, Q in slots 8-11, dO in 12-15."""
        fr = {}
        base = {"Q": 8, "dO": 12}
        for ks in range(4):
            for name in ("Q", "dO"):
                k = base[name] + ks
                fr[(ks, name)] = Frag(k, [f"ds_read_b128 {frag(k)}, {v(ADDR_R + ks)} offset:{TOFF[name]}"])
        return fr

    def tr_frags(self, addr0):
        """Output-product A operands of one tile: per (column block dt, query
        half s) the Q and dO fragments read transposed, slots 0-7."""
        fr = {}
        k = 0
        for dt in range(2):
            for s in range(2):
                for name in ("Q", "dO"):
                    off = TOFF[name] + 2048 * s
                    a, b = v(addr0 + dt), v(addr0 + 2 + dt)
                    fr[(dt, s, name)] = Frag(k, [
                        f"ds_read_b64_tr_b16 a[{FRAG0 + 4 * k}:{FRAG0 + 4 * k + 1}], {a} offset:{off}",
                        f"ds_read_b64_tr_b16 a[{FRAG0 + 4 * k + 2}:{FRAG0 + 4 * k + 3}], {b} offset:{off + 1024}"])
                    k += 1
        return fr

    @staticmethod
    def tr_order(fr):
        return [fr[(dt, s, n)] for dt in range(2) for s in range(2) for n in ("Q", "dO")]

    def stats_frag(self):
        """The tile's raw statistics L and D; no matrix instruction reads them
        (slot 'st')."""
        return Frag("st", [f"ds_read_b32 {v(STR)}, {v(ADDR_SA)}",
                           f"ds_read_b32 {v(STR + 1)}, {v(ADDR_SA)} offset:256"])

    # ----- matrix instruction lists -----
    def score_mfmas(self, fr):
        """(text, frags) of a tile's 20 score products: chains S (h = 0, 1)
        and dP (h = 0, 1), each started by the constants product."""
        op = self.mfma_op
        st = vr(STATA, 4)
        m = []
        for h in range(NH):
            m.append((f"{self.const_op} {vr(SC[h], 16)}, {st}, %[sels], 0", []))
            for ks in range(4):
                m.append((f"{op} {vr(SC[h], 16)}, {frag(fr[(ks, 'Q')].slot)}, %[k{h}{ks}], {vr(SC[h], 16)}",
                          [fr[(ks, "Q")]]))
        for h in range(NH):
            m.append((f"{self.const_op} {vr(DPC[h], 16)}, {st}, %[selp], 0", []))
            for ks in range(4):
                m.append((f"{op} {vr(DPC[h], 16)}, {frag(fr[(ks, 'dO')].slot)}, %[v{h}{ks}], {vr(DPC[h], 16)}",
                          [fr[(ks, "dO")]]))
        return m

    def output_mfmas(self, fr):
        """(text, frags) of a tile's 16 output products."""
        op = self.mfma_op
        m = []
        for dt in range(2):
            for s in range(2):
                Q, dO = fr[(dt, s, "Q")], fr[(dt, s, "dO")]
                for h in range(NH):
                    m.append((f"{op} %[ak{h}{dt}], {frag(Q.slot)}, {vr(EDS[h] + 4 * s, 4)}, %[ak{h}{dt}]", [Q]))
                for h in range(NH):
                    m.append((f"{op} %[av{h}{dt}], {frag(dO.slot)}, {vr(EP[h] + 4 * s, 4)}, %[av{h}{dt}]", [dO]))
        return m

    @staticmethod
    def uses(mfmas):
        u = {}
        for _, fs in mfmas:
            for f in fs:
                u[f] = u.get(f, 0) + 1
        return u

    @staticmethod
    def first_use(mfmas, offset=0):
        fu = {}
        for i, (_, fs) in enumerate(mfmas):
            for f in fs:
                fu.setdefault(f, offset + i)
        return fu

    # ----- vector work -----
    def e_mul(self, h):
        """The read of S of half h: P = S c2 (before exp2)."""
        return [f"v_mul_f32 {v(TP[h] + r)}, %[c2], {v(SC[h] + r)}" for r in range(16)]

    def e_exp(self, h, masked):
        """P = exp2(P), masked. masked = "both": row 8 (r / 4) + 4 g + r % 4
        of the tile is kept iff (8 (r / 4) + r % 4) - MLO < width (unsigned),
        i.e. qfirst <= query < nq; "lo" (a tile inside nq): iff
        8 (r / 4) + r % 4 >= MLO (signed), i.e. qfirst <= query."""
        ops = []
        for b in range(4):
            rs = range(4 * b, 4 * b + 4)
            for r in rs:
                ops.append(f"v_exp_f32 {v(TP[h] + r)}, {v(TP[h] + r)}")
            for r in rs:
                const = 8 * (r // 4) + r % 4
                if masked == "both":
                    ops.append((f"v_sub_u32 {v(TX[h] + r)}, {const}, {v(MLO[h])}",
                                f"v_cmp_gt_u32 vcc, %[qw{h}], {v(TX[h] + r)}",
                                f"v_cndmask_b32 {v(TP[h] + r)}, 0, {v(TP[h] + r)}, vcc"))
                elif masked == "lo":
                    ops.append((f"v_cmp_ge_i32 vcc, {const}, {v(MLO[h])}",
                                f"v_cndmask_b32 {v(TP[h] + r)}, 0, {v(TP[h] + r)}, vcc"))
                else:
                    assert not masked
        return ops

    def e_ds(self, h):
        """dS = P u (reads dP of half h)."""
        return [f"v_mul_f32 {v(TX[h] + r)}, {v(TP[h] + r)}, {v(DPC[h] + r)}" for r in range(16)]

    def e_cvt(self, h):
        ops = []
        for s in range(2):
            for k in range(4):
                r0, r1 = 8 * s + 2 * k, 8 * s + 2 * k + 1
                ops.append(f"{self.cvt} {v(EP[h] + 4 * s + k)}, {v(TP[h] + r0)}, {v(TP[h] + r1)}")
                ops.append(f"{self.cvt} {v(EDS[h] + 4 * s + k)}, {v(TX[h] + r0)}, {v(TX[h] + r1)}")
        return ops

    def stats_ops(self):
        """The constants operand from the raw statistics (see the module
        docstring); the first entry is a marker for the LDS wait."""
        a, b, x, y = (v(STT + i) for i in range(4))
        r1, r2 = v(STR), v(STR + 1)
        hi, mid, lo = (v(STATA + i) for i in range(3))
        cvt = "v_cvt_pk_bf16_f32"
        return [
            "WAIT_STATS",
            # a row that sees no key has L = +inf; its parts would be -inf and
            # NaN, and the selectors' zero products (inf 0) would turn every
            # chain of the row into NaN. 1e30 keeps P = exp2(S c2) at 0.
            f"v_min_f32 {r1}, 0x7149f2ca, {r1}",
            f"v_mul_f32 {a}, {r1}, %[ca]",                       # -L k1 (lanes of half 0), else 0
            f"v_mul_f32 {b}, {r2}, %[cb]",                       # -D (lanes of half 0), else 0
            f"{cvt} {hi}, {a}, {b}",
            f"v_lshlrev_b32 {x}, 16, {hi}",
            f"v_and_b32 {y}, 0xffff0000, {hi}",
            f"v_sub_f32 {a}, {a}, {x}",
            f"v_sub_f32 {b}, {b}, {y}",
            f"{cvt} {mid}, {a}, {b}",
            f"v_lshlrev_b32 {x}, 16, {mid}",
            f"v_and_b32 {y}, 0xffff0000, {mid}",
            f"v_sub_f32 {a}, {a}, {x}",
            f"v_sub_f32 {b}, {b}, {y}",
            f"{cvt} {lo}, {a}, {b}",
        ]

    # ----- scalar pieces -----
    def stage_ops(self, dst, delta):
        """SGPR dst = lds base of the stage of tile t + delta."""
        k = f"s{SG[dst]}"
        return [f"s_add_u32 {k}, s{SG['t']}, {delta}", f"s_and_b32 {k}, {k}, {NST - 1}",
                f"s_lshl_b32 {k}, {k}, 14", f"s_add_u32 {k}, {k}, %[ldsq]"]

    def addr_row_ops(self, delta):
        """Row-fragment and statistics addresses of tile t + delta."""
        ops = self.stage_ops("k2", delta)
        ops += [f"v_add_u32 {v(ADDR_R + ks)}, s{SG['k2']}, %[ro{ks}]" for ks in range(4)]
        ops += [f"v_add_u32 {v(ADDR_SA)}, s{SG['k2']}, %[sta]"]
        return ops

    def addr_tr_ops(self, delta, base=ADDR_TC):
        ops = self.stage_ops("k3", delta)
        ops += [f"v_add_u32 {v(base + i)}, s{SG['k3']}, %[{n}]" for i, n in enumerate(("ta0", "ta1", "tb0", "tb1"))]
        return ops

    def mlo_ops(self):
        """MLO(h) = qfirst(h) - 4 g - q0 of tile t (masked steps)."""
        return [f"v_subrev_u32 {v(MLO[h])}, s{SG['eq0']}, %[qlo{h}]" for h in range(NH)]

    def ecursor_ops(self):
        """Advance the element-wise step's (head, query tile) cursor."""
        egi, eq0, k0 = (f"s{SG[n]}" for n in ("egi", "eq0", "k0"))
        return [f"s_add_u32 {egi}, {egi}, 1", f"s_cmp_eq_u32 {egi}, %[grp]", f"s_cselect_b32 {egi}, 0, {egi}",
                f"s_cselect_b32 {k0}, 32, 0", f"s_add_u32 {eq0}, {eq0}, {k0}"]

    def dma_ops(self, which, L):
        """DMA of the tile whose stage base is in k1: waves 0-1 four 16-byte
        loads of their tensor's tile, wave 2 four 4-byte loads of the
        statistics, wave 3 none. which: vo (full tile) or vp (the ragged last
        query tile)."""
        k1 = f"s{SG['k1']}"
        ops = [f"s_cmp_eq_u32 %[ldsw], {ST_OFF}", f"s_cbranch_scc1 {L('st_' + which)}",
               f"s_cmp_eq_u32 %[ldsw], {WAVE_NONE}", f"s_cbranch_scc1 {L('dc_' + which)}",
               f"s_add_u32 m0, {k1}, %[ldsw]"]
        for i in range(4):
            if i:
                ops.append("s_add_u32 m0, m0, 0x400")
            ops.append("s_nop 4" if i == 0 else "s_nop 0")
            ops.append(f"global_load_lds_dwordx4 %[{which}{i}], s[{SG['p0']}:{SG['p0'] + 1}]")
        ops.append(f"s_branch {L('dc_' + which)}")
        ops.append(f"{L('st_' + which)}:")
        ops.append(f"s_add_u32 m0, {k1}, {ST_OFF}")
        for i in range(4):
            if i:
                ops.append("s_add_u32 m0, m0, 0x100")
            ops.append("s_nop 4")  # each from its own base
            p = SG[f"p{i}"]
            ops.append(f"global_load_lds_dword %[{which}{i}], s[{p}:{p + 1}]")
        ops.append(f"{L('dc_' + which)}:")
        return ops

    def dcursor_ops(self):
        dgi, dq0, k0, k2, k3 = (f"s{SG[n]}" for n in ("dgi", "dq0", "k0", "k2", "k3"))
        ops = [f"s_add_u32 {dgi}, {dgi}, 1", f"s_cmp_eq_u32 {dgi}, %[grp]", f"s_cselect_b32 {dgi}, 0, {dgi}",
               f"s_cselect_b64 s[{SG['k2']}:{SG['k3']}], %[stepb], %[stepa]", f"s_cselect_b32 {k0}, 32, 0",
               f"s_add_u32 {dq0}, {dq0}, {k0}"]
        for i in range(4):
            p = SG[f"p{i}"]
            ops += [f"s_add_u32 s{p}, s{p}, {k2}", f"s_addc_u32 s{p + 1}, s{p + 1}, {k3}"]
        return ops

    def advance(self, need_delta, name):
        """Wait for tile t + need_delta (own DMAs), barrier, then the DMA of
        tile hi + 1 if there is one."""
        t, hi, k0, k1 = (f"s{SG[n]}" for n in ("t", "hi", "k0", "k1"))
        L = lambda x: self.lbl(f"{name}_{x}")
        out = [f"s_add_u32 {k0}, {t}, {need_delta}", f"s_sub_u32 {k0}, {hi}, {k0}"]
        for n in (4, 3, 2, 1):
            out += [f"s_cmp_{'ge' if n == 4 else 'eq'}_u32 {k0}, {n}", f"s_cbranch_scc1 {L(f'w{n}')}"]
        out += ["s_waitcnt vmcnt(0)", f"s_branch {L('wd')}"]
        for n in (1, 2, 3):
            out += [f"{L(f'w{n}')}:", f"s_waitcnt vmcnt({4 * n})", f"s_branch {L('wd')}"]
        out += [f"{L('w4')}:", "s_waitcnt vmcnt(16)", f"{L('wd')}:", "s_barrier"]
        out += [f"s_add_u32 {k0}, {hi}, 1", f"s_cmp_lt_u32 {k0}, %[ntot]", f"s_cbranch_scc0 {L('ni')}",
                f"s_mov_b32 {hi}, {k0}", f"s_and_b32 {k1}, {k0}, {NST - 1}", f"s_lshl_b32 {k1}, {k1}, 14",
                f"s_add_u32 {k1}, {k1}, %[ldsq]",
                f"s_cmp_eq_u32 s{SG['dq0']}, %[ragq0]", f"s_cbranch_scc1 {L('part')}"]
        out += self.dma_ops("vo", L)
        out += [f"s_branch {L('adv')}", f"{L('part')}:"]
        out += self.dma_ops("vp", L)
        out += [f"{L('adv')}:"]
        out += self.dcursor_ops()
        out += [f"{L('ni')}:"]
        for x in out:
            self.emit(x)

    def advance_steady(self, L):
        """advance(1) where tiles t + 2 .. t + 5 are in flight and tile t + 6
        exists and is a full query tile: no branches but the wave's DMA type.
        The DMA cursor's update (dcursor_ops) is left to the caller."""
        hi, k1 = (f"s{SG[n]}" for n in ("hi", "k1"))
        out = ["s_waitcnt vmcnt(16)", "s_barrier", f"s_add_u32 {hi}, {hi}, 1", f"s_and_b32 {k1}, {hi}, {NST - 1}",
               f"s_lshl_b32 {k1}, {k1}, 14", f"s_add_u32 {k1}, {k1}, %[ldsq]"]
        out += self.dma_ops("vo", L)
        return out

    # ----- emission -----
    @staticmethod
    def spread(ops, lo, hi):
        """slot -> ops: ops (strings or tuples kept together) spread evenly
        over slots lo .. hi - 1 (a slot is the gap after that matrix
        instruction)."""
        n = hi - lo
        res = {}
        for i, op in enumerate(ops):
            s = lo + (i * n) // max(1, len(ops))
            res.setdefault(s, []).append(op)
        return res

    @staticmethod
    def merge(*maps):
        res = {}
        for m in maps:
            for k, ops in m.items():
                res.setdefault(k, []).extend(ops)
        return res

    def run(self, sch, mfmas, slots, side, stfrag=None):
        """Emits mfmas; after matrix instruction i its side ops, then the
        paced LDS reads, then slots[i]. Slot -1 comes before the
        first matrix instruction. A side op "ADDR_TC" emits the transposed
        addresses of tile t (the caller's addr_tc) once every older
        transposed read has been issued."""
        def put(op):
            if op == "WAIT_STATS":
                sch.wait_for(stfrag)
            elif isinstance(op, tuple):
                for x in op:
                    sch.emit(x)
            else:
                sch.emit(op)

        def put_side(x):
            if isinstance(x, tuple) and x[0] == "ADDR_TC":
                old, ops = x[1], x[2]
                assert all(e[0] not in old for e in sch.queue), "old transposed reads pending"
                for y in ops:
                    sch.emit(y)
            else:
                sch.emit(x)

        for x in side.get(-1, []):
            put_side(x)
        if not mfmas:
            sch.issue_reads(greedy=True)
            for j, op in enumerate(slots.get(-1, [])):
                put(op)
                if j % 4 == 3:
                    sch.issue_reads(greedy=True)
            sch.issue_reads(greedy=True)
            return
        for op in slots.get(-1, []):
            put(op)
        sch.issue_reads()
        for i, (text, frags) in enumerate(mfmas):
            sch.mfma(text, frags)
            for x in side.get(i, []):
                put_side(x)
            # the gap's LDS reads first: their data returns while its vector ops issue
            sch.issue_reads()
            for op in slots.get(i, []):
                put(op)

    PREF_KEEP = 8

    def start_after_prefetch(self, sch, tf, mf_o):
        """The previous step read all eight transposed fragments of this
        step's output products; the last four (eight reads) may be in flight."""
        u = self.uses(mf_o)
        sch.ds = self.PREF_KEEP
        sch.done_upto = 0
        for k, f in enumerate(self.tr_order(tf)):
            f.last_ds = -1 if k < 4 else 2 * (k - 4) + 1
            sch.pending_uses[f.slot] = u[f]

    def end_with_prefetch(self, sch):
        sch.flush_reads()
        keep = min(self.PREF_KEEP, sch.ds - sch.done_upto)
        sch.emit(f"s_waitcnt lgkmcnt({keep})")

    def phase_b_vector(self, lo):
        """Phase B's vector work (the matrix instructions of phase B are
        lo .. lo + 19: S0 lo, S1 lo + 5, dP0 lo + 10, dP1 lo + 15): exp2 (and
        mask) of half 1 and dS of half 0 before dP0 is overwritten, dS of
        half 1 before dP1, and the conversions after their inputs."""
        return None  # built per block (the mask variant changes the exp2 part)

    def slots_b(self, lo, masked, exp1_before):
        """slot map of phase B's vector work; exp1_before: exp2 (and mask)
        of half 1 still to do (False when it already ran in phase A)."""
        exp1 = self.e_exp(1, masked) if exp1_before else []
        ds0, ds1 = self.e_ds(0), self.e_ds(1)
        cvt0, cvt1 = self.e_cvt(0), self.e_cvt(1)
        h = len(exp1) // 2
        return self.merge(
            self.spread(ds0 + exp1[:h], lo - 1, lo + 5),         # dS0 before dP0 (lo + 10)
            self.spread(exp1[h:] + cvt0[:8], lo + 5, lo + 10),
            self.spread(ds1 + cvt0[8:], lo + 10, lo + 15),       # dS1 before dP1 (lo + 15)
            self.spread(cvt1, lo + 15, lo + 20))

    # ----- blocks -----
    def block_prologue(self):
        """Pinned state, tile 0's DMA wait, its constants and score products."""
        self.emit(f"s_mov_b32 s{SG['m0s']}, m0")
        self.emit(f"s_mov_b32 s{SG['egi']}, 0")
        self.emit(f"s_mov_b32 s{SG['t']}, 0")
        self.emit(f"v_mov_b32 {v(STATA + 3)}, 0")
        self.advance(0, "pro")
        for x in self.addr_row_ops(0):
            self.emit(x)
        rf = self.row_frags()
        mf = self.score_mfmas(rf)
        st = self.stats_frag()
        sch = Sched(self.out, len(mf))
        sch.start()
        sch.enqueue([st], {st: 0}, {st: q.MIN_LEAD})
        sch.enqueue([rf[(ks, n)] for n in ("Q", "dO") for ks in range(4)], self.uses(mf), self.first_use(mf))
        self.run(sch, [], {-1: self.stats_ops()}, {}, st)
        self.emit("s_nop 1")
        self.run(sch, mf, {}, {})
        sch.flush_reads()
        self.emit("s_waitcnt lgkmcnt(0)")

    def next_step_frags(self, sch, n_block, not_before):
        tf_next = self.tr_frags(ADDR_TC)
        mf_next = self.output_mfmas(tf_next)
        sch.enqueue(self.tr_order(tf_next), self.uses(mf_next), self.first_use(mf_next, n_block), not_before)

    def block_first(self, masked):
        """t = 0: tile 0's element-wise step, tile 1's constants and score
        products; reads tile 0's transposed fragments for step 1."""
        masked = "both" if masked else False
        self.advance(1, f"first{int(bool(masked))}")
        for x in self.addr_row_ops(1) + self.addr_tr_ops(0) + (self.mlo_ops() if masked else []):
            self.emit(x)
        rf = self.row_frags()
        mf = self.score_mfmas(rf)
        st = self.stats_frag()
        sch = Sched(self.out, len(mf))
        sch.start()
        sch.enqueue([st], {st: 0}, {st: q.MIN_LEAD})
        sch.enqueue([rf[(ks, n)] for n in ("Q", "dO") for ks in range(4)], self.uses(mf), self.first_use(mf))
        # no matrix work beside the part of the step that reads S
        pre = self.e_mul(0) + self.e_exp(0, masked) + self.e_mul(1) + self.stats_ops()
        self.run(sch, [], {-1: pre}, {}, st)
        self.emit("s_nop 1")
        # the transposed fragments of tile 0 once the row fragments are out
        self.next_step_frags(sch, len(mf), 0)
        self.run(sch, mf, self.slots_b(0, masked, True), {})
        self.end_with_prefetch(sch)
        for x in self.ecursor_ops():
            self.emit(x)

    def block_mid(self, masked, steady=False):
        """Step t: output products of tile t - 1 (phase A), score products of
        tile t + 1 (phase B). masked: False, "lo" or "both" (e_exp)."""
        code = {False: "0", "lo": "1", "both": "2"}[masked]
        L = lambda x: self.lbl(f"mid{code}{int(steady)}_{x}")
        tf = self.tr_frags(ADDR_TC)
        mf_o = self.output_mfmas(tf)
        rf = self.row_frags()
        mf_s = self.score_mfmas(rf)
        mf = mf_o + mf_s
        no = len(mf_o)
        side = {}
        if steady:
            # DMA wait, barrier and DMA, then the row and statistics
            # addresses of tile t + 1, then the DMA cursor two scalar
            # instructions per gap (a burst of them would stall the matrix
            # unit)
            side[ADV_POS] = self.advance_steady(L)
            side[ADV_POS + 1] = self.addr_row_ops(1)
            # (instructions that read SCC stay in the gap of the one that set it)
            dc = self.dcursor_ops()
            groups = [dc[:5], dc[5:6]] + [dc[i:i + 2] for i in range(6, len(dc), 2)]
            for i, grp_ops in enumerate(groups):
                side[ADV_POS + 2 + i] = grp_ops
            nb = ADV_POS + 2
        else:
            self.advance(1, f"mid{code}")
            for x in self.addr_row_ops(1):
                self.emit(x)
            nb = 0
        if masked:
            for x in self.mlo_ops():
                self.emit(x)
        st = self.stats_frag()
        sch = Sched(self.out, len(mf))
        self.start_after_prefetch(sch, tf, mf_o)
        fu = self.first_use(mf)
        sch.enqueue([st], {st: 0}, {st: nb + q.MIN_LEAD + 2}, nb)
        sch.enqueue([rf[(ks, n)] for n in ("Q", "dO") for ks in range(4)], self.uses(mf_s), fu, nb)
        # phase A: S of both halves read (S0 before B0 = no, S1 before
        # no + 5), exp2 of half 0, and the constants of tile t + 1 before B0
        k = min(nb + 3, no - 6)  # the constants start once their reads can have landed
        slots = self.merge(
            self.spread(self.e_mul(0) + self.e_exp(0, masked)[:8], -1, k),
            self.spread(self.stats_ops(), k, no - 2),
            self.spread(self.e_exp(0, masked)[8:], k, no - 1),
            self.spread(self.e_mul(1), no - 2, no + 3),
            self.slots_b(no, masked, True))
        # the transposed addresses of tile t for the next step once every read
        # through those of tile t - 1 has been issued; then the element-wise
        # step's cursor and t (its last reader is ADDR_TC), one per gap
        side = self.merge(side, {no - 1: [("ADDR_TC", self.tr_order(tf), self.addr_tr_ops(0))]})
        ec = self.ecursor_ops()
        side = self.merge(side, {no + 2: ec[:4], no + 3: ec[4:] + [f"s_add_u32 s{SG['t']}, s{SG['t']}, 1"]})
        self.next_step_frags(sch, len(mf), no + 1)
        self.run(sch, mf, slots, side, st)
        self.end_with_prefetch(sch)

    def block_last(self, masked, single=False):
        """t = ntot - 1: output products of tile t - 1 (none when single)
        beside tile t's element-wise step, then tile t's output products."""
        masked = "both" if masked else False
        self.emit("s_nop 7")  # matrix results (the last score products) are read next
        self.emit("s_nop 7")
        for x in self.addr_tr_ops(0, ADDR_TN) + (self.mlo_ops() if masked else []):
            self.emit(x)
        tn = self.tr_frags(ADDR_TN)
        mf_n = self.output_mfmas(tn)
        ops = (self.e_mul(0) + self.e_exp(0, masked) + self.e_mul(1) + self.e_exp(1, masked)
               + self.e_ds(0) + self.e_ds(1))
        if not single:
            tf = self.tr_frags(ADDR_TC)
            mf_o = self.output_mfmas(tf)
            sch = Sched(self.out, len(mf_o) + len(mf_n))
            self.start_after_prefetch(sch, tf, mf_o)
            fu = self.first_use(mf_o + mf_n)
            sch.enqueue(self.tr_order(tn), self.uses(mf_n), fu)
            self.run(sch, mf_o, self.spread(ops, -1, len(mf_o)), {})
        else:
            sch = Sched(self.out, len(mf_n))
            sch.start()
            sch.enqueue(self.tr_order(tn), self.uses(mf_n), self.first_use(mf_n))
            self.run(sch, [], {-1: ops}, {})
        self.run(sch, [], {-1: self.e_cvt(0) + self.e_cvt(1)}, {})
        self.emit("s_nop 1")  # the last conversions are read by the matrix instructions below
        self.run(sch, mf_n, {}, {})
        sch.flush_reads()

    def generate(self):
        L = self.lbl
        t, k0 = f"s{SG['t']}", f"s{SG['k0']}"
        self.block_prologue()
        self.emit(f"s_cmp_eq_u32 %[ntot], 1")
        self.emit(f"s_cbranch_scc1 {L('single_sel')}")
        # t = 0 masked iff 0 < mlo or 0 >= mhi
        self.emit(f"s_cmp_lg_u32 %[mlo], 0")
        self.emit(f"s_cbranch_scc1 {L('first_m')}")
        self.emit(f"s_cmp_eq_u32 %[mhi], 0")
        self.emit(f"s_cbranch_scc1 {L('first_m')}")
        self.block_first(masked=False)
        self.emit(f"s_branch {L('first_done')}")
        self.emit(f"{L('first_m')}:")
        self.block_first(masked=True)
        self.emit(f"{L('first_done')}:")
        self.emit(f"s_mov_b32 {t}, 1")
        self.emit(f"{L('loop')}:")
        self.emit(f"s_add_u32 {k0}, {t}, 1")
        self.emit(f"s_cmp_ge_u32 {k0}, %[ntot]")
        self.emit(f"s_cbranch_scc1 {L('last_sel')}")
        self.emit(f"s_cmp_lt_u32 {t}, %[mlo]")
        self.emit(f"s_cbranch_scc1 {L('mid_m')}")
        self.emit(f"s_cmp_ge_u32 {t}, %[mhi]")
        self.emit(f"s_cbranch_scc1 {L('mid_m')}")
        self.emit(f"s_add_u32 {k0}, {t}, 7")
        self.emit(f"s_cmp_lt_u32 {k0}, %[nsd]")
        self.emit(f"s_cbranch_scc1 {L('mid_s')}")
        self.block_mid(masked=False)
        self.emit(f"s_branch {L('loop')}")
        self.emit(f"{L('mid_s')}:")
        self.block_mid(masked=False, steady=True)
        self.emit(f"s_branch {L('loop')}")
        self.emit(f"{L('mid_m')}:")
        # the ragged last query tile needs both bounds; the causal diagonal
        # only the lower one, and when tile t + 6 is a full tile its step is
        # a steady one
        self.emit(f"s_cmp_ge_u32 {t}, %[mhi]")
        self.emit(f"s_cbranch_scc1 {L('mid_mb')}")
        self.emit(f"s_add_u32 {k0}, {t}, 7")
        self.emit(f"s_cmp_lt_u32 {k0}, %[nsd]")
        self.emit(f"s_cbranch_scc1 {L('mid_ms')}")
        self.block_mid(masked="lo")
        self.emit(f"s_branch {L('loop')}")
        self.emit(f"{L('mid_ms')}:")
        self.block_mid(masked="lo", steady=True)
        self.emit(f"s_branch {L('loop')}")
        self.emit(f"{L('mid_mb')}:")
        self.block_mid(masked="both")
        self.emit(f"s_branch {L('loop')}")
        self.emit(f"{L('last_sel')}:")
        self.emit(f"s_cmp_lt_u32 {t}, %[mlo]")
        self.emit(f"s_cbranch_scc1 {L('last_m')}")
        self.emit(f"s_cmp_ge_u32 {t}, %[mhi]")
        self.emit(f"s_cbranch_scc1 {L('last_m')}")
        self.block_last(masked=False)
        self.emit(f"s_branch {L('end')}")
        self.emit(f"{L('last_m')}:")
        self.block_last(masked=True)
        self.emit(f"s_branch {L('end')}")
        self.emit(f"{L('single_sel')}:")
        self.emit(f"s_cmp_lg_u32 %[mlo], 0")
        self.emit(f"s_cbranch_scc1 {L('single_m')}")
        self.emit(f"s_cmp_eq_u32 %[mhi], 0")
        self.emit(f"s_cbranch_scc1 {L('single_m')}")
        self.block_last(masked=False, single=True)
        self.emit(f"s_branch {L('end')}")
        self.emit(f"{L('single_m')}:")
        self.block_last(masked=True, single=True)
        self.emit(f"{L('end')}:")
        self.emit("s_waitcnt lgkmcnt(0)")
        self.emit(f"s_mov_b32 m0, s{SG['m0s']}")
        # the accumulators are read by code the compiler places after this
        # statement, which cannot see the last matrix instructions
        self.emit("s_nop 7")
        self.emit("s_nop 7")
        self.emit("s_nop 3")
        return self.out


VARIANTS = (("BF16", "bf16"), ("F16", "f16"))


def render() -> str:
    lines = [
        "// Generated by gen_bwd_k64_loop.py; do not edit. The query sweep of",
        "// bwd_k64_kernel (fhog_bwd_k64.hip) as inline assembly, one string per",
        "// input type; operands and pinned registers are described there.",
        "#pragma once",
        "",
        "// registers the statements use beyond their operands",
        "#define FHOG_BK64_CLOBBERS \\",
    ]
    clob = [f'"v{i}"' for i in range(NVGPR_PINNED)] + [f'"a{i}"' for i in range(FRAG0, 256)]
    bound = set()
    for n in BOUND:
        bound |= {SG[n], SG[n] + 1} if n.startswith("p") else {SG[n]}
    clob += [f'"s{i}"' for i in range(min(SG.values()), max(SG.values()) + 2) if i not in bound]
    clob += ['"vcc"', '"scc"', '"memory"']
    for i in range(0, len(clob), 12):
        lines.append("  " + ", ".join(clob[i:i + 12]) + ("," if i + 12 < len(clob) else "") + " \\")
    lines.append("")
    lines.append("")
    lines.append("// the in/out operands bound to the registers the sweep keeps its DMA cursor in;")
    lines.append("// early-clobber, so that no input shares one of them")
    cons = []
    for n in BOUND:
        r = SG[n]
        cons.append(f'"+&{{s[{r}:{r + 1}]}}"({n})' if n.startswith("p") else f'"+&{{s{r}}}"({n})')
    lines.append(f"#define FHOG_BK64_BOUND({', '.join(BOUND)}) \\")
    lines.append("  " + ", ".join(cons))
    lines.append("")
    lines.append(f"#define FHOG_BK64_WAVE_NONE {WAVE_NONE}")
    lines.append(f"#define FHOG_BK64_STAT_OFF {ST_OFF}")
    lines.append("")
    for name, dtype in VARIANTS:
        body = BK64(dtype).generate()
        lines.append(f"#define FHOG_BK64_LOOP_{name} \\")
        for ins in body:
            lines.append(f'  "{ins}\\n\\t" \\')
        lines.append('  ""')
        lines.append("")
    return "\n".join(lines) + "\n"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--check", action="store_true")
    args = ap.parse_args(argv)
    text = render()
    if args.check:
        if not OUT.exists() or OUT.read_text() != text:
            print(f"{OUT} is out of date: run {pathlib.Path(__file__).name}", file=sys.stderr)
            return 1
        return 0
    OUT.write_text(text)
    print(OUT)
    return 0


if __name__ == "__main__":
    sys.exit(main())

#!/usr/bin/env python3
"""Writes fhog_k32_loop.inc: the query sweep of bwdbwd_k32_kernel
(fhog_bwdbwd_k32.hip, stage 2 of the double backward: dK2 and dV2) as one
inline-assembly statement per variant (bf16 with the scale folded into K and
ddK, bf16).

A workgroup owns 128 keys (32 per wave, one wave per SIMD) and streams
32-query tiles of Q, dO and ddQ and the tiles' row statistics through an
8-stage LDS ring. Waves 0-2 stream one query-side tensor each (four
global_load_lds_dwordx4 per tile); wave 3 streams the four statistics L, D,
dD, B (four global_load_lds_dword per tile, lanes 32-63 repeating lanes
0-31). Score tiles are S = Q K^T (queries x keys), so a lane holds one key
column and sixteen query rows.

Per-query constants. The score accumulators must start at -L (S), -dD (ddS),
-D (dP) and -(D dD + B) (dPa), sixteen values per lane each. Instead of
reading them from LDS, each wave turns the tile's raw statistics into one
matrix operand: lane (query m, half h) holds, for h = 0, the bf16 parts
hi, mid, lo of a = -L and b = -dD, for h = 1 those of a = -D and b = -c, at
k = 8 h + {0, 2, 4} (a) and 8 h + {1, 3, 5} (b). Each chain of score products
starts with one matrix product of that operand and a 0/1 selector whose ones
pick the three parts of its constant, so the accumulator starts at
hi + mid + lo, which is the fp32 constant to within an ulp (the parts are
exact successive roundings: x - hi is exact in fp32, and so on). That costs
three 4-byte LDS reads and 16 vector instructions per tile instead of sixteen
16-byte reads. A row that sees no key (L = +inf) takes L = 1e30: the product
multiplies every part, zero selectors included, and inf 0 is NaN.

Step t (tile t's element-wise step):
  phase A: the 12 output products of tile t - 1 (dK2 += ddQ^T dS, Q^T dS2;
           dV2 += dO^T ddP; LDS fragments read transposed) beside the part of
           the element-wise step that reads S and ddS, and the constants of
           tile t + 1;
  phase B: the 24 score products of tile t + 1, in chains S, ddS, dP, dPa
           (each register set is overwritten only after the element-wise
           step has read it), beside the rest of the element-wise step and
           the conversions to bf16.
The DMA wait, barrier and DMA of tile t + 6 sit after phase A's third matrix
instruction in the steady step. Hazard distances follow gen_q32_loop.py.

Usage: python gen_k32_loop.py [--check]   (--check: compare with the file on disk)
"""

from __future__ import annotations

import argparse
import pathlib
import sys

import gen_q32_loop as q

HERE = pathlib.Path(__file__).resolve().parent
OUT = HERE / "fhog_k32_loop.inc"

Frag, Sched, v, vr, frag = q.Frag, q.Sched, q.v, q.vr, q.frag

QTILE = 4096                  # bytes of one 32 x 64 bf16 tile
STAGE = 16384                 # Q, dO, ddQ, statistics
NST = 8
TOFF = {"Q": 0, "dO": QTILE, "dQ": 2 * QTILE}
ST_OFF = 3 * QTILE            # statistic j at ST_OFF + 256 j + 4 lane
ADV_POS = 2                   # steady step: DMA wait, barrier, DMA after this matrix instruction

# pinned registers
S0, DDS0, DP0, DPA0 = 0, 16, 32, 48          # score tiles (fp32, 16 each)
EDS0, EDS20, EDP0 = 64, 72, 80               # bf16 dS, dS2, ddP (2 halves x 4 regs)
TP0, TX0, T10 = 88, 104, 120                 # element-wise temporaries (16 each)
ADDR_R = 136                                 # 4: row fragments of tile t + 1, per 16-deep step
ADDR_TC = 140                                # 4: transposed fragments (a0, a1, b0, b1)
ADDR_TN = 144                                # 4: transposed fragments of tile t (last step)
MLO = 148                                    # masked steps: first kept row offset (see e1)
STATA = 150                                  # 4: constants operand (hi, mid, lo, zero pairs; even)
STR = 154                                    # 3: raw statistics r1, r2, r3
STT = 157                                    # 4: temporaries of the constants
ADDR_SA, ADDR_SB = 161, 162                  # statistics reads of tile t + 1
NVGPR_PINNED = 163
FRAG0 = q.FRAG0
# s100 and s101 are outside the compiler's allocatable set and are not
# touched; m0 is saved in m0s and restored at the end. k2 is even (a pair).
SG = {"m0s": 80, "t": 81, "hi": 82, "dgi": 83, "dq0": 84, "egi": 85, "eq0": 86, "k0": 87,
      "k2": 88, "k3": 89, "k1": 90, "p0": 92, "p1": 94, "p2": 96, "p3": 98}
# Registers the kernel binds as in/out operands ("+{sN}") with their start
# values (the DMA cursor after the kernel's own first tiles): not clobbered.
BOUND = ("hi", "dgi", "dq0", "eq0", "p0", "p1", "p2", "p3")


class K32:
    def __init__(self, pre: bool):
        self.pre = pre
        self.mfma_op = "v_mfma_f32_32x32x16_bf16"
        self.cvt = "v_cvt_pk_bf16_f32"
        self.out: list[str] = []

    def lbl(self, name):
        return f"Lk32_{name}_%="

    def emit(self, s):
        self.out.append(s)

    # ----- fragments -----
    def row_frags(self):
        """Score-product A operands of one tile: per 16-deep step ks the Q,
        ddQ and dO row fragments. Q in slots 12-15 (free during phase A),
        ddQ in 4-7, dO in 8-11."""
        fr = {}
        base = {"Q": 12, "dQ": 4, "dO": 8}
        for ks in range(4):
            for name in ("Q", "dQ", "dO"):
                k = base[name] + ks
                fr[(ks, name)] = Frag(k, [f"ds_read_b128 {frag(k)}, {v(ADDR_R + ks)} offset:{TOFF[name]}"])
        return fr

    def tr_frags(self, addr0):
        """Output-product A operands of one tile: per (column block dt, query
        half s) the ddQ, Q, dO fragments read transposed, slots 0-11."""
        fr = {}
        k = 0
        for dt in range(2):
            for s in range(2):
                for name in ("dQ", "Q", "dO"):
                    off = TOFF[name] + 2048 * s
                    a, b = v(addr0 + dt), v(addr0 + 2 + dt)
                    fr[(dt, s, name)] = Frag(k, [
                        f"ds_read_b64_tr_b16 a[{FRAG0 + 4 * k}:{FRAG0 + 4 * k + 1}], {a} offset:{off}",
                        f"ds_read_b64_tr_b16 a[{FRAG0 + 4 * k + 2}:{FRAG0 + 4 * k + 3}], {b} offset:{off + 1024}"])
                    k += 1
        return fr

    @staticmethod
    def first_tr(fr):
        """The first eight transposed fragments in use order."""
        order = [fr[(dt, s, n)] for dt in range(2) for s in range(2) for n in ("dQ", "Q", "dO")]
        return order[:8]

    @staticmethod
    def rest_tr(fr):
        order = [fr[(dt, s, n)] for dt in range(2) for s in range(2) for n in ("dQ", "Q", "dO")]
        return order[8:]

    def stats_frag(self):
        """The tile's raw statistics: r1 = L (h = 0) or D (h = 1), r2 = dD,
        r3 = B; no matrix instruction reads them (slot 'st')."""
        return Frag("st", [f"ds_read_b32 {v(STR)}, {v(ADDR_SA)}",
                           f"ds_read_b32 {v(STR + 1)}, {v(ADDR_SB)} offset:512",
                           f"ds_read_b32 {v(STR + 2)}, {v(ADDR_SB)} offset:768"])

    # ----- matrix instruction lists -----
    def score_mfmas(self, fr):
        """(text, frags) of a tile's 24 score products: chains S, ddS, dP,
        dPa, each started by the constants product."""
        op = self.mfma_op
        st = vr(STATA, 4)
        m = []
        m.append((f"{op} {vr(S0, 16)}, {st}, %[sels], 0", []))
        for ks in range(4):
            m.append((f"{op} {vr(S0, 16)}, {frag(fr[(ks, 'Q')].slot)}, %[k{ks}], {vr(S0, 16)}", [fr[(ks, "Q")]]))
        m.append((f"{op} {vr(DDS0, 16)}, {st}, %[seld], 0", []))
        for ks in range(4):
            m.append((f"{op} {vr(DDS0, 16)}, {frag(fr[(ks, 'dQ')].slot)}, %[k{ks}], {vr(DDS0, 16)}",
                      [fr[(ks, "dQ")]]))
            m.append((f"{op} {vr(DDS0, 16)}, {frag(fr[(ks, 'Q')].slot)}, %[dk{ks}], {vr(DDS0, 16)}",
                      [fr[(ks, "Q")]]))
        m.append((f"{op} {vr(DP0, 16)}, {st}, %[selp], 0", []))
        for ks in range(4):
            m.append((f"{op} {vr(DP0, 16)}, {frag(fr[(ks, 'dO')].slot)}, %[v{ks}], {vr(DP0, 16)}", [fr[(ks, "dO")]]))
        m.append((f"{op} {vr(DPA0, 16)}, {st}, %[sela], 0", []))
        for ks in range(4):
            m.append((f"{op} {vr(DPA0, 16)}, {frag(fr[(ks, 'dO')].slot)}, %[dv{ks}], {vr(DPA0, 16)}",
                      [fr[(ks, "dO")]]))
        return m

    def output_mfmas(self, fr):
        """(text, frags) of a tile's 12 output products."""
        op = self.mfma_op
        m = []
        for dt in range(2):
            for s in range(2):
                dQ, Q, dO = (fr[(dt, s, n)] for n in ("dQ", "Q", "dO"))
                m.append((f"{op} %[ak{dt}], {frag(dQ.slot)}, {vr(EDS0 + 4 * s, 4)}, %[ak{dt}]", [dQ]))
                m.append((f"{op} %[ak{dt}], {frag(Q.slot)}, {vr(EDS20 + 4 * s, 4)}, %[ak{dt}]", [Q]))
                m.append((f"{op} %[av{dt}], {frag(dO.slot)}, {vr(EDP0 + 4 * s, 4)}, %[av{dt}]", [dO]))
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
    def e1a(self, masked):
        """The part of tile t's element-wise step that reads S (and ddS
        without the folded scale): P = exp2(S c2), masked; t = ddS scale."""
        ops = []
        for b in range(4):
            rs = range(4 * b, 4 * b + 4)
            if not self.pre:
                for r in rs:
                    ops.append(f"v_mul_f32 {v(T10 + r)}, %[scl], {v(DDS0 + r)}")
            for r in rs:
                ops.append(f"v_mul_f32 {v(TP0 + r)}, %[c2], {v(S0 + r)}")
            for r in rs:
                ops.append(f"v_exp_f32 {v(TP0 + r)}, {v(TP0 + r)}")
            if masked:
                # row 8 (r / 4) + 4 g + r % 4 of the tile is kept iff
                # (8 (r / 4) + r % 4) - MLO < width (unsigned)
                for r in rs:
                    const = 8 * (r // 4) + r % 4
                    ops.append((f"v_sub_u32 {v(TX0 + r)}, {const}, {v(MLO)}",
                                f"v_cmp_gt_u32 vcc, %[qw], {v(TX0 + r)}",
                                f"v_cndmask_b32 {v(TP0 + r)}, 0, {v(TP0 + r)}, vcc"))
        return ops

    def e1b(self):
        """x = u t + dPa' and ddP = P t (reads ddS, dP, dPa)."""
        ops = []
        t = (lambda r: v(DDS0 + r)) if self.pre else (lambda r: v(T10 + r))
        for b in range(4):
            rs = range(4 * b, 4 * b + 4)
            for r in rs:
                ops.append(f"v_fma_f32 {v(TX0 + r)}, {v(DP0 + r)}, {t(r)}, {v(DPA0 + r)}")
            for r in rs:
                ops.append(f"v_mul_f32 {v(T10 + r)}, {v(TP0 + r)}, {t(r)}")
        return ops

    def e1c(self):
        """dS2 = P x and dS = P u (the last use of P; reads dP)."""
        ops = []
        for b in range(4):
            rs = range(4 * b, 4 * b + 4)
            for r in rs:
                ops.append(f"v_mul_f32 {v(TX0 + r)}, {v(TP0 + r)}, {v(TX0 + r)}")
            for r in rs:
                ops.append(f"v_mul_f32 {v(TP0 + r)}, {v(TP0 + r)}, {v(DP0 + r)}")
        return ops

    def e2(self):
        ops = []
        for s in range(2):
            for k in range(4):
                r0, r1 = 8 * s + 2 * k, 8 * s + 2 * k + 1
                ops.append(f"{self.cvt} {v(EDS0 + 4 * s + k)}, {v(TP0 + r0)}, {v(TP0 + r1)}")
                ops.append(f"{self.cvt} {v(EDS20 + 4 * s + k)}, {v(TX0 + r0)}, {v(TX0 + r1)}")
                ops.append(f"{self.cvt} {v(EDP0 + 4 * s + k)}, {v(T10 + r0)}, {v(T10 + r1)}")
        return ops

    def stats_ops(self):
        """The constants operand from the raw statistics (see the module
        docstring); the first entry is a marker for the LDS wait."""
        a, b, x, y = (v(STT + i) for i in range(4))
        r1, r2, r3 = (v(STR + i) for i in range(3))
        hi, mid, lo = (v(STATA + i) for i in range(3))
        return [
            "WAIT_STATS",
            # a row that sees no key has L = +inf; its parts would be -inf and
            # NaN, and the selectors' zero products (inf 0) would turn every
            # chain of the row into NaN. 1e30 keeps P = exp2(S c2) at 0.
            f"v_min_f32 {r1}, 0x7149f2ca, {r1}",
            f"v_mul_f32 {a}, {r1}, %[ca]",                       # -L k1 (h = 0) or -D
            f"v_fma_f32 {x}, {r1}, %[cnb], %[knb]",              # -k2 (h = 0) or -D
            f"v_mul_f32 {y}, {r3}, %[cb]",                       # 0 (h = 0) or -B
            f"v_fma_f32 {b}, {r2}, {x}, {y}",                    # -dD k2 or -(D dD + B)
            f"{self.cvt} {hi}, {a}, {b}",
            f"v_lshlrev_b32 {x}, 16, {hi}",
            f"v_and_b32 {y}, 0xffff0000, {hi}",
            f"v_sub_f32 {a}, {a}, {x}",
            f"v_sub_f32 {b}, {b}, {y}",
            f"{self.cvt} {mid}, {a}, {b}",
            f"v_lshlrev_b32 {x}, 16, {mid}",
            f"v_and_b32 {y}, 0xffff0000, {mid}",
            f"v_sub_f32 {a}, {a}, {x}",
            f"v_sub_f32 {b}, {b}, {y}",
            f"{self.cvt} {lo}, {a}, {b}",
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
        ops += [f"v_add_u32 {v(ADDR_SA)}, s{SG['k2']}, %[sta]", f"v_add_u32 {v(ADDR_SB)}, s{SG['k2']}, %[stb]"]
        return ops

    def addr_tr_ops(self, delta, base=ADDR_TC):
        ops = self.stage_ops("k3", delta)
        ops += [f"v_add_u32 {v(base + i)}, s{SG['k3']}, %[{n}]" for i, n in enumerate(("ta0", "ta1", "tb0", "tb1"))]
        return ops

    def mlo_ops(self):
        """MLO = qfirst - 4 g - q0 of tile t (masked steps)."""
        return [f"v_subrev_u32 {v(MLO)}, s{SG['eq0']}, %[qlo]"]

    def ecursor_ops(self):
        """Advance the element-wise step's (head, query tile) cursor."""
        egi, eq0, k0 = (f"s{SG[n]}" for n in ("egi", "eq0", "k0"))
        return [f"s_add_u32 {egi}, {egi}, 1", f"s_cmp_eq_u32 {egi}, %[grp]", f"s_cselect_b32 {egi}, 0, {egi}",
                f"s_cselect_b32 {k0}, 32, 0", f"s_add_u32 {eq0}, {eq0}, {k0}"]

    def dma_ops(self, which, L):
        """DMA of the tile whose stage base is in k1: waves 0-2 four 16-byte
        loads of their tensor's tile, wave 3 four 4-byte loads of the
        statistics; then the DMA cursor advances. which: vo (full tile) or
        vp (the ragged last query tile)."""
        k1 = f"s{SG['k1']}"
        ops = [f"s_cmp_eq_u32 %[ldsw], {ST_OFF}", f"s_cbranch_scc1 {L('st_' + which)}",
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

    def run(self, sch, mfmas, slots, side, stfrag=None):
        """Emits mfmas; after matrix instruction i its side ops, then the
        paced LDS reads, then slots[i]. Slot -1 comes before the
        first matrix instruction."""
        def put(op):
            if op == "WAIT_STATS":
                sch.wait_for(stfrag)
            elif isinstance(op, tuple):
                for x in op:
                    sch.emit(x)
            else:
                sch.emit(op)

        for x in side.get(-1, []):
            sch.emit(x)
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
                sch.emit(x)
            # the gap's LDS reads first: their data returns while its vector ops issue
            sch.issue_reads()
            for op in slots.get(i, []):
                put(op)

    def merge(self, *maps):
        res = {}
        for m in maps:
            for k, ops in m.items():
                res.setdefault(k, []).extend(ops)
        return res

    PREF_KEEP = 8

    def start_after_prefetch(self, sch, tf, mf_o):
        u = self.uses(mf_o)
        sch.ds = self.PREF_KEEP
        sch.done_upto = 0
        for k, f in enumerate(self.first_tr(tf)):
            f.last_ds = -1 if k < 4 else 2 * (k - 4) + 1
            sch.pending_uses[f.slot] = u[f]

    def end_with_prefetch(self, sch):
        sch.flush_reads()
        keep = min(self.PREF_KEEP, sch.ds - sch.done_upto)
        sch.emit(f"s_waitcnt lgkmcnt({keep})")

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
        sch.enqueue([rf[(ks, n)] for n in ("Q", "dQ", "dO") for ks in range(4)], self.uses(mf), self.first_use(mf))
        self.run(sch, [], {-1: self.stats_ops()}, {}, st)
        self.emit("s_nop 1")
        self.run(sch, mf, {}, {})
        sch.flush_reads()
        self.emit("s_waitcnt lgkmcnt(0)")

    def next_step_frags(self, sch, n_block, not_before):
        tf_next = self.tr_frags(ADDR_TC)
        mf_next = self.output_mfmas(tf_next)
        sch.enqueue(self.first_tr(tf_next), self.uses(mf_next), self.first_use(mf_next, n_block), not_before)

    def block_first(self, masked):
        """t = 0: tile 0's element-wise step, tile 1's constants and score
        products; reads tile 0's first transposed fragments for step 1."""
        self.advance(1, f"first{int(masked)}")
        for x in self.addr_row_ops(1) + self.addr_tr_ops(0) + (self.mlo_ops() if masked else []):
            self.emit(x)
        rf = self.row_frags()
        mf = self.score_mfmas(rf)
        st = self.stats_frag()
        sch = Sched(self.out, len(mf))
        sch.start()
        sch.enqueue([st], {st: 0}, {st: q.MIN_LEAD})
        sch.enqueue([rf[(ks, n)] for n in ("Q", "dQ", "dO") for ks in range(4)], self.uses(mf), self.first_use(mf))
        # no matrix work beside the first part of the step
        self.run(sch, [], {-1: self.e1a(masked) + self.stats_ops() + self.e1b()}, {}, st)
        self.emit("s_nop 1")
        self.next_step_frags(sch, len(mf), 0)
        slots = self.merge(self.spread(self.e1c(), 0, 9), self.spread(self.e2(), 9, len(mf)))
        self.run(sch, mf, slots, {})
        self.end_with_prefetch(sch)
        for x in self.ecursor_ops():
            self.emit(x)

    def block_mid(self, masked, steady=False):
        """Step t: output products of tile t - 1 (phase A), score products of
        tile t + 1 (phase B)."""
        L = lambda x: self.lbl(f"mid{int(masked)}{int(steady)}_{x}")
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
            self.advance(1, f"mid{int(masked)}")
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
        sch.enqueue(self.rest_tr(tf), self.uses(mf_o), fu)
        sch.enqueue([st], {st: 0}, {st: nb + q.MIN_LEAD + 2}, nb)
        sch.enqueue([rf[(ks, n)] for n in ("Q", "dQ", "dO") for ks in range(4)], self.uses(mf_s), fu, nb)
        # phase A and the first chain of phase B: the S-reading part and the
        # constants before B0, x and ddP before B5 (the ddS chain)
        e1a, stats, e1b = self.e1a(masked), self.stats_ops(), self.e1b()
        k = min(nb + 3, no - 4)  # the constants start once their reads can have landed
        first = self.spread(e1a, -1, k)
        second = self.spread(stats, k, no - 1)
        third = self.spread(e1b, no - 1, no + 5)
        fourth = self.merge(self.spread(self.e1c(), no + 5, no + 14), self.spread(self.e2(), no + 14, len(mf)))
        slots = self.merge(first, second, third, fourth)
        # the transposed addresses of tile t for the next step once every read
        # through those of tile t - 1 has been issued; then the element-wise
        # step's cursor and t (its last reader is ADDR_TC), one per gap
        side = self.merge(side, {no - 1: ["ADDR_TC"]})
        ec = self.ecursor_ops()
        side = self.merge(side, {no + 2: ec[:4], no + 3: ec[4:] + [f"s_add_u32 s{SG['t']}, s{SG['t']}, 1"]})
        self.next_step_frags(sch, len(mf), no + 1)
        addr_tc = self.addr_tr_ops(0)

        def run_with_addr():
            for x in side.get(-1, []):
                sch.emit(x)
            for op in slots.get(-1, []):
                put(op)
            sch.issue_reads()
            for i, (text, frags) in enumerate(mf):
                sch.mfma(text, frags)
                for x in side.get(i, []):
                    if x == "ADDR_TC":
                        assert all(e[0] not in self.rest_tr(tf) for e in sch.queue), "old transposed reads pending"
                        for y in addr_tc:
                            sch.emit(y)
                    else:
                        sch.emit(x)
                # the gap's LDS reads first: their data returns while its vector ops issue
                sch.issue_reads()
                for op in slots.get(i, []):
                    put(op)

        def put(op):
            if op == "WAIT_STATS":
                sch.wait_for(st)
            elif isinstance(op, tuple):
                for x in op:
                    sch.emit(x)
            else:
                sch.emit(op)

        run_with_addr()
        self.end_with_prefetch(sch)

    def block_last(self, masked, single=False):
        """t = ntot - 1: output products of tile t - 1 (none when single)
        beside tile t's element-wise step, then tile t's output products."""
        self.emit("s_nop 7")  # matrix results (the last score products) are read next
        self.emit("s_nop 7")
        for x in self.addr_tr_ops(0, ADDR_TN) + (self.mlo_ops() if masked else []):
            self.emit(x)
        tn = self.tr_frags(ADDR_TN)
        mf_n = self.output_mfmas(tn)
        ops = self.e1a(masked) + self.e1b() + self.e1c()
        if not single:
            tf = self.tr_frags(ADDR_TC)
            mf_o = self.output_mfmas(tf)
            sch = Sched(self.out, len(mf_o) + len(mf_n))
            self.start_after_prefetch(sch, tf, mf_o)
            fu = self.first_use(mf_o + mf_n)
            sch.enqueue(self.rest_tr(tf), self.uses(mf_o), fu)
            sch.enqueue(self.first_tr(tn) + self.rest_tr(tn), self.uses(mf_n), fu)
            self.run(sch, mf_o, self.spread(ops, -1, len(mf_o)), {})
        else:
            sch = Sched(self.out, len(mf_n))
            sch.start()
            sch.enqueue(self.first_tr(tn) + self.rest_tr(tn), self.uses(mf_n), self.first_use(mf_n))
            self.run(sch, [], {-1: ops}, {})
        self.run(sch, [], {-1: self.e2()}, {})
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
        self.block_mid(masked=True)
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


VARIANTS = (("BF16_PRE", True), ("BF16", False))


def render() -> str:
    lines = [
        "// Generated by gen_k32_loop.py; do not edit. The query sweep of",
        "// bwdbwd_k32_kernel (fhog_bwdbwd_k32.hip) as inline assembly, one string",
        "// per variant; operands and pinned registers are described there.",
        "#pragma once",
        "",
        "// registers the statements use beyond their operands",
        "#define FHOG_K32_CLOBBERS \\",
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
        # early-clobber: the sweep writes them before it has read every input,
        # so no input may share their register (an input holding the same
        # value, say 0, otherwise can)
        cons.append(f'"+&{{s[{r}:{r + 1}]}}"({n})' if n.startswith("p") else f'"+&{{s{r}}}"({n})')
    lines.append(f"#define FHOG_K32_BOUND({', '.join(BOUND)}) \\")
    lines.append("  " + ", ".join(cons))
    lines.append("")
    for name, pre in VARIANTS:
        body = K32(pre).generate()
        lines.append(f"#define FHOG_K32_LOOP_{name} \\")
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

#!/usr/bin/env python3
"""Writes fhog_bwd_q64_loop.inc: the key sweep of bwd_q64_kernel
(fhog_bwd_q64.hip, the dQ kernel of the first backward) as one
inline-assembly statement per input type (bf16, fp16).

A workgroup owns 256 queries (64 per wave, one wave per SIMD) and streams
32-key tiles of K (wave 0) and V (wave 1, four global_load_lds_dwordx4 per
tile each; waves 2 and 3 stream nothing) through an 8-stage LDS ring. Score
tiles are transposed, S^T = K Q^T (keys x queries): a lane holds one query
column and sixteen key rows, so the row statistics are per-lane scalars. The
wave's queries are two halves of 32 (h = 0, 1), each with its own resident Q
and dO, score tiles and dQ accumulators; the key-side fragments a step reads
from LDS serve both halves, which halves the LDS bytes per pair against 32
queries per wave.

Step t (tile t's element-wise step):
  phase A: the 8 output products of tile t - 1 (dQ^T += K^T dS^T for both
           halves; K fragments read transposed) beside the part of the
           element-wise step that reads S: P = exp2(S c2 - L log2 e),
           masked (keys past the lane's last visible key);
  phase B: the 16 score products of tile t + 1, in chains S (h = 0), S
           (h = 1), dP (h = 0), dP (h = 1), the dP chains starting at the
           per-lane tuple -D, each register set overwritten only after the
           element-wise step has read it, beside dS = P u (u = dP - D) and
           the conversions to the input type.
The DMA wait, barrier and DMA of tile t + 6 sit after phase A's third
matrix instruction in the steady step. Hazard distances follow
gen_q32_loop.py.

Usage: python gen_bwd_q64_loop.py [--check]   (--check: compare with the file on disk)
"""

from __future__ import annotations

import argparse
import pathlib
import sys

import gen_q32_loop as q

HERE = pathlib.Path(__file__).resolve().parent
OUT = HERE / "fhog_bwd_q64_loop.inc"

Frag, Sched, v, vr, frag = q.Frag, q.Sched, q.v, q.vr, q.frag

QTILE = 4096                  # bytes of one 32 x 64 tile of a 2-byte type
NST = 8
STAGE_SHIFT = 13              # 8 KiB stages: K, V
TOFF = {"K": 0, "V": QTILE}
ADV_POS = 2                   # steady step: DMA wait, barrier, DMA after this matrix instruction
NH = 2                        # query halves per wave

# pinned registers
SC = (0, 32)                                 # S^T of half h (fp32, 16)
DPC = (16, 48)                               # dP^T of half h
EDS = (64, 72)                               # bf16 dS of half h (2 key halves x 4 regs)
TP = (80, 112)                               # element-wise temporaries: P of half h (16)
TX = (96, 128)                               # dS of half h (16)
INITU = (144, 160)                           # 16 x (-D) of half h: start of its dP chain
ADDR_R = 176                                 # 4: row fragments of tile t + 1, per 16-deep step
ADDR_TC = 180                                # 4: transposed fragments (a0, a1, b0, b1)
ADDR_TN = 184                                # 4: transposed fragments of tile t (last step)
KLIM = (188, 189)                            # masked steps: last visible key - 4 g of half h, tile-relative
NVGPR_PINNED = 190
FRAG0 = q.FRAG0
# s100 and s101 are outside the compiler's allocatable set and are not
# touched; m0 is saved in m0s and restored at the end. k2 is even (a pair).
SG = {"m0s": 80, "t": 81, "hi": 82, "dgi": 83, "dq0": 84, "egi": 85, "eq0": 86, "k0": 87,
      "k2": 88, "k3": 89, "k1": 90, "p0": 92}
# Registers the kernel binds as in/out operands ("+{sN}") with their start
# values (the DMA cursor after the kernel's own first tiles): not clobbered.
BOUND = ("hi", "dgi", "dq0", "eq0", "p0")
WAVE_NONE = 0xFFFF            # ldsw of a wave that streams nothing


class BQ64:
    def __init__(self, dtype: str):
        self.dtype = dtype
        self.mfma_op = f"v_mfma_f32_32x32x16_{'bf16' if dtype == 'bf16' else 'f16'}"
        self.cvt = f"v_cvt_pk_{'bf16' if dtype == 'bf16' else 'f16'}_f32"
        self.out: list[str] = []

    def lbl(self, name):
        return f"Lbq64_{name}_%="

    def emit(self, s):
        self.out.append(s)

    # ----- fragments -----
    def row_frags(self):
        """Score-product A operands of one tile: per 16-deep step ks the K
        and V row fragments, K in slots 8-11, V in 12-15."""
        fr = {}
        base = {"K": 8, "V": 12}
        for ks in range(4):
            for name in ("K", "V"):
                k = base[name] + ks
                fr[(ks, name)] = Frag(k, [f"ds_read_b128 {frag(k)}, {v(ADDR_R + ks)} offset:{TOFF[name]}"])
        return fr

    def tr_frags(self, addr0):
        """Output-product A operands of one tile: per (column block dt, key
        half s) the K fragment read transposed, slots 0-3."""
        fr = {}
        k = 0
        for dt in range(2):
            for s in range(2):
                off = TOFF["K"] + 2048 * s
                a, b = v(addr0 + dt), v(addr0 + 2 + dt)
                fr[(dt, s)] = Frag(k, [
                    f"ds_read_b64_tr_b16 a[{FRAG0 + 4 * k}:{FRAG0 + 4 * k + 1}], {a} offset:{off}",
                    f"ds_read_b64_tr_b16 a[{FRAG0 + 4 * k + 2}:{FRAG0 + 4 * k + 3}], {b} offset:{off + 1024}"])
                k += 1
        return fr

    @staticmethod
    def tr_order(fr):
        return [fr[(dt, s)] for dt in range(2) for s in range(2)]

    # ----- matrix instruction lists -----
    def score_mfmas(self, fr):
        """(text, frags) of a tile's 16 score products: chains S (h = 0, 1)
        and dP (h = 0, 1); the dP chains start at the -D tuple."""
        op = self.mfma_op
        m = []
        for h in range(NH):
            for ks in range(4):
                c = "0" if ks == 0 else vr(SC[h], 16)
                m.append((f"{op} {vr(SC[h], 16)}, {frag(fr[(ks, 'K')].slot)}, %[q{h}{ks}], {c}", [fr[(ks, "K")]]))
        for h in range(NH):
            for ks in range(4):
                c = vr(INITU[h], 16) if ks == 0 else vr(DPC[h], 16)
                m.append((f"{op} {vr(DPC[h], 16)}, {frag(fr[(ks, 'V')].slot)}, %[o{h}{ks}], {c}",
                          [fr[(ks, "V")]]))
        return m

    def output_mfmas(self, fr):
        """(text, frags) of a tile's 8 output products."""
        op = self.mfma_op
        m = []
        for dt in range(2):
            for s in range(2):
                K = fr[(dt, s)]
                for h in range(NH):
                    m.append((f"{op} %[aq{h}{dt}], {frag(K.slot)}, {vr(EDS[h] + 4 * s, 4)}, %[aq{h}{dt}]", [K]))
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
        """The read of S of half h: P = S c2 - L log2 e (before exp2)."""
        return [f"v_fma_f32 {v(TP[h] + r)}, {v(SC[h] + r)}, %[c2], %[nl{h}]" for r in range(16)]

    def e_exp(self, h, masked):
        """P = exp2(P), masked: key 8 (r / 4) + 4 g + r % 4 of the tile is
        kept iff 8 (r / 4) + r % 4 <= KLIM (the lane's last visible key, less
        4 g, tile-relative)."""
        ops = []
        for b in range(4):
            rs = range(4 * b, 4 * b + 4)
            for r in rs:
                ops.append(f"v_exp_f32 {v(TP[h] + r)}, {v(TP[h] + r)}")
            if masked:
                for r in rs:
                    const = 8 * (r // 4) + r % 4
                    ops.append((f"v_cmp_gt_i32 vcc, {const}, {v(KLIM[h])}",
                                f"v_cndmask_b32_e64 {v(TP[h] + r)}, {v(TP[h] + r)}, 0, vcc"))
        return ops

    def e_ds(self, h):
        """dS = P u (reads dP of half h, which started at -D)."""
        return [f"v_mul_f32 {v(TX[h] + r)}, {v(TP[h] + r)}, {v(DPC[h] + r)}" for r in range(16)]

    def e_cvt(self, h):
        ops = []
        for s in range(2):
            for k in range(4):
                r0, r1 = 8 * s + 2 * k, 8 * s + 2 * k + 1
                ops.append(f"{self.cvt} {v(EDS[h] + 4 * s + k)}, {v(TX[h] + r0)}, {v(TX[h] + r1)}")
        return ops

    # ----- scalar pieces -----
    def stage_ops(self, dst, delta):
        """SGPR dst = lds base of the stage of tile t + delta."""
        k = f"s{SG[dst]}"
        return [f"s_add_u32 {k}, s{SG['t']}, {delta}", f"s_and_b32 {k}, {k}, {NST - 1}",
                f"s_lshl_b32 {k}, {k}, {STAGE_SHIFT}", f"s_add_u32 {k}, {k}, %[ldsk]"]

    def addr_row_ops(self, delta):
        """Row-fragment addresses of tile t + delta."""
        ops = self.stage_ops("k2", delta)
        ops += [f"v_add_u32 {v(ADDR_R + ks)}, s{SG['k2']}, %[ro{ks}]" for ks in range(4)]
        return ops

    def addr_tr_ops(self, delta, base=ADDR_TC):
        ops = self.stage_ops("k3", delta)
        ops += [f"v_add_u32 {v(base + i)}, s{SG['k3']}, %[{n}]" for i, n in enumerate(("ta0", "ta1", "tb0", "tb1"))]
        return ops

    def klim_ops(self):
        """KLIM(h) = klb(h) - k0 of tile t (masked steps)."""
        return [f"v_subrev_u32 {v(KLIM[h])}, s{SG['eq0']}, %[klb{h}]" for h in range(NH)]

    def ecursor_ops(self):
        """Advance the element-wise step's key offset."""
        return [f"s_add_u32 s{SG['eq0']}, s{SG['eq0']}, 32"]

    def dma_ops(self, which, L):
        """DMA of the tile whose stage base is in k1: waves 0-1 four 16-byte
        loads of their tensor's tile, waves 2-3 none. which: vo (full tile)
        or vp (the ragged last key tile)."""
        k1 = f"s{SG['k1']}"
        ops = [f"s_cmp_eq_u32 %[ldsw], {WAVE_NONE}", f"s_cbranch_scc1 {L('dc_' + which)}",
               f"s_add_u32 m0, {k1}, %[ldsw]"]
        for i in range(4):
            if i:
                ops.append("s_add_u32 m0, m0, 0x400")
            ops.append("s_nop 4" if i == 0 else "s_nop 0")
            ops.append(f"global_load_lds_dwordx4 %[{which}{i}], s[{SG['p0']}:{SG['p0'] + 1}]")
        ops.append(f"{L('dc_' + which)}:")
        return ops

    def dcursor_ops(self):
        """The DMA cursor: key offset and source pointer of the next tile."""
        dq0, p = f"s{SG['dq0']}", SG["p0"]
        return [f"s_add_u32 {dq0}, {dq0}, 32",
                f"s_add_u32 s{p}, s{p}, %[gstep_lo]", f"s_addc_u32 s{p + 1}, s{p + 1}, %[gstep_hi]"]

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
                f"s_mov_b32 {hi}, {k0}", f"s_and_b32 {k1}, {k0}, {NST - 1}",
                f"s_lshl_b32 {k1}, {k1}, {STAGE_SHIFT}", f"s_add_u32 {k1}, {k1}, %[ldsk]",
                f"s_cmp_eq_u32 s{SG['dq0']}, %[ragk0]", f"s_cbranch_scc1 {L('part')}"]
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
        exists and is a full key tile: no branches but the wave's DMA type.
        The DMA cursor's update (dcursor_ops) is left to the caller."""
        hi, k1 = (f"s{SG[n]}" for n in ("hi", "k1"))
        out = ["s_waitcnt vmcnt(16)", "s_barrier", f"s_add_u32 {hi}, {hi}, 1", f"s_and_b32 {k1}, {hi}, {NST - 1}",
               f"s_lshl_b32 {k1}, {k1}, {STAGE_SHIFT}", f"s_add_u32 {k1}, {k1}, %[ldsk]"]
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

    def run(self, sch, mfmas, slots, side):
        """Emits mfmas; after matrix instruction i its side ops, then the
        paced LDS reads, then slots[i]. Slot -1 comes before the
        first matrix instruction. A side op ("ADDR_TC", old, ops) emits ops
        (the transposed addresses of tile t) once every older transposed read
        has been issued."""
        def put(op):
            if isinstance(op, tuple):
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

    PREF_KEEP = 4

    def start_after_prefetch(self, sch, tf, mf_o):
        """The previous step read all four transposed fragments of this
        step's output products; the last two (four reads) may be in flight."""
        u = self.uses(mf_o)
        sch.ds = self.PREF_KEEP
        sch.done_upto = 0
        for k, f in enumerate(self.tr_order(tf)):
            f.last_ds = -1 if k < 2 else 2 * (k - 2) + 1
            sch.pending_uses[f.slot] = u[f]

    def end_with_prefetch(self, sch):
        sch.flush_reads()
        keep = min(self.PREF_KEEP, sch.ds - sch.done_upto)
        sch.emit(f"s_waitcnt lgkmcnt({keep})")

    def slots_b(self, lo, masked):
        """slot map of phase B's vector work (its matrix instructions are
        lo .. lo + 15: S0 lo, S1 lo + 4, dP0 lo + 8, dP1 lo + 12): exp2 (and
        mask) of half 1, dS of half 0 before dP0 is overwritten and of half 1
        before dP1, the conversions after their inputs."""
        exp1 = self.e_exp(1, masked)
        ds0, ds1 = self.e_ds(0), self.e_ds(1)
        cvt0, cvt1 = self.e_cvt(0), self.e_cvt(1)
        h = len(exp1) // 2
        return self.merge(
            self.spread(ds0 + exp1[:h], lo - 1, lo + 4),
            self.spread(exp1[h:] + cvt0[:4], lo + 4, lo + 8),        # dS0 done before dP0 (lo + 8)
            self.spread(ds1 + cvt0[4:], lo + 8, lo + 12),           # dS1 before dP1 (lo + 12)
            self.spread(cvt1, lo + 12, lo + 16))

    # ----- blocks -----
    def block_prologue(self):
        """Pinned state, tile 0's DMA wait and its score products."""
        self.emit(f"s_mov_b32 s{SG['m0s']}, m0")
        self.emit(f"s_mov_b32 s{SG['t']}, 0")
        for h in range(NH):
            for r in range(16):
                self.emit(f"v_mov_b32 {v(INITU[h] + r)}, %[nd{h}]")
        self.advance(0, "pro")
        for x in self.addr_row_ops(0):
            self.emit(x)
        rf = self.row_frags()
        mf = self.score_mfmas(rf)
        sch = Sched(self.out, len(mf))
        sch.start()
        sch.enqueue([rf[(ks, n)] for n in ("K", "V") for ks in range(4)], self.uses(mf), self.first_use(mf))
        self.run(sch, mf, {}, {})
        sch.flush_reads()
        self.emit("s_waitcnt lgkmcnt(0)")

    def next_step_frags(self, sch, n_block, not_before):
        tf_next = self.tr_frags(ADDR_TC)
        mf_next = self.output_mfmas(tf_next)
        sch.enqueue(self.tr_order(tf_next), self.uses(mf_next), self.first_use(mf_next, n_block), not_before)

    def block_first(self, masked):
        """t = 0: tile 0's element-wise step, tile 1's score products; reads
        tile 0's transposed fragments for step 1."""
        self.emit("s_nop 7")  # matrix results (the prologue's score products) are read next
        self.emit("s_nop 4")
        self.advance(1, f"first{int(masked)}")
        for x in self.addr_row_ops(1) + self.addr_tr_ops(0) + (self.klim_ops() if masked else []):
            self.emit(x)
        rf = self.row_frags()
        mf = self.score_mfmas(rf)
        sch = Sched(self.out, len(mf))
        sch.start()
        sch.enqueue([rf[(ks, n)] for n in ("K", "V") for ks in range(4)], self.uses(mf), self.first_use(mf))
        # no matrix work beside the part of the step that reads S
        pre = self.e_mul(0) + self.e_exp(0, masked) + self.e_mul(1)
        self.run(sch, [], {-1: pre}, {})
        self.next_step_frags(sch, len(mf), 0)
        self.run(sch, mf, self.slots_b(0, masked), {})
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
            # DMA wait, barrier and DMA, then the row addresses of tile t + 1,
            # then the DMA cursor
            side[ADV_POS] = self.advance_steady(L)
            side[ADV_POS + 1] = self.addr_row_ops(1)
            dc = self.dcursor_ops()
            side[ADV_POS + 2] = dc[:1]
            side[ADV_POS + 3] = dc[1:]   # (s_addc reads the carry of the s_add before it)
            nb = ADV_POS + 2
        else:
            self.advance(1, f"mid{int(masked)}")
            for x in self.addr_row_ops(1):
                self.emit(x)
            nb = 0
        if masked:
            for x in self.klim_ops():
                self.emit(x)
        sch = Sched(self.out, len(mf))
        self.start_after_prefetch(sch, tf, mf_o)
        fu = self.first_use(mf)
        sch.enqueue([rf[(ks, n)] for n in ("K", "V") for ks in range(4)], self.uses(mf_s), fu, nb)
        # phase A: S of half 0 read before B0 (= no), of half 1 before no + 4;
        # exp2 of half 0
        slots = self.merge(
            self.spread(self.e_mul(0) + self.e_exp(0, masked), -1, no - 1),
            self.spread(self.e_mul(1), no - 2, no + 3),
            self.slots_b(no, masked))
        # the transposed addresses of tile t for the next step; then the
        # element-wise step's cursor and t (its last reader is ADDR_TC)
        side = self.merge(side, {no - 1: [("ADDR_TC", self.tr_order(tf), self.addr_tr_ops(0))]})
        side = self.merge(side, {no + 2: self.ecursor_ops() + [f"s_add_u32 s{SG['t']}, s{SG['t']}, 1"]})
        self.next_step_frags(sch, len(mf), no + 1)
        self.run(sch, mf, slots, side)
        self.end_with_prefetch(sch)

    def block_last(self, masked, single=False):
        """t = ntot - 1: output products of tile t - 1 (none when single)
        beside tile t's element-wise step, then tile t's output products."""
        self.emit("s_nop 7")  # matrix results (the last score products) are read next
        self.emit("s_nop 7")
        for x in self.addr_tr_ops(0, ADDR_TN) + (self.klim_ops() if masked else []):
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
        # t = 0 masked iff 0 >= nfull
        self.emit(f"s_cmp_eq_u32 %[nfull], 0")
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
        self.emit(f"s_cmp_ge_u32 {t}, %[nfull]")
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
        self.emit(f"s_cmp_ge_u32 {t}, %[nfull]")
        self.emit(f"s_cbranch_scc1 {L('last_m')}")
        self.block_last(masked=False)
        self.emit(f"s_branch {L('end')}")
        self.emit(f"{L('last_m')}:")
        self.block_last(masked=True)
        self.emit(f"s_branch {L('end')}")
        self.emit(f"{L('single_sel')}:")
        self.emit(f"s_cmp_eq_u32 %[nfull], 0")
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
        "// Generated by gen_bwd_q64_loop.py; do not edit. The key sweep of",
        "// bwd_q64_kernel (fhog_bwd_q64.hip) as inline assembly, one string per",
        "// input type; operands and pinned registers are described there.",
        "#pragma once",
        "",
        "// registers the statements use beyond their operands",
        "#define FHOG_BQ64_CLOBBERS \\",
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
    lines.append(f"#define FHOG_BQ64_BOUND({', '.join(BOUND)}) \\")
    lines.append("  " + ", ".join(cons))
    lines.append("")
    lines.append(f"#define FHOG_BQ64_WAVE_NONE {WAVE_NONE}")
    lines.append("")
    for name, dtype in VARIANTS:
        body = BQ64(dtype).generate()
        lines.append(f"#define FHOG_BQ64_LOOP_{name} \\")
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

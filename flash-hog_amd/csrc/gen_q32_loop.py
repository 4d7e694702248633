#!/usr/bin/env python3
"""Writes fhog_q32_loop.inc: the key sweep of bwdbwd_q32_kernel
(fhog_bwdbwd_q32.hip) as one inline-assembly statement per instruction
variant (bf16 with the scale folded into Q and ddQ, bf16, fp16).

Why assembly. At one wave per SIMD nothing hides a stall, so every LDS read
must be issued several matrix instructions before its use and every matrix
instruction must have vector work beside it. Left to itself the compiler keeps
the score tiles in AGPRs (at one wave per SIMD it selects the AGPR form of
every matrix instruction) and copies every element out before the
element-wise step, and it issues most LDS reads directly before the
instruction that consumes them; that version ran at about 3460 cycles per
32-key step against 1650 for a hand-interleaved loop of the same instruction
mix.

Structure. A step t of the sweep issues
  phase A: the 26 output products of tile t - 1 (their LDS fragments are
           tile t - 1's key-side tiles read transposed; two of them take a
           ones operand and sum the rounded x over the keys, which a
           dot-product instruction would do at several times the cost)
           beside the first half
           of tile t's element-wise step, which reads the four score tiles
           into temporaries (P, x = P ddS, P u, X = x u + P dPa);
  phase B: the 20 score products of tile t + 1 (written into the score
           registers phase A has finished reading) beside the second half
           (conversions to the input type, row sums);
so only one score set and one set of converted results are alive. LDS
fragments rotate through 16 AGPR slots and are read up to about 10 LDS
instructions ahead; the last fragments a step reads are the first ones the
next step needs. Each step begins by waiting for tile t + 1's LDS DMA,
the workgroup barrier and the DMA of tile t + 6 into the stage tile t - 2
left (an 8-stage ring).

Tile numbers are ring positions: the block's key tile j is ring tile t0 + j
(operand t0, less than 8), in stage (t0 + j) mod 8, and the operands nkt,
nfull, hi0 and rag count in those numbers (t0 + the block's tile count, and so
on; rag stays 0xffffffff without a ragged tail), klb in keys (its value plus
32 t0). A workgroup that sweeps several blocks starts each one where the
previous one left the ring, so it can issue the next block's first tiles
while waves still read the last stages of the current one.

Hazards. The statement is opaque to the compiler's hazard recognizer, so
the generated code keeps the distances the compiler itself inserts for
v_mfma_f32_32x32x16 on gfx950 (measured by compiling the patterns): a matrix
result is read by a vector instruction at least 12 wait states later (12
s_nop states are added where no barrier separates them), a vector result is
read by a matrix instruction at least 2 later, and no vector or LDS
instruction writes a register that a matrix instruction reads as its
accumulator input. The first LDS DMA of each tile follows `s_nop 4`, the
others `s_nop 0` after M0 is written (tests/test_dma_wait_states.py checks
the built library).

Usage: python gen_q32_loop.py [--check]   (--check: compare with the file on disk)
"""

from __future__ import annotations

import argparse
import pathlib
import sys

HERE = pathlib.Path(__file__).resolve().parent
OUT = HERE / "fhog_q32_loop.inc"

KTILE = 4096          # bytes of one 32 x 64 tile of a 2-byte type
STAGE = 4 * KTILE     # K, V, ddK, ddV
NST = 8               # ring stages
TOFF = {"K": 0, "V": KTILE, "dK": 2 * KTILE, "dV": 3 * KTILE}
LGKM_MAX = 15         # LDS instructions counted in flight (the counter's limit)
LGKM_RETIRE = 7       # a wait at that limit leaves this many in flight
MIN_LEAD = 6          # a fragment is read at least this many matrix instructions before its use
DS_AHEAD = 3          # the uniform read rate runs this many matrix instructions ahead
GAP_MAX = 3           # LDS reads issued in one gap between matrix instructions unless one is due
ADV_POS = 2           # steady step: DMA wait, barrier and DMA after this matrix instruction

# pinned registers
S0, DDS0, DP0, DPA0 = 0, 16, 32, 48          # score tiles (fp32, 16 each)
EP0, EX0, EU0, EXX0 = 64, 72, 80, 88        # converted results P, x, P u, X (2 halves x 4 regs)
TP0, TX0, TU0, TXX0 = 96, 112, 128, 144     # element-wise temporaries (16 each)
INITU = 160                                 # 16 x (-D): accumulator start of dP
ADDR_R = 176                                # 4: row fragments of the score tile, per 16-deep step
ADDR_TC = 180                               # 4: transposed fragments, tile t - 1 (a0, a1, b0, b1)
KLIM = 184                                  # masked steps: last visible key - 4 g, tile-relative
ADDR_TN = 185                               # 4: transposed fragments, tile t
NVGPR_PINNED = 189
FRAG0 = 192                                 # AGPR fragment slots a[192 + 4 k .. + 3], k < 16
# s100 and s101 are outside the compiler's allocatable set (it reserves them)
# and are not touched; m0 is saved in m0s and restored at the end.
SG = {"m0s": 89, "gptr": 90, "gstep": 92, "hi": 94, "t": 95, "k0": 96, "k1": 97, "k2": 98, "k3": 99}


def v(i):
    return f"v{i}"


def vr(i, n):
    return f"v[{i}:{i + n - 1}]"


def frag(k):
    return f"a[{FRAG0 + 4 * k}:{FRAG0 + 4 * k + 3}]"


def issue_cost(x):
    """Approximate issue cycles of an instruction at one wave per SIMD, as
    measured by looping instruction mixes: a wave-wide vector instruction
    about 5 (an exponential about 8.6), an LDS DMA about 10, s_nop n n + 1,
    a scalar instruction 1-4 (more in dependent chains). LDS reads are paced
    separately and waits and barriers cost what they wait for; both count 0.
    A matrix instruction leaves about 32 cycles for the others."""
    op = x.split()[0]
    if op.startswith("ds_read") or op in ("s_waitcnt", "s_barrier") or op.endswith(":"):
        return 0.0
    if op == "v_exp_f32":
        return 8.6
    if op.startswith("v_"):
        return 5.2
    if op.startswith("global_load"):
        return 10.0
    if op == "s_nop":
        return int(x.split()[1]) + 1.0
    if op.startswith("s_"):
        return 2.0
    return 0.0


class Frag:
    """An MFMA A operand read from LDS into fragment slot `slot`: one
    ds_read_b128 (row fragment) or two ds_read_b64_tr_b16 (transposed)."""

    def __init__(self, slot, reads):
        self.slot = slot
        self.reads = reads     # list of (instruction text)
        self.last_ds = None    # index of its last DS instruction once issued


class Sched:
    """Interleaves one block's matrix, vector, LDS and scalar instructions.

    Every fragment read has a release point (its slot's previous occupant has
    had its last matrix use emitted, and, for tiles another wave streams, the
    step's barrier has passed) and a deadline (its first matrix use less
    MIN_LEAD matrix instructions). Reads leave the queue in order at a
    uniform rate over the block's matrix instructions, earlier only when a
    deadline is near. Before a matrix instruction, s_waitcnt lgkmcnt makes
    its fragments resident. At most LGKM_MAX LDS reads are counted as in
    flight; beyond that one wait retires the oldest ones, issued many matrix
    instructions earlier, so every lgkmcnt value fits the counter. A block
    starts either with every read complete (start) or with the previous
    block's last PREF_KEEP reads in flight (Gen.start_after_prefetch)."""

    def __init__(self, out, n_mfma):
        self.out = out
        self.ds = 0             # DS instructions issued in this block
        self.done_upto = 0      # DS instructions known complete
        self.queue = []         # [frag, uses, not_before, deadline]
        self.pending_uses = {}  # slot -> remaining matrix uses of its current frag
        self.mi = 0             # matrix instructions emitted in this block
        self.n_mfma = max(1, n_mfma)
        self.ds_total = 0       # DS instructions enqueued in this block
        self.issued = 0         # of those, issued

    def emit(self, s):
        self.out.append(s)

    def start(self):
        self.emit("s_waitcnt lgkmcnt(0)")
        self.ds = 0
        self.done_upto = 0

    def enqueue(self, frags, uses, first_use, not_before=0):
        for f in frags:
            self.queue.append([f, uses[f], not_before, first_use[f] - MIN_LEAD])
            self.ds_total += len(f.reads)

    def _issue(self, f, nuses):
        for r in f.reads:
            if self.ds - self.done_upto >= LGKM_MAX:
                self.emit(f"s_waitcnt lgkmcnt({LGKM_RETIRE})")
                self.done_upto = self.ds - LGKM_RETIRE
            self.emit(r)
            self.ds += 1
            self.issued += 1
        f.last_ds = self.ds - 1
        self.pending_uses[f.slot] = nuses

    def issue_reads(self, greedy=False):
        """Issues reads from the queue head: those due by the uniform rate,
        or urgent ones, or (greedy) all whose slots are free."""
        want = -(-(self.mi + DS_AHEAD) * self.ds_total // self.n_mfma)
        n = 0
        while self.queue:
            f, nuses, nb, dl = self.queue[0]
            if self.pending_uses.get(f.slot, 0) > 0 or self.mi < nb:
                break
            if not greedy and dl > self.mi and (self.issued >= want or n >= GAP_MAX):
                break
            self.queue.pop(0)
            self._issue(f, nuses)
            n += len(f.reads)

    def wait_for(self, f):
        assert f.last_ds is not None, "fragment used before it was read"
        need = f.last_ds + 1
        if need > self.done_upto:
            self.emit(f"s_waitcnt lgkmcnt({self.ds - need})")
            self.done_upto = need

    def mfma(self, text, frags):
        for f in frags:
            self.wait_for(f)
        self.emit(text)
        for f in frags:
            self.pending_uses[f.slot] -= 1
        self.mi += 1

    def flush_reads(self):
        while self.queue:
            f, nuses, nb, dl = self.queue[0]
            if self.pending_uses.get(f.slot, 0) > 0:
                raise RuntimeError("flush: fragment slot still in use")
            self.queue.pop(0)
            self._issue(f, nuses)


class Gen:
    def __init__(self, dtype: str, pre: bool):
        self.dtype, self.pre = dtype, pre
        self.mfma_op = f"v_mfma_f32_32x32x16_{'bf16' if dtype == 'bf16' else 'f16'}"
        self.cvt = f"v_cvt_pk_{'bf16' if dtype == 'bf16' else 'f16'}_f32"
        self.out: list[str] = []
        self.uid = 0

    def lbl(self, name):
        return f"Lq32_{name}_%="

    def emit(self, s):
        self.out.append(s)

    # ----- fragments -----
    def row_frags(self):
        """Score-product A operands of one tile: per 16-deep step ks, the K, V,
        ddV, ddK row fragments (their first-use order), slots 0..15."""
        fr = {}
        k = 0
        for ks in range(4):
            for name in ("K", "V", "dV", "dK"):
                fr[(ks, name)] = Frag(k, [f"ds_read_b128 {frag(k)}, {v(ADDR_R + ks)} offset:{TOFF[name]}"])
                k += 1
        return fr

    def tr_frags(self, addr0):
        """Output-product A operands of one tile: per (column block dt, key
        half s) the ddK, K, ddV, V fragments read transposed, slots 0..15."""
        fr = {}
        k = 0
        for dt in range(2):
            for s in range(2):
                for name in ("dK", "K", "dV", "V"):
                    off = TOFF[name] + 2048 * s
                    a, b = v(addr0 + dt), v(addr0 + 2 + dt)
                    fr[(dt, s, name)] = Frag(k, [
                        f"ds_read_b64_tr_b16 a[{FRAG0 + 4 * k}:{FRAG0 + 4 * k + 1}], {a} offset:{off}",
                        f"ds_read_b64_tr_b16 a[{FRAG0 + 4 * k + 2}:{FRAG0 + 4 * k + 3}], {b} offset:{off + 1024}"])
                    k += 1
        return fr

    # ----- matrix instruction lists -----
    def score_mfmas(self, fr):
        """(text, frags) of tile's 20 score products in issue order."""
        m = []
        op = self.mfma_op
        for ks in range(4):
            K, V, dV, dK = fr[(ks, "K")], fr[(ks, "V")], fr[(ks, "dV")], fr[(ks, "dK")]
            q, dq, do = f"%[q{ks}]", f"%[dq{ks}]", f"%[do{ks}]"
            c = lambda base, init: vr(base, 16) if ks else init
            m.append((f"{op} {vr(S0, 16)}, {frag(K.slot)}, {q}, {c(S0, '0')}", [K]))
            m.append((f"{op} {vr(DDS0, 16)}, {frag(K.slot)}, {dq}, {c(DDS0, '0')}", [K]))
            m.append((f"{op} {vr(DP0, 16)}, {frag(V.slot)}, {do}, {c(DP0, vr(INITU, 16))}", [V]))
            m.append((f"{op} {vr(DPA0, 16)}, {frag(dV.slot)}, {do}, {c(DPA0, '0')}", [dV]))
            m.append((f"{op} {vr(DDS0, 16)}, {frag(dK.slot)}, {q}, {vr(DDS0, 16)}", [dK]))
        return m

    def output_mfmas(self, fr):
        """(text, frags) of a tile's 26 output products in issue order."""
        m = []
        op = self.mfma_op
        for dt in range(2):
            for s in range(2):
                dK, K, dV, V = (fr[(dt, s, n)] for n in ("dK", "K", "dV", "V"))
                Eu, EX, EP, Ex = (vr(b + 4 * s, 4) for b in (EU0, EXX0, EP0, EX0))
                m.append((f"{op} %[aa{dt}], {frag(dK.slot)}, {Eu}, %[aa{dt}]", [dK]))
                m.append((f"{op} %[as{dt}], {frag(K.slot)}, {Eu}, %[as{dt}]", [K]))
                m.append((f"{op} %[aa{dt}], {frag(K.slot)}, {EX}, %[aa{dt}]", [K]))
                m.append((f"{op} %[ap{dt}], {frag(K.slot)}, {EP}, %[ap{dt}]", [K]))
                m.append((f"{op} %[ao{dt}], {frag(dV.slot)}, {EP}, %[ao{dt}]", [dV]))
                m.append((f"{op} %[ao{dt}], {frag(V.slot)}, {Ex}, %[ao{dt}]", [V]))
                if dt == 0:
                    # every row of ddm accumulates the column sums of x rounded to T
                    m.append((f"{op} %[ddm], %[ones], {Ex}, %[ddm]", []))
        return m

    @staticmethod
    def first_tr(fr):
        """The first eight transposed fragments in use order (column block 0)."""
        return [fr[(0, s, n)] for s in range(2) for n in ("dK", "K", "dV", "V")]

    @staticmethod
    def rest_tr(fr):
        return [fr[(1, s, n)] for s in range(2) for n in ("dK", "K", "dV", "V")]

    @staticmethod
    def uses(mfmas):
        u = {}
        for _, fs in mfmas:
            for f in fs:
                u[f] = u.get(f, 0) + 1
        return u

    # ----- element-wise step -----
    def e1(self, masked):
        """First half of the element-wise step: reads the four score tiles."""
        ops = []
        for b in range(4):
            rs = range(4 * b, 4 * b + 4)
            for r in rs:
                ops.append(f"v_fma_f32 {v(TP0 + r)}, {v(S0 + r)}, %[c2], %[nl2]")
            for r in rs:
                ops.append(f"v_exp_f32 {v(TP0 + r)}, {v(TP0 + r)}")
            if not self.pre:
                for r in rs:
                    ops.append(f"v_mul_f32 {v(TX0 + r)}, %[scl], {v(DDS0 + r)}")
            if masked:
                for r in rs:
                    const = 8 * (r // 4) + r % 4  # tile key 8 (r / 4) + 4 g + r % 4, less 4 g
                    ops.append((f"v_cmp_gt_i32 vcc, {const}, {v(KLIM)}",
                                f"v_cndmask_b32_e64 {v(TP0 + r)}, {v(TP0 + r)}, 0, vcc"))
            for r in rs:
                src = v(DDS0 + r) if self.pre else v(TX0 + r)
                ops.append(f"v_mul_f32 {v(TX0 + r)}, {v(TP0 + r)}, {src}")       # x = P ddS
            for r in rs:
                ops.append(f"v_mul_f32 {v(TU0 + r)}, {v(TP0 + r)}, {v(DP0 + r)}")   # P u
            for r in rs:
                ops.append(f"v_mul_f32 {v(TXX0 + r)}, {v(TP0 + r)}, {v(DPA0 + r)}")  # P dPa
            for r in rs:
                ops.append(f"v_fmac_f32 {v(TXX0 + r)}, {v(TX0 + r)}, {v(DP0 + r)}")  # X = x u + P dPa
        return ops

    def e2(self):
        """Second half: conversions of P, x, P u, X to the input type and the
        fp32 row sums (dD, sum X, sum P u)."""
        ops = []
        for s in range(2):
            for k in range(4):
                r0, r1 = 8 * s + 2 * k, 8 * s + 2 * k + 1
                ops.append(f"{self.cvt} {v(EP0 + 4 * s + k)}, {v(TP0 + r0)}, {v(TP0 + r1)}")
                ops.append(f"{self.cvt} {v(EX0 + 4 * s + k)}, {v(TX0 + r0)}, {v(TX0 + r1)}")
                ops.append(f"{self.cvt} {v(EU0 + 4 * s + k)}, {v(TU0 + r0)}, {v(TU0 + r1)}")
                ops.append(f"{self.cvt} {v(EXX0 + 4 * s + k)}, {v(TXX0 + r0)}, {v(TXX0 + r1)}")
                for r in (r0, r1):
                    ops.append(f"v_add_f32 %[dd], %[dd], {v(TX0 + r)}")
                    ops.append(f"v_add_f32 %[xs], %[xs], {v(TXX0 + r)}")
                    ops.append(f"v_add_f32 %[pu], %[pu], {v(TU0 + r)}")
        return ops

    # ----- SALU pieces -----
    def stage_addr(self, dst_sgpr, tile_expr_sgpr, delta):
        """dst = lds_kv + ((tile + delta) & 7) * STAGE."""
        k = f"s{dst_sgpr}"
        self.emit(f"s_add_u32 {k}, s{tile_expr_sgpr}, {delta & 0xffffffff}" if delta >= 0 else
                  f"s_sub_u32 {k}, s{tile_expr_sgpr}, {-delta}")
        self.emit(f"s_and_b32 {k}, {k}, {NST - 1}")
        self.emit(f"s_lshl_b32 {k}, {k}, 14")
        self.emit(f"s_add_u32 {k}, {k}, %[ldskv]")

    def advance(self, need_delta, name):
        """Wait for tile t + need_delta (own LDS DMAs), barrier, then DMA the
        next tile (hi + 1) if there is one."""
        t, hi, k0, k1 = SG["t"], SG["hi"], SG["k0"], SG["k1"]
        L = lambda x: self.lbl(f"{name}_{x}")
        self.emit(f"s_add_u32 s{k0}, s{t}, {need_delta}")
        self.emit(f"s_sub_u32 s{k0}, s{hi}, s{k0}")          # tiles issued after the one needed
        for n in (4, 3, 2, 1):
            self.emit(f"s_cmp_{'ge' if n == 4 else 'eq'}_u32 s{k0}, {n}")
            self.emit(f"s_cbranch_scc1 {L(f'w{n}')}")
        self.emit("s_waitcnt vmcnt(0)")
        self.emit(f"s_branch {L('wd')}")
        for n in (1, 2, 3):
            self.emit(f"{L(f'w{n}')}:")
            self.emit(f"s_waitcnt vmcnt({4 * n})")
            self.emit(f"s_branch {L('wd')}")
        self.emit(f"{L('w4')}:")
        self.emit("s_waitcnt vmcnt(16)")
        self.emit(f"{L('wd')}:")
        self.emit("s_barrier")
        # DMA of tile hi + 1 into stage (hi + 1) mod 8
        self.emit(f"s_add_u32 s{k0}, s{hi}, 1")
        self.emit(f"s_cmp_lt_u32 s{k0}, %[nkt]")
        self.emit(f"s_cbranch_scc0 {L('ni')}")
        self.emit(f"s_mov_b32 s{hi}, s{k0}")
        self.emit(f"s_and_b32 s{k1}, s{k0}, {NST - 1}")
        self.emit(f"s_lshl_b32 s{k1}, s{k1}, 14")
        self.emit(f"s_cmp_eq_u32 s{k0}, %[rag]")
        self.emit(f"s_cbranch_scc1 {L('part')}")
        for which, lab in (("vo", None), ("vp", "part")):
            if lab:
                self.emit(f"{L(lab)}:")
            self.emit(f"s_add_u32 m0, s{k1}, %[ldsw]")
            for i in range(4):
                if i:
                    self.emit("s_add_u32 m0, m0, 0x400")
                self.emit("s_nop 4" if i == 0 else "s_nop 0")
                self.emit(f"global_load_lds_dwordx4 %[{which}{i}], s[{SG['gptr']}:{SG['gptr'] + 1}]")
            if not lab:
                self.emit(f"s_branch {L('adv')}")
        self.emit(f"{L('adv')}:")
        self.emit(f"s_add_u32 s{SG['gptr']}, s{SG['gptr']}, s{SG['gstep']}")
        self.emit(f"s_addc_u32 s{SG['gptr'] + 1}, s{SG['gptr'] + 1}, s{SG['gstep'] + 1}")
        self.emit(f"{L('ni')}:")

    def advance_steady(self):
        """advance(1) where tiles t + 2 .. t + 5 are in flight and tile t + 6
        exists and is not the ragged tail (t + 7 < nkt): no branches."""
        hi, k1 = SG["hi"], SG["k1"]
        self.emit("s_waitcnt vmcnt(16)")
        self.emit("s_barrier")
        self.emit(f"s_add_u32 s{hi}, s{hi}, 1")
        self.emit(f"s_and_b32 s{k1}, s{hi}, {NST - 1}")
        self.emit(f"s_lshl_b32 s{k1}, s{k1}, 14")
        self.emit(f"s_add_u32 m0, s{k1}, %[ldsw]")
        for i in range(4):
            if i:
                self.emit("s_add_u32 m0, m0, 0x400")
            self.emit("s_nop 4" if i == 0 else "s_nop 0")
            self.emit(f"global_load_lds_dwordx4 %[vo{i}], s[{SG['gptr']}:{SG['gptr'] + 1}]")
        self.emit(f"s_add_u32 s{SG['gptr']}, s{SG['gptr']}, s{SG['gstep']}")
        self.emit(f"s_addc_u32 s{SG['gptr'] + 1}, s{SG['gptr'] + 1}, s{SG['gstep'] + 1}")

    def addr_rows(self, delta):
        """ADDR_R[ks] = stage(t + delta) + row offset of step ks."""
        self.stage_addr(SG["k2"], SG["t"], delta)
        return [f"v_add_u32 {v(ADDR_R + ks)}, s{SG['k2']}, %[ro{ks}]" for ks in range(4)]

    def addr_tr(self, base, delta, sg):
        """base[0..3] = stage(t + delta) + transposed offsets a0, a1, b0, b1."""
        self.stage_addr(sg, SG["t"], delta)
        return [f"v_add_u32 {v(base + i)}, s{sg}, %[{n}]" for i, n in enumerate(("ta0", "ta1", "tb0", "tb1"))]

    def klim(self):
        """KLIM = klim base - 32 t (masked steps)."""
        self.emit(f"s_lshl_b32 s{SG['k3']}, s{SG['t']}, 5")
        return [f"v_subrev_u32 {v(KLIM)}, s{SG['k3']}, %[klb]"]

    # ----- phases -----
    def phase(self, sch, mfmas, valu, side=None):
        """Issues mfmas with the vector ops between them and LDS reads paced
        by the scheduler. side maps a matrix instruction's index in this phase
        (-1: before the first) to instructions emitted right after it. The
        vector ops keep their order and fill the gaps so that each gap's
        issue cost (issue_cost: its side instructions and vector ops) is about
        the phase's average: a gap that holds the DMAs or an address chain
        takes fewer vector ops."""
        side = side or {}
        groups = [list(op) if isinstance(op, tuple) else [op] for op in valu]
        for x in side.get(-1, []):
            sch.emit(x)
        n = len(mfmas)
        if n == 0:
            sch.issue_reads(greedy=True)
            for gi, g in enumerate(groups):
                for x in g:
                    sch.emit(x)
                if gi % 3 == 2:
                    sch.issue_reads(greedy=True)
            sch.issue_reads(greedy=True)
            return
        sch.issue_reads()
        gi = 0
        gcost = [sum(issue_cost(x) for x in g) for g in groups]
        scost = [sum(issue_cost(x) for x in side.get(i, [])) for i in range(n)]
        placed = sum(issue_cost(x) for x in side.get(-1, []))  # falls in the first gap
        total = placed + sum(gcost) + sum(scost)
        for i, (text, frags) in enumerate(mfmas):
            sch.mfma(text, frags)
            for x in side.get(i, []):
                sch.emit(x)
            placed += scost[i]
            goal = (i + 1) * total / n
            target = gi
            while target < len(groups) and (i == n - 1 or placed + gcost[target] / 2 <= goal):
                placed += gcost[target]
                target += 1
            # the gap's LDS reads first: their data returns while its vector
            # ops issue (reads after half or all of them: 6 % slower steps)
            sch.issue_reads()
            while gi < target:
                for x in groups[gi]:
                    sch.emit(x)
                gi += 1
        assert gi == len(groups)

    @staticmethod
    def first_use(mfmas, offset=0):
        fu = {}
        for i, (_, fs) in enumerate(mfmas):
            for f in fs:
                fu.setdefault(f, offset + i)
        return fu

    # Block boundaries. Every block that is followed by a step ends having
    # read the next step's first eight transposed fragments (groups (0, 0)
    # and (0, 1), 16 LDS reads) and waits until at most the last PREF_KEEP of
    # its reads are in flight: the first four fragments have landed, the
    # next four may not have. The following block starts from that state.
    PREF_KEEP = 8

    def start_after_prefetch(self, sch, tf, mf_o):
        """Block start after a prefetching block: fragments 0..3 resident,
        4..7 (the last PREF_KEEP LDS reads) possibly in flight."""
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

    def next_step_frags(self, sch, n_block, not_before):
        """Queues the next step's first transposed fragments (tile t, through
        ADDR_TC as recomputed in this block)."""
        tf_next = self.tr_frags(ADDR_TC)
        mf_next = self.output_mfmas(tf_next)
        sch.enqueue(self.first_tr(tf_next), self.uses(mf_next), self.first_use(mf_next, n_block), not_before)

    def addr_tr_ops(self, delta, sg, base=ADDR_TC):
        """SALU + VALU computing base[0..3] = stage(t + delta) + transposed offsets."""
        ops = [f"s_add_u32 s{sg}, s{SG['t']}, {delta}" if delta >= 0 else f"s_sub_u32 s{sg}, s{SG['t']}, {-delta}",
               f"s_and_b32 s{sg}, s{sg}, {NST - 1}", f"s_lshl_b32 s{sg}, s{sg}, 14", f"s_add_u32 s{sg}, s{sg}, %[ldskv]"]
        ops += [f"v_add_u32 {v(base + i)}, s{sg}, %[{n}]" for i, n in enumerate(("ta0", "ta1", "tb0", "tb1"))]
        return ops

    def addr_row_ops(self, delta, sg):
        ops = [f"s_add_u32 s{sg}, s{SG['t']}, {delta}", f"s_and_b32 s{sg}, s{sg}, {NST - 1}",
               f"s_lshl_b32 s{sg}, s{sg}, 14", f"s_add_u32 s{sg}, s{sg}, %[ldskv]"]
        ops += [f"v_add_u32 {v(ADDR_R + ks)}, s{sg}, %[ro{ks}]" for ks in range(4)]
        return ops

    def klim_ops(self):
        return [f"s_lshl_b32 s{SG['k3']}, s{SG['t']}, 5", f"v_subrev_u32 {v(KLIM)}, s{SG['k3']}, %[klb]"]

    # ----- blocks -----
    def block_prologue(self):
        """Pinned SGPR state, the -D start tuple, tile 0's DMA wait and its
        score products."""
        for r in range(16):
            self.emit(f"v_mov_b32 {v(INITU + r)}, %[nd]")
        self.emit(f"s_mov_b32 s{SG['m0s']}, m0")
        self.emit(f"s_mov_b64 s[{SG['gptr']}:{SG['gptr'] + 1}], %[gptr]")
        self.emit(f"s_mov_b64 s[{SG['gstep']}:{SG['gstep'] + 1}], %[gstep]")
        self.emit(f"s_mov_b32 s{SG['hi']}, %[hi0]")
        self.emit(f"s_mov_b32 s{SG['t']}, %[t0]")
        self.advance(0, "pro")
        for x in self.addr_row_ops(0, SG["k2"]):
            self.emit(x)
        rf = self.row_frags()
        mf = self.score_mfmas(rf)
        sch = Sched(self.out, len(mf))
        sch.start()
        sch.enqueue([rf[(ks, n)] for ks in range(4) for n in ("K", "V", "dV", "dK")], self.uses(mf), self.first_use(mf))
        self.phase(sch, mf, [])
        sch.flush_reads()
        self.emit("s_waitcnt lgkmcnt(0)")

    def block_first(self, masked):
        """t = 0: element-wise step of tile 0, score products of tile 1; reads
        tile 0's first transposed fragments for step 1."""
        self.advance(1, f"first{int(masked)}")
        for x in self.addr_row_ops(1, SG["k2"]) + self.addr_tr_ops(0, SG["k1"]) + (self.klim_ops() if masked else []):
            self.emit(x)
        rf = self.row_frags()
        mf_s = self.score_mfmas(rf)
        sch = Sched(self.out, len(mf_s))
        sch.start()
        sch.enqueue([rf[(ks, n)] for ks in range(4) for n in ("K", "V", "dV", "dK")], self.uses(mf_s), self.first_use(mf_s))
        self.phase(sch, [], self.e1(masked))
        self.next_step_frags(sch, len(mf_s), 0)
        self.phase(sch, mf_s, self.e2())
        self.end_with_prefetch(sch)

    def block_mid(self, masked, steady=False):
        """Step t: output products of tile t - 1 beside the element-wise step's
        first half (tile t); score products of tile t + 1 beside its second
        half. The steady form (t + 7 < nkt, unmasked) places the DMA wait,
        barrier and DMA after its third matrix instruction, so that the
        matrix unit works through them."""
        tf = self.tr_frags(ADDR_TC)
        mf_o = self.output_mfmas(tf)
        rf = self.row_frags()
        mf_s = self.score_mfmas(rf)
        n_blk = len(mf_o) + len(mf_s)
        side_a = {}
        if steady:
            adv = []
            saved = self.out
            self.out = adv
            self.advance_steady()
            self.out = saved
            # wait + barrier + M0 set-up, then the DMAs two per matrix
            # instruction, then the row addresses of tile t + 1
            cut = [i for i, x in enumerate(adv) if x.startswith("global_load_lds")]
            side_a[ADV_POS] = adv[:cut[0] + 1]
            side_a[ADV_POS + 1] = adv[cut[0] + 1:cut[2] + 1]
            side_a[ADV_POS + 2] = adv[cut[2] + 1:] + self.addr_row_ops(1, SG["k2"])
            s_nb = ADV_POS + 3
        else:
            self.advance(1, f"mid{int(masked)}")
            for x in self.addr_row_ops(1, SG["k2"]) + (self.klim_ops() if masked else []):
                self.emit(x)
            s_nb = 0
        sch = Sched(self.out, n_blk)
        self.start_after_prefetch(sch, tf, mf_o)
        fu = self.first_use(mf_o + mf_s)
        sch.enqueue(self.rest_tr(tf), self.uses(mf_o), fu)
        sch.enqueue([rf[(ks, n)] for ks in range(4) for n in ("K", "V", "dV", "dK")], self.uses(mf_s), fu, s_nb)
        self.phase(sch, mf_o, self.e1(masked), side_a)
        # every read through the old transposed addresses has been issued
        assert all(e[0] not in self.rest_tr(tf) for e in sch.queue)
        # tile t's transposed addresses after the first score product (the gap
        # before it holds phase A's last vector ops); the next step's reads
        # through them are queued from there on
        side_b = {0: self.addr_tr_ops(0, SG["k1"])}
        self.next_step_frags(sch, n_blk, len(mf_o) + 1)
        self.phase(sch, mf_s, self.e2(), side_b)
        self.end_with_prefetch(sch)
        self.emit(f"s_add_u32 s{SG['t']}, s{SG['t']}, 1")

    def block_last(self, masked, single=False):
        """t = nkt - 1: output products of tile t - 1 (none when single) beside
        the element-wise step of tile t, then tile t's output products."""
        self.emit("s_nop 7")  # a matrix result (the last score products) is read next
        self.emit("s_nop 7")
        for x in self.addr_tr_ops(0, SG["k1"], ADDR_TN) + (self.klim_ops() if masked else []):
            self.emit(x)
        tn = self.tr_frags(ADDR_TN)
        mf_n = self.output_mfmas(tn)
        if not single:
            tf = self.tr_frags(ADDR_TC)
            mf_o = self.output_mfmas(tf)
            sch = Sched(self.out, len(mf_o) + len(mf_n))
            self.start_after_prefetch(sch, tf, mf_o)
            fu = self.first_use(mf_o + mf_n)
            sch.enqueue(self.rest_tr(tf), self.uses(mf_o), fu)
            sch.enqueue(self.first_tr(tn) + self.rest_tr(tn), self.uses(mf_n), fu)
            self.phase(sch, mf_o, self.e1(masked))
        else:
            sch = Sched(self.out, len(mf_n))
            sch.start()
            sch.enqueue(self.first_tr(tn) + self.rest_tr(tn), self.uses(mf_n), self.first_use(mf_n))
            self.phase(sch, [], self.e1(masked))
        self.phase(sch, [], self.e2())
        self.emit("s_nop 1")  # the last conversions are read by the first matrix instructions below
        self.phase(sch, mf_n, [])
        sch.flush_reads()

    def generate(self):
        out = self.out
        L = self.lbl
        self.block_prologue()
        self.emit(f"s_add_u32 s{SG['k0']}, s{SG['t']}, 1")
        self.emit(f"s_cmp_eq_u32 %[nkt], s{SG['k0']}")
        self.emit(f"s_cbranch_scc1 {L('single_sel')}")
        self.emit(f"s_cmp_eq_u32 %[nfull], s{SG['t']}")
        self.emit(f"s_cbranch_scc1 {L('first_m')}")
        self.block_first(masked=False)
        self.emit(f"s_add_u32 s{SG['t']}, s{SG['t']}, 1")
        self.emit(f"s_branch {L('loop')}")
        self.emit(f"{L('first_m')}:")
        self.block_first(masked=True)
        self.emit(f"s_add_u32 s{SG['t']}, s{SG['t']}, 1")
        self.emit(f"{L('loop')}:")
        self.emit(f"s_add_u32 s{SG['k0']}, s{SG['t']}, 1")
        self.emit(f"s_cmp_ge_u32 s{SG['k0']}, %[nkt]")
        self.emit(f"s_cbranch_scc1 {L('last_sel')}")
        self.emit(f"s_cmp_ge_u32 s{SG['t']}, %[nfull]")
        self.emit(f"s_cbranch_scc1 {L('mid_m')}")
        self.emit(f"s_add_u32 s{SG['k0']}, s{SG['t']}, 7")
        self.emit(f"s_cmp_lt_u32 s{SG['k0']}, %[nkt]")
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
        self.emit(f"s_cmp_ge_u32 s{SG['t']}, %[nfull]")
        self.emit(f"s_cbranch_scc1 {L('last_m')}")
        self.block_last(masked=False)
        self.emit(f"s_branch {L('end')}")
        self.emit(f"{L('last_m')}:")
        self.block_last(masked=True)
        self.emit(f"s_branch {L('end')}")
        self.emit(f"{L('single_sel')}:")
        self.emit(f"s_cmp_eq_u32 %[nfull], s{SG['t']}")
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
        return out


VARIANTS = (("BF16_PRE", "bf16", True), ("BF16", "bf16", False), ("F16", "f16", False))


def render() -> str:
    lines = [
        "// Generated by gen_q32_loop.py; do not edit. The key sweep of",
        "// bwdbwd_q32_kernel (fhog_bwdbwd_q32.hip) as inline assembly, one string",
        "// per variant; operands and pinned registers are described there.",
        "#pragma once",
        "",
        f"#define FHOG_Q32_NVGPR_PINNED {NVGPR_PINNED}",
        f"#define FHOG_Q32_FRAG_AGPR0 {FRAG0}",
        "",
        "// registers the statements use beyond their operands",
        "#define FHOG_Q32_CLOBBERS \\",
    ]
    clob = [f'"v{i}"' for i in range(NVGPR_PINNED)] + [f'"a{i}"' for i in range(FRAG0, 256)]
    clob += [f'"s{i}"' for i in range(min(SG.values()), max(SG.values()) + 1)]
    clob += ['"vcc"', '"scc"', '"memory"']
    for i in range(0, len(clob), 12):
        lines.append("  " + ", ".join(clob[i:i + 12]) + ("," if i + 12 < len(clob) else "") + " \\")
    lines.append("")
    lines.append("")
    for name, dtype, pre in VARIANTS:
        body = Gen(dtype, pre).generate()
        lines.append(f"#define FHOG_Q32_LOOP_{name} \\")
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

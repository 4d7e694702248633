"""The generated sweeps issue each gap's LDS reads before its element-wise work.

Between two matrix instructions of a steady step (a gap) the generators emit
the gap's side instructions (DMA, barrier, address updates), then the paced
LDS fragment reads, then the gap's share of the element-wise step. With the
reads first their data returns while the vector work issues: the looped
stage-1 step went from 1974 to 1848 cycles, and the kernels took 2 % (stage
1, first backward) to 5 % (one-wave stage 2) less time with the same results.
This test keeps that order in every variant's steady step. CPU only.
"""

from __future__ import annotations

import importlib.util
import pathlib
import sys

import pytest

CSRC = pathlib.Path(__file__).resolve().parent.parent / "flash-hog_amd" / "csrc"
sys.path.insert(0, str(CSRC))


def _load(name):
    spec = importlib.util.spec_from_file_location(name, CSRC / f"{name}.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


Q32, K32, BK64, BQ64 = (_load(n) for n in ("gen_q32_loop", "gen_k32_loop", "gen_bwd_k64_loop", "gen_bwd_q64_loop"))

VARIANTS = {
    "q32 bf16 folded scale": lambda: Q32.Gen("bf16", True).generate(),
    "q32 bf16": lambda: Q32.Gen("bf16", False).generate(),
    "q32 fp16": lambda: Q32.Gen("f16", False).generate(),
    "k32 folded scale": lambda: K32.K32(True).generate(),
    "k32": lambda: K32.K32(False).generate(),
    "k64 bf16": lambda: BK64.BK64("bf16").generate(),
    "k64 fp16": lambda: BK64.BK64("f16").generate(),
    "q64 bf16": lambda: BQ64.BQ64("bf16").generate(),
    "q64 fp16": lambda: BQ64.BQ64("f16").generate(),
}

# vector instructions of the element-wise step (address arithmetic such as
# v_add_u32 belongs to the side instructions and may precede the reads)
ELEMENT = ("v_fma_f32", "v_fmac_f32", "v_mul_f32", "v_exp_f32", "v_cvt_pk", "v_add_f32", "v_sub_f32",
           "v_min_f32", "v_cndmask", "v_dot2")


def steady_step(prog):
    """The instructions of the steady (branch-free) middle step: from its
    label to the branch back to the loop head."""
    start = next(i for i, x in enumerate(prog) if x.endswith("mid_s_%=:")) + 1
    end = next(i for i in range(start, len(prog))
               if prog[i].startswith("s_branch") and prog[i].endswith("_loop_%="))
    return prog[start:end]


def gaps(step):
    out = [[]]
    for ins in step:
        if ins.split()[0].startswith("v_mfma"):
            out.append([])
        else:
            out[-1].append(ins)
    return out


def interleaved_reads(gap):
    """LDS reads of a gap that sit between two of its element-wise
    instructions (a read before all of them, or after all of them where a
    gap also holds the next phase's first reads, is in order)."""
    elem = [i for i, ins in enumerate(gap) if ins.split()[0].startswith(ELEMENT)]
    if not elem:
        return []
    return [ins for ins in gap[elem[0]:elem[-1]] if ins.startswith("ds_read")]


@pytest.mark.parametrize("name", sorted(VARIANTS))
def test_reads_precede_element_work_in_every_gap(name):
    step = steady_step(VARIANTS[name]())
    g = gaps(step)
    assert len(g) > 20, "steady step not found"
    assert sum(x.startswith("ds_read") for x in step) > 0
    for k, gap in enumerate(g):
        assert not interleaved_reads(gap), f"{name}, gap {k}: LDS reads inside the element-wise work: {interleaved_reads(gap)}"


def test_an_interleaved_gap_is_caught():
    """The check itself: half the vector work, then the reads, then the rest
    (the order the generators had before) fails; reads first passes."""
    half = ["v_mul_f32 v1, v2, v3", "ds_read_b128 a[4:7], v9", "v_mul_f32 v4, v2, v3"]
    first = ["ds_read_b128 a[4:7], v9", "v_mul_f32 v1, v2, v3", "v_mul_f32 v4, v2, v3"]
    assert interleaved_reads(half) == ["ds_read_b128 a[4:7], v9"]
    assert interleaved_reads(first) == []

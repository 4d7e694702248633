"""The LDS DMA statements of the built library keep their manual wait states.

The kernels issue global_load_lds_* as inline assembly, which the compiler's
hazard check does not look inside. Two hazards then need explicit wait
states, which fhog_device.h puts in each statement as an s_nop:
  - an SALU write of M0 (the LDS destination) before an LDS DMA: 1 state;
  - a VALU write of an SGPR (v_readlane, as when the compiler reloads a
    spilled SGPR) before a vector-memory instruction that reads that SGPR
    (the scalar base of the DMA): 5 states.
A DMA whose base was read stale faulted the GPU now and then. This test
disassembles the gfx950 code objects of the library built here and checks that
every LDS DMA directly follows an s_nop (five wait states for a scalar base,
unless the DMA just before it used the same base), that no DMA with a
scalar base has a VALU write of that base within the five preceding wait
states (a straight-line scan), and that M0 is written by an SALU instruction
in the DMA's own block: the statement's single wait state covers only that
(a v_readfirstlane into M0 would need five). CPU only.
"""

from __future__ import annotations

import re
import shutil
import struct
import subprocess

import pytest

from flash_hog import _hip

OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _gfx950_code_objects(lib: bytes):
    """The gfx950 device code objects of every clang offload bundle in lib."""
    out = []
    for m in re.finditer(re.escape(MAGIC), lib):
        base = m.start()
        pos = base + len(MAGIC)
        (n,) = struct.unpack_from("<Q", lib, pos)
        pos += 8
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", lib, pos)
            pos += 24
            triple = lib[pos:pos + tlen].decode()
            pos += tlen
            if triple.endswith("gfx950"):
                out.append(lib[base + off:base + off + size])
    return out


LABEL = "<label>"


def _instructions(text: str):
    """(function, [mnemonic line or LABEL, ...]) for each function of an objdump
    listing; LABEL marks a branch target (a block another block may jump to)."""
    funcs, cur, name = [], [], None
    for line in text.splitlines():
        m = re.match(r"^[0-9a-f]+ <(\S+)>:", line)
        if m:
            if name is not None:
                funcs.append((name, cur))
            name, cur = m.group(1), []
            continue
        t = line.split("//")[0].strip()
        if name is None or not t:
            continue
        cur.append(LABEL if t.endswith(":") else t)
    if name is not None:
        funcs.append((name, cur))
    return funcs


def _sregs(tok: str) -> set[int]:
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"s(\d+)", tok)
    return {int(m.group(1))} if m else set()


@pytest.fixture(scope="module")
def listing(tmp_path_factory):
    if not shutil.which(OBJDUMP) and not shutil.os.path.exists(OBJDUMP):
        pytest.skip("llvm-objdump not available")
    path = _hip.library_path()
    if not path.exists():
        pytest.fail(f"{path} missing: run python flash-hog_amd/build.py")
    objs = _gfx950_code_objects(path.read_bytes())
    assert objs, "no gfx950 code object in the library"
    d = tmp_path_factory.mktemp("co")
    funcs = []
    for i, co in enumerate(objs):
        f = d / f"co{i}.o"
        f.write_bytes(co)
        text = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", str(f)], capture_output=True, text=True,
                              check=True).stdout
        funcs += _instructions(text)
    return funcs


def test_every_lds_dma_follows_its_wait_states(listing):
    seen = 0
    for name, ins in listing:
        for i, t in enumerate(ins):
            if not t.startswith("global_load_lds"):
                continue
            seen += 1
            ops = t.replace(",", " ").split()
            scalar_base = len(ops) > 2 and ops[2] != "off"
            prev = ins[i - 1].split() if i else []
            assert prev[:1] == ["s_nop"], (name, i, ins[i - 1], t)
            if scalar_base and int(prev[1], 0) < 4:
                # allowed only after an earlier DMA from the same base in the same
                # straight-line code (no branch target or branch in between)
                found = False
                for j in range(i - 2, max(-1, i - 64), -1):
                    b = ins[j].replace(",", " ").split()
                    if ins[j] == LABEL or b[0].startswith(("s_branch", "s_cbranch", "s_setpc")):
                        break
                    if b[0].startswith("global_load_lds") and b[2:3] == ops[2:3]:
                        found = True
                        break
                assert found, (name, i, ins[max(0, i - 8):i + 1])
    assert seen > 1000, seen


def test_no_dma_base_written_by_valu_within_five_states(listing):
    for name, ins in listing:
        for i, t in enumerate(ins):
            if not t.startswith("global_load_lds"):
                continue
            ops = t.replace(",", " ").split()
            base = _sregs(ops[2]) if len(ops) > 2 else set()
            if not base:
                continue
            states = 0
            for j in range(i - 1, max(-1, i - 32), -1):
                if ins[j] == LABEL:
                    # another block may jump here: only the wait states already counted hold
                    assert states >= 5, (name, i, t, states)
                    break
                op, *rest = ins[j].replace(",", " ").split()
                if op == "s_nop":
                    states += int(rest[0], 0) + 1
                    continue
                if rest and _sregs(rest[0]) & base:
                    assert not (op.startswith("v_") and states < 5), (name, i, ins[j], t, states)
                    break
                states += 1
                if states >= 5:
                    break


def test_m0_of_every_lds_dma_is_written_by_salu_in_its_block(listing):
    """The last write of M0 before each DMA is in the same straight-line code
    (no branch target in between) and is an SALU instruction."""
    seen = 0
    for name, ins in listing:
        for i, t in enumerate(ins):
            if not t.startswith("global_load_lds"):
                continue
            seen += 1
            writer = None
            for j in range(i - 1, -1, -1):
                if ins[j] == LABEL:
                    break
                op, *rest = ins[j].replace(",", " ").split()
                if rest and rest[0] == "m0":
                    writer = op
                    break
            assert writer is not None, (name, i, "M0 written in another block", ins[max(0, i - 8):i + 1])
            assert writer.startswith("s_"), (name, i, writer, t)
    assert seen > 1000, seen

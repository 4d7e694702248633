"""Build libflash_hog_hip.so (the C-ABI kernel library) for gfx950 with hipcc,
and the torch extension that calls it from C++ (_fhog_torch).

Usage: python flash-hog_amd/build.py [--jobs N] [--out DIR]

Each .hip source under csrc/ is compiled to an object in parallel, then the
objects are linked into flash_hog/_lib/libflash_hog_hip.so next to the Python
package that loads it. hipcc cross-compiles without a GPU. csrc/fhog_torch.cpp
is compiled with g++ against the installed torch's headers into
flash_hog/_lib/_fhog_torch<ext suffix>: tensor-level calls of the C ABI that
flash_hog/_hip.py prefers to its Python wrappers (less host time per call). It
links no kernel code; it calls the entry points of the library _hip.py loaded.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
LIB_DIR = HERE / "flash_hog" / "_lib"
LIB_NAME = "libflash_hog_hip.so"
ARCH = "gfx950"

# -packed-fp32-ops: hipcc may not emit v_pk_{add,mul,fma}_f32; ordinary scalar
# float code is compiled to unpacked VALU instructions.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]


# Extra flags for single sources. The double-backward kernels and the
# forward are scheduled for instruction-level parallelism rather than for
# occupancy (their occupancy is fixed by amdgpu_waves_per_eu anyway): the
# matrix instructions interleave better with the vector ones, and at
# B4 N2048 H16 D64 the double backward takes 0.314 instead of 0.323 ms
# (stage 1 180 -> 177 us, stage 2 146 -> 142 us), B1 N32768 H8 8.84 instead of
# 8.97 ms, B8 N1000 H12 fp16 0.263 instead of 0.266 ms; B2 N8192 H16 D128 is
# unchanged within noise. The first backward is not faster with it.
_MAX_ILP = ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]
SOURCE_FLAGS: dict[str, list[str]] = {
    "fhog_bwdbwd_fused.hip": _MAX_ILP,
    "fhog_bwdbwd_q32.hip": _MAX_ILP,
    "fhog_bwdbwd_k32.hip": _MAX_ILP,
    "fhog_bwd_k64.hip": _MAX_ILP,
    "fhog_bwd_q64.hip": _MAX_ILP,
    "fhog_bwdbwd.hip": _MAX_ILP,
    "fhog_bwdbwd_k16.hip": _MAX_ILP,
    "fhog_fwd.hip": _MAX_ILP,
}


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found (expected under /opt/rocm/bin)")
    return exe


def _compile(src: pathlib.Path, obj: pathlib.Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")


def build(jobs: int | None = None, out_dir: pathlib.Path | None = None) -> pathlib.Path:
    out_dir = pathlib.Path(out_dir) if out_dir else LIB_DIR
    obj_dir = HERE / "_build"
    obj_dir.mkdir(parents=True, exist_ok=True)
    out_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no .hip sources under {CSRC}")
    objs = [obj_dir / (s.stem + ".o") for s in sources]
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_compile, sources, objs))
    lib = out_dir / LIB_NAME
    tmp = out_dir / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, lib)
    return lib


TORCH_EXT_SRC = CSRC / "fhog_torch.cpp"
TORCH_EXT_NAME = "_fhog_torch"


def build_torch_ext(out_dir: pathlib.Path | None = None) -> pathlib.Path:
    """Compiles csrc/fhog_torch.cpp into a Python extension module for the
    installed torch (ROCm build) and this interpreter."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    out_dir = pathlib.Path(out_dir) if out_dir else LIB_DIR
    out_dir.mkdir(parents=True, exist_ok=True)
    lib_dirs = cpp_extension.library_paths()
    out = out_dir / (TORCH_EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_name(out.name + ".tmp")
    cmd = [
        shutil.which("g++") or "g++", "-O2", "-std=c++17", "-shared", "-fPIC",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        f"-DTORCH_EXTENSION_NAME={TORCH_EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
        *[f"-I{p}" for p in cpp_extension.include_paths()],
        f"-I{sysconfig.get_paths()['include']}", "-I/opt/rocm/include", f"-I{REPO / 'include'}",
        str(TORCH_EXT_SRC), "-o", str(tmp),
        *[f"-L{p}" for p in lib_dirs], *[f"-Wl,-rpath,{p}" for p in lib_dirs],
        "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
    ]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed for {TORCH_EXT_SRC.name}:\n{res.stderr}")
    os.replace(tmp, out)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--out", type=pathlib.Path, default=None)
    args = ap.parse_args(argv)
    with cf.ThreadPoolExecutor(max_workers=1) as ex:
        ext = ex.submit(build_torch_ext, args.out)
        lib = build(args.jobs, args.out)
        print(lib)
        print(ext.result())
    return 0


if __name__ == "__main__":
    sys.exit(main())

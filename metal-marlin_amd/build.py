"""Build libmmfp4.so (gfx950) in-tree: every csrc/*.hip -> object -> one shared
library next to the Python package (mmfp4/libmmfp4.so), plus the per-call torch
binding mmfp4/_mmfp4_torch.so (csrc/mm_pybind.cpp, host C++ linked to it) and
bench.py's measurement aids bench_aids/libmmfp4_bench.so (not part of the
GEMM library's ABI).

Usage: python metal-marlin_amd/build.py [-j N]
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "mmfp4" / "libmmfp4.so"
BIND_SRC = CSRC / "mm_pybind.cpp"
BIND = HERE / "mmfp4" / "_mmfp4_torch.so"
# Measurement aids for bench.py, kept out of the GEMM library's ABI.
AIDS_SRC = HERE / "bench_aids" / "mm_bench_aids.hip"
AIDS = HERE / "bench_aids" / "libmmfp4_bench.so"
ROOT = HERE.parent

ARCH = "gfx950"
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # Keep the compiler from forming packed-fp32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    f"-I{CSRC}", f"-I{ROOT / 'include'}",
]
# Per-file extra flags: the quantizers reproduce numpy's float32 arithmetic
# operation by operation, so no contraction there.
EXTRA = {"mm_quant.hip": ["-ffp-contract=off"], "mm_fp4flat.hip": ["-ffp-contract=off"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmmfp4.so)")


def _compile(cc: str, src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [cc, *COMMON, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stderr}")
    return obj


def build(jobs: int | None = None) -> Path:
    cc = hipcc()
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(jobs + 1) as ex:
        bind_obj = ex.submit(compile_binding)
        aids_obj = ex.submit(_compile, cc, AIDS_SRC)
        objs = list(ex.map(lambda s: _compile(cc, s), srcs))
        bind_obj = bind_obj.result()
        aids_obj = aids_obj.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, LIB)
    link_binding(bind_obj)
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-Bsymbolic", "-o",
           str(AIDS.with_suffix(".so.tmp")), str(aids_obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
    os.replace(AIDS.with_suffix(".so.tmp"), AIDS)
    return LIB


def _binding_flags() -> list[str]:
    import sysconfig

    import torch
    from torch.utils import cpp_extension
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    flags = ["-O2", "-std=c++17", "-fPIC", "-DTORCH_EXTENSION_NAME=_mmfp4_torch",
             f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-I{ROOT / 'include'}",
             f"-I{sysconfig.get_paths()['include']}"]
    return flags + [f"-I{p}" for p in cpp_extension.include_paths()]


def compile_binding() -> Path:
    """Object of the per-call torch binding (host C++ against torch's headers)."""
    obj = BUILD / "mm_pybind.o"
    cmd = ["g++", *_binding_flags(), "-c", str(BIND_SRC), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"binding compile failed: {' '.join(cmd)}\n{r.stderr[-4000:]}")
    return obj


def link_binding(obj: Path) -> Path:
    """_mmfp4_torch.so, linked to libmmfp4.so next to it."""
    from torch.utils import cpp_extension
    cmd = ["g++", "-shared", "-fPIC", str(obj), "-o", str(BIND.with_suffix(".so.tmp"))]
    cmd += [f"-L{p}" for p in cpp_extension.library_paths()]
    cmd += [f"-L{LIB.parent}", "-l:libmmfp4.so", "-Wl,-rpath,$ORIGIN",
            "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"binding link failed: {' '.join(cmd)}\n{r.stderr[-4000:]}")
    os.replace(BIND.with_suffix(".so.tmp"), BIND)
    return BIND


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    print(build(a.j))
    sys.exit(0)

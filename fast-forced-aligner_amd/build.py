"""Build the MI355X alignment libraries in place.

Produces, inside ``fast_forced_aligner/``:
  * ``libffa_hip.so``  - the HIP kernels and the C ABI of ``include/ffa.h``
    (hipcc, gfx950 only);
  * ``_ffa_torch.so``  - the PyTorch operators ``fast_forced_aligner_cuda::align``
    and ``::emission_validity`` on top of that ABI, plus the Python module
    ``_ffa_torch`` whose ``align`` the package calls (g++ against torch's headers).

Run ``python fast-forced-aligner_amd/build.py`` (or ``__graft_entry__.build()``).
hipcc cross-compiles for gfx950 without a GPU.
"""
from __future__ import annotations

import os
import shlex
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
OUT = PKG_ROOT / "fast_forced_aligner"
INCLUDE = REPO / "include"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

# -ffp-contract=off: the recurrence is one fp32 add per state and frame; no
# contraction may fuse it with anything (the reference builds with --fmad=false).
# Packed FP32 instructions are disabled for all device code.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(shlex.quote(c) for c in cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        sys.stderr.write(result.stdout + result.stderr)
        raise RuntimeError(f"build step failed: {cmd[0]} (exit {result.returncode})")


def build_hip(verbose: bool = False) -> Path:
    target = OUT / "libffa_hip.so"
    tmp = target.with_suffix(".so.tmp")
    _run([str(ROCM / "bin" / "hipcc"), *HIP_FLAGS, f"-I{INCLUDE}", str(CSRC / "ffa_kernels.hip"),
          "-o", str(tmp)], verbose)
    os.replace(tmp, target)
    return target


def build_torch(verbose: bool = False) -> Path:
    import torch
    from torch.utils import cpp_extension

    target = OUT / "_ffa_torch.so"
    tmp = target.with_suffix(".so.tmp")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    import sysconfig

    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w", "-fvisibility=hidden",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-I{INCLUDE}", f"-I{ROCM / 'include'}", f"-I{sysconfig.get_paths()['include']}"]
    cmd += [f"-I{p}" for p in cpp_extension.include_paths()]
    cmd += [str(CSRC / "ffa_torch.cpp"), "-o", str(tmp), f"-L{OUT}", "-lffa_hip"]
    for lib_dir in cpp_extension.library_paths():
        cmd += [f"-L{lib_dir}"]
    cmd += ["-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python", "-Wl,-rpath,$ORIGIN"]
    _run(cmd, verbose)
    os.replace(tmp, target)
    return target


def build(verbose: bool = False) -> None:
    OUT.mkdir(parents=True, exist_ok=True)
    build_hip(verbose)
    build_torch(verbose)


if __name__ == "__main__":
    build(verbose=True)

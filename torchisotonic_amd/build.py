"""Builds the package's two libraries in place.

    python -m torchisotonic_amd.build

``libtorchisotonic_amd.so``: every ``csrc/*.hip`` file compiled for gfx950 with hipcc (in
parallel) and linked; packed float32 instructions are switched off (``-packed-fp32-ops``) for
all device code. This is the C ABI of ``include/torchisotonic_amd.h``.

``libtorchisotonic_amd_ops.so``: ``csrc/ti_torch.cpp`` (host code only) compiled with g++
against torch's headers and linked to the first library: the ``torchisotonic_amd.isotonic_fit``
operator with its autograd node in C++.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libtorchisotonic_amd.so"
OPS_LIB = PKG / "libtorchisotonic_amd_ops.so"
INCLUDE = PKG.parent / "include"
OBJ = PKG / "_build"
ARCH = os.environ.get("TI_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build_ops(verbose: bool = True) -> Path:
    import torch
    from torch.utils import cpp_extension

    torch_lib = cpp_extension.library_paths()[0]
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *(f"-I{p}" for p in cpp_extension.include_paths()),
        "-I/opt/rocm/include", f"-I{INCLUDE}",
        str(CSRC / "ti_torch.cpp"),
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-lamdhip64",
        f"-L{PKG}", "-ltorchisotonic_amd",
        f"-Wl,-rpath,{torch_lib}", "-Wl,-rpath,$ORIGIN",
    ]
    tmp = OPS_LIB.with_suffix(".so.tmp")
    _run([*cmd, "-o", str(tmp)])
    tmp.replace(OPS_LIB)
    if verbose:
        print(f"built {OPS_LIB}")
    return OPS_LIB


def build(verbose: bool = True) -> Path:
    sources = sorted(CSRC.glob("*.hip"))
    OBJ.mkdir(exist_ok=True)
    objects = [OBJ / (s.stem + ".o") for s in sources]
    cmds = [[HIPCC, *FLAGS, "-c", str(s), "-o", str(o)] for s, o in zip(sources, objects)]
    with ThreadPoolExecutor(max_workers=min(8, len(cmds))) as pool:
        list(pool.map(_run, cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)])
    tmp.replace(LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    build_ops(verbose)
    return LIB


if __name__ == "__main__":
    build()

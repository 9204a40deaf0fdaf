"""Builds libtorchisotonic_amd.so in place, for gfx950, with hipcc.

    python -m torchisotonic_amd.build

Every ``csrc/*.hip`` file is compiled to an object (in parallel) and linked into
``torchisotonic_amd/libtorchisotonic_amd.so``. Packed float32 instructions are switched off
(``-packed-fp32-ops``) for all device code.
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
    return LIB


if __name__ == "__main__":
    build()

"""Build the gfx950 C-ABI library ``kernelfuser_amd/_lib/libkfmi.so`` in-tree.

``python -m kernelfuser_amd.build`` compiles every ``csrc/*.hip`` file with
hipcc for gfx950 (one process per file), then links the shared library.  The
library only needs the HIP runtime; it has no libtorch dependency, so it works
with whichever HIP runtime torch has already loaded (same soname).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIBDIR = PKG / "_lib"
LIB = LIBDIR / "libkfmi.so"
ARCH = "gfx950"

# Packed-FP32 instructions are disabled for all device code (hipcc's host pass
# warns that it does not know the feature; that warning is harmless).
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-I", str(INCLUDE), "-I", str(CSRC),
          "-Wall", "-Wno-unused-function"]


# Per-file flags.  attention.hip: no NaN inputs reach its max reductions
# (masked scores are -inf, not NaN), and without NaN semantics fmaxf needs no
# canonicalising instructions, so max trees map onto v_max3_f32.
FILE_FLAGS = {"attention.hip": ["-fno-honor-nans"]}


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the gfx950 library cannot be built")
    return exe


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # Drop the host pass's known warning about the device-only feature flag.
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all HIP sources for gfx950 and link ``libkfmi.so``; returns its path."""
    cc = hipcc()
    objdir = LIBDIR / "obj"
    objdir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [objdir / (s.stem + ".o") for s in sources]
    cmds = [[cc, *COMMON, *DEVICE_FLAGS, *FILE_FLAGS.get(s.name, []), "-c", str(s), "-o", str(o)]
            for s, o in zip(sources, objs)]
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB.with_suffix(".so.tmp")
    # -z defs: an unresolved symbol (e.g. a kernel stub the host pass did not
    # emit) fails the build instead of the first dlopen.
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))

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


# Per-file flags.  The attention kernels: no NaN inputs reach their max reductions
# (masked scores are -inf, not NaN), and without NaN semantics fmaxf needs no
# canonicalising instructions, so max trees map onto v_max3_f32.
_NO_NANS = ["-fno-honor-nans"]
FILE_FLAGS = {"attention.hip": _NO_NANS, "attn_pp.hip": _NO_NANS, "attn_wide.hip": _NO_NANS}


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


def resources() -> list[dict]:
    """Per-kernel resource usage of every template instance in ``csrc/``, from
    the compiler's own report (``-Rpass-analysis=kernel-resource-usage``, the
    same flags as the build, device pass only): VGPRs, AGPRs, SGPRs, spills,
    scratch, LDS and waves per SIMD."""
    import re
    cc = hipcc()
    rows: list[dict] = []
    for src in sorted(CSRC.glob("*.hip")):
        cmd = [cc, *COMMON, *DEVICE_FLAGS, *FILE_FLAGS.get(src.name, []), "--cuda-device-only", "-c", str(src),
               "-o", os.devnull, "-Rpass-analysis=kernel-resource-usage"]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"resource report failed for {src.name}:\n{res.stderr[-2000:]}")
        cur = None
        for line in res.stderr.splitlines():
            m = re.search(r"remark: Function Name: (\S+)", line)
            if m:
                cur = {"file": src.name, "symbol": m.group(1)}
                rows.append(cur)
                continue
            m = re.search(r"remark:\s+([A-Za-z][A-Za-z /\[\]]*?):\s+(\S+) \[-Rpass", line)
            if m and cur is not None:
                cur[m.group(1).strip()] = m.group(2)
    filt = shutil.which("llvm-cxxfilt") or shutil.which("c++filt")
    if filt and rows:
        out = subprocess.run([filt], input="\n".join(r["symbol"] for r in rows), capture_output=True, text=True)
        for r, name in zip(rows, out.stdout.splitlines()):
            r["name"] = name.replace("kfmi::(anonymous namespace)::", "").replace("(kfmi::(anonymous namespace)::", "(")
    return rows


def resources_markdown(rows: list[dict]) -> str:
    cols = [("VGPRs", "VGPRs"), ("AGPRs", "AGPRs"), ("TotalSGPRs", "SGPRs"), ("VGPRs Spill", "VGPR spill"),
            ("SGPRs Spill", "SGPR spill"), ("ScratchSize [bytes/lane]", "scratch B/lane"),
            ("LDS Size [bytes/block]", "LDS B/block"), ("Occupancy [waves/SIMD]", "waves/SIMD")]
    lines = ["| file | kernel instance | " + " | ".join(c[1] for c in cols) + " |",
             "|" + "---|" * (2 + len(cols))]
    for r in rows:
        lines.append(f"| {r['file']} | `{r.get('name', r['symbol'])}` | "
                     + " | ".join(str(r.get(c[0], "")) for c in cols) + " |")
    return "\n".join(lines) + "\n"


if __name__ == "__main__":
    if "--resources" in sys.argv:
        print(resources_markdown(resources()), end="")
    else:
        print(build(verbose="-v" in sys.argv))

"""Host-side AddressSanitizer / UndefinedBehaviorSanitizer run of the library
(no GPU).  Not collected by pytest; run it by hand:

    python tests/host_asan.py [OUT_DIR]

It compiles every HIP source with the build's own flags plus host-only
sanitizers (each sanitizer flag behind -Xarch_host, so device code is built
as usual), links libkfmi.so into OUT_DIR (default: a temporary directory), and
runs the CPU test suite against that copy with clang's ASAN runtime preloaded
and leak detection off (the Python interpreter itself is not instrumented).
The library's host code (argument checks, dispatch and split plans, launch
records, per-thread tuning, clock-stamp bookkeeping) runs under the
sanitizers; a report stops the run with a non-zero status.  Two CPU tests are
left out: the C caller (gcc cannot link the sanitized copy without the
runtime) and the device-IR check (it compiles the sources itself).
"""
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

from kernelfuser_amd import build as B  # noqa: E402

HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-omit-frame-pointer", "-g"]
PLUGIN = """
from pathlib import Path


def pytest_configure(config):
    from kernelfuser_amd import _lib
    _lib.LIB_PATH = Path({lib!r})
"""


def build_sanitized(out: Path) -> Path:
    out.mkdir(parents=True, exist_ok=True)
    cc = B.hipcc()
    srcs = sorted(B.CSRC.glob("*.hip"))
    objs = [out / (s.stem + ".o") for s in srcs]
    cmds = [[cc, *B.COMMON, *B.DEVICE_FLAGS, *B.FILE_FLAGS.get(s.name, []), *HOST_SAN, "-c", str(s), "-o", str(o)]
            for s, o in zip(srcs, objs)]
    with ThreadPoolExecutor(8) as ex:
        list(ex.map(lambda c: B._run(c, False), cmds))
    lib = out / "libkfmi.so"
    B._run([cc, f"--offload-arch={B.ARCH}", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address",
            "-Xarch_host", "-fsanitize=undefined", "-shared-libsan", "-o", str(lib), *map(str, objs)], False)
    return lib


def asan_runtime() -> str:
    clang = Path(B.hipcc()).resolve().parent.parent / "llvm" / "bin" / "clang"
    if not clang.exists():
        clang = Path("/opt/rocm/llvm/bin/clang")
    path = subprocess.run([str(clang), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                          text=True, check=True).stdout.strip()
    if not Path(path).is_file():
        raise RuntimeError(f"clang's ASAN runtime not found ({path})")
    return path


def main(argv: list[str]) -> int:
    out = Path(argv[0]) if argv else Path(tempfile.mkdtemp(prefix="kfmi-asan-"))
    lib = build_sanitized(out)
    (out / "kfmi_asan_plugin.py").write_text(PLUGIN.format(lib=str(lib)))
    # the ASAN runtime first; whatever the environment already preloads stays
    preload = " ".join(p for p in (asan_runtime(), os.environ.get("LD_PRELOAD", "")) if p)
    env = {"LD_PRELOAD": preload, "ASAN_OPTIONS": "detect_leaks=0:verify_asan_link_order=0:halt_on_error=1",
           "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1", "PYTHONPATH": str(out)}
    cmd = [sys.executable, "-m", "pytest", "-p", "kfmi_asan_plugin", str(ROOT / "tests"), "-q", "-m", "not gpu",
           "--deselect", "tests/test_c_caller.py", "--deselect", "tests/test_nan_checks_ir.py"]
    return subprocess.run(cmd, cwd=ROOT, env={**os.environ, **env}).returncode


if __name__ == "__main__":
    raise SystemExit(main(sys.argv[1:]))

"""The C ABI from C: a C99 program compiled with gcc against include/kfmi.h
and linked to the built libkfmi.so (as a cgo, JNI or N-API binding would
link it) sees the header's struct layouts, the query entry points and the
argument errors, without touching a GPU."""
import ctypes
import shutil
import subprocess
from pathlib import Path

import pytest

from kernelfuser_amd import _lib

ROOT = Path(__file__).resolve().parent.parent

PROGRAM = r"""
#include <stdio.h>
#include <string.h>
#include "kfmi.h"

int main(void) {
  printf("abi %d\n", kfmi_abi_version());
  printf("sizes %zu %zu %zu\n", sizeof(kfmi_tuning), sizeof(kfmi_clock_stamp), sizeof(kfmi_launch_info));
  printf("work %lld\n", (long long)kfmi_attention_workspace_bytes(1, 8, 4, 2048, 256, 1));
  printf("kernel %d\n", kfmi_attention_kernel(1, 32, 8, 4096, 128, 1, KFMI_MODE_QUERY));
  /* an invalid shape is rejected before any device access */
  int rc = kfmi_prepare_bf16((void *)16, (void *)16, NULL, (void *)16, (void *)16, (void *)16, (void *)16,
                             (void *)16, (void *)16, NULL, 0, 32, 8, 16, 128, 1e-6f, KFMI_NORM_FP32, 0, NULL);
  printf("einval %d %d\n", rc == KFMI_EINVAL, strstr(kfmi_last_error(), ">= 1") != NULL);
  kfmi_tuning t;
  memset(&t, 0, sizeof t);
  t.attn_kernel = KFMI_KERNEL_WIDE + 1;
  printf("tuning %d\n", kfmi_set_tuning(&t) == KFMI_EINVAL);
  printf("stamps %d\n", kfmi_clock_stamps(NULL, 4));
  return 0;
}
"""


@pytest.fixture(scope="module")
def c_output(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    lib = _lib.LIB_PATH
    if not lib.exists():
        pytest.skip("libkfmi.so not built")
    d = tmp_path_factory.mktemp("ccaller")
    src = d / "caller.c"
    src.write_text(PROGRAM)
    exe = d / "caller"
    cmd = [gcc, "-std=c99", "-Wall", "-Werror", "-I", str(ROOT / "include"), str(src), "-o", str(exe),
           "-L", str(lib.parent), "-l:" + lib.name, "-Wl,-rpath," + str(lib.parent)]
    subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=120)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    return dict(line.split(" ", 1) for line in res.stdout.strip().splitlines())


def test_c_caller_sees_the_abi(c_output):
    assert int(c_output["abi"]) == _lib.ABI_VERSION
    tuning, stamp, info = (int(x) for x in c_output["sizes"].split())
    assert tuning == ctypes.sizeof(_lib.Tuning)
    assert stamp == ctypes.sizeof(_lib.ClockStamp)
    assert info == ctypes.sizeof(_lib.LaunchInfo)
    # the same answers the Python binding gets from the same library
    assert int(c_output["work"]) == _lib.load().kfmi_attention_workspace_bytes(1, 8, 4, 2048, 256, 1)
    assert int(c_output["kernel"]) == _lib.KERNELS[_lib.attention_kernel(1, 32, 8, 4096, 128, True, 0)]


def test_c_caller_gets_errors(c_output):
    assert c_output["einval"] == "1 1"
    assert c_output["tuning"] == "1"
    assert int(c_output["stamps"]) == -_lib.KFMI_EINVAL

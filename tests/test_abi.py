"""The C-ABI library on a host without a GPU: it loads, reports its ABI
version, exports every entry point ``include/kfmi.h`` declares, and rejects
invalid arguments with KFMI_EINVAL and a message before touching a device.
No compute call is made here."""
import ctypes
import re
from pathlib import Path

import pytest

from kernelfuser_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "kfmi.h"
EINVAL = _lib.KFMI_EINVAL


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(kfmi_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_declares_the_bound_entry_points():
    names = _declared()
    queries = {"kfmi_abi_version", "kfmi_last_error", "kfmi_attention_workspace_bytes", "kfmi_last_launches",
               "kfmi_set_tuning", "kfmi_get_tuning", "kfmi_attention_kernel", "kfmi_clock_stamps"}
    assert queries <= set(names)
    assert set(_lib.SIGNATURES) == set(names) - queries


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    m = re.search(r"#define KFMI_ABI_VERSION (\d+)", HEADER.read_text())
    assert lib.kfmi_abi_version() == int(m.group(1)) == _lib.ABI_VERSION


def _err(lib):
    return lib.kfmi_last_error().decode()


# (entry point, arguments, fragment of the expected message); pointers are
# NULL or a fake aligned value that is never dereferenced because an earlier
# argument check fails first.
FAKE = 1 << 20
P = FAKE
CASES = [
    ("kfmi_prepare_bf16", (P, P, None, P, P, P, P, P, P, None, 0, 32, 8, 16, 128, 1e-6, 2, 2, None), "must be >= 1"),
    ("kfmi_prepare_bf16", (P, P, None, P, P, P, P, P, P, None, 1, 32, 8, 16, 64, 1e-6, 2, 2, None), "D must be"),
    ("kfmi_prepare_bf16", (P, P, None, P, P, P, P, P, P, None, 1, 30, 8, 16, 128, 1e-6, 2, 2, None), "multiple of Hkv"),
    ("kfmi_prepare_bf16", (P, P, None, P, P, P, P, P, P, None, 1, 32, 8, 16, 128, 1e-6, 7, 2, None), "norm_style"),
    ("kfmi_prepare_bf16", (P, P, None, P, P, P, P, P, P, None, 1, 32, 8, 16, 128, 1e-6, 2, 64, None), "flags"),
    ("kfmi_prepare_bf16", (P, None, None, P, P, P, P, P, P, None, 1, 32, 8, 16, 128, 1e-6, 2, 2, None), "k must not"),
    ("kfmi_prepare_bf16", (P, P, None, P, P, None, P, P, P, None, 1, 32, 8, 16, 128, 1e-6, 2, 2, None), "cos"),
    ("kfmi_prepare_bf16", (P, P, None, P, P, P, P, P, P, P, 1, 32, 8, 16, 128, 1e-6, 2, 2, None), "v must not"),
    ("kfmi_prepare_bf16", (P, P, P, P, P, P, P, P, P, P, 1, 32, 8, 12, 128, 1e-6, 2, 2, None), "S % 8"),
    ("kfmi_prepare_bf16", (P + 2, P, None, P, P, P, P, P, P, None, 1, 32, 8, 16, 128, 1e-6, 2, 0, None), "aligned"),
    ("kfmi_attention_bf16", (P, P, P, None, P, P, P, P, 1, 32, 8, 16, 128, 0.1, 1e-6, 1, 1, 2, 33, 64, None, 0, None), "bm"),
    ("kfmi_attention_bf16", (P, P, P, None, P, P, P, P, 1, 32, 8, 16, 128, 0.1, 1e-6, 1, 1, 2, 128, 48, None, 0, None), "bn"),
    ("kfmi_attention_bf16", (P, P, P, None, P, P, None, P, 1, 32, 8, 16, 128, 0.1, 1e-6, 1, 1, 2, 128, 64, None, 0, None),
     "both rotary"),
    ("kfmi_attention_bf16", (P, P, P, None, P, P, P, P, 1, 32, 8, 16, 128, 0.0, 1e-6, 1, 1, 2, 128, 64, None, 0, None),
     "scale"),
    ("kfmi_attention_bf16", (P, P, P, None, None, P, P, P, 1, 32, 8, 16, 128, 0.1, 1e-6, 1, 1, 2, 128, 64, None, 0, None),
     "gq"),
    ("kfmi_attention_bf16", (P, P, P, None, P, P, P, P, 1, 2 ** 16, 8, 2 ** 12, 256, 0.1, 1e-6, 1, 1, 2, 128, 64,
                             None, 0, None), "2^31"),
    ("kfmi_attention_bf16", (P, P, P, None, P, P, P, P, 1, 32, 8, 16, 128, 0.1, 1e-6, 1, 1, 2, 128, 64, None, -1, None),
     "work_bytes"),
    ("kfmi_attention_bf16", (P, P, P, None, P, P, P, P, 1, 32, 8, 16, 128, 0.1, 1e-6, 1, 1, 2, 128, 64, P + 4, 64, None),
     "work must be"),
    ("kfmi_launch_attention_bf16", (P, P, P, P, P, P, P, P, None, P, None, 1, 32, 8, 16, 128, 0.1, 1e-6, 1, 5, 2,
                                    128, 64, None, 0, None), "Invalid fusion mode"),
    ("kfmi_launch_attention_bf16", (P, P, P, P, None, P, P, P, None, None, None, 1, 32, 8, 16, 128, 0.1, 1e-6, 1, 2,
                                    2, 128, 64, None, 0, None), "gk must not"),
    ("kfmi_launch_attention_bf16", (P, P, P, P, P, P, None, P, None, None, None, 1, 32, 8, 16, 128, 0.1, 1e-6, 1, 2,
                                    2, 128, 64, None, 0, None), "both rotary"),
    ("kfmi_launch_attention_bf16", (P, P, P, P, P, P, P, P, None, None, None, 1, 32, 8, 16, 128, 0.1, 1e-6, 1, 0, 2,
                                    128, 64, None, 0, None), "Missing scratch buffers"),
    ("kfmi_launch_attention_bf16", (P, P, P, P, P, P, P, P, None, P, None, 1, 32, 8, 16, 128, 0.1, 1e-6, 1, 1, 2,
                                    128, 64, None, 0, None), "Missing scratch buffers"),
    ("kfmi_transpose_v_bf16", (P, P, 4, 100, 128, None), "multiple of 8"),
    ("kfmi_transpose_v_bf16", (P, P, 4, 64, 96, None), "D must be"),
    ("kfmi_transpose_v_bf16", (P, None, 4, 64, 128, None), "vt must not"),
    ("kfmi_factored_prepare_bf16", (P, P, P, P, None, P, 1, 16, 8, 16, 256, 1e-6, None), "inv must not"),
    ("kfmi_factored_prepare_bf16", (P, P, P, P, P, P, 1, 16, 8, 16, 256, -1.0, None), "eps"),
    ("kfmi_factored_attention_bf16", (P, P, P, P, P, 1, 16, 8, 16, 256, 1e-6, 1, 2, 128, 64, None, 0, None), "inv_mode"),
    ("kfmi_factored_attention_bf16", (P, P, P, None, P, 1, 16, 8, 16, 256, 1e-6, 1, 0, 128, 64, None, 0, None),
     "inv must not"),
    ("kfmi_factored_attention_bf16", (P, P, P, P + 2, P, 1, 16, 8, 16, 256, 1e-6, 1, 1, 128, 64, None, 0, None),
     "4-byte"),
    ("kfmi_launch_factored_attention_bf16", (P, P, P, P, P, P, P, P, 1, 16, 8, 16, 256, 1e-6, 1, 128, 16, None, 0, None),
     "bn"),
    ("kfmi_launch_factored_attention_bf16", (P, P, P, P, P, P, P, P, 1, 16, 8, 16, 256, 1e-6, 1, 128, 64, None, -1,
                                             None), "work_bytes"),
    ("kfmi_factored_attention_bf16", (P, P, P, P, P, 1, 16, 8, 16, 256, 1e-6, 1, 1, 128, 64, P + 8, 4096, None),
     "16-byte"),
]


@pytest.mark.parametrize("name,args,fragment", CASES, ids=[f"{c[0]}-{i}" for i, c in enumerate(CASES)])
def test_invalid_arguments_fail_before_launch(lib, name, args, fragment):
    rc = getattr(lib, name)(*args)
    assert rc == EINVAL, (rc, _err(lib))
    assert fragment in _err(lib), _err(lib)


def test_workspace_bytes_query(lib):
    f = lib.kfmi_attention_workspace_bytes
    assert f(1, 32, 8, 0, 128, 1) == -1  # invalid shape
    assert f(1, 32, 8, 8192, 128, 1) == 0  # runs the ping-pong kernel: no split
    assert f(1, 32, 8, 2048, 128, 1) == 0  # D = 128: two workgroups per CU, no split
    assert f(1, 16, 8, 2048, 256, 0) == 0  # not causal: nothing to balance
    assert f(4, 16, 8, 2048, 256, 1) == 0  # more work items than CUs
    assert f(1, 16, 8, 2048, 256, 1) == 0  # 256 items = 256 CUs: already one per CU
    n = f(1, 8, 4, 2048, 256, 1)  # 128 items on 256 CUs: the long blocks split
    # 8 split blocks x 8 heads: a 4 KiB counter region (the same for every
    # shape) + 2 halves of 256 threads x (128 + 2) floats per pair
    pairs = 8 * 8
    assert n == 4096 + pairs * 2 * 130 * 256 * 4
    # a 12-pair plan keeps the same counter region: its partials start where
    # the 64-pair plan's do
    assert f(1, 4, 2, 640, 256, 1) == 4096 + 12 * 2 * 130 * 256 * 4


def test_attention_kernel_query(lib):
    """The kernel choice by shape, as measured by the tuning runner (CU
    count 256 where no device can be queried)."""
    k = lambda *a: _lib.attention_kernel(*a)
    assert k(1, 32, 8, 2048, 128, True, 0) == "general"     # causal, 16 blocks: half the CUs paired
    assert k(1, 32, 8, 3072, 128, True, 0) == "pingpong"    # causal, 24 blocks
    assert k(1, 64, 8, 2048, 128, True, 0) == "pingpong"    # Qwen3-32B: the pairing fills every CU
    assert k(1, 32, 8, 2048, 128, False, 0) == "pingpong"   # 256 items: one round
    assert k(1, 32, 8, 3072, 128, False, 0) == "general"    # 384 items: 1.5 rounds
    assert k(4, 32, 8, 1000, 128, True, 0) == "pingpong"    # 8 blocks, one paired unit per CU
    assert k(8, 32, 8, 1024, 128, True, 0) == "general"     # 8 blocks, two paired units per CU
    assert k(4, 32, 8, 1000, 128, False, 0) == "general"    # 8 blocks, not causal
    assert k(1, 32, 8, 1024, 128, True, 0) == "general"     # 8 blocks, not paired
    assert k(32, 32, 8, 128, 128, True, 0) == "general"     # one unit per CU, but of 3 tiles
    assert k(1, 32, 8, 8192, 128, True, 2) == "general"     # mode 'full'
    assert k(1, 16, 8, 8192, 256, True, 0) == "general"     # D = 256
    assert k(1, 40, 8, 8192, 128, True, 0) == "general"     # odd GQA ratio
    with _lib.tuning(attn_kernel="wide"):
        assert k(4, 32, 8, 1000, 128, True, 0) == "wide"
    with _lib.tuning(persistent=1):
        assert k(1, 64, 8, 2048, 128, True, 0) == "general"  # without the pairing the grid does not fill
        assert k(4, 32, 8, 1000, 128, True, 0) == "general"
    assert lib.kfmi_attention_kernel(1, 32, 8, 0, 128, 1, 0) == -EINVAL
    assert lib.kfmi_attention_kernel(1, 32, 8, 16, 128, 1, 7) == -EINVAL
    with _lib.tuning(attn_kernel="pingpong"):
        assert lib.kfmi_attention_kernel(1, 16, 8, 16, 256, 1, 0) == -EINVAL
        assert "ping-pong" in _err(lib)


def test_call_maps_einval_to_value_error(lib):
    with pytest.raises(ValueError, match="Invalid fusion mode"):
        _lib.call("kfmi_launch_attention_bf16", P, P, P, P, P, P, P, P, None, P, None, 1, 32, 8, 16, 128, 0.1,
                  1e-6, 1, 9, 2, 128, 64, None, 0, None)


def test_last_error_is_per_thread(lib):
    import threading
    lib.kfmi_transpose_v_bf16(P, P, 4, 100, 128, None)
    seen = {}

    def other():
        seen["msg"] = lib.kfmi_last_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == "" and "multiple of 8" in _err(lib)


def test_failed_call_reports_no_launches(lib):
    lib.kfmi_transpose_v_bf16(P, P, 4, 100, 128, None)  # rejected before any launch
    assert lib.kfmi_last_launches(None, 0) == 0
    assert _lib.last_launches() == []


def test_tuning_overrides_validate_and_scope(lib):
    """kfmi_set_tuning rejects out-of-range fields, keeps settings per
    thread, and a forced kernel that cannot run a shape fails the call with
    KFMI_EINVAL before any device access."""
    assert _lib.get_tuning() == dict.fromkeys(_lib.TUNING_FIELDS, 0)
    for bad in ({"attn_kernel": 4}, {"pp_heads": 3}, {"rows_heads": 1}, {"split": 2}, {"persistent": -1},
                {"clock_stamps": 2}):
        with pytest.raises(ValueError):
            _lib.set_tuning(**bad)
    assert _lib.get_tuning() == dict.fromkeys(_lib.TUNING_FIELDS, 0)
    args = (P, P, P, None, P, P, P, P, 1, 16, 8, 4096, 128, 0.1, 1e-6, 1, 1, 2, 128, 64, None, 0, None)
    with _lib.tuning(attn_kernel="wide"):
        assert lib.kfmi_attention_bf16(*args) == EINVAL  # GQA ratio 2
        assert "wide kernel" in _err(lib)
        import threading
        seen = {}
        th = threading.Thread(target=lambda: seen.update(_lib.get_tuning()))
        th.start()
        th.join()
        assert seen["attn_kernel"] == 0  # another thread keeps its own settings
    with _lib.tuning(attn_kernel="pingpong", pp_heads=2):
        assert lib.kfmi_attention_bf16(*args) == EINVAL  # four heads per item need a ratio of 4
    args256 = args[:12] + (256,) + args[13:]
    with _lib.tuning(attn_kernel="pingpong"):
        assert lib.kfmi_attention_bf16(*args256) == EINVAL
    assert _lib.get_tuning()["attn_kernel"] == 0


def test_clock_stamp_layout_and_arguments(lib):
    """kfmi_clock_stamp and kfmi_tuning sizes match the header's fields;
    kfmi_clock_stamps rejects a NULL buffer with room for entries."""
    assert ctypes.sizeof(_lib.ClockStamp) == 32
    assert ctypes.sizeof(_lib.Tuning) == 4 * 6
    m = re.search(r"#define KFMI_CLOCK_STAMPS_MAX (\d+)", HEADER.read_text())
    assert int(m.group(1)) == _lib.CLOCK_STAMPS_MAX
    assert lib.kfmi_clock_stamps(None, 4) == -EINVAL
    assert "NULL" in _err(lib)
    s = [(0, 2000, 0, 100), (0, 4200, 10, 110), (5, 1805, 20, 120)]  # 2.0, 4.2, 1.8 GHz
    c = _lib.clock_summary(s)
    assert (round(c["ghz_median"], 6), round(c["ghz_min"], 6), round(c["ghz_max"], 6)) == (2.0, 1.8, 4.2)
    assert c["workgroups"] == 3 and c["workgroup_us_median"] == 1.0 and round(c["span_us"], 6) == 1.2


def test_launch_handle_reads_only_its_own_call():
    """A launcher's lazy record handle is valid until the thread's next
    compute call; a read after it raises (no GPU call is made here)."""
    h = _lib.Launches()
    assert list(h) == [] and len(h) == 0  # this thread's last call launched nothing
    stale = _lib.Launches()
    _lib._tls.calls = _lib._calls() + 1  # as a later successful call would
    with pytest.raises(RuntimeError):
        len(stale)
    with _lib.record_launches() as outer:
        with _lib.record_launches() as inner:
            pass
    assert outer.launches == [] and inner.kernels() == []

"""ctypes binding of the gfx950 C-ABI library (``include/kfmi.h``).

The library is built in-tree by ``python -m kernelfuser_amd.build``.  There is
no fallback: if the library is missing or cannot be loaded, every op raises.
torch is imported first so the HIP runtime torch ships is the one the library
binds to (both use the ``libamdhip64.so.7`` soname).
"""
from __future__ import annotations

import ctypes
import threading
from collections.abc import Sequence
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime before the library)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libkfmi.so"
ABI_VERSION = 10

KFMI_OK, KFMI_EINVAL, KFMI_ELAUNCH, KFMI_EDEVICE = 0, 1, 2, 3
NORM_STYLES = {"hf": 0, "legacy": 1, "fp32": 2}
PREP_ONLY_K, PREP_ROPE = 1, 2
MODE_QUERY, MODE_UNFUSED, MODE_FULL = 0, 1, 2
# attention kernels (KFMI_KERNEL_*)
KERNEL_AUTO, KERNEL_GENERAL, KERNEL_PINGPONG, KERNEL_WIDE = 0, 1, 2, 3
KERNELS = {"auto": KERNEL_AUTO, "general": KERNEL_GENERAL, "pingpong": KERNEL_PINGPONG, "wide": KERNEL_WIDE}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_D = ctypes.c_double

# name -> argtypes (restype is int for all compute entry points)
SIGNATURES = {
    "kfmi_prepare_bf16": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _I, _I, _P],
    "kfmi_attention_bf16": [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _D, _F, _I, _I, _I, _I, _I,
                            _P, _I64, _P],
    "kfmi_transpose_v_bf16": [_P, _P, _I64, _I64, _I64, _P],
    "kfmi_launch_attention_bf16": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _D,
                                   _F, _I, _I, _I, _I, _I, _P, _I64, _P],
    "kfmi_launch_attention_bf16_noalloc": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                           _D, _F, _I, _I, _I, _I, _I, _P],
    "kfmi_factored_prepare_bf16": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _P],
    "kfmi_factored_attention_bf16": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _I, _I, _I, _I, _P,
                                     _I64, _P],
    "kfmi_launch_factored_attention_bf16": [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _I,
                                            _I, _I, _P, _I64, _P],
}

_lock = threading.Lock()
_lib = None


class KfmiError(RuntimeError):
    """A non-argument failure reported by the native library."""


def load() -> ctypes.CDLL:
    """Load (once) and return the native library; raises if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"kfmi native library not found at {LIB_PATH}; build it with "
                "`python -m kernelfuser_amd.build` (there is no CPU fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.kfmi_abi_version.restype = ctypes.c_int
        lib.kfmi_abi_version.argtypes = []
        lib.kfmi_last_error.restype = ctypes.c_char_p
        lib.kfmi_last_error.argtypes = []
        lib.kfmi_attention_workspace_bytes.restype = ctypes.c_int64
        lib.kfmi_attention_workspace_bytes.argtypes = [_I64, _I64, _I64, _I64, _I64, _I]
        lib.kfmi_attention_kernel.restype = ctypes.c_int
        lib.kfmi_attention_kernel.argtypes = [_I64, _I64, _I64, _I64, _I64, _I, _I]
        lib.kfmi_last_launches.restype = ctypes.c_int
        lib.kfmi_last_launches.argtypes = [ctypes.POINTER(LaunchInfo), _I]
        lib.kfmi_set_tuning.restype = ctypes.c_int
        lib.kfmi_set_tuning.argtypes = [ctypes.POINTER(Tuning)]
        lib.kfmi_get_tuning.restype = None
        lib.kfmi_get_tuning.argtypes = [ctypes.POINTER(Tuning)]
        lib.kfmi_clock_stamps.restype = ctypes.c_int
        lib.kfmi_clock_stamps.argtypes = [ctypes.POINTER(ClockStamp), _I]
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        if lib.kfmi_abi_version() != ABI_VERSION:
            raise RuntimeError(f"kfmi ABI version {lib.kfmi_abi_version()} != {ABI_VERSION}")
        _lib = lib
    return _lib


class LaunchInfo(ctypes.Structure):
    """kfmi_launch_info of include/kfmi.h."""
    _fields_ = [("kernel", ctypes.c_char * 96), ("grid", ctypes.c_int64), ("block", ctypes.c_int32),
                ("registers", ctypes.c_int32), ("lds_bytes", ctypes.c_int32), ("scratch_bytes", ctypes.c_int32),
                ("plan", ctypes.c_char * 64)]


def attention_kernel(b: int, hq: int, hkv: int, s: int, d: int, causal: bool, mode: int) -> str:
    """Name (a key of KERNELS) of the attention kernel that a call of this
    shape and mode launches on the current device under the calling
    thread's overrides (kfmi_attention_kernel)."""
    lib = load()
    k = lib.kfmi_attention_kernel(b, hq, hkv, s, d, int(bool(causal)), mode)
    if k < 0:
        raise ValueError(f"kfmi_attention_kernel: {lib.kfmi_last_error().decode(errors='replace')}")
    return {v: n for n, v in KERNELS.items()}[k]


class Tuning(ctypes.Structure):
    """kfmi_tuning of include/kfmi.h: dispatch choices the library otherwise
    makes by shape (0 = by shape)."""
    _fields_ = [("attn_kernel", ctypes.c_int32), ("pp_heads", ctypes.c_int32), ("rows_heads", ctypes.c_int32),
                ("split", ctypes.c_int32), ("persistent", ctypes.c_int32), ("clock_stamps", ctypes.c_int32)]


class ClockStamp(ctypes.Structure):
    """kfmi_clock_stamp of include/kfmi.h."""
    _fields_ = [("t0", ctypes.c_uint64), ("t1", ctypes.c_uint64), ("r0", ctypes.c_uint64), ("r1", ctypes.c_uint64)]


CLOCK_STAMPS_MAX = 2048
REALTIME_HZ = 100e6  # s_memrealtime


def clock_stamps() -> list[tuple[int, int, int, int]]:
    """(t0, t1, r0, r1) per workgroup of the last attention launch on the
    current device that recorded clock stamps (kfmi_clock_stamps; launches
    record them under ``tuning(clock_stamps=1)``).  Waits for the device."""
    lib = load()
    buf = (ClockStamp * CLOCK_STAMPS_MAX)()
    n = lib.kfmi_clock_stamps(buf, CLOCK_STAMPS_MAX)
    if n < 0:
        raise RuntimeError(f"kfmi_clock_stamps: {lib.kfmi_last_error().decode(errors='replace')}")
    return [(r.t0, r.t1, r.r0, r.r1) for r in buf[:n]]


def clock_summary(stamps) -> dict:
    """Shader clock per workgroup, (t1 - t0) / (r1 - r0) x 100 MHz, in GHz
    (median, min, max), the workgroups' median lifetime and the span from the
    first start to the last end (microseconds)."""
    ghz = sorted((t1 - t0) / (r1 - r0) * REALTIME_HZ / 1e9 for t0, t1, r0, r1 in stamps if r1 > r0)
    if not ghz:
        raise ValueError("no clock stamps")
    life = sorted((r1 - r0) / REALTIME_HZ * 1e6 for _, _, r0, r1 in stamps)
    span = (max(r1 for *_, r1 in stamps) - min(r0 for _, _, r0, _ in stamps)) / REALTIME_HZ * 1e6
    return {"ghz_median": ghz[len(ghz) // 2], "ghz_min": ghz[0], "ghz_max": ghz[-1], "workgroups": len(stamps),
            "workgroup_us_median": life[len(life) // 2], "span_us": span}


TUNING_FIELDS = tuple(f for f, _ in Tuning._fields_)


def get_tuning() -> dict:
    """The calling thread's dispatch overrides (kfmi_get_tuning)."""
    t = Tuning()
    load().kfmi_get_tuning(ctypes.byref(t))
    return {f: getattr(t, f) for f in TUNING_FIELDS}


def set_tuning(**fields) -> None:
    """Set the calling thread's dispatch overrides (kfmi_set_tuning); fields
    not given are 0 (by shape).  ``attn_kernel`` also takes a name of
    KERNELS.  For tuning runs and tests: the reference-signature ops never
    call this."""
    unknown = set(fields) - set(TUNING_FIELDS)
    if unknown:
        raise ValueError(f"unknown tuning fields {sorted(unknown)}")
    if isinstance(fields.get("attn_kernel"), str):
        fields["attn_kernel"] = KERNELS[fields["attn_kernel"]]
    t = Tuning(**{f: int(fields.get(f, 0)) for f in TUNING_FIELDS})
    lib = load()
    if lib.kfmi_set_tuning(ctypes.byref(t)) != KFMI_OK:
        raise ValueError(f"kfmi_set_tuning: {lib.kfmi_last_error().decode(errors='replace')}")


class tuning:
    """``with tuning(attn_kernel='wide'): ...`` -- overrides for the block,
    then the previous ones again."""

    def __init__(self, **fields):
        self.fields = fields
        self.saved: dict | None = None

    def __enter__(self):
        self.saved = get_tuning()
        set_tuning(**self.fields)
        return self

    def __exit__(self, *exc):
        set_tuning(**self.saved)
        return False


def last_launches(max_records: int = 8) -> list[dict]:
    """The kernels launched by this thread's last successful compute call
    (kfmi_last_launches), in launch order: kernel instance, workgroups,
    threads per workgroup, registers per thread, static LDS and scratch bytes,
    and the launch-time choices (``plan``, e.g. "hpg=2 persistent=1 xcd=1")."""
    lib = load()
    buf = (LaunchInfo * max_records)()
    n = lib.kfmi_last_launches(buf, max_records)
    return [{"kernel": r.kernel.decode(errors="replace"), "grid": r.grid, "block": r.block,
             "registers": r.registers, "lds_bytes": r.lds_bytes, "scratch_bytes": r.scratch_bytes,
             "plan": r.plan.decode(errors="replace")}
            for r in buf[:min(n, max_records)]]


_tls = threading.local()


def _calls() -> int:
    """Successful compute calls made by this thread so far."""
    return getattr(_tls, "calls", 0)


class Launches(Sequence):
    """The kernels one compute call launched, read from the library only when
    first used (so an eager launch costs one ctypes call).  The library keeps
    the records of a thread's last call only: reading a handle after a later
    call on the same thread raises instead of returning that call's kernels."""

    def __init__(self):
        self._thread = threading.get_ident()
        self._call = _calls()
        self._records = None

    def _get(self) -> list:
        if self._records is None:
            if threading.get_ident() != self._thread or _calls() != self._call:
                raise RuntimeError("launch records are read before the next compute call of the same thread")
            self._records = last_launches()
        return self._records

    def __getitem__(self, i):
        return self._get()[i]

    def __len__(self) -> int:
        return len(self._get())

    def __eq__(self, other) -> bool:
        return list(self._get()) == list(other)

    def __repr__(self) -> str:
        return f"Launches({self._get()!r})"


class record_launches:
    """``with record_launches() as rec: ...`` -- collects the launch records of
    every compute call the block makes on this thread into ``rec.launches``
    (the runners' per-arm kernel evidence).  Nests; each level sees its own
    block's calls."""

    def __init__(self):
        self.launches: list[dict] = []

    def __enter__(self):
        stack = getattr(_tls, "recorders", None)
        if stack is None:
            stack = _tls.recorders = []
        stack.append(self)
        return self

    def __exit__(self, *exc):
        _tls.recorders.remove(self)
        return False

    def kernels(self) -> list[str]:
        """The distinct kernel instances, in first-launch order."""
        seen = []
        for r in self.launches:
            if r["kernel"] not in seen:
                seen.append(r["kernel"])
        return seen


def call(name: str, *args) -> None:
    """Call a compute entry point; map its status to ValueError / KfmiError."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc == KFMI_OK:
        _tls.calls = _calls() + 1
        recs = getattr(_tls, "recorders", None)
        if recs:
            got = last_launches()
            for r in recs:
                r.launches.extend(got)
        return
    msg = lib.kfmi_last_error().decode(errors="replace")
    if rc == KFMI_EINVAL:
        raise ValueError(f"{name}: {msg}")
    raise KfmiError(f"{name} failed (status {rc}): {msg}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of torch's current stream on ``t``'s device."""
    return torch.cuda.current_stream(t.device).cuda_stream

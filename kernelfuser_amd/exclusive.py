"""Timing-validity guard: does another process share the selected GPU while a
runner times it?  Counterpart of the reference's ``gpu_snapshot`` /
``ExclusiveMonitor`` (src/e1_rope_publication_v1.py:304-342), its per-row use
in the A/A runner (src/e7_rope_aa.py:250-290) and the Qwen3 runner's
``_snapshot`` (src/e2_qwen3_rope_prefill.py:70-90).

``amd-smi`` names GPUs by PCI address, so the selected torch device is matched
to its ``amd-smi`` index through its PCI domain/bus/device.  A snapshot lists
the compute processes on that GPU.  ``exclusive`` is

* ``True``  when the list can be read and holds no process but this one,
* ``False`` when it holds another process (the reference's failing case),
* ``None``  when the list cannot be read: ``amd-smi`` is absent, fails, or
  cannot see processes (it reports "No running processes" even though this
  process holds a context on the GPU, which happens where the per-process
  driver directory it reads is not visible, as in some containers).

Unknown is recorded as unknown, never as exclusive.  A runner marks a row
``tested_invalid`` only on ``False``; receipts carry the summary either way.
"""
from __future__ import annotations

import json
import os
import shutil
import subprocess
import threading
import time
from typing import Any, Callable

Runner = Callable[[list], "tuple[int, str, str]"]


def _run_smi(args: list, timeout: float = 15.0) -> tuple[int, str, str]:
    """Run amd-smi as a child process: (return code, stdout, stderr)."""
    exe = shutil.which("amd-smi")
    if exe is None:
        return 127, "", "amd-smi not found"
    try:
        r = subprocess.run([exe, *args], capture_output=True, text=True, timeout=timeout)
    except (OSError, subprocess.TimeoutExpired) as e:
        return 124, "", repr(e)
    return r.returncode, r.stdout, r.stderr


def _json_payload(text: str) -> Any:
    """The JSON document in amd-smi's output (it may print notes before it)."""
    starts = [i for i in (text.find("["), text.find("{")) if i >= 0]
    if not starts:
        raise ValueError("no JSON in amd-smi output")
    return json.loads(text[min(starts):])


def _as_int(v: Any) -> int | None:
    if isinstance(v, dict):
        v = v.get("value")
    try:
        return int(v)
    except (TypeError, ValueError):
        return None


def device_bdf(device: int = 0) -> str:
    """PCI address "dddd:bb:dd" of a torch CUDA/HIP device."""
    import torch

    p = torch.cuda.get_device_properties(device)
    return f"{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}"


def smi_index(bdf: str, listing: str) -> int | None:
    """amd-smi GPU index whose PCI address matches ``bdf`` (``amd-smi list --json``)."""
    for gpu in _json_payload(listing):
        addr = str(gpu.get("bdf", "")).lower()
        if addr.startswith(bdf.lower()):
            return _as_int(gpu.get("gpu"))
    return None


def parse_processes(text: str, gpu: int) -> list[dict] | None:
    """Processes that ``amd-smi process --json`` lists on GPU ``gpu``, as
    ``{"pid", "name"}``; None when the output has no readable list for it."""
    try:
        doc = _json_payload(text)
    except ValueError:
        return None
    for entry in doc if isinstance(doc, list) else [doc]:
        if _as_int(entry.get("gpu")) != gpu:
            continue
        apps = []
        for item in entry.get("process_list", []):
            info = item.get("process_info", item) if isinstance(item, dict) else item
            if isinstance(info, str):  # "No running processes detected"
                continue
            pid = _as_int(info.get("pid")) if isinstance(info, dict) else None
            if pid is None:
                return None  # a format this parser does not know: unreadable, not empty
            apps.append({"pid": pid, "name": str(info.get("name", ""))})
        return apps
    return None


def gpu_snapshot(device: int = 0, *, holds_context: bool = True, run: Runner = _run_smi,
                 bdf: str | None = None) -> dict:
    """One observation of the selected GPU's compute processes.

    ``holds_context``: this process has a context on the GPU, so a readable
    list that does not name it is incomplete (``exclusive`` None)."""
    own = os.getpid()
    snap: dict[str, Any] = {"utc": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime()), "t": time.time(),
                            "device": device, "pid": own, "exclusive": None}
    try:
        snap["bdf"] = bdf if bdf is not None else device_bdf(device)
        rc, out, err = run(["list", "--json"])
        if rc != 0:
            snap["note"] = f"amd-smi list failed ({rc}): {err.strip()[:200]}"
            return snap
        gpu = smi_index(snap["bdf"], out)
        snap["gpu"] = gpu
        if gpu is None:
            snap["note"] = "selected device not found in amd-smi list"
            return snap
        rc, out, err = run(["process", "--json", "-g", str(gpu)])
        if rc != 0:
            snap["note"] = f"amd-smi process failed ({rc}): {err.strip()[:200]}"
            return snap
        apps = parse_processes(out, gpu)
        if apps is None:
            snap["note"] = "amd-smi process output not readable"
            return snap
        snap["apps"] = apps
        snap["foreign_apps"] = [a for a in apps if a["pid"] != own]
        if snap["foreign_apps"]:
            snap["exclusive"] = False
        elif holds_context and not any(a["pid"] == own for a in apps):
            snap["note"] = ("process list does not include this process: not visible to this user "
                            + (err.strip()[:120] if err.strip() else "")).strip()
        else:
            snap["exclusive"] = True
    except Exception as e:  # the guard must never break a timing run
        snap["note"] = f"snapshot failed: {e!r}"[:240]
    return snap


def summarize(records: list[dict]) -> dict:
    """``exclusive``: False if any observation saw another process, True if
    every one (at least one) saw none, None otherwise."""
    seen = [r.get("exclusive") for r in records]
    foreign = sorted({a["pid"] for r in records for a in r.get("foreign_apps", [])})
    if any(x is False for x in seen):
        ex = False
    elif seen and all(x is True for x in seen):
        ex = True
    else:
        ex = None
    notes = sorted({r["note"] for r in records if r.get("note")})
    return {"observations": len(records), "exclusive": ex, "foreign_pids": foreign, "notes": notes[:4]}


class ExclusiveMonitor:
    """Snapshots of the selected GPU every ``interval`` seconds on a daemon
    thread, from ``start()`` to ``finish()``."""

    def __init__(self, device: int = 0, interval: float = 1.0, run: Runner = _run_smi):
        self.device, self.interval, self._run = device, interval, run
        self.records: list[dict] = []
        self._stop = threading.Event()
        self._bdf: str | None = None
        self._thread = threading.Thread(target=self._loop, daemon=True)

    def _loop(self):
        while not self._stop.is_set():
            self.records.append(gpu_snapshot(self.device, run=self._run, bdf=self._bdf))
            self._stop.wait(self.interval)

    def start(self) -> "ExclusiveMonitor":
        try:  # resolve the PCI address on the caller's thread (a device query)
            self._bdf = device_bdf(self.device)
        except Exception:
            self._bdf = None
        self._thread.start()
        return self

    def between(self, t0: float, t1: float) -> list[dict]:
        """Observations taken in [t0, t1] (seconds since the epoch)."""
        return [r for r in list(self.records) if t0 <= r["t"] <= t1]

    def finish(self) -> list[dict]:
        self._stop.set()
        self._thread.join(timeout=max(5.0, 3 * self.interval))
        return list(self.records)


def guarded(row: dict, records: list[dict]) -> dict:
    """Attach the exclusivity summary of a row's observations; a row that saw
    another process on the GPU becomes ``tested_invalid``."""
    row["gpu_exclusivity"] = summarize(records)
    if row["gpu_exclusivity"]["exclusive"] is False:
        row["status"] = "tested_invalid"
    return row

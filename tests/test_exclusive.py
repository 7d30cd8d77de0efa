"""Timing-validity guard (kernelfuser_amd.exclusive) on recorded amd-smi
outputs: the selected device is matched by PCI address, another process on it
makes the snapshot non-exclusive and the row tested_invalid, and a process
list that cannot be read (or that omits this process although it holds a
context) is recorded as unknown, never as exclusive."""
import json
import os

from kernelfuser_amd import exclusive

LIST = json.dumps([{"gpu": 0, "bdf": "0000:05:00.0", "uuid": "a"}, {"gpu": 1, "bdf": "0000:72:00.0", "uuid": "b"}])
NONE = "Unable to open process directory: No such file or directory\n" + json.dumps(
    [{"gpu": 1, "process_list": [{"process_info": "No running processes detected"}]}])


def procs(gpu, *pids):
    return json.dumps([{"gpu": gpu, "process_list": [
        {"process_info": {"name": f"p{p}", "pid": p, "memory_usage": {"vram_mem": {"value": 1, "unit": "B"}}}}
        for p in pids]}])


def runner(process_out, calls=None, list_out=LIST, rc=0):
    def run(args):
        if calls is not None:
            calls.append(args)
        return (rc, list_out, "") if args[0] == "list" else (rc, process_out, "")
    return run


def test_selected_gpu_by_pci_address():
    calls = []
    s = exclusive.gpu_snapshot(0, run=runner(procs(1, os.getpid()), calls), bdf="0000:72:00")
    assert s["gpu"] == 1 and calls[1] == ["process", "--json", "-g", "1"]
    assert s["exclusive"] is True and s["foreign_apps"] == []


def test_foreign_process_is_not_exclusive():
    s = exclusive.gpu_snapshot(0, run=runner(procs(1, os.getpid(), 4242)), bdf="0000:72:00")
    assert s["exclusive"] is False and [a["pid"] for a in s["foreign_apps"]] == [4242]
    row = exclusive.guarded({"status": "passed"}, [s])
    assert row["status"] == "tested_invalid" and row["gpu_exclusivity"]["foreign_pids"] == [4242]


def test_unreadable_process_list_is_unknown():
    s = exclusive.gpu_snapshot(0, run=runner(NONE), bdf="0000:72:00")
    assert s["exclusive"] is None and "not visible" in s["note"]
    # no context held: an empty list is a readable, exclusive answer
    s2 = exclusive.gpu_snapshot(0, run=runner(NONE), bdf="0000:72:00", holds_context=False)
    assert s2["exclusive"] is True
    row = exclusive.guarded({"status": "passed"}, [s])
    assert row["status"] == "passed" and row["gpu_exclusivity"]["exclusive"] is None


def test_missing_tool_device_or_format_is_unknown():
    assert exclusive.gpu_snapshot(0, run=lambda a: (127, "", "amd-smi not found"), bdf="0000:72:00")["exclusive"] is None
    assert exclusive.gpu_snapshot(0, run=runner(procs(1)), bdf="0000:99:00")["exclusive"] is None
    odd = json.dumps([{"gpu": 1, "process_list": [{"process_info": {"name": "x"}}]}])
    assert exclusive.gpu_snapshot(0, run=runner(odd), bdf="0000:72:00")["exclusive"] is None
    assert exclusive.gpu_snapshot(0, run=runner("garbage"), bdf="0000:72:00")["exclusive"] is None


def test_summary_rules():
    t, f, n = {"exclusive": True}, {"exclusive": False, "foreign_apps": [{"pid": 7}]}, {"exclusive": None}
    assert exclusive.summarize([t, t])["exclusive"] is True
    assert exclusive.summarize([t, f, n])["exclusive"] is False
    assert exclusive.summarize([t, n])["exclusive"] is None
    assert exclusive.summarize([])["exclusive"] is None


def test_monitor_collects_and_windows():
    mon = exclusive.ExclusiveMonitor(0, interval=0.01, run=runner(procs(1, os.getpid())))
    mon._bdf = "0000:72:00"
    mon._thread.start()
    import time
    t0 = time.time()
    time.sleep(0.08)
    recs = mon.finish()
    assert len(recs) >= 2 and all(r["exclusive"] is True for r in recs)
    assert mon.between(t0, time.time())

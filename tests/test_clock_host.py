"""Host logic of the clock runner (no GPU): parsing of ``amd-smi metric
--power --clock --json`` output and the clock-stamp summary."""
import json

from kernelfuser_amd import _lib, clock
from kernelfuser_amd import exclusive as ex


def _metric_doc(watts, clocks):
    return {"gpu_data": [{"gpu": 0,
                          "power": {"socket_power": {"value": watts, "unit": "W"}, "gfx_voltage": "N/A"},
                          "clock": {**{f"gfx_{i}": {"clk": {"value": c, "unit": "MHz"},
                                                    "max_clk": {"value": 2400, "unit": "MHz"}}
                                       for i, c in enumerate(clocks)},
                                    "mem_0": {"clk": {"value": 1900, "unit": "MHz"}}}}]}


def test_power_sample_parses_socket_power_and_gfx_clocks(monkeypatch):
    doc = _metric_doc(1340, [1881, 1797, 1873, 1775])
    monkeypatch.setattr(ex, "_run_smi", lambda args, timeout=15.0: (0, "note: something\n" + json.dumps(doc), ""))
    w, clks = clock._smi_power_sample(0)
    assert w == 1340.0 and clks == [1881.0, 1797.0, 1873.0, 1775.0]  # mem clocks left out


def test_power_sample_unreadable(monkeypatch):
    monkeypatch.setattr(ex, "_run_smi", lambda args, timeout=15.0: (1, "", "no device"))
    assert clock._smi_power_sample(0) == (None, [])
    monkeypatch.setattr(ex, "_run_smi", lambda args, timeout=15.0: (0, "not json", ""))
    assert clock._smi_power_sample(0) == (None, [])
    doc = _metric_doc(1340, [])
    doc["gpu_data"][0]["power"]["socket_power"] = "N/A"
    monkeypatch.setattr(ex, "_run_smi", lambda args, timeout=15.0: (0, json.dumps(doc), ""))
    assert clock._smi_power_sample(0) == (None, [])


def test_table_marks_missing_power():
    row = {"B": 1, "S": 4096, "case": "random", "kernel": "attn_pp_kernel<true, 2, 2, false>(AttnParams)",
           "us": 127.0, "clock": _lib.clock_summary([(0, 1778, 0, 100)]), "power": None, "kcycles": 225.8,
           "tflops": 1082.0, "frac_mfma": 0.433, "frac_mfma_at_clock": 0.584}
    lines = clock.table([row, dict(row, power={"socket_w_median": 1368.0})]).splitlines()
    assert lines[2].endswith("| n/a |") and lines[3].endswith("| 1368 |")
    assert "1.778 (1.778-1.778)" in lines[2]

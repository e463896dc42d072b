"""Host-side logic of bench.py that needs no GPU: range verdicts, the idle
gate and the sysfs readers (on a fake sysfs tree), the previous-record
lookup, and the one-GPU refusal.  The reference's suite driver decides
"improved / regressed" only from non-overlapping ranges measured on an idle
GPU (agent/tools/bench.py:29-33, 78-119; agent/tools/_common.py:217-327)."""

import importlib.util
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_range_verdicts(bench):
    assert bench.ranges_overlap([1.0, 2.0], [1.5, 3.0])
    assert bench.ranges_overlap([1.0, 2.0], [2.0, 3.0])  # touching ranges overlap
    assert not bench.ranges_overlap([1.0, 1.9], [2.0, 3.0])
    c = bench.compare_range([1.0, 1.1], [1.2, 1.3], "old")
    assert c["verdict"] == "improved" and not c["ranges_overlap"] and c["median_delta_pct"] < 0
    c = bench.compare_range([1.4, 1.5], [1.2, 1.3], "old")
    assert c["verdict"] == "regressed" and c["median_delta_pct"] > 0
    c = bench.compare_range([1.25, 1.35], [1.2, 1.3], "old")
    assert c["verdict"] == "noise" and c["source"] == "old"


def test_range_of_rounds(bench):
    r = bench.range_of([[1.0, 2.0, 3.0], [2.0, 2.5, 2.0], [0.5, 1.5]])
    assert r["runs"] == 3
    assert (r["min"], r["max"]) == (1.0, 2.0)
    assert r["per_run_median_ms"] == [2.0, 2.0, 1.0]


def test_old_range_of_records(bench):
    assert bench.old_range_of(None) is None
    assert bench.old_range_of({"range_ms": {"min": 1.0, "max": 1.5}}) == [1.0, 1.5]
    assert bench.old_range_of({"value": 0.2}) == [0.2, 0.2]  # a record without repeated runs
    assert bench.old_range_of({"latency_ms_p50": 3.0}) == [3.0, 3.0]


def _fake_sysfs(tmp_path, busy):
    d = tmp_path / "0000:8e:00.0"
    (d / "hwmon" / "hwmon3").mkdir(parents=True)
    if busy is not None:
        (d / "gpu_busy_percent").write_text(f"{busy}\n")
    (d / "pp_dpm_sclk").write_text("0: 500Mhz\n1: 1400Mhz *\n2: 2400Mhz\n")
    (d / "pp_dpm_mclk").write_text("0: 900Mhz\n1: 2000Mhz *\n")
    (d / "hwmon" / "hwmon3" / "power1_average").write_text("271000000\n")
    (d / "hwmon" / "hwmon3" / "temp2_input").write_text("48000\n")
    return d


def test_gpu_state_reads_sysfs(bench, tmp_path):
    st = bench.gpu_state(_fake_sysfs(tmp_path, 7))
    assert st["busy_pct"] == 7.0
    assert st["sclk"] == "1400Mhz" and st["mclk"] == "2000Mhz"
    assert st["power_w"] == 271.0 and st["temp_c"] == 48.0


def test_idle_gate_passes_an_idle_device(bench, tmp_path):
    gate = bench.wait_for_idle(_fake_sysfs(tmp_path, 3), timeout_s=5.0, hold_s=0.3, poll_s=0.05)
    assert gate["idle"] and gate["measurable"]
    assert 0.3 <= gate["waited_s"] < 5.0
    assert gate["max_busy_pct_in_hold"] == 3.0


def test_idle_gate_refuses_a_busy_device(bench, tmp_path):
    gate = bench.wait_for_idle(_fake_sysfs(tmp_path, 55), timeout_s=0.4, hold_s=0.2, poll_s=0.05)
    assert not gate["idle"] and gate["measurable"]
    assert gate["last_busy_pct"] == 55.0 and "reason" in gate


def test_idle_gate_waits_for_the_device_to_settle(bench, tmp_path):
    """Busy at first, idle later: the gate holds until it has seen hold_s of
    idle readings."""
    import threading
    import time

    d = _fake_sysfs(tmp_path, 80)
    t = threading.Timer(0.3, lambda: (d / "gpu_busy_percent").write_text("2\n"))
    t.start()
    t0 = time.time()
    gate = bench.wait_for_idle(d, timeout_s=5.0, hold_s=0.3, poll_s=0.05)
    t.join()
    assert gate["idle"] and time.time() - t0 >= 0.6


def test_idle_gate_without_a_busy_counter(bench, tmp_path):
    gate = bench.wait_for_idle(_fake_sysfs(tmp_path, None), timeout_s=1.0, hold_s=0.2, poll_s=0.05)
    assert gate["idle"] and not gate["measurable"] and "note" in gate


def test_previous_record_is_the_newest_driver_record(bench):
    name, rec = bench.previous_record()
    records = sorted(ROOT.glob("BENCH_r*.json"))
    if not records:
        assert (name, rec) == (None, None)
        return
    newest = max(records, key=lambda p: int(p.stem[len("BENCH_r"):]))
    assert name == newest.name
    data = json.loads(newest.read_text())
    assert rec == data.get("parsed", data)


def test_committed_ranges_cover_the_bench_configs(bench):
    label, ranges = bench.committed_ranges()
    assert label is not None
    for key in ("c2", "c3", "c4", "c5", "c3:causal", "c4:causal"):
        lo, hi = ranges[key]
        assert 0 < lo <= hi


def test_bench_refuses_more_than_one_gpu():
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 2
    assert "one GPU only" in out.stderr

"""bench.py's host-side contract (no GPU needed): the one-GPU scope message,
and the GPU-state monitor's child process ending cleanly on any host."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one MI355X" in r.stderr and "out of scope" in r.stderr
    assert r.stdout == ""


def test_device_monitor_child_reports_and_exits():
    sys.path.insert(0, ROOT)
    import bench
    m = bench.DeviceMonitor()
    if m.p is None:          # not startable here (e.g. under a profiler)
        return
    # never started: the child reports without sampling and exits
    out = m.stop()
    assert isinstance(out, dict) and out["samples"] == 0
    assert m.p.returncode == 0
    json.dumps(out)


def test_device_monitor_disabled():
    sys.path.insert(0, ROOT)
    import bench
    m = bench.DeviceMonitor(enabled=False)
    assert m.p is None and m.stop() is None

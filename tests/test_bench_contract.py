"""bench.py's contract, on the CPU: --gpus above 1 exits with a message and no JSON line, and a config-1 run on the
stand-in device (tests/fake_device.py) prints one line with every field the driver reads, the roofline and the HIP
graph replay included."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

import fake_device
from anvil_mi355x import runtime as rt

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_exits_with_a_message():
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 2 and "one MI355X" in out.stderr and not out.stdout.strip()


def test_block_line_has_the_contract_fields(monkeypatch, capsys):
    sys.path.insert(0, str(ROOT))
    import bench
    dev = fake_device.FakeDevice()
    dev.elapsed_ms = lambda a, b: 0.01                   # the stand-in's events: 10 us a timed span
    monkeypatch.setattr(rt, "device", lambda index=0: dev)
    monkeypatch.setattr(bench, "stream_copy", lambda d: {"GBs": None, "peak": bench.PEAK_HBM_GBS})
    monkeypatch.setattr(sys, "argv", ["bench.py", "--config", "1", "--steps", "3", "--warmup", "1",
                                      "--no-cpu-baseline"])
    bench.main()
    lines = [ln for ln in capsys.readouterr().out.splitlines() if ln.startswith("{")]
    assert len(lines) == 1
    d = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline", "hip_graph", "end_to_end", "kernels"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1 and d["higher_is_better"] is True
    assert d["config"]["workload"].startswith("config1")
    r = d["roofline"]
    assert r["bound"] in ("mfma", "hbm") and r["unit"] in ("TOPS", "GB/s") and "frac" in r and "traffic" in r
    assert d["hip_graph"]["steps"] == 3 and dev.captures == 1

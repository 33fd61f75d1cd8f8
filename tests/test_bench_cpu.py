"""bench.py's CPU baseline on the host (no GPU): the cpu-eigen restatement
and the reference's "cpu" device legs are both timed for the MLP configs, and
the oracle is left in its default (cpu-eigen) mode afterwards."""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

import bench  # noqa: E402


def test_cpu_baseline_times_both_reference_devices(oracle):
    r = bench.cpu_baseline(1, 0.4)
    devices = [leg["device"] for leg in r["legs"]]
    assert devices[0] == "cpu-eigen" and "cpu" in devices, devices
    assert r["value"] == r["legs"][0]["samples_per_s"] > 0
    assert all(leg["samples_per_s"] > 0 and leg["steps"] >= 1 for leg in r["legs"])
    assert "\"cpu\" device" in r["sample"]
    assert oracle.cnref_get_cpu_loops() == 0

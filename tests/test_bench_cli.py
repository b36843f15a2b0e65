"""bench.py's command line on the host: the one-GPU contract and the paired mode's workloads."""

import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err


@pytest.mark.parametrize("key", ["c1", "c2", "c3", "c4", "c5a", "c5b", "c5c", "conv"])
def test_paired_workloads_have_a_reference_point(key):
    # --vs-vendor times WORKLOADS[key] against WORKLOADS["vendor_" + key]
    assert key in bench.WORKLOADS and f"vendor_{key}" in bench.WORKLOADS


def test_paired_mode_needs_a_device_or_a_reference_point(capsys):
    # without a device the run stops before any timing; with one, a workload without a
    # vendor_ reference point is refused
    assert bench.main(["--workload", "copy", "--vs-vendor"]) == 2
    err = capsys.readouterr().err
    assert "no ROCm device" in err or "reference point" in err

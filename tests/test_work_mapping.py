"""CPU: the kernels' workgroup -> work item mappings (kerneldev_amd/csrc/kd_work.h,
compiled for the host by tests/host/work_mapping.cpp) are bijections that keep
each XCD on its own range of items, and the forward's takes a range that
splits a head in rank-major order."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_work_mappings_on_the_host(tmp_path):
    exe = tmp_path / "work_mapping"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", os.path.join(HERE, "host", "work_mapping.cpp"),
                    "-o", str(exe)], check=True, capture_output=True, text=True, timeout=120)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout
    assert r.stdout.strip().endswith("failures 0"), r.stdout

"""GPU: the C ABI from a C program (tests/c_abi/attn_from_c.c), without Python
or torch in the calling process: plan, forward and fused backward through
include/kdattn.h, checked inside the program against its own double-precision
causal attention (per-element bar as the Python parity tests); then again with
fp8 e4m3 scores from kd_absmax and kd_quant_fp8, against the same attention
with the decoded e4m3 scores."""
import os
import subprocess

import pytest

from kerneldev_amd.build import C_ABI_BIN

pytestmark = pytest.mark.gpu


def test_c_program_calls_the_library():
    assert os.path.exists(C_ABI_BIN), "build first: python __graft_entry__.py build"
    print(f"running {C_ABI_BIN}", flush=True)
    r = subprocess.run([C_ABI_BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and "c abi ok" in r.stdout and "fp8 scores dK" in r.stdout

"""The namespace-qwen C++ layer as the reference's layer code sees it.

qwen-3.5-cuda_amd/bin/dropin_check (built from tests/dropin_check.cpp by
`make -C qwen-3.5-cuda_amd check`) is compiled against include/*.hpp together
with the forward declarations the reference's layer files make, and re-runs the
reference's own host-side checks (tests/kernel_tests.cu: dequant fixtures, the
RMSNorm closed form, the RoPE fixture) through the C++ API, plus the exception
messages of rope_forward and dequantize_row.
"""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

PKG = Path(__file__).resolve().parent.parent / "qwen-3.5-cuda_amd"
BIN = PKG / "bin" / "dropin_check"


def test_dropin_headers_and_exceptions():
    if not BIN.exists():  # CPU side only: build it here (the GPU box uses the prebuilt binary)
        subprocess.run(["make", "-s", "-C", str(PKG), "check"], check=True)
    r = subprocess.run([str(BIN), "--cpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout


@pytest.mark.gpu
def test_dropin_reference_checks_on_gpu():
    assert BIN.exists(), "build first: make -C qwen-3.5-cuda_amd all check"
    r = subprocess.run([str(BIN), "--gpu"], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout

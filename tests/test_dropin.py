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


REF = Path("/root/reference")
ROOT = PKG.parent
# The reference's callers of the kernel API: the four .cpp files and the headers
# they declare their classes in (include/cuda_utils.hpp:30-87 is what they take
# CUDA_CHECK and CudaContext from).
CALLER_SOURCES = ["src/layer_attn.cpp", "src/layer_gdn.cpp", "src/layer_moe.cpp", "src/model.cpp"]
CALLER_HEADERS = ["include/layer_attn.hpp", "include/layer_gdn.hpp", "include/layer_moe.hpp", "include/model.hpp",
                  "include/config.hpp"]


def _rename_table() -> list[tuple[str, str]]:
    """(reference name, HIP name) pairs of INTEGRATION.md section 2's table."""
    import re

    text = (ROOT / "INTEGRATION.md").read_text()
    sec = text[text.index("| Reference name | HIP name |"):]
    sec = sec[:sec.index("\n\n")]
    pairs = re.findall(r"^\| `([^`]+)` \| `([^`]+)` \|", sec, flags=re.M)
    assert len(pairs) >= 10, pairs
    return pairs


def test_rename_table_names_no_cuda_compat_shim():
    """Every rename maps a CUDA name to a HIP name (none to a CUDA-named alias)."""
    for old, new in _rename_table():
        assert "cuda" in old.lower() or "CUDA" in old
        assert "cuda" not in new.lower()


@pytest.mark.skipif(not (REF / "src/layer_attn.cpp").exists(), reason="reference sources absent (GPU box)")
def test_reference_callers_link_after_renames(tmp_path):
    """The reference's layer files and model.cpp, with only INTEGRATION.md's renames
    applied (to temporary copies), compile against include/ and link with
    --no-undefined against libqwen35_hip.so: the rename list is complete and every
    kernel, matmul_dispatch, dequantize_row and GgufLoader symbol they call is
    exported with the reference's signature. Nothing is run."""
    lib = PKG / "libqwen35_hip.so"
    if not lib.exists():
        subprocess.run(["make", "-s", "-C", str(PKG), "all"], check=True)
    pairs = _rename_table()
    (tmp_path / "src").mkdir()
    (tmp_path / "include").mkdir()
    for rel in CALLER_SOURCES + CALLER_HEADERS:
        text = (REF / rel).read_text()
        for old, new in pairs:
            text = text.replace(old, new)
        (tmp_path / rel).write_text(text)
    import re

    for rel in CALLER_SOURCES + CALLER_HEADERS:
        code = "\n".join(line.split("//")[0] for line in (tmp_path / rel).read_text().splitlines())
        left = set(re.findall(r"\b(?:cuda|Cuda|CUDA|cublas|CUBLAS)\w*", code))
        assert not left, f"{rel}: CUDA names left after the renames: {sorted(left)}"
    hipcc = "/opt/rocm/bin/hipcc"
    objs = []
    for rel in CALLER_SOURCES:
        obj = tmp_path / (Path(rel).stem + ".o")
        r = subprocess.run([hipcc, "-std=c++17", "-fPIC", "-c", f"-I{ROOT / 'include'}", f"-I{tmp_path / 'include'}",
                            str(tmp_path / rel), "-o", str(obj)], capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, f"{rel}:\n{r.stderr[-3000:]}"
        objs.append(str(obj))
    r = subprocess.run([hipcc, "-shared", "-fPIC", "-o", str(tmp_path / "liblayers.so"), *objs, f"-L{PKG}",
                        "-lqwen35_hip", "-Wl,--no-undefined"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]

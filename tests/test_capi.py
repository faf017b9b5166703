"""C ABI checks that need no GPU: the library loads, exports every function the
header declares, and rejects bad arguments on the host before any launch (the
reference's throw conditions, src/cuda/rope.cu:33-43 and
src/cuda/matmul_q4.cu:210-217, map to status codes). Zero-size calls return OK
without touching the device.
"""

from __future__ import annotations

import ctypes
import subprocess

import pytest

from qwen35_hip import _lib

NULL = None
ST = None  # default stream; never reached by these calls


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def msg(lib) -> str:
    return lib.qwen_last_error().decode()


def test_exports_every_declared_function(lib):
    declared = _lib.header_functions()
    assert len(declared) >= 27
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [f for f in declared if f not in exported]
    assert not missing, missing
    assert set(declared) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_cxx_dropin_symbols_exported():
    out = subprocess.run(["nm", "-DC", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    for sig in [
        "qwen::rmsnorm_forward(float const*, float const*, float*, int, float, ihipStream_t*)",
        "qwen::rmsnorm_gated_forward(float const*, float const*, float const*, float*, int, float, ihipStream_t*)",
        "qwen::residual_add(float const*, float const*, float*, int, ihipStream_t*)",
        "qwen::encoder_forward(int, float const*, float*, int, ihipStream_t*)",
        "qwen::rope_forward(float*, int, int, int, int, float, ihipStream_t*)",
        "qwen::attn_head_norm(float*, float const*, int, int, float, ihipStream_t*)",
        "qwen::gdn_conv_step(float const*, float const*, float*, float*, int, int, ihipStream_t*)",
        "qwen::gdn_qk_normalize(float*, float*, int, int, float, ihipStream_t*)",
        "qwen::gdn_norm_gate(float const*, float const*, float const*, float*, int, int, float, ihipStream_t*)",
        "qwen::moe_silu_mul(float const*, float const*, float*, int, ihipStream_t*)",
        "qwen::moe_shared_add(float*, float const*, float const*, int, ihipStream_t*)",
        "qwen::dequantize_row(qwen::QuantTensor const&, float*, int, int, ihipStream_t*)",
        "qwen::matmul_type_supported(qwen::GgmlType)",
    ]:
        assert sig in out, sig


def test_status_names(lib):
    assert lib.qwen_abi_version() == 2
    names = [lib.qwen_status_name(i).decode() for i in range(5)]
    assert names == ["QWEN_STATUS_OK", "QWEN_STATUS_INVALID_ARGUMENT", "QWEN_STATUS_UNSUPPORTED_TYPE",
                     "QWEN_STATUS_OUT_OF_RANGE", "QWEN_STATUS_LAUNCH_FAILED"]


FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails validation first


@pytest.mark.parametrize("args", [
    (NULL, 3, 2, 8, 4, 100.0),        # null pointer
    (FAKE, -1, 2, 8, 4, 100.0),       # negative position
    (FAKE, 3, 0, 8, 4, 100.0),        # no heads
    (FAKE, 3, 2, 0, 4, 100.0),        # head_dim 0
    (FAKE, 3, 2, 8, 0, 100.0),        # rope_dim 0
    (FAKE, 3, 2, 8, 10, 100.0),       # rope_dim > head_dim
    (FAKE, 3, 2, 8, 3, 100.0),        # odd rope_dim
    (FAKE, 3, 2, 4096, 2050, 100.0),  # rope_dim / 2 > 1024
    (FAKE, 3, 2, 8, 4, 0.0),          # theta <= 0
    (FAKE, 3, 2, 8, 4, float("nan")),  # theta not > 0
])
def test_rope_rejects_reference_conditions(lib, args):
    assert lib.qwen_rope_forward(*args, ST) == _lib.STATUS_INVALID_ARGUMENT
    assert msg(lib) == "invalid RoPE arguments"


def test_dequantize_row_errors(lib):
    Q4_K, Q4_1 = 12, 3
    assert lib.qwen_dequantize_row(NULL, Q4_K, 256, FAKE, 0, 256, ST) == _lib.STATUS_UNSUPPORTED_TYPE
    assert msg(lib) == "cannot dequantize tensor"
    assert lib.qwen_dequantize_row(FAKE, Q4_1, 256, FAKE, 0, 256, ST) == _lib.STATUS_UNSUPPORTED_TYPE
    for row, cols, n in [(-1, 256, 512), (0, 0, 512), (0, -5, 512), (1, 256, 256), (2, 256, 767)]:
        assert lib.qwen_dequantize_row(FAKE, Q4_K, n, FAKE, row, cols, ST) == _lib.STATUS_OUT_OF_RANGE
        assert msg(lib) == "row is outside tensor"
    assert lib.qwen_dequantize_row(FAKE, Q4_K, 512, NULL, 1, 256, ST) == _lib.STATUS_INVALID_ARGUMENT
    assert lib.qwen_dequant_gather_rows(FAKE, 3, 512, FAKE, 1, 256, FAKE, ST) == _lib.STATUS_UNSUPPORTED_TYPE
    assert lib.qwen_dequant_gather_rows(FAKE, Q4_K, 512, FAKE, -1, 256, FAKE, ST) == _lib.STATUS_INVALID_ARGUMENT
    assert lib.qwen_dequant_gather_rows(FAKE, Q4_K, 512, NULL, 4, 256, FAKE, ST) == _lib.STATUS_INVALID_ARGUMENT
    assert lib.qwen_dequant_gather_rows(FAKE, Q4_K, 512, FAKE, 0, 256, FAKE, ST) == _lib.STATUS_OK


def test_type_supported(lib):
    for t in range(40):
        assert lib.qwen_type_supported(t) == (1 if t in (0, 1, 2, 6, 8, 12, 13, 14, 30) else 0)


def test_size_and_pointer_validation(lib):
    INV, OK = _lib.STATUS_INVALID_ARGUMENT, _lib.STATUS_OK
    assert lib.qwen_rmsnorm_rows(FAKE, FAKE, FAKE, -1, 8, 1e-6, ST) == INV
    assert lib.qwen_rmsnorm_rows(NULL, FAKE, FAKE, 2, 8, 1e-6, ST) == INV
    assert lib.qwen_rmsnorm_rows(NULL, NULL, NULL, 0, 8, 1e-6, ST) == OK  # nothing to do
    assert lib.qwen_rmsnorm_forward(NULL, NULL, NULL, 0, 1e-6, ST) == OK
    assert lib.qwen_rmsnorm_gated_rows(FAKE, NULL, FAKE, FAKE, 1, 8, 1e-6, ST) == INV
    assert lib.qwen_residual_add(FAKE, FAKE, FAKE, -4, ST) == INV
    assert lib.qwen_residual_rmsnorm_rows_bf16(FAKE, FAKE, NULL, FAKE, FAKE, 1, 8, 1e-6, ST) == INV
    assert lib.qwen_encoder_forward(-1, FAKE, FAKE, 16, ST) == INV
    assert lib.qwen_attn_head_norm(NULL, FAKE, 2, 8, 1e-6, ST) == INV
    assert lib.qwen_attn_qk_norm_rope_rows(FAKE, FAKE, FAKE, FAKE, NULL, 0, 4, 2, 1, 8, 10, 1e7, 1e-6, ST) == INV
    assert lib.qwen_attn_qk_norm_rope_rows(FAKE, FAKE, FAKE, FAKE, NULL, -1, 4, 2, 1, 8, 4, 1e7, 1e-6, ST) == INV
    assert lib.qwen_attn_qk_norm_rope_rows(FAKE, NULL, FAKE, NULL, NULL, 0, 4, 2, 1, 8, 4, 1e7, 1e-6, ST) == INV
    assert lib.qwen_attn_qk_norm_rope_rows(FAKE, FAKE, FAKE, FAKE, NULL, 0, 4, 2, 1, 8, 4, 0.0, 1e-6, ST) == INV
    assert lib.qwen_gdn_frontend_rows(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 64, 1, 0, 0, 1e-6, ST) == INV
    assert lib.qwen_gdn_frontend_rows(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 64, 4, 1, 64, 1e-6, ST) == INV
    assert lib.qwen_gdn_frontend_rows(FAKE, FAKE, NULL, FAKE, FAKE, 4, 64, 4, 0, 0, 1e-6, ST) == INV
    assert lib.qwen_gdn_qk_normalize(FAKE, NULL, 2, 8, 1e-6, ST) == INV
    assert lib.qwen_gdn_norm_gate_rows(FAKE, FAKE, FAKE, FAKE, 1, -2, 8, 1e-6, ST) == INV
    assert lib.qwen_moe_silu_mul(FAKE, NULL, FAKE, 8, ST) == INV
    assert lib.qwen_moe_shared_add_rows(FAKE, FAKE, FAKE, 70000, 8, ST) == INV
    assert lib.qwen_swiglu_bf16(FAKE, FAKE, FAKE, -1, ST) == INV
    assert lib.qwen_shared_swiglu_sigmoid_rows_bf16(FAKE, FAKE, NULL, FAKE, 2, 8, ST) == INV
    assert "null" in msg(lib)


def test_matmul_rows_host_validation(lib):
    """matmul_rows / matmul_rows_multi reject bad arguments on the host, in
    matmul_dispatch's order (src/cuda/matmul_q4.cu:187-195), before any launch;
    the workspace size is the prep layout (exponents, group sums, fp16 parts)."""
    INV, OK = _lib.STATUS_INVALID_ARGUMENT, _lib.STATUS_OK
    UNS, OOR = _lib.STATUS_UNSUPPORTED_TYPE, _lib.STATUS_OUT_OF_RANGE
    q4 = 12
    assert lib.qwen_matmul_rows(NULL, q4, 4096, FAKE, FAKE, 32, 16, 256, 0, NULL, 0, ST) == INV
    assert "not loaded" in msg(lib)
    assert lib.qwen_matmul_rows(FAKE, 3, 4096, FAKE, FAKE, 32, 16, 256, 0, NULL, 0, ST) == UNS
    assert lib.qwen_matmul_rows(FAKE, q4, 4096, FAKE, FAKE, 32, 17, 256, 0, NULL, 0, ST) == OOR
    assert lib.qwen_matmul_rows(FAKE, q4, 4096, FAKE, FAKE, 32, 16, 256, 256, NULL, 0, ST) == OOR
    assert lib.qwen_matmul_rows(FAKE, q4, 4096, FAKE, FAKE, -1, 16, 256, 0, NULL, 0, ST) == INV
    assert lib.qwen_matmul_rows(FAKE, q4, 4096, NULL, NULL, 0, 16, 256, 0, NULL, 0, ST) == OK
    # the matrix-core path needs its workspace: checked before the prep launch
    aligned = 1 << 20
    assert lib.qwen_matmul_rows(FAKE, q4, 4096, aligned, aligned, 32, 16, 256, 0, NULL, 0, ST) == INV
    assert "workspace" in msg(lib)
    assert lib.qwen_matmul_rows_workspace_bytes(15, 2048) == 0
    assert lib.qwen_matmul_rows_workspace_bytes(64, 300) == 0
    # 64 tokens x 2048: 256 B of exponents, 64 x 64 sums, 64 x 2048 x 2 halves
    assert lib.qwen_matmul_rows_workspace_bytes(64, 2048) == 256 + 64 * 64 * 4 + 64 * 2048 * 4
    assert lib.qwen_matmul_rows_multi(NULL, 65, FAKE, 32, 256, NULL, 0, ST) == INV
    assert lib.qwen_matmul_rows_multi(NULL, 0, NULL, 32, 256, NULL, 0, ST) == OK


def test_gdn_chunked_workspace_bytes(lib):
    """Per 64-token chunk and value head: T' and Bm (64 x 64 fp32 each), gamma and
    R[C-1][.] (64 fp32 each) and 4 scalars; then the chunk's K and Q of one key head
    as fp16 pairs (64 tokens x 128 dims x hi/lo x 2 bytes each), sized per value
    head (key heads read by some value head are at most the value heads)."""
    per_head = (2 * 64 * 64 + 2 * 64 + 4) * 4 + 2 * 64 * 128 * 2 * 2
    f = lib.qwen_gdn_recurrent_chunked_workspace_bytes
    assert f(0, 32) == 0 and f(16, 0) == 0 and f(-1, 32) == 0
    assert f(1, 32) == 32 * per_head
    assert f(64, 2) == 2 * per_head and f(65, 2) == 2 * 2 * per_head
    assert f(4096, 32) == 64 * 32 * per_head   # 202 MB at the Qwen3.5 GDN shape
    assert f(4096, 32) % 16 == 0 and (2 * 64 * 64 + 2 * 64 + 4) * 4 % 16 == 0   # the pairs region stays 16-byte aligned


def test_gdn_value_dim_limit_on_every_recurrent_path(lib):
    """value_dim above 256 is rejected with the reference's message
    (src/cuda/gdn.cu:167-169) by the token loop and by the chunked entry point
    whatever the pointers' alignment (which would otherwise pick the path)."""
    INV = _lib.STATUS_INVALID_ARGUMENT
    aligned, odd = ctypes.c_void_p(1 << 20), ctypes.c_void_p((1 << 20) + 4)
    for p in (aligned, odd):
        st = lib.qwen_gdn_recurrent_chunked(p, p, p, p, p, p, p, 64, 16, 32, 128, 512, 8192, 4096, p, 1 << 30, ST)
        assert st == INV and msg(lib) == "GDN value dimension exceeds kernel limit"
    assert lib.qwen_gdn_recurrent_rows(aligned, aligned, aligned, aligned, aligned, aligned, aligned, 4, 16, 32, 128,
                                       512, 8192, 4096, ST) == INV
    assert msg(lib) == "GDN value dimension exceeds kernel limit"


def test_swiglu_routed_shared_validation(lib):
    INV, OK = _lib.STATUS_INVALID_ARGUMENT, _lib.STATUS_OK
    f = lib.qwen_swiglu_routed_shared_bf16
    assert f(FAKE, FAKE, FAKE, -8, FAKE, FAKE, FAKE, FAKE, 1, 8, ST) == INV
    assert f(FAKE, FAKE, FAKE, 8, FAKE, FAKE, FAKE, FAKE, -1, 8, ST) == INV
    assert f(NULL, FAKE, FAKE, 8, FAKE, FAKE, FAKE, FAKE, 1, 8, ST) == INV and "routed" in msg(lib)
    assert f(FAKE, FAKE, FAKE, 8, FAKE, FAKE, NULL, FAKE, 1, 8, ST) == INV and "shared" in msg(lib)
    assert f(NULL, NULL, NULL, 0, NULL, NULL, NULL, NULL, 0, 512, ST) == OK  # both parts empty


def test_attn_decode_noalloc_host_validation(lib):
    """Shape, pointer and scratch-size checks come before any device call."""
    INV = _lib.STATUS_INVALID_ARGUMENT
    f = lib.qwen_attn_decode_noalloc
    assert lib.qwen_attn_decode_noalloc_max_scratch_bytes() == 8 << 20
    assert f(FAKE, FAKE, FAKE, NULL, FAKE, 6, 4, 64, 3, ST) == INV  # heads not a multiple of kv_heads
    assert f(NULL, FAKE, FAKE, NULL, FAKE, 16, 2, 256, 3, ST) == INV and "null" in msg(lib)
    assert lib.qwen_attn_decode_workspace_bytes(64, 8, 256, 19999) > 8 << 20
    assert f(FAKE, FAKE, FAKE, NULL, FAKE, 64, 8, 256, 19999, ST) == INV and "scratch" in msg(lib)


def test_gdn_norm_gate_matmul_host_validation(lib):
    """The fused gated norm + output projection rejects what either call would
    (sizes, null pointers, a shape past the tensor, an unloaded tensor) before any
    launch."""
    INV, OOR = _lib.STATUS_INVALID_ARGUMENT, _lib.STATUS_OUT_OF_RANGE
    p = ctypes.c_void_p(1 << 20)
    assert lib.qwen_gdn_norm_gate_matmul(p, p, p, p, 0, 128, 1e-6, p, 12, 1 << 20, p, 8, 0, ST) == INV
    assert "bad heads" in msg(lib)
    assert lib.qwen_gdn_norm_gate_matmul(p, NULL, p, p, 32, 128, 1e-6, p, 12, 1 << 20, p, 8, 0, ST) == INV
    assert "null pointer" in msg(lib)
    assert lib.qwen_gdn_norm_gate_matmul(p, p, p, p, 32, 128, 1e-6, NULL, 12, 1 << 20, p, 8, 0, ST) == INV
    assert msg(lib) == "tensor is not loaded"
    # 2048 rows x 4096 inputs need 8 Mi elements
    assert lib.qwen_gdn_norm_gate_matmul(p, p, p, p, 32, 128, 1e-6, p, 12, 4096 * 2047, p, 2048, 0, ST) == OOR
    assert "GEMV shape exceeds tensor" in msg(lib)


def test_attn_decode_norm_rope_host_validation(lib):
    """The folded attention decode rejects bad shapes, null pointers, a partly
    overlapping q_normed and a short workspace before any launch."""
    INV = _lib.STATUS_INVALID_ARGUMENT
    p = ctypes.c_void_p(1 << 20)
    big = 1 << 30
    assert lib.qwen_attn_decode_norm_rope(p, ctypes.c_void_p((1 << 20) + 4096), p, p, NULL, p, 16, 3, 256, 10, p, p,
                                          64, 1e7, 1e-6, p, big, ST) == INV
    assert "not a multiple" in msg(lib)
    assert lib.qwen_attn_decode_norm_rope(p, ctypes.c_void_p((1 << 20) + 65536), p, p, NULL, p, 16, 2, 256, 10, NULL,
                                          p, 64, 1e7, 1e-6, p, big, ST) == INV
    assert "null pointer" in msg(lib)
    assert lib.qwen_attn_decode_norm_rope(p, ctypes.c_void_p((1 << 20) + 64), p, p, NULL, p, 16, 2, 256, 10, p, p,
                                          64, 1e7, 1e-6, p, big, ST) == INV
    assert "overlaps q" in msg(lib)
    assert lib.qwen_attn_decode_norm_rope(p, p, p, p, NULL, p, 16, 2, 256, 10, p, p, 65, 1e7, 1e-6, p, big, ST) == INV
    assert "rope_dim" in msg(lib)
    assert lib.qwen_attn_decode_norm_rope(p, p, p, p, NULL, p, 16, 2, 256, 10, p, p, 64, 1e7, 1e-6, p, 16, ST) == INV
    assert "workspace" in msg(lib)

"""ctypes view of libqwen35_hip.so (the C ABI declared in include/qwen35_hip.h and
include/qwen35_gguf.h).

The library is built in-tree by the package Makefile. Loading fails loudly when
it is missing: there is no fallback implementation.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent.parent
# The in-tree build; QWEN35_HIP_LIB names another build of the same library.
LIB_PATH = Path(os.environ.get("QWEN35_HIP_LIB") or PACKAGE_DIR / "libqwen35_hip.so")

STATUS_OK = 0
STATUS_INVALID_ARGUMENT = 1
STATUS_UNSUPPORTED_TYPE = 2
STATUS_OUT_OF_RANGE = 3
STATUS_LAUNCH_FAILED = 4
STATUS_IO_ERROR = 5
STATUS_MALFORMED = 6
STATUS_OUT_OF_MEMORY = 7

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64

# name -> argument types (all functions return int unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "qwen_abi_version": [],
    "qwen_last_error": [],
    "qwen_status_name": [_I],
    "qwen_rmsnorm_forward": [_P, _P, _P, _I, _F, _P],
    "qwen_rmsnorm_rows": [_P, _P, _P, _I, _I, _F, _P],
    "qwen_rmsnorm_gated_forward": [_P, _P, _P, _P, _I, _F, _P],
    "qwen_rmsnorm_gated_rows": [_P, _P, _P, _P, _I, _I, _F, _P],
    "qwen_residual_add": [_P, _P, _P, _I, _P],
    "qwen_residual_rmsnorm_rows_f32": [_P, _P, _P, _P, _P, _I, _I, _F, _P],
    "qwen_residual_rmsnorm_rows_bf16": [_P, _P, _P, _P, _P, _I, _I, _F, _P],
    "qwen_encoder_forward": [_I, _P, _P, _I, _P],
    "qwen_attn_head_norm": [_P, _P, _I, _I, _F, _P],
    "qwen_rope_forward": [_P, _I, _I, _I, _I, _F, _P],
    "qwen_attn_qk_norm_rope_rows": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _F, _P],
    "qwen_gdn_conv_step": [_P, _P, _P, _P, _I, _I, _P],
    "qwen_gdn_qk_normalize": [_P, _P, _I, _I, _F, _P],
    "qwen_gdn_frontend_rows": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P],
    "qwen_gdn_norm_gate": [_P, _P, _P, _P, _I, _I, _F, _P],
    "qwen_gdn_norm_gate_rows": [_P, _P, _P, _P, _I, _I, _I, _F, _P],
    "qwen_gdn_norm_gate_matmul": [_P, _P, _P, _P, _I, _I, _F, _P, _I, _U64, _P, _I, _U64, _P],
    "qwen_moe_silu_mul": [_P, _P, _P, _I, _P],
    "qwen_moe_shared_add": [_P, _P, _P, _I, _P],
    "qwen_moe_shared_add_rows": [_P, _P, _P, _I, _I, _P],
    "qwen_swiglu_bf16": [_P, _P, _P, _I64, _P],
    "qwen_shared_swiglu_sigmoid_rows_bf16": [_P, _P, _P, _P, _I, _I, _P],
    "qwen_swiglu_routed_shared_bf16": [_P, _P, _P, _I64, _P, _P, _P, _P, _I, _I, _P],
    "qwen_type_supported": [_I],
    "qwen_dequantize_row": [_P, _I, _U64, _P, _I, _I, _P],
    "qwen_dequant_gather_rows": [_P, _I, _U64, _P, _I, _I, _P, _P],
    "qwen_gdn_gate_values": [_P] * 6 + [_I, _P],
    "qwen_gdn_gate_values_rows": [_P] * 6 + [_I, _I, _P],
    "qwen_gdn_recurrent_step": [_P] * 7 + [_I, _I, _I, _I, _P],
    "qwen_gdn_recurrent_rows": [_P] * 7 + [_I, _I, _I, _I, _I, _I64, _I64, _P],
    "qwen_gdn_gated_recurrent_rows": [_P] * 9 + [_I, _I, _I, _I, _I, _I64, _I64, _P],
    "qwen_gdn_recurrent_chunked_workspace_bytes": [_I, _I],
    "qwen_gdn_recurrent_chunked": [_P] * 7 + [_I, _I, _I, _I, _I, _I64, _I64, _P, ctypes.c_size_t, _P],
    "qwen_attn_split_qg": [_P, _P, _P, _I, _I, _P],
    "qwen_attn_scores": [_P, _P, _P, _I, _I, _I, _I, _P],
    "qwen_attn_softmax": [_P, _I, _I, _P],
    "qwen_attn_values": [_P, _P, _P, _I, _I, _I, _I, _P],
    "qwen_attn_sigmoid_gate": [_P, _P, _P, _I, _P],
    "qwen_attn_kv_store": [_P, _P, _P, _P, _I, _I, _I, _P],
    "qwen_attn_decode_workspace_bytes": [_I, _I, _I, _I],
    "qwen_attn_decode": [_P] * 5 + [_I, _I, _I, _I, _P, ctypes.c_size_t, _P],
    "qwen_attn_decode_norm_rope": [_P] * 6 + [_I, _I, _I, _I, _P, _P, _I, _F, _F, _P, ctypes.c_size_t, _P],
    "qwen_attn_decode_noalloc_max_scratch_bytes": [],
    "qwen_attn_decode_noalloc": [_P] * 5 + [_I, _I, _I, _I, _P],
    "qwen_moe_topk": [_P, _P, _P, _I, _I, _P],
    "qwen_moe_topk_rows": [_P, _P, _P, _I, _I, _I, _P],
    "qwen_moe_add": [_P, _P, _F, _I, _P],
    "qwen_moe_weighted_sum_rows": [_P, _P, _P, _I, _I, _I, _P],
    "qwen_moe_expert_matmul": [_P, _I, _U64, _U64, _I, _P, _I, _P, _I64, _P, _I, _I, _P],
    "qwen_gdn_decode_step": [_P] * 11 + [_I, _I, _I, _I, _I, _F, _P],
    "qwen_moe_expert_gate_up": [_P, _P, _I, _U64, _U64, _I, _P, _I, _P, _P, _P, _I, _I, _P],
    "qwen_moe_expert_swiglu_workspace_bytes": [_I, _I, _I],
    "qwen_moe_expert_swiglu": [_P, _P, _I, _U64, _U64, _I, _P, _I, _I, _P, _P, _I, _U64, _I, _P, _I, _P, _P, _P,
                               ctypes.c_size_t, _P],
    "qwen_moe_route_swiglu": [_P, _P, _P, _I, _P, _P, _I, _U64, _U64, _I, _I, _P, _P, _I, _U64, _I, _P, _I, _P, _P,
                              _P, ctypes.c_size_t, _P],
    "qwen_moe_down_combine_workspace_bytes": [_I, _I],
    "qwen_moe_down_combine": [_P, _I, _U64, _U64, _I, _P, _P, _I, _P, _I, _P, _I, _U64, _P, _I, _P, _P, _I,
                              _P, ctypes.c_size_t, _P],
    "qwen_matmul_type_supported": [_I],
    "qwen_matmul_dispatch": [_P, _I, _U64, _P, _P, _I, _I, _U64, _P],
    "qwen_matmul_dispatch_multi": [_P, _I, _P, _I, _P],
    "qwen_matmul_rows": [_P, _I, _U64, _P, _P, _I, _I, _I, _U64, _P, ctypes.c_size_t, _P],
    "qwen_matmul_rows_workspace_bytes": [_I, _I],
    "qwen_matmul_rows_multi": [_P, _I, _P, _I, _I, _P, ctypes.c_size_t, _P],
    # GGUF loader (include/qwen35_gguf.h)
    "qwen_gguf_open": [ctypes.c_char_p, _P],
    "qwen_gguf_close": [_P],
    "qwen_gguf_get_info": [_P, _P],
    "qwen_gguf_get_tensor": [_P, _U64, _P],
    "qwen_gguf_find_tensor": [_P, ctypes.c_char_p, _P],
    "qwen_gguf_get_meta": [_P, ctypes.c_char_p, _P],
    "qwen_gguf_get_meta_array_size": [_P, ctypes.c_char_p, _P],
    "qwen_gguf_get_meta_array_item": [_P, ctypes.c_char_p, _U64, _P],
    "qwen_gguf_get_meta_key": [_P, _U64, _P, _P],
    "qwen_gguf_load": [_P, _I, _P],
    "qwen_gguf_unload": [_P],
}

_RESTYPES = {"qwen_last_error": ctypes.c_char_p, "qwen_status_name": ctypes.c_char_p,
             "qwen_attn_decode_workspace_bytes": ctypes.c_size_t,
             "qwen_attn_decode_noalloc_max_scratch_bytes": ctypes.c_size_t,
             "qwen_matmul_rows_workspace_bytes": ctypes.c_size_t,
             "qwen_gdn_recurrent_chunked_workspace_bytes": ctypes.c_size_t,
             "qwen_moe_down_combine_workspace_bytes": ctypes.c_size_t,
             "qwen_moe_expert_swiglu_workspace_bytes": ctypes.c_size_t}

_lib = None


def header_functions(header: Path | None = None) -> list[str]:
    """Names of the functions the C headers (include/*.h) declare (for export checks)."""
    import re

    headers = [header] if header else sorted((PACKAGE_DIR.parent / "include").glob("*.h"))
    text = "\n".join(h.read_text() for h in headers)
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(qwen_\w+)\s*\(", text, flags=re.M)))


def load(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Load the library once and attach the C signatures. Raises if it is absent."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is missing: build it with `make -C {PACKAGE_DIR}` (or __graft_entry__.build()); "
            "the kernels have no non-HIP implementation"
        )
    lib = ctypes.CDLL(str(p))
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPES.get(name, ctypes.c_int)
    if path is None:
        _lib = lib
    return lib


class QwenError(RuntimeError):
    """A C entry point returned a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status})")
        self.status = status
        self.message = message


def check(status: int) -> None:
    if status != STATUS_OK:
        raise QwenError(status, load().qwen_last_error().decode())

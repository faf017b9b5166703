"""MI355X (gfx950) fused per-layer kernels of the Qwen3.5 hybrid-MoE decoder.

`qwen35_hip.ops` exposes every C entry point of include/qwen35_hip.h on torch
device tensors; `qwen35_hip.synth` builds the deterministic synthetic inputs of
the benchmark configurations.
"""

from ._lib import LIB_PATH, PACKAGE_DIR, QwenError, load  # noqa: F401

__all__ = ["LIB_PATH", "PACKAGE_DIR", "QwenError", "load"]

"""Shared test setup: import paths, the `gpu` marker and the parity metrics.

Parity bars (from the task's north star):
  * integer/byte work (dequant-gather): bit-exact, compared on raw float bits;
  * fp32 outputs: |got - ref| <= 1e-5 * max(|ref|, rms(ref over its row or head)).
    The rms floor applies only where an output is a cancelling sum (a RoPE
    rotation, a conv sum near zero); for a product of factors |ref| dominates;
  * bf16 outputs: at most 1 unit in the last place of bf16 apart.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "qwen-3.5-cuda_amd"))
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "tests"))

RTOL_F32 = 1e-5
MAX_BF16_ULP = 1


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs with -m gpu on the GPU box)")


def rel_err(got: np.ndarray, ref: np.ndarray, group: int | None = None) -> np.ndarray:
    """|got - ref| / max(|ref|, rms(ref over the last `group` elements))."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.abs(ref)
    if group:
        g = ref.reshape(-1, group)
        rms = np.sqrt(np.mean(g * g, axis=1, keepdims=True))
        denom = np.maximum(denom, np.broadcast_to(rms, g.shape).reshape(ref.shape))
    denom = np.where(denom == 0, 1.0, denom)
    return np.abs(got - ref) / denom


def assert_f32_close(got, ref, group: int | None = None, rtol: float = RTOL_F32, what: str = ""):
    got = np.asarray(got, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    assert np.array_equal(nan_g, nan_r), f"{what}: NaN pattern differs"
    ok = ~nan_r
    e = rel_err(np.where(ok, got, 0), np.where(ok, ref, 0), group)
    worst = int(np.argmax(e)) if e.size else 0
    assert e.size == 0 or e.flat[worst] <= rtol, (
        f"{what}: rel err {e.flat[worst]:.3e} > {rtol:g} at {np.unravel_index(worst, e.shape)}: "
        f"got {got.flat[worst]!r} ref {ref.flat[worst]!r}")


def floor_audit(got, ref, group: int, what: str = "") -> dict:
    """How much of an fp32 comparison the rms floor carries: the largest plain
    relative error |got - ref| / |ref|, how many elements exceed RTOL_F32 by that
    measure (they pass only because of the floor), the largest error of those
    measured against the floor, and the largest |ref| / rms among them (so a
    reader can see they are the near-zero outputs of cancelling sums). Printed
    with a fixed prefix so a test log can be searched for it."""
    g = np.asarray(got, dtype=np.float64).reshape(-1, group)
    r = np.asarray(ref, dtype=np.float64).reshape(-1, group)
    ok = ~np.isnan(r)
    err = np.where(ok, np.abs(g - r), 0.0)
    plain = np.where(np.abs(r) > 0, err / np.where(np.abs(r) > 0, np.abs(r), 1.0), np.where(err > 0, np.inf, 0.0))
    rms = np.sqrt(np.mean(np.where(ok, r * r, 0.0), axis=1, keepdims=True))
    rms = np.where(rms == 0, 1.0, rms)
    floor_only = ok & (plain > RTOL_F32)
    rep = {"what": what, "elements": int(r.size), "max_plain_rel_err": float(plain[ok].max()) if ok.any() else 0.0,
           "floor_only": int(floor_only.sum()),
           "floor_only_max_err_over_rms": float((err / rms)[floor_only].max()) if floor_only.any() else 0.0,
           "floor_only_max_abs_ref_over_rms": float((np.abs(r) / rms)[floor_only].max()) if floor_only.any() else 0.0,
           "max_err_over_rms": float((err / rms).max())}
    print(f"FLOOR-AUDIT {rep}", flush=True)
    return rep


def bf16_ordered(bits: np.ndarray) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16).astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def assert_bf16_close(got_bits, ref_bits, max_ulp: int = MAX_BF16_ULP, what: str = ""):
    g = np.asarray(got_bits, dtype=np.uint16)
    r = np.asarray(ref_bits, dtype=np.uint16)
    assert g.shape == r.shape
    nan_g = ((g & 0x7F80) == 0x7F80) & ((g & 0x7F) != 0)
    nan_r = ((r & 0x7F80) == 0x7F80) & ((r & 0x7F) != 0)
    assert np.array_equal(nan_g, nan_r), f"{what}: NaN pattern differs"
    d = np.abs(bf16_ordered(g) - bf16_ordered(r))
    d = np.where(nan_r, 0, d)
    worst = int(np.argmax(d)) if d.size else 0
    assert d.size == 0 or d.flat[worst] <= max_ulp, (
        f"{what}: {d.flat[worst]} bf16 ulp apart at {np.unravel_index(worst, d.shape)}: "
        f"got {g.flat[worst]:#06x} ref {r.flat[worst]:#06x}")


def assert_bits_equal(got, ref, what: str = ""):
    g = np.ascontiguousarray(got, dtype=np.float32).view(np.uint32)
    r = np.ascontiguousarray(ref, dtype=np.float32).view(np.uint32)
    assert g.shape == r.shape
    bad = np.nonzero(g != r)[0] if g.ndim == 1 else np.argwhere(g != r)
    assert len(bad) == 0, (f"{what}: {len(bad)} elements differ, first at {bad[0]}: "
                           f"got {g[tuple(np.atleast_1d(bad[0]))]:#010x} ref {r[tuple(np.atleast_1d(bad[0]))]:#010x}")


@pytest.fixture(scope="session")
def oracle():
    import pyoracle

    pyoracle.build()
    return pyoracle

"""Block dequantizers in the loop form of ggml's dequantize_row_* (llama.cpp
b9222, the GGML formats the reference transcribes per element in
src/cuda/matmul_q4.cu:30-129; ggml itself is not vendored in the reference).

Test infrastructure: an independent restatement used to pin the oracle's
per-element decoder. It walks each block the way ggml does (64-element groups
with scale pairs for Q4_K/Q5_K, 128-element halves with four quarter streams
for Q6_K, explicit high-bit masks for Q5_0), so a wrong index, shift or nibble
order in either form shows up as a mismatch. Arithmetic is float32 with the same
association as ggml: (d * sc) * q - dmin * m.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def _f16(col: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(col).view(np.float16).astype(F32).reshape(-1, 1)


def _scale_min_k4(j: int, s: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    s = s.astype(np.int32)
    if j < 4:
        return (s[:, j] & 63).reshape(-1, 1), (s[:, j + 4] & 63).reshape(-1, 1)
    d = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
    m = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    return d.reshape(-1, 1), m.reshape(-1, 1)


def q4_0(raw: np.ndarray) -> np.ndarray:
    b = raw.reshape(-1, 18)
    d = _f16(b[:, 0:2])
    qs = b[:, 2:18].astype(np.int32)
    y = np.empty((b.shape[0], 32), dtype=F32)
    y[:, :16] = ((qs & 0xF) - 8).astype(F32) * d
    y[:, 16:] = ((qs >> 4) - 8).astype(F32) * d
    return y.reshape(-1)


def q5_0(raw: np.ndarray) -> np.ndarray:
    b = raw.reshape(-1, 22)
    d = _f16(b[:, 0:2])
    qh = np.ascontiguousarray(b[:, 2:6]).view(np.uint32).astype(np.int64).reshape(-1, 1)
    qs = b[:, 6:22].astype(np.int64)
    j = np.arange(16, dtype=np.int64).reshape(1, -1)
    xh0 = ((qh >> j) << 4) & 0x10
    xh1 = (qh >> (j + 12)) & 0x10
    y = np.empty((b.shape[0], 32), dtype=F32)
    y[:, :16] = (((qs & 0x0F) | xh0) - 16).astype(F32) * d
    y[:, 16:] = (((qs >> 4) | xh1) - 16).astype(F32) * d
    return y.reshape(-1)


def q8_0(raw: np.ndarray) -> np.ndarray:
    b = raw.reshape(-1, 34)
    d = _f16(b[:, 0:2])
    return (b[:, 2:34].view(np.int8).astype(F32) * d).reshape(-1)


def q4_k(raw: np.ndarray) -> np.ndarray:
    b = raw.reshape(-1, 144)
    d, dmin = _f16(b[:, 0:2]), _f16(b[:, 2:4])
    scales = b[:, 4:16]
    qs = b[:, 16:144].astype(np.int32)
    y = np.empty((b.shape[0], 256), dtype=F32)
    is_ = 0
    for j in range(0, 256, 64):
        sc, m = _scale_min_k4(is_, scales)
        d1, m1 = d * sc.astype(F32), dmin * m.astype(F32)
        sc, m = _scale_min_k4(is_ + 1, scales)
        d2, m2 = d * sc.astype(F32), dmin * m.astype(F32)
        q = qs[:, (j // 64) * 32:(j // 64) * 32 + 32]
        y[:, j:j + 32] = d1 * (q & 0xF).astype(F32) - m1
        y[:, j + 32:j + 64] = d2 * (q >> 4).astype(F32) - m2
        is_ += 2
    return y.reshape(-1)


def q5_k(raw: np.ndarray) -> np.ndarray:
    b = raw.reshape(-1, 176)
    d, dmin = _f16(b[:, 0:2]), _f16(b[:, 2:4])
    scales = b[:, 4:16]
    qh = b[:, 16:48].astype(np.int32)
    ql = b[:, 48:176].astype(np.int32)
    y = np.empty((b.shape[0], 256), dtype=F32)
    is_, u1, u2 = 0, 1, 2
    for j in range(0, 256, 64):
        sc, m = _scale_min_k4(is_, scales)
        d1, m1 = d * sc.astype(F32), dmin * m.astype(F32)
        sc, m = _scale_min_k4(is_ + 1, scales)
        d2, m2 = d * sc.astype(F32), dmin * m.astype(F32)
        q = ql[:, (j // 64) * 32:(j // 64) * 32 + 32]
        y[:, j:j + 32] = d1 * ((q & 0xF) + np.where(qh & u1, 16, 0)).astype(F32) - m1
        y[:, j + 32:j + 64] = d2 * ((q >> 4) + np.where(qh & u2, 16, 0)).astype(F32) - m2
        is_ += 2
        u1 <<= 2
        u2 <<= 2
    return y.reshape(-1)


def q6_k(raw: np.ndarray) -> np.ndarray:
    b = raw.reshape(-1, 210)
    d = _f16(b[:, 208:210])
    y = np.empty((b.shape[0], 256), dtype=F32)
    for n in range(2):  # two 128-element halves
        ql = b[:, n * 64:n * 64 + 64].astype(np.int32)
        qh = b[:, 128 + n * 32:128 + n * 32 + 32].astype(np.int32)
        sc = b[:, 192 + n * 8:192 + n * 8 + 8].view(np.int8).astype(F32)
        for l in range(32):
            is_ = l // 16
            q1 = ((ql[:, l] & 0xF) | (((qh[:, l] >> 0) & 3) << 4)) - 32
            q2 = ((ql[:, l + 32] & 0xF) | (((qh[:, l] >> 2) & 3) << 4)) - 32
            q3 = ((ql[:, l] >> 4) | (((qh[:, l] >> 4) & 3) << 4)) - 32
            q4 = ((ql[:, l + 32] >> 4) | (((qh[:, l] >> 6) & 3) << 4)) - 32
            base = n * 128
            y[:, base + l] = (d[:, 0] * sc[:, is_ + 0]) * q1.astype(F32)
            y[:, base + l + 32] = (d[:, 0] * sc[:, is_ + 2]) * q2.astype(F32)
            y[:, base + l + 64] = (d[:, 0] * sc[:, is_ + 4]) * q3.astype(F32)
            y[:, base + l + 96] = (d[:, 0] * sc[:, is_ + 6]) * q4.astype(F32)
    return y.reshape(-1)


DEQUANT = {2: q4_0, 6: q5_0, 8: q8_0, 12: q4_k, 13: q5_k, 14: q6_k}
BLOCK = {2: (32, 18), 6: (32, 22), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}
HALF_OFFSETS = {2: [0], 6: [0], 8: [0], 12: [0, 2], 13: [0, 2], 14: [208]}


def random_blocks(rng: np.random.Generator, ggml_type: int, n_blocks: int, finite: bool = True) -> np.ndarray:
    """Uniform random bytes with every fp16 field replaced by a finite random
    half (both signs, subnormals included) when `finite`."""
    elems, nbytes = BLOCK[ggml_type]
    raw = rng.integers(0, 256, size=(n_blocks, nbytes), dtype=np.uint8)
    if finite:
        for off in HALF_OFFSETS[ggml_type]:
            h = rng.integers(0, 1 << 16, size=n_blocks, dtype=np.uint32)
            h = np.where((h & 0x7C00) == 0x7C00, h & 0x83FF, h).astype(np.uint16)  # exponent 31 -> 0
            raw[:, off:off + 2] = h.view(np.uint8).reshape(n_blocks, 2)
    return raw.reshape(-1)

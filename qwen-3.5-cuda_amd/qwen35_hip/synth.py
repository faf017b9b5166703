"""Deterministic synthetic inputs of the benchmark configurations (numpy, host).

Generator: splitmix64 -> 53-bit uniforms in [0, 1); normals by Box-Muller with
N(mu, sigma) meaning mean and standard deviation. Config k uses base seed
0x5EED0000 + k; tensor s inside a config uses seed (base << 8) | s. The same
host arrays feed the GPU kernels and the CPU oracle, so both see bit-identical
inputs.

Configurations (BASELINE.json `configs`, in order):
  C1  RMSNorm fp32 x [36 x 2048] N(0,1), w [2048] N(1,0.1), eps 1e-6
  C2  Q [512 x 16 x 256], K [512 x 2 x 256] N(0,1), norm weights [256] N(1,0.1),
      rope_dim 64, theta 1e7, positions 0..511
  C3  bf16 x, branch [4096 x 2048] N(0,1), w [2048] N(1,0.1);
      SwiGLU g, u bf16 [4096 x 8 x 512] N(0,2); shared g, u [4096 x 512] N(0,2),
      logits [4096] N(0,1)
  C4  conv x [4096 x 8192] N(0,1), w [8192 x 4] N(0,0.5), zero history;
      16 key heads x 128; gated norm x, z [4096 x 32 x 128] N(0,1), w [128] N(1,0.1)
  C5  vocab 248320 x 2048 as Q4_K (d, dmin fp16 U(0,0.01), uniform scale bytes and
      nibbles) and as Q6_K (uniform ql/qh/scale bytes, d fp16 U(0,0.01));
      8192 uniform token ids
"""

from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22

BASE_SEED = 0x5EED0000


def seed_for(config: int, tensor: int) -> int:
    return ((BASE_SEED + config) << 8) | tensor


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Outputs offset+1 .. offset+n of the splitmix64 stream started at `seed`."""
    i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int) -> np.ndarray:
    """float64 uniforms in [0, 1) with 53 random bits."""
    out = np.empty(n, dtype=np.float64)
    for lo in range(0, n, _CHUNK):
        m = min(_CHUNK, n - lo)
        out[lo:lo + m] = (splitmix64(seed, m, lo) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
    return out


def normal(seed: int, shape, mu: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    """float32 N(mu, sigma) by Box-Muller on consecutive uniform pairs."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    pairs = (n + 1) // 2
    for lo in range(0, pairs, _CHUNK):
        m = min(_CHUNK, pairs - lo)
        u = (splitmix64(seed, 2 * m, 2 * lo) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
        r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
        a = 2.0 * np.pi * u[1::2]
        z = np.empty(2 * m, dtype=np.float64)
        z[0::2] = r * np.cos(a)
        z[1::2] = r * np.sin(a)
        k = min(2 * m, n - 2 * lo)
        out[2 * lo:2 * lo + k] = (mu + sigma * z[:k]).astype(np.float32)
    return out.reshape(shape)


def random_bytes(seed: int, n: int) -> np.ndarray:
    words = (n + 7) // 8
    out = np.empty(words * 8, dtype=np.uint8)
    for lo in range(0, words, _CHUNK):
        m = min(_CHUNK, words - lo)
        out[8 * lo:8 * (lo + m)] = splitmix64(seed, m, lo).view(np.uint8)
    return out[:n]


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return u.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


# ---------------------------------------------------------------- configs
def c1_rmsnorm(rows: int = 36, n: int = 2048):
    return {"x": normal(seed_for(1, 0), (rows, n)), "w": normal(seed_for(1, 1), (n,), 1.0, 0.1), "eps": 1e-6}


def c2_qk_rope(rows: int = 512, q_heads: int = 16, k_heads: int = 2, head_dim: int = 256):
    return {
        "q": normal(seed_for(2, 0), (rows, q_heads, head_dim)),
        "k": normal(seed_for(2, 1), (rows, k_heads, head_dim)),
        "qw": normal(seed_for(2, 2), (head_dim,), 1.0, 0.1),
        "kw": normal(seed_for(2, 3), (head_dim,), 1.0, 0.1),
        "pos": np.arange(rows, dtype=np.int32),
        "rope_dim": 64,
        "theta": 1e7,
        "eps": 1e-6,
    }


def c3_residual(rows: int = 4096, n: int = 2048):
    return {
        "x": to_bf16_bits(normal(seed_for(3, 0), (rows, n))),
        "branch": to_bf16_bits(normal(seed_for(3, 1), (rows, n))),
        "w": normal(seed_for(3, 2), (n,), 1.0, 0.1),
        "eps": 1e-6,
    }


def c3_swiglu(rows: int = 4096, experts: int = 8, dim: int = 512):
    return {
        "g": to_bf16_bits(normal(seed_for(3, 3), (rows, experts, dim), 0.0, 2.0)),
        "u": to_bf16_bits(normal(seed_for(3, 4), (rows, experts, dim), 0.0, 2.0)),
    }


def c3_shared(rows: int = 4096, dim: int = 512):
    return {
        "g": to_bf16_bits(normal(seed_for(3, 5), (rows, dim), 0.0, 2.0)),
        "u": to_bf16_bits(normal(seed_for(3, 6), (rows, dim), 0.0, 2.0)),
        "logits": normal(seed_for(3, 7), (rows,)),
    }


def c4_frontend(rows: int = 4096, channels: int = 8192, kernel: int = 4, random_history: bool = False):
    hist = (normal(seed_for(4, 2), (channels, kernel - 1)) if random_history
            else np.zeros((channels, kernel - 1), dtype=np.float32))
    return {
        "x": normal(seed_for(4, 0), (rows, channels)),
        "w": normal(seed_for(4, 1), (channels, kernel), 0.0, 0.5),
        "hist": hist,
        "k_heads": 16,
        "key_dim": 128,
        "eps": 1e-6,
    }


def c4_norm_gate(rows: int = 4096, heads: int = 32, dim: int = 128):
    return {
        "x": normal(seed_for(4, 3), (rows, heads, dim)),
        "z": normal(seed_for(4, 4), (rows, heads, dim)),
        "w": normal(seed_for(4, 5), (dim,), 1.0, 0.1),
        "eps": 1e-6,
    }


def _fp16_bits(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float16).view(np.uint16)


def q4k_table(rows: int = 248320, cols: int = 2048, seed_tensor: int = 0) -> np.ndarray:
    """uint8 [rows * cols/256 * 144]: d, dmin fp16 U(0,0.01); 12 scale bytes and
    128 nibble bytes uniform."""
    nb = rows * (cols // 256)
    blocks = random_bytes(seed_for(5, seed_tensor), nb * 144).reshape(nb, 144)
    d = _fp16_bits(uniform(seed_for(5, seed_tensor + 1), nb) * 0.01)
    dmin = _fp16_bits(uniform(seed_for(5, seed_tensor + 2), nb) * 0.01)
    blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blocks[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return blocks.reshape(-1)


def q6k_table(rows: int = 248320, cols: int = 2048, seed_tensor: int = 4) -> np.ndarray:
    """uint8 [rows * cols/256 * 210]: ql, qh, int8 scales uniform; d fp16 U(0,0.01)."""
    nb = rows * (cols // 256)
    blocks = random_bytes(seed_for(5, seed_tensor), nb * 210).reshape(nb, 210)
    d = _fp16_bits(uniform(seed_for(5, seed_tensor + 1), nb) * 0.01)
    blocks[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return blocks.reshape(-1)


def token_ids(n: int = 8192, vocab: int = 248320, seed_tensor: int = 8) -> np.ndarray:
    return np.minimum((uniform(seed_for(5, seed_tensor), n) * vocab).astype(np.int64), vocab - 1).astype(np.int32)

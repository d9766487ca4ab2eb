"""Seeded synthetic inputs for the IQ3_XXS path (weights, activations, router logits).

Counter-based generator: splitmix64 applied to ``key + (i+1) * golden`` for
element ``i`` of a named stream, so any prefix of any stream is reproducible
from ``(seed, stream)`` alone and generation vectorises in numpy. Normals are
Box-Muller in float64, rounded once to the requested dtype.

Block distribution (one 98-byte IQ3_XXS super-block of 256 weights):
  d      = fp16_RNE(|z| * d_scale), z ~ N(0,1)       (d_scale = 0.02)
  qs[64] = uniform bytes 0..255                      (grid indices)
  aux[8] = uniform u32: bits 28..31 scale 0..15, bits 7l..7l+6 sign index 0..127
which is the byte layout the reference decodes at quant.cpp:186-210.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

BLOCK_BYTES = 98
QK = 256


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def u64(seed: int, stream: int, n: int, offset: int = 0) -> np.ndarray:
    """``n`` uint64 values of stream ``stream`` starting at element ``offset``."""
    with np.errstate(over="ignore"):
        key = _mix(np.array([(seed & 0xFFFFFFFF) | ((stream & 0xFFFFFFFF) << 32)], dtype=np.uint64))[0]
        ctr = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        return _mix(key + ctr * _GOLDEN)


def normal(seed: int, stream: int, n: int, dtype=np.float32) -> np.ndarray:
    """``n`` N(0,1) samples (Box-Muller over pairs of 53-bit uniforms)."""
    m = (n + 1) // 2
    r = u64(seed, stream, 2 * m)
    scale = 1.0 / 9007199254740992.0  # 2^-53
    u1 = ((r[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * scale  # (0, 1]
    u2 = (r[1::2] >> np.uint64(11)).astype(np.float64) * scale  # [0, 1)
    rad = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = rad * np.cos(2.0 * np.pi * u2)
    z[1::2] = rad * np.sin(2.0 * np.pi * u2)
    return z[:n].astype(dtype)


def iq3xxs_blocks(seed: int, stream: int, n_blocks: int, d_scale: float = 0.02) -> np.ndarray:
    """``n_blocks`` packed IQ3_XXS blocks as a uint8 array of shape [n_blocks, 98]."""
    out = np.empty((n_blocks, BLOCK_BYTES), dtype=np.uint8)
    d = (np.abs(normal(seed, stream * 4 + 0, n_blocks, np.float64)) * d_scale).astype(np.float16)
    out[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
    qs = u64(seed, stream * 4 + 1, n_blocks * 8)
    out[:, 2:66] = qs.view(np.uint8).reshape(n_blocks, 64)
    aux = (u64(seed, stream * 4 + 2, n_blocks * 8) & np.uint64(0xFFFFFFFF)).astype("<u4")
    out[:, 66:98] = aux.view(np.uint8).reshape(n_blocks, 32)
    return out


def iq3xxs_matrix(seed: int, stream: int, n_rows: int, in_dim: int, d_scale: float = 0.02) -> np.ndarray:
    """GGUF row-major IQ3_XXS payload for an [n_rows, in_dim] weight: uint8 [n_rows, in_dim/256*98]."""
    if in_dim % QK:
        raise ValueError("in_dim must be a multiple of 256")
    nb = in_dim // QK
    return iq3xxs_blocks(seed, stream, n_rows * nb, d_scale).reshape(n_rows, nb * BLOCK_BYTES)


def row_bytes(in_dim: int) -> int:
    return in_dim // QK * BLOCK_BYTES

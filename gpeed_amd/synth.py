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


# GGUF block formats other than IQ3_XXS (quant.cpp:83-114, 165-502): ggml
# type id -> (weights per block, bytes per block, byte offsets of the fp16
# scale fields)
FORMATS = {
    8: (32, 34, (0,)),          # Q8_0: d
    10: (256, 84, (80, 82)),    # Q2_K: d, dmin
    11: (256, 110, (108,)),     # Q3_K: d
    14: (256, 210, (208,)),     # Q6_K: d
    18: (256, 98, (0,)),        # IQ3_XXS: d
    21: (256, 110, (0,)),       # IQ3_S: d
    22: (256, 82, (0,)),        # IQ2_S: d
    23: (256, 136, (0,)),       # IQ4_XS: d
}
SCALAR_FORMATS = {0: np.float32, 1: np.float16, 30: "bf16"}


def quant_blocks(seed: int, stream: int, dtype: int, n_blocks: int, d_scale: float = 0.02) -> np.ndarray:
    """``n_blocks`` blocks of a GGUF block format: uniform random bytes with
    every fp16 scale field set to |N(0,1)| * d_scale. uint8 [n_blocks, bytes]."""
    _, nbytes, d_offs = FORMATS[dtype]
    words = u64(seed, stream * 4 + 0, (n_blocks * nbytes + 7) // 8)
    out = words.view(np.uint8)[: n_blocks * nbytes].reshape(n_blocks, nbytes).copy()
    for k, off in enumerate(d_offs):
        d = (np.abs(normal(seed, stream * 4 + 1 + k, n_blocks, np.float64)) * d_scale).astype(np.float16)
        out[:, off:off + 2] = d.view(np.uint8).reshape(n_blocks, 2)
    return out


def quant_matrix(seed: int, stream: int, dtype: int, n_rows: int, in_dim: int, d_scale: float = 0.02) -> np.ndarray:
    """GGUF row-major payload of an [n_rows, in_dim] weight of any decoded type:
    uint8 [n_rows, row_bytes]. Scalar types hold N(0,1) * d_scale * 16."""
    if dtype in SCALAR_FORMATS:
        v = normal(seed, stream, n_rows * in_dim, np.float64) * d_scale * 16
        if dtype == 30:
            bits = np.asarray(v, np.float32).view(np.uint32)
            raw = ((bits + np.uint32(0x7FFF) + ((bits >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
        else:
            raw = v.astype(SCALAR_FORMATS[dtype])
        return raw.view(np.uint8).reshape(n_rows, -1)
    elems, nbytes, _ = FORMATS[dtype]
    if in_dim % elems:
        raise ValueError(f"in_dim must be a multiple of {elems}")
    nb = in_dim // elems
    return quant_blocks(seed, stream, dtype, n_rows * nb, d_scale).reshape(n_rows, nb * nbytes)

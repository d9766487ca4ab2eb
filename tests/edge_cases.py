"""IQ3_XXS weight matrices with edge-case block scales, for the product tests.

Every row starts from seeded synthetic blocks (gpeed_amd.synth); the fp16 d of
chosen blocks is then overwritten (bytes 0..1 of the 98-byte block,
quant.cpp:186-191):

* finite edges, cycled along a row: +0, -0, the smallest subnormal 2^-24, a
  mid subnormal, the largest subnormal, the smallest normal, +-65504 (the
  largest finite), +-1 and 0.1;
* jump rows: consecutive blocks whose d differs by 2^20 or 2^-20, with
  unequal mantissas too (1.5 x 2^-5 next to 1.25 x 2^15), so the GEMM's
  running-d rescale meets ratios that are not powers of two;
* zero rows: every d +0 or -0 (the row is exactly zero);
* a big-then-tiny row: block 0 at 65504, the rest subnormal.

Rows r % 8 in 4..7 keep their synthetic d. ``nonfinite=True`` also puts
+inf, -inf or NaN into one block of a few of those rows (at the first, a
middle and the last block); the reference then sums +-inf products of both
signs (or NaN products), so those rows are NaN.
"""
from __future__ import annotations

import numpy as np

from gpeed_amd import synth

FINITE_D = [0x0000, 0x8000, 0x0001, 0x0200, 0x03FF, 0x0400, 0x7BFF, 0xFBFF, 0x3C00, 0xBC00, 0x2E66]
# 2^-5, 2^15, 1.5*2^-5, 1.25*2^15, 2^-20 (subnormal), 1.0, 2^-20, 1.5, -2^-5, -2^15
JUMP_D = [0x2800, 0x7800, 0x2A00, 0x7900, 0x0010, 0x3C00, 0x0010, 0x3E00, 0xA800, 0xF800]
POS_INF, NEG_INF, NAN = 0x7C00, 0xFC00, 0x7E00


def edge_matrix(seed: int, stream: int, n_rows: int, in_dim: int, nonfinite: bool = False) -> np.ndarray:
    """GGUF rows [n_rows, in_dim/256*98] with the edge scales described above."""
    w = synth.iq3xxs_matrix(seed, stream, n_rows, in_dim)
    nb = in_dim // synth.QK
    blocks = w.reshape(n_rows, nb, synth.BLOCK_BYTES)
    d = blocks[:, :, 0].astype(np.uint32) | (blocks[:, :, 1].astype(np.uint32) << 8)
    r = np.arange(n_rows)[:, None]
    b = np.arange(nb)[None, :]
    kind = np.broadcast_to(r % 8, d.shape)
    fin = np.asarray(FINITE_D, np.uint32)[(r // 8 + b) % len(FINITE_D)]
    jump = np.asarray(JUMP_D, np.uint32)[(r // 8 + b) % len(JUMP_D)]
    zero = np.where((r + b) & 1, 0x8000, 0x0000).astype(np.uint32)
    tiny = np.where(b == 0, 0x7BFF, 0x0001 + ((r + b) % 7) * 0x80).astype(np.uint32)
    d = np.where(kind == 0, fin, np.where(kind == 1, jump, np.where(kind == 2, zero, np.where(kind == 3, tiny, d))))
    if nonfinite:
        rows = np.nonzero(np.arange(n_rows) % 8 >= 5)[0]
        k = rows % 8
        which = (rows // 8) % 3
        col = np.array([0, nb // 2, nb - 1])[(rows // 8 + k) % 3]
        d[rows, col] = np.array([POS_INF, NEG_INF, NAN], np.uint32)[which]
    blocks[:, :, 0] = (d & 0xFF).astype(np.uint8)
    blocks[:, :, 1] = (d >> 8).astype(np.uint8)
    return w


def outlier_rows(x: np.ndarray, seed: int) -> np.ndarray:
    """Activation rows with a few channels at 1000x the row's rms."""
    x = np.array(x, np.float32, copy=True)
    rng = synth.u64(seed, 7, x.shape[0] * 3)
    for t in range(x.shape[0]):
        rms = float(np.sqrt(np.mean(x[t].astype(np.float64) ** 2)))
        for k in range(3):
            c = int(rng[3 * t + k] % np.uint64(x.shape[1]))
            x[t, c] = np.float32((1000.0 if k != 1 else -1000.0) * rms)
    return x


def row_kinds(n_rows: int) -> np.ndarray:
    """The edge kind of each row (r % 8; 4..7 are synthetic d)."""
    k = np.arange(n_rows) % 8
    return np.where(k >= 4, 4, k)


def check(y, ref, tol: float, kinds=None, what: str = "") -> None:
    """Every non-finite output of the same class as the reference's (NaN,
    +inf or -inf); finite outputs within tol under rel_err, taken per row
    kind (``kinds`` broadcast against the output's last axis) so that rows
    of d = 65504 do not set the scale for the others."""
    from conftest import rel_err

    y = np.asarray(y, np.float32)
    ref = np.asarray(ref, np.float32)
    assert y.shape == ref.shape, (what, y.shape, ref.shape)
    assert np.array_equal(np.isnan(y), np.isnan(ref)), (what, np.argwhere(np.isnan(y) != np.isnan(ref))[:8])
    assert np.array_equal(np.isposinf(y), np.isposinf(ref)), what
    assert np.array_equal(np.isneginf(y), np.isneginf(ref)), what
    kinds = np.zeros(y.shape[-1], int) if kinds is None else np.asarray(kinds)
    kinds = np.broadcast_to(kinds, y.shape)
    fin = np.isfinite(ref)
    for k in np.unique(kinds):
        sel = fin & (kinds == k)
        if sel.any():
            e = rel_err(y[sel], ref[sel])
            assert e < tol, (what, int(k), e)

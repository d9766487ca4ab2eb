"""CPU checks of the other GGUF block formats (Q8_0, Q2_K, Q3_K, Q6_K, IQ3_S,
IQ2_S, IQ4_XS, F16, BF16, F32): the oracle's restatement against the
reference's own code (oracle/_ref, quant.cpp compiled from source) and the
committed vectors it wrote, the codebooks against the reference header, and
the geometry the C ABI reports. No GPU needed.
"""
import os
import re
import struct

import numpy as np
import pytest

import gpeed_amd as G
import oracle
from gpeed_amd import synth
from conftest import ROOT

GOLD = os.path.join(ROOT, "tests", "golden")
REF_QTABLES = "/root/reference/cpp/core/include/glm5/quant_tables.h"
BLOCK_TYPES = [8, 10, 11, 14, 21, 22, 23]
SCALAR_TYPES = [0, 1, 30]
# ggml block geometry (weights, bytes): quant.cpp:52-114
GEOMETRY = {0: (1, 4), 1: (1, 2), 30: (1, 2), 8: (32, 34), 10: (256, 84), 11: (256, 110), 14: (256, 210),
            18: (256, 98), 21: (256, 110), 22: (256, 82), 23: (256, 136)}


def same_bits_or_nan(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) | np.isnan(b)
    return bool(np.array_equal(np.isnan(a), np.isnan(b))
                and np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32)))


def _table(text, name):
    body = re.search(name + r"\[(\d+)\]\s*=\s*\{(.*?)\};", text, re.S)
    vals = [int(v, 0) for v in re.findall(r"-?0x[0-9a-fA-F]+|-?\d+", body.group(2))]
    assert len(vals) == int(body.group(1))
    return vals


def test_geometry_oracle_and_abi():
    for dt, (be, bb) in GEOMETRY.items():
        assert oracle.block_geometry(dt) == (be, bb)
        assert G.dtype_block_size(dt) == be
        assert G.dtype_row_bytes(dt, 512) == 512 // be * bb
    # quant.cpp:119-126: 0 for a partial block or a type that is not decoded
    assert G.dtype_row_bytes(10, 300) == 0
    for dt in (2, 3, 12, 13, 15, 16, 17, 19, 20, 24, 29, 34):
        assert G.dtype_block_size(dt) == 0 and G.dtype_row_bytes(dt, 256) == 0


def test_codebooks_match_reference_header():
    """The packed codebooks expand, in the oracle and in the product library,
    to the reference's tables (quant_tables.h:15, 275, 343)."""
    g2, g3, v4 = oracle.iq2s_grid(), oracle.iq3s_grid(), oracle.iq4nl_values()
    assert np.array_equal(G.codebook(22), g2)
    assert np.array_equal(G.codebook(21), g3)
    assert np.array_equal(G.codebook(18), np.array([oracle.lib().orc_grid_entry(i) for i in range(256)], np.uint64))
    # level sets: IQ2_S bytes in {8, 25, 43}, IQ3_S bytes odd in 1..15, IQ4 levels sorted
    assert set(np.unique(g2.view(np.uint8))) == {8, 25, 43}
    assert set(np.unique(g3.astype(np.uint32).view(np.uint8))) <= set(range(1, 16, 2))
    assert len(set(g2.tolist())) == 1024 and len(set(g3.tolist())) == 512
    assert np.all(np.diff(v4) > 0)
    if not os.path.exists(REF_QTABLES):
        pytest.skip("reference header not present")
    text = open(REF_QTABLES, encoding="utf-8").read()
    assert _table(text, "kIq2sGrid") == g2.tolist()
    assert _table(text, "kIq3sGrid") == g3.tolist()
    assert _table(text, "kValuesIq4nl") == v4.tolist()


@pytest.mark.parametrize("dt", BLOCK_TYPES + SCALAR_TYPES)
def test_oracle_dequant_golden(dt):
    z = np.load(os.path.join(GOLD, "quant_formats.npz"))
    raw, deq = z[f"raw_{dt}"], z[f"deq_{dt}"]
    assert same_bits_or_nan(oracle.dequantize(raw.reshape(-1), deq.size, dtype=dt), deq)


@pytest.mark.parametrize("dt", BLOCK_TYPES + SCALAR_TYPES)
def test_oracle_rows_product_golden(dt):
    z = np.load(os.path.join(GOLD, "quant_formats.npz"))
    Y = oracle.matmul_rows(dt, z[f"w_{dt}"], 2, 512, 8, z[f"X_{dt}"])
    assert same_bits_or_nan(Y, z[f"Y_{dt}"])


@pytest.mark.parametrize("dt", BLOCK_TYPES)
def test_oracle_dequant_random_vs_ref(dt):
    """Uniform random bytes (scales included: every fp16 class, every scale
    byte) against the reference's quant.cpp."""
    R = oracle.ref()
    if R is None:
        pytest.skip("oracle/_ref is not built")
    be, bb = GEOMETRY[dt]
    n_blk = 4000
    raw = synth.u64(31, dt, n_blk * bb // 8 + 1).view(np.uint8)[: n_blk * bb].copy()
    n = n_blk * be
    ref = np.empty(n, np.float32)
    assert R.ref_dequantize(dt, raw.ctypes.data, ref, n) == 0
    assert same_bits_or_nan(oracle.dequantize(raw, n, dtype=dt), ref)


@pytest.mark.parametrize("dt", BLOCK_TYPES + SCALAR_TYPES)
def test_oracle_rows_product_vs_ref(dt):
    R = oracle.ref()
    if R is None:
        pytest.skip("oracle/_ref is not built")
    in_dim, rows = 1024, 24
    w = synth.quant_matrix(32, dt, dt, rows, in_dim)
    X = synth.normal(32, 7, 3 * in_dim).reshape(3, in_dim)
    st = oracle.RefStore(w, rows, in_dim, name="t.weight", dtype=dt)
    try:
        assert same_bits_or_nan(oracle.matmul_rows(dt, w, 5, in_dim, 16, X), st.matmul(5, in_dim, 16, X))
        assert same_bits_or_nan(oracle.matmul_rows(dt, w, 0, in_dim, 24, X[1]), st.matvec(0, in_dim, 24, X[1])[None])
    finally:
        st.close()


@pytest.mark.parametrize("dt", BLOCK_TYPES)
def test_oracle_scale_linearity(dt):
    """Doubling the fp16 scale fields (exactly) doubles every weight: the
    scales multiply every term, with nothing added that does not scale."""
    be, bb = GEOMETRY[dt]
    raw = synth.quant_blocks(33, dt, dt, 64)
    d_offs = synth.FORMATS[dt][2]
    raw2 = raw.copy()
    for off in d_offs:
        d = np.frombuffer(raw[:, off:off + 2].tobytes(), np.float16).astype(np.float32)
        raw2[:, off:off + 2] = np.frombuffer((d * 2).astype(np.float16).tobytes(), np.uint8).reshape(-1, 2)
    a = oracle.dequantize(raw.reshape(-1), 64 * be, dtype=dt)
    b = oracle.dequantize(raw2.reshape(-1), 64 * be, dtype=dt)
    assert np.array_equal(b, a * 2)


def test_oracle_q8_0_closed_form():
    """Q8_0 with d = 1: the weights are the int8 codes (make_test_gguf.py's
    test.q8_0 tensor decodes the same way)."""
    raw = synth.quant_blocks(34, 8, 8, 32)
    raw[:, 0:2] = np.frombuffer(struct.pack("<e", 1.0), np.uint8)
    y = oracle.dequantize(raw.reshape(-1), 32 * 32, dtype=8)
    assert np.array_equal(y, raw[:, 2:].view(np.int8).reshape(-1).astype(np.float32))


def test_oracle_iq4_xs_closed_form():
    """IQ4_XS with scale 33 (dl = d) and d = 1: weight i < 16 of sub-block ib
    is level[low nibble of qs[16 ib + i]], weight 16 + i the high nibble."""
    raw = synth.quant_blocks(35, 23, 23, 8)
    raw[:, 0:2] = np.frombuffer(struct.pack("<e", 1.0), np.uint8)
    raw[:, 2:4] = np.frombuffer(struct.pack("<H", 0xAAAA), np.uint8)  # top bits 10 for every sub-block
    raw[:, 4:8] = 0x11  # low nibbles 1 -> 6-bit scale 0b100001 = 33
    y = oracle.dequantize(raw.reshape(-1), 8 * 256, dtype=23).reshape(8, 8, 32)
    lv = oracle.iq4nl_values()
    qs = raw[:, 8:].reshape(8, 8, 16)
    assert np.array_equal(y[:, :, :16], lv[qs & 15].astype(np.float32))
    assert np.array_equal(y[:, :, 16:], lv[qs >> 4].astype(np.float32))

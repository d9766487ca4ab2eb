"""CPU-side checks of the C ABI library (no device compute).

* libgpeed_iq3.so loads and exports every entry point include/gpeed_iq3.h declares;
* host-only geometry and layout helpers answer correctly;
* a numpy model of the GPU decode (T16 unit -> perm addresses -> the library's
  own 64 KiB LDS table -> (2s+1) -> d/4) reproduces the oracle's dequantized
  weights bit for bit, so the layout and table are right before any kernel
  runs.
"""
import ctypes as C
import os
import re

import numpy as np
import pytest

import gpeed_amd
import oracle
from gpeed_amd import synth
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "gpeed_iq3.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gpeed_\w+)\s*\(", text)))


def test_header_symbols_exported():
    L = gpeed_amd.lib()
    names = declared_symbols()
    assert len(names) >= 15
    for n in names:
        assert hasattr(L, n), n


def test_geometry():
    L = gpeed_amd.lib()
    assert L.gpeed_iq3xxs_row_bytes(4096) == 16 * 98
    assert L.gpeed_iq3xxs_row_bytes(12288) == 4704
    assert L.gpeed_iq3xxs_row_bytes(100) == 0
    assert L.gpeed_iq3xxs_t16_bytes(6144, 12288) == 6144 * 4704
    assert L.gpeed_iq3xxs_t16_bytes(17, 256) == 32 * 98
    assert L.gpeed_iq3xxs_t16_bytes(1, 200) == 0


def aux_t16_model(aux):
    """T16 sign/scale word, restated from the layout definition."""
    out = 0
    for l in range(4):
        s7 = (aux >> (7 * l)) & 127
        s = [(s7 >> i) & 1 for i in range(7)]
        t3 = s[0] ^ s[1] ^ s[2] ^ s[3]
        b = s[0] | s[1] << 1 | s[2] << 2 | t3 << 3 | s[4] << 4 | s[5] << 5 | s[6] << 6
        b |= ((aux >> (28 + l)) & 1) << 7
        out |= b << (8 * l)
    return out


def test_aux_word_matches_model():
    L = gpeed_amd.lib()
    words = synth.u64(3, 0, 4000) & np.uint64(0xFFFFFFFF)
    for w in [0, 0xFFFFFFFF, 0x80000000, 0x0FFFFFFF] + [int(v) for v in words]:
        assert L.gpeed_t16_aux_word(w) == aux_t16_model(w), hex(w)


@pytest.fixture(scope="module")
def sign_table():
    t = np.empty(32768, np.uint16)
    assert gpeed_amd.lib().gpeed_t16_sign_table(t.ctypes.data, t.size) == 0
    assert gpeed_amd.lib().gpeed_t16_sign_table(t.ctypes.data, 100) != 0
    return t.view(np.float16)


def test_decode_model_matches_oracle(sign_table):
    L = gpeed_amd.lib()
    blocks = synth.iq3xxs_blocks(5, 0, 48)
    want = oracle.dequantize(blocks, 48 * 256).reshape(48, 256)
    for bi, raw in enumerate(blocks):
        d = np.float32(np.frombuffer(raw[0:2].tobytes(), np.float16)[0])
        aux = np.frombuffer(raw[66:98].tobytes(), "<u4")
        got = np.empty(256, np.float32)
        for ib in range(8):
            a = L.gpeed_t16_aux_word(int(aux[ib]))
            q = raw[2 + 8 * ib: 10 + 8 * ib]
            cb1 = (a << 3) & 0x78787878
            cb2 = (a & 0x78787878) | 0x80808080
            s = sum(((a >> (8 * l + 7)) & 1) << l for l in range(4))
            assert s == int(aux[ib]) >> 28
            f = np.float16(2 * s + 1)
            for l in range(4):
                a1 = (int(q[2 * l]) << 8) | ((cb1 >> (8 * l)) & 255)
                a2 = (int(q[2 * l + 1]) << 8) | ((cb2 >> (8 * l)) & 255)
                v = np.concatenate([sign_table[a1 // 2: a1 // 2 + 4], sign_table[a2 // 2: a2 // 2 + 4]])
                vf = (v * f).astype(np.float16)  # exact: |q*(2s+1)| <= 1922
                assert np.array_equal(vf.astype(np.float64), v.astype(np.float64) * (2 * s + 1))
                got[32 * ib + 8 * l: 32 * ib + 8 * l + 8] = vf.astype(np.float32) * (d * np.float32(0.25))
        assert np.array_equal(got.view(np.uint32), want[bi].view(np.uint32)), bi


def test_device_count_without_gpu_is_nonnegative():
    assert gpeed_amd.device_count() >= 0

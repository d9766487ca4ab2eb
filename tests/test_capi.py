"""CPU-side checks of the C ABI library (no device compute).

* libgpeed_iq3.so loads and exports every entry point include/gpeed_iq3.h declares;
* host-only geometry and layout helpers answer correctly;
* a numpy model of the GPU decode (T16 unit -> perm addresses -> the library's
  own 64 KiB replicated LDS table -> sign bits from the T16 word -> (2s+1)d/4)
  reproduces the oracle's dequantized weights bit for bit, so the layout and
  table are right before any kernel runs.
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
    """T16 sign/scale word, restated bit by bit from the layout definition:
    sign j (< 7) of group l at bit 15-k (j even) or 31-k (j odd), k = 4(j//2)+l;
    the scale nibble at bits 16..19."""
    out = ((aux >> 28) & 15) << 16
    for l in range(4):
        for j in range(7):
            k = 4 * (j // 2) + l
            out |= ((aux >> (7 * l + j)) & 1) << (31 - k if j & 1 else 15 - k)
    return out


def test_aux_word_matches_model():
    L = gpeed_amd.lib()
    words = synth.u64(3, 0, 4000) & np.uint64(0xFFFFFFFF)
    for w in [0, 0xFFFFFFFF, 0x80000000, 0x0FFFFFFF] + [int(v) for v in words]:
        assert L.gpeed_t16_aux_word(w) == aux_t16_model(w), hex(w)


def test_aux_word_is_a_bijection_on_used_bits():
    """Every one of the 32 aux bits lands on a distinct T16 bit."""
    L = gpeed_amd.lib()
    seen = 0
    for b in range(32):
        t = L.gpeed_t16_aux_word(1 << b)
        assert t and (t & (t - 1)) == 0, b
        assert not (seen & t), b
        seen |= t
    assert seen == 0xFFFFFFFF


@pytest.fixture(scope="module")
def grid_table():
    t = np.empty(32768, np.uint16)
    assert gpeed_amd.lib().gpeed_t16_grid_table(t.ctypes.data, t.size) == 0
    assert gpeed_amd.lib().gpeed_t16_grid_table(t.ctypes.data, 100) != 0
    return t


def full_signs_model(w):
    """The kernel's sign word: implied 8th signs (even parity per group) folded
    in over the scale nibble with three xor-folds (t16_full_signs)."""
    m = w & 0xFFF0FFFF
    t = m ^ (m >> 16)
    t ^= t >> 8
    t ^= t >> 4
    return m | ((t & 15) << 16)


def test_grid_table_replicas_conflict_free(grid_table):
    """Each lane's 8-byte entry for any index sits in its own bank pair among
    the 32 lanes of an LDS pass (64 banks x 4 B)."""
    for idx in (0, 1, 77, 255):
        banks = [(((idx << 8) | (lane << 3)) // 4) % 64 for lane in range(32)]
        assert len(set(banks)) == 32
        ref = grid_table[(idx << 8) // 2: (idx << 8) // 2 + 4]
        for lane in range(32):
            a = ((idx << 8) | (lane << 3)) // 2
            assert np.array_equal(grid_table[a: a + 4], ref)
    assert not (grid_table & 0x8000).any()  # unsigned entries


def test_decode_model_matches_oracle(grid_table):
    """T16 unit -> v_perm addresses -> replicated table -> sign insertion ->
    db = (2s+1) * d/4: bit-exact with the oracle's dequantized weights."""
    L = gpeed_amd.lib()
    blocks = synth.iq3xxs_blocks(5, 0, 48)
    want = oracle.dequantize(blocks, 48 * 256).reshape(48, 256)
    for bi, raw in enumerate(blocks):
        d = np.float32(np.frombuffer(raw[0:2].tobytes(), np.float16)[0])
        aux = np.frombuffer(raw[66:98].tobytes(), "<u4")
        got = np.empty(256, np.float32)
        for ib in range(8):
            lane = (7 * bi + 13 * ib) % 64
            lb = (lane & 31) << 3
            w = L.gpeed_t16_aux_word(int(aux[ib]))
            sw = full_signs_model(w)
            s = (w >> 16) & 15
            db = np.float32(2 * s + 1) * (d * np.float32(0.25))
            q = raw[2 + 8 * ib: 10 + 8 * ib]
            for l in range(4):
                h = np.empty(8, np.uint16)
                for half in range(2):
                    a = ((int(q[2 * l + half]) << 8) | lb) // 2
                    h[4 * half: 4 * half + 4] = grid_table[a: a + 4]
                for e in range(8):
                    k = 4 * (e // 2) + l
                    h[e] |= ((sw >> (31 - k if e & 1 else 15 - k)) & 1) << 15
                got[32 * ib + 8 * l: 32 * ib + 8 * l + 8] = h.view(np.float16).astype(np.float32) * db
        assert np.array_equal(got.view(np.uint32), want[bi].view(np.uint32)), bi


def test_device_count_without_gpu_is_nonnegative():
    assert gpeed_amd.device_count() >= 0

"""CPU-side checks of the C ABI library (no device compute).

* libgpeed_iq3.so loads and exports every entry point include/gpeed_iq3.h declares;
* host-only geometry and layout helpers answer correctly;
* a numpy model of the GPU decode (T64 lane data -> perm addresses -> the
  library's 64 KiB replicated LDS table -> sign bits from the T64 word ->
  (2s+1) d/4) reproduces the oracle's dequantized weights bit for bit, so the
  layout and table are right before any kernel runs.
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


def test_host_layer_exports_reference_signatures():
    """libgpeed_glm5.so (C++ host layer) exports the reference's kernel-slot
    functions (kernels.h:7-11) and the WeightStore product methods
    (weights.h:41-48) under the glm5 namespace."""
    import subprocess

    lib = os.path.join(ROOT, "gpeed_amd", "libgpeed_glm5.so")
    syms = subprocess.run(["nm", "-D", "--defined-only", "-C", lib], stdout=subprocess.PIPE, text=True,
                          check=True).stdout
    for want in ["glm5::cuda_device_count()", "glm5::cuda_device_name[abi:cxx11](int)",
                 "glm5::cuda_add(float const*, float const*, float*, int)",
                 "glm5::gpu::WeightStore::matvec_quant(std::__cxx11::basic_string<char, std::char_traits<char>, "
                 "std::allocator<char> > const&, unsigned long, int, int, float const*, float*)",
                 "glm5::gpu::WeightStore::matmul_quant(std::__cxx11::basic_string<char, std::char_traits<char>, "
                 "std::allocator<char> > const&, unsigned long, int, int, float const*, int, float*)"]:
        assert want in syms, want
    assert os.access(os.path.join(ROOT, "tests", "cpp", "host_check"), os.X_OK)


def test_geometry():
    L = gpeed_amd.lib()
    assert L.gpeed_iq3xxs_row_bytes(4096) == 16 * 98
    assert L.gpeed_iq3xxs_row_bytes(12288) == 4704
    assert L.gpeed_iq3xxs_row_bytes(100) == 0
    assert L.gpeed_iq3xxs_t64_bytes(6144, 12288) == 6144 * 4704
    assert L.gpeed_iq3xxs_t64_bytes(17, 256) == 64 * 98
    assert L.gpeed_iq3xxs_t64_bytes(1, 200) == 0


def sign_bit(e):
    """T64 bit of the sign of element e = 8l + j of a sub-block, restated from
    the layout definition: pair c = j // 2 of group l owns bits a = 4c + l
    (lower element) and a + 16 (upper element)."""
    l, j = divmod(e, 8)
    return 4 * (j // 2) + l + 16 * (j & 1)


CHAIN = [0, 2, 4, 6, 1, 3, 5, 7]  # group element at chain position k (bit 4k + l)


def aux_t64_model(aux):
    """T64 sign/scale word restated from the layout definition: at chain
    position k < 7 of group l (bit 4k + l) the parity of the group's signs at
    chain positions 0..k; the scale in bits 28..31."""
    out = (aux >> 28) << 28
    for l in range(4):
        p = 0
        for k in range(7):
            p ^= (aux >> (7 * l + CHAIN[k])) & 1
            out |= p << (4 * k + l)
    return out


def test_sign_bits_layout():
    """The 32 element signs use 32 distinct bits; the implied ones (j = 7)
    sit on the scale nibble; group l uses the bits = l (mod 4)."""
    bits = [sign_bit(e) for e in range(32)]
    assert sorted(bits) == list(range(32))
    assert [sign_bit(8 * l + 7) for l in range(4)] == [28, 29, 30, 31]
    assert all(sign_bit(e) % 4 == e // 8 for e in range(32))


def test_sign_chain_positions():
    """Chain position k of group l is bit 4k + l and holds element CHAIN[k],
    which is the layout's sign bit of that element."""
    for l in range(4):
        for k in range(8):
            assert sign_bit(8 * l + CHAIN[k]) == 4 * k + l


def test_aux_word_matches_model():
    L = gpeed_amd.lib()
    words = synth.u64(3, 0, 4000) & np.uint64(0xFFFFFFFF)
    for w in [0, 0xFFFFFFFF, 0x80000000, 0x0FFFFFFF] + [int(v) for v in words]:
        assert L.gpeed_t64_aux_word(w) == aux_t64_model(w), hex(w)


def test_sign_decode_exhaustive():
    """For every group and every 7-bit sign index (and both extreme scales),
    the kernels' decode S = (W & 0x0FFFFFFF) ^ (W << 4) of the library's T64
    word puts each of the group's 8 signs -- the implied eighth, the parity of
    the seven, included (quant.cpp:196-205) -- on its layout bit."""
    L = gpeed_amd.lib()
    for l in range(4):
        for idx in range(128):
            for sc in (0, 15):
                aux = (sc << 28) | (idx << (7 * l))
                w = L.gpeed_t64_aux_word(aux)
                assert w >> 28 == sc
                dec = full_signs_model(w)
                signs = [(idx >> j) & 1 for j in range(7)]
                signs.append(sum(signs) & 1)
                for j in range(8):
                    assert (dec >> sign_bit(8 * l + j)) & 1 == signs[j], (l, idx, j)
                for e in range(32):  # the other groups' signs are all +
                    if e // 8 != l:
                        assert (dec >> sign_bit(e)) & 1 == 0


@pytest.fixture(scope="module")
def grid_table():
    t = np.empty(32768, np.uint16)
    assert gpeed_amd.lib().gpeed_t64_grid_table(t.ctypes.data, t.size) == 0
    assert gpeed_amd.lib().gpeed_t64_grid_table(t.ctypes.data, 100) != 0
    return t


def full_signs_model(w):
    """The kernels' decoded sign word (t64_signs): each chain bit XORed with
    the one before it in its group, the eighth signs shifted up from the
    stored parity at chain position 6 (over the scale nibble)."""
    return ((w & 0x0FFFFFFF) ^ (w << 4)) & 0xFFFFFFFF


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


def rotr(w, r):
    r &= 31
    return ((w >> r) | (w << (32 - r))) & 0xFFFFFFFF if r else w


def test_decode_model_matches_oracle(grid_table):
    """T64 lane data -> v_perm addresses -> replicated table -> sign bits by
    rotate-and-mask (rotr(W, a+17) & 0x80008000) -> (2s+1) * d/4: bit-exact
    with the oracle's dequantized weights."""
    L = gpeed_amd.lib()
    blocks = synth.iq3xxs_blocks(5, 0, 48)
    want = oracle.dequantize(blocks, 48 * 256).reshape(48, 256)
    for bi, raw in enumerate(blocks):
        d = np.float32(np.frombuffer(raw[0:2].tobytes(), np.float16)[0])
        aux = np.frombuffer(raw[66:98].tobytes(), "<u4")
        got = np.empty(256, np.float32)
        lane = (7 * bi) % 64
        lb = (lane & 31) << 3
        for ib in range(8):
            w = L.gpeed_t64_aux_word(int(aux[ib]))
            sw = full_signs_model(w)
            sc = np.float32((w >> 27) | 1)
            q = raw[2 + 8 * ib: 10 + 8 * ib]
            for m in range(8):  # one MFMA: grid index q[m], elements 4m..4m+3
                l, h = m >> 1, m & 1
                a = ((int(q[m]) << 8) | lb) // 2
                v = grid_table[a: a + 4].copy()
                for p in range(2):
                    bits = rotr(sw, 4 * (2 * h + p) + l + 17) & 0x80008000
                    v[2 * p] |= (bits >> 0) & 0x8000
                    v[2 * p + 1] |= (bits >> 16) & 0x8000
                got[32 * ib + 4 * m: 32 * ib + 4 * m + 4] = v.view(np.float16).astype(np.float32) * sc
        got *= d * np.float32(0.25)
        assert np.array_equal(got.view(np.uint32), want[bi].view(np.uint32)), bi


def test_device_count_without_gpu_is_nonnegative():
    assert gpeed_amd.device_count() >= 0


def test_moe_check_buckets_host():
    """The host-side bucket check (gpeed_moe_check_buckets) accepts what the
    router makes and rejects each broken invariant the device plan rejects."""
    T, E, K = 9, 12, 3
    logits = synth.normal(97, 0, T * E).reshape(T, E)
    eptr, tok, _, _ = oracle.moe_route(logits, K, 1)
    gpeed_amd.moe_check_buckets(eptr, tok, E, T, K)
    cases = []
    e = eptr.copy(); e[0] = 1; cases.append((e, tok, "eptr[0]"))
    e = eptr.copy(); e[E] -= 1; cases.append((e, tok, "eptr[n_exp]"))
    nz = int(np.nonzero(np.diff(eptr))[0][0])  # first expert with tokens
    e = eptr.copy(); e[nz + 1] = e[nz] - 1; cases.append((e, tok, "decreases"))
    t = tok.copy(); t[4] = T; cases.append((eptr, t, "out of range"))
    t = tok.copy(); t[4] = -1; cases.append((eptr, t, "out of range"))
    t = tok.copy(); t[0:K + 1] = t[0]; cases.append((eptr, t, "appears"))
    for e, t, what in cases:
        with pytest.raises(gpeed_amd.GpeedError) as err:
            gpeed_amd.moe_check_buckets(e, t, E, T, K)
        assert err.value.code == -1 and what in str(err.value), (what, str(err.value))


@pytest.mark.parametrize("in_dim,out_dim", [(6144, 12288), (12288, 6144), (6144, 3072), (6144, 576),
                                            (6144, 1536), (2048, 6144), (6144, 2048)])
@pytest.mark.parametrize("num_cus", [256, 304, 80])
def test_matmul_workspace_covers_every_smaller_call(in_dim, out_dim, num_cus):
    """A matmul workspace sized for n tokens serves every call with fewer
    tokens (the header's promise): the size is non-decreasing in n_tok on the
    GLM5 dense and latent shapes, for several CU counts (host arithmetic
    only; the split-K count is not monotonic in the token tile count)."""
    f = gpeed_amd.lib().gpeed_iq3xxs_matmul_ws_bytes_for
    sizes = np.array([f(in_dim, out_dim, n, num_cus) for n in range(1, 1025)], np.int64)
    assert (sizes > 0).all()
    prefix_max = np.maximum.accumulate(sizes)
    bad = np.nonzero(sizes < prefix_max)[0]
    assert bad.size == 0, [(int(i) + 1, int(sizes[i]), int(prefix_max[i])) for i in bad[:5]]


def test_matmul_rows_refuses_rows_past_the_offset_range():
    """gpeed_matmul_rows refuses a row length whose per-wavefront row group
    passes the kernels' 2 GiB buffer offsets (before any launch, so this
    runs without a device: the pointers are never dereferenced)."""
    L = gpeed_amd.lib()
    fake = C.c_void_p(1 << 20)
    # (F32 rows go through the dot_f32-order kernel, which addresses rows
    # with 64-bit offsets and has no such limit)
    for dt, in_dim in ((1, 1 << 28), (30, 1 << 28), (8, 1 << 28)):
        rc = L.gpeed_matmul_rows(dt, fake, 8, 0, in_dim, 4, fake, 1, fake, None)
        assert rc == -1, (dt, rc, L.gpeed_last_error())
        assert b"rows too long" in L.gpeed_last_error()

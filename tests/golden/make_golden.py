"""Writes the golden vectors under tests/golden/ from the reference's own CPU code.

Outputs come from oracle/_ref/libgpeed_ref.so, i.e. the reference's
cpp/core/src/{quant,gguf,weights}.cpp compiled unmodified from the reference
checkout (oracle/Makefile), so the committed vectors pin the plain-C oracle
and the GPU kernels where the checkout is absent. Inputs are built here:

* selftest_block: the one IQ3_XXS block the reference's known-answer test
  decodes (tests/gguf_selftest.cpp:69-94 over make_test_gguf.py:139-146):
  fp16 d = 0.0625 followed by 96 bytes from Python's random.Random(1234),
  drawn after the 32 bytes of the Q8_0 tensor, in randint(0, 255) order.
  The draw procedure is restated from the generator's text; only the
  standard library's random module runs.
* edge_blocks: 64 seeded blocks whose fp16 d covers +-0, subnormals, the
  largest finite, +-inf and NaN, plus every scale value 0..15.
* matvec: a 48-row x 1024 weight (seeded), one x and three tokens through
  WeightStore::matvec_quant / matmul_quant (rows 16..47 and 8..39).
* dot: dot_f32 over lengths that exercise the 16-wide, 8-wide and scalar tails.
* quant_formats: for Q8_0, Q2_K, Q3_K, Q6_K, IQ3_S, IQ2_S, IQ4_XS, F16, BF16
  and F32, seeded blocks (the first eight with fp16 scales +-0, the smallest
  subnormal, the largest finite, +-inf, NaN and 1.0) through dequantize, and
  a 12-row x 512 weight with two tokens through WeightStore::matmul_quant
  (rows 2..9).

Run: python tests/golden/make_golden.py   (needs `make -C oracle ref`)
"""
from __future__ import annotations

import os
import random
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from gpeed_amd import synth  # noqa: E402


def ref_dequant(R, raw: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    rc = R.ref_dequantize(18, np.ascontiguousarray(raw).ctypes.data, out, n)
    assert rc == 0
    return out


def selftest_block() -> np.ndarray:
    rng = random.Random(1234)
    _q8 = bytes(rng.randint(0, 255) for _ in range(32))
    body = bytes(rng.randint(0, 255) for _ in range(96))
    return np.frombuffer(struct.pack("<e", 0.0625) + body, dtype=np.uint8).copy()


def edge_blocks() -> np.ndarray:
    blocks = synth.iq3xxs_blocks(7, 0, 64)
    specials = [0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x0200, 0x0400, 0x7BFF, 0xFBFF,
                0x7C00, 0xFC00, 0x7E00, 0x7C01, 0x3C00, 0xBC00, 0x2E66]
    for i, h in enumerate(specials):
        blocks[i, 0:2] = np.frombuffer(struct.pack("<H", h), dtype=np.uint8)
    # every scale value 0..15 in sub-block 0 of blocks 16..31
    for s in range(16):
        aux = int(np.frombuffer(blocks[16 + s, 66:70].tobytes(), "<u4")[0])
        aux = (aux & 0x0FFFFFFF) | (s << 28)
        blocks[16 + s, 66:70] = np.frombuffer(struct.pack("<I", aux), dtype=np.uint8)
    return blocks


SPECIAL_D = [0x0000, 0x8000, 0x0001, 0x7BFF, 0x7C00, 0xFC00, 0x7E00, 0x3C00]


def quant_formats(R) -> dict:
    out = {}
    for dt in [8, 10, 11, 14, 21, 22, 23, 0, 1, 30]:
        if dt in synth.FORMATS:
            elems, nbytes, d_offs = synth.FORMATS[dt]
            raw = synth.quant_blocks(21, dt, dt, 16)
            for i, h in enumerate(SPECIAL_D):
                for off in d_offs:
                    raw[i, off:off + 2] = np.frombuffer(struct.pack("<H", h), dtype=np.uint8)
            n = 16 * elems
        else:
            n = 600
            raw = synth.quant_matrix(21, dt, dt, 1, n).reshape(-1)
            if dt != 0:
                raw[: 2 * len(SPECIAL_D)] = np.frombuffer(struct.pack("<8H", *SPECIAL_D), dtype=np.uint8)
        deq = np.empty(n, np.float32)
        assert R.ref_dequantize(dt, np.ascontiguousarray(raw).ctypes.data, deq, n) == 0
        w = synth.quant_matrix(22, dt, dt, 12, 512)
        X = synth.normal(22, 100 + dt, 2 * 512).reshape(2, 512)
        st = oracle.RefStore(w, 12, 512, name="t.weight", dtype=dt)
        Y = st.matmul(2, 512, 8, X)
        st.close()
        out.update({f"raw_{dt}": raw, f"deq_{dt}": deq, f"w_{dt}": w, f"X_{dt}": X, f"Y_{dt}": Y})
    return out


def main():
    R = oracle.ref()
    if R is None:
        raise SystemExit("oracle/_ref is not built: run `make -C oracle ref`")
    out = {}

    blk = selftest_block()
    np.savez(os.path.join(HERE, "selftest_block.npz"), raw=blk, deq=ref_dequant(R, blk, 256))

    eb = edge_blocks()
    np.savez(os.path.join(HERE, "edge_blocks.npz"), raw=eb, deq=ref_dequant(R, eb, 64 * 256))

    in_dim, n_rows = 1024, 48
    w = synth.iq3xxs_matrix(11, 0, n_rows, in_dim)
    x = synth.normal(11, 100, in_dim)
    X = synth.normal(11, 101, 3 * in_dim).reshape(3, in_dim)
    st = oracle.RefStore(w, n_rows, in_dim)
    y = st.matvec(16, in_dim, 32, x)
    Y = st.matmul(8, in_dim, 32, X)
    st.close()
    np.savez(os.path.join(HERE, "matvec.npz"), w=w, x=x, X=X, y_row16=y, Y_row8=Y)

    lens = np.array([16, 24, 31, 256, 1000], np.int32)
    a = synth.normal(12, 0, 1000)
    b = synth.normal(12, 1, 1000)
    dots = np.array([R.ref_dot_f32(a, b, int(n)) for n in lens], np.float32)
    np.savez(os.path.join(HERE, "dot.npz"), a=a, b=b, lens=lens, dots=dots)
    np.savez(os.path.join(HERE, "quant_formats.npz"), **quant_formats(R))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()

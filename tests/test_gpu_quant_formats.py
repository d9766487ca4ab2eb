"""GPU parity of the other GGUF formats (Q8_0, Q2_K, Q3_K, Q6_K, IQ3_S, IQ2_S,
IQ4_XS, F16, BF16, F32, and IQ3_XXS through the same raw-row kernels),
through the C ABI.

Bars: dequantized weights bit-exact with the reference's vectors and the
oracle (NaN payloads aside); products (fp32 accumulation of exactly
dequantized weights, in another order than the reference) within 2e-5 of
the oracle under rel_err.
"""
import os

import numpy as np
import pytest

import gpeed_amd as G
import oracle
from gpeed_amd import synth
from conftest import ROOT, rel_err

pytestmark = pytest.mark.gpu
GOLD = os.path.join(ROOT, "tests", "golden")
TIGHT = 2e-5
BLOCK_TYPES = [8, 10, 11, 14, 21, 22, 23]
ALL_TYPES = BLOCK_TYPES + [0, 1, 30, 18]


def dev(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def same_bits_or_nan(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) | np.isnan(b)
    return bool(np.array_equal(np.isnan(a), np.isnan(b))
                and np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32)))


@pytest.mark.parametrize("dt", BLOCK_TYPES + [0, 1, 30])
def test_dequant_golden(gpu, dt):
    z = np.load(os.path.join(GOLD, "quant_formats.npz"))
    raw, deq = z[f"raw_{dt}"], z[f"deq_{dt}"]
    out = G.dequantize(dev(raw.reshape(-1), gpu), deq.size, dtype=dt)
    assert same_bits_or_nan(out.cpu().numpy(), deq)


@pytest.mark.parametrize("dt", BLOCK_TYPES + [18])
def test_dequant_random_bytes_vs_oracle(gpu, dt):
    be, bb = oracle.block_geometry(dt)
    n_blk = 5000
    raw = synth.u64(41, dt, n_blk * bb // 8 + 1).view(np.uint8)[: n_blk * bb].copy()
    out = G.dequantize(dev(raw, gpu), n_blk * be, dtype=dt)
    assert same_bits_or_nan(out.cpu().numpy(), oracle.dequantize(raw, n_blk * be, dtype=dt))


@pytest.mark.parametrize("dt", [0, 1, 30])
def test_dequant_scalar_any_length(gpu, dt):
    n = 1001  # not a multiple of 8 or 32
    raw = synth.quant_matrix(42, dt, dt, 1, n).reshape(-1)
    out = G.dequantize(dev(raw, gpu), n, dtype=dt)
    assert same_bits_or_nan(out.cpu().numpy(), oracle.dequantize(raw, n, dtype=dt))


@pytest.mark.parametrize("dt", BLOCK_TYPES + [0, 1, 30])
def test_rows_product_golden(gpu, dt):
    z = np.load(os.path.join(GOLD, "quant_formats.npz"))
    w = z[f"w_{dt}"]
    Y = G.matmul_rows(dt, dev(w.reshape(-1), gpu), 12, 2, 512, 8, dev(z[f"X_{dt}"], gpu))
    assert rel_err(Y.cpu().numpy(), z[f"Y_{dt}"]) < TIGHT


@pytest.mark.parametrize("dt", ALL_TYPES)
@pytest.mark.parametrize("n_tok", [1, 2, 3, 8, 13, 24, 70])
def test_rows_product_vs_oracle(gpu, dt, n_tok):
    """The 8-token-slice kernel below 32 tokens (16 for F16/BF16), the
    fp32-MFMA GEMM from there (24 tokens: F16/BF16 only; F32: dot_f32's order
    at every size); 150 rows and 70 tokens leave partial row tiles (16 rows
    each at 70 tokens: 10 x 2 workgroups) and a partial 64-token tile."""
    in_dim, rows, row0, out_dim = 2048, 200, 37, 150
    w = synth.quant_matrix(43, dt, dt, rows, in_dim)
    X = synth.normal(43, 100 + n_tok, n_tok * in_dim).reshape(n_tok, in_dim)
    Y = G.matmul_rows(dt, dev(w.reshape(-1), gpu), rows, row0, in_dim, out_dim, dev(X, gpu))
    ref = oracle.matmul_rows(dt, w, row0, in_dim, out_dim, X)
    assert rel_err(Y.cpu().numpy(), ref) < TIGHT


@pytest.mark.parametrize("dt", [8, 14, 23])
def test_rows_product_model_width(gpu, dt):
    """A 6144-wide projection slice (the model's hidden size), one token and
    a 32-token prefill chunk."""
    in_dim, rows = 6144, 512
    w = synth.quant_matrix(44, dt, dt, rows, in_dim)
    wd = dev(w.reshape(-1), gpu)
    for n_tok in (1, 32):
        X = synth.normal(44, n_tok, n_tok * in_dim).reshape(n_tok, in_dim)
        Y = G.matmul_rows(dt, wd, rows, 0, in_dim, rows, dev(X, gpu))
        assert rel_err(Y.cpu().numpy(), oracle.matmul_rows(dt, w, 0, in_dim, rows, X)) < TIGHT


@pytest.mark.parametrize("dt", [8, 14, 22, 30])
def test_rows_product_prefill_chunk(gpu, dt):
    """A 512-token prefill chunk (model_batch.cpp:30-95 call matmul_quant with
    n = the chunk) through the fp32-MFMA GEMM over a 6144-wide slice."""
    in_dim, rows, row0, out_dim = 6144, 200, 5, 190
    w = synth.quant_matrix(45, dt, dt, rows, in_dim)
    X = synth.normal(45, 512, 512 * in_dim).reshape(512, in_dim)
    Y = G.matmul_rows(dt, dev(w.reshape(-1), gpu), rows, row0, in_dim, out_dim, dev(X, gpu))
    assert rel_err(Y.cpu().numpy(), oracle.matmul_rows(dt, w, row0, in_dim, out_dim, X)) < TIGHT


@pytest.mark.parametrize("dt", [8, 14])
@pytest.mark.parametrize("rows", [4096, 2048])
def test_rows_product_gemm_row_tiles(gpu, dt, rows):
    """The fp32-MFMA GEMM's row tiles: 4096 rows x 256 tokens take 64-row
    tiles (256 workgroups), 2048 rows 32-row tiles (and the suite's smaller
    cases 16-row tiles)."""
    in_dim, n_tok = 512, 256
    w = synth.quant_matrix(46, dt, dt, rows, in_dim)
    X = synth.normal(46, rows, n_tok * in_dim).reshape(n_tok, in_dim)
    Y = G.matmul_rows(dt, dev(w.reshape(-1), gpu), rows, 0, in_dim, rows, dev(X, gpu))
    assert rel_err(Y.cpu().numpy(), oracle.matmul_rows(dt, w, 0, in_dim, rows, X)) < TIGHT


def test_rows_product_errors(gpu):
    import torch

    w = dev(synth.quant_matrix(45, 8, 8, 4, 64).reshape(-1), gpu)
    x = torch.zeros(64, device=gpu)
    with pytest.raises(G.GpeedError) as e:
        G.matmul_rows(2, w, 4, 0, 64, 4, x)  # Q4_0 is not decoded
    assert e.value.code == -4
    with pytest.raises(G.GpeedError) as e:
        G.matmul_rows(8, w, 4, 1, 64, 4, x)  # rows past the tensor
    assert e.value.code == -1
    with pytest.raises(G.GpeedError) as e:
        G.matmul_rows(10, w, 4, 0, 64, 4, x)  # Q2_K rows need in_dim % 256 == 0
    assert e.value.code == -3
    with pytest.raises(G.GpeedError) as e:
        G.dequantize(w, 100, dtype=10)
    assert e.value.code == -2


def test_weight_store_mixed_types(gpu):
    """The Python store keeps IQ3_XXS tensors in T64 and the others as GGUF
    rows; matvec_quant / matmul_quant by name match the oracle either way."""
    ws = G.WeightStore(gpu)
    in_dim = 1024
    mats = {}
    for dt in (8, 14, 23, 18, 30):
        w = synth.quant_matrix(46, dt, dt, 128, in_dim)
        ws.add(f"t{dt}.weight", w, in_dim, 128, dtype=dt)
        mats[dt] = w
    x = synth.normal(46, 1, in_dim)
    X = synth.normal(46, 2, 5 * in_dim).reshape(5, in_dim)
    for dt, w in mats.items():
        y = ws.matvec_quant(f"t{dt}.weight", 64, in_dim, 64, x)
        assert rel_err(y, oracle.matmul_rows(dt, w, 64, in_dim, 64, x)[0]) < TIGHT
        Y = ws.matmul_quant(f"t{dt}.weight", 0, in_dim, 128, X, 5)
        assert rel_err(Y, oracle.matmul_rows(dt, w, 0, in_dim, 128, X)) < TIGHT


def test_host_dequantize_reference_signature(gpu, tmp_path):
    """glm5::gpu::dequantize(DType, const void*, float*, uint64_t) (quant.h:18-22)
    over host arrays, through the C++ layer, and its error for a type that
    is not decoded."""
    import subprocess

    exe = os.path.join(ROOT, "tests", "cpp", "host_check")
    z = np.load(os.path.join(GOLD, "quant_formats.npz"))
    for dt in (8, 10, 11, 14, 21, 22, 23, 1, 30, 0):
        raw, deq = z[f"raw_{dt}"], z[f"deq_{dt}"]
        raw.tofile(tmp_path / "raw.bin")
        r = subprocess.run([exe, "dequant", str(dt), str(tmp_path / "raw.bin"), str(deq.size),
                            str(tmp_path / "out.bin")], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stdout + r.stderr
        assert same_bits_or_nan(np.fromfile(tmp_path / "out.bin", np.float32), deq), dt
    r = subprocess.run([exe, "dequant", "2", str(tmp_path / "raw.bin"), "32", str(tmp_path / "out.bin")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "dequantize: unimplemented type Q4_0" in (r.stdout + r.stderr)


@pytest.mark.parametrize("in_dim", [6144, 1000, 24, 7])
@pytest.mark.parametrize("n_tok", [1, 5, 300])
def test_f32_rows_bitwise_reference_order(gpu, in_dim, n_tok):
    """F32 rows (matmul_quant of an F32 tensor: the router ffn_gate_inp,
    model_batch.cpp:172) are multiplied in dot_f32's own order (simd.h:
    12-37: 16 fma chains, their add tree, the fma tail), so the products are
    bitwise the oracle's, which is bitwise the reference's build; lengths
    with and without the 8-wide step and the tail (7 columns: the dword
    copies of rows that are not a multiple of 4 long), 4 x 4 tiles (1 and 5 tokens)
    and 8 x 8 tiles (300 tokens x 60 rows: 304 tiles)."""
    rows = 64
    w = (synth.normal(88, in_dim, rows * in_dim) * np.float32(0.05)).astype(np.float32).reshape(rows, in_dim)
    X = synth.normal(88, 1, n_tok * in_dim).reshape(n_tok, in_dim)
    Y = G.matmul_rows(0, dev(w.reshape(-1).view(np.uint8), gpu), rows, 3, in_dim, 60, dev(X, gpu)).cpu().numpy()
    ref = oracle.matmul_rows(0, w.view(np.uint8), 3, in_dim, 60, X)
    assert np.array_equal(Y.reshape(ref.shape).view(np.uint32), ref.view(np.uint32))

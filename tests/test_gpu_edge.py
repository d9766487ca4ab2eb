"""GPU parity of every IQ3_XXS product kernel on edge-case block scales and
outlier activations (tests/edge_cases.py builds the weights).

The blocks carry d = +-0, subnormals, +-65504, d jumping by 2^+-20 between
consecutive blocks (unequal mantissas too) and, in the non-finite cases, +inf,
-inf or NaN. Bars (quant.cpp:186-210, weights.cpp:86-203): finite outputs
within 2e-5 of the oracle under rel_err, taken per row kind; non-finite
outputs of the same class (the reference sums an infinite block's +-inf
products of both signs, so such a row is NaN). The oracle is pinned to the
reference's own build on these matrices by
tests/test_oracle.py::test_oracle_edge_blocks_bitwise_vs_reference_build.
"""
import numpy as np
import pytest

import gpeed_amd as G
import oracle
from edge_cases import check, edge_matrix, outlier_rows, row_kinds
from gpeed_amd import synth

pytestmark = pytest.mark.gpu
TIGHT = 2e-5


def dev(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    return t.cpu().numpy()


def bf16_round(x):
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("nonfinite", [False, True])
@pytest.mark.parametrize("n_rows,in_dim,row0,out_dim", [(192, 4096, 0, 192), (256, 2048, 64, 136),
                                                        (6144, 12288, 0, 6144)])
def test_matvec_edge(gpu, nonfinite, n_rows, in_dim, row0, out_dim):
    """k_gemv_t64 with the activation prepared in the kernel (matvec) and
    from prepared images (gemv_act, 1..8 vectors), and the raw-row GEMV."""
    w = edge_matrix(70, 0, n_rows, in_dim, nonfinite)
    t64 = G.tile(dev(w.reshape(-1), gpu), n_rows, in_dim)
    kinds = row_kinds(n_rows)[row0:row0 + out_dim]
    x = synth.normal(70, 1, in_dim)
    ref = oracle.matvec(w, row0, in_dim, out_dim, x)
    check(host(G.matvec(t64, n_rows, row0, in_dim, out_dim, dev(x, gpu))), ref, TIGHT, kinds, "matvec")
    check(host(G.matvec_raw(dev(w.reshape(-1), gpu), n_rows, row0, in_dim, out_dim, dev(x, gpu))), ref, TIGHT,
          kinds, "matvec_raw")
    for n_tok in (1, 2, 5, 8):
        X = synth.normal(70, 2 + n_tok, n_tok * in_dim).reshape(n_tok, in_dim)
        act = G.prep_act(dev(X, gpu), G.act_buffer(in_dim, n_tok, gpu))
        Y = host(G.gemv_act(t64, n_rows, row0, in_dim, out_dim, act, n_tok))
        check(Y, oracle.matmul(w, row0, in_dim, out_dim, X), TIGHT, kinds, f"gemv_act {n_tok}")


@pytest.mark.parametrize("nonfinite", [False, True])
@pytest.mark.parametrize("M,x_bf16", [(40, True), (100, True), (300, True), (16, False), (70, False)])
def test_gemm_edge(gpu, nonfinite, M, x_bf16):
    """k_gemm3 (bf16, <= 64 tokens), k_gemm5 (bf16 above 64 tokens; fp32 X as
    hi + lo images, split K at few tiles): the running-d rescale across
    blocks of +-0, subnormal, 65504 and 2^+-20 jumps, and NaN poison."""
    n_rows, in_dim = 448, 4096
    w = edge_matrix(71, M, n_rows, in_dim, nonfinite)
    t64 = G.tile(dev(w.reshape(-1), gpu), n_rows, in_dim)
    X = synth.normal(71, 1000 + M, M * in_dim).reshape(M, in_dim)
    import torch

    if x_bf16:
        X = bf16_round(X)
        Xd = dev(X, gpu).to(torch.bfloat16)
    else:
        Xd = dev(X, gpu)
    Y = host(G.gemm(t64, n_rows, 64, in_dim, 320, Xd))
    check(Y, oracle.matmul(w, 64, in_dim, 320, X), TIGHT, row_kinds(n_rows)[64:384], f"gemm {M}")


def test_gemm_wide_form_edge(gpu):
    """k_gemm6 (32x32x16 MFMAs on 256-row tiles, where the tiles cover every
    CU: 2048 bf16 tokens x 4096 rows) on edge rows, checked on two 128-row
    slices (the first and last row tiles) with non-finite scales."""
    import torch

    n_rows, in_dim, M = 4096, 2048, 2048
    w = edge_matrix(72, 0, n_rows, in_dim, nonfinite=True)
    t64 = G.tile(dev(w.reshape(-1), gpu), n_rows, in_dim)
    X = bf16_round(synth.normal(72, 1, M * in_dim).reshape(M, in_dim))
    Y = host(G.gemm(t64, n_rows, 0, in_dim, n_rows, dev(X, gpu).to(torch.bfloat16)))
    kinds = row_kinds(n_rows)
    for r0 in (0, n_rows - 128):
        ref = oracle.matmul(w, r0, in_dim, 128, X)
        check(Y[:, r0:r0 + 128], ref, TIGHT, kinds[r0:r0 + 128], f"gemm6 rows {r0}")


@pytest.mark.parametrize("n_tok", [5, 40])
def test_matmul_outlier_activations(gpu, n_tok):
    """matmul_quant (fp32 X) with a few channels per token at 1000x the row's
    rms: the GEMV scales X per 256 values, the GEMM (from 9 tokens) once per
    token row, so the GEMM's fp16 hi + lo images carry the other channels
    1000x below the row's largest."""
    n_rows, in_dim = 256, 6144
    w = edge_matrix(73, n_tok, n_rows, in_dim)
    t64 = G.tile(dev(w.reshape(-1), gpu), n_rows, in_dim)
    X = outlier_rows(synth.normal(73, 1, n_tok * in_dim).reshape(n_tok, in_dim), 73)
    Y = host(G.matmul(t64, n_rows, 0, in_dim, n_rows, dev(X, gpu)))
    check(Y, oracle.matmul(w, 0, in_dim, n_rows, X), TIGHT, row_kinds(n_rows), f"matmul {n_tok}")


def test_gemm_bf16_outlier_activations(gpu):
    """bf16 X with outlier channels (1000x rms) through the 128-token tiles."""
    import torch

    n_rows, in_dim, M = 384, 4096, 200
    w = edge_matrix(74, 0, n_rows, in_dim)
    t64 = G.tile(dev(w.reshape(-1), gpu), n_rows, in_dim)
    X = bf16_round(outlier_rows(synth.normal(74, 1, M * in_dim).reshape(M, in_dim), 74))
    Y = host(G.gemm(t64, n_rows, 0, in_dim, n_rows, dev(X, gpu).to(torch.bfloat16)))
    check(Y, oracle.matmul(w, 0, in_dim, n_rows, X), TIGHT, row_kinds(n_rows), "gemm bf16 outliers")


@pytest.mark.parametrize("nonfinite", [False, True])
def test_matmul_rows_iq3_edge(gpu, nonfinite):
    """The raw-row products over GGUF rows for IQ3_XXS edge blocks: the
    8-token-slice kernel (1, 2 and 9 tokens) and the fp32-MFMA GEMM (40)."""
    n_rows, in_dim = 200, 2048
    w = edge_matrix(75, 0, n_rows, in_dim, nonfinite)
    wd = dev(w.reshape(-1), gpu)
    for n_tok in (1, 2, 9, 40):
        X = synth.normal(75, n_tok, n_tok * in_dim).reshape(n_tok, in_dim)
        Y = host(G.matmul_rows(18, wd, n_rows, 3, in_dim, 190, dev(X, gpu)))
        check(Y, oracle.matmul_rows(18, w, 3, in_dim, 190, X), TIGHT, row_kinds(n_rows)[3:193],
              f"matmul_rows {n_tok}")


def test_dense_mlp_edge(gpu):
    """Model::dense_mlp (gate+up launch with the SwiGLU epilogue, then down)
    with edge scales in all three tensors; finite scales, so the output is
    finite (65504-scaled gate/up rows meet the SwiGLU clamp)."""
    H, I = 1024, 2048
    wg = edge_matrix(76, 0, I, H)
    wu = edge_matrix(76, 1, I, H)
    wd = edge_matrix(76, 2, H, I)
    t = lambda a, r, c: G.tile(dev(a.reshape(-1), gpu), r, c)  # noqa: E731
    x = synth.normal(76, 3, H)
    y = host(G.dense_mlp(t(wg, I, H), t(wu, I, H), t(wd, H, I), H, I, dev(x, gpu), 10.0))
    ref = oracle.dense_mlp(wg, wu, wd, H, I, x.reshape(1, H), 10.0)[0]
    check(y, ref, TIGHT, row_kinds(H), "dense_mlp")


def test_dense_mlp_nan_gate_row(gpu):
    """A NaN scale in one gate row: the reference's SwiGLU keeps the NaN
    (std::min(NaN, lim) is NaN) and every down output becomes NaN."""
    H, I = 512, 1024
    wg = edge_matrix(77, 0, I, H, nonfinite=True)
    wu = synth.iq3xxs_matrix(77, 1, I, H)
    wd = synth.iq3xxs_matrix(77, 2, H, I)
    t = lambda a, r, c: G.tile(dev(a.reshape(-1), gpu), r, c)  # noqa: E731
    x = synth.normal(77, 3, H)
    y = host(G.dense_mlp(t(wg, I, H), t(wu, I, H), t(wd, H, I), H, I, dev(x, gpu), 10.0))
    ref = oracle.dense_mlp(wg, wu, wd, H, I, x.reshape(1, H), 10.0)[0]
    assert np.isnan(ref).all()
    check(y, ref, TIGHT, None, "dense_mlp nan")


@pytest.mark.parametrize("nonfinite", [False, True])
def test_moe_batch_edge(gpu, nonfinite):
    """The routed step (grouped GEMVs, shared expert, combine) with edge
    scales in every expert tensor; with non-finite scales, the NaN rows of
    gate/up and down reach the tokens routed to those experts."""
    T, E, K, H, I = 12, 8, 3, 1024, 512
    wg = edge_matrix(78, 0, E * I, H, nonfinite)
    wu = edge_matrix(78, 1, E * I, H)
    wd = edge_matrix(78, 2, E * H, I, nonfinite)
    sh = (edge_matrix(78, 5, I, H), edge_matrix(78, 6, I, H), edge_matrix(78, 7, H, I))
    X = synth.normal(78, 3, T * H).reshape(T, H)
    logits = synth.normal(78, 4, T * E).reshape(T, E)
    t = lambda a, r, c: G.tile(dev(a.reshape(-1), gpu), r, c)  # noqa: E731
    tsh = (t(sh[0], I, H), t(sh[1], I, H), t(sh[2], H, I))
    Y = host(G.moe_batch(dev(logits, gpu), dev(X, gpu), t(wg, E * I, H), t(wu, E * I, H), t(wd, E * H, I), E, H,
                         I, K, 1, None, 1.0, True, 10.0, shared=tsh))
    ref = oracle.moe_batch(logits, X, wg, wu, wd, H, I, K, 1, None, 1.0, True, 10.0, shared=sh)
    check(Y, ref, TIGHT, row_kinds(H), "moe_batch")

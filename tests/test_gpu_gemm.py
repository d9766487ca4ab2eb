"""GPU parity tests for the prefill GEMM (gpeed_iq3xxs_gemm): W dequantized
into LDS as exact fp16 q*(2s+1), X as fp16 images (bf16 input exact, fp32
input as hi+lo), fp32 MFMA accumulation. Checked against the oracle's
matmul_quant (weights.cpp:86-165) on the same bf16-representable or fp32
inputs: rel_err < 2e-5 (north-star bar 1e-3). Full-size shapes are checked on
row slices the CPU oracle finishes quickly."""
import numpy as np
import pytest

import gpeed_amd as G
import oracle
from gpeed_amd import synth
from conftest import rel_err

pytestmark = pytest.mark.gpu
TIGHT = 2e-5


def dev(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def bf16_round(x):
    """Round-to-nearest-even to bf16, returned as float32 (exactly representable)."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def as_bf16_tensor(xf, device):
    import torch

    return dev(xf, device).to(torch.bfloat16)  # exact: xf holds bf16 values


@pytest.mark.parametrize("M,N,K,row0,x_bf16", [
    (100, 200, 768, 64, True),      # partial token and row tiles, 3 blocks
    (128, 128, 256, 0, False),      # one tile, fp32 input (hi + lo images)
    (300, 384, 1536, 0, True),
    (64, 576, 6144, 0, False),      # the decode-mix latent projection, fp32
    (37, 1536, 6144, 0, True),
])
def test_gemm_small(gpu, M, N, K, row0, x_bf16):
    n_rows = row0 + N
    w = synth.iq3xxs_matrix(90, M, n_rows, K)
    X = synth.normal(90, 1000 + K, M * K).reshape(M, K)
    if x_bf16:
        X = bf16_round(X)
    t64 = G.tile(dev(w.reshape(-1), gpu), n_rows, K)
    Xd = as_bf16_tensor(X, gpu) if x_bf16 else dev(X, gpu)
    Y = G.gemm(t64, n_rows, row0, K, N, Xd).cpu().numpy()
    ref = oracle.matmul(w, row0, K, N, X)
    e = max(rel_err(Y[t], ref[t]) for t in range(M))
    assert e < TIGHT, e


@pytest.mark.parametrize("M", [512, 2048])
def test_gemm_prefill_full_size(gpu, M):
    """W 12288 x 6144, X bf16 [M, 6144]: every output computed on the GPU,
    six 64-row slices (all tokens) checked against the oracle."""
    N, K = 12288, 6144
    w = synth.iq3xxs_matrix(91, 0, N, K)
    X = bf16_round(synth.normal(91, M, M * K).reshape(M, K))
    t64 = G.tile(dev(w.reshape(-1), gpu), N, K)
    Y = G.gemm(t64, N, 0, K, N, as_bf16_tensor(X, gpu)).cpu().numpy()
    assert np.isfinite(Y).all()
    for r0 in (0, 64 * 37, 64 * 95, 64 * 128, 64 * 160, N - 64):
        ref = oracle.matmul(w, r0, K, 64, X[:: max(1, M // 128)])
        got = Y[:: max(1, M // 128), r0:r0 + 64]
        e = max(rel_err(got[t], ref[t]) for t in range(ref.shape[0]))
        assert e < TIGHT, (r0, e)


def test_gemm_matches_gemv(gpu):
    """Same fp32 tokens through the GEMM and the multi-token GEMV."""
    M, N, K = 8, 640, 2048
    w = synth.iq3xxs_matrix(92, 0, N, K)
    X = synth.normal(92, 1, M * K).reshape(M, K)
    t64 = G.tile(dev(w.reshape(-1), gpu), N, K)
    Yg = G.gemm(t64, N, 0, K, N, dev(X, gpu)).cpu().numpy()
    Yv = G.matmul(t64, N, 0, K, N, dev(X, gpu)).cpu().numpy()
    assert max(rel_err(Yg[t], Yv[t]) for t in range(M)) < TIGHT


def test_gemm_errors(gpu):
    import torch

    w = synth.iq3xxs_matrix(93, 0, 128, 512)
    t64 = G.tile(dev(w.reshape(-1), gpu), 128, 512)
    X = torch.zeros(4, 512, device=gpu)
    with pytest.raises(G.GpeedError) as e:
        G.gemm(t64, 128, 32, 512, 64, X)
    assert e.value.code == -6
    with pytest.raises(G.GpeedError) as e:
        G.gemm(t64, 128, 0, 500, 64, X)
    assert e.value.code == -3

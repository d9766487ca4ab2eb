"""GPU parity tests for the prefill GEMM (gpeed_iq3xxs_gemm): W dequantized
into LDS as exact fp16 q*(2s+1), X as fp16 images (bf16 input exact, fp32
input as hi+lo), fp32 MFMA accumulation. Checked against the oracle's
matmul_quant (weights.cpp:86-165) on the same bf16-representable or fp32
inputs: rel_err < 2e-5 (the parity bar is 1e-3). Full-size shapes are checked on
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
    (1, 64, 256, 0, True),          # one token, one row tile, one block
    (65, 192, 512, 0, False),       # one token past the 64-token tile: 128-token tiles, fp32 input
    # X preparation with 2, 4 and 8 register chunks per thread, and the
    # two-pass form past 2048 chunks per row (K = 65 blocks: an odd block
    # count under K halves keeps its split count)
    (16, 64, 4096, 0, False),
    (80, 64, 8192, 0, True),
    (9, 64, 16384, 0, False),
    (70, 64, 16640, 0, True),
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


@pytest.mark.parametrize("N,K,x_bf16", [
    (576, 6144, False),    # MLA kv_a at 64 tokens, fp32 X: 3 row tiles, K split 8 ways
    (1536, 6144, True),    # q_a
    (12288, 6144, False),  # shared-expert gate/up: 64 row tiles, K split 4 ways
    (6144, 12288, True),   # shared-expert down: 32 row tiles, K split 8 ways
])
def test_gemm_decode_mix_split_k(gpu, N, K, x_bf16):
    """64 concurrent decode tokens through the latent projections and the
    shared-expert FFN shapes: few result tiles, so K is split over
    workgroups and the partials added in split order. Row slices against
    the oracle; a second call on the same workspace gives the same bits
    (its tickets are back at zero)."""
    import torch

    M = 64
    w = synth.iq3xxs_matrix(94, N, N, K)
    X = synth.normal(94, K, M * K).reshape(M, K)
    if x_bf16:
        X = bf16_round(X)
    t64 = G.tile(dev(w.reshape(-1), gpu), N, K)
    Xd = as_bf16_tensor(X, gpu) if x_bf16 else dev(X, gpu)
    xd = G.X_BF16 if x_bf16 else G.X_F32
    ws = torch.zeros(G.lib().gpeed_iq3xxs_gemm_ws_bytes(M, K, N, xd), dtype=torch.uint8, device=gpu)
    Y = G.gemm(t64, N, 0, K, N, Xd, ws=ws).cpu().numpy()
    for r0 in sorted({0, 64 * ((N // 64) // 2), N - 64}):
        ref = oracle.matmul(w, r0, K, 64, X[::4])
        e = max(rel_err(Y[::4, r0:r0 + 64][t], ref[t]) for t in range(ref.shape[0]))
        assert e < TIGHT, (r0, e)
    Y2 = G.gemm(t64, N, 0, K, N, Xd, ws=ws).cpu().numpy()
    assert np.array_equal(Y, Y2)


# (16, 256, 16640): the SwiGLU images of a row past 2048 register chunks
# (two-pass preparation); (24, 512, 4096): two chunks per thread
@pytest.mark.parametrize("M,H,I", [(64, 1024, 2048), (200, 512, 768), (64, 6144, 12288), (16, 256, 16640),
                                   (24, 512, 4096)])
def test_dense_mlp_batch_gemm(gpu, M, H, I):
    """dense_mlp_batch (model_batch.cpp:145-163) through the GEMM: gate and
    up GEMMs, then the down GEMM with SwiGLU formed while its images are
    prepared (gpeed_iq3xxs_gemm_swiglu). Against the oracle's dense MLP
    (silu through the device expf differs by ulps from glibc's); the full
    decode-mix shape on token slices."""
    wg = synth.iq3xxs_matrix(95, 0, I, H)
    wu = synth.iq3xxs_matrix(95, 1, I, H)
    wd = synth.iq3xxs_matrix(95, 2, H, I)
    X = synth.normal(95, M, M * H).reshape(M, H) * np.float32(3.0)
    tg, tu, td = (G.tile(dev(a.reshape(-1), gpu), r, c) for a, r, c in ((wg, I, H), (wu, I, H), (wd, H, I)))
    Xd = dev(X, gpu)
    Gm = G.gemm(tg, I, 0, H, I, Xd)
    Um = G.gemm(tu, I, 0, H, I, Xd)
    Y = G.gemm_swiglu(td, H, 0, I, H, Gm, Um, 10.0).cpu().numpy()
    step = 1 if H * I <= 1 << 22 else 16
    ref = oracle.dense_mlp(wg, wu, wd, H, I, X[::step], 10.0)
    e = max(rel_err(Y[::step][t], ref[t]) for t in range(ref.shape[0]))
    assert e < 1e-4, e


@pytest.mark.parametrize("M,Na,Nb,K,row0a,row0b,x_bf16", [
    (64, 576, 1536, 6144, 0, 0, False),    # decode-mix kv_a + q_a, K split over workgroups
    (100, 200, 330, 768, 64, 128, True),   # partial token and row tiles, row offsets
    (200, 384, 192, 512, 0, 64, False),    # fp32 X over 64 tokens (the hi/lo form)
    (512, 6144, 6144, 1024, 0, 0, True),   # one K split, XCD bands across both tensors
])
def test_gemm2_two_tensors(gpu, M, Na, Nb, K, row0a, row0b, x_bf16):
    """Two products on one X in one launch (gpeed_iq3xxs_gemm2): each output
    against the oracle's matmul_quant of its own tensor, on token slices; a
    second call on the same workspace gives the same bits."""
    import torch

    wa = synth.iq3xxs_matrix(96, 0, row0a + Na, K)
    wb = synth.iq3xxs_matrix(96, 1, row0b + Nb, K)
    X = synth.normal(96, M, M * K).reshape(M, K)
    if x_bf16:
        X = bf16_round(X)
    ta = G.tile(dev(wa.reshape(-1), gpu), row0a + Na, K)
    tb = G.tile(dev(wb.reshape(-1), gpu), row0b + Nb, K)
    Xd = as_bf16_tensor(X, gpu) if x_bf16 else dev(X, gpu)
    xd = G.X_BF16 if x_bf16 else G.X_F32
    ws = torch.zeros(G.lib().gpeed_iq3xxs_gemm2_ws_bytes(M, K, Na, Nb, xd), dtype=torch.uint8, device=gpu)
    Ya, Yb = G.gemm2(ta, row0a + Na, row0a, Na, tb, row0b + Nb, row0b, Nb, K, Xd, ws=ws)
    Ya, Yb = Ya.cpu().numpy(), Yb.cpu().numpy()
    step = 1 if M * K <= 1 << 16 else 8
    for Y, w, r0, N in ((Ya, wa, row0a, Na), (Yb, wb, row0b, Nb)):
        ref = oracle.matmul(w, r0, K, N, X[::step])
        e = max(rel_err(Y[::step][t], ref[t]) for t in range(ref.shape[0]))
        assert e < TIGHT, (N, e)
    Ya2, Yb2 = G.gemm2(ta, row0a + Na, row0a, Na, tb, row0b + Nb, row0b, Nb, K, Xd, ws=ws)
    assert np.array_equal(Ya, Ya2.cpu().numpy()) and np.array_equal(Yb, Yb2.cpu().numpy())


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


@pytest.mark.parametrize("M,H,I,extra,x_bf16", [
    (64, 2048, 4096, (576, 1536), False),   # the down launch holds two problems (balanced K splits)
    (37, 2048, 4096, (192,), False),        # partial token tile, one extra tensor
    (1, 1024, 2048, (), False),             # no extra tensor: gate+up, SwiGLU images, down
    (100, 1024, 2048, (320, 64), False),    # over 64 tokens: the extra tensors as a launch of their own
    (40, 1024, 2048, (576,), True),         # bf16 X: likewise
])
def test_mlp_gemm(gpu, M, H, I, extra, x_bf16):
    """dense_mlp_batch as GEMMs (gpeed_iq3xxs_mlp_gemm, model_batch.cpp:145-163)
    with up to two extra tensors of the same X computed in the down launch:
    every output against the oracle (dense_mlp, matmul_quant), and a second
    call on the same workspace gives the same bits."""
    import torch

    wg = synth.iq3xxs_matrix(97, 0, I, H)
    wu = synth.iq3xxs_matrix(97, 1, I, H)
    wd = synth.iq3xxs_matrix(97, 2, H, I)
    we = [synth.iq3xxs_matrix(97, 3 + i, r, H) for i, r in enumerate(extra)]
    X = synth.normal(97, M, M * H).reshape(M, H)
    if x_bf16:
        X = bf16_round(X)
    t = lambda a, r, c: G.tile(dev(a.reshape(-1), gpu), r, c)  # noqa: E731
    tg, tu, td = t(wg, I, H), t(wu, I, H), t(wd, H, I)
    te = [(t(w, r, H), r) for w, r in zip(we, extra)]
    Xd = as_bf16_tensor(X, gpu) if x_bf16 else dev(X, gpu)
    ws = G.mlp_gemm_workspace(M, H, I, G.X_BF16 if x_bf16 else G.X_F32, list(extra), gpu)
    Y, Ye = G.mlp_gemm(tg, tu, td, H, I, Xd, 10.0, extra=te, ws=ws)
    Y, Ye = Y.cpu().numpy(), [y.cpu().numpy() for y in Ye]
    ref = oracle.dense_mlp(wg, wu, wd, H, I, X, 10.0)
    assert max(rel_err(Y[i], ref[i]) for i in range(M)) < TIGHT
    for y, w, r in zip(Ye, we, extra):
        ref_e = oracle.matmul(w, 0, H, r, X)
        assert max(rel_err(y[i], ref_e[i]) for i in range(M)) < TIGHT, r
    Y2, Ye2 = G.mlp_gemm(tg, tu, td, H, I, Xd, 10.0, extra=te, ws=ws)
    assert np.array_equal(Y, Y2.cpu().numpy())
    assert all(np.array_equal(a, b.cpu().numpy()) for a, b in zip(Ye, Ye2))


def test_mlp_gemm_decode_mix_full_size(gpu):
    """The decode-mix shapes: 64 fp32 tokens through gate/up 12288x6144 and
    down 6144x12288 with kv_a 576x6144 and q_a 1536x6144 in the down launch;
    the five outputs against the oracle on 8 of the tokens."""
    H, I, M = 6144, 12288, 64
    wg = synth.iq3xxs_matrix(98, 0, I, H)
    wu = synth.iq3xxs_matrix(98, 1, I, H)
    wd = synth.iq3xxs_matrix(98, 2, H, I)
    wk = synth.iq3xxs_matrix(98, 3, 576, H)
    wq = synth.iq3xxs_matrix(98, 4, 1536, H)
    X = synth.normal(98, 5, M * H).reshape(M, H)
    t = lambda a, r, c: G.tile(dev(a.reshape(-1), gpu), r, c)  # noqa: E731
    Y, (Yk, Yq) = G.mlp_gemm(t(wg, I, H), t(wu, I, H), t(wd, H, I), H, I, dev(X, gpu), 10.0,
                             extra=((t(wk, 576, H), 576), (t(wq, 1536, H), 1536)))
    sel = np.arange(0, M, 8)
    ref = oracle.dense_mlp(wg, wu, wd, H, I, X[sel], 10.0)
    Y, Yk, Yq = Y.cpu().numpy()[sel], Yk.cpu().numpy()[sel], Yq.cpu().numpy()[sel]
    assert max(rel_err(Y[i], ref[i]) for i in range(len(sel))) < TIGHT
    for y, w, r in ((Yk, wk, 576), (Yq, wq, 1536)):
        ref_e = oracle.matmul(w, 0, H, r, X[sel])
        assert max(rel_err(y[i], ref_e[i]) for i in range(len(sel))) < TIGHT, r

"""GPU parity tests for the IQ3_XXS path, through the C ABI (gpeed_amd -> libgpeed_iq3.so).

Bars: dequantized weights and layout conversions bit-exact; products within
1e-3 of the oracle under rel_err (conftest.rel_err, the parity bar) and,
as a tighter design check, within 2e-5 -- the MFMA path multiplies exactly
(fp16 signed grid values times fp16 hi/lo activation halves, then the exact
(2s+1) and d/4 scales), so only fp32 accumulation order separates it from the
CPU. Dropping the low activation half would still pass 1e-3 (it costs
~3e-4), so the tight bound is what catches it.
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
TOL = 1e-3
TIGHT = 2e-5


def dev(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    return t.cpu().numpy()


def same_bits_or_nan(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) | np.isnan(b)
    return bool(np.array_equal(np.isnan(a), np.isnan(b))
                and np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32)))


# ------------------------------------------------------------------ dequant / layout

@pytest.mark.parametrize("name", ["selftest_block", "edge_blocks"])
def test_dequant_golden(gpu, name):
    z = np.load(os.path.join(GOLD, name + ".npz"))
    n = z["raw"].size // 98 * 256
    out = G.dequantize(dev(z["raw"].reshape(-1), gpu), n)
    assert same_bits_or_nan(host(out), z["deq"])


def test_dequant_random_vs_oracle(gpu):
    raw = synth.iq3xxs_blocks(41, 0, 3000)
    out = G.dequantize(dev(raw.reshape(-1), gpu), 3000 * 256)
    assert same_bits_or_nan(host(out), oracle.dequantize(raw, 3000 * 256))


def test_dequant_errors(gpu):
    import torch

    raw = torch.zeros(98, dtype=torch.uint8, device=gpu)
    with pytest.raises(G.GpeedError) as e:
        G.dequantize(raw, 255)
    assert e.value.code == -2
    with pytest.raises(G.GpeedError) as e:
        G.dequantize(raw, 256, dtype=12)
    assert e.value.code == -4


@pytest.mark.parametrize("n_rows,in_dim", [(64, 256), (65, 768), (130, 4096), (45, 2048)])
def test_tile_roundtrip(gpu, n_rows, in_dim):
    raw = synth.iq3xxs_matrix(42, n_rows, n_rows, in_dim)
    t64 = G.tile(dev(raw.reshape(-1), gpu), n_rows, in_dim)
    assert t64.numel() == ((n_rows + 63) // 64) * 64 * in_dim // 256 * 98
    back = host(G.untile(t64, n_rows, in_dim))
    assert np.array_equal(back, raw.reshape(-1))


def test_tile_record_layout(gpu):
    """One record checked field by field against the layout definition;
    padding rows of the partial tile are zero bytes."""
    n_rows, in_dim = 50, 512
    raw = synth.iq3xxs_matrix(43, 0, n_rows, in_dim)
    t64 = host(G.tile(dev(raw.reshape(-1), gpu), n_rows, in_dim))
    L = G.lib()
    rec = t64[6272:2 * 6272]  # tile 0, block 1
    for n in range(64):
        seq = np.concatenate([rec[u * 1024 + 16 * n: u * 1024 + 16 * n + 16] for u in range(6)]).view("<u4")
        d = rec[6144 + 2 * n: 6146 + 2 * n]
        if n >= n_rows:
            assert not seq.any() and not d.any()
            continue
        blk = raw[n, 98:196]
        assert np.array_equal(d, blk[0:2])
        for ib in range(8):
            assert seq[3 * ib: 3 * ib + 2].tobytes() == blk[2 + 8 * ib: 10 + 8 * ib].tobytes()
            aux = int(np.frombuffer(blk[66 + 4 * ib: 70 + 4 * ib].tobytes(), "<u4")[0])
            assert int(seq[3 * ib + 2]) == L.gpeed_t64_aux_word(aux)


# ------------------------------------------------------------------ GEMV

def run_matvec(gpu, w, n_rows, in_dim, row0, out_dim, x):
    t64 = G.tile(dev(w.reshape(-1), gpu), n_rows, in_dim)
    return host(G.matvec(t64, n_rows, row0, in_dim, out_dim, dev(x, gpu)))


def test_matvec_golden(gpu):
    """Fixture written by the reference's own WeightStore (oracle/_ref)."""
    z = np.load(os.path.join(GOLD, "matvec.npz"))
    y = run_matvec(gpu, z["w"], 48, 1024, 0, 48, z["x"])
    e = rel_err(y[16:48], z["y_row16"])
    assert e < TIGHT, e
    t64 = G.tile(dev(z["w"].reshape(-1), gpu), 48, 1024)
    Y = host(G.matmul(t64, 48, 0, 1024, 48, dev(z["X"], gpu)))
    e = rel_err(Y[:, 8:40], z["Y_row8"])
    assert e < TIGHT, e


@pytest.mark.parametrize("n_rows,in_dim,row0,out_dim", [
    (4096, 4096, 0, 4096),    # single IQ3_XXS GEMV, 4096 x 4096
    (64, 256, 0, 64),         # one block per row
    (35, 768, 0, 35),         # 3 blocks per row, partial last tile
    (200, 1280, 64, 100),     # row0 inside the tensor, partial tile
    (300, 512, 128, 172),     # ends on the tensor's partial last tile
    (16, 2048, 0, 16),
])
def test_matvec_shapes(gpu, n_rows, in_dim, row0, out_dim):
    w = synth.iq3xxs_matrix(50, n_rows, n_rows, in_dim)
    x = synth.normal(50, 1000 + in_dim, in_dim)
    y = run_matvec(gpu, w, n_rows, in_dim, row0, out_dim, x)
    ref = oracle.matvec(w, row0, in_dim, out_dim, x)
    e = rel_err(y, ref)
    assert e < TIGHT, e


@pytest.mark.parametrize("scale", [1e-6, 3e4, 1.0])
def test_matvec_activation_range(gpu, scale):
    n_rows, in_dim = 64, 2048
    w = synth.iq3xxs_matrix(51, 0, n_rows, in_dim)
    x = synth.normal(51, 1, in_dim) * np.float32(scale)
    x[::97] *= np.float32(50.0)  # outliers
    y = run_matvec(gpu, w, n_rows, in_dim, 0, n_rows, x)
    e = rel_err(y, oracle.matvec(w, 0, in_dim, n_rows, x))
    assert e < TIGHT, e


@pytest.mark.parametrize("n_rows,in_dim,row0,out_dim", [
    (128, 20480, 64, 64),     # 80 blocks per row, one tile cut into many chunks
    (128, 12288, 0, 128),     # 96 records over 96 workgroups: 48 partials per tile
    (33000, 256, 0, 33000),   # 516 one-block tiles, several tiles per chunk
])
def test_matvec_split_and_many_tiles(gpu, n_rows, in_dim, row0, out_dim):
    w = synth.iq3xxs_matrix(59, 0, n_rows, in_dim)
    x = synth.normal(59, 1, in_dim)
    y = run_matvec(gpu, w, n_rows, in_dim, row0, out_dim, x)
    e = rel_err(y, oracle.matvec(w, row0, in_dim, out_dim, x))
    assert e < TIGHT, e


def test_gemv_deterministic_and_workspace_reset(gpu):
    """Shared tiles are summed in chunk order (bitwise repeatable) and every
    launch leaves the workspace tickets at zero."""
    import torch

    n_rows, in_dim = 6144, 12288
    w = synth.iq3xxs_matrix(61, 0, n_rows, in_dim)
    t64 = G.tile(dev(w.reshape(-1), gpu), n_rows, in_dim)
    x = synth.normal(61, 1, in_dim)
    act = G.prep_act(dev(x, gpu), G.act_buffer(in_dim, 1, gpu))
    ws = G.gemv_workspace(in_dim, n_rows, 1, 1, gpu)
    ys = [host(G.gemv_act(t64, n_rows, 0, in_dim, n_rows, act, 1, ws=ws)) for _ in range(3)]
    assert all(np.array_equal(ys[0].view(np.uint32), y.view(np.uint32)) for y in ys[1:])
    torch.cuda.synchronize()
    n_tiles = n_rows // 64
    assert not host(ws[:256 + 4 * n_tiles]).any()  # header (error word) and tickets
    G.ws_status(ws)
    assert rel_err(ys[0][0], oracle.matvec(w, 0, in_dim, n_rows, x)) < TIGHT


@pytest.mark.parametrize("n_tok", [1, 2, 3, 4, 5, 6, 7, 8, 11])
def test_matmul_tokens(gpu, n_tok):
    """matmul_quant (weights.cpp:86-165): Y[t] = W X[t]; row t equals the
    token's own matvec up to accumulation order."""
    n_rows, in_dim = 200, 1536
    w = synth.iq3xxs_matrix(62, n_tok, n_rows, in_dim)
    X = np.stack([synth.normal(62, 100 + t, in_dim) * np.float32(1 + t) for t in range(n_tok)])
    t64 = G.tile(dev(w.reshape(-1), gpu), n_rows, in_dim)
    Y = host(G.matmul(t64, n_rows, 64, in_dim, 136, dev(X, gpu)))
    ref = oracle.matmul(w, 64, in_dim, 136, X)
    for t in range(n_tok):
        e = rel_err(Y[t], ref[t])
        assert e < TIGHT, (t, e)


def test_gemv2_shared_activation(gpu):
    n_rows, in_dim = 200, 1536
    wa = synth.iq3xxs_matrix(60, 0, n_rows, in_dim)
    wb = synth.iq3xxs_matrix(60, 1, n_rows, in_dim)
    X = np.stack([synth.normal(60, 2, in_dim), synth.normal(60, 3, in_dim)])
    ta = G.tile(dev(wa.reshape(-1), gpu), n_rows, in_dim)
    tb = G.tile(dev(wb.reshape(-1), gpu), n_rows, in_dim)
    act = G.prep_act(dev(X, gpu), G.act_buffer(in_dim, 2, gpu))
    ya, yb = G.gemv2_act(ta, tb, n_rows, 64, in_dim, 136, act, 2)
    ra, rb = oracle.matmul(wa, 64, in_dim, 136, X), oracle.matmul(wb, 64, in_dim, 136, X)
    for t in range(2):
        assert rel_err(host(ya)[t], ra[t]) < TIGHT
        assert rel_err(host(yb)[t], rb[t]) < TIGHT


def test_matvec_zero_activation(gpu):
    w = synth.iq3xxs_matrix(52, 0, 64, 512)
    y = run_matvec(gpu, w, 64, 512, 0, 64, np.zeros(512, np.float32))
    assert np.all(y == 0)


@pytest.mark.parametrize("n_rows,in_dim", [(12288, 6144), (6144, 12288)])
def test_matvec_dense_mlp_shapes(gpu, n_rows, in_dim):
    """Gate/up 12288 x 6144 and down 6144 x 12288 at full size."""
    w = synth.iq3xxs_matrix(53, n_rows, n_rows, in_dim)
    x = synth.normal(53, 7, in_dim)
    y = run_matvec(gpu, w, n_rows, in_dim, 0, n_rows, x)
    ref = oracle.matvec(w, 0, in_dim, n_rows, x)
    e = rel_err(y, ref)
    assert e < TOL and e < TIGHT, e


def test_matvec_raw(gpu):
    n_rows, in_dim = 70, 1536
    w = synth.iq3xxs_matrix(54, 0, n_rows, in_dim)
    x = synth.normal(54, 1, in_dim)
    y = host(G.matvec_raw(dev(w.reshape(-1), gpu), n_rows, 3, in_dim, 60, dev(x, gpu)))
    e = rel_err(y, oracle.matvec(w, 3, in_dim, 60, x))
    assert e < TIGHT, e


def test_matvec_errors(gpu):
    import torch

    w = synth.iq3xxs_matrix(55, 0, 128, 512)
    t64 = G.tile(dev(w.reshape(-1), gpu), 128, 512)
    x = torch.zeros(512, device=gpu)
    with pytest.raises(G.GpeedError) as e:
        G.matvec(t64, 128, 16, 512, 16, x)
    assert e.value.code == -6
    with pytest.raises(G.GpeedError) as e:
        G.matvec(t64, 128, 64, 512, 65, x)
    assert e.value.code == -1
    with pytest.raises(G.GpeedError) as e:
        G.matvec(t64, 128, 0, 500, 16, x)
    assert e.value.code == -3
    with pytest.raises(G.GpeedError) as e:
        G.matvec(t64, 128, 0, 512, 16, x, ws=torch.zeros(256, dtype=torch.uint8, device=gpu))
    assert e.value.code == -7
    act = G.act_buffer(512, 8, gpu)
    with pytest.raises(G.GpeedError) as e:
        G.gemv_act(t64, 128, 0, 512, 64, act, 9, ws=torch.zeros(1 << 20, dtype=torch.uint8, device=gpu))
    assert e.value.code == -1
    # out_dim <= 0 / n_tok <= 0 return without touching dst (weights.cpp:88)
    G.matvec(t64, 128, 0, 512, 0, x, out=torch.empty(1, device=gpu))


@pytest.mark.parametrize("n_tok", [1, 4])
def test_dense_mlp_step(gpu, n_tok):
    """dense_mlp / dense_mlp_batch (model.cpp:677-690, model_batch.cpp:145-163):
    gate/up share one prepared activation, SwiGLU fused into the down
    projection's activation prep."""
    import torch

    H, I = 1024, 2048
    wg = synth.iq3xxs_matrix(56, 0, I, H)
    wu = synth.iq3xxs_matrix(56, 1, I, H)
    wd = synth.iq3xxs_matrix(56, 2, H, I)
    X = np.stack([synth.normal(56, 9 + t, H) * np.float32(4.0) for t in range(n_tok)])
    tg, tu, td = (G.tile(dev(a.reshape(-1), gpu), r, c) for a, r, c in ((wg, I, H), (wu, I, H), (wd, H, I)))
    act = G.act_buffer(H, n_tok, gpu)
    G.prep_act(dev(X, gpu), act)
    g, u = G.gemv2_act(tg, tu, I, 0, H, I, act, n_tok)
    for t in range(n_tok):
        assert rel_err(host(g)[t], oracle.matvec(wg, 0, H, I, X[t])) < TIGHT
        assert rel_err(host(u)[t], oracle.matvec(wu, 0, H, I, X[t])) < TIGHT
    act2 = G.act_buffer(I, n_tok, gpu)
    G.prep_swiglu(g, u, act2, 10.0)
    y = host(G.gemv_act(td, H, 0, I, H, act2, n_tok))
    ref = oracle.dense_mlp(wg, wu, wd, H, I, X, 10.0)
    for t in range(n_tok):
        e = rel_err(y[t], ref[t])
        assert e < TOL, e
        assert e < 1e-4, e  # silu via the device expf differs by ulps from glibc's
    torch.cuda.synchronize()


@pytest.mark.parametrize("n_rows,in_dim,row0,out_dim", [(6144, 12288, 0, 6144), (12288, 6144, 0, 12288),
                                                      (200, 1280, 64, 100), (128, 16384, 0, 128), (33000, 256, 0, 33000)])
def test_gemv_x_fused_preparation(gpu, n_rows, in_dim, row0, out_dim):
    """One-launch GEMV (activation blocks prepared inside the workgroups)."""
    w = synth.iq3xxs_matrix(64, 0, n_rows, in_dim)
    t64 = G.tile(dev(w.reshape(-1), gpu), n_rows, in_dim)
    x = synth.normal(64, 1, in_dim)
    x[::89] *= np.float32(40.0)
    y = host(G.gemv_x(t64, n_rows, row0, in_dim, out_dim, dev(x, gpu)))
    e = rel_err(y, oracle.matvec(w, row0, in_dim, out_dim, x))
    assert e < TIGHT, e


def test_dense_mlp_fused_launches(gpu):
    """dense_mlp (model.cpp:677-690) as two launches: gate+up with the
    preparation fused, down with SwiGLU fused."""
    H, I = 6144, 12288
    wg = synth.iq3xxs_matrix(65, 0, I, H)
    wu = synth.iq3xxs_matrix(65, 1, I, H)
    wd = synth.iq3xxs_matrix(65, 2, H, I)
    x = synth.normal(65, 9, H) * np.float32(4.0)
    tg, tu, td = (G.tile(dev(a.reshape(-1), gpu), r, c) for a, r, c in ((wg, I, H), (wu, I, H), (wd, H, I)))
    g, u = G.gemv2_x(tg, tu, I, 0, H, I, dev(x, gpu))
    assert rel_err(host(g), oracle.matvec(wg, 0, H, I, x)) < TIGHT
    assert rel_err(host(u), oracle.matvec(wu, 0, H, I, x)) < TIGHT
    y = host(G.gemv_swiglu(td, H, 0, I, H, g, u, 10.0))
    ref = oracle.dense_mlp(wg, wu, wd, H, I, x[None, :], 10.0)[0]
    e = rel_err(y, ref)
    assert e < 1e-4, e
    with pytest.raises(G.GpeedError) as err:
        G.gemv_x(td, H, 32, I, 64, dev(np.zeros(I, np.float32), gpu))  # row0 off the 64-row tiles
    assert err.value.code < 0


@pytest.mark.parametrize("H,I", [(6144, 12288), (1024, 2048), (256, 768), (512, 256), (2304, 5376)])
def test_dense_mlp(gpu, H, I):
    """dense_mlp (model.cpp:677-690) through gpeed_iq3xxs_dense_mlp: gate and
    up in one launch, the workgroup completing 64 rows writing their SwiGLU
    as the down projection's activation; down in a second launch, whose
    shared row tiles are added into y (zero-filled by the first launch) with
    atomic adds. Repeated calls on one workspace agree to within the fp32
    rounding of those two to four adds, whose order varies."""
    wg = synth.iq3xxs_matrix(66, 0, I, H)
    wu = synth.iq3xxs_matrix(66, 1, I, H)
    wd = synth.iq3xxs_matrix(66, 2, H, I)
    x = synth.normal(66, 9, H) * np.float32(4.0)
    x[::97] *= np.float32(30.0)
    tg, tu, td = (G.tile(dev(a.reshape(-1), gpu), r, c) for a, r, c in ((wg, I, H), (wu, I, H), (wd, H, I)))
    ws = G.dense_mlp_workspace(H, I, gpu)
    xd = dev(x, gpu)
    y = host(G.dense_mlp(tg, tu, td, H, I, xd, 10.0, ws=ws))
    ref = oracle.dense_mlp(wg, wu, wd, H, I, x[None, :], 10.0)[0]
    e = rel_err(y, ref)
    assert e < 1e-4, e  # silu via the device expf differs by ulps from glibc's
    for _ in range(3):
        y2 = host(G.dense_mlp(tg, tu, td, H, I, xd, 10.0, ws=ws))
        assert rel_err(y2, y) < 1e-6
    # a second input on the same workspace (the completion counters move on)
    x2 = synth.normal(66, 10, H)
    y3 = host(G.dense_mlp(tg, tu, td, H, I, dev(x2, gpu), 10.0, ws=ws))
    ref2 = oracle.dense_mlp(wg, wu, wd, H, I, x2[None, :], 10.0)[0]
    assert rel_err(y3, ref2) < 1e-4
    # in place (y over x: the down launch finishes shared row tiles by
    # ticket), then the atomic path again on the same workspace
    xin = dev(x2, gpu)
    y4 = host(G.dense_mlp(tg, tu, td, H, I, xin, 10.0, out=xin, ws=ws))
    assert rel_err(y4, ref2) < 1e-4
    y5 = host(G.dense_mlp(tg, tu, td, H, I, xd, 10.0, ws=ws))
    assert rel_err(y5, y) < 1e-6


def test_dense_mlp_errors(gpu):
    t = dev(np.zeros(16, np.uint8), gpu)
    x = dev(np.zeros(512, np.float32), gpu)
    with pytest.raises(ValueError):
        G.dense_mlp_workspace(500, 256, gpu)
    ws = G.dense_mlp_workspace(512, 256, gpu)
    small = dev(np.zeros(256, np.uint8), gpu)
    with pytest.raises(G.GpeedError) as err:
        G.dense_mlp(t, t, t, 512, 256, x, 10.0, ws=small)
    assert err.value.code == -7
    with pytest.raises(G.GpeedError):
        G.dense_mlp(t, t, t, 500, 256, x, 10.0, ws=ws)


def test_weight_store_mirror(gpu):
    w = synth.iq3xxs_matrix(57, 0, 128, 512)
    ws = G.WeightStore(device=gpu)
    ws.add("blk.0.ffn_up.weight", w, 512, 128)
    x = synth.normal(57, 1, 512)
    y = ws.matvec_quant("blk.0.ffn_up.weight", 64, 512, 32, x)
    assert rel_err(y, oracle.matvec(w, 64, 512, 32, x)) < TIGHT
    X = np.stack([synth.normal(57, 2 + t, 512) for t in range(5)])
    Y = ws.matmul_quant("blk.0.ffn_up.weight", 0, 512, 100, X, 5)
    ref = oracle.matmul(w, 0, 512, 100, X)
    assert max(rel_err(Y[t], ref[t]) for t in range(5)) < TIGHT
    assert ws.matmul_quant("blk.0.ffn_up.weight", 0, 512, 100, X, 0) is None
    # any row0, as weights.cpp:86-203: a row0 inside a 64-row tile
    y = ws.matvec_quant("blk.0.ffn_up.weight", 3, 512, 70, x)
    assert y.shape == (70,) and rel_err(y, oracle.matvec(w, 3, 512, 70, x)) < TIGHT
    for n_tok in (5, 12):
        Xn = np.stack([synth.normal(57, 20 + t, 512) for t in range(n_tok)])
        Y = ws.matmul_quant("blk.0.ffn_up.weight", 3, 512, 125, Xn, n_tok)
        ref = oracle.matmul(w, 3, 512, 125, Xn)
        assert Y.shape == (n_tok, 125) and max(rel_err(Y[t], ref[t]) for t in range(n_tok)) < TIGHT
    with pytest.raises(RuntimeError, match="rows outside"):
        ws.matvec_quant("blk.0.ffn_up.weight", 100, 512, 29, x)
    with pytest.raises(RuntimeError, match="missing tensor"):
        ws.matvec_quant("nope", 0, 512, 16, x)
    with pytest.raises(RuntimeError, match="not block aligned"):
        ws.matvec_quant("blk.0.ffn_up.weight", 0, 500, 16, x)


def test_graph_replay_matches_eager(gpu):
    """The GEMV launches captured in a HIP graph (no memset nodes; the
    workspace tickets reset inside the kernel) give the eager result on
    every replay, with eager work in between."""
    import torch

    n_rows, in_dim = 6144, 12288
    w = synth.iq3xxs_matrix(63, 0, n_rows, in_dim)
    t64 = G.tile(dev(w.reshape(-1), gpu), n_rows, in_dim)
    x = dev(synth.normal(63, 1, in_dim), gpu)
    act = G.prep_act(x, G.act_buffer(in_dim, 1, gpu))
    ws = G.gemv_workspace(in_dim, n_rows, 1, 1, gpu)
    y = torch.empty(1, n_rows, device=gpu)
    G.gemv_act(t64, n_rows, 0, in_dim, n_rows, act, 1, out=y, ws=ws)
    torch.cuda.synchronize()
    want = host(y).copy()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            G.gemv_act(t64, n_rows, 0, in_dim, n_rows, act, 1, out=y, ws=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for r in range(4):
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32)), r
        G.gemv_act(t64, n_rows, 0, in_dim, n_rows, act, 1, ws=ws)  # eager work between replays
        torch.cuda.synchronize()


def test_dense_mlp_graph_replay(gpu):
    """dense_mlp captured in a HIP graph: the gate/up launch's zero fill of y
    and the down launch's atomic tile sums hold on every replay (y garbage
    before each), with eager calls on the same workspace in between."""
    import torch

    H, I = 1024, 2048
    wg = synth.iq3xxs_matrix(67, 0, I, H)
    wu = synth.iq3xxs_matrix(67, 1, I, H)
    wd = synth.iq3xxs_matrix(67, 2, H, I)
    x = synth.normal(67, 9, H)
    tg, tu, td = (G.tile(dev(a.reshape(-1), gpu), r, c) for a, r, c in ((wg, I, H), (wu, I, H), (wd, H, I)))
    ws = G.dense_mlp_workspace(H, I, gpu)
    xd = dev(x, gpu)
    y = torch.empty(H, device=gpu)
    G.dense_mlp(tg, tu, td, H, I, xd, 10.0, out=y, ws=ws)
    torch.cuda.synchronize()
    want = host(y).copy()
    assert rel_err(want, oracle.dense_mlp(wg, wu, wd, H, I, x[None, :], 10.0)[0]) < 1e-4
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            G.dense_mlp(tg, tu, td, H, I, xd, 10.0, out=y, ws=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for r in range(4):
        y.fill_(float(r + 1) * 1e6)
        graph.replay()
        torch.cuda.synchronize()
        assert rel_err(host(y), want) < 1e-6, r
        G.dense_mlp(tg, tu, td, H, I, xd, 10.0, ws=ws)  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("n_bytes,groups", [(16, 1), (4096 * 5 + 48, 3), (1 << 20, 256), (3 * (1 << 20) + 4080, 1024)])
def test_stream_read_covers_every_byte(gpu, n_bytes, groups):
    """Workgroup i folds (XOR of 32-bit words) exactly its share: shares are
    ceil(bytes / groups) rounded up to 4 KiB, the last ones short or empty."""
    rng = np.random.default_rng(n_bytes + groups)
    words = rng.integers(0, 2**32, n_bytes // 4, dtype=np.uint64).astype(np.uint32)
    got = host(G.stream_read(dev(words.view(np.int32), gpu), groups)).view(np.uint32)
    share = (n_bytes // groups + 4095) & ~4095
    want = np.zeros(groups, np.uint32)
    for i in range(groups):
        seg = words[i * share // 4:min((i + 1) * share, n_bytes) // 4]
        want[i] = np.bitwise_xor.reduce(seg) if seg.size else 0
    assert np.array_equal(got, want)


def test_stream_read_errors(gpu):
    import ctypes

    buf = dev(np.zeros(64, np.int32), gpu)
    out = dev(np.zeros(4, np.int32), gpu)
    p, o = ctypes.c_void_p(buf.data_ptr()), ctypes.c_void_p(out.data_ptr())
    assert G.lib().gpeed_stream_read(p, 20, o, 4, None) != 0  # not a multiple of 16
    assert G.lib().gpeed_stream_read(ctypes.c_void_p(buf.data_ptr() + 4), 32, o, 4, None) != 0
    assert G.lib().gpeed_stream_read(p, 32, o, 0, None) != 0
    assert G.lib().gpeed_stream_read(p, 0, o, 4, None) == 0  # nothing to read


def test_device_smoke(gpu):
    assert G.device_count() >= 1
    assert G.device_name(0) not in ("", "<none>")
    a = synth.normal(58, 0, 1000)
    b = synth.normal(58, 1, 1000)
    assert np.array_equal(G.add_f32(a, b), a + b)

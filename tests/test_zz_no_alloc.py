"""GPU test of gpeed_iq3xxs_matvec_noalloc, the entry point that allocates
nothing (no reference counterpart: for callers that cannot allocate). Called
through the C ABI and checked against gpeed_iq3xxs_matvec (same kernel: bit
for bit) and the oracle, on two calls in a row, the second smaller, which
share the GPU's fixed scratch array."""
import ctypes as C

import numpy as np
import pytest

import gpeed_amd as G
import oracle
from gpeed_amd import synth
from conftest import rel_err

pytestmark = pytest.mark.gpu
TIGHT = 2e-5


def _noalloc(t64, n_rows, row0, in_dim, out_dim, x, out):
    import torch

    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    return G.lib().gpeed_iq3xxs_matvec_noalloc(C.c_void_p(t64.data_ptr()), n_rows, row0, in_dim, out_dim,
                                               C.c_void_p(x.data_ptr()), C.c_void_p(out.data_ptr()), s)


@pytest.mark.parametrize("order", ["large_then_small", "small_then_large"])
def test_matvec_noalloc_matches_matvec(gpu, order):
    import torch

    cases = [(6144, 12288, 0, 6144), (200, 1536, 64, 136)]  # many shared tiles; then a small slice
    if order == "small_then_large":
        cases = cases[::-1]
    for i, (n_rows, in_dim, row0, out_dim) in enumerate(cases):
        w = synth.iq3xxs_matrix(98, i, n_rows, in_dim)
        t64 = G.tile(torch.from_numpy(w.reshape(-1)).to(gpu), n_rows, in_dim)
        x_h = synth.normal(98, 10 + i, in_dim)
        x = torch.from_numpy(x_h).to(gpu)
        y0 = torch.full((out_dim,), float("nan"), device=gpu)
        y1 = torch.full((out_dim,), float("nan"), device=gpu)
        G.matvec(t64, n_rows, row0, in_dim, out_dim, x, out=y0)
        assert _noalloc(t64, n_rows, row0, in_dim, out_dim, x, y1) == 0, G.lib().gpeed_last_error()
        a, b = y0.cpu().numpy(), y1.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (n_rows, in_dim)
        assert rel_err(b, oracle.matvec(w, row0, in_dim, out_dim, x_h)) < TIGHT


def test_matvec_noalloc_repeats_and_refuses_oversize(gpu):
    import torch

    n_rows, in_dim = 448, 4096
    w = synth.iq3xxs_matrix(99, 0, n_rows, in_dim)
    t64 = G.tile(torch.from_numpy(w.reshape(-1)).to(gpu), n_rows, in_dim)
    x = torch.from_numpy(synth.normal(99, 1, in_dim)).to(gpu)
    ys = []
    for _ in range(3):
        y = torch.empty(n_rows, device=gpu)
        assert _noalloc(t64, n_rows, 0, in_dim, n_rows, x, y) == 0
        ys.append(y.cpu().numpy())
    assert all(np.array_equal(ys[0].view(np.uint32), v.view(np.uint32)) for v in ys[1:])
    # 9375 one-block tiles need ~4.8 MB of tickets and partials: refused
    # before any launch (the weights are real and in bounds all the same)
    big_rows, big_in = 600000, 256
    tbig = torch.zeros(G.t64_bytes(big_rows, big_in), dtype=torch.uint8, device=gpu)
    xb = torch.zeros(big_in, device=gpu)
    yb = torch.empty(big_rows, device=gpu)
    assert _noalloc(tbig, big_rows, 0, big_in, big_rows, xb, yb) == -1
    assert b"scratch" in G.lib().gpeed_last_error()
    torch.cuda.synchronize()


def test_matvec_noalloc_status_reports_and_clears(gpu):
    """A stale ticket in the fixed scratch (what overlapping calls leave) is
    reported by gpeed_iq3xxs_matvec_noalloc_status, which then zero-fills the
    scratch: the next call is bitwise equal to the workspace entry point.
    The preset ticket only makes every part of tile 0 see a count past its
    last, so no workgroup waits on it and every kernel exits normally."""
    import torch

    L = G.lib()
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    n_rows, in_dim = 6144, 12288  # tile 0's 48 records span three workgroups' chunks
    w = synth.iq3xxs_matrix(97, 0, n_rows, in_dim)
    t64 = G.tile(torch.from_numpy(w.reshape(-1)).to(gpu), n_rows, in_dim)
    x = torch.from_numpy(synth.normal(97, 1, in_dim)).to(gpu)
    assert L.gpeed_iq3xxs_matvec_noalloc_status(s) == 0, L.gpeed_last_error()
    assert L.gpeed_iq3xxs_matvec_noalloc_poke(256, 1000) == 0, L.gpeed_last_error()  # tile 0's ticket
    y = torch.empty(n_rows, device=gpu)
    assert _noalloc(t64, n_rows, 0, in_dim, n_rows, x, y) == 0
    assert L.gpeed_iq3xxs_matvec_noalloc_status(s) == -9
    assert b"ticket" in L.gpeed_last_error() and b"cleared" in L.gpeed_last_error()
    assert L.gpeed_iq3xxs_matvec_noalloc_status(s) == 0, L.gpeed_last_error()
    y0 = torch.empty(n_rows, device=gpu)
    G.matvec(t64, n_rows, 0, in_dim, n_rows, x, out=y0)
    assert _noalloc(t64, n_rows, 0, in_dim, n_rows, x, y) == 0
    assert L.gpeed_iq3xxs_matvec_noalloc_status(s) == 0, L.gpeed_last_error()
    a, b = y0.cpu().numpy(), y.cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert L.gpeed_iq3xxs_matvec_noalloc_poke(3, 0) == -1  # not a word offset

"""GPU tests of the workspace contract and of matmul_quant's dispatch.

* matmul_quant (weights.cpp:86-165) runs 8-token GEMV passes for decode-sized
  batches and the prefill GEMM from matmul_gemm_min_tok() tokens on, as the
  reference's prefill call sites need (model_batch.cpp:30-95, 151-162); the
  launch-timing pool shows which kernel ran.
* One matmul workspace serves every token count up to the one it was sized
  for, in any order.
* Workspaces report what the kernels find wrong with them (gpeed_ws_status)
  instead of producing silently wrong rows: a pre-set ticket, buckets that
  break the router's invariants. Every kernel still exits normally: nothing
  here waits on a partial that is never written.
* GEMM workspaces need no initialisation beyond the header (the X
  preparation clears the split-K tickets on every call).
"""
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


def host(t):
    return t.cpu().numpy()


def _tensor(gpu, seed, n_rows, in_dim):
    w = synth.iq3xxs_matrix(seed, 0, n_rows, in_dim)
    return w, G.tile(dev(w.reshape(-1), gpu), n_rows, in_dim)


@pytest.mark.parametrize("n_tok", [1, 2, 9, 15, 16, 17, 64, 100, 512])
def test_matmul_quant_dispatch(gpu, n_tok):
    """WeightStore.matmul_quant on host arrays: parity at every token count,
    and the GEMM (not n_tok / 8 GEMV passes) from the crossover on."""
    n_rows, in_dim, row0, out_dim = 704, 1536, 64, 600
    w = synth.iq3xxs_matrix(90, 0, n_rows, in_dim)
    X = synth.normal(90, 1, n_tok * in_dim).reshape(n_tok, in_dim)
    st = G.WeightStore(gpu)
    st.add("blk.0.attn_q_a.weight", w, in_dim, n_rows)
    G.prof_start(256)
    Y = st.matmul_quant("blk.0.attn_q_a.weight", row0, in_dim, out_dim, X, n_tok)
    n_gemm, n_gemv = len(G.prof_read(G.PROF_GEMM)), len(G.prof_read(G.PROF_GEMV))
    ref = oracle.matmul(w, row0, in_dim, out_dim, X)
    e = max(rel_err(Y[t], ref[t]) for t in range(n_tok))
    assert e < TIGHT, e
    if n_tok >= G.matmul_gemm_min_tok():
        assert n_gemm == 1 and n_gemv == 0, (n_gemm, n_gemv)
    else:
        assert n_gemm == 0 and n_gemv == (n_tok + 7) // 8, (n_gemm, n_gemv)


def test_matmul_prefill_full_width(gpu):
    """A 512-token matmul_quant on the 12288 x 6144 prefill tensor runs one
    GEMM; rows checked against the oracle on slices it finishes quickly."""
    n_rows, in_dim, n_tok = 12288, 6144, 512
    w, t64 = _tensor(gpu, 91, n_rows, in_dim)
    X = synth.normal(91, 1, n_tok * in_dim).reshape(n_tok, in_dim)
    ws = G.matmul_workspace(in_dim, n_rows, n_tok, gpu)
    G.prof_start(64)
    Y = host(G.matmul(t64, n_rows, 0, in_dim, n_rows, dev(X, gpu), ws=ws))
    assert len(G.prof_read(G.PROF_GEMM)) == 1
    G.ws_status(ws)
    for r0 in (0, 6080, 12224):
        ref = oracle.matmul(w, r0, in_dim, 64, X[::37])
        e = max(rel_err(Y[::37][t, r0:r0 + 64], ref[t]) for t in range(ref.shape[0]))
        assert e < TIGHT, (r0, e)


def test_matmul_workspace_serves_smaller_calls(gpu):
    """One workspace sized for 512 tokens, calls of 512, 1, 9, 300, 16, 2 and
    64 tokens in turn: every result matches, the workspace stays clean."""
    n_rows, in_dim = 448, 2048
    w, t64 = _tensor(gpu, 92, n_rows, in_dim)
    ws = G.matmul_workspace(in_dim, n_rows, 512, gpu)
    for n_tok in (512, 1, 9, 300, 16, 2, 64):
        X = synth.normal(92, n_tok, n_tok * in_dim).reshape(n_tok, in_dim)
        Y = host(G.matmul(t64, n_rows, 0, in_dim, n_rows, dev(X, gpu), ws=ws))
        ref = oracle.matmul(w, 0, in_dim, n_rows, X[::7])
        e = max(rel_err(Y[::7][t], ref[t]) for t in range(ref.shape[0]))
        assert e < TIGHT, (n_tok, e)
        G.ws_status(ws)


def test_matmul_workspace_too_small(gpu):
    """A matvec-sized workspace is refused for a multi-token call."""
    n_rows, in_dim = 128, 512
    _, t64 = _tensor(gpu, 93, n_rows, in_dim)
    ws = G.matvec_workspace(in_dim, n_rows, gpu)
    X = dev(synth.normal(93, 1, 4 * in_dim).reshape(4, in_dim), gpu)
    with pytest.raises(G.GpeedError) as e:
        G.matmul(t64, n_rows, 0, in_dim, n_rows, X, ws=ws)
    assert e.value.code == -7


def test_preset_ticket_is_reported(gpu):
    """Tickets left non-zero (a workspace never initialised, or shared by two
    calls at once) are reported by gpeed_ws_status, not silently summed; after
    gpeed_ws_init the same workspace gives the right result again."""
    import torch

    n_rows, in_dim = 256, 12288  # 4 tiles x 48 blocks: every tile cut over many workgroups
    w, t64 = _tensor(gpu, 94, n_rows, in_dim)
    x = synth.normal(94, 1, in_dim)
    ws = G.matvec_workspace(in_dim, n_rows, gpu)
    tickets = ws[256:256 + 16].view(torch.int32)
    tickets.fill_(1000)  # more arrivals than any tile has parts: no workgroup is last
    torch.cuda.synchronize()
    G.matvec(t64, n_rows, 0, in_dim, n_rows, dev(x, gpu), ws=ws)
    with pytest.raises(G.GpeedError) as e:
        G.ws_status(ws)
    assert e.value.code == -9 and "ticket" in str(e.value)
    G.ws_status(ws)  # the flags were cleared by the read
    G.ws_init(ws)
    y = host(G.matvec(t64, n_rows, 0, in_dim, n_rows, dev(x, gpu), ws=ws))
    G.ws_status(ws)
    assert rel_err(y, oracle.matvec(w, 0, in_dim, n_rows, x)) < TIGHT


def test_gemm_workspace_needs_no_zero_fill(gpu):
    """Split-K GEMM (few result tiles) on a workspace full of garbage except
    its header: the X preparation clears the tickets, the result is the same
    bits as on a zero-filled workspace, and nothing is flagged."""
    import torch

    n_rows, in_dim, n_tok = 384, 4096, 40
    w, t64 = _tensor(gpu, 95, n_rows, in_dim)
    X = dev(synth.normal(95, 1, n_tok * in_dim).reshape(n_tok, in_dim), gpu)
    nb = G.lib().gpeed_iq3xxs_gemm_ws_bytes(n_tok, in_dim, n_rows, G.X_F32)
    clean = G._zeros(nb, gpu)
    dirty = torch.full(((nb + 255) // 256 * 256,), 0xA5, dtype=torch.uint8, device=gpu)
    dirty[:256] = 0
    y0 = host(G.gemm(t64, n_rows, 0, in_dim, n_rows, X, ws=clean))
    y1 = host(G.gemm(t64, n_rows, 0, in_dim, n_rows, X, ws=dirty))
    y2 = host(G.gemm(t64, n_rows, 0, in_dim, n_rows, X, ws=dirty))
    G.ws_status(dirty)
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
    assert np.array_equal(y0.view(np.uint32), y2.view(np.uint32))
    ref = oracle.matmul(w, 0, in_dim, n_rows, host(X))
    assert max(rel_err(y0[t], ref[t]) for t in range(n_tok)) < TIGHT


@pytest.mark.parametrize("bad", ["total", "decreasing", "token_range", "token_count"])
def test_moe_bad_buckets_flagged(gpu, bad):
    """Buckets that break the router's invariants are not multiplied: Y = 0,
    GPEED_WS_BUCKETS reported; good buckets on the same workspace work after."""
    E, H, I, T, K = 8, 512, 256, 6, 2
    wg = G.tile(dev(synth.iq3xxs_matrix(96, 0, E * I, H).reshape(-1), gpu), E * I, H)
    wu = G.tile(dev(synth.iq3xxs_matrix(96, 1, E * I, H).reshape(-1), gpu), E * I, H)
    wd_raw = synth.iq3xxs_matrix(96, 2, E * H, I)
    wd = G.tile(dev(wd_raw.reshape(-1), gpu), E * H, I)
    X = synth.normal(96, 3, T * H).reshape(T, H)
    logits = synth.normal(96, 4, T * E).reshape(T, E)
    eptr, tok, wt, _ = oracle.moe_route(logits, K, 1)
    eptr_b, tok_b = eptr.copy(), tok.copy()
    if bad == "total":
        eptr_b[E] -= 1
    elif bad == "decreasing":
        eptr_b[3], eptr_b[4] = eptr_b[4] + 1, eptr_b[3]
    elif bad == "token_range":
        tok_b[5] = T + 3
    else:
        tok_b[0] = tok_b[1] = 0  # token 0 three times or more, another token short
        tok_b[2] = 0
    with pytest.raises(G.GpeedError):
        G.moe_check_buckets(eptr_b, tok_b, E, T, K)
    ws = G._zeros(G.lib().gpeed_iq3xxs_moe_ws_bytes(T, E, K, H, I), gpu)
    Xd = dev(X, gpu)
    Y = host(G.moe_experts(wg, wu, wd, E, H, I, Xd, K, dev(eptr_b.astype(np.int32), gpu),
                           dev(tok_b.astype(np.int32), gpu), dev(wt, gpu), ws=ws))
    assert not Y.any()
    with pytest.raises(G.GpeedError) as e:
        G.ws_status(ws)
    assert e.value.code == -9 and "bucket" in str(e.value)
    G.moe_check_buckets(eptr, tok, E, T, K)
    Y = host(G.moe_experts(wg, wu, wd, E, H, I, Xd, K, dev(eptr.astype(np.int32), gpu),
                           dev(tok.astype(np.int32), gpu), dev(wt, gpu), ws=ws))
    G.ws_status(ws)
    ref = oracle.moe_experts(synth.iq3xxs_matrix(96, 0, E * I, H), synth.iq3xxs_matrix(96, 1, E * I, H), wd_raw,
                             H, I, X, eptr, tok, wt, 10.0)
    assert max(rel_err(Y[t], ref[t]) for t in range(T)) < TIGHT

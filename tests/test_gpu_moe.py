"""GPU parity tests for the routed-expert path (model_batch.cpp:165-262).

The router's integer outputs (bucket offsets, token order, ranked choices)
must equal the oracle's bit for bit; combine weights differ from the CPU's
only by the last-ulp of expf (rel 1e-6); the experts' output is held to the
product bar (rel_err < 2e-5; the parity bar is 1e-3).
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


@pytest.mark.parametrize("T,E,K,mode", [
    (32, 64, 8, 1),      # the routed-expert decode batch: softmax top-8 of 64
    (32, 64, 8, 0),      # reference router: sigmoid + bias, routed_scale 2.5
    (32, 64, 8, 2),      # the same without norm_topk (weights score * routed_scale)
    (300, 256, 8, 0),    # 2400 assignments: the scatter runs in three chunks
    (7, 100, 1, 1),      # experts not a multiple of 64, top-1
    (5, 1024, 32, 1),    # widest router
])
def test_route_matches_oracle(gpu, T, E, K, mode):
    # mode 2 here: the reference router (mode 0) with norm_topk off
    norm = mode != 2
    mode = 0 if mode == 2 else mode
    logits = synth.normal(70, T * 1000 + E, T * E).reshape(T, E)
    bias = synth.normal(71, E, E) * np.float32(0.05) if mode == 0 else None
    eptr, tok, wt, sel = G.moe_route(dev(logits, gpu), K, mode, None if bias is None else dev(bias, gpu),
                                     routed_scale=2.5 if mode == 0 else 1.0, norm_topk=norm)
    r_eptr, r_tok, r_wt, r_sel = oracle.moe_route(logits, K, mode, bias=bias, routed_scale=2.5 if mode == 0 else 1.0,
                                                  norm_topk=norm)
    assert np.array_equal(host(eptr), r_eptr)
    assert np.array_equal(host(tok), r_tok)
    assert np.array_equal(host(sel), r_sel)
    np.testing.assert_allclose(host(wt), r_wt, rtol=1e-6, atol=0)
    # invariants: counts sum to T*K; each token appears K times; in-bucket order by token
    e = host(eptr)
    assert e[0] == 0 and e[-1] == T * K and np.all(np.diff(e) >= 0)
    assert np.array_equal(np.bincount(host(tok), minlength=T), np.full(T, K))
    for x in range(E):
        seg = host(tok)[e[x]:e[x + 1]]
        assert np.all(np.diff(seg) > 0)


def test_route_ties_lower_id_first(gpu):
    logits = np.zeros((3, 16), np.float32)
    logits[1, 5] = 1.0
    eptr, tok, wt, sel = G.moe_route(dev(logits, gpu), 4, 1)
    assert host(sel).tolist() == [[0, 1, 2, 3], [5, 0, 1, 2], [0, 1, 2, 3]]


@pytest.mark.parametrize("E", [16, 100])  # one rank slot per lane, and two (E > 64)
def test_route_signed_zero_ties(gpu, E):
    # -0.0 and +0.0 compare equal (model_batch.cpp ranks with float >): ties
    # go to the lower id whichever zero a logit holds
    logits = np.zeros((3, E), np.float32)
    logits[0, 0] = -0.0
    logits[1, 1] = -0.0
    logits[1, E - 1] = 0.5
    logits[2, :] = -0.0
    logits[2, 70 % E] = 0.0
    eptr, tok, wt, sel = G.moe_route(dev(logits, gpu), 4, 1)
    r_sel = oracle.moe_route(logits, 4, 1)[3]
    assert host(sel).tolist() == r_sel.tolist() == [[0, 1, 2, 3], [E - 1, 0, 1, 2], [0, 1, 2, 3]]


def experts_case(gpu, seed, T, E, K, H, I, mode=1):
    wg = synth.iq3xxs_matrix(seed, 0, E * I, H)
    wu = synth.iq3xxs_matrix(seed, 1, E * I, H)
    wd = synth.iq3xxs_matrix(seed, 2, E * H, I)
    X = synth.normal(seed, 3, T * H).reshape(T, H)
    logits = synth.normal(seed, 4, T * E).reshape(T, E)
    tg = G.tile(dev(wg.reshape(-1), gpu), E * I, H)
    tu = G.tile(dev(wu.reshape(-1), gpu), E * I, H)
    td = G.tile(dev(wd.reshape(-1), gpu), E * H, I)
    eptr, tok, wt, _ = G.moe_route(dev(logits, gpu), K, mode, routed_scale=2.5 if mode == 0 else 1.0)
    Y = host(G.moe_experts(tg, tu, td, E, H, I, dev(X, gpu), K, eptr, tok, wt, 10.0))
    r_eptr, r_tok, r_wt, _ = oracle.moe_route(logits, K, mode, routed_scale=2.5 if mode == 0 else 1.0)
    ref = oracle.moe_experts(wg, wu, wd, H, I, X, r_eptr, r_tok, r_wt, 10.0)
    return Y, ref


@pytest.mark.parametrize("T,E,K,H,I,mode", [
    (5, 8, 2, 512, 256, 1),
    (32, 16, 4, 1024, 512, 0),     # experts with up to ~20 tokens: several segments each
    (3, 4, 4, 768, 1280, 1),       # every expert touched by every token
    (1, 64, 8, 1024, 512, 0),      # one token (moe_forward, model.cpp:692-756): 8 experts of one token each
    (1, 4, 1, 256, 256, 1),        # one token, top-1: a single expert, a single segment
])
def test_experts_small(gpu, T, E, K, H, I, mode):
    Y, ref = experts_case(gpu, 72, T, E, K, H, I, mode)
    for t in range(T):
        e = rel_err(Y[t], ref[t])
        assert e < TIGHT, (t, e)


def test_experts_decode_batch_full_size(gpu):
    """64 experts of gate/up 2048x6144 and down 6144x2048, 32 tokens, top-8."""
    Y, ref = experts_case(gpu, 73, 32, 64, 8, 6144, 2048, 1)
    e = max(rel_err(Y[t], ref[t]) for t in range(32))
    assert e < TIGHT, e


def test_experts_repeatable(gpu):
    """Dynamic work distribution, fixed arithmetic: bitwise repeatable."""
    import torch

    T, E, K, H, I = 16, 8, 4, 512, 512
    wg = synth.iq3xxs_matrix(74, 0, E * I, H)
    wu = synth.iq3xxs_matrix(74, 1, E * I, H)
    wd = synth.iq3xxs_matrix(74, 2, E * H, I)
    tg, tu, td = (G.tile(dev(a.reshape(-1), gpu), r, c) for a, r, c in ((wg, E * I, H), (wu, E * I, H), (wd, E * H, I)))
    X = dev(synth.normal(74, 3, T * H).reshape(T, H), gpu)
    eptr, tok, wt, _ = G.moe_route(dev(synth.normal(74, 4, T * E).reshape(T, E), gpu), K, 1)
    ys = [host(G.moe_experts(tg, tu, td, E, H, I, X, K, eptr, tok, wt)) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(np.array_equal(ys[0].view(np.uint32), y.view(np.uint32)) for y in ys[1:])


def test_moe_errors(gpu):
    import torch

    logits = torch.zeros(2, 8, device=gpu)
    with pytest.raises(G.GpeedError) as e:
        G.moe_route(logits, 9, 1)
    assert e.value.code == -4
    with pytest.raises(G.GpeedError) as e:
        G.moe_route(logits, 2, 3)
    assert e.value.code == -1


# ------------------------------------------------------------------ the whole step (moe_batch)

def batch_case(gpu, seed, T, E, K, H, I, mode, shared, norm=True):
    wg = synth.iq3xxs_matrix(seed, 0, E * I, H)
    wu = synth.iq3xxs_matrix(seed, 1, E * I, H)
    wd = synth.iq3xxs_matrix(seed, 2, E * H, I)
    sh = tuple(synth.iq3xxs_matrix(seed, 5 + i, r, c) for i, (r, c) in enumerate(((I, H), (I, H), (H, I)))) \
        if shared else None
    X = synth.normal(seed, 3, T * H).reshape(T, H)
    logits = synth.normal(seed, 4, T * E).reshape(T, E)
    bias = synth.normal(seed, 8, E) * np.float32(0.05) if mode == 0 else None
    scale = 2.5 if mode == 0 else 1.0
    t = lambda a, r, c: G.tile(dev(a.reshape(-1), gpu), r, c)  # noqa: E731
    tg, tu, td = t(wg, E * I, H), t(wu, E * I, H), t(wd, E * H, I)
    tsh = (t(sh[0], I, H), t(sh[1], I, H), t(sh[2], H, I)) if shared else None
    Y, eptr, tok, wt = G.moe_batch(dev(logits, gpu), dev(X, gpu), tg, tu, td, E, H, I, K, mode,
                                   None if bias is None else dev(bias, gpu), scale, norm, 10.0, shared=tsh,
                                   routing=True)
    ref = oracle.moe_batch(logits, X, wg, wu, wd, H, I, K, mode, bias, scale, norm, 10.0, shared=sh)
    r_eptr, r_tok, r_wt, _ = oracle.moe_route(logits, K, mode, bias=bias, routed_scale=scale, norm_topk=norm)
    assert np.array_equal(host(eptr), r_eptr) and np.array_equal(host(tok), r_tok)
    np.testing.assert_allclose(host(wt), r_wt, rtol=1e-6, atol=0)
    return host(Y), ref, (tg, tu, td, X, eptr, tok, wt, logits, bias, sh, wg, wu, wd)


@pytest.mark.parametrize("T,E,K,H,I,mode,shared,norm", [
    (5, 8, 2, 512, 256, 0, True, True),
    (32, 16, 4, 1024, 512, 0, True, False),   # reference router without norm_topk
    (3, 4, 4, 768, 1280, 1, False, True),      # no shared expert
    (17, 8, 3, 512, 512, 1, True, True),       # shared expert over 17 tokens: three segments, the last of one
])
def test_moe_batch_matches_oracle(gpu, T, E, K, H, I, mode, shared, norm):
    Y, ref, _ = batch_case(gpu, 80, T, E, K, H, I, mode, shared, norm)
    e = max(rel_err(Y[t], ref[t]) for t in range(T))
    assert e < TIGHT, e


def test_moe_batch_decode_batch_full_size(gpu):
    """The routed-expert decode batch (64 experts of gate/up 2048x6144 and
    down 6144x2048, 32 tokens, top-8 softmax routing) with a shared expert of
    the same shape, from the logits in five launches."""
    Y, ref, _ = batch_case(gpu, 81, 32, 64, 8, 6144, 2048, 1, True)
    e = max(rel_err(Y[t], ref[t]) for t in range(32))
    assert e < TIGHT, e


def test_moe_batch_routed_part_equals_moe_experts(gpu):
    """Without the shared expert, the whole step (activations gathered from
    per-token images) gives bit for bit what moe_route + moe_experts give
    (per-segment images)."""
    T, E, K, H, I = 20, 8, 3, 512, 512
    Y, _, (tg, tu, td, X, eptr, tok, wt, logits, bias, _, _, _, _) = batch_case(gpu, 82, T, E, K, H, I, 1, False)
    Y2 = host(G.moe_experts(tg, tu, td, E, H, I, dev(X, gpu), K, eptr, tok, wt, 10.0))
    assert np.array_equal(Y.view(np.uint32), Y2.view(np.uint32))


@pytest.mark.parametrize("norm", [True, False])
def test_moe_batch_one_token_vs_moe_forward(gpu, norm):
    """One token (model.cpp:692-755): the reference's rank-order combine with
    (score / denom) * routed_scale, and the shared expert."""
    H, I, E, K = 1024, 512, 64, 8
    Y, _, (tg, tu, td, X, eptr, tok, wt, logits, bias, sh, wg, wu, wd) = batch_case(gpu, 83, 1, E, K, H, I, 0, True,
                                                                                     norm)
    ref = oracle.moe_forward(logits[0], X[0], wg, wu, wd, H, I, K, bias, 2.5, norm, 10.0, shared=sh)
    assert rel_err(Y[0], ref) < TIGHT


def test_moe_batch_errors(gpu):
    import torch

    T, E, K, H, I = 2, 4, 2, 256, 256
    w = G.tile(dev(synth.iq3xxs_matrix(84, 0, E * I, H).reshape(-1), gpu), E * I, H)
    X = torch.zeros(T, H, device=gpu)
    lg = torch.zeros(T, E, device=gpu)
    with pytest.raises(G.GpeedError) as e:  # only part of the shared expert
        G.moe_batch(lg, X, w, w, w, E, H, I, K, shared=(w, w, None))
    assert e.value.code == -1
    with pytest.raises(G.GpeedError) as e:
        G.moe_batch(lg, X, w, w, w, E, H, I, K, mode=3)
    assert e.value.code == -1
    ws = torch.zeros(256, dtype=torch.uint8, device=gpu)
    with pytest.raises(G.GpeedError) as e:
        G.moe_batch(lg, X, w, w, w, E, H, I, K, ws=ws)
    assert e.value.code == -7


# ------------------------------------------------------------------ prefill-sized batches (grouped GEMM)

@pytest.mark.parametrize("T,E,K,H,I,mode,shared", [
    (128, 16, 4, 1024, 512, 0, True),    # 32 tokens per expert on average: grouped GEMMs
    (72, 64, 8, 512, 256, 1, True),      # 9 per expert: the crossover
    (200, 8, 2, 768, 1280, 1, False),    # no shared expert; 50 per expert, partial 80-token tiles
    (300, 32, 6, 512, 512, 0, True),     # buckets of many tiles
    # 40 per expert: 64-token tiles; the shared expert's gate/up (5 x 2 x 32
    # tiles of the 32x32 form) fills the CUs, so it runs as GEMMs of its own
    (320, 16, 2, 512, 8192, 1, True),
])
def test_moe_batch_prefill_matches_oracle(gpu, T, E, K, H, I, mode, shared):
    """moe_batch at prefill chunk sizes (model_batch.cpp:165-281 called with
    n = the chunk, :391): from an average of 9 tokens per expert every
    expert's gate/up and down run as grouped MFMA GEMMs over its bucket
    (row0 = e*I, e*H; tiles of 32 to 80 tokens from the mean bucket), the
    shared expert as one more bucket of those launches or as GEMMs of its
    own; the router integers stay bit-exact and the outputs match the
    oracle."""
    assert G.lib().gpeed_iq3xxs_moe_batch_ws_bytes(T, E, K, H, I, int(shared)) > 0
    Y, ref, _ = batch_case(gpu, 85, T, E, K, H, I, mode, shared)
    e = max(rel_err(Y[t], ref[t]) for t in range(T))
    assert e < TIGHT, e


def test_moe_batch_prefill_full_size(gpu):
    """The routed-expert prefill chunk at the model's size: 512 tokens, 64
    experts of gate/up 2048x6144 and down 6144x2048, top-8 (reference
    router), with a shared expert of the same shape, from the logits. Every
    output is computed on the GPU; the oracle recomputes 6 sampled tokens
    (a token's output depends only on its own experts, so a sub-batch of
    those tokens gives the same rows)."""
    T, E, K, H, I = 512, 64, 8, 6144, 2048
    wg = synth.iq3xxs_matrix(86, 0, E * I, H)
    wu = synth.iq3xxs_matrix(86, 1, E * I, H)
    wd = synth.iq3xxs_matrix(86, 2, E * H, I)
    sh = tuple(synth.iq3xxs_matrix(86, 5 + i, r, c) for i, (r, c) in enumerate(((I, H), (I, H), (H, I))))
    X = synth.normal(86, 3, T * H).reshape(T, H)
    logits = synth.normal(86, 4, T * E).reshape(T, E)
    t = lambda a, r, c: G.tile(dev(a.reshape(-1), gpu), r, c)  # noqa: E731
    tsh = (t(sh[0], I, H), t(sh[1], I, H), t(sh[2], H, I))
    Y, eptr, tok, wt = G.moe_batch(dev(logits, gpu), dev(X, gpu), t(wg, E * I, H), t(wu, E * I, H),
                                   t(wd, E * H, I), E, H, I, K, 0, None, 2.5, True, 10.0, shared=tsh, routing=True)
    Y = host(Y)
    r_eptr, r_tok, _, _ = oracle.moe_route(logits, K, 0, routed_scale=2.5)
    assert np.array_equal(host(eptr), r_eptr) and np.array_equal(host(tok), r_tok)
    assert np.isfinite(Y).all()
    idx = np.array([0, 1, 97, 255, 400, 511])
    ref = oracle.moe_batch(logits[idx], X[idx], wg, wu, wd, H, I, K, 0, None, 2.5, True, 10.0, shared=sh)
    e = max(rel_err(Y[i], ref[j]) for j, i in enumerate(idx))
    # the full-size bar of the dense MLP tests (1e-4, against the parity bar
    # of 1e-3): at K = 6144 the fp32 summation-order noise of either side
    # alone is ~3e-6 of a row's rms, and its maximum over 6 x 6144 outputs,
    # through SwiGLU and a nine-term combine, reaches 2-3e-5
    assert e < 1e-4, e

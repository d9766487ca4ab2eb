"""Pins the CPU oracle (oracle/iq3_oracle.c) before it is trusted as the reference.

Each check is chosen so that a plausible slip in the restatement (a dropped
term, a wrong shift, a transposed operand, a different summation order) fails:
golden vectors written by the reference's own code, bitwise comparison with
the reference compiled from source (when built here), closed forms, brute
force, and fp64 products.
"""
import os
import re

import numpy as np
import pytest

import oracle
from gpeed_amd import synth
from conftest import ROOT, rel_err

GOLD = os.path.join(ROOT, "tests", "golden")
REF_TABLES = "/root/reference/cpp/core/include/glm5/iq3xxs_tables.h"
LEVELS = {4, 12, 20, 28, 36, 44, 52, 62}


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def same_bits_or_nan(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) | np.isnan(b)
    return bool(np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(bits(a)[~nan], bits(b)[~nan]))


# ------------------------------------------------------------------ tables

def _grid_from_header(path):
    text = open(path, encoding="utf-8").read()
    body = re.search(r"\[256\]\s*=\s*\{(.*?)\};", text, re.S).group(1)
    return [int(v, 0) for v in body.replace("\n", " ").split(",") if v.strip()]


def test_grid_invariants():
    g = [oracle.lib().orc_grid_entry(i) for i in range(256)]
    assert len(set(g)) == 256
    assert g == sorted(g)
    for v in g:
        assert {(v >> (8 * j)) & 255 for j in range(4)} <= LEVELS


def test_grid_copies_agree():
    g = [oracle.lib().orc_grid_entry(i) for i in range(256)]
    assert _grid_from_header(os.path.join(ROOT, "gpeed_amd", "csrc", "iq3_tables.h")) == g
    if os.path.exists(REF_TABLES):
        assert _grid_from_header(REF_TABLES) == g
        text = open(REF_TABLES, encoding="utf-8").read()
        body = re.search(r"kSignsIq2xs\[128\]\s*=\s*\{(.*?)\};", text, re.S).group(1)
        signs = [int(v, 0) for v in body.replace("\n", " ").split(",") if v.strip()]
        assert signs == [oracle.lib().orc_sign_byte(i) for i in range(128)]


def test_sign_byte_even_parity_closed_form():
    L = oracle.lib()
    for i in range(128):
        s = L.orc_sign_byte(i)
        assert s & 127 == i
        assert bin(s).count("1") % 2 == 0


# ------------------------------------------------------------------ fp16

def test_f16_all_patterns():
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    # through the F16 dequantize path (array output keeps NaN payloads intact;
    # a ctypes float return would quiet signalling NaNs)
    got = oracle.dequantize(h.view(np.uint8), 65536, dtype=1)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # NaN payload kept as man << 13 (quant.cpp:148)
    u = got.view(np.uint32)[nan]
    hv = h[nan].astype(np.uint32)
    assert np.array_equal(u, ((hv & 0x8000) << 16) | 0x7F800000 | ((hv & 0x3FF) << 13))


# ------------------------------------------------------------------ block decode

def _closed_form_block(raw):
    """w[32ib+8l+j] = d*(0.5+s)*0.5 * grid(qs[8ib+2l+j//4])[j%4] * (-1)^sign_j, in fp64."""
    d = float(np.frombuffer(raw[0:2].tobytes(), np.float16)[0])
    qs = raw[2:66]
    aux = np.frombuffer(raw[66:98].tobytes(), "<u4")
    out = np.zeros(256)
    grid = [oracle.lib().orc_grid_entry(i) for i in range(256)]
    for ib in range(8):
        a = int(aux[ib])
        db = d * (0.5 + (a >> 28)) * 0.5
        for l in range(4):
            s7 = (a >> (7 * l)) & 127
            sg = s7 | ((bin(s7).count("1") & 1) << 7)
            for j in range(8):
                g = (grid[qs[8 * ib + 2 * l + j // 4]] >> (8 * (j % 4))) & 255
                out[32 * ib + 8 * l + j] = db * g * (-1.0 if (sg >> j) & 1 else 1.0)
    return out


def test_block_golden_selftest():
    z = np.load(os.path.join(GOLD, "selftest_block.npz"))
    got = oracle.dequantize(z["raw"], 256)
    assert same_bits_or_nan(got, z["deq"])
    # the reference test's own criterion (gguf_selftest.cpp:14-18) also holds
    assert np.all(np.abs(got - z["deq"]) <= 1e-4 * np.maximum(1.0, np.abs(z["deq"])))


def test_block_golden_edges():
    z = np.load(os.path.join(GOLD, "edge_blocks.npz"))
    got = oracle.dequantize(z["raw"], z["raw"].shape[0] * 256)
    assert same_bits_or_nan(got, z["deq"])


def test_block_closed_form_and_exactness():
    blocks = synth.iq3xxs_blocks(3, 0, 16)
    for b in blocks:
        got = oracle.dequantize(b, 256)
        want = _closed_form_block(b)
        # every product has <= 21 significant bits: fp32 holds it exactly
        assert np.array_equal(got.astype(np.float64), want)


def test_block_brute_force_grid_sign_scale():
    """All 256 grid indices x 128 sign indices x 16 scales for one group, d = 1."""
    L = oracle.lib()
    grid = [L.orc_grid_entry(i) for i in range(256)]
    raw = np.zeros(98, np.uint8)
    raw[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    y = np.empty(256, np.float32)
    for s in range(16):
        for si in range(0, 128, 1 if s in (0, 15) else 37):
            aux = (s << 28) | si
            raw[66:70] = np.frombuffer(np.uint32(aux).tobytes(), np.uint8)
            for idx in range(0, 256, 1 if si in (0, 127) else 17):
                raw[2] = idx
                raw[3] = 255 - idx
                L.orc_iq3xxs_block(raw, y)
                sg = L.orc_sign_byte(si)
                db = (0.5 + s) * 0.5
                for j in range(8):
                    g = (grid[idx if j < 4 else 255 - idx] >> (8 * (j % 4))) & 255
                    assert y[j] == np.float32(db * g * (-1 if (sg >> j) & 1 else 1))


def test_dequantize_errors():
    L = oracle.lib()
    raw = np.zeros(98, np.uint8)
    out = np.empty(256, np.float32)
    assert L.orc_dequantize(18, raw.ctypes.data, out, 255) == -1
    assert L.orc_dequantize(12, raw.ctypes.data, out, 256) == -2


# ------------------------------------------------------------------ dot / matvec

def test_dot_golden():
    z = np.load(os.path.join(GOLD, "dot.npz"))
    for n, want in zip(z["lens"], z["dots"]):
        got = np.float32(oracle.lib().orc_dot_f32(z["a"], z["b"], int(n)))
        assert got.view(np.uint32) == np.float32(want).view(np.uint32), n


def test_dot_fp64_bound():
    a = synth.normal(5, 0, 12288)
    b = synth.normal(5, 1, 12288)
    got = oracle.dot_f32(a, b)
    exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
    bound = 12288 * 2 ** -24 * float(np.dot(np.abs(a).astype(np.float64), np.abs(b)))
    assert abs(got - exact) <= bound
    # and a reordering is detectable: the naive sequential sum differs in bits
    seq = np.float32(0)
    for i in range(12288):
        seq = np.float32(seq + a[i] * b[i])
    assert np.float32(got) != seq


def test_matvec_golden():
    z = np.load(os.path.join(GOLD, "matvec.npz"))
    y = oracle.matvec(z["w"], 16, 1024, 32, z["x"])
    assert np.array_equal(bits(y), bits(z["y_row16"]))
    Y = oracle.matmul(z["w"], 8, 1024, 32, z["X"])
    assert np.array_equal(bits(Y), bits(z["Y_row8"]))


def test_matmul_equals_per_token_matvec():
    w = synth.iq3xxs_matrix(4, 0, 40, 768)
    X = synth.normal(4, 9, 4 * 768).reshape(4, 768)
    Y = oracle.matmul(w, 0, 768, 40, X)
    for t in range(4):
        assert np.array_equal(bits(Y[t]), bits(oracle.matvec(w, 0, 768, 40, X[t])))


def test_matvec_fp64():
    w = synth.iq3xxs_matrix(6, 0, 64, 4096)
    x = synth.normal(6, 9, 4096)
    W = oracle.dequantize(w, 64 * 4096).reshape(64, 4096).astype(np.float64)
    assert rel_err(oracle.matvec(w, 0, 4096, 64, x), W @ x) < 1e-5


@pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref not built (needs the reference checkout)")
def test_oracle_bitwise_vs_reference_build():
    R = oracle.ref()
    w = synth.iq3xxs_matrix(8, 0, 96, 2048)
    deq = np.empty(96 * 2048, np.float32)
    assert R.ref_dequantize(18, w.ctypes.data, deq, deq.size) == 0
    assert same_bits_or_nan(oracle.dequantize(w, deq.size), deq)
    st = oracle.RefStore(w, 96, 2048)
    x = synth.normal(8, 1, 2048)
    assert np.array_equal(bits(oracle.matvec(w, 32, 2048, 48, x)), bits(st.matvec(32, 2048, 48, x)))
    X = synth.normal(8, 2, 5 * 2048).reshape(5, 2048)
    assert np.array_equal(bits(oracle.matmul(w, 16, 2048, 64, X)), bits(st.matmul(16, 2048, 64, X)))
    a = synth.normal(8, 3, 1000)
    b = synth.normal(8, 4, 1000)
    for n in list(range(1, 40)) + [999, 1000]:
        r = np.float32(R.ref_dot_f32(a, b, n))
        o = np.float32(oracle.lib().orc_dot_f32(a, b, n))
        assert r.view(np.uint32) == o.view(np.uint32), n
    for n in range(1, 65):
        p = a[:64].copy()
        q = p.copy()
        R.ref_axpy_f32(p, b[:64], np.float32(0.37), n)
        oracle.lib().orc_axpy_f32(q, b[:64], np.float32(0.37), n)
        assert np.array_equal(bits(p), bits(q))


@pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref not built (needs the reference checkout)")
@pytest.mark.parametrize("in_dim", [2048, 4096])
def test_oracle_edge_blocks_bitwise_vs_reference_build(in_dim):
    """The oracle's dequant, matvec and matmul on the edge-case matrices the
    GPU edge tests use (d = +-0, subnormal, +-65504, 2^+-20 jumps, +-inf,
    NaN): bit for bit the reference's own build, NaN positions included;
    and every row holding an infinite or NaN d is NaN in the reference
    (its +-inf products have both signs), the class the GPU must give."""
    from edge_cases import edge_matrix

    n_rows = 96
    w = edge_matrix(70, 9, n_rows, in_dim, nonfinite=True)
    R = oracle.ref()
    deq = np.empty(n_rows * in_dim, np.float32)
    assert R.ref_dequantize(18, w.ctypes.data, deq, deq.size) == 0
    assert same_bits_or_nan(oracle.dequantize(w, deq.size), deq)
    st = oracle.RefStore(w, n_rows, in_dim)
    x = synth.normal(70, 1, in_dim)
    yr = st.matvec(0, in_dim, n_rows, x)
    assert same_bits_or_nan(oracle.matvec(w, 0, in_dim, n_rows, x), yr)
    X = synth.normal(70, 2, 3 * in_dim).reshape(3, in_dim)
    assert same_bits_or_nan(oracle.matmul(w, 0, in_dim, n_rows, X), st.matmul(0, in_dim, n_rows, X))
    d = w.reshape(n_rows, -1, 98)[:, :, 0:2].copy().view(np.float16)[:, :, 0].astype(np.float32)
    bad = ~np.isfinite(d).all(axis=1)
    assert bad.any() and np.array_equal(np.isnan(yr), bad)


def test_oracle_swiglu_keeps_nan():
    """std::min(g, lim) and std::clamp(u, -lim, lim) (model.cpp:683-688,
    model_batch.cpp:245-253) return a NaN argument: a gate row that is NaN
    makes every down output NaN in the oracle's dense MLP, where fminf-style
    clamps would give finite outputs."""
    from edge_cases import edge_matrix

    H, I = 256, 512
    wg = edge_matrix(77, 0, I, H, nonfinite=True)
    wu = synth.iq3xxs_matrix(77, 1, I, H)
    wd = synth.iq3xxs_matrix(77, 2, H, I)
    x = synth.normal(77, 3, H).reshape(1, H)
    assert np.isnan(oracle.dense_mlp(wg, wu, wd, H, I, x, 10.0)).all()
    # a NaN up value alone (gate finite) also passes the clamp
    wu2 = edge_matrix(77, 4, I, H, nonfinite=True)
    wg2 = synth.iq3xxs_matrix(77, 5, I, H)
    assert np.isnan(oracle.dense_mlp(wg2, wu2, wd, H, I, x, 10.0)).all()


# ------------------------------------------------------------------ routing

def _brute_topk(key, k):
    order = sorted(range(len(key)), key=lambda e: (-key[e], e))
    return order[:k]


@pytest.mark.parametrize("mode", [0, 1])
def test_route_invariants_and_brute_force(mode):
    T, E, K = 32, 64, 8
    logits = synth.normal(21, mode, T * E).reshape(T, E)
    bias = synth.normal(21, 9, E) * np.float32(0.1) if mode == 0 else None
    eptr, tok, wt, sel = oracle.moe_route(logits, K, mode, bias=bias, routed_scale=2.5)
    assert eptr[0] == 0 and eptr[-1] == T * K and np.all(np.diff(eptr) >= 0)
    counts = np.bincount(sel.reshape(-1), minlength=E)
    assert np.array_equal(np.diff(eptr), counts)
    for e in range(E):
        seg = tok[eptr[e]:eptr[e + 1]]
        assert np.all(np.diff(seg) > 0)  # stable: ascending token, each once
        for t in seg:
            assert e in sel[t]
    assert np.array_equal(np.bincount(tok, minlength=T), np.full(T, K))
    for t in range(T):
        lg = logits[t].astype(np.float64)
        if mode == 0:
            score = 1.0 / (1.0 + np.exp(-lg))
            key = score + bias
        else:
            key = lg
        assert list(sel[t]) == _brute_topk(list(key.astype(np.float32)), K)
        w_t = np.array([wt[np.where((tok == t) & (np.arange(T * K) >= eptr[e]) & (np.arange(T * K) < eptr[e + 1]))[0][0]]
                        for e in sel[t]], np.float64)
        if mode == 0:
            want = score[sel[t]] / score[sel[t]].sum() * 2.5
        else:
            p = np.exp(lg[sel[t]] - lg[sel[t]].max())
            want = p / p.sum()
        assert np.allclose(w_t, want, rtol=2e-6, atol=0)


def test_route_ties_prefer_lower_expert():
    logits = np.zeros((2, 16), np.float32)
    logits[1, [3, 9]] = 1.0
    _, _, _, sel = oracle.moe_route(logits, 4, 1)
    assert list(sel[0]) == [0, 1, 2, 3]
    assert list(sel[1]) == [3, 9, 0, 1]


def test_moe_batch_with_shared_expert_fp64():
    """The whole moe_batch step (model_batch.cpp:165-281) with the reference
    router (mode 0: sigmoid, bias, routed_scale, norm_topk) and the shared
    expert added last, against an fp64 restatement of every piece: top-k of
    sigmoid(logit) + bias, weights score * scale / (1e-20 + sum), each expert
    FFN and the shared FFN over every token."""
    H, I, E, T, K = 512, 256, 8, 6, 3
    wg = synth.iq3xxs_matrix(32, 0, E * I, H)
    wu = synth.iq3xxs_matrix(32, 1, E * I, H)
    wd = synth.iq3xxs_matrix(32, 2, E * H, I)
    sg = synth.iq3xxs_matrix(32, 3, I, H)
    su = synth.iq3xxs_matrix(32, 4, I, H)
    sd = synth.iq3xxs_matrix(32, 5, H, I)
    X = synth.normal(32, 10, T * H).reshape(T, H)
    logits = synth.normal(32, 11, T * E).reshape(T, E)
    bias = synth.normal(32, 12, E) * 0.1
    scale = 2.5
    Y = oracle.moe_batch(logits, X, wg, wu, wd, H, I, K, 0, bias, scale, True, 10.0, shared=(sg, su, sd))
    deq = lambda w, r, c: oracle.dequantize(w, r * c).reshape(r, c).astype(np.float64)  # noqa: E731
    G, U, D = deq(wg, E * I, H).reshape(E, I, H), deq(wu, E * I, H).reshape(E, I, H), deq(wd, E * H, I).reshape(E, H, I)
    SG, SU, SD = deq(sg, I, H), deq(su, I, H), deq(sd, H, I)

    def ffn(g_m, u_m, d_m, x):
        g = np.minimum(g_m @ x, 10.0)
        u = np.clip(u_m @ x, -10.0, 10.0)
        return d_m @ (g / (1.0 + np.exp(-g)) * u)

    want = np.zeros((T, H))
    for t in range(T):
        s_e = 1.0 / (1.0 + np.exp(-logits[t].astype(np.float64)))
        top = np.argsort(-(s_e + bias), kind="stable")[:K]
        denom = 1e-20 + s_e[top].sum()
        for e in sorted(top):
            want[t] += s_e[e] * scale / denom * ffn(G[e], U[e], D[e], X[t])
        want[t] += ffn(SG, SU, SD, X[t])
    assert rel_err(Y, want) < 1e-5
    # without the shared expert it is the routed part alone
    Y0 = oracle.moe_batch(logits, X, wg, wu, wd, H, I, K, 0, bias, scale, True, 10.0)
    shared = np.stack([ffn(SG, SU, SD, X[t]) for t in range(T)])
    assert rel_err(Y0, want - shared) < 1e-5


def test_moe_forward_one_token_fp64():
    """moe_forward (model.cpp:692-755): the rank-order combine with
    (score / denom) * routed_scale, against fp64, and against the batched
    step at one token (same value, other rounding order)."""
    H, I, E, K = 512, 256, 16, 4
    wg = synth.iq3xxs_matrix(33, 0, E * I, H)
    wu = synth.iq3xxs_matrix(33, 1, E * I, H)
    wd = synth.iq3xxs_matrix(33, 2, E * H, I)
    sh = tuple(synth.iq3xxs_matrix(33, 3 + i, r, c) for i, (r, c) in enumerate(((I, H), (I, H), (H, I))))
    x = synth.normal(33, 10, H)
    logits = synth.normal(33, 11, E)
    bias = synth.normal(33, 12, E) * 0.1
    for norm in (True, False):
        y = oracle.moe_forward(logits, x, wg, wu, wd, H, I, K, bias, 2.5, norm, 10.0, shared=sh)
        deq = lambda w, r, c: oracle.dequantize(w, r * c).reshape(r, c).astype(np.float64)  # noqa: E731
        G, U, D = deq(wg, E * I, H).reshape(E, I, H), deq(wu, E * I, H).reshape(E, I, H), deq(wd, E * H, I).reshape(E, H, I)

        def ffn(g_m, u_m, d_m):
            g = np.minimum(g_m @ x, 10.0)
            u = np.clip(u_m @ x, -10.0, 10.0)
            return d_m @ (g / (1.0 + np.exp(-g)) * u)

        s_e = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
        top = np.argsort(-(s_e + bias), kind="stable")[:K]
        w = s_e[top] * 2.5 / ((1e-20 + s_e[top].sum()) if norm else 1.0)
        want = sum(w[k] * ffn(G[e], U[e], D[e]) for k, e in enumerate(top)) + ffn(deq(sh[0], I, H), deq(sh[1], I, H),
                                                                                 deq(sh[2], H, I))
        assert rel_err(y, want) < 1e-5
        yb = oracle.moe_batch(logits[None], x[None], wg, wu, wd, H, I, K, 0, bias, 2.5, norm, 10.0, shared=sh)[0]
        assert rel_err(y, yb) < 1e-6


def test_moe_experts_fp64():
    H, I, E, T, K = 512, 256, 6, 5, 2
    wg = synth.iq3xxs_matrix(31, 0, E * I, H)
    wu = synth.iq3xxs_matrix(31, 1, E * I, H)
    wd = synth.iq3xxs_matrix(31, 2, E * H, I)
    X = synth.normal(31, 10, T * H).reshape(T, H)
    logits = synth.normal(31, 11, T * E).reshape(T, E)
    eptr, tok, wt, sel = oracle.moe_route(logits, K, 1)
    Y = oracle.moe_experts(wg, wu, wd, H, I, X, eptr, tok, wt, 10.0)
    G = oracle.dequantize(wg, E * I * H).reshape(E, I, H).astype(np.float64)
    U = oracle.dequantize(wu, E * I * H).reshape(E, I, H).astype(np.float64)
    D = oracle.dequantize(wd, E * H * I).reshape(E, H, I).astype(np.float64)
    want = np.zeros((T, H))
    for e in range(E):
        for p in range(eptr[e], eptr[e + 1]):
            t = tok[p]
            g = np.minimum(G[e] @ X[t], 10.0)
            u = np.clip(U[e] @ X[t], -10.0, 10.0)
            want[t] += wt[p] * (D[e] @ (g / (1.0 + np.exp(-g)) * u))
    assert rel_err(Y, want) < 1e-5

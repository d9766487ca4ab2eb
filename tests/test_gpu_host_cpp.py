"""GPU tests of the C++ host layer (gpeed_amd/host/glm5_gpu.{h,cpp}): the
reference's call signatures -- glm5::cuda_device_count / cuda_device_name /
cuda_add (kernels.h:7-11) and WeightStore::matvec_quant / matmul_quant
(weights.h:41-48) plus the moe_batch expert step -- driven through
tests/cpp/host_check with host arrays, checked against the oracle."""
import os
import subprocess

import numpy as np
import pytest

import oracle
from gpeed_amd import synth
from conftest import ROOT, rel_err

pytestmark = pytest.mark.gpu
EXE = os.path.join(ROOT, "tests", "cpp", "host_check")
TIGHT = 2e-5


def run(*args):
    r = subprocess.run([EXE, *map(str, args)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=240)
    assert r.returncode == 0, r.stdout
    return r.stdout


def test_kernels_parity_set(gpu):
    out = run("kernels")
    assert "add=ok" in out and "devices=" in out and "name=<none>" not in out


def test_errors_match_reference(gpu):
    assert "missing=1 unaligned=1 zero=1" in run("errors")


@pytest.mark.parametrize("n_rows,in_dim,row0,out_dim,n_tok", [(200, 1536, 64, 136, 3), (6144, 12288, 0, 6144, 1),
                                                             (300, 512, 0, 300, 11), (704, 1536, 64, 600, 9),
                                                             (704, 1536, 64, 600, 64), (704, 1536, 64, 600, 512),
                                                             # row0 inside a 64-row tile (weights.cpp:86-203
                                                             # takes any row0): GEMV and GEMM sides
                                                             (200, 1536, 3, 136, 1), (200, 1536, 3, 136, 5),
                                                             (704, 1536, 67, 600, 33), (300, 512, 299, 1, 2)])
def test_matvec_matmul_quant(gpu, tmp_path, n_rows, in_dim, row0, out_dim, n_tok):
    w = synth.iq3xxs_matrix(80, n_tok, n_rows, in_dim)
    X = synth.normal(80, 1, n_tok * in_dim).reshape(n_tok, in_dim)
    w.tofile(tmp_path / "w.bin")
    X.tofile(tmp_path / "x.bin")
    run("matmul", tmp_path, n_rows, in_dim, row0, out_dim, n_tok)
    y = np.fromfile(tmp_path / "y.bin", np.float32)
    Y = np.fromfile(tmp_path / "Y.bin", np.float32).reshape(n_tok, out_dim)
    assert rel_err(y, oracle.matvec(w, row0, in_dim, out_dim, X[0])) < TIGHT
    ref = oracle.matmul(w, row0, in_dim, out_dim, X)
    assert max(rel_err(Y[t], ref[t]) for t in range(n_tok)) < TIGHT


@pytest.mark.parametrize("mode", [0, 1])
def test_moe_experts(gpu, tmp_path, mode):
    E, H, I, T, K = 16, 1024, 512, 12, 4
    wg = synth.iq3xxs_matrix(81, 0, E * I, H)
    wu = synth.iq3xxs_matrix(81, 1, E * I, H)
    wd = synth.iq3xxs_matrix(81, 2, E * H, I)
    X = synth.normal(81, 3, T * H).reshape(T, H)
    logits = synth.normal(81, 4, T * E).reshape(T, E)
    for name, a in (("gate", wg), ("up", wu), ("down", wd), ("x", X), ("logits", logits)):
        a.tofile(tmp_path / f"{name}.bin")
    run("moe", tmp_path, E, H, I, T, K, mode)
    Y = np.fromfile(tmp_path / "Y.bin", np.float32).reshape(T, H)
    eptr, tok, wt, _ = oracle.moe_route(logits, K, mode, routed_scale=2.5 if mode == 0 else 1.0)
    ref = oracle.moe_experts(wg, wu, wd, H, I, X, eptr, tok, wt, 10.0)
    assert max(rel_err(Y[t], ref[t]) for t in range(T)) < TIGHT


@pytest.mark.parametrize("shared", [False, True])
def test_moe_batch_whole_step(gpu, tmp_path, shared):
    """WeightStore::moe_batch (model_batch.cpp:174-280 after the router
    product) through the C++ layer, with and without the shared expert,
    against the oracle's moe_batch."""
    E, H, I, T, K, mode = 16, 1024, 512, 12, 4, 0
    wg = synth.iq3xxs_matrix(82, 0, E * I, H)
    wu = synth.iq3xxs_matrix(82, 1, E * I, H)
    wd = synth.iq3xxs_matrix(82, 2, E * H, I)
    sg = synth.iq3xxs_matrix(82, 5, I, H)
    su = synth.iq3xxs_matrix(82, 6, I, H)
    sd = synth.iq3xxs_matrix(82, 7, H, I)
    X = synth.normal(82, 3, T * H).reshape(T, H)
    logits = synth.normal(82, 4, T * E).reshape(T, E)
    for name, a in (("gate", wg), ("up", wu), ("down", wd), ("gate_sh", sg), ("up_sh", su), ("down_sh", sd),
                    ("x", X), ("logits", logits)):
        a.tofile(tmp_path / f"{name}.bin")
    run("moe-batch", tmp_path, E, H, I, T, K, mode, int(shared))
    Y = np.fromfile(tmp_path / "Y.bin", np.float32).reshape(T, H)
    ref = oracle.moe_batch(logits, X, wg, wu, wd, H, I, K, mode, None, 2.5, True, 10.0,
                           shared=(sg, su, sd) if shared else None)
    assert max(rel_err(Y[t], ref[t]) for t in range(T)) < TIGHT


@pytest.mark.parametrize("T", [12, 96])
def test_moe_batch_with_router_product(gpu, tmp_path, T):
    """WeightStore::moe_batch from X with the router product on the device
    (model_batch.cpp:172, ffn_gate_inp F32 [E, H]): its logits are bitwise
    the reference's dot_f32, so the routing equals the oracle's from the
    oracle's logits; 12 tokens run the grouped GEMVs, 96 the grouped GEMMs."""
    E, H, I, K, mode = 16, 1024, 512, 4, 0
    wr = (synth.normal(87, 9, E * H) * np.float32(0.05)).astype(np.float32).reshape(E, H)
    wg = synth.iq3xxs_matrix(87, 0, E * I, H)
    wu = synth.iq3xxs_matrix(87, 1, E * I, H)
    wd = synth.iq3xxs_matrix(87, 2, E * H, I)
    sg = synth.iq3xxs_matrix(87, 5, I, H)
    su = synth.iq3xxs_matrix(87, 6, I, H)
    sd = synth.iq3xxs_matrix(87, 7, H, I)
    X = synth.normal(87, 3, T * H).reshape(T, H)
    for name, a in (("router", wr), ("gate", wg), ("up", wu), ("down", wd), ("gate_sh", sg), ("up_sh", su),
                    ("down_sh", sd), ("x", X)):
        a.tofile(tmp_path / f"{name}.bin")
    run("moe-router", tmp_path, E, H, I, T, K, mode)
    Y = np.fromfile(tmp_path / "Y.bin", np.float32).reshape(T, H)
    logits = oracle.matmul_rows(0, wr.view(np.uint8).reshape(E, -1), 0, H, E, X)
    ref = oracle.moe_batch(logits, X, wg, wu, wd, H, I, K, mode, None, 2.5, True, 10.0, shared=(sg, su, sd))
    assert max(rel_err(Y[t], ref[t]) for t in range(T)) < TIGHT


@pytest.mark.parametrize("T", [1, 5, 70])
def test_dense_mlp_host(gpu, tmp_path, T):
    """WeightStore::dense_mlp: Model::dense_mlp (model.cpp:677-690) at one
    token through the dense GEMV pair, dense_mlp_batch (model_batch.cpp:
    145-163) at 5 and 70 through gpeed_iq3xxs_mlp_gemm, against the oracle."""
    H, I = 1024, 2048
    wg = synth.iq3xxs_matrix(89, 0, I, H)
    wu = synth.iq3xxs_matrix(89, 1, I, H)
    wd = synth.iq3xxs_matrix(89, 2, H, I)
    X = synth.normal(89, T, T * H).reshape(T, H)
    for name, a in (("gate", wg), ("up", wu), ("down", wd), ("x", X)):
        a.tofile(tmp_path / f"{name}.bin")
    run("dense-mlp", tmp_path, H, I, T)
    Y = np.fromfile(tmp_path / "Y.bin", np.float32).reshape(T, H)
    ref = oracle.dense_mlp(wg, wu, wd, H, I, X, 10.0)
    assert max(rel_err(Y[t], ref[t]) for t in range(T)) < TIGHT

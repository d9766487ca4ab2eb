#!/usr/bin/env python3
"""IQ3_XXS decode benchmark on one MI355X.

Workload: the dense-layer decode step at batch 1 (dense_mlp, model.cpp:677-690)
with IQ3_XXS weights gate/up 12288x6144 (K=6144) and down 6144x12288
(K=12288): prepare x, gate and up matvecs sharing the prepared activation,
SwiGLU fused into the down projection's activation prep, down matvec.
Weights are synthetic (seeded, the block distribution of gpeed_amd.synth),
x ~ N(0,1) fp32, resident in HBM before timing. To measure HBM rather than
the 256 MB Infinity Cache, `--copies` distinct copies of the three tensors
(default 8, 694 MB) are rotated step by step.

value = packed weight bytes per step (3 x 28,901,376) / step time, GB/s.
roofline = the GEMV kernel (k_gemv_t64, launched once for gate+up and
once for down per step): algorithmic bytes of its launches (packed W +
prepared activation + outputs) / their summed duration, each launch timed
with HIP events on the launch stream during the timed steps, against 8 TB/s.
cpu_baseline = the reference's own CPU path (oracle/_ref: WeightStore::
matvec_quant compiled from the reference sources, single-threaded as the
reference builds on Linux) on one full step of the same workload; the
oracle's C restatement stands in if oracle/_ref was not built.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "IQ3_XXS GEMV weight GB/s (% of HBM peak) at batch 1; prefill GEMM TFLOP/s"
HBM_PEAK_GBS = 8000.0
H, I = 6144, 12288
SWIGLU_LIMIT = 10.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_baseline(wg, wu, wd, x):
    """Reference CPU dense-MLP decode step; returns (record, y_ref)."""
    import oracle

    W_BYTES = wg.nbytes + wu.nbytes + wd.nbytes
    ref = oracle.ref(openmp=False)
    out = {}
    if ref is not None:
        stores = [oracle.RefStore(wg, I, H, name="blk.0.ffn_gate.weight"),
                  oracle.RefStore(wu, I, H, name="blk.0.ffn_up.weight"),
                  oracle.RefStore(wd, H, I, name="blk.0.ffn_down.weight")]

        def step():
            g = stores[0].matvec(0, H, I, x)
            u = stores[1].matvec(0, H, I, x)
            gi = np.minimum(g, np.float32(SWIGLU_LIMIT))
            ui = np.clip(u, -SWIGLU_LIMIT, SWIGLU_LIMIT).astype(np.float32)
            h = (gi / (np.float32(1.0) + np.exp(-gi))) * ui
            return stores[2].matvec(0, I, H, h.astype(np.float32))

        kind = "reference"
    else:
        def step():
            return oracle.dense_mlp(wg, wu, wd, H, I, x[None, :], SWIGLU_LIMIT)[0]

        kind = "port"
    y_ref = step()  # warm-up
    times = []
    t_end = time.time() + 20.0
    while len(times) < 5 and (time.time() < t_end or len(times) < 2):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    out = {"value": round(W_BYTES / med / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
           "sample": f"{len(times)} dense-MLP decode steps (3 matvecs, {W_BYTES} packed bytes each), "
                     f"median; best {W_BYTES / min(times) / 1e9:.4f} GB/s"}
    ref_omp = oracle.ref(openmp=True) if kind == "reference" else None
    if ref_omp is not None:
        ncores = len(os.sched_getaffinity(0))
        nth = ref_omp.ref_openmp_threads()
        st = oracle.RefStore(wd, H, I, openmp=True, name="blk.0.ffn_down.weight")
        h1 = np.ones(I, np.float32)
        st.matvec(0, I, H, h1)  # warm-up
        tt = []
        t_end = time.time() + 10.0
        while len(tt) < 10 and (time.time() < t_end or len(tt) < 2):
            t0 = time.perf_counter()
            st.matvec(0, I, H, h1)
            tt.append(time.perf_counter() - t0)
        out["all_cores"] = {"value": round(wd.nbytes / statistics.median(tt) / 1e9, 4), "unit": "GB/s",
                            "cores": nth, "host_cpus": ncores,
                            "sample": f"{len(tt)} down-projection matvecs (6144x12288), median"}
        st.close()
    for s in (stores if kind == "reference" else []):
        s.close()
    return out, y_ref


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the multi-GPU "
              "sharding of this path is a design note, not a measured configuration).", file=sys.stderr)
        sys.exit(2)

    import torch

    import gpeed_amd as G
    from gpeed_amd import synth

    dev = torch.device("cuda:0")
    G.init()
    log("generating weights")
    wg = synth.iq3xxs_matrix(2024, 0, I, H)
    wu = synth.iq3xxs_matrix(2024, 1, I, H)
    wd = synth.iq3xxs_matrix(2024, 2, H, I)
    x = synth.normal(2024, 100, H)
    W_BYTES = wg.nbytes + wu.nbytes + wd.nbytes

    base = [G.tile(torch.from_numpy(a.reshape(-1)).to(dev), r, c) for a, r, c in ((wg, I, H), (wu, I, H), (wd, H, I))]
    copies = [base] + [[t.clone() for t in base] for _ in range(args.copies - 1)]
    xd = torch.from_numpy(x).to(dev)
    act = G.act_buffer(H, 1, dev)
    act2 = G.act_buffer(I, 1, dev)
    ws_gu = G.gemv_workspace(H, I, 1, 2, dev)
    ws_d = G.gemv_workspace(I, H, 1, 1, dev)
    g = torch.empty(1, I, device=dev)
    u = torch.empty(1, I, device=dev)
    y = torch.empty(1, H, device=dev)
    stream = torch.cuda.current_stream()

    def timed_launch(ev, kind, fn):
        if ev is None:
            fn()
            return
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn()
        b.record(stream)
        ev.append((kind, a, b))

    def step(c, ev=None):
        tg, tu, td = copies[c]
        G.prep_act(xd, act)
        timed_launch(ev, "gate+up", lambda: G.gemv2_act(tg, tu, I, 0, H, I, act, 1, out_a=g, out_b=u, ws=ws_gu))
        G.prep_swiglu(g, u, act2, SWIGLU_LIMIT)
        timed_launch(ev, "down", lambda: G.gemv_act(td, H, 0, I, H, act2, 1, out=y, ws=ws_d))

    log("warmup")
    for i in range(args.warmup):
        step(i % args.copies)
    torch.cuda.synchronize()
    step(0)
    torch.cuda.synchronize()
    y_gpu = y.cpu().numpy()[0].copy()

    log("timed")
    ev = []
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for i in range(args.steps):
        step(i % args.copies, ev)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    # k_gemv_t64 launches: bytes = packed W + prepared activation + outputs
    act_bytes = {"gate+up": G.lib().gpeed_iq3xxs_act_bytes(H, 1), "down": G.lib().gpeed_iq3xxs_act_bytes(I, 1)}
    launch_bytes = {"gate+up": 2 * (W_BYTES // 3) + act_bytes["gate+up"] + 2 * I * 4,
                    "down": W_BYTES // 3 + act_bytes["down"] + H * 4}
    per_kind = {}
    for kind, a, b in ev:
        per_kind.setdefault(kind, []).append(a.elapsed_time(b))
    tot_ms = sum(sum(v) for v in per_kind.values())
    tot_bytes = sum(launch_bytes[k] * len(v) for k, v in per_kind.items())
    achieved = tot_bytes / (tot_ms * 1e-3) / 1e9
    value = W_BYTES / (ms * 1e-3) / 1e9
    kinds = {k: {"mean_us": round(statistics.fmean(v) * 1e3, 3), "launches": len(v),
                 "algorithmic_bytes": launch_bytes[k],
                 "GBps": round(launch_bytes[k] / (statistics.fmean(v) * 1e-3) / 1e9, 1)}
             for k, v in per_kind.items()}

    rec = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "iq3_xxs weights, fp32 activations; f16 MFMA on exact operands, f32 accumulate",
        "data": "synthetic (seeded IQ3_XXS blocks, x ~ N(0,1)); weights resident in HBM, "
                f"{args.copies} rotated copies ({args.copies * W_BYTES / 1e6:.0f} MB)",
        "config": {"workload": "dense-layer decode at batch 1: IQ3_XXS gate/up 12288x6144, "
                               "down 6144x12288 (prep, 2 matvec, SwiGLU-prep, matvec)",
                   "packed_weight_bytes_per_step": W_BYTES, "batch": 1},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "k_gemv_t64", "launch_kinds": kinds},
    }
    if not args.no_cpu:
        log("cpu baseline")
        cb, y_ref = cpu_baseline(wg, wu, wd, x)
        rec["cpu_baseline"] = cb
        y_ref = np.asarray(y_ref, np.float64)
        rms = float(np.sqrt(np.mean(y_ref * y_ref)))
        rec["parity_rel_err"] = float(np.max(np.abs(y_gpu - y_ref) / np.maximum(np.abs(y_ref), rms)))
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()

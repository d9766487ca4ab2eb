#!/usr/bin/env python3
"""IQ3_XXS dequantize-and-multiply benchmark on one MI355X.

Headline workload (value / metric): the dense-layer decode step at batch 1
(dense_mlp, model.cpp:677-690) with IQ3_XXS weights gate/up 12288x6144
(K=6144) and down 6144x12288 (K=12288) through gpeed_iq3xxs_dense_mlp: a
gate+up launch (each wavefront prepares the activation blocks of its
records; the workgroup that completes 64 rows writes SwiGLU(gate, up) as the
down projection's prepared activation), then the down launch.
Weights are synthetic (seeded, the block distribution
of gpeed_amd.synth), x ~ N(0,1) fp32, resident in HBM before timing. To
measure HBM rather than the 256 MB Infinity Cache, `--copies` distinct
copies of the three tensors (default 8, 694 MB) are rotated step by step.

value = packed weight bytes per step (3 x 28,901,376) / step time, GB/s, over
the --steps timed steps; before the --warmup steps the step runs untimed for
about 0.25 s so that a freshly leased GPU's clocks and launch path settle.
roofline = the GEMV kernel (k_gemv_t64: the gate+up launch and the down
launch of a step): algorithmic bytes of the pair (packed W + fp32 x + the
SwiGLU activation written and read + y) / the pair's duration, timed with
HIP events on the launch stream around back-to-back steps of all copies in
turn, as C-ABI calls or as replays of a HIP graph, whichever is faster (no
host gaps either way; still HBM-bound). roofline.down: the 6144x12288 shape
alone (gpeed_iq3xxs_matvec on an fp32 vector, rotated copies), timed the
same way, as its own field.
cpu_baseline = the reference's own CPU path (oracle/_ref: WeightStore::
matvec_quant compiled from the reference sources, single-threaded as the
reference builds on Linux) on one full step of the same workload; the
oracle's C restatement stands in if oracle/_ref was not built.

Secondary line items (same JSON object, key "extra"): the routed-expert
decode batch (64 experts of gate/up 2048x6144 and down 6144x2048, 32
tokens, softmax top-8: GB/s over the packed bytes of the touched experts),
the prefill GEMM (W 12288x6144, X bf16 [M,6144], M = 512 and 2048:
TFLOP/s = 2*M*N*K / kernel time from dispatch-stamped events, against the
2.5 PFLOP/s dense bf16/fp16 MFMA peak), and the continuous-batching decode
mix (64 tokens through the latent projections and the shared-expert FFN:
GB/s over the packed weights and TFLOP/s, both fractions), the MLA
per-head projections attn_k_b / attn_v_b (64 heads each, one launch per
tensor, against 64 matvec launches), the router product of moe_batch (F32
64x6144 in dot_f32's order, 32 and 512 tokens), and the other GGUF formats
over raw rows (one token: GB/s; a 512-token chunk: fp32-MFMA TFLOP/s).
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
# Kernel arguments in device memory (set before the HIP runtime starts): a
# launch's first scalar loads of its arguments then come from HBM instead of
# host memory, about 1.1 us less per launch on this stack (measured: dense
# step 35.7 -> 33.2 us on one box). The library's callers get the same by
# exporting the variable.
os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "1")

METRIC = "IQ3_XXS GEMV weight GB/s (% of HBM peak) at batch 1; prefill GEMM TFLOP/s"
HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix peak
H, I = 6144, 12288
SWIGLU_LIMIT = 10.0
# HBM traffic of the GEMV pair, measured with rocprofv3 --pmc (FETCH_SIZE and
# WRITE_SIZE per dispatch, each scaled by what the counter reads for an
# elementwise copy of known size); see the summary file for the commands.
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "k_gemv_t64_dense_decode_traffic.md")


def measured_traffic():
    """HBM bytes per gate+up + down pair from the committed counter summary, or None."""
    try:
        with open(TRAFFIC_SUMMARY) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_pair:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


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
            with np.errstate(over="ignore"):  # exp(-g) overflows to inf for g << 0: silu -> -0, as in C
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
    out = {"value": round(W_BYTES / med / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind, "cpu_model": _cpu_model(),
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


def moe_decode(torch, G, synth, dev, steps, warmup_s):
    """Routed-expert decode batch: route + grouped gate/up + SwiGLU + grouped down + combine."""
    E, T, K, HM, IM = 64, 32, 8, 6144, 2048
    log("moe: generating 64 experts")
    tens = []
    for i, (r, c) in enumerate(((E * IM, HM), (E * IM, HM), (E * HM, IM))):
        raw = torch.from_numpy(synth.iq3xxs_matrix(2025, i, r, c).reshape(-1)).to(dev)
        tens.append(G.tile(raw, r, c))
        del raw
    X = torch.from_numpy(synth.normal(2025, 10, T * HM).reshape(T, HM)).to(dev)
    logits = torch.from_numpy(synth.normal(2025, 11, T * E).reshape(T, E)).to(dev)
    ws_r = torch.zeros(G.lib().gpeed_moe_route_ws_bytes(T, E, K), dtype=torch.uint8, device=dev)
    ws_e = torch.zeros(G.lib().gpeed_iq3xxs_moe_ws_bytes(T, E, K, HM, IM), dtype=torch.uint8, device=dev)
    Y = torch.empty(T, HM, device=dev)

    def step():
        eptr, tok, wt, _ = G.moe_route(logits, K, 1, ws=ws_r)
        G.moe_experts(tens[0], tens[1], tens[2], E, HM, IM, X, K, eptr, tok, wt, SWIGLU_LIMIT, out=Y, ws=ws_e)
        return eptr

    # timed through the C ABI with prebuilt arguments (as the dense step):
    # the Python wrappers' host time per step is of the order of the GPU's
    import ctypes
    L = G.lib()
    cur = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    r_eptr = torch.empty(E + 1, dtype=torch.int32, device=dev)
    r_tok = torch.empty(T * K, dtype=torch.int32, device=dev)
    r_wt = torch.empty(T * K, dtype=torch.float32, device=dev)
    r_sel = torch.empty(T, K, dtype=torch.int32, device=dev)
    route_args = (vp(logits), T, E, K, 1, ctypes.c_void_p(0), ctypes.c_float(1.0), 1, vp(r_eptr), vp(r_tok),
                  vp(r_wt), vp(r_sel), vp(ws_r), ws_r.numel(), cur)
    exp_args = (vp(tens[0]), vp(tens[1]), vp(tens[2]), E, HM, IM, vp(X), T, K, vp(r_eptr), vp(r_tok), vp(r_wt),
                ctypes.c_float(SWIGLU_LIMIT), vp(Y), vp(ws_e), ws_e.numel(), cur)

    def step_fast():
        if L.gpeed_moe_route(*route_args) != 0 or L.gpeed_iq3xxs_moe_experts(*exp_args) != 0:
            raise RuntimeError(f"moe: {L.gpeed_last_error().decode(errors='replace')}")

    # warm-up by time, not count: after the CPU-bound weight generation the
    # GPU runs the first ~100 ms of steps measurably slower
    import time
    eptr = step()
    t_end = time.perf_counter() + warmup_s
    while time.perf_counter() < t_end:
        for _ in range(20):
            step_fast()
        torch.cuda.synchronize()
    if not torch.equal(r_eptr, eptr):
        raise RuntimeError("moe: prebuilt and wrapper routes differ")
    counts = np.diff(eptr.cpu().numpy())
    touched = int((counts > 0).sum())
    blk_bytes = IM * HM // 256 * 98  # one expert's gate (or up, or down) tensor
    moe_bytes = touched * 3 * blk_bytes
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    # each timed loop follows an untimed lead-in of the same length with no
    # synchronisation between them, so it measures back-to-back steps
    for _ in range(steps):
        step_fast()
    t0.record()
    for _ in range(steps):
        step_fast()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    for _ in range(steps):
        step()
    t0.record()
    for _ in range(steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    ms_wrapped = t0.elapsed_time(t1) / steps
    # kernel durations from dispatch-stamped launches, in a loop of their own
    # (the stamps add to the step)
    G.prof_start(4 * steps + 8)
    for _ in range(steps):
        step_fast()
    torch.cuda.synchronize()
    d = G.prof_read(G.PROF_GROUPED).astype(np.float64)  # launch order: gate+up, down, ...
    gu, dn = d[0::2], d[1::2]
    n_asg = T * K
    gu_bytes = touched * 2 * blk_bytes + n_asg * (HM // 256) * 1028 + 2 * n_asg * IM * 4
    dn_bytes = touched * blk_bytes + n_asg * (IM // 256) * 1028 + n_asg * HM * 4
    k_ms = float(gu.mean() + dn.mean())

    # the whole step from the logits with a shared expert of the same shape
    # (gpeed_iq3xxs_moe_batch: five launches)
    sh = []
    for i, (r, c) in enumerate(((IM, HM), (IM, HM), (HM, IM))):
        raw = torch.from_numpy(synth.iq3xxs_matrix(2025, 20 + i, r, c).reshape(-1)).to(dev)
        sh.append(G.tile(raw, r, c))
        del raw
    ws_b = G.moe_batch_workspace(T, E, K, HM, IM, True, dev)
    nul = ctypes.c_void_p(0)
    batch_args = (vp(logits), T, E, K, 1, nul, ctypes.c_float(1.0), 1, vp(tens[0]), vp(tens[1]), vp(tens[2]),
                  vp(sh[0]), vp(sh[1]), vp(sh[2]), HM, IM, vp(X), ctypes.c_float(SWIGLU_LIMIT), vp(Y), nul, nul,
                  nul, vp(ws_b), ws_b.numel(), cur)

    def step_batch():
        if L.gpeed_iq3xxs_moe_batch(*batch_args) != 0:
            raise RuntimeError(f"moe: {L.gpeed_last_error().decode(errors='replace')}")

    t_end = time.perf_counter() + warmup_s
    while time.perf_counter() < t_end:
        for _ in range(20):
            step_batch()
        torch.cuda.synchronize()
    for _ in range(steps):
        step_batch()
    t0.record()
    for _ in range(steps):
        step_batch()
    t1.record()
    torch.cuda.synchronize()
    ms_b = t0.elapsed_time(t1) / steps
    G.prof_start(4 * steps + 8)
    for _ in range(steps):
        step_batch()
    torch.cuda.synchronize()
    d = G.prof_read(G.PROF_GROUPED).astype(np.float64)
    b_bytes = moe_bytes + 3 * blk_bytes
    whole = {"entry": "gpeed_iq3xxs_moe_batch", "launches": 5,
             "workload": "the same batch from the logits with a shared expert (gate/up 2048x6144, down "
                         "6144x2048) over every token, added last",
             "packed_bytes_per_step": b_bytes, "ms_per_step": round(ms_b, 4),
             "GBps": round(b_bytes / (ms_b * 1e-3) / 1e9, 1),
             "frac_of_hbm_peak": round(b_bytes / (ms_b * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
             "grouped_gate_up_us": round(float(d[0::2].mean()) * 1e3, 2),
             "grouped_down_us": round(float(d[1::2].mean()) * 1e3, 2)}
    prefill = moe_prefill(torch, G, synth, dev, tens, sh, 20)
    return prefill, {
        "workload": "routed-expert decode batch: 64 experts x (gate/up 2048x6144 + down 6144x2048) IQ3_XXS, "
                    "32 tokens, softmax top-8, router + grouped GEMVs + combine on the GPU",
        "touched_experts": touched, "packed_bytes_per_step": moe_bytes,
        "ms_per_step": round(ms, 4), "ms_per_step_python_wrappers": round(ms_wrapped, 4),
        "GBps": round(moe_bytes / (ms * 1e-3) / 1e9, 1),
        "frac_of_hbm_peak": round(moe_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "grouped_gemv": {"kernel": "k_gemv_grouped", "gate_up_us": round(float(gu.mean()) * 1e3, 2),
                         "down_us": round(float(dn.mean()) * 1e3, 2),
                         "algorithmic_bytes": gu_bytes + dn_bytes,
                         "GBps": round((gu_bytes + dn_bytes) / (k_ms * 1e-3) / 1e9, 1),
                         "frac": round((gu_bytes + dn_bytes) / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "whole_step": whole,
    }


def moe_prefill(torch, G, synth, dev, tens, sh, reps):
    """Routed-expert prefill chunk: moe_batch over 512 tokens (64 experts,
    top-8 softmax, shared expert), the experts as grouped MFMA GEMMs."""
    import ctypes
    E, T, K, HM, IM = 64, 512, 8, 6144, 2048
    L = G.lib()
    cur = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    X = torch.from_numpy(synth.normal(2027, 10, T * HM).reshape(T, HM)).to(dev)
    logits = torch.from_numpy(synth.normal(2027, 11, T * E).reshape(T, E)).to(dev)
    Y = torch.empty(T, HM, device=dev)
    eptr = torch.empty(E + 1, dtype=torch.int32, device=dev)
    ws = G.moe_batch_workspace(T, E, K, HM, IM, True, dev)
    nul = ctypes.c_void_p(0)
    args = (vp(logits), T, E, K, 1, nul, ctypes.c_float(1.0), 1, vp(tens[0]), vp(tens[1]), vp(tens[2]),
            vp(sh[0]), vp(sh[1]), vp(sh[2]), HM, IM, vp(X), ctypes.c_float(SWIGLU_LIMIT), vp(Y), vp(eptr), nul,
            nul, vp(ws), ws.numel(), cur)

    def step():
        if L.gpeed_iq3xxs_moe_batch(*args) != 0:
            raise RuntimeError(f"moe prefill: {L.gpeed_last_error().decode(errors='replace')}")

    for _ in range(5):
        step()
    torch.cuda.synchronize()
    counts = np.diff(eptr.cpu().numpy())
    touched = int((counts > 0).sum())
    blk_bytes = IM * HM // 256 * 98
    # every touched expert's three tensors and the shared expert's, once
    packed = (touched + 1) * 3 * blk_bytes
    flops = 2.0 * (T * K + T) * 3 * HM * IM
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    G.prof_start(8 * reps + 8)
    for _ in range(reps):
        step()
    torch.cuda.synchronize()
    # per step: the grouped gate/up and down GEMMs (the shared expert among
    # their buckets), or those and the shared expert's two GEMMs
    d = G.prof_read(G.PROF_GEMM).astype(np.float64) * 1e3
    per = max(1, int(round(len(d) / reps)))
    names = ["grouped_gate_up_us", "grouped_down_us", "shared_gate_up_us", "shared_down_us"][:per]
    kern = {n: round(float(d[i::per].mean()), 2) for i, n in enumerate(names)}
    return {"workload": "routed-expert prefill chunk: 512 tokens, 64 experts x (gate/up 2048x6144 + down "
                        "6144x2048) IQ3_XXS, softmax top-8, shared expert of the same shape; fp32 X; the experts' "
                        "buckets as grouped MFMA GEMMs (k_gemm5, 32-80-token tiles of hi + lo images, the shared expert as one more bucket)",
            "entry": "gpeed_iq3xxs_moe_batch", "touched_experts": touched,
            "packed_bytes_read_once": packed, "gflop_per_step": round(flops / 1e9, 2),
            "ms_per_step": round(ms, 4), "GBps": round(packed / (ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(packed / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1),
            "frac_of_fp16_peak": round(flops / (ms * 1e-3) / 1e12 / 2500.0, 4), "gemm_kernels": kern}


def router_product(torch, G, synth, dev, reps):
    """moe_batch step 1 (model_batch.cpp:172): logits = X . ffn_gate_inp^T, an
    F32 [64, 6144] tensor, for 32 and 512 tokens, through gpeed_matmul_rows
    (dot_f32's own order: bitwise the reference's logits)."""
    import ctypes
    E, HM = 64, 6144
    L = G.lib()
    cur = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    wr = torch.from_numpy((synth.normal(2028, 0, E * HM) * np.float32(0.05)).astype(np.float32)).to(dev)
    out = {}
    for T in (32, 512):
        X = torch.from_numpy(synth.normal(2028, T, T * HM).reshape(T, HM)).to(dev)
        lg = torch.empty(T, E, device=dev)
        a = (0, vp(wr), E, 0, HM, E, vp(X), T, vp(lg), cur)
        for _ in range(5):
            L.gpeed_matmul_rows(*a)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            if L.gpeed_matmul_rows(*a) != 0:
                raise RuntimeError(L.gpeed_last_error().decode(errors="replace"))
        e1.record()
        torch.cuda.synchronize()
        out[f"T{T}_us"] = round(e0.elapsed_time(e1) / reps * 1e3, 2)
    return {"workload": "router product of moe_batch: F32 ffn_gate_inp [64, 6144] times X [T, 6144] "
                        "(k_dot_rows_f32, dot_f32's order), back-to-back launches", **out}


def prefill_gemm(torch, G, synth, dev, reps, copies=12):
    """Prefill GEMM: IQ3_XXS W 12288x6144, X bf16 [M, 6144], Y fp32 [M, 12288], M = 512 and 2048.
    `copies` rotated weight copies (28.9 MB each, 347 MB in all: above the 256 MB Infinity Cache),
    so each call reads its W from HBM as a prefill over a model's layers does. kernel_us comes
    from dispatch-stamped launches in a loop of their own; stamp_overhead_us is that loop's time
    per call less the unstamped loop's."""
    N, K = 12288, 6144
    w = synth.iq3xxs_matrix(2026, 0, N, K)
    t64 = G.tile(torch.from_numpy(w.reshape(-1)).to(dev), N, K)
    ts = [t64] + [t64.clone() for _ in range(copies - 1)]
    out = {"workload": "prefill GEMM: IQ3_XXS W 12288x6144 (record units staged through LDS, decoded to exact "
                       "fp16 q*(2s+1) MFMA operands, d/4 per block in fp32), X bf16 [M,6144] ~ N(0,1), "
                       f"Y fp32 [M,12288]; {copies} rotated weight copies",
           "peak_TFLOPs": 2500.0}

    def loop(M, X, Y, ws, n):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for r in range(n):
            G.gemm(ts[r % copies], N, 0, K, N, X, out=Y, ws=ws)
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    for M in (512, 2048):
        X = torch.from_numpy(synth.normal(2026, M, M * K).reshape(M, K)).to(dev).to(torch.bfloat16)
        Y = torch.empty(M, N, device=dev)
        ws = torch.zeros(G.lib().gpeed_iq3xxs_gemm_ws_bytes(M, K, N, G.X_BF16), dtype=torch.uint8, device=dev)
        n = max(reps, 2 * copies)
        loop(M, X, Y, ws, copies)
        call_ms = loop(M, X, Y, ws, n)
        G.prof_start(n + 8)  # kernel durations, dispatch-stamped, in a loop of their own
        stamped_ms = loop(M, X, Y, ws, n)
        k_ms = float(G.prof_read(G.PROF_GEMM).astype(np.float64).mean())
        # the unstamped loop again: the better of the two (one loop's spread
        # on rotated weights exceeds the stamps' cost)
        call_ms = min(call_ms, loop(M, X, Y, ws, n))
        fl = 2.0 * M * N * K
        # the GEMM kernel takes at most the stamped duration and at most the
        # whole call (X images + GEMM), whichever is less: the stamps add
        # their own cost, which can exceed the X images' launch
        kb_ms = min(k_ms, call_ms)
        out[f"M{M}"] = {"kernel_us": round(k_ms * 1e3, 2), "call_us": round(call_ms * 1e3, 2),
                        "stamp_overhead_us": round((stamped_ms - call_ms) * 1e3, 2),
                        "TFLOPs_kernel": round(fl / (k_ms * 1e-3) / 1e12, 1),
                        "TFLOPs_call": round(fl / (call_ms * 1e-3) / 1e12, 1),
                        "kernel_bound_us": round(kb_ms * 1e3, 2),
                        "frac_of_bf16_peak": round(fl / (kb_ms * 1e-3) / 1e12 / 2500.0, 4)}
    del ts
    return out


def mla_heads(torch, G, synth, dev, reps, copies=64):
    """MLA per-head absorbed projections of one layer (model.cpp:638-643, 664-665): attn_k_b (64 heads of
    512 rows over 256) and attn_v_b (64 heads of 256 rows over 512), each one launch of
    gpeed_iq3xxs_matvec_heads, against the reference's pattern of 64 matvec_quant calls per tensor.
    `copies` rotated weight sets (2 x 3.2 MB each) keep the reads in HBM."""
    NH, KVL, DK, DV = 64, 512, 256, 256
    shapes = {"attn_k_b": (NH * KVL, DK, KVL), "attn_v_b": (NH * DV, KVL, DV)}
    out = {"workload": "MLA per-head projections, one launch each: attn_k_b 64 heads x (512x256), "
                       "attn_v_b 64 heads x (256x512), fp32 per-head inputs"}
    for i, (name, (rows, k, rph)) in enumerate(shapes.items()):
        base = G.tile(torch.from_numpy(synth.iq3xxs_matrix(2030, i, rows, k).reshape(-1)).to(dev), rows, k)
        ws_list = [base] + [base.clone() for _ in range(copies - 1)]
        x = torch.from_numpy(synth.normal(2030, 10 + i, NH * k).reshape(NH, k)).to(dev)
        y = torch.empty(NH, rph, device=dev)
        ws = G.gemv_workspace(k, rows, 1, 1, dev)
        wsv = G.matvec_workspace(k, rph, dev)
        for c in range(copies):
            G.matvec_heads(ws_list[c], rows, 0, k, rph, x, out=y, ws=ws)
        torch.cuda.synchronize()
        G.prof_start(reps * copies + 8)
        for r in range(reps * copies):
            G.matvec_heads(ws_list[r % copies], rows, 0, k, rph, x, out=y, ws=ws)
        torch.cuda.synchronize()
        one = G.prof_read(G.PROF_GEMV).astype(np.float64) * 1e3
        G.prof_start(reps * NH * 4 + 8)  # the reference's pattern: one matvec per head
        for r in range(reps):
            for h in range(NH):
                G.matvec(ws_list[(r * NH + h) % copies], rows, h * rph, k, rph, x[h], out=y[h], ws=wsv)
        torch.cuda.synchronize()
        per = G.prof_read(G.PROF_GEMV).astype(np.float64) * 1e3
        nbytes = rows * k // 256 * 98
        out[name] = {"one_launch_kernel_us": round(float(np.median(one)), 2),
                     "GBs": round(nbytes / (float(np.median(one)) * 1e-6) / 1e9, 1),
                     "per_head_launches_kernel_us_sum": round(float(np.median(per)) * NH, 2),
                     "packed_bytes": nbytes}
        del ws_list
    return out


def other_formats(torch, G, synth, dev, reps, min_bytes=600e6):
    """Batch-1 products over raw GGUF rows of the other formats of a UD-IQ3_XXS file
    (gpeed_matmul_rows; weights.cpp:167-203 for any decoded type): a 6144x6144 weight per
    format, rotated copies (at least `min_bytes` in all) so the reads come from HBM. Time per
    launch from events around `reps` back-to-back launches."""
    K = N = 6144
    out = {"workload": "matvec over 6144x6144 GGUF rows, one token, fp32 x, per format; prefill512: the "
                       "same weight times X [512, 6144] (k_gemm_rows: exact decode to fp32 tiles, fp32 MFMA)",
           "prefill_peak_TFLOPs": FP32_MFMA_PEAK_TFLOPS}
    X512 = torch.from_numpy(synth.normal(2031, 1, 512 * K).reshape(512, K)).to(dev)
    Y512 = torch.empty(512, N, device=dev)
    names = {8: "Q8_0", 10: "Q2_K", 11: "Q3_K", 14: "Q6_K", 21: "IQ3_S", 22: "IQ2_S", 23: "IQ4_XS", 1: "F16",
             30: "BF16", 18: "IQ3_XXS (raw rows)"}
    x = torch.from_numpy(synth.normal(2031, 0, K)).to(dev)
    y = torch.empty(N, device=dev)
    for dt, name in names.items():
        w = torch.from_numpy(synth.quant_matrix(2031, dt, dt, N, K).reshape(-1)).to(dev)
        nbytes = w.numel()
        copies = max(2, int(min_bytes // nbytes) + 1)
        ws = [w] + [w.clone() for _ in range(copies - 1)]
        for c in range(copies):
            G.matmul_rows(dt, ws[c], N, 0, K, N, x, out=y)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for r in range(reps * copies):
            G.matmul_rows(dt, ws[r % copies], N, 0, K, N, x, out=y)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * copies)
        gbs = nbytes / (us * 1e-6) / 1e9
        G.matmul_rows(dt, w, N, 0, K, N, X512, out=Y512)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            G.matmul_rows(dt, w, N, 0, K, N, X512, out=Y512)
        e1.record()
        torch.cuda.synchronize()
        pus = e0.elapsed_time(e1) * 1e3 / reps
        tf = 2.0 * 512 * N * K / (pus * 1e-6) / 1e12
        out[name] = {"us": round(us, 2), "packed_bytes": nbytes, "GBs": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "prefill512": {"us": round(pus, 1), "TFLOPs": round(tf, 1),
                                    "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}}
        del ws, w
        torch.cuda.empty_cache()
    return out


def moe_probe(torch, G, synth, dev, steps):
    """The routed-expert decode step of the bench (gpeed_iq3xxs_moe_batch: 32 tokens, 64 experts,
    softmax top-8, a shared expert over every token; five launches), `steps` times after three
    warm-up steps, for counter runs. The experts (925 MB) exceed the Infinity Cache, so every
    step streams them from HBM."""
    import ctypes
    E, T, K, HM, IM = 64, 32, 8, 6144, 2048
    log("moe probe: generating 64 experts and a shared expert")
    tens = []
    for i, (r, c) in enumerate(((E * IM, HM), (E * IM, HM), (E * HM, IM))):
        raw = torch.from_numpy(synth.iq3xxs_matrix(2025, i, r, c).reshape(-1)).to(dev)
        tens.append(G.tile(raw, r, c))
        del raw
    sh = []
    for i, (r, c) in enumerate(((IM, HM), (IM, HM), (HM, IM))):
        raw = torch.from_numpy(synth.iq3xxs_matrix(2025, 20 + i, r, c).reshape(-1)).to(dev)
        sh.append(G.tile(raw, r, c))
        del raw
    X = torch.from_numpy(synth.normal(2025, 10, T * HM).reshape(T, HM)).to(dev)
    logits = torch.from_numpy(synth.normal(2025, 11, T * E).reshape(T, E)).to(dev)
    Y = torch.empty(T, HM, device=dev)
    L = G.lib()
    cur = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    nul = ctypes.c_void_p(0)
    ws_b = G.moe_batch_workspace(T, E, K, HM, IM, True, dev)
    args = (vp(logits), T, E, K, 1, nul, ctypes.c_float(1.0), 1, vp(tens[0]), vp(tens[1]), vp(tens[2]),
            vp(sh[0]), vp(sh[1]), vp(sh[2]), HM, IM, vp(X), ctypes.c_float(SWIGLU_LIMIT), vp(Y), nul, nul,
            nul, vp(ws_b), ws_b.numel(), cur)
    for _ in range(3 + steps):
        if L.gpeed_iq3xxs_moe_batch(*args) != 0:
            raise RuntimeError(f"moe: {L.gpeed_last_error().decode(errors='replace')}")
    torch.cuda.synchronize()
    counts = np.diff(G.moe_route(logits, K, 1)[0].cpu().numpy())
    log(f"moe probe done: {int((counts > 0).sum())} experts touched")


def rows_probe(torch, G, synth, dev, reps, min_bytes=600e6):
    """One-token products over raw GGUF rows (k_matmul_rows) of a Q8_0 and a Q6_K 6144x6144
    weight, `reps` launches each over rotated copies (at least `min_bytes`, so the reads come from
    HBM), then five 512-token products (k_gemm_rows) of each, for counter runs."""
    K = N = 6144
    x = torch.from_numpy(synth.normal(2031, 0, K)).to(dev)
    X512 = torch.from_numpy(synth.normal(2031, 1, 512 * K).reshape(512, K)).to(dev)
    y = torch.empty(N, device=dev)
    Y512 = torch.empty(512, N, device=dev)
    for dt in (8, 14):
        w = torch.from_numpy(synth.quant_matrix(2031, dt, dt, N, K).reshape(-1)).to(dev)
        copies = max(2, int(min_bytes // w.numel()) + 1)
        ws = [w] + [w.clone() for _ in range(copies - 1)]
        for r in range(reps):
            G.matmul_rows(dt, ws[r % copies], N, 0, K, N, x, out=y)
        for _ in range(5):
            G.matmul_rows(dt, w, N, 0, K, N, X512, out=Y512)
        torch.cuda.synchronize()
        del ws, w
        torch.cuda.empty_cache()
    log("rows probe done")


def decode_mix(torch, G, synth, dev, reps, copies=4, probe_steps=0):
    """Continuous-batching decode mix: 64 tokens (fp32 X [64, 6144]) through the MLA latent projections
    kv_a 576x6144 and q_a 1536x6144 and the shared-expert FFN (gate, up 12288x6144; down 6144x12288),
    all IQ3_XXS GEMMs, as one gpeed_iq3xxs_mlp_gemm call: X images, the gate+up two-tensor GEMM, the
    SwiGLU images, and one launch holding down and kv_a + q_a (K splits balanced over the CUs).
    `copies` rotated weight sets keep it out of the Infinity Cache. The same products as three
    calls (gemm2 kv_a+q_a, gemm2 gate+up, gemm_swiglu down) are timed beside it. With probe_steps,
    runs that many steps (after three warm-up steps) and returns None (for counter runs)."""
    M, HM, IM = 64, 6144, 12288
    shapes = [("kv_a", 576, HM), ("q_a", 1536, HM), ("gate", IM, HM), ("up", IM, HM), ("down", HM, IM)]
    log("decode mix: generating weights")
    sets = []
    for c in range(copies):
        if c == 0:
            base = {n: G.tile(torch.from_numpy(synth.iq3xxs_matrix(2027, i, r, k).reshape(-1)).to(dev), r, k)
                    for i, (n, r, k) in enumerate(shapes)}
            sets.append(base)
        else:
            sets.append({n: t.clone() for n, t in sets[0].items()})
    X = torch.from_numpy(synth.normal(2027, 10, M * HM).reshape(M, HM)).to(dev)
    out = {n: torch.empty(M, r, device=dev) for n, r, _ in shapes}
    ws_m = G.mlp_gemm_workspace(M, HM, IM, G.X_F32, [576, 1536], dev)

    def step(c):
        W = sets[c % copies]
        G.mlp_gemm(W["gate"], W["up"], W["down"], HM, IM, X, SWIGLU_LIMIT,
                   extra=((W["kv_a"], 576), (W["q_a"], 1536)), out=out["down"],
                   extra_out=[out["kv_a"], out["q_a"]], ws=ws_m)

    # timed through the C ABI with prebuilt arguments (see the dense step)
    import ctypes
    L = G.lib()
    cur = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    eo = (ctypes.c_int * 2)(576, 1536)
    ey = (ctypes.c_void_p * 2)(out["kv_a"].data_ptr(), out["q_a"].data_ptr())
    ew = [(ctypes.c_void_p * 2)(sets[c]["kv_a"].data_ptr(), sets[c]["q_a"].data_ptr()) for c in range(copies)]
    args = [(vp(sets[c]["gate"]), vp(sets[c]["up"]), vp(sets[c]["down"]), HM, IM, vp(X), G.X_F32, M,
             ctypes.c_float(SWIGLU_LIMIT), vp(out["down"]), 2, ew[c], eo, ey, vp(ws_m), ws_m.numel(), cur)
            for c in range(copies)]

    def step_fast(c):
        if L.gpeed_iq3xxs_mlp_gemm(*args[c % copies]) != 0:
            raise RuntimeError(f"decode mix: {L.gpeed_last_error().decode(errors='replace')}")

    # the same products as three calls
    ws3 = {"lat": G.lib().gpeed_iq3xxs_gemm2_ws_bytes(M, HM, 576, 1536, G.X_F32),
           "ffn": G.lib().gpeed_iq3xxs_gemm2_ws_bytes(M, HM, IM, IM, G.X_F32),
           "down": G.lib().gpeed_iq3xxs_gemm_ws_bytes(M, IM, HM, G.X_F32)}
    ws3 = {n: torch.zeros(b, dtype=torch.uint8, device=dev) for n, b in ws3.items()}
    g_u = (torch.empty(M, IM, device=dev), torch.empty(M, IM, device=dev))
    calls3 = []
    for c in range(copies):
        W = sets[c]
        calls3.append([
            (L.gpeed_iq3xxs_gemm2, (vp(W["kv_a"]), 576, 0, 576, vp(W["q_a"]), 1536, 0, 1536, HM, vp(X), G.X_F32, M,
                                    vp(out["kv_a"]), vp(out["q_a"]), vp(ws3["lat"]), ws3["lat"].numel(), cur)),
            (L.gpeed_iq3xxs_gemm2, (vp(W["gate"]), IM, 0, IM, vp(W["up"]), IM, 0, IM, HM, vp(X), G.X_F32, M,
                                    vp(g_u[0]), vp(g_u[1]), vp(ws3["ffn"]), ws3["ffn"].numel(), cur)),
            (L.gpeed_iq3xxs_gemm_swiglu, (vp(W["down"]), HM, 0, IM, HM, vp(g_u[0]), vp(g_u[1]),
                                          ctypes.c_float(SWIGLU_LIMIT), M, vp(out["down"]), vp(ws3["down"]),
                                          ws3["down"].numel(), cur))])

    def step_three(c):
        for f, a in calls3[c % copies]:
            if f(*a) != 0:
                raise RuntimeError(f"decode mix: {L.gpeed_last_error().decode(errors='replace')}")

    for c in range(3):
        step(c)
        step_fast(c)
    torch.cuda.synchronize()
    if probe_steps:
        for c in range(probe_steps):
            step_fast(c)
        torch.cuda.synchronize()
        return None

    def timed(f):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        for c in range(copies):
            f(c)
        a.record()
        for c in range(reps):
            f(c)
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    ms = timed(step_fast)
    ms_three = timed(step_three)
    # GEMM kernel durations (gate+up, down + kv_a/q_a) from dispatch-stamped
    # launches, in a loop of their own (the stamps add to the step)
    G.prof_start(2 * (reps + copies) + 8)
    stamped_ms = timed(step_fast)
    d = G.prof_read(G.PROF_GEMM).astype(np.float64)[-2 * reps:]
    gu_ms, dl_ms = float(np.median(d[0::2])), float(np.median(d[1::2]))
    w_bytes = sum(r * k // 256 * 98 for _, r, k in shapes)
    flops = sum(2.0 * M * r * k for _, r, k in shapes)
    return {"workload": "continuous-batching decode mix: 64 tokens, fp32 X [64,6144], IQ3_XXS kv_a 576x6144, "
                        "q_a 1536x6144, shared expert gate/up 12288x6144 and down 6144x12288, one "
                        "gpeed_iq3xxs_mlp_gemm call: X images, gate+up GEMM (K split 2), SwiGLU images, one "
                        "launch of down (6 K splits of 8 blocks) and kv_a+q_a (3 of 8), 225 workgroups",
            "packed_bytes_per_step": w_bytes, "gflop_per_step": round(flops / 1e9, 2),
            "ms_per_step": round(ms, 4),
            "gemm_kernel_us": {"gate_up": round(gu_ms * 1e3, 2), "down_kv_a_q_a": round(dl_ms * 1e3, 2)},
            "stamp_overhead_us_per_step": round((stamped_ms - ms) * 1e3, 2),
            "three_calls_ms_per_step": round(ms_three, 4),
            "GBps": round(w_bytes / (ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(w_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1),
            "frac_of_fp16_peak": round(flops / (ms * 1e-3) / 1e12 / 2500.0, 4)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary workloads")
    ap.add_argument("--stream-probe", action="store_true",
                    help="gpeed_stream_read over rotated buffers of the GEMV sizes, "
                         "for the read-ceiling profile (run under rocprofv3 --kernel-trace --stats)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run 5 elementwise copies of 256 MiB (counter calibration), then 20 dense steps, and "
                         "exit; meant to run under rocprofv3 --pmc FETCH_SIZE (or WRITE_SIZE)")
    ap.add_argument("--gemm-probe", action="store_true",
                    help="run the prefill GEMM (W 12288x6144, bf16 X [M, 6144]) 20 times and the dense "
                         "decode step 20 times, and exit; meant to run under rocprofv3 --pmc")
    ap.add_argument("--gemm-m", type=int, default=512,
                    help="tokens of the --gemm-probe GEMM (512 runs k_gemm5, 2048 k_gemm6)")
    ap.add_argument("--probe", choices=("moe", "mix", "rows"),
                    help="run 5 elementwise copies of 256 MiB (counter calibration), then 20 steps of the "
                         "routed-expert decode step (moe), the decode mix (mix) or the raw-row products "
                         "(rows), and exit; meant to run under rocprofv3 --pmc")
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
    ws_mlp = G.dense_mlp_workspace(H, I, dev)
    y = torch.empty(H, device=dev)

    def step(c):
        tg, tu, td = copies[c]
        G.dense_mlp(tg, tu, td, H, I, xd, SWIGLU_LIMIT, out=y, ws=ws_mlp)

    # The timed loops call the C ABI with argument tuples built beforehand:
    # a call then costs the host a few microseconds, well under the GPU's
    # step, so the launches queue back to back (the Python wrapper's checks
    # would leave the GPU waiting for the host).
    import ctypes
    fn_mlp = G.lib().gpeed_iq3xxs_dense_mlp
    cur = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = lambda t: ctypes.c_void_p(t.data_ptr())
    call_args = [(vp(tg), vp(tu), vp(td), H, I, vp(xd), ctypes.c_float(SWIGLU_LIMIT), vp(y), vp(ws_mlp),
                  ws_mlp.numel(), cur) for tg, tu, td in copies]

    def step_fast(c):
        if fn_mlp(*call_args[c]) != 0:
            raise RuntimeError(f"dense_mlp: {G.lib().gpeed_last_error().decode(errors='replace')}")

    if args.stream_probe:
        # one streaming read per launch at each GEMV weight size (down; gate+up;
        # the whole step), buffers rotated over the GEMV steps' 694 MB so every
        # byte comes from HBM, not the 256 MB Infinity Cache
        import ctypes
        out = torch.zeros(1024, dtype=torch.int32, device=dev)
        cur = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for nbytes in (W_BYTES // 3, 2 * (W_BYTES // 3), W_BYTES):
            n_bufs = -(-args.copies * W_BYTES // nbytes)  # as many bytes rotated as the GEMV steps rotate
            bufs = [torch.ones(nbytes // 16 * 4, device=dev) for _ in range(n_bufs)]
            for groups in (256, 512, 1024):  # workgroups of 512 threads: 1, 2, 4 per CU
                for _ in range(10):
                    for b in bufs:
                        if G.lib().gpeed_stream_read(ctypes.c_void_p(b.data_ptr()), b.numel() * 4,
                                                     ctypes.c_void_p(out.data_ptr()), groups, cur) != 0:
                            raise RuntimeError("stream_read failed")
                torch.cuda.synchronize()
                log(f"stream probe: {nbytes} B, {groups} workgroups, x {10 * len(bufs)} reads")
            if nbytes == W_BYTES // 3:
                # independent readers of the same bytes: the runtime's
                # device-to-device copy (reads and writes them) and torch's
                # sum reduction (reads them)
                dst = [torch.empty_like(bufs[0]) for _ in range(4)]
                for _ in range(10):
                    for i, b in enumerate(bufs):
                        dst[i % 4].copy_(b)
                for _ in range(10):
                    for b in bufs:
                        torch.sum(b)
                torch.cuda.synchronize()
                log(f"stream probe: {nbytes} B, runtime copy and torch.sum, x {10 * len(bufs)} each")
                del dst
            del bufs
            torch.cuda.empty_cache()
        # the same two readers at 256 MiB (the asymptotic rate)
        big = [torch.ones(64 << 20, device=dev) for _ in range(3)]
        for _ in range(8):
            for i in range(3):
                big[(i + 1) % 3].copy_(big[i])
                torch.sum(big[i])
        torch.cuda.synchronize()
        log("stream probe: 256 MiB runtime copy and torch.sum, x 24 each")
        return

    if args.gemm_probe:
        N_, K_, M_ = 12288, 6144, args.gemm_m
        t64 = G.tile(torch.from_numpy(synth.iq3xxs_matrix(2026, 0, N_, K_).reshape(-1)).to(dev), N_, K_)
        X = torch.from_numpy(synth.normal(2026, M_, M_ * K_).reshape(M_, K_)).to(dev).to(torch.bfloat16)
        Yg = torch.empty(M_, N_, device=dev)
        wsg = torch.zeros(G.lib().gpeed_iq3xxs_gemm_ws_bytes(M_, K_, N_, G.X_BF16), dtype=torch.uint8, device=dev)
        for _ in range(20):
            G.gemm(t64, N_, 0, K_, N_, X, out=Yg, ws=wsg)
        for i in range(20):
            step(i % args.copies)
        torch.cuda.synchronize()
        log("gemm probe done")
        return

    if args.probe:
        src = torch.ones(64 << 20, device=dev)  # 256 MiB fp32
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.add(src, 0.0, out=dst)  # reads 256 MiB, writes 256 MiB
        torch.cuda.synchronize()
        del src, dst, copies, base
        torch.cuda.empty_cache()
        if args.probe == "moe":
            moe_probe(torch, G, synth, dev, 20)
        elif args.probe == "mix":
            decode_mix(torch, G, synth, dev, 20, probe_steps=20)
        else:
            rows_probe(torch, G, synth, dev, 20)
        log(f"{args.probe} probe done")
        return

    if args.traffic_probe:
        src = torch.ones(64 << 20, device=dev)  # 256 MiB fp32
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.add(src, 0.0, out=dst)  # reads 256 MiB, writes 256 MiB
        for i in range(20):
            step(i % args.copies)
        torch.cuda.synchronize()
        log("traffic probe done")
        return

    # Before the warm-up steps, the step runs untimed for about a quarter of
    # a second through the C ABI: on a freshly leased GPU the clocks and the
    # launch path take that long to settle (5 warm-up steps left a cold box's
    # 20-step line ~11% below its steady state).
    log("settle")
    t_end = time.perf_counter() + 0.25
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(64):
            step_fast(i % args.copies)
            i += 1
        torch.cuda.synchronize()
    log("warmup")
    for i in range(args.warmup):
        step(i % args.copies)
    torch.cuda.synchronize()
    step(0)
    torch.cuda.synchronize()
    y_gpu = y.cpu().numpy().copy()

    log("timed")
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for i in range(args.steps):
        step_fast(i % args.copies)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    value = W_BYTES / (ms * 1e-3) / 1e9

    # Kernel timing: the step's two GEMV launches for every copy in turn,
    # captured in one HIP graph so consecutive launches leave no host gaps;
    # one event pair on the launch stream brackets the replays. Per-launch
    # duration = elapsed / launches (inter-launch gaps included, so it errs
    # low).
    log("kernel timing")

    def time_per_step(fn):
        """ms per step: the faster of HIP graph replays of all copies in turn
        and back-to-back eager steps (graph kernel nodes carry their own
        per-node cost on this stack; neither leaves host gaps)."""
        reps = max(4, args.steps // args.copies)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(reps * args.copies):
            step_fast(i % args.copies)
        e1.record()
        torch.cuda.synchronize()
        eager_ms = e0.elapsed_time(e1) / (reps * args.copies)
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=side):
                    for c in range(args.copies):
                        fn(c)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
            graph_ms = e0.elapsed_time(e1) / (reps * args.copies)
        except Exception as exc:  # capture unsupported for this launch
            log(f"graph capture unavailable ({type(exc).__name__}): eager timing")
            return eager_ms, "eager"
        return (graph_ms, "graph") if graph_ms < eager_ms else (eager_ms, "eager")

    pair_ms, pair_timing = time_per_step(step)
    # dispatch-stamped events split the pair per kind (they add a little each)
    G.prof_start(2 * 64 + 8)
    for i in range(64):
        step(i % args.copies)
    dur = G.prof_read(G.PROF_GEMV).astype(np.float64)  # launch order: gate+up, down, ...
    per_kind = {"gate+up": dur[0::2], "down": dur[1::2]}
    # algorithmic bytes: packed W + x + the SwiGLU activation written and read
    # (I/256 blocks of 1024 B images + 16 B unscales) + y
    act64 = (I // 256) * (1024 + 16)
    launch_bytes = {"gate+up": 2 * (W_BYTES // 3) + H * 4 + act64,
                    "down": W_BYTES // 3 + act64 + H * 4}
    pair_bytes = launch_bytes["gate+up"] + launch_bytes["down"]
    achieved = pair_bytes / (pair_ms * 1e-3) / 1e9
    kinds = {k: {"dispatch_event_us": round(float(v.mean()) * 1e3, 3), "algorithmic_bytes": launch_bytes[k]}
             for k, v in per_kind.items()}
    down_us = float(per_kind["down"].mean()) * 1e3

    # the 6144x12288 shape alone: matvec_quant of the down weights on an
    # fp32 vector (gpeed_iq3xxs_matvec, one launch), rotated copies
    xdn = torch.from_numpy(synth.normal(2024, 101, I)).to(dev)
    ws_mv = G.matvec_workspace(I, H, dev)
    fn_mv = G.lib().gpeed_iq3xxs_matvec
    mv_args = [(vp(c[2]), H, 0, I, H, vp(xdn), vp(y), vp(ws_mv), ws_mv.numel(), cur) for c in copies]
    reps = max(8, args.steps // args.copies) * args.copies
    for i in range(2 * args.copies):
        fn_mv(*mv_args[i % args.copies])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(reps):
        if fn_mv(*mv_args[i % args.copies]) != 0:
            raise RuntimeError(G.lib().gpeed_last_error().decode(errors="replace"))
    e1.record()
    torch.cuda.synchronize()
    mv_us = e0.elapsed_time(e1) / reps * 1e3
    G.prof_start(64 + 8)
    for i in range(64):
        fn_mv(*mv_args[i % args.copies])
    mv_stamped_us = float(G.prof_read(G.PROF_GEMV).astype(np.float64).mean()) * 1e3
    mv_bytes = W_BYTES // 3 + I * 4 + H * 4
    mv_gbs = mv_bytes / (mv_us * 1e-6) / 1e9

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
        "dtype": "iq3_xxs",
        "data": "synthetic (seeded IQ3_XXS blocks, x ~ N(0,1)); weights resident in HBM, "
                f"{args.copies} rotated copies ({args.copies * W_BYTES / 1e6:.0f} MB)",
        "config": {"workload": "dense-layer decode at batch 1: IQ3_XXS gate/up 12288x6144, "
                               "down 6144x12288 (gate+up GEMV writing the SwiGLU activation, down GEMV)",
                   "packed_weight_bytes_per_step": W_BYTES, "batch": 1,
                   "arithmetic": "iq3_xxs weights decoded to exact fp16, fp32 activations as fp16 hi+lo, "
                                 "f16 MFMA with fp32 accumulation"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_per": "gate+up + down launch pair, bytes (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                                    "copy-calibrated)",
                     "kernel": "k_gemv_t64", "avg_launch_us": round(pair_ms * 1e3 / 2, 3),
                     "pair_us": round(pair_ms * 1e3, 3), "timing": pair_timing,
                     "pair_algorithmic_bytes": pair_bytes, "launch_kinds": kinds,
                     "down": {"shape": "6144x12288", "in_step_launch_us": round(down_us, 3),
                              "entry": "gpeed_iq3xxs_matvec (fp32 x, one launch), rotated copies",
                              "launch_us": round(mv_us, 3), "dispatch_event_us": round(mv_stamped_us, 3),
                              "algorithmic_bytes": mv_bytes, "achieved": round(mv_gbs, 1),
                              "frac": round(mv_gbs / HBM_PEAK_GBS, 4)}},
    }
    if not args.no_extra:
        del copies, base
        torch.cuda.empty_cache()
        pre, dec = moe_decode(torch, G, synth, dev, max(30, args.steps // 5), 0.3)
        rec["extra"] = {"moe_decode": dec, "moe_prefill": pre}
        torch.cuda.empty_cache()
        rec["extra"]["router_product"] = router_product(torch, G, synth, dev, 50)
        rec["extra"]["prefill_gemm"] = prefill_gemm(torch, G, synth, dev, 20)
        torch.cuda.empty_cache()
        rec["extra"]["decode_mix"] = decode_mix(torch, G, synth, dev, 20)
        torch.cuda.empty_cache()
        rec["extra"]["mla_heads"] = mla_heads(torch, G, synth, dev, 20)
        torch.cuda.empty_cache()
        rec["extra"]["other_formats"] = other_formats(torch, G, synth, dev, 5)
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

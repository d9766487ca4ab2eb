"""gpeed_amd - MI355X (gfx950) IQ3_XXS dequantize-and-multiply path.

Python host layer over the C ABI in include/gpeed_iq3.h (libgpeed_iq3.so,
built in-tree by ``gpeed_amd.build``). Device memory and streams come from
PyTorch; every computation runs in the HIP library. There is no CPU fallback:
if the library is missing or no GPU is visible, the calls raise.

The WeightStore class mirrors the reference's WeightStore::matvec_quant /
matmul_quant contract (cpp/core/include/glm5/weights.h:41-48): same argument
meaning (tensor name, first row, in_dim, out_dim), same errors (missing
tensor, row not block aligned) raised as RuntimeError.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgpeed_iq3.so")

GPEED_OK = 0
ERRORS = {
    -1: "invalid argument",
    -2: "element count not a multiple of block size",
    -3: "row not block aligned",
    -4: "dtype not implemented on the GPU path",
    -5: "HIP error",
    -6: "T64 operand off a 64-row tile boundary",
    -7: "workspace missing or too small",
    -8: "no HIP device",
    -9: "a kernel flagged its workspace",
}
WS_TICKET, WS_TIMEOUT, WS_BUCKETS = 1, 2, 4
DTYPE_IQ3_XXS = 18
# ggml type ids of the formats a UD-IQ3_XXS file holds (common.h:10-43)
DTYPE_F32, DTYPE_F16, DTYPE_Q8_0, DTYPE_Q2_K, DTYPE_Q3_K, DTYPE_Q6_K = 0, 1, 8, 10, 11, 14
DTYPE_IQ3_S, DTYPE_IQ2_S, DTYPE_IQ4_XS, DTYPE_BF16 = 21, 22, 23, 30
DTYPES_DECODED = (DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_Q8_0, DTYPE_Q2_K, DTYPE_Q3_K, DTYPE_Q6_K, DTYPE_IQ3_XXS,
                  DTYPE_IQ3_S, DTYPE_IQ2_S, DTYPE_IQ4_XS)
QK = 256
BLOCK_BYTES = 98

_lib = None


class GpeedError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (status {code}: {ERRORS.get(code, 'unknown')})")
        self.code = code


def lib():
    """The loaded libgpeed_iq3.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run gpeed_amd.build.build() first")
        L = C.CDLL(LIB_PATH)
        vp, u64, i64, i32, sz = C.c_void_p, C.c_uint64, C.c_int64, C.c_int, C.c_size_t
        sig = {
            "gpeed_device_count": ([], i32),
            "gpeed_device_name": ([i32, C.c_char_p, sz], i32),
            "gpeed_add_f32": ([vp, vp, vp, i32], i32),
            "gpeed_init": ([], i32),
            "gpeed_last_error": ([], C.c_char_p),
            "gpeed_iq3xxs_row_bytes": ([i64], sz),
            "gpeed_iq3xxs_t64_bytes": ([u64, i64], sz),
            "gpeed_dequantize": ([i32, vp, vp, u64, vp], i32),
            "gpeed_dtype_block_size": ([i32], i32),
            "gpeed_dtype_row_bytes": ([i32, u64], sz),
            "gpeed_matmul_rows": ([i32, vp, u64, u64, i32, i32, vp, i32, vp, vp], i32),
            "gpeed_codebook": ([i32, vp, sz], i32),
            "gpeed_t64_grid_table": ([vp, sz], i32),
            "gpeed_t64_aux_word": ([C.c_uint32], C.c_uint32),
            "gpeed_iq3xxs_tile": ([vp, u64, i64, vp, vp], i32),
            "gpeed_iq3xxs_untile": ([vp, u64, i64, vp, vp], i32),
            "gpeed_iq3xxs_matvec_ws_bytes": ([i64, i64], sz),
            "gpeed_iq3xxs_matmul_ws_bytes": ([i64, i64, i32], sz),
            "gpeed_iq3xxs_matmul_ws_bytes_for": ([i64, i64, i32, i32], sz),
            "gpeed_iq3xxs_matvec": ([vp, u64, u64, i32, i32, vp, vp, vp, sz, vp], i32),
            "gpeed_iq3xxs_matmul": ([vp, u64, u64, i32, i32, vp, i32, vp, vp, sz, vp], i32),
            "gpeed_iq3xxs_matvec_raw": ([vp, u64, u64, i32, i32, vp, vp, vp], i32),
            "gpeed_iq3xxs_matvec_noalloc": ([vp, u64, u64, i32, i32, vp, vp, vp], i32),
            "gpeed_iq3xxs_matvec_noalloc_status": ([vp], i32),
            "gpeed_iq3xxs_matvec_noalloc_poke": ([sz, C.c_uint32], i32),
            "gpeed_iq3xxs_act_bytes": ([i64, i32], sz),
            "gpeed_iq3xxs_prep_act": ([vp, i64, i32, vp, sz, vp], i32),
            "gpeed_iq3xxs_prep_swiglu": ([vp, vp, i64, i32, C.c_float, vp, sz, vp], i32),
            "gpeed_iq3xxs_gemv_ws_bytes": ([i32, i64, i64, i32], sz),
            "gpeed_iq3xxs_gemv_act": ([vp, u64, u64, i32, i32, vp, i32, vp, vp, sz, vp], i32),
            "gpeed_iq3xxs_gemv2_act": ([vp, vp, u64, u64, i32, i32, vp, i32, vp, vp, vp, sz, vp], i32),
            "gpeed_iq3xxs_gemv_x": ([vp, u64, u64, i32, i32, vp, vp, vp, sz, vp], i32),
            "gpeed_iq3xxs_gemv2_x": ([vp, vp, u64, u64, i32, i32, vp, vp, vp, vp, sz, vp], i32),
            "gpeed_iq3xxs_gemv_swiglu": ([vp, u64, u64, i32, i32, vp, vp, C.c_float, vp, vp, sz, vp], i32),
            "gpeed_iq3xxs_matvec_heads": ([vp, u64, u64, i32, i32, i32, vp, vp, vp, sz, vp], i32),
            "gpeed_iq3xxs_dense_mlp_ws_bytes": ([i64, i64], sz),
            "gpeed_iq3xxs_dense_mlp": ([vp, vp, vp, i32, i32, vp, C.c_float, vp, vp, sz, vp], i32),
            "gpeed_iq3xxs_gemm_ws_bytes": ([i64, i64, i64, i32], sz),
            "gpeed_iq3xxs_gemm_swiglu": ([vp, u64, u64, i32, i32, vp, vp, C.c_float, i32, vp, vp, sz, vp], i32),
            "gpeed_iq3xxs_gemm": ([vp, u64, u64, i32, i32, vp, i32, i32, vp, vp, sz, vp], i32),
            "gpeed_iq3xxs_gemm2_ws_bytes": ([i64, i64, i64, i64, i32], sz),
            "gpeed_iq3xxs_gemm2": ([vp, u64, u64, i32, vp, u64, u64, i32, i32, vp, i32, i32, vp, vp, vp, sz, vp],
                                   i32),
            "gpeed_iq3xxs_mlp_gemm_ws_bytes": ([i64, i64, i64, i32, i32, vp], sz),
            "gpeed_iq3xxs_mlp_gemm": ([vp, vp, vp, i32, i32, vp, i32, i32, C.c_float, vp, i32, vp, vp, vp, vp, sz,
                                       vp], i32),
            "gpeed_stream_read": ([vp, sz, vp, sz, vp], i32),
            "gpeed_prof_start": ([i32], i32),
            "gpeed_prof_read": ([i32, vp, i32, vp], i32),
            "gpeed_ws_status": ([vp, vp], i32),
            "gpeed_ws_init": ([vp, sz, vp], i32),
            "gpeed_moe_check_buckets": ([vp, vp, i32, i32, i32], i32),
            "gpeed_iq3xxs_matmul_gemm_min_tok": ([], i32),
            "gpeed_moe_route_ws_bytes": ([i32, i32, i32], sz),
            "gpeed_moe_route": ([vp, i32, i32, i32, i32, vp, C.c_float, i32, vp, vp, vp, vp, vp, sz, vp], i32),
            "gpeed_iq3xxs_moe_ws_bytes": ([i32, i32, i32, i32, i32], sz),
            "gpeed_iq3xxs_moe_experts": ([vp, vp, vp, i32, i32, i32, vp, i32, i32, vp, vp, vp, C.c_float, vp, vp,
                                          sz, vp], i32),
            "gpeed_iq3xxs_moe_batch_ws_bytes": ([i32, i32, i32, i32, i32, i32], sz),
            "gpeed_iq3xxs_moe_batch": ([vp, i32, i32, i32, i32, vp, C.c_float, i32, vp, vp, vp, vp, vp, vp, i32, i32,
                                        vp, C.c_float, vp, vp, vp, vp, vp, sz, vp], i32),
        }
        for name, (args, res) in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def _check(rc: int, what: str):
    if rc != GPEED_OK:
        msg = lib().gpeed_last_error().decode(errors="replace")
        raise GpeedError(rc, f"{what}: {msg}")


def _torch():
    import torch

    return torch


def _stream(stream=None):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def _ptr(t) -> C.c_void_p:
    return C.c_void_p(t.data_ptr())


def _require_cuda(*ts):
    for t in ts:
        if not t.is_cuda:
            raise ValueError("gpeed_amd operates on device tensors (tensor.is_cuda is False)")
        if not t.is_contiguous():
            raise ValueError("gpeed_amd expects contiguous tensors")


def init():
    _check(lib().gpeed_init(), "gpeed_init")


PROF_GEMV, PROF_GROUPED, PROF_GEMM = 0, 1, 2


def prof_start(max_launches: int = 4096):
    """Time every following hot-kernel launch (kernel execution only)."""
    _check(lib().gpeed_prof_start(max_launches), "prof_start")


def prof_read(kind: int) -> np.ndarray:
    """Stop timing; per-launch durations (ms) of one kernel kind, launch order."""
    n = C.c_int(0)
    _check(lib().gpeed_prof_read(kind, None, 0, C.byref(n)), "prof_read")
    out = np.zeros(max(n.value, 1), np.float32)
    _check(lib().gpeed_prof_read(kind, out.ctypes.data, n.value, C.byref(n)), "prof_read")
    return out[:n.value]


def device_count() -> int:
    return lib().gpeed_device_count()


def device_name(index: int = 0) -> str:
    buf = C.create_string_buffer(256)
    _check(lib().gpeed_device_name(index, buf, 256), "gpeed_device_name")
    return buf.value.decode()


def add_f32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Host-array a + b through the device (the reference's cuda_add smoke test)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty_like(a)
    _check(lib().gpeed_add_f32(a.ctypes.data, b.ctypes.data, out.ctypes.data, a.size), "gpeed_add_f32")
    return out


def stream_read(buf, groups: int, out=None, stream=None):
    """Reads the bytes of device tensor `buf` once (gpeed_stream_read: `groups`
    workgroups, each a contiguous share) and returns the int32 per-workgroup
    XOR folds. A measurement aid: its duration is a plain streaming read of
    buf.nbytes bytes."""
    torch = _torch()
    _require_cuda(buf)
    if out is None:
        out = torch.empty(groups, dtype=torch.int32, device=buf.device)
    _check(lib().gpeed_stream_read(_ptr(buf), buf.numel() * buf.element_size(), _ptr(out), groups,
                                   _stream(stream)), "gpeed_stream_read")
    return out


def row_bytes(in_dim: int) -> int:
    return lib().gpeed_iq3xxs_row_bytes(in_dim)


def t64_bytes(n_rows: int, in_dim: int) -> int:
    return lib().gpeed_iq3xxs_t64_bytes(n_rows, in_dim)


def dtype_block_size(dtype: int) -> int:
    """dtype_block_size (quant.cpp:52-81) for the decoded types, else 0."""
    return lib().gpeed_dtype_block_size(dtype)


def dtype_row_bytes(dtype: int, n: int) -> int:
    """dtype_row_bytes (quant.cpp:119-126) for the decoded types, else 0."""
    return lib().gpeed_dtype_row_bytes(dtype, n)


def codebook(dtype: int) -> np.ndarray:
    """The expanded grid the kernels use for IQ2_S, IQ3_S or IQ3_XXS (uint64 per entry)."""
    n = {DTYPE_IQ2_S: 1024, DTYPE_IQ3_S: 512, DTYPE_IQ3_XXS: 256}[dtype]
    out = np.zeros(n, np.uint64)
    _check(lib().gpeed_codebook(dtype, out.ctypes.data, n), "codebook")
    return out


def dequantize(raw, n: int, out=None, dtype: int = DTYPE_IQ3_XXS, stream=None):
    """fp32 [n] from GGUF bytes of any decoded type on the device (bit-exact
    with quant.cpp:165-563)."""
    torch = _torch()
    _require_cuda(raw)
    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=raw.device)
    _check(lib().gpeed_dequantize(dtype, _ptr(raw), _ptr(out), n, _stream(stream)), "dequantize")
    return out


def tile(raw, n_rows: int, in_dim: int, out=None, stream=None):
    """T64 copy of [n_rows, in_dim] GGUF rows held on the device."""
    torch = _torch()
    _require_cuda(raw)
    if out is None:
        out = torch.empty(t64_bytes(n_rows, in_dim), dtype=torch.uint8, device=raw.device)
    _check(lib().gpeed_iq3xxs_tile(_ptr(raw), n_rows, in_dim, _ptr(out), _stream(stream)), "tile")
    return out


def untile(t64, n_rows: int, in_dim: int, out=None, stream=None):
    torch = _torch()
    _require_cuda(t64)
    if out is None:
        out = torch.empty(n_rows * row_bytes(in_dim), dtype=torch.uint8, device=t64.device)
    _check(lib().gpeed_iq3xxs_untile(_ptr(t64), n_rows, in_dim, _ptr(out), _stream(stream)), "untile")
    return out


def _zeros(nbytes: int, device):
    """Initialised workspace (gpeed_ws_init); a size the library rejects (0)
    still gets a small buffer so that the call itself reports why."""
    torch = _torch()
    ws = torch.empty((max(nbytes, 256) + 255) // 256 * 256, dtype=torch.uint8, device=device)
    ws_init(ws)
    return ws


def ws_init(ws, stream=None):
    """Zero-fill a workspace with the library's fill kernel (gpeed_ws_init)."""
    _require_cuda(ws)
    _check(lib().gpeed_ws_init(_ptr(ws), ws.numel() * ws.element_size(), _stream(stream)), "ws_init")
    return ws


def ws_status(ws, stream=None):
    """Waits for the stream; raises GpeedError (status -9) if a kernel flagged
    the workspace since the last check (the flags are cleared)."""
    _require_cuda(ws)
    _check(lib().gpeed_ws_status(_ptr(ws), _stream(stream)), "ws_status")


def moe_check_buckets(eptr: np.ndarray, tok: np.ndarray, n_exp: int, n_tok: int, top_k: int):
    """Checks host expert buckets against the router's invariants (raises GpeedError)."""
    e = np.ascontiguousarray(eptr, np.int32)
    t = np.ascontiguousarray(tok, np.int32)
    if e.size < n_exp + 1 or t.size < n_tok * top_k:
        raise ValueError("moe_check_buckets: arrays shorter than n_exp + 1 / n_tok * top_k")
    _check(lib().gpeed_moe_check_buckets(e.ctypes.data, t.ctypes.data, n_exp, n_tok, top_k), "moe_check_buckets")


def matmul_gemm_min_tok() -> int:
    """Token count from which matmul runs the prefill GEMM instead of GEMV passes."""
    return lib().gpeed_iq3xxs_matmul_gemm_min_tok()


def matmul_workspace(in_dim: int, out_dim: int, n_tok: int = 1, device="cuda"):
    """Initialised workspace for matvec / matmul of up to n_tok tokens (one per stream)."""
    return _zeros(lib().gpeed_iq3xxs_matmul_ws_bytes(in_dim, out_dim, n_tok), device)


def matvec_workspace(in_dim: int, out_dim: int, device="cuda"):
    return matmul_workspace(in_dim, out_dim, 1, device)


def matvec(w_t64, n_rows: int, row0: int, in_dim: int, out_dim: int, x, out=None, ws=None, stream=None):
    """dst = W[row0:row0+out_dim] @ x from a T64 tensor (batch 1, fp32)."""
    torch = _torch()
    _require_cuda(w_t64, x)
    if out is None:
        out = torch.empty(out_dim, dtype=torch.float32, device=x.device)
    if ws is None:
        ws = matvec_workspace(in_dim, out_dim, x.device)
    _check(lib().gpeed_iq3xxs_matvec(_ptr(w_t64), n_rows, row0, in_dim, out_dim, _ptr(x), _ptr(out),
                                     _ptr(ws), ws.numel(), _stream(stream)), "matvec")
    return out


def matmul(w_t64, n_rows: int, row0: int, in_dim: int, out_dim: int, X, out=None, ws=None, stream=None):
    """Y[t] = W[row0:row0+out_dim] @ X[t] for X [n_tok, in_dim] fp32; Y [n_tok, out_dim].

    GEMV passes of up to 8 tokens below matmul_gemm_min_tok() tokens, the
    prefill GEMM with fp32 X from there on."""
    torch = _torch()
    _require_cuda(w_t64, X)
    n_tok = X.shape[0] if X.dim() == 2 else 1
    if out is None:
        out = torch.empty(n_tok, out_dim, dtype=torch.float32, device=X.device)
    if ws is None:
        ws = matmul_workspace(in_dim, out_dim, n_tok, X.device)
    _check(lib().gpeed_iq3xxs_matmul(_ptr(w_t64), n_rows, row0, in_dim, out_dim, _ptr(X), n_tok, _ptr(out),
                                     _ptr(ws), ws.numel(), _stream(stream)), "matmul")
    return out


X_F32, X_BF16 = 0, 1


def gemm(w_t64, n_rows: int, row0: int, in_dim: int, out_dim: int, X, out=None, ws=None, stream=None):
    """Prefill GEMM: Y [n_tok, out_dim] = X [n_tok, in_dim] (fp32 or bf16) @ W[row0:row0+out_dim]^T."""
    torch = _torch()
    _require_cuda(w_t64, X)
    n_tok = X.shape[0]
    xd = X_BF16 if X.dtype == torch.bfloat16 else X_F32
    if xd == X_F32 and X.dtype != torch.float32:
        raise ValueError("gemm: X must be float32 or bfloat16")
    if out is None:
        out = torch.empty(n_tok, out_dim, dtype=torch.float32, device=X.device)
    if ws is None:
        ws = _zeros(lib().gpeed_iq3xxs_gemm_ws_bytes(n_tok, in_dim, out_dim, xd), X.device)
    _check(lib().gpeed_iq3xxs_gemm(_ptr(w_t64), n_rows, row0, in_dim, out_dim, _ptr(X), xd, n_tok, _ptr(out),
                                   _ptr(ws), ws.numel(), _stream(stream)), "gemm")
    return out


def gemm2(w_a, n_rows_a: int, row0_a: int, out_a: int, w_b, n_rows_b: int, row0_b: int, out_b: int, in_dim: int, X,
          out_a_t=None, out_b_t=None, ws=None, stream=None):
    """Two prefill GEMMs on one X in one launch: (Y_a [n_tok, out_a], Y_b [n_tok, out_b])."""
    torch = _torch()
    _require_cuda(w_a, w_b, X)
    n_tok = X.shape[0]
    xd = X_BF16 if X.dtype == torch.bfloat16 else X_F32
    if xd == X_F32 and X.dtype != torch.float32:
        raise ValueError("gemm2: X must be float32 or bfloat16")
    if out_a_t is None:
        out_a_t = torch.empty(n_tok, out_a, dtype=torch.float32, device=X.device)
    if out_b_t is None:
        out_b_t = torch.empty(n_tok, out_b, dtype=torch.float32, device=X.device)
    if ws is None:
        ws = _zeros(lib().gpeed_iq3xxs_gemm2_ws_bytes(n_tok, in_dim, out_a, out_b, xd), X.device)
    _check(lib().gpeed_iq3xxs_gemm2(_ptr(w_a), n_rows_a, row0_a, out_a, _ptr(w_b), n_rows_b, row0_b, out_b, in_dim,
                                    _ptr(X), xd, n_tok, _ptr(out_a_t), _ptr(out_b_t), _ptr(ws), ws.numel(),
                                    _stream(stream)), "gemm2")
    return out_a_t, out_b_t


def gemm_swiglu(w_t64, n_rows: int, row0: int, in_dim: int, out_dim: int, G, U, limit: float = 10.0, out=None,
                ws=None, stream=None):
    """Y [n_tok, out_dim] = SwiGLU(G, U) [n_tok, in_dim] (fp32) @ W[row0:row0+out_dim]^T, one GEMM."""
    torch = _torch()
    _require_cuda(w_t64, G, U)
    if G.dtype != torch.float32 or U.dtype != torch.float32 or G.shape != U.shape:
        raise ValueError("gemm_swiglu: G and U must be float32 of one shape")
    n_tok = G.shape[0]
    if out is None:
        out = torch.empty(n_tok, out_dim, dtype=torch.float32, device=G.device)
    if ws is None:
        ws = _zeros(lib().gpeed_iq3xxs_gemm_ws_bytes(n_tok, in_dim, out_dim, X_F32), G.device)
    _check(lib().gpeed_iq3xxs_gemm_swiglu(_ptr(w_t64), n_rows, row0, in_dim, out_dim, _ptr(G), _ptr(U), limit, n_tok,
                                          _ptr(out), _ptr(ws), ws.numel(), _stream(stream)), "gemm_swiglu")
    return out


def mlp_gemm_workspace(n_tok: int, hidden: int, inter: int, x_dtype: int = None, extra_out=(), device="cuda"):
    """Workspace of mlp_gemm (zeroed: its header holds the error word)."""
    xd = X_F32 if x_dtype is None else x_dtype
    eo = (C.c_int * max(1, len(extra_out)))(*extra_out)
    n = lib().gpeed_iq3xxs_mlp_gemm_ws_bytes(n_tok, hidden, inter, xd, len(extra_out), eo)
    if n == 0:
        raise ValueError("mlp_gemm: unsupported sizes")
    return _zeros(n, device)


def mlp_gemm(w_gate, w_up, w_down, hidden: int, inter: int, X, limit: float = 10.0, extra=(), out=None,
             extra_out=None, ws=None, stream=None):
    """dense_mlp_batch as GEMMs: Y [n_tok, hidden] = down(SwiGLU(gate X, up X)) for whole T64 tensors,
    plus the products of up to two more whole T64 tensors of the same X, extra = ((w, out_dim), ...),
    computed in the down launch. Returns (Y, [Y_extra ...])."""
    torch = _torch()
    _require_cuda(w_gate, w_up, w_down, X)
    n_tok = X.shape[0]
    xd = X_BF16 if X.dtype == torch.bfloat16 else X_F32
    if xd == X_F32 and X.dtype != torch.float32:
        raise ValueError("mlp_gemm: X must be float32 or bfloat16")
    if len(extra) > 2:
        raise ValueError("mlp_gemm: at most two extra tensors")
    if out is None:
        out = torch.empty(n_tok, hidden, dtype=torch.float32, device=X.device)
    if extra_out is None:
        extra_out = [torch.empty(n_tok, r, dtype=torch.float32, device=X.device) for _, r in extra]
    dims = [r for _, r in extra]
    if ws is None:
        ws = mlp_gemm_workspace(n_tok, hidden, inter, xd, dims, X.device)
    k = max(1, len(extra))
    ew = (C.c_void_p * k)(*[_ptr(w) for w, _ in extra])
    eo = (C.c_int * k)(*dims)
    ey = (C.c_void_p * k)(*[_ptr(y) for y in extra_out])
    _check(lib().gpeed_iq3xxs_mlp_gemm(_ptr(w_gate), _ptr(w_up), _ptr(w_down), hidden, inter, _ptr(X), xd, n_tok,
                                       limit, _ptr(out), len(extra), ew, eo, ey, _ptr(ws), ws.numel(),
                                       _stream(stream)), "mlp_gemm")
    return out, extra_out


def act_buffer(in_dim: int, n_tok: int = 1, device="cuda"):
    """Device buffer for n_tok prepared activations (fp16 hi/lo operand + scales)."""
    torch = _torch()
    return torch.empty(lib().gpeed_iq3xxs_act_bytes(in_dim, n_tok), dtype=torch.uint8, device=device)


def gemv_workspace(in_dim: int, out_dim: int, n_tok: int = 1, n_tensors: int = 1, device="cuda"):
    """Zero-filled GEMV workspace (shared-tile partials and tickets), one per stream."""
    return _zeros(lib().gpeed_iq3xxs_gemv_ws_bytes(n_tensors, in_dim, out_dim, n_tok), device)


def prep_act(x, act, stream=None):
    """Prepare x ([in_dim] or [n_tok, in_dim], fp32) into act."""
    _require_cuda(x, act)
    n_tok = x.shape[0] if x.dim() == 2 else 1
    _check(lib().gpeed_iq3xxs_prep_act(_ptr(x), x.shape[-1], n_tok, _ptr(act), act.numel(), _stream(stream)),
           "prep_act")
    return act


def prep_swiglu(g, u, act, limit: float = 10.0, stream=None):
    _require_cuda(g, u, act)
    n_tok = g.shape[0] if g.dim() == 2 else 1
    _check(lib().gpeed_iq3xxs_prep_swiglu(_ptr(g), _ptr(u), g.shape[-1], n_tok, limit, _ptr(act), act.numel(),
                                          _stream(stream)), "prep_swiglu")
    return act


def gemv_act(w_t64, n_rows: int, row0: int, in_dim: int, out_dim: int, act, n_tok: int = 1, out=None,
             ws=None, stream=None):
    """dst[t] = W[row0:row0+out_dim] @ x_t for the n_tok prepared vectors in act."""
    torch = _torch()
    _require_cuda(w_t64, act)
    if out is None:
        out = torch.empty(n_tok, out_dim, dtype=torch.float32, device=act.device)
    if ws is None:
        ws = gemv_workspace(in_dim, out_dim, n_tok, 1, act.device)
    _check(lib().gpeed_iq3xxs_gemv_act(_ptr(w_t64), n_rows, row0, in_dim, out_dim, _ptr(act), n_tok, _ptr(out),
                                       _ptr(ws), ws.numel(), _stream(stream)), "gemv_act")
    return out


def gemv_x(w_t64, n_rows: int, row0: int, in_dim: int, out_dim: int, x, out=None, ws=None, stream=None):
    """y = W[row0:row0+out_dim] @ x for one fp32 vector, preparation fused (one launch)."""
    torch = _torch()
    _require_cuda(w_t64, x)
    if out is None:
        out = torch.empty(out_dim, dtype=torch.float32, device=x.device)
    if ws is None:
        ws = gemv_workspace(in_dim, out_dim, 1, 1, x.device)
    _check(lib().gpeed_iq3xxs_gemv_x(_ptr(w_t64), n_rows, row0, in_dim, out_dim, _ptr(x), _ptr(out), _ptr(ws),
                                     ws.numel(), _stream(stream)), "gemv_x")
    return out


def gemv2_x(w_a, w_b, n_rows: int, row0: int, in_dim: int, out_dim: int, x, out_a=None, out_b=None, ws=None,
            stream=None):
    """Two same-shape tensors against one fp32 vector, preparation fused (one launch)."""
    torch = _torch()
    _require_cuda(w_a, w_b, x)
    if out_a is None:
        out_a = torch.empty(out_dim, dtype=torch.float32, device=x.device)
    if out_b is None:
        out_b = torch.empty(out_dim, dtype=torch.float32, device=x.device)
    if ws is None:
        ws = gemv_workspace(in_dim, out_dim, 1, 2, x.device)
    _check(lib().gpeed_iq3xxs_gemv2_x(_ptr(w_a), _ptr(w_b), n_rows, row0, in_dim, out_dim, _ptr(x), _ptr(out_a),
                                      _ptr(out_b), _ptr(ws), ws.numel(), _stream(stream)), "gemv2_x")
    return out_a, out_b


def matvec_heads(w_t64, n_rows: int, row0: int, in_dim: int, rows_per_head: int, x, out=None, ws=None,
                 stream=None):
    """Per-head projections in one launch: x [n_heads, in_dim] -> [n_heads, rows_per_head], head h
    using rows row0 + h*rows_per_head .. (attn_k_b / attn_v_b, model.cpp:638-643, 664-665)."""
    torch = _torch()
    _require_cuda(w_t64, x)
    n_heads = x.shape[0]
    if out is None:
        out = torch.empty(n_heads, rows_per_head, dtype=torch.float32, device=x.device)
    if ws is None:
        ws = gemv_workspace(in_dim, n_heads * rows_per_head, 1, 1, x.device)
    _check(lib().gpeed_iq3xxs_matvec_heads(_ptr(w_t64), n_rows, row0, in_dim, rows_per_head, n_heads, _ptr(x),
                                           _ptr(out), _ptr(ws), ws.numel(), _stream(stream)), "matvec_heads")
    return out


def dense_mlp_workspace(hidden: int, inter: int, device="cuda"):
    """Zero-filled workspace of dense_mlp for one (hidden, inter) shape."""
    n = lib().gpeed_iq3xxs_dense_mlp_ws_bytes(hidden, inter)
    if n == 0:
        raise ValueError("dense_mlp: hidden and inter must be positive multiples of 256")
    return _zeros(n, device)


def dense_mlp(w_gate, w_up, w_down, hidden: int, inter: int, x, limit: float = 10.0, out=None, ws=None,
              stream=None):
    """Model::dense_mlp (model.cpp:677-690): y = W_down swiglu(W_gate x, W_up x), two launches."""
    torch = _torch()
    _require_cuda(w_gate, w_up, w_down, x)
    if out is None:
        out = torch.empty(hidden, dtype=torch.float32, device=x.device)
    if ws is None:
        ws = dense_mlp_workspace(hidden, inter, x.device)
    _check(lib().gpeed_iq3xxs_dense_mlp(_ptr(w_gate), _ptr(w_up), _ptr(w_down), hidden, inter, _ptr(x), limit,
                                        _ptr(out), _ptr(ws), ws.numel(), _stream(stream)), "dense_mlp")
    return out


def gemv_swiglu(w_t64, n_rows: int, row0: int, in_dim: int, out_dim: int, g, u, limit: float = 10.0, out=None,
                ws=None, stream=None):
    """y = W @ (silu(min(g,limit)) * clamp(u,-limit,limit)), SwiGLU computed inside the GEMV (one launch)."""
    torch = _torch()
    _require_cuda(w_t64, g, u)
    if out is None:
        out = torch.empty(out_dim, dtype=torch.float32, device=g.device)
    if ws is None:
        ws = gemv_workspace(in_dim, out_dim, 1, 1, g.device)
    _check(lib().gpeed_iq3xxs_gemv_swiglu(_ptr(w_t64), n_rows, row0, in_dim, out_dim, _ptr(g), _ptr(u), limit,
                                          _ptr(out), _ptr(ws), ws.numel(), _stream(stream)), "gemv_swiglu")
    return out


def gemv2_act(w_a, w_b, n_rows: int, row0: int, in_dim: int, out_dim: int, act, n_tok: int = 1, out_a=None,
              out_b=None, ws=None, stream=None):
    """Two same-shape T64 tensors against one prepared activation, one launch."""
    torch = _torch()
    _require_cuda(w_a, w_b, act)
    if out_a is None:
        out_a = torch.empty(n_tok, out_dim, dtype=torch.float32, device=act.device)
    if out_b is None:
        out_b = torch.empty(n_tok, out_dim, dtype=torch.float32, device=act.device)
    if ws is None:
        ws = gemv_workspace(in_dim, out_dim, n_tok, 2, act.device)
    _check(lib().gpeed_iq3xxs_gemv2_act(_ptr(w_a), _ptr(w_b), n_rows, row0, in_dim, out_dim, _ptr(act), n_tok,
                                        _ptr(out_a), _ptr(out_b), _ptr(ws), ws.numel(), _stream(stream)),
           "gemv2_act")
    return out_a, out_b


def matvec_raw(w, n_rows: int, row0: int, in_dim: int, out_dim: int, x, out=None, stream=None):
    """dst = W[row0:row0+out_dim] @ x straight from GGUF rows on the device."""
    torch = _torch()
    _require_cuda(w, x)
    if out is None:
        out = torch.empty(out_dim, dtype=torch.float32, device=x.device)
    _check(lib().gpeed_iq3xxs_matvec_raw(_ptr(w), n_rows, row0, in_dim, out_dim, _ptr(x), _ptr(out),
                                         _stream(stream)), "matvec_raw")
    return out


def moe_route(logits, top_k: int, mode: int = 1, bias=None, routed_scale: float = 1.0, norm_topk: bool = True,
              ws=None, stream=None):
    """Router top-k and stable expert buckets on the device (model_batch.cpp:178-219).

    logits: [n_tok, n_exp] fp32 device tensor. Returns (eptr [n_exp+1],
    tok [n_tok*top_k], wt [n_tok*top_k], sel [n_tok, top_k]) device tensors.
    """
    torch = _torch()
    _require_cuda(logits)
    T, E = logits.shape
    dev_ = logits.device
    eptr = torch.empty(E + 1, dtype=torch.int32, device=dev_)
    tok = torch.empty(T * top_k, dtype=torch.int32, device=dev_)
    wt = torch.empty(T * top_k, dtype=torch.float32, device=dev_)
    sel = torch.empty(T, top_k, dtype=torch.int32, device=dev_)
    if ws is None:
        ws = _zeros(lib().gpeed_moe_route_ws_bytes(T, E, top_k), dev_)
    b = C.c_void_p(0) if bias is None else _ptr(bias)
    _check(lib().gpeed_moe_route(_ptr(logits), T, E, top_k, mode, b, routed_scale, int(norm_topk), _ptr(eptr),
                                 _ptr(tok), _ptr(wt), _ptr(sel), _ptr(ws), ws.numel(), _stream(stream)), "moe_route")
    return eptr, tok, wt, sel


def moe_experts(w_gate, w_up, w_down, n_exp: int, hidden: int, inter: int, X, top_k: int, eptr, tok, wt,
                swiglu_limit: float = 10.0, out=None, ws=None, stream=None):
    """Routed experts (model_batch.cpp:221-262) over T64 expert tensors; Y [n_tok, hidden]."""
    torch = _torch()
    _require_cuda(w_gate, w_up, w_down, X, eptr, tok, wt)
    T = X.shape[0]
    if out is None:
        out = torch.empty(T, hidden, dtype=torch.float32, device=X.device)
    if ws is None:
        ws = _zeros(lib().gpeed_iq3xxs_moe_ws_bytes(T, n_exp, top_k, hidden, inter), X.device)
    _check(lib().gpeed_iq3xxs_moe_experts(_ptr(w_gate), _ptr(w_up), _ptr(w_down), n_exp, hidden, inter, _ptr(X), T,
                                          top_k, _ptr(eptr), _ptr(tok), _ptr(wt), swiglu_limit, _ptr(out), _ptr(ws),
                                          ws.numel(), _stream(stream)), "moe_experts")
    return out


def moe_batch_workspace(n_tok: int, n_exp: int, top_k: int, hidden: int, inter: int, shared: bool = True,
                        device="cuda"):
    return _zeros(lib().gpeed_iq3xxs_moe_batch_ws_bytes(n_tok, n_exp, top_k, hidden, inter, int(shared)), device)


def moe_batch(logits, X, w_gate, w_up, w_down, n_exp: int, hidden: int, inter: int, top_k: int, mode: int = 0,
              bias=None, routed_scale: float = 1.0, norm_topk: bool = True, swiglu_limit: float = 10.0,
              shared=None, out=None, ws=None, routing: bool = False, stream=None):
    """The whole routed step of Model::moe_batch from the router logits
    (model_batch.cpp:174-280) in five launches: router + buckets, routed
    experts (T64 tensors), and the shared expert (shared = (gate, up, down)
    T64 tensors, or None) added last. Returns Y [n_tok, hidden], or
    (Y, eptr, tok, wt) with routing=True."""
    torch = _torch()
    _require_cuda(logits, X, w_gate, w_up, w_down)
    T = X.shape[0]
    dev_ = X.device
    if out is None:
        out = torch.empty(T, hidden, dtype=torch.float32, device=dev_)
    if ws is None:
        ws = moe_batch_workspace(T, n_exp, top_k, hidden, inter, shared is not None, dev_)
    gs, us, ds = (C.c_void_p(0),) * 3 if shared is None else \
        tuple(C.c_void_p(0) if t is None else _ptr(t) for t in shared)
    eptr = tok = wt = None
    if routing:
        eptr = torch.empty(n_exp + 1, dtype=torch.int32, device=dev_)
        tok = torch.empty(T * top_k, dtype=torch.int32, device=dev_)
        wt = torch.empty(T * top_k, dtype=torch.float32, device=dev_)
    nul = C.c_void_p(0)
    b = nul if bias is None else _ptr(bias)
    _check(lib().gpeed_iq3xxs_moe_batch(_ptr(logits), T, n_exp, top_k, mode, b, routed_scale, int(norm_topk),
                                        _ptr(w_gate), _ptr(w_up), _ptr(w_down), gs, us, ds, hidden, inter, _ptr(X),
                                        swiglu_limit, _ptr(out), _ptr(eptr) if routing else nul,
                                        _ptr(tok) if routing else nul, _ptr(wt) if routing else nul, _ptr(ws),
                                        ws.numel(), _stream(stream)), "moe_batch")
    return (out, eptr, tok, wt) if routing else out


def matmul_rows(dtype: int, w, n_rows: int, row0: int, in_dim: int, out_dim: int, X, out=None, stream=None):
    """Y[t][j] = sum_i W[row0+j][i] * X[t][i] over GGUF rows of any decoded type
    kept on the device (weights.cpp:86-203). X: [in_dim] or [n_tok, in_dim]."""
    torch = _torch()
    _require_cuda(w, X)
    vec = X.dim() == 1
    X2 = X.reshape(1 if vec else X.shape[0], in_dim)
    n_tok = X2.shape[0]
    if out is None:
        out = torch.empty((n_tok, out_dim), dtype=torch.float32, device=X.device)
    _check(lib().gpeed_matmul_rows(dtype, _ptr(w), n_rows, row0, in_dim, out_dim, _ptr(X2), n_tok, _ptr(out),
                                   _stream(stream)), "matmul_rows")
    return out.reshape(out_dim) if vec else out


class WeightStore:
    """Device-resident IQ3_XXS tensors behind the reference's matvec_quant contract.

    ``add(name, payload, in_dim, n_rows)`` uploads GGUF rows once and keeps
    their T64 copy in HBM (the role of pin_nonexpert, weights.cpp:70-84).
    ``matvec_quant`` follows weights.cpp:167-203: ``dst[j] = sum_i
    W[row0+j][i] * x[i]`` for ``j < out_dim`` (one launch); ``matmul_quant``
    follows weights.cpp:86-165 (``Y[t][j]`` for ``t < n_tok``, nothing done
    when ``n_tok <= 0`` or ``out_dim <= 0``): 8-token GEMV passes below
    ``matmul_gemm_min_tok()`` tokens, the prefill GEMM (one pass over W) from
    there on, as at the reference's prefill call sites
    (model_batch.cpp:30-95, 151-162). Host numpy arrays in, host numpy out
    (synchronous, like the reference), or device tensors in and out.
    """

    def __init__(self, device="cuda"):
        self.device = device
        self.tensors = {}
        self._ws = {}

    def add(self, name: str, payload, in_dim: int, n_rows: int, dtype: int = DTYPE_IQ3_XXS):
        """IQ3_XXS rows are kept in the T64 layout; the other decoded types as
        their GGUF rows."""
        torch = _torch()
        bs = dtype_block_size(dtype)
        if bs == 0:
            raise RuntimeError(f"weights: type {dtype} is not decoded")
        if in_dim % bs:
            raise RuntimeError(f"weights: row not block aligned for {name}")
        if isinstance(payload, np.ndarray):
            raw = torch.from_numpy(np.ascontiguousarray(payload).reshape(-1).view(np.uint8)).to(self.device)
        else:
            raw = payload.reshape(-1)
        dev = tile(raw, n_rows, in_dim) if dtype == DTYPE_IQ3_XXS else raw.clone()
        self.tensors[name] = (dev, in_dim, n_rows, dtype)
        return dev

    def has(self, name: str) -> bool:
        return name in self.tensors

    def _get(self, name: str, in_dim: int):
        if name not in self.tensors:
            raise RuntimeError(f"weights: missing tensor {name}")
        if in_dim % dtype_block_size(self.tensors[name][3]):
            raise RuntimeError(f"weights: row not block aligned for {name}")
        return self.tensors[name]

    def _workspace(self, in_dim: int, out_dim: int, n_tok: int):
        # one workspace per shape, grown when a call needs more (a workspace
        # sized for n_tok tokens serves every smaller call)
        key = (in_dim, out_dim)
        need = lib().gpeed_iq3xxs_matmul_ws_bytes(in_dim, out_dim, n_tok)
        ws = self._ws.get(key)
        if ws is None or ws.numel() < need:
            ws = self._ws[key] = matmul_workspace(in_dim, out_dim, n_tok, self.device)
        return ws

    @staticmethod
    def _row0_shift(row0: int, out_dim: int, n_rows: int, name: str) -> int:
        if row0 < 0 or row0 + out_dim > n_rows:
            raise GpeedError(-1, f"weights: rows outside {name}")
        return row0 % 64

    def matvec_quant(self, name: str, row0: int, in_dim: int, out_dim: int, x, dst=None):
        torch = _torch()
        t64, _, n_rows, dtype = self._get(name, in_dim)
        host = isinstance(x, np.ndarray)
        if out_dim <= 0:
            return dst
        xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(self.device) if host else x
        if dtype != DTYPE_IQ3_XXS:
            yd = matmul_rows(dtype, t64, n_rows, row0, in_dim, out_dim, xd.reshape(in_dim))
            ws = None
        else:
            # T64 products start on a 64-row tile; a row0 inside one runs from
            # the tile's first row and keeps rows row0.. (weights.cpp:167-203
            # takes any row0)
            shift = self._row0_shift(row0, out_dim, n_rows, name)
            ws = self._workspace(in_dim, out_dim + shift, 1)
            yd = matvec(t64, n_rows, row0 - shift, in_dim, out_dim + shift, xd, ws=ws)[shift:]
        if host:
            if ws is not None:
                ws_status(ws)  # synchronous, like the reference: report a flagged workspace here
            y = yd.cpu().numpy()
            if dst is not None:
                dst[:out_dim] = y
                return dst
            return y
        if dst is not None:
            dst.copy_(yd)
            return dst
        return yd

    def matmul_quant(self, name: str, row0: int, in_dim: int, out_dim: int, X, n_tok: int, Y=None):
        torch = _torch()
        t64, _, n_rows, dtype = self._get(name, in_dim)
        if n_tok <= 0 or out_dim <= 0:
            return Y
        host = isinstance(X, np.ndarray)
        Xd = torch.from_numpy(np.ascontiguousarray(X, np.float32).reshape(n_tok, in_dim)).to(self.device) \
            if host else X.reshape(n_tok, in_dim)
        if dtype != DTYPE_IQ3_XXS:
            Yd = matmul_rows(dtype, t64, n_rows, row0, in_dim, out_dim, Xd)
            ws = None
        else:
            shift = self._row0_shift(row0, out_dim, n_rows, name)
            ws = self._workspace(in_dim, out_dim + shift, n_tok)
            Yd = matmul(t64, n_rows, row0 - shift, in_dim, out_dim + shift, Xd, ws=ws)
            if shift:
                Yd = Yd.reshape(n_tok, out_dim + shift)[:, shift:].contiguous()
        if host:
            if ws is not None:
                ws_status(ws)
            y = Yd.cpu().numpy()
            if Y is not None:
                Y.reshape(n_tok, out_dim)[:] = y
                return Y
            return y
        if Y is not None:
            Y.copy_(Yd.reshape(Y.shape))
            return Y
        return Yd

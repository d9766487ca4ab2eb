"""CPU oracle for the IQ3_XXS dequantize-and-multiply path (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this package, and only as the correctness reference / the timed CPU
baseline. The
product (``gpeed_amd``) never imports it and has no CPU fallback.

``lib()``  -> liboracle.so, the plain-C restatement (iq3_oracle.c), with numpy
              wrappers below.
``ref()``  -> oracle/_ref/libgpeed_ref.so, the reference's own CPU sources
              compiled in place (see Makefile), or None when not built.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_lib = None
_ref = {}

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


def build(with_ref: bool = True) -> None:
    """Compile liboracle.so (and _ref when the reference checkout is present)."""
    targets = ["all"]
    if with_ref and os.path.isdir("/root/reference/cpp/core/src"):
        targets.append("ref")
    subprocess.run(["make", "-s", "-C", HERE] + targets, check=True)


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build(with_ref=False)
        L = C.CDLL(path)
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_sign_byte.argtypes = [C.c_uint]
        L.orc_sign_byte.restype = C.c_uint8
        L.orc_grid_entry.argtypes = [C.c_uint]
        L.orc_grid_entry.restype = C.c_uint32
        L.orc_iq3xxs_block.argtypes = [_u8p, _f32p]
        L.orc_dequantize.argtypes = [C.c_int, C.c_void_p, _f32p, C.c_uint64]
        L.orc_matmul_rows.argtypes = [C.c_int, C.c_void_p, C.c_uint64, C.c_int, C.c_int, _f32p, C.c_int, _f32p,
                                      _f32p]
        L.orc_block_elems.argtypes = [C.c_int]
        L.orc_block_bytes.argtypes = [C.c_int]
        L.orc_iq2s_grid.argtypes = [C.c_uint32]
        L.orc_iq2s_grid.restype = C.c_uint64
        L.orc_iq3s_grid.argtypes = [C.c_uint32]
        L.orc_iq3s_grid.restype = C.c_uint32
        L.orc_iq4nl_value.argtypes = [C.c_int]
        L.orc_dot_f32.argtypes = [_f32p, _f32p, C.c_int]
        L.orc_dot_f32.restype = C.c_float
        L.orc_axpy_f32.argtypes = [_f32p, _f32p, C.c_float, C.c_int]
        L.orc_matvec_quant.argtypes = [C.c_void_p, C.c_uint64, C.c_int, C.c_int, _f32p, _f32p]
        L.orc_matmul_quant.argtypes = [C.c_void_p, C.c_uint64, C.c_int, C.c_int, _f32p, C.c_int, _f32p]
        L.orc_moe_route.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_float,
                                    C.c_int, _i32p, _i32p, _f32p, _i32p]
        L.orc_moe_experts.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, _f32p, C.c_int,
                                      C.c_int, _i32p, _i32p, _f32p, C.c_float, _f32p]
        L.orc_dense_mlp.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, _f32p, C.c_int,
                                    C.c_float, _f32p]
        L.orc_moe_forward.argtypes = [_f32p, C.c_int, C.c_int, C.c_void_p, C.c_float, C.c_int, C.c_void_p,
                                      C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                      _f32p, C.c_float, _f32p]
        L.orc_moe_batch.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_float, C.c_int,
                                    C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_int, C.c_int, _f32p, C.c_float, _f32p]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def dequantize(raw: np.ndarray, n: int, dtype: int = 18) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    rc = lib().orc_dequantize(dtype, _ptr(np.ascontiguousarray(raw)), out, n)
    if rc != 0:
        raise RuntimeError(f"orc_dequantize rc={rc}")
    return out


def matmul_rows(dtype: int, w: np.ndarray, row0: int, in_dim: int, out_dim: int, X: np.ndarray) -> np.ndarray:
    """weights.cpp:86-203 over GGUF rows of any decoded type (Y[t][j], reference order)."""
    X = np.ascontiguousarray(np.atleast_2d(X), np.float32)
    Y = np.empty((X.shape[0], out_dim), np.float32)
    buf = np.empty(in_dim, np.float32)
    rc = lib().orc_matmul_rows(dtype, _ptr(np.ascontiguousarray(w)), row0, in_dim, out_dim, X, X.shape[0], Y, buf)
    if rc != 0:
        raise RuntimeError(f"orc_matmul_rows rc={rc}")
    return Y


def block_geometry(dtype: int):
    """(weights per block, bytes per block) of a decoded type (quant.cpp:52-114), else (0, 0)."""
    return lib().orc_block_elems(dtype), lib().orc_block_bytes(dtype)


def iq2s_grid() -> np.ndarray:
    return np.array([lib().orc_iq2s_grid(i) for i in range(1024)], np.uint64)


def iq3s_grid() -> np.ndarray:
    return np.array([lib().orc_iq3s_grid(i) for i in range(512)], np.uint64)


def iq4nl_values() -> np.ndarray:
    return np.array([lib().orc_iq4nl_value(i) for i in range(16)], np.int64)


def dot_f32(a: np.ndarray, b: np.ndarray) -> float:
    return float(lib().orc_dot_f32(np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32), a.size))


def matvec(w: np.ndarray, row0: int, in_dim: int, out_dim: int, x: np.ndarray) -> np.ndarray:
    y = np.empty(out_dim, dtype=np.float32)
    rc = lib().orc_matvec_quant(_ptr(w), row0, in_dim, out_dim, np.ascontiguousarray(x, np.float32), y)
    if rc != 0:
        raise RuntimeError(f"orc_matvec_quant rc={rc}")
    return y


def matmul(w: np.ndarray, row0: int, in_dim: int, out_dim: int, X: np.ndarray) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    n_tok = X.shape[0]
    Y = np.empty((n_tok, out_dim), dtype=np.float32)
    rc = lib().orc_matmul_quant(_ptr(w), row0, in_dim, out_dim, X, n_tok, Y)
    if rc != 0:
        raise RuntimeError(f"orc_matmul_quant rc={rc}")
    return Y


def moe_route(logits: np.ndarray, top_k: int, mode: int, bias=None, routed_scale=1.0, norm_topk=True):
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    eptr = np.empty(E + 1, np.int32)
    tok = np.empty(T * top_k, np.int32)
    wt = np.empty(T * top_k, np.float32)
    sel = np.empty(T * top_k, np.int32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    rc = lib().orc_moe_route(logits, T, E, top_k, mode, None if b is None else _ptr(b), routed_scale,
                             int(norm_topk), eptr, tok, wt, sel)
    if rc != 0:
        raise RuntimeError(f"orc_moe_route rc={rc}")
    return eptr, tok, wt, sel.reshape(T, top_k)


def moe_experts(w_gate, w_up, w_down, hidden, inter, X, eptr, tok, wt, swiglu_limit=10.0):
    X = np.ascontiguousarray(X, np.float32)
    T = X.shape[0]
    E = eptr.size - 1
    Y = np.empty((T, hidden), np.float32)
    rc = lib().orc_moe_experts(_ptr(w_gate), _ptr(w_up), _ptr(w_down), hidden, inter, X, T, E,
                               np.ascontiguousarray(eptr, np.int32), np.ascontiguousarray(tok, np.int32),
                               np.ascontiguousarray(wt, np.float32), swiglu_limit, Y)
    if rc != 0:
        raise RuntimeError(f"orc_moe_experts rc={rc}")
    return Y


def moe_batch(logits, X, w_gate, w_up, w_down, hidden, inter, top_k, mode=0, bias=None, routed_scale=1.0,
              norm_topk=True, swiglu_limit=10.0, shared=None):
    """model_batch.cpp:165-281 from the logits; shared = (gate, up, down) GGUF payloads or None."""
    logits = np.ascontiguousarray(logits, np.float32)
    X = np.ascontiguousarray(X, np.float32)
    T, E = logits.shape
    Y = np.empty((T, hidden), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    sh = (None, None, None) if shared is None else tuple(_ptr(np.ascontiguousarray(a)) for a in shared)
    rc = lib().orc_moe_batch(logits, T, E, top_k, mode, None if b is None else _ptr(b), routed_scale,
                             int(norm_topk), _ptr(w_gate), _ptr(w_up), _ptr(w_down), *sh, hidden, inter, X,
                             swiglu_limit, Y)
    if rc != 0:
        raise RuntimeError(f"orc_moe_batch rc={rc}")
    return Y


def moe_forward(logits, x, w_gate, w_up, w_down, hidden, inter, top_k, bias=None, routed_scale=1.0,
                norm_topk=True, swiglu_limit=10.0, shared=None):
    """model.cpp:692-755 for one token (rank-order combine); shared = (gate, up, down) or None."""
    logits = np.ascontiguousarray(logits, np.float32).reshape(-1)
    y = np.empty(hidden, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    sh = (None, None, None) if shared is None else tuple(_ptr(np.ascontiguousarray(a)) for a in shared)
    rc = lib().orc_moe_forward(logits, logits.size, top_k, None if b is None else _ptr(b), routed_scale,
                               int(norm_topk), _ptr(w_gate), _ptr(w_up), _ptr(w_down), *sh, hidden, inter,
                               np.ascontiguousarray(x, np.float32).reshape(-1), swiglu_limit, y)
    if rc != 0:
        raise RuntimeError(f"orc_moe_forward rc={rc}")
    return y


def dense_mlp(w_gate, w_up, w_down, hidden, inter, X, swiglu_limit=10.0):
    X = np.ascontiguousarray(X, np.float32)
    Y = np.empty((X.shape[0], hidden), np.float32)
    rc = lib().orc_dense_mlp(_ptr(w_gate), _ptr(w_up), _ptr(w_down), hidden, inter, X, X.shape[0],
                             swiglu_limit, Y)
    if rc != 0:
        raise RuntimeError(f"orc_dense_mlp rc={rc}")
    return Y


# --------------------------------------------------------------------------- reference (_ref)

def ref(openmp: bool = False):
    """The reference's own CPU path (oracle/_ref), or None if it was not built here."""
    key = "omp" if openmp else "st"
    if key not in _ref:
        path = os.path.join(HERE, "_ref", "libgpeed_ref_omp.so" if openmp else "libgpeed_ref.so")
        if not os.path.exists(path):
            _ref[key] = None
        else:
            L = C.CDLL(path)
            L.ref_last_error.restype = C.c_char_p
            L.ref_dequantize.argtypes = [C.c_int, C.c_void_p, _f32p, C.c_uint64]
            L.ref_dot_f32.argtypes = [_f32p, _f32p, C.c_int]
            L.ref_dot_f32.restype = C.c_float
            L.ref_axpy_f32.argtypes = [_f32p, _f32p, C.c_float, C.c_int]
            L.ref_store_open.argtypes = [C.c_void_p, C.c_uint64, C.c_int, C.c_char_p, C.c_char_p]
            L.ref_store_open.restype = C.c_void_p
            L.ref_store_open_typed.argtypes = [C.c_void_p, C.c_uint64, C.c_int, C.c_int, C.c_char_p, C.c_char_p]
            L.ref_store_open_typed.restype = C.c_void_p
            L.ref_store_matvec.argtypes = [C.c_void_p, C.c_uint64, C.c_int, C.c_int, _f32p, _f32p]
            L.ref_store_matmul.argtypes = [C.c_void_p, C.c_uint64, C.c_int, C.c_int, _f32p, C.c_int, _f32p]
            L.ref_store_close.argtypes = [C.c_void_p]
            L.ref_openmp_threads.restype = C.c_int
            L.ref_gguf_dump.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
            L.ref_gguf_dump.restype = C.c_long
            L.ref_gguf_read.argtypes = [C.c_char_p, C.c_char_p, C.c_void_p, C.c_size_t]
            L.ref_gguf_read.restype = C.c_long
            _ref[key] = L
    return _ref[key]


def ref_gguf_dump(path: str) -> dict:
    """What the reference's own GGUF loader parses from a file (JSON dict)."""
    import json

    L = ref()
    if L is None:
        raise RuntimeError("oracle/_ref is not built")
    buf = C.create_string_buffer(1 << 22)
    n = L.ref_gguf_dump(path.encode(), buf, len(buf))
    if n < 0:
        raise RuntimeError(L.ref_last_error().decode())
    return json.loads(buf.value.decode())


def ref_gguf_read(path: str, name: str, nbytes: int) -> bytes:
    """GgufModel::read_tensor of one tensor, by the reference's loader."""
    L = ref()
    if L is None:
        raise RuntimeError("oracle/_ref is not built")
    out = C.create_string_buffer(max(nbytes, 1))
    n = L.ref_gguf_read(path.encode(), name.encode(), out, nbytes)
    if n < 0:
        raise RuntimeError(L.ref_last_error().decode())
    return out.raw[:n]


class RefStore:
    """One tensor (IQ3_XXS unless dtype says otherwise) held by the reference's
    WeightStore (pinned in RAM)."""

    def __init__(self, payload: np.ndarray, n_rows: int, in_dim: int, openmp: bool = False,
                 name: str = "blk.0.ffn_down.weight", dtype: int = 18):
        self.L = ref(openmp)
        if self.L is None:
            raise RuntimeError("oracle/_ref is not built")
        self.payload = np.ascontiguousarray(payload)
        tmp = os.environ.get("TMPDIR", "/tmp")
        self.h = self.L.ref_store_open_typed(_ptr(self.payload), n_rows, in_dim, dtype, name.encode(), tmp.encode())
        if not self.h:
            raise RuntimeError(self.L.ref_last_error().decode())

    def matvec(self, row0, in_dim, out_dim, x):
        y = np.empty(out_dim, np.float32)
        if self.L.ref_store_matvec(self.h, row0, in_dim, out_dim, np.ascontiguousarray(x, np.float32), y):
            raise RuntimeError(self.L.ref_last_error().decode())
        return y

    def matmul(self, row0, in_dim, out_dim, X):
        X = np.ascontiguousarray(X, np.float32)
        Y = np.empty((X.shape[0], out_dim), np.float32)
        if self.L.ref_store_matmul(self.h, row0, in_dim, out_dim, X, X.shape[0], Y):
            raise RuntimeError(self.L.ref_last_error().decode())
        return Y

    def close(self):
        if self.h:
            self.L.ref_store_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

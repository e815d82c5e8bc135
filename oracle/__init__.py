"""ctypes binding of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU restatement of
recipe's CPU path. The product (librqmv and the rqmv package) never imports it.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int, c_int64, c_uint16, c_uint32, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
FORMATS = {"f32": F32, "f16": F16, "q4_0": Q4_0, "q8_0": Q8_0, "q4_k": Q4_K, "q6_k": Q6_K}

_lib = None



def _as_bytes(a) -> np.ndarray:
    """The array's bytes as stored (a view, never a value conversion)."""
    return np.ascontiguousarray(a).view(np.uint8).reshape(-1)

def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        L.orc_fp16_from_f32.argtypes = [c_float]
        L.orc_fp16_from_f32.restype = c_uint16
        L.orc_f32_from_fp16.argtypes = [c_uint16]
        L.orc_f32_from_fp16.restype = c_float
        L.orc_fp16_from_f32_n.argtypes = [c_void_p, c_void_p, ctypes.c_size_t]
        L.orc_dequant_value.argtypes = [c_int, c_void_p, c_int]
        L.orc_dequant_value.restype = c_double
        L.orc_dequant_rows.argtypes = [c_int, c_void_p, c_int64, c_int64, c_void_p]
        L.orc_matvec_f64.argtypes = [c_int, c_void_p, c_int64, c_int64, c_void_p, c_int, c_int64, c_void_p, c_int64]
        L.orc_matvec_recipe_f32.argtypes = [c_int, c_void_p, c_int64, c_int64, c_void_p, c_int, c_int64, c_void_p,
                                            c_int64, c_int]
        L.orc_matvec_recipe_fast.argtypes = [c_int, c_void_p, c_int64, c_int64, c_void_p, c_int, c_int64, c_void_p,
                                             c_int64, c_int]
        L.orc_topk.argtypes = [c_void_p, c_int, c_int, c_int, c_int, c_void_p]
        L.orc_topk_biased.argtypes = [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p]
        L.orc_activation.argtypes = [c_int, c_double, c_double, c_void_p]
        L.orc_moe_f64.argtypes = [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_double, c_int, c_double,
                                  c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]
        L.orc_q4k_q81_reference.argtypes = [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p]
        L.orc_q4k_xorshift_rows.argtypes = [c_uint32, c_int64, c_uint16, c_void_p]
        L.orc_q8_records.argtypes = [c_void_p, c_int64, c_int, c_void_p, c_void_p]
        L.orc_int8_matvec.argtypes = [c_int, c_void_p, c_int64, c_int64, c_void_p, c_int, c_int, c_int, c_void_p]
        L.orc_fp16_rne.argtypes = [c_float]
        L.orc_fp16_rne.restype = c_uint16
        L.orc_requantize_q8_0.argtypes = [c_int, c_void_p, c_int64, c_int64, c_void_p]
        _lib = L
    return _lib


def _fmt(fmt):
    return FORMATS[fmt] if isinstance(fmt, str) else int(fmt)


def _ptr(a: np.ndarray):
    return a.ctypes.data if a is not None else None


def fp16_from_f32(values) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = np.empty(v.size, np.uint16)
    lib().orc_fp16_from_f32_n(v.ctypes.data, out.ctypes.data, v.size)
    return out


def f32_from_fp16(bits) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16).reshape(-1)
    return np.array([lib().orc_f32_from_fp16(int(v)) for v in b], dtype=np.float32)


def _row_split(g: np.ndarray, rows: int, threads: int, call) -> None:
    """Run call(r0, r1, row_bytes) over contiguous row ranges on `threads`
    threads (the C routines work row by row and release the GIL)."""
    if rows <= 0 or g.size % rows:
        raise ValueError("GGUF bytes must hold whole rows")
    row_bytes = g.size // rows
    threads = max(1, min(int(threads), rows))
    edges = [rows * t // threads for t in range(threads + 1)]
    if threads == 1:
        call(0, rows, row_bytes)
        return
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(threads) as pool:
        for f in [pool.submit(call, edges[t], edges[t + 1], row_bytes) for t in range(threads)]:
            f.result()


def dequant_rows(fmt, gguf: np.ndarray, rows: int, cols: int, threads: int = 1) -> np.ndarray:
    g = _as_bytes(gguf)
    out = np.empty(rows * cols, np.float32)

    def run(r0, r1, row_bytes):
        rc = lib().orc_dequant_rows(_fmt(fmt), g.ctypes.data + r0 * row_bytes, r1 - r0, cols,
                                    out.ctypes.data + 4 * r0 * cols)
        assert rc == 0, rc

    _row_split(g, rows, threads, run)
    return out.reshape(rows, cols)


def dequant_value(fmt, block: np.ndarray, index: int) -> float:
    b = _as_bytes(block)
    return lib().orc_dequant_value(_fmt(fmt), b.ctypes.data, index)


def matvec_f64(fmt, gguf: np.ndarray, rows: int, cols: int, x: np.ndarray, threads: int = 1) -> np.ndarray:
    """x (M, K) float64 -> y (M, N) float64."""
    g = _as_bytes(gguf)
    x2 = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float64)
    m = x2.shape[0]
    y = np.empty((m, rows), np.float64)

    def run(r0, r1, row_bytes):
        rc = lib().orc_matvec_f64(_fmt(fmt), g.ctypes.data + r0 * row_bytes, r1 - r0, cols, x2.ctypes.data, m, cols,
                                  y.ctypes.data + 8 * r0, rows)
        assert rc == 0, rc

    _row_split(g, rows, threads, run)
    return y


def matvec_recipe_f32(fmt, gguf: np.ndarray, rows: int, cols: int, x: np.ndarray, threads: int = 1) -> np.ndarray:
    """recipe's fp32 float packed path: x (M, K) float32 -> y (M, N) float32."""
    g = _as_bytes(gguf)
    x2 = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    m = x2.shape[0]
    y = np.empty((m, rows), np.float32)
    rc = lib().orc_matvec_recipe_f32(_fmt(fmt), g.ctypes.data, rows, cols, x2.ctypes.data, m, cols, y.ctypes.data,
                                     rows, threads)
    assert rc == 0, rc
    return y


def matvec_recipe_fast(fmt, gguf: np.ndarray, rows: int, cols: int, x: np.ndarray, threads: int = 1) -> np.ndarray:
    """matvec_recipe_f32's products bit for bit, on recipe's compiled schedule
    (the timed CPU baseline)."""
    g = _as_bytes(gguf)
    x2 = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    m = x2.shape[0]
    y = np.empty((m, rows), np.float32)
    rc = lib().orc_matvec_recipe_fast(_fmt(fmt), g.ctypes.data, rows, cols, x2.ctypes.data, m, cols, y.ctypes.data,
                                      rows, threads)
    assert rc == 0, rc
    return y


# recipe's Activation::code() values (recipe.rs:13925-13950); "gelu_fp16" is
# Gelu under the llama.cpp profile's gelu table.
ACTIVATIONS = {"linear": 0, "cos": 1, "exp": 2, "log": 3, "ln": 4, "huber": 5, "tan": 6, "relu": 7, "leak": 8,
               "sigmoid": 9, "tanh": 10, "selu": 11, "gelu": 12, "silu": 13, "elu": 14, "prelu": 15, "scale": 16,
               "sqrt": 17, "softplus": 18, "gelu_fp16": 32}


def _act(a) -> int:
    return ACTIVATIONS[a] if isinstance(a, str) else int(a)


def activation(act, x, factor: float = 0.0) -> np.ndarray:
    """recipe's activation program applied elementwise in f64."""
    xs = np.asarray(x, dtype=np.float64).reshape(-1)
    out = np.empty_like(xs)
    r = c_double()
    for i, v in enumerate(xs):
        assert lib().orc_activation(_act(act), factor, float(v), ctypes.byref(r)) == 1
        out[i] = r.value
    return out.reshape(np.shape(x))


def topk(scores: np.ndarray, top: int, scoring: int = 0, renormalize: bool = True, bias=None) -> np.ndarray:
    s = np.ascontiguousarray(scores, dtype=np.float64)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float64)
    w = np.empty_like(s)
    rc = lib().orc_topk_biased(s.ctypes.data, s.size, top, scoring, 1 if renormalize else 0, _ptr(b), w.ctypes.data)
    assert rc == 0, rc
    return w


def moe_f64(fmt, d_model, experts, top, hidden, router_bits, gate, up, down, x, scoring=0, renormalize=True,
            scale=1.0, hidden_shared=0, shared_gate_bits=None, gate_sh=None, up_sh=None, down_sh=None,
            activation="silu", shared_gate_activation="sigmoid", activation_factor=0.0, selection_bias=None):
    """Returns (y float64 (d_model,), routing weights float64 (experts,)).
    A shared expert (gate_sh, up_sh, down_sh) is weighted by
    shared_gate_activation(shared_gate . x), or by one without shared_gate_bits."""
    r = np.ascontiguousarray(router_bits, dtype=np.uint16)
    xs = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty(d_model, np.float64)
    rw = np.empty(experts, np.float64)
    conv = lambda a, t: None if a is None else np.ascontiguousarray(a, dtype=t)  # noqa: E731
    sg, gs, us, ds = conv(shared_gate_bits, np.uint16), conv(gate_sh, np.uint8), conv(up_sh, np.uint8), conv(down_sh, np.uint8)
    g, u, d = conv(gate, np.uint8), conv(up, np.uint8), conv(down, np.uint8)
    sb = conv(selection_bias, np.float64)
    rc = lib().orc_moe_f64(_fmt(fmt), d_model, experts, top, hidden, scoring, 1 if renormalize else 0, scale,
                           _act(activation), activation_factor, _ptr(sb), r.ctypes.data, g.ctypes.data, u.ctypes.data,
                           d.ctypes.data, hidden_shared, _ptr(sg), _act(shared_gate_activation), _ptr(gs), _ptr(us),
                           _ptr(ds), xs.ctypes.data, y.ctypes.data, rw.ctypes.data)
    assert rc == 0, rc
    return y, rw


def q4k_q81_reference(w: np.ndarray, rows: int, cols: int, x: np.ndarray):
    """evidence bench.rs algebra: returns (y float32 (rows,), x as used float64 (cols,))."""
    g = _as_bytes(w)
    xs = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, np.float32)
    xu = np.empty(cols, np.float64)
    rc = lib().orc_q4k_q81_reference(g.ctypes.data, rows, cols, xs.ctypes.data, y.ctypes.data, xu.ctypes.data)
    assert rc == 0, rc
    return y, xu


def q4k_xorshift_rows(seed: int, rows: int, scale_bits: int) -> np.ndarray:
    out = np.empty(rows * 16 * 144, np.uint8)
    lib().orc_q4k_xorshift_rows(seed, rows, scale_bits, out.ctypes.data)
    return out


def q8_records(x: np.ndarray, step: int):
    """recipe's int(8) activation records of one position: (d float32 (K/32,), codes int8 (K,))."""
    xs = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    d = np.empty(xs.size // 32, np.float32)
    codes = np.empty(xs.size, np.int8)
    rc = lib().orc_q8_records(xs.ctypes.data, xs.size, step, d.ctypes.data, codes.ctypes.data)
    assert rc == 0, rc
    return d, codes


def int8_matvec(fmt, gguf: np.ndarray, rows: int, cols: int, x: np.ndarray, step: int = 32,
                tail: bool = False) -> np.ndarray:
    """recipe's int(8) sum over GGUF block rows: x (M, cols) float32 -> y (M, rows) float32."""
    g = _as_bytes(gguf)
    xs = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
    y = np.empty((xs.shape[0], rows), np.float32)
    rc = lib().orc_int8_matvec(_fmt(fmt), g.ctypes.data, rows, cols, xs.ctypes.data, xs.shape[0], step,
                               1 if tail else 0, y.ctypes.data)
    assert rc == 0, rc
    return y


def requantize_q8_0(fmt, gguf: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """recipe's int(8) storage for a non-Q4_K weight: the Q8_0 blocks (uint8)."""
    g = _as_bytes(gguf)
    out = np.empty(rows * (cols // 32) * 34, np.uint8)
    rc = lib().orc_requantize_q8_0(_fmt(fmt), g.ctypes.data, rows, cols, out.ctypes.data)
    assert rc == 0, rc
    return out

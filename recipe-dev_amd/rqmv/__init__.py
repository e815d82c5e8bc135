"""Python binding of librqmv, the gfx950 GGUF quantized matrix-vector library.

A thin ctypes layer over the C ABI in include/rqmv.h plus the few HIP runtime
calls a host program needs (device buffers, streams, events), taken from the
same libamdhip64 that librqmv links. Nothing here computes: every product runs
in librqmv's HIP kernels, and loading fails loudly when the library is absent.

The host-side names mirror recipe's single-op API (recipe.rs:17126-17199):
`contract(weight, x)` is Gguf::contract (one projection, fp32 out) and
`expert(bank, index, x)` is Gguf::expert; `moe(...)` runs one gguf_moe block.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, byref, c_char_p, c_double, c_float, c_int, c_int64, c_size_t, c_void_p

import numpy as np

from . import synth  # noqa: F401

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "librqmv.so")

F16, Q4_0, Q8_0, Q4_K, Q6_K = 1, 2, 8, 12, 14
FORMATS = {"f16": F16, "q4_0": Q4_0, "q8_0": Q8_0, "q4_k": Q4_K, "q6_k": Q6_K}
DTYPE_F32, DTYPE_F16 = 0, 1
SCORE_SOFTMAX, SCORE_SIGMOID = 0, 1

_H2D, _D2H, _D2D = 1, 2, 3


class RqmvError(RuntimeError):
    pass


class _Lib:
    def __init__(self):
        if not os.path.exists(LIB_PATH):
            raise RqmvError(f"librqmv.so is not built ({LIB_PATH}); run __graft_entry__.build()")
        self.lib = ctypes.CDLL(LIB_PATH)
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        L, H = self.lib, self.hip
        L.rqmv_init.argtypes = [c_int]
        L.rqmv_last_error.restype = c_char_p
        L.rqmv_weight_create.argtypes = [c_int, c_int64, c_int64, c_void_p, c_size_t, POINTER(c_void_p)]
        L.rqmv_expert_bank_create.argtypes = [c_int, c_int64, c_int64, c_int64, c_void_p, c_size_t, POINTER(c_void_p)]
        L.rqmv_weight_destroy.argtypes = [c_void_p]
        L.rqmv_weight_info.argtypes = [c_void_p, POINTER(c_int), POINTER(c_int64), POINTER(c_int64), POINTER(c_int64),
                                       POINTER(c_size_t)]
        L.rqmv_weight_unpack.argtypes = [c_void_p, c_void_p, c_size_t]
        L.rqmv_weight_dequantize.argtypes = [c_void_p, c_void_p, c_void_p]
        L.rqmv_matvec.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int64, c_void_p, c_int64, c_void_p]
        L.rqmv_matvec_timed.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int64, c_void_p, c_int64, c_void_p,
                                        c_void_p, c_void_p]
        L.rqmv_expert_matvec.argtypes = [c_void_p, c_int64, c_void_p, c_int, c_int, c_int64, c_void_p, c_int64, c_void_p]
        L.rqmv_moe_workspace_size.argtypes = [c_void_p, POINTER(c_size_t)]
        L.rqmv_moe.argtypes = [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]
        L.rqmv_moe_batch_noalloc.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int64, c_void_p, c_int64, c_void_p,
                                             c_void_p]
        L.rqmv_moe_batch.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int64, c_void_p, c_int64, c_void_p, c_void_p,
                                     c_size_t, c_void_p]
        L.rqmv_add_rmsnorm.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_float, c_void_p, c_void_p]
        L.rqmv_rope_kv.argtypes = [c_void_p, c_void_p, c_int, c_int, c_int, ctypes.c_double, c_void_p, c_void_p, c_int,
                                   c_void_p]
        L.rqmv_attention_workspace_size.argtypes = [c_int, c_int, c_int, c_int, POINTER(c_size_t)]
        L.rqmv_attention.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p,
                                     c_size_t, c_void_p, c_void_p]
        L.rqmv_silu_mul.argtypes = [c_void_p, c_int, c_void_p, c_void_p]
        L.rqmv_argmax.argtypes = [c_void_p, c_int, c_void_p, c_void_p, c_size_t, c_void_p]
        L.rqmv_argmax_workspace_size.argtypes = [POINTER(c_size_t)]
        L.rqmv_advance.argtypes = [c_void_p, c_void_p]
        L.rqmv_capability.argtypes = [ctypes.c_char_p, POINTER(ctypes.c_char_p), POINTER(ctypes.c_char_p)]
        L.rqmv_weight_create_int8.argtypes = [c_int, c_int64, c_int64, c_int64, c_void_p, c_size_t, POINTER(c_void_p)]
        L.rqmv_requantize_q8_0_host.argtypes = [c_int, c_int64, c_int64, c_void_p, c_size_t, c_void_p]
        L.rqmv_matvec_int8.argtypes = [c_void_p, c_void_p, c_int, c_int64, c_void_p, c_int64, c_int, c_int, c_void_p]
        L.rqmv_q8_records.argtypes = [c_void_p, c_int64, c_int, c_void_p, c_void_p, c_void_p]
        L.rqmv_embed_row.argtypes = [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p]
        L.rqmv_gguf_open.argtypes = [c_char_p, c_void_p]
        L.rqmv_gguf_close.argtypes = [c_void_p]
        L.rqmv_gguf_tensor_count.argtypes = [c_void_p, POINTER(c_int64)]
        L.rqmv_gguf_tensor_info.argtypes = [c_void_p, c_int64, POINTER(c_char_p), POINTER(c_int), POINTER(c_int),
                                            POINTER(c_int64), POINTER(c_size_t)]
        L.rqmv_gguf_find_tensor.argtypes = [c_void_p, c_char_p, POINTER(c_int64)]
        L.rqmv_gguf_tensor_data.argtypes = [c_void_p, c_int64, POINTER(c_void_p), POINTER(c_size_t)]
        L.rqmv_gguf_metadata_count.argtypes = [c_void_p, POINTER(c_int64)]
        L.rqmv_gguf_metadata_key.argtypes = [c_void_p, c_int64, POINTER(c_char_p), POINTER(c_int)]
        L.rqmv_gguf_get_int.argtypes = [c_void_p, c_char_p, POINTER(c_int64)]
        L.rqmv_gguf_get_float.argtypes = [c_void_p, c_char_p, POINTER(c_double)]
        L.rqmv_gguf_get_string.argtypes = [c_void_p, c_char_p, POINTER(c_char_p)]
        L.rqmv_gguf_get_array.argtypes = [c_void_p, c_char_p, POINTER(c_int), POINTER(c_int64)]
        L.rqmv_gguf_get_array_int.argtypes = [c_void_p, c_char_p, c_int64, POINTER(c_int64)]
        L.rqmv_gguf_get_array_string.argtypes = [c_void_p, c_char_p, c_int64, POINTER(c_char_p)]
        L.rqmv_gguf_weight_create.argtypes = [c_void_p, c_char_p, c_void_p]
        L.rqmv_rope_table.argtypes = [c_void_p, c_int, c_double, c_int, c_void_p]
        L.rqmv_attention_rope.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                          c_void_p, c_size_t, c_void_p, c_void_p]
        L.rqmv_glu_weight_create.argtypes = [c_int, c_int64, c_int64, c_void_p, c_void_p, c_size_t, c_void_p]
        L.rqmv_matvec_fused.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]
        L.rqmv_layout_bytes.argtypes = [c_int, c_int64, c_int64, POINTER(c_size_t)]
        L.rqmv_repack_host.argtypes = [c_int, c_int64, c_int64, c_void_p, c_void_p]
        L.rqmv_unpack_host.argtypes = [c_int, c_int64, c_int64, c_void_p, c_void_p]
        H.hipMalloc.argtypes = [POINTER(c_void_p), c_size_t]
        H.hipFree.argtypes = [c_void_p]
        H.hipMemcpy.argtypes = [c_void_p, c_void_p, c_size_t, c_int]
        H.hipMemcpyAsync.argtypes = [c_void_p, c_void_p, c_size_t, c_int, c_void_p]
        H.hipMemset.argtypes = [c_void_p, c_int, c_size_t]
        H.hipDeviceSynchronize.argtypes = []
        H.hipStreamCreate.argtypes = [POINTER(c_void_p)]
        H.hipStreamDestroy.argtypes = [c_void_p]
        H.hipStreamSynchronize.argtypes = [c_void_p]
        H.hipEventCreate.argtypes = [POINTER(c_void_p)]
        H.hipEventDestroy.argtypes = [c_void_p]
        H.hipEventRecord.argtypes = [c_void_p, c_void_p]
        H.hipEventSynchronize.argtypes = [c_void_p]
        H.hipEventElapsedTime.argtypes = [POINTER(c_float), c_void_p, c_void_p]
        H.hipGetErrorString.restype = c_char_p
        H.hipGetErrorString.argtypes = [c_int]
        H.hipGetDeviceCount.argtypes = [POINTER(c_int)]
        H.hipStreamBeginCapture.argtypes = [c_void_p, c_int]
        H.hipStreamEndCapture.argtypes = [c_void_p, POINTER(c_void_p)]
        H.hipGraphInstantiate.argtypes = [POINTER(c_void_p), c_void_p, c_void_p, c_char_p, c_size_t]
        H.hipGraphLaunch.argtypes = [c_void_p, c_void_p]
        H.hipGraphExecDestroy.argtypes = [c_void_p]
        H.hipGraphDestroy.argtypes = [c_void_p]


_lib = None



def _as_bytes(a) -> np.ndarray:
    """The array's bytes as stored (a view, never a value conversion)."""
    return np.ascontiguousarray(a).view(np.uint8).reshape(-1)

def lib() -> _Lib:
    global _lib
    if _lib is None:
        _lib = _Lib()
    return _lib


def _check(rc: int, what: str):
    if rc != 0:
        raise RqmvError(f"{what} failed ({rc}): {lib().lib.rqmv_last_error().decode()}")


def _hip(rc: int, what: str):
    if rc != 0:
        raise RqmvError(f"{what}: {lib().hip.hipGetErrorString(rc).decode()}")


def device_count() -> int:
    n = c_int(0)
    rc = lib().hip.hipGetDeviceCount(byref(n))
    return n.value if rc == 0 else 0


def init(device: int = 0):
    _check(lib().lib.rqmv_init(device), "rqmv_init")


def synchronize():
    _hip(lib().hip.hipDeviceSynchronize(), "hipDeviceSynchronize")


class DeviceBuffer:
    """A device allocation (freed on close/garbage collection)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = c_void_p()
        _hip(lib().hip.hipMalloc(byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        _hip(lib().hip.hipMemcpy(self.ptr, arr.ctypes.data, arr.nbytes, _H2D), "hipMemcpy H2D")

    def download(self, dtype, count: int | None = None) -> np.ndarray:
        return _download(self.ptr, self.nbytes, dtype, count)

    def fill_zero(self):
        _hip(lib().hip.hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def copy_from(self, src: "DeviceBuffer", nbytes: int, stream=None):
        """Stream-ordered device-to-device copy of src's first nbytes."""
        assert nbytes <= self.nbytes and nbytes <= src.nbytes
        _hip(lib().hip.hipMemcpyAsync(self.ptr, src.ptr, nbytes, _D2D, stream.handle if stream else None),
             "hipMemcpyAsync D2D")

    def view(self, offset: int, nbytes: int) -> "BufferView":
        """A non-owning window [offset, offset + nbytes) of this allocation."""
        if offset < 0 or nbytes < 0 or offset + nbytes > self.nbytes:
            raise ValueError("view outside the buffer")
        return BufferView(self, self.ptr + offset, nbytes)

    def close(self):
        if self.ptr:
            lib().hip.hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class BufferView:
    """Part of a DeviceBuffer, usable wherever a kernel takes a device pointer;
    it keeps its parent alive and frees nothing itself."""

    def __init__(self, parent: DeviceBuffer, ptr: int, nbytes: int):
        self.parent, self.ptr, self.nbytes = parent, ptr, nbytes

    def download(self, dtype, count: int | None = None) -> np.ndarray:
        return _download(self.ptr, self.nbytes, dtype, count)


def _download(ptr: int, nbytes: int, dtype, count: int | None) -> np.ndarray:
    """`count` values of `dtype` (all that fit when None) copied from device memory."""
    dtype = np.dtype(dtype)
    n = nbytes // dtype.itemsize if count is None else int(count)
    if not 0 <= n * dtype.itemsize <= nbytes:
        raise ValueError(f"{n} values of {dtype} do not fit in {nbytes} bytes")
    out = np.empty(n, dtype=dtype)
    _hip(lib().hip.hipMemcpy(out.ctypes.data, ptr, out.nbytes, _D2H), "hipMemcpy D2H")
    return out


class Stream:
    def __init__(self):
        s = c_void_p()
        _hip(lib().hip.hipStreamCreate(byref(s)), "hipStreamCreate")
        self.handle = s.value

    def synchronize(self):
        _hip(lib().hip.hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def close(self):
        if self.handle:
            lib().hip.hipStreamDestroy(self.handle)
            self.handle = None


class Event:
    def __init__(self):
        e = c_void_p()
        _hip(lib().hip.hipEventCreate(byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream=None):
        _hip(lib().hip.hipEventRecord(self.handle, stream.handle if stream else None), "hipEventRecord")

    def synchronize(self):
        _hip(lib().hip.hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, later: "Event") -> float:
        ms = c_float(0.0)
        _hip(lib().hip.hipEventElapsedTime(byref(ms), self.handle, later.handle), "hipEventElapsedTime")
        return ms.value

    def close(self):
        if self.handle:
            lib().hip.hipEventDestroy(self.handle)
            self.handle = None


class Graph:
    """A HIP graph captured from the work a callable enqueues on `stream`."""

    def __init__(self, stream: Stream, enqueue):
        H = lib().hip
        _hip(H.hipStreamBeginCapture(stream.handle, 2), "hipStreamBeginCapture")  # relaxed mode
        try:
            enqueue()
        finally:
            g = c_void_p()
            _hip(H.hipStreamEndCapture(stream.handle, byref(g)), "hipStreamEndCapture")
        self.graph = g.value
        ex = c_void_p()
        _hip(H.hipGraphInstantiate(byref(ex), self.graph, None, None, 0), "hipGraphInstantiate")
        self.exec = ex.value

    def launch(self, stream: Stream):
        _hip(lib().hip.hipGraphLaunch(self.exec, stream.handle), "hipGraphLaunch")

    def close(self):
        if self.exec:
            lib().hip.hipGraphExecDestroy(self.exec)
            lib().hip.hipGraphDestroy(self.graph)
            self.exec = None


def _fmt(fmt) -> int:
    return FORMATS[fmt] if isinstance(fmt, str) else int(fmt)


class Weight:
    """A repacked weight (or expert bank) resident on the device."""

    def __init__(self, fmt, rows: int, cols: int, gguf: np.ndarray, experts: int | None = None):
        # the tensor's bytes as stored (an F16 tensor may come as uint16 or float16 values)
        gguf = np.ascontiguousarray(gguf).view(np.uint8).reshape(-1)
        h = c_void_p()
        if experts is None:
            _check(lib().lib.rqmv_weight_create(_fmt(fmt), rows, cols, gguf.ctypes.data, gguf.nbytes, byref(h)),
                   "rqmv_weight_create")
        else:
            _check(lib().lib.rqmv_expert_bank_create(_fmt(fmt), experts, rows, cols, gguf.ctypes.data, gguf.nbytes,
                                                     byref(h)), "rqmv_expert_bank_create")
        self.handle = h.value
        self.fmt, self.rows, self.cols = _fmt(fmt), rows, cols
        self.experts = 1 if experts is None else experts
        self.gguf_nbytes = gguf.nbytes
        self.glu = False

    def info(self):
        f, r, c, e, b = c_int(), c_int64(), c_int64(), c_int64(), c_size_t()
        _check(lib().lib.rqmv_weight_info(self.handle, byref(f), byref(r), byref(c), byref(e), byref(b)), "info")
        return {"format": f.value, "rows": r.value, "cols": c.value, "experts": e.value, "device_bytes": b.value}

    def unpack(self) -> np.ndarray:
        out = np.empty(self.gguf_nbytes, dtype=np.uint8)
        _check(lib().lib.rqmv_weight_unpack(self.handle, out.ctypes.data, out.nbytes), "rqmv_weight_unpack")
        return out

    def dequantize(self, out: DeviceBuffer, stream: Stream | None = None):
        _check(lib().lib.rqmv_weight_dequantize(self.handle, out.ptr, stream.handle if stream else None),
               "rqmv_weight_dequantize")

    def matvec(self, x: DeviceBuffer, x_dtype: int, m: int, ldx: int, y: DeviceBuffer, ldy: int,
               stream: Stream | None = None, x_offset: int = 0, y_offset: int = 0):
        _check(lib().lib.rqmv_matvec(self.handle, x.ptr + x_offset, x_dtype, m, ldx, y.ptr + y_offset, ldy,
                                     stream.handle if stream else None), "rqmv_matvec")

    def matvec_timed(self, x: DeviceBuffer, x_dtype: int, m: int, ldx: int, y: DeviceBuffer, ldy: int,
                     stream: Stream | None, start: "Event", stop: "Event"):
        """matvec whose kernel dispatch records `start` and `stop` itself."""
        _check(lib().lib.rqmv_matvec_timed(self.handle, x.ptr, x_dtype, m, ldx, y.ptr, ldy,
                                           stream.handle if stream else None, start.handle, stop.handle),
               "rqmv_matvec_timed")

    def expert_matvec(self, expert: int, x: DeviceBuffer, x_dtype: int, m: int, ldx: int, y: DeviceBuffer, ldy: int,
                      stream: Stream | None = None):
        _check(lib().lib.rqmv_expert_matvec(self.handle, expert, x.ptr, x_dtype, m, ldx, y.ptr, ldy,
                                            stream.handle if stream else None), "rqmv_expert_matvec")

    def close(self):
        if self.handle:
            lib().lib.rqmv_weight_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _x_host(x: np.ndarray):
    if x.dtype == np.float16:
        return x.view(np.uint16), DTYPE_F16
    if x.dtype == np.uint16:
        return x, DTYPE_F16
    return x.astype(np.float32), DTYPE_F32


def contract(weight: Weight, x: np.ndarray) -> np.ndarray:
    """One projection of host activations (Gguf::contract, recipe.rs:17130):
    x is (K,) or (M, K) as float16 (or uint16 bits) or float32; returns fp32 (M, N)."""
    x2 = np.atleast_2d(x)
    xh, dt = _x_host(np.ascontiguousarray(x2))
    m, k = xh.shape
    xb = DeviceBuffer.from_array(xh)
    yb = DeviceBuffer(4 * m * weight.rows * weight.experts)
    weight.matvec(xb, dt, m, k, yb, weight.rows * weight.experts)
    synchronize()
    y = yb.download(np.float32).reshape(m, -1)
    return y[0] if x.ndim == 1 else y


def expert(bank: Weight, index: int, x: np.ndarray) -> np.ndarray:
    """One expert of a bank (Gguf::expert, recipe.rs:17135)."""
    x2 = np.atleast_2d(x)
    xh, dt = _x_host(np.ascontiguousarray(x2))
    m, k = xh.shape
    xb = DeviceBuffer.from_array(xh)
    yb = DeviceBuffer(4 * m * bank.rows)
    bank.expert_matvec(index, xb, dt, m, k, yb, bank.rows)
    synchronize()
    y = yb.download(np.float32).reshape(m, -1)
    return y[0] if x.ndim == 1 else y


INT8_TAIL = 1


def matvec_int8(weight: Weight, x: DeviceBuffer, m: int, ldx: int, y: DeviceBuffer, ldy: int, step: int = 32,
                tail: bool = False, stream: Stream | None = None):
    """recipe's int(8) sum (rqmv_matvec_int8): fp32 activation rows, Q8 records
    of `step` inputs, recipe's fp32 order."""
    _check(lib().lib.rqmv_matvec_int8(weight.handle, x.ptr, m, ldx, y.ptr, ldy, step, INT8_TAIL if tail else 0,
                                      _sh(stream)), "rqmv_matvec_int8")


def capability(fmt: str):
    """(vector, matrix) instruction descriptions for a compute format on gfx950
    (rqmv_capability); raises RqmvError where there is neither."""
    v, m = ctypes.c_char_p(), ctypes.c_char_p()
    _check(lib().lib.rqmv_capability(fmt.encode(), byref(v), byref(m)), "rqmv_capability")
    return (v.value.decode() if v.value else None, m.value.decode() if m.value else None)


def int8_weight(fmt, rows: int, cols: int, gguf: np.ndarray, experts: int | None = None) -> Weight:
    """A weight stored as recipe's int(8) profile stores it (rqmv_weight_create_int8):
    Q4_K and Q8_0 as they are, F16/Q4_0/Q6_K re-encoded to Q8_0."""
    gguf = np.ascontiguousarray(gguf).view(np.uint8).reshape(-1)
    h = c_void_p()
    _check(lib().lib.rqmv_weight_create_int8(_fmt(fmt), experts or 1, rows, cols, gguf.ctypes.data, gguf.nbytes,
                                             byref(h)), "rqmv_weight_create_int8")
    w = Weight.__new__(Weight)
    w.handle = h.value
    w.rows, w.cols, w.experts = rows, cols, experts or 1
    w.fmt = w.info()["format"]
    w.gguf_nbytes = rows * (experts or 1) * cols // 32 * 34 if w.fmt == FORMATS["q8_0"] else gguf.nbytes
    w.glu = False
    return w


def requantize_q8_0_host(fmt, rows: int, cols: int, gguf: np.ndarray) -> np.ndarray:
    """rqmv_requantize_q8_0_host: the Q8_0 blocks recipe's int(8) profile stores."""
    gguf = np.ascontiguousarray(gguf).view(np.uint8).reshape(-1)
    out = np.empty(rows * (cols // 32) * 34, np.uint8)
    _check(lib().lib.rqmv_requantize_q8_0_host(_fmt(fmt), rows, cols, gguf.ctypes.data, gguf.nbytes, out.ctypes.data),
           "rqmv_requantize_q8_0_host")
    return out


def contract_int8(weight: Weight, x: np.ndarray, step: int = 32, tail: bool = False) -> np.ndarray:
    """contract() under recipe's int(8) sum: x (K,) or (M, K) float32 -> fp32 (M, N)."""
    x2 = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    m, k = x2.shape
    xb = DeviceBuffer.from_array(x2)
    n = weight.rows * weight.experts
    yb = DeviceBuffer(4 * m * n)
    matvec_int8(weight, xb, m, k, yb, n, step, tail)
    synchronize()
    y = yb.download(np.float32).reshape(m, n)
    return y[0] if x.ndim == 1 else y


def q8_records(x: np.ndarray, step: int = 32):
    """The Q8 records rqmv_matvec_int8 forms for one fp32 row: (d (K/32,), codes int8 (K,))."""
    xs = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    xb = DeviceBuffer.from_array(xs)
    db = DeviceBuffer(4 * (xs.size // 32))
    cb = DeviceBuffer(xs.size)
    _check(lib().lib.rqmv_q8_records(xb.ptr, xs.size, step, db.ptr, cb.ptr, None), "rqmv_q8_records")
    synchronize()
    return db.download(np.float32), cb.download(np.int8)


class MoeParams(ctypes.Structure):
    _fields_ = [("router", c_void_p), ("gate_exps", c_void_p), ("up_exps", c_void_p), ("down_exps", c_void_p),
                ("shared_gate_inp", c_void_p), ("gate_shexp", c_void_p), ("up_shexp", c_void_p),
                ("down_shexp", c_void_p), ("top_k", c_int), ("scoring", c_int), ("renormalize", c_int),
                ("scale", c_float), ("activation", c_int), ("shared_gate_activation", c_int),
                ("activation_factor", c_float), ("selection_bias", c_void_p)]


# recipe's Activation::code() values (recipe.rs:13925-13950), as rqmv_activation
# names them; "gelu_fp16" is Gelu under the llama.cpp profile's gelu table.
ACTIVATIONS = {"linear": 0, "cos": 1, "exp": 2, "log": 3, "ln": 4, "huber": 5, "tan": 6, "relu": 7, "leak": 8,
               "sigmoid": 9, "tanh": 10, "selu": 11, "gelu": 12, "silu": 13, "elu": 14, "prelu": 15, "scale": 16,
               "sqrt": 17, "softplus": 18, "gelu_fp16": 32}


def _act(a) -> int:
    return ACTIVATIONS[a] if isinstance(a, str) else int(a)


class Moe:
    """A gguf_moe block's weights and workspace on the device: gguf_moe(experts,
    top_k, hidden, activation, scoring, renormalize, shared, scale,
    selection_bias) (recipe.rs:14722). The shared expert is absent (no shared
    weights), ungated (shared weights without shared_gate_inp: weight one) or
    gated by shared_gate_activation(shared_gate_inp . x). selection_bias is a
    device buffer of `experts` fp32 values (exp_probs_b.bias) or None."""

    def __init__(self, router: Weight, gate: Weight, up: Weight, down: Weight, top_k: int, scoring: int = SCORE_SOFTMAX,
                 renormalize: bool = True, scale: float = 1.0, shared_gate_inp: Weight | None = None,
                 gate_sh: Weight | None = None, up_sh: Weight | None = None, down_sh: Weight | None = None,
                 activation="silu", shared_gate_activation="sigmoid", activation_factor: float = 0.0,
                 selection_bias: "DeviceBuffer | None" = None):
        h = lambda w: w.handle if w is not None else None  # noqa: E731
        self.params = MoeParams(h(router), h(gate), h(up), h(down), h(shared_gate_inp), h(gate_sh), h(up_sh),
                                h(down_sh), top_k, scoring, 1 if renormalize else 0, scale, _act(activation),
                                _act(shared_gate_activation), activation_factor,
                                selection_bias.ptr if selection_bias is not None else None)
        self.keep = (router, gate, up, down, shared_gate_inp, gate_sh, up_sh, down_sh, selection_bias)
        self.d_model = router.cols
        self.experts = router.rows
        n = c_size_t()
        _check(lib().lib.rqmv_moe_workspace_size(byref(self.params), byref(n)), "rqmv_moe_workspace_size")
        self.workspace = DeviceBuffer(n.value)

    def run(self, x: DeviceBuffer, x_dtype: int, y: DeviceBuffer, route: DeviceBuffer | None = None,
            stream: Stream | None = None):
        _check(lib().lib.rqmv_moe(byref(self.params), x.ptr, x_dtype, y.ptr, route.ptr if route else None,
                                  self.workspace.ptr, self.workspace.nbytes, stream.handle if stream else None),
               "rqmv_moe")

    def run_batch(self, x: DeviceBuffer, x_dtype: int, m: int, ldx: int, y: DeviceBuffer, ldy: int,
                  route: DeviceBuffer | None = None, workspace: DeviceBuffer | None = None,
                  stream: Stream | None = None):
        """m positions (rqmv_moe_batch); the workspace holds m per-position workspaces."""
        if workspace is None:
            workspace = self.batch_workspace(m)
        _check(lib().lib.rqmv_moe_batch(byref(self.params), x.ptr, x_dtype, m, ldx, y.ptr, ldy,
                                        route.ptr if route else None, workspace.ptr, workspace.nbytes,
                                        stream.handle if stream else None), "rqmv_moe_batch")

    def run_batch_noalloc(self, x: DeviceBuffer, x_dtype: int, m: int, ldx: int, y: DeviceBuffer, ldy: int,
                          route: DeviceBuffer | None = None, stream: Stream | None = None):
        """m positions on the library's own per-GPU scratch (rqmv_moe_batch_noalloc):
        no workspace and no allocation; calls on one GPU must not overlap."""
        _check(lib().lib.rqmv_moe_batch_noalloc(byref(self.params), x.ptr, x_dtype, m, ldx, y.ptr, ldy,
                                                route.ptr if route else None, stream.handle if stream else None),
               "rqmv_moe_batch_noalloc")

    def batch_workspace(self, m: int) -> DeviceBuffer:
        return DeviceBuffer(self.workspace.nbytes * m)

    def __call__(self, x: np.ndarray):
        """Host convenience: x (d_model,) or (m, d_model) -> (y fp32, routing weights fp32),
        shaped (d_model,) / (experts,) or (m, d_model) / (m, experts)."""
        x2 = np.atleast_2d(np.ascontiguousarray(x))
        xh, dt = _x_host(x2)
        m = xh.shape[0]
        xb = DeviceBuffer.from_array(xh)
        yb = DeviceBuffer(4 * self.d_model * m)
        rb = DeviceBuffer(4 * self.experts * m)
        if m == 1:
            self.run(xb, dt, yb, rb)
        else:
            self.run_batch(xb, dt, m, self.d_model, yb, self.d_model, rb)
        synchronize()
        y, r = yb.download(np.float32).reshape(m, -1), rb.download(np.float32).reshape(m, -1)
        return (y[0], r[0]) if x.ndim == 1 else (y, r)


def layout_bytes(fmt, rows: int, cols: int) -> int:
    n = c_size_t()
    _check(lib().lib.rqmv_layout_bytes(_fmt(fmt), rows, cols, byref(n)), "rqmv_layout_bytes")
    return n.value


def repack_host(fmt, rows: int, cols: int, gguf: np.ndarray) -> np.ndarray:
    """GGUF bytes -> the kernels' repacked layout, on the host."""
    out = np.zeros(layout_bytes(fmt, rows, cols), np.uint8)
    g = _as_bytes(gguf)
    _check(lib().lib.rqmv_repack_host(_fmt(fmt), rows, cols, g.ctypes.data, out.ctypes.data), "rqmv_repack_host")
    return out


def unpack_host(fmt, rows: int, cols: int, packed: np.ndarray, nbytes: int) -> np.ndarray:
    out = np.zeros(nbytes, np.uint8)
    pk = _as_bytes(packed)
    _check(lib().lib.rqmv_unpack_host(_fmt(fmt), rows, cols, pk.ctypes.data, out.ctypes.data), "rqmv_unpack_host")
    return out


# ------------------------------------------------- decode-step helpers ----
# Thin wrappers of the decode-step entry points (device buffers in and out).

def _sh(stream):
    return stream.handle if stream else None


def add_rmsnorm(x: DeviceBuffer, delta: DeviceBuffer | None, weight: DeviceBuffer, n: int, eps: float,
                out: DeviceBuffer, stream: Stream | None = None, delta_offset: int = 0):
    _check(lib().lib.rqmv_add_rmsnorm(x.ptr, (delta.ptr + delta_offset) if delta else None, weight.ptr, n, eps,
                                      out.ptr, _sh(stream)), "rqmv_add_rmsnorm")


def rope_kv(qkv: DeviceBuffer, pos: DeviceBuffer, q_heads: int, kv_heads: int, head_dim: int, base: float,
            k_cache: DeviceBuffer, v_cache: DeviceBuffer, max_ctx: int, stream: Stream | None = None):
    _check(lib().lib.rqmv_rope_kv(qkv.ptr, pos.ptr, q_heads, kv_heads, head_dim, base, k_cache.ptr, v_cache.ptr,
                                  max_ctx, _sh(stream)), "rqmv_rope_kv")


def attention_workspace_size(q_heads: int, kv_heads: int, head_dim: int, max_ctx: int) -> int:
    n = c_size_t()
    _check(lib().lib.rqmv_attention_workspace_size(q_heads, kv_heads, head_dim, max_ctx, byref(n)),
           "rqmv_attention_workspace_size")
    return n.value


def attention_workspace(q_heads: int, kv_heads: int, head_dim: int, max_ctx: int) -> DeviceBuffer:
    return DeviceBuffer(attention_workspace_size(q_heads, kv_heads, head_dim, max_ctx))


def argmax_workspace() -> DeviceBuffer:
    n = c_size_t()
    _check(lib().lib.rqmv_argmax_workspace_size(byref(n)), "rqmv_argmax_workspace_size")
    return DeviceBuffer(n.value)


def attention(q: DeviceBuffer, k_cache: DeviceBuffer, v_cache: DeviceBuffer, pos: DeviceBuffer, q_heads: int,
              kv_heads: int, head_dim: int, max_ctx: int, workspace: DeviceBuffer, out: DeviceBuffer,
              stream: Stream | None = None):
    _check(lib().lib.rqmv_attention(q.ptr, k_cache.ptr, v_cache.ptr, pos.ptr, q_heads, kv_heads, head_dim, max_ctx,
                                    workspace.ptr, workspace.nbytes, out.ptr, _sh(stream)), "rqmv_attention")


def rope_table(head_dim: int, base: float, rows: int, stream: Stream | None = None) -> DeviceBuffer:
    t = DeviceBuffer(rows * head_dim * 4)
    _check(lib().lib.rqmv_rope_table(t.ptr, head_dim, base, rows, _sh(stream)), "rqmv_rope_table")
    return t


def attention_rope(qkv: DeviceBuffer, table: DeviceBuffer, k_cache: DeviceBuffer, v_cache: DeviceBuffer,
                   pos: DeviceBuffer, q_heads: int, kv_heads: int, head_dim: int, max_ctx: int, workspace: DeviceBuffer,
                   out: DeviceBuffer, stream: Stream | None = None):
    _check(lib().lib.rqmv_attention_rope(qkv.ptr, table.ptr, k_cache.ptr, v_cache.ptr, pos.ptr, q_heads, kv_heads,
                                         head_dim, max_ctx, workspace.ptr, workspace.nbytes, out.ptr, _sh(stream)),
           "rqmv_attention_rope")


def silu_mul(gate_up: DeviceBuffer, n: int, out: DeviceBuffer, stream: Stream | None = None):
    _check(lib().lib.rqmv_silu_mul(gate_up.ptr, n, out.ptr, _sh(stream)), "rqmv_silu_mul")


def argmax(values: DeviceBuffer, n: int, out: DeviceBuffer, workspace: DeviceBuffer, stream: Stream | None = None):
    _check(lib().lib.rqmv_argmax(values.ptr, n, out.ptr, workspace.ptr, workspace.nbytes, _sh(stream)), "rqmv_argmax")


def advance(pos: DeviceBuffer, stream: Stream | None = None):
    _check(lib().lib.rqmv_advance(pos.ptr, _sh(stream)), "rqmv_advance")


def embed_row(table: DeviceBuffer, rows: int, n: int, token: DeviceBuffer, out: DeviceBuffer,
              stream: Stream | None = None):
    _check(lib().lib.rqmv_embed_row(table.ptr, rows, n, token.ptr, out.ptr, _sh(stream)), "rqmv_embed_row")


# ------------------------------------------------------- fused products ----

EPI_PLAIN, EPI_GLU = 0, 1


class Fusion(ctypes.Structure):
    _fields_ = [("norm_weight", c_void_p), ("eps", c_float), ("delta", c_void_p), ("x_out", c_void_p),
                ("epilogue", c_int)]


def glu_weight(fmt, rows: int, cols: int, gate: np.ndarray, up: np.ndarray) -> Weight:
    """A (gate, up) pair as one weight of 2 x rows interleaved rows."""
    g = np.ascontiguousarray(gate).view(np.uint8).reshape(-1)
    u = np.ascontiguousarray(up).view(np.uint8).reshape(-1)
    if g.nbytes != u.nbytes:
        raise ValueError("gate and up differ in size")
    h = c_void_p()
    _check(lib().lib.rqmv_glu_weight_create(_fmt(fmt), rows, cols, g.ctypes.data, u.ctypes.data, g.nbytes, byref(h)),
           "rqmv_glu_weight_create")
    w = Weight.__new__(Weight)
    w.handle = h.value
    w.fmt, w.rows, w.cols, w.experts = _fmt(fmt), 2 * rows, cols, 1
    w.gguf_nbytes = 2 * g.nbytes
    w.glu = True
    return w


def matvec_fused(weight: Weight, x: DeviceBuffer, y: DeviceBuffer, epilogue: int = EPI_PLAIN,
                 norm_weight: DeviceBuffer | None = None, eps: float = 0.0, delta: DeviceBuffer | None = None,
                 x_out: DeviceBuffer | None = None, stream: Stream | None = None):
    f = Fusion(norm_weight.ptr if norm_weight else None, eps, delta.ptr if delta else None,
               x_out.ptr if x_out else None, epilogue)
    _check(lib().lib.rqmv_matvec_fused(weight.handle, x.ptr, y.ptr, byref(f), _sh(stream)), "rqmv_matvec_fused")


# ------------------------------------------------------------ GGUF files ----

GGUF_ARRAY = 9


class GgufTensorInfo:
    def __init__(self, name: str, ggml_type: int, shape: tuple, nbytes: int, index: int):
        self.name, self.ggml_type, self.shape, self.nbytes, self.index = name, ggml_type, shape, nbytes, index

    def __repr__(self):
        return f"GgufTensorInfo({self.name!r}, type={self.ggml_type}, shape={self.shape}, nbytes={self.nbytes})"


class Gguf:
    """A GGUF v3 file (or split model) opened by librqmv's reader (Gguf::open,
    recipe.rs:10069): metadata, tensor descriptors, mapped tensor bytes and
    device weights by tensor name."""

    def __init__(self, path: str):
        h = c_void_p()
        _check(lib().lib.rqmv_gguf_open(os.fsencode(path), byref(h)), "rqmv_gguf_open")
        self.handle = h.value
        n = c_int64()
        _check(lib().lib.rqmv_gguf_tensor_count(self.handle, byref(n)), "rqmv_gguf_tensor_count")
        self._tensors = []
        for i in range(n.value):
            name, ty, nd, nb = c_char_p(), c_int(), c_int(), c_size_t()
            dims = (c_int64 * 8)()
            _check(lib().lib.rqmv_gguf_tensor_info(self.handle, i, byref(name), byref(ty), byref(nd), dims, byref(nb)),
                   "rqmv_gguf_tensor_info")
            self._tensors.append(GgufTensorInfo(name.value.decode(), ty.value, tuple(dims[:nd.value]), nb.value, i))
        self._by_name = {t.name: t for t in self._tensors}

    def tensors(self) -> list:
        return list(self._tensors)

    def tensor(self, name: str) -> GgufTensorInfo | None:
        return self._by_name.get(name)

    def data(self, name: str) -> np.ndarray:
        """The tensor's bytes as stored (a copy out of the mapping)."""
        t = self._by_name[name]
        p, nb = c_void_p(), c_size_t()
        _check(lib().lib.rqmv_gguf_tensor_data(self.handle, t.index, byref(p), byref(nb)), "rqmv_gguf_tensor_data")
        return np.ctypeslib.as_array((ctypes.c_uint8 * nb.value).from_address(p.value)).copy()

    def keys(self) -> list:
        n = c_int64()
        _check(lib().lib.rqmv_gguf_metadata_count(self.handle, byref(n)), "rqmv_gguf_metadata_count")
        out = []
        for i in range(n.value):
            k, ty = c_char_p(), c_int()
            _check(lib().lib.rqmv_gguf_metadata_key(self.handle, i, byref(k), byref(ty)), "rqmv_gguf_metadata_key")
            out.append((k.value.decode(), ty.value))
        return out

    def get_int(self, key: str) -> int:
        v = c_int64()
        _check(lib().lib.rqmv_gguf_get_int(self.handle, key.encode(), byref(v)), "rqmv_gguf_get_int")
        return v.value

    def get_float(self, key: str) -> float:
        v = c_double()
        _check(lib().lib.rqmv_gguf_get_float(self.handle, key.encode(), byref(v)), "rqmv_gguf_get_float")
        return v.value

    def get_string(self, key: str) -> str:
        v = c_char_p()
        _check(lib().lib.rqmv_gguf_get_string(self.handle, key.encode(), byref(v)), "rqmv_gguf_get_string")
        return v.value.decode()

    def get_array(self, key: str) -> list:
        ty, n = c_int(), c_int64()
        _check(lib().lib.rqmv_gguf_get_array(self.handle, key.encode(), byref(ty), byref(n)), "rqmv_gguf_get_array")
        out = []
        for i in range(n.value):
            if ty.value == 8:
                v = c_char_p()
                _check(lib().lib.rqmv_gguf_get_array_string(self.handle, key.encode(), i, byref(v)), "array")
                out.append(v.value.decode())
            else:
                v = c_int64()
                _check(lib().lib.rqmv_gguf_get_array_int(self.handle, key.encode(), i, byref(v)), "array")
                out.append(v.value)
        return out

    def weight(self, name: str) -> Weight:
        """A device weight straight from the mapped tensor ([k, n]: n rows of k;
        [k, n, experts]: an expert bank)."""
        t = self._by_name.get(name)
        h = c_void_p()
        _check(lib().lib.rqmv_gguf_weight_create(self.handle, name.encode(), byref(h)), "rqmv_gguf_weight_create")
        w = Weight.__new__(Weight)
        w.handle = h.value
        w.fmt = t.ggml_type
        w.cols = t.shape[0]
        w.rows = t.shape[1] if len(t.shape) > 1 else 1
        w.experts = t.shape[2] if len(t.shape) > 2 else 1
        w.gguf_nbytes = t.nbytes
        w.glu = False
        return w

    def close(self):
        if self.handle:
            lib().lib.rqmv_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

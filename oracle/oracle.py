"""ctypes wrapper of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the CPU restatement of Stream-PT's quantized MoE
path: the results tests/ and ``__graft_entry__.smoke()`` compare the HIP
library against, and the timed CPU baseline of bench.py.  The product library never imports it.

Every function here wraps one C function of spt_oracle.c; the C file cites the
reference Go source line each one follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


class MoEWeights(C.Structure):
    _fields_ = [
        ("hidden", C.c_int), ("expert_dim", C.c_int), ("experts", C.c_int), ("topk", C.c_int),
        ("router", C.c_void_p), ("router_bias", C.c_void_p), ("router_bias_type", C.c_int),
        ("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
        ("gate_bias", C.c_void_p), ("up_bias", C.c_void_p), ("down_bias", C.c_void_p),
        ("gate_bias_type", C.c_int), ("up_bias_type", C.c_int), ("down_bias_type", C.c_int),
    ]


class MoEDebug(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "logits", "ids", "weights", "counts", "offsets", "list", "active", "n_active",
        "xq", "gate", "up", "act", "actq", "results")]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.so_fp16_to_f32.argtypes = [C.c_uint16]
        L.so_fp16_to_f32.restype = C.c_float
        L.so_f32_to_fp16.argtypes = [C.c_float]
        L.so_f32_to_fp16.restype = C.c_uint16
        L.so_e8m0.argtypes = [C.c_uint8]
        L.so_e8m0.restype = C.c_float
        for n in ("so_mxfp4_decode_row", "so_mxfp4_decode_row_scalar"):
            getattr(L, n).argtypes = [u8p, C.c_int, f32p]
            getattr(L, n).restype = None
        for n in ("so_dot_mxfp4_f32", "so_dot_mxfp4_f32_scalar", "so_dot_q40_f32", "so_dot_q80_f32"):
            getattr(L, n).argtypes = [u8p, f32p, C.c_int]
            getattr(L, n).restype = C.c_float
        L.so_dot_q40_batch_f32.argtypes = [u8p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int]
        L.so_dot_q40_batch_f32.restype = None
        for n in ("so_dot_f32", "so_dot_f32_scalar"):
            getattr(L, n).argtypes = [f32p, f32p, C.c_int]
            getattr(L, n).restype = C.c_float
        L.so_mul_q40_f32.argtypes = [u8p, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int]
        L.so_mul_q40_f32.restype = None
        L.so_mul_q80_f32.argtypes = [u8p, f32p, f32p, C.c_int, C.c_int, C.c_int]
        L.so_mul_q80_f32.restype = None
        L.so_mul_q80_argmax.argtypes = [u8p, f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                        C.POINTER(C.c_int64), C.POINTER(C.c_float)]
        L.so_mul_q80_argmax.restype = None
        L.so_rmsnorm_f32.argtypes = [f32p, f32p, C.c_int, C.c_float, f32p]
        L.so_rmsnorm_f32.restype = None
        L.so_rmsnorm_batch_f32.argtypes = [f32p, f32p, C.c_int, C.c_int, C.c_float, f32p]
        L.so_rmsnorm_batch_f32.restype = None
        L.so_route.argtypes = [f32p, C.c_void_p, f32p, C.c_int, C.c_int, C.c_int, f32p]
        L.so_route.restype = None
        L.so_select.argtypes = [f32p, C.c_int, C.c_int, i32p, f32p]
        L.so_select.restype = None
        L.so_swiglu.argtypes = [C.c_float, C.c_float]
        L.so_swiglu.restype = C.c_float
        L.so_combine.argtypes = [f32p, f32p, C.c_int, C.c_int, C.c_int, f32p]
        L.so_combine.restype = None
        L.so_group.argtypes = [i32p, f32p, C.c_int, C.c_int, C.c_int, i32p, i32p, i32p, i32p, i32p]
        L.so_group.restype = None
        L.so_quantize_q8_0.argtypes = [f32p, C.c_int64, u8p]
        L.so_quantize_q8_0.restype = None
        L.so_isum_mxfp4_q8.argtypes = [u8p, i8p]
        L.so_isum_mxfp4_q8.restype = C.c_int32
        L.so_isum_q40_q8.argtypes = [u8p, i8p]
        L.so_isum_q40_q8.restype = C.c_int32
        for n in ("so_dot_mxfp4_q8", "so_dot_q40_q8"):
            getattr(L, n).argtypes = [u8p, u8p, C.c_int]
            getattr(L, n).restype = C.c_float
        L.so_mul_q40_q8.argtypes = [u8p, f32p, f32p, C.c_int, C.c_int, C.c_int]
        L.so_mul_q40_q8.restype = None
        L.so_mul_mxfp4_q8.argtypes = [u8p, u8p, C.c_void_p, f32p, C.c_int, C.c_int]
        L.so_mul_mxfp4_q8.restype = None
        for n in ("so_forward_moe_batch_f32", "so_forward_moe_batch_q8"):
            getattr(L, n).argtypes = [C.POINTER(MoEWeights), f32p, f32p, C.c_int, C.c_int,
                                      C.POINTER(MoEDebug)]
            getattr(L, n).restype = C.c_int
        _lib = L
    return _lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- codecs ------------------------------------------------------------------

def fp16_to_f32(bits: int) -> float:
    return lib().so_fp16_to_f32(bits)


def f32_to_fp16(value: float) -> int:
    return lib().so_f32_to_fp16(value)


def e8m0(e: int) -> float:
    return lib().so_e8m0(e)


def mxfp4_decode_row(row: np.ndarray, scalar: bool = False) -> np.ndarray:
    row = _c(row, np.uint8)
    nb = row.size // 17
    out = np.empty(nb * 32, np.float32)
    (lib().so_mxfp4_decode_row_scalar if scalar else lib().so_mxfp4_decode_row)(row, nb, out)
    return out


# ---- fp32-activation reference ----------------------------------------------------

def dot_mxfp4_f32(row, x, scalar=False):
    row, x = _c(row, np.uint8), _c(x, np.float32)
    f = lib().so_dot_mxfp4_f32_scalar if scalar else lib().so_dot_mxfp4_f32
    return np.float32(f(row, x, row.size // 17))


def dot_q40_f32(row, x):
    row, x = _c(row, np.uint8), _c(x, np.float32)
    return np.float32(lib().so_dot_q40_f32(row, x, row.size // 18))


def dot_q80_f32(row, x):
    row, x = _c(row, np.uint8), _c(x, np.float32)
    return np.float32(lib().so_dot_q80_f32(row, x, row.size // 34))


def dot_f32(w, x, scalar=False):
    w, x = _c(w, np.float32), _c(x, np.float32)
    f = lib().so_dot_f32_scalar if scalar else lib().so_dot_f32
    return np.float32(f(w, x, x.size))


def mul_q40_f32(w, x, input_dim, output_dim, batch, threads=1):
    w, x = _c(w, np.uint8), _c(x, np.float32)
    y = np.empty(batch * output_dim, np.float32)
    lib().so_mul_q40_f32(w, x, y, input_dim, output_dim, batch, threads)
    return y


def mul_q80_f32(w, x, input_dim, output_dim, threads=1):
    """MulQ80Into numerics: y[row] = quantQ80AVX2(row, x)."""
    w, x = _c(w, np.uint8), _c(x, np.float32)
    y = np.empty(output_dim, np.float32)
    lib().so_mul_q80_f32(w, x, y, input_dim, output_dim, threads)
    return y


def mul_q80_argmax(w, x, input_dim, output_dim, workers=1, window_rows=0):
    """MulQ80Argmax: (best_token, best_logit) with the reference's worker and
    window merge (window_rows 0: one window)."""
    w, x = _c(w, np.uint8), _c(x, np.float32)
    tok, logit = C.c_int64(), C.c_float()
    lib().so_mul_q80_argmax(w, x, input_dim, output_dim, workers, window_rows, C.byref(tok), C.byref(logit))
    return tok.value, np.float32(logit.value)


def rmsnorm_f32(x, w, eps):
    """RMSNormInto numerics (one vector)."""
    x, w = _c(x, np.float32), _c(w, np.float32)
    y = np.empty_like(x)
    lib().so_rmsnorm_f32(x, w, x.size, eps, y)
    return y


def rmsnorm_batch_f32(x, w, batch, eps):
    """normBatch numerics (batch consecutive vectors of len(w))."""
    x, w = _c(x, np.float32), _c(w, np.float32)
    y = np.empty_like(x)
    lib().so_rmsnorm_batch_f32(x, w, w.size, batch, eps, y)
    return y


def decode_norm_weight(raw, typ):
    """F32 (0), F16 (1) or BF16 (28 / 30) vector bytes -> float32."""
    raw = np.ascontiguousarray(raw, np.uint8)
    if typ == 0:
        return raw.view(np.float32).copy()
    h = raw.view(np.uint16)
    if typ == 1:
        return h.view(np.float16).astype(np.float32)
    return (h.astype(np.uint32) << 16).view(np.float32)


def route(router, bias, x, batch, hidden, experts):
    router, x = _c(router, np.float32), _c(x, np.float32)
    logits = np.empty(batch * experts, np.float32)
    b = None
    if bias is not None:
        b = _c(bias, np.float32)
    lib().so_route(router, b.ctypes.data if b is not None else None, x, batch, hidden, experts, logits)
    return logits


def select(logits, k):
    logits = _c(logits, np.float32)
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    lib().so_select(logits, logits.size, k, ids, w)
    return ids, w


def swiglu(gate, up):
    return np.float32(lib().so_swiglu(gate, up))


def combine(results, weights, batch, k, h):
    results, weights = _c(results, np.float32), _c(weights, np.float32)
    out = np.empty(batch * h, np.float32)
    lib().so_combine(results, weights, batch, k, h, out)
    return out


def group(ids, weights, batch, k, experts):
    ids, weights = _c(ids, np.int32), _c(weights, np.float32)
    counts = np.empty(experts, np.int32)
    offsets = np.empty(experts + 1, np.int32)
    lst = np.zeros(max(batch * k, 1), np.int32)
    active = np.zeros(experts, np.int32)
    na = np.zeros(1, np.int32)
    lib().so_group(ids, weights, batch, k, experts, counts, offsets, lst, active, na)
    return counts, offsets, lst[:offsets[-1]], active[:na[0]]


# ---- Q8_0 activation path ------------------------------------------------------------

def quantize_q8_0(x):
    x = _c(x, np.float32).ravel()
    out = np.empty(x.size // 32 * 34, np.uint8)
    lib().so_quantize_q8_0(x, x.size, out)
    return out


def isum_mxfp4_q8(wblk, q):
    return int(lib().so_isum_mxfp4_q8(_c(wblk, np.uint8), _c(q, np.int8)))


def isum_q40_q8(wblk, q):
    return int(lib().so_isum_q40_q8(_c(wblk, np.uint8), _c(q, np.int8)))


def dot_mxfp4_q8(row, xq):
    row, xq = _c(row, np.uint8), _c(xq, np.uint8)
    return np.float32(lib().so_dot_mxfp4_q8(row, xq, row.size // 17))


def dot_q40_q8(row, xq):
    row, xq = _c(row, np.uint8), _c(xq, np.uint8)
    return np.float32(lib().so_dot_q40_q8(row, xq, row.size // 18))


def mul_q40_q8(w, x, input_dim, output_dim, batch):
    w, x = _c(w, np.uint8), _c(x, np.float32)
    y = np.empty(batch * output_dim, np.float32)
    lib().so_mul_q40_q8(w, x, y, input_dim, output_dim, batch)
    return y


def mul_mxfp4_q8(w, xq, bias, input_dim, output_dim):
    w, xq = _c(w, np.uint8), _c(xq, np.uint8)
    y = np.empty(output_dim, np.float32)
    b = _c(bias, np.float32) if bias is not None else None
    lib().so_mul_mxfp4_q8(w, xq, b.ctypes.data if b is not None else None, y, input_dim, output_dim)
    return y


# ---- full layer ----------------------------------------------------------------------------

_BIAS_DTYPE = {0: np.float32, 1: np.uint16, 30: np.uint16}


def forward_moe_batch(layer, x, batch, q8: bool, threads: int = 1, debug: bool = False):
    """Run one MoE layer on the CPU.

    ``layer`` is a dict with keys hidden, expert_dim, experts, topk, router
    (f32 [E*H]), gate/up/down (uint8 expert tensors) and optional router_bias,
    gate_bias, up_bias, down_bias as (array, ggml_type) pairs.
    """
    h, d, E, k = layer["hidden"], layer["expert_dim"], layer["experts"], layer["topk"]
    keep = []

    def ptr(a):
        keep.append(a)
        return a.ctypes.data

    w = MoEWeights()
    w.hidden, w.expert_dim, w.experts, w.topk = h, d, E, k
    w.router = ptr(_c(layer["router"], np.float32))
    for name in ("gate", "up", "down"):
        setattr(w, name, ptr(_c(layer[name], np.uint8)))
    for name in ("router_bias", "gate_bias", "up_bias", "down_bias"):
        b = layer.get(name)
        if b is None:
            setattr(w, name, None)
            setattr(w, name + "_type", 0)
        else:
            arr, typ = b
            setattr(w, name, ptr(_c(arr, _BIAS_DTYPE[typ])))
            setattr(w, name + "_type", typ)
    x = _c(x, np.float32)
    out = np.empty(batch * h, np.float32)
    n = batch * k
    dbg = MoEDebug()
    res = {}
    if debug:
        shapes = {
            "logits": (batch * E, np.float32), "ids": (n, np.int32), "weights": (n, np.float32),
            "counts": (E, np.int32), "offsets": (E + 1, np.int32), "list": (max(n, 1), np.int32),
            "active": (E, np.int32), "n_active": (1, np.int32),
            "xq": (batch * (h // 32) * 34, np.uint8), "gate": (n * d, np.float32),
            "up": (n * d, np.float32), "act": (n * d, np.float32),
            "actq": (n * (d // 32) * 34, np.uint8), "results": (n * h, np.float32),
        }
        for name, (size, dt) in shapes.items():
            res[name] = np.zeros(size, dt)
            setattr(dbg, name, res[name].ctypes.data)
    f = lib().so_forward_moe_batch_q8 if q8 else lib().so_forward_moe_batch_f32
    rc = f(C.byref(w), x, out, batch, threads, C.byref(dbg))
    if rc != 0:
        raise RuntimeError(f"oracle forward_moe_batch failed: {rc}")
    if debug:
        res["list"] = res["list"][: res["offsets"][-1]]
        res["active"] = res["active"][: res["n_active"][0]]
        if not q8:
            del res["xq"], res["actq"]
        return out, res
    return out

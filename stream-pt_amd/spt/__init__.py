"""spt -- Python binding of libspt_moe.so (include/spt_moe.h).

The operator names and argument meanings follow Stream-PT's forward package
(MulQ40Into, MulQ40BatchInto, forwardMoE, forwardMoEBatch, routeMoEBatch,
mulMoEBatchExpert); tensors are passed as device memory (torch tensors on a
ROCm device) plus ggufindex-style descriptors.  Errors raise SptError with
the library's message.  There is no fallback: if the HIP library is missing
the import fails.
"""
from __future__ import annotations

import ctypes as C
import os

__all__ = ["SptError", "Tensor", "MoEConfig", "MoELayer", "MoETaps", "Context", "lib", "LIB_PATH",
           "TYPE_F32", "TYPE_F16", "TYPE_Q4_0", "TYPE_Q8_0", "TYPE_BF16", "TYPE_MXFP4",
           "OK", "ERR_INVALID", "ERR_DEVICE", "ERR_NOMEM", "ERR_CANCELED", "ERR_IO"]

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "libspt_moe.so")

OK, ERR_INVALID, ERR_DEVICE, ERR_NOMEM, ERR_CANCELED, ERR_IO = 0, 1, 2, 3, 4, 5
TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q8_0, TYPE_BF16, TYPE_MXFP4 = 0, 1, 2, 8, 30, 39

EXPORTED = (
    "spt_last_error", "spt_ctx_create", "spt_ctx_destroy", "spt_ctx_synchronize",
    "spt_ctx_set_cancel_flag", "spt_alloc", "spt_free", "spt_copy_h2d", "spt_copy_d2h",
    "spt_tensor_upload", "spt_quantize_q8_0", "spt_mul_q40_into", "spt_mul_q40_batch_into",
    "spt_mul_q40_batch_into_host", "spt_mul_mxfp4_expert", "spt_route_moe_batch",
    "spt_forward_moe", "spt_forward_moe_batch", "spt_forward_moe_batch_ex",
    "spt_forward_moe_batch_host", "spt_block_sums", "spt_synth_mxfp4",
    "spt_ctx_enable_timing", "spt_ctx_read_timing", "spt_ctx_set_gemm_min_group",
    "spt_mul_q80_into", "spt_mul_q80_argmax", "spt_mul_q80_into_host", "spt_mul_q80_argmax_host",
    "spt_rmsnorm_into", "spt_rmsnorm_batch_into", "spt_mul_q40_batch_bias_into",
    "spt_mul_q40_batch_q8_into", "spt_mul_q40_qkv_batch_into", "spt_forward_moe_batch_q8",
    "spt_forward_moe_batch_noalloc", "spt_ctx_set_decode_max_selections", "spt_upload_range", "spt_ctx_memory",
)
KERNEL_KINDS = ("quantize", "route", "gate_up", "down", "combine", "q40", "select", "gate_up_gemm", "down_gemm",
                "q80", "rmsnorm")


class SptError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"spt error {code}: {message}")
        self.code = code
        self.message = message


class Tensor(C.Structure):
    """spt_tensor: ggufindex.Tensor with its HBM-resident bytes."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_uint32), ("n_dims", C.c_uint32),
                ("shape", C.c_uint64 * 4), ("nbytes", C.c_uint64), ("data", C.c_void_p)]

    @classmethod
    def make(cls, name, typ, shape, data_ptr, nbytes):
        t = cls()
        t.name = name.encode() if name else None
        t.type = typ
        t.n_dims = len(shape)
        for i, s in enumerate(shape):
            t.shape[i] = int(s)
        t.nbytes = int(nbytes)
        t.data = int(data_ptr) if data_ptr else None
        return t

    @classmethod
    def absent(cls):
        return cls()


class MoEConfig(C.Structure):
    _fields_ = [("hidden_dim", C.c_int32), ("expert_hidden_dim", C.c_int32),
                ("num_experts", C.c_int32), ("num_experts_used", C.c_int32)]


class MoELayer(C.Structure):
    _fields_ = [(n, Tensor) for n in (
        "ffn_gate_inp", "ffn_gate_inp_bias", "ffn_gate_exps", "ffn_gate_exps_bias",
        "ffn_up_exps", "ffn_up_exps_bias", "ffn_down_exps", "ffn_down_exps_bias")]


class MoETaps(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "logits_in", "logits", "ids", "weights", "counts", "offsets", "list", "active",
        "n_active", "xq", "gate", "up", "act", "actq", "results")]


_lib = None


def lib():
    """Load libspt_moe.so; raise if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
    L = C.CDLL(LIB_PATH)
    vp, i64, i32, u64 = C.c_void_p, C.c_int64, C.c_int32, C.c_uint64
    T = C.POINTER(Tensor)
    sig = {
        "spt_last_error": ([], C.c_char_p),
        "spt_ctx_create": ([C.c_int, vp, C.POINTER(vp)], C.c_int),
        "spt_ctx_destroy": ([vp], C.c_int),
        "spt_ctx_synchronize": ([vp], C.c_int),
        "spt_ctx_set_cancel_flag": ([vp, vp], C.c_int),
        "spt_ctx_set_gemm_min_group": ([vp, i32], C.c_int),
        "spt_ctx_set_decode_max_selections": ([vp, i32], C.c_int),
        "spt_alloc": ([vp, u64, C.POINTER(vp)], C.c_int),
        "spt_free": ([vp, vp], C.c_int),
        "spt_copy_h2d": ([vp, vp, vp, u64], C.c_int),
        "spt_copy_d2h": ([vp, vp, vp, u64], C.c_int),
        "spt_tensor_upload": ([vp, T, vp], C.c_int),
        "spt_quantize_q8_0": ([vp, vp, i64, vp], C.c_int),
        "spt_mul_q40_into": ([vp, T, vp, i64, vp, i64], C.c_int),
        "spt_mul_q40_batch_into": ([vp, T, vp, i64, vp, i64, i64], C.c_int),
        "spt_mul_q40_batch_into_host": ([vp, T, vp, i64, vp, i64, i64], C.c_int),
        "spt_mul_q40_batch_bias_into": ([vp, T, T, vp, i64, vp, i64, i64, vp], C.c_int),
        "spt_mul_q40_batch_q8_into": ([vp, T, T, vp, i64, vp, i64, vp], C.c_int),
        "spt_mul_q40_qkv_batch_into": ([vp, T, T, vp, vp, i64, i64, C.POINTER(vp), C.POINTER(i64)], C.c_int),
        "spt_mul_q80_into": ([vp, T, vp, i64, vp, i64], C.c_int),
        "spt_mul_q80_argmax": ([vp, T, vp, i64, C.POINTER(C.c_int64), C.POINTER(C.c_float)], C.c_int),
        "spt_mul_q80_into_host": ([vp, T, vp, i64, vp, i64], C.c_int),
        "spt_rmsnorm_into": ([vp, T, vp, i64, vp, i64, C.c_float, vp], C.c_int),
        "spt_rmsnorm_batch_into": ([vp, T, vp, i64, vp, i64, i64, C.c_float, vp], C.c_int),
        "spt_mul_q80_argmax_host": ([vp, T, vp, i64, C.POINTER(C.c_int64), C.POINTER(C.c_float)], C.c_int),
        "spt_mul_mxfp4_expert": ([vp, T, T, i32, vp, i64, vp, i64, i64], C.c_int),
        "spt_route_moe_batch": ([vp, T, T, vp, i64, vp], C.c_int),
        "spt_forward_moe": ([vp, C.POINTER(MoEConfig), C.POINTER(MoELayer), vp, i64, vp, i64], C.c_int),
        "spt_forward_moe_batch": ([vp, C.POINTER(MoEConfig), C.POINTER(MoELayer), vp, i64, vp, i64, i64],
                                  C.c_int),
        "spt_forward_moe_batch_ex": ([vp, C.POINTER(MoEConfig), C.POINTER(MoELayer), vp, i64, vp, i64, i64,
                                      C.POINTER(MoETaps)], C.c_int),
        "spt_forward_moe_batch_host": ([vp, C.POINTER(MoEConfig), C.POINTER(MoELayer), vp, i64, vp, i64,
                                        i64], C.c_int),
        "spt_forward_moe_batch_q8": ([vp, C.POINTER(MoEConfig), C.POINTER(MoELayer), vp, vp, i64, vp, i64, i64],
                                     C.c_int),
        "spt_forward_moe_batch_noalloc": ([vp, C.POINTER(MoEConfig), C.POINTER(MoELayer), vp, i64, vp, i64, i64],
                                          C.c_int),
        "spt_block_sums": ([vp, T, i32, vp, i64, vp], C.c_int),
        "spt_synth_mxfp4": ([vp, vp, u64, u64, u64, i32, i32], C.c_int),
        "spt_ctx_enable_timing": ([vp, C.c_int], C.c_int),
        "spt_ctx_read_timing": ([vp, C.POINTER(C.c_double), C.POINTER(C.c_int64)], C.c_int),
        "spt_upload_range": ([vp, C.c_char_p, u64, u64, T], C.c_int),
        "spt_ctx_memory": ([vp, C.POINTER(u64), C.POINTER(u64)], C.c_int),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


def _ptr(t):
    """Device or host address of a torch tensor / numpy array / int / None."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    if hasattr(t, "ctypes"):
        return t.ctypes.data
    raise TypeError(f"cannot take the address of {type(t)}")


def _numel(t):
    if hasattr(t, "numel") and callable(t.numel):
        return int(t.numel())
    return int(t.size)


def _check(rc):
    if rc != OK:
        raise SptError(rc, lib().spt_last_error().decode(errors="replace"))


def _ref(t):
    return C.byref(t) if t is not None else None


class Context:
    """An spt_ctx: one HIP stream, one scratch arena (device=-1: validation
    only)."""

    def __init__(self, device: int = 0, stream=None):
        h = C.c_void_p()
        _check(lib().spt_ctx_create(device, stream, C.byref(h)))
        self.handle = h
        self.device = device
        self._cancel = None

    def close(self):
        if self.handle:
            lib().spt_ctx_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self):
        _check(lib().spt_ctx_synchronize(self.handle))

    def enable_timing(self, enable: bool = True):
        _check(lib().spt_ctx_enable_timing(self.handle, 1 if enable else 0))

    def read_timing(self) -> dict:
        """{kind: (total_ms, launches)} since the last read."""
        ms = (C.c_double * len(KERNEL_KINDS))()
        n = (C.c_int64 * len(KERNEL_KINDS))()
        _check(lib().spt_ctx_read_timing(self.handle, ms, n))
        return {k: (ms[i], n[i]) for i, k in enumerate(KERNEL_KINDS)}

    def memory(self):
        """(arena_bytes, staging_bytes) the context holds."""
        a, b = C.c_uint64(), C.c_uint64()
        _check(lib().spt_ctx_memory(self.handle, C.byref(a), C.byref(b)))
        return a.value, b.value

    def upload_range(self, path, start: int, end: int, name, typ: int, shape) -> Tensor:
        """Bytes [start, end) of the file at path (a ggufindex.Tensor's
        Range) copied to a new device allocation: the resident Tensor (free
        with ctx.free(t.data)).  The name bytes are kept on the Tensor."""
        t = Tensor.make(name, typ, shape, None, 0)
        _check(lib().spt_upload_range(self.handle, os.fspath(path).encode(), int(start), int(end), C.byref(t)))
        return t

    def free(self, dev):
        if dev:
            _check(lib().spt_free(self.handle, dev))

    def set_gemm_min_group(self, min_group: int):
        """Expert groups of at least min_group selections use the grouped
        GEMM, smaller ones the grouped GEMV; 0 restores the default."""
        _check(lib().spt_ctx_set_gemm_min_group(self.handle, int(min_group)))

    def set_decode_max_selections(self, max_selections: int):
        """Batches of up to max_selections selections take the two-launch
        decode path; 0 restores the default, a negative value turns it off."""
        _check(lib().spt_ctx_set_decode_max_selections(self.handle, int(max_selections)))

    def set_cancel_flag(self, flag_array):
        """flag_array: a host int32 numpy array of one element, or None."""
        self._cancel = flag_array
        _check(lib().spt_ctx_set_cancel_flag(self.handle, _ptr(flag_array)))

    # -- operators -----------------------------------------------------------
    def quantize_q8_0(self, x, out):
        _check(lib().spt_quantize_q8_0(self.handle, _ptr(x), _numel(x), _ptr(out)))

    def mul_q40_into(self, w: Tensor, x, y):
        _check(lib().spt_mul_q40_into(self.handle, C.byref(w), _ptr(x), _numel(x), _ptr(y), _numel(y)))

    def mul_q40_batch_into(self, w: Tensor, x, y, batch: int):
        _check(lib().spt_mul_q40_batch_into(self.handle, C.byref(w), _ptr(x), _numel(x), _ptr(y),
                                            _numel(y), batch))

    def mul_q40_batch_bias_into(self, w: Tensor, bias, x, y, batch: int, resid=None):
        b = bias if bias is not None else Tensor.absent()
        _check(lib().spt_mul_q40_batch_bias_into(self.handle, C.byref(w), C.byref(b), _ptr(x), _numel(x), _ptr(y),
                                                 _numel(y), batch, _ptr(resid)))

    def mul_q40_batch_q8_into(self, w: Tensor, bias, xq, y, batch: int, resid=None):
        """MulQ40BatchInto (+ bias, + residual) on an input given as GGML Q8_0
        blocks (a uint8 buffer of batch * in/32 * 34 bytes)."""
        b = bias if bias is not None else Tensor.absent()
        _check(lib().spt_mul_q40_batch_q8_into(self.handle, C.byref(w), C.byref(b), _ptr(xq), batch, _ptr(y),
                                               _numel(y), _ptr(resid)))

    def mul_q40_qkv_batch_into(self, ws, biases, x, ys, batch: int, xq=None, x_len=None):
        """The Q, K, V projections of one input: ws / biases / ys are three
        Tensors / Tensors-or-None / output buffers; the input is the fp32 x
        or, with x None, the GGML Q8_0 blocks xq (x_len elements)."""
        wa = (Tensor * 3)(*ws)
        ba = (Tensor * 3)(*[b if b is not None else Tensor.absent() for b in biases]) if biases else None
        ya = (C.c_void_p * 3)(*[_ptr(y) for y in ys])
        yl = (C.c_int64 * 3)(*[_numel(y) for y in ys])
        n = _numel(x) if x is not None else int(x_len)
        _check(lib().spt_mul_q40_qkv_batch_into(self.handle, wa, ba, _ptr(x), _ptr(xq), n, batch, ya, yl))

    def mul_q40_batch_into_host(self, w: Tensor, x, y, batch: int):
        _check(lib().spt_mul_q40_batch_into_host(self.handle, C.byref(w), _ptr(x), _numel(x), _ptr(y),
                                                 _numel(y), batch))

    def mul_q80_into(self, w: Tensor, x, y):
        _check(lib().spt_mul_q80_into(self.handle, C.byref(w), _ptr(x), _numel(x), _ptr(y), _numel(y)))

    def mul_q80_argmax(self, w: Tensor, x):
        """(best_token, best_logit) of W x (forward.MulQ80Argmax)."""
        tok, logit = C.c_int64(), C.c_float()
        _check(lib().spt_mul_q80_argmax(self.handle, C.byref(w), _ptr(x), _numel(x), C.byref(tok),
                                        C.byref(logit)))
        return tok.value, logit.value

    def mul_q80_into_host(self, w: Tensor, x, y):
        _check(lib().spt_mul_q80_into_host(self.handle, C.byref(w), _ptr(x), _numel(x), _ptr(y), _numel(y)))

    def mul_q80_argmax_host(self, w: Tensor, x):
        tok, logit = C.c_int64(), C.c_float()
        _check(lib().spt_mul_q80_argmax_host(self.handle, C.byref(w), _ptr(x), _numel(x), C.byref(tok),
                                             C.byref(logit)))
        return tok.value, logit.value

    def rmsnorm_into(self, w: Tensor, x, y, eps: float, q8=None):
        _check(lib().spt_rmsnorm_into(self.handle, C.byref(w), _ptr(x), _numel(x), _ptr(y), _numel(y), eps,
                                      _ptr(q8)))

    def rmsnorm_batch_into(self, w: Tensor, x, y, batch: int, eps: float, q8=None):
        _check(lib().spt_rmsnorm_batch_into(self.handle, C.byref(w), _ptr(x), _numel(x), _ptr(y), _numel(y),
                                            batch, eps, _ptr(q8)))

    def mul_mxfp4_expert(self, w: Tensor, bias, expert: int, x, y, batch: int):
        b = bias if bias is not None else Tensor.absent()
        _check(lib().spt_mul_mxfp4_expert(self.handle, C.byref(w), C.byref(b), expert, _ptr(x), _numel(x),
                                          _ptr(y), _numel(y), batch))

    def route_moe_batch(self, router: Tensor, bias, x, batch: int, logits):
        b = bias if bias is not None else Tensor.absent()
        _check(lib().spt_route_moe_batch(self.handle, C.byref(router), C.byref(b), _ptr(x), batch,
                                         _ptr(logits)))

    def forward_moe(self, cfg: MoEConfig, lw: MoELayer, x, out):
        _check(lib().spt_forward_moe(self.handle, _ref(cfg), _ref(lw), _ptr(x), _numel(x), _ptr(out),
                                     _numel(out)))

    def forward_moe_batch(self, cfg: MoEConfig, lw: MoELayer, x, out, batch: int, taps: MoETaps = None):
        if taps is None:
            rc = lib().spt_forward_moe_batch(self.handle, _ref(cfg), _ref(lw), _ptr(x), _numel(x), _ptr(out),
                                             _numel(out), batch)
        else:
            rc = lib().spt_forward_moe_batch_ex(self.handle, _ref(cfg), _ref(lw), _ptr(x), _numel(x),
                                                _ptr(out), _numel(out), batch, C.byref(taps))
        _check(rc)

    def forward_moe_batch_host(self, cfg: MoEConfig, lw: MoELayer, x, out, batch: int):
        _check(lib().spt_forward_moe_batch_host(self.handle, _ref(cfg), _ref(lw), _ptr(x), _numel(x),
                                                _ptr(out), _numel(out), batch))

    def forward_moe_batch_q8(self, cfg: MoEConfig, lw: MoELayer, x, xq, out, batch: int):
        _check(lib().spt_forward_moe_batch_q8(self.handle, _ref(cfg), _ref(lw), _ptr(x), _ptr(xq), _numel(x),
                                              _ptr(out), _numel(out), batch))

    def block_sums(self, w: Tensor, expert: int, xq, rows: int, sums):
        _check(lib().spt_block_sums(self.handle, C.byref(w), expert, _ptr(xq), rows, _ptr(sums)))

    def synth_mxfp4(self, dst, key: int, first_block: int, nblocks: int, scale_lo=118, scale_hi=124):
        _check(lib().spt_synth_mxfp4(self.handle, _ptr(dst), key, first_block, nblocks, scale_lo, scale_hi))


def make_taps(**bufs) -> MoETaps:
    taps = MoETaps()
    for name, t in bufs.items():
        setattr(taps, name, _ptr(t))
    return taps

"""CPU tests of the C ABI: every symbol include/*.h declares is
exported, and argument validation follows the reference's rules (a
validation-only context, device -1, runs every check without a GPU).

Validation cases: tests/testdata/forward/moe_batch_test.go:170-237
(TestForwardMoEBatchValidation) and q40_stream_test.go:107-151."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import spt

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    inc = os.path.join(ROOT, "include")
    text = "".join(open(os.path.join(inc, f)).read() for f in sorted(os.listdir(inc)) if f.endswith(".h"))
    return sorted(set(re.findall(r"\b(spt_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported():
    L = spt.lib()
    declared = _declared()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(L, name), f"{name} not exported"
    assert set(declared) == set(spt.EXPORTED)


@pytest.fixture()
def vctx():
    ctx = spt.Context(-1)
    yield ctx
    ctx.close()


def _moe_descriptors(H=32, D=64, E=4, k=2, biases=True):
    """Descriptors with fake (never dereferenced) device addresses."""
    base = 0x10000000
    lw = spt.MoELayer()
    lw.ffn_gate_inp = spt.Tensor.make("router", spt.TYPE_F32, [H, E], base, H * E * 4)
    lw.ffn_gate_exps = spt.Tensor.make("gate", spt.TYPE_MXFP4, [H, D, E], base, H // 32 * 17 * D * E)
    lw.ffn_up_exps = spt.Tensor.make("up", spt.TYPE_MXFP4, [H, D, E], base, H // 32 * 17 * D * E)
    lw.ffn_down_exps = spt.Tensor.make("down", spt.TYPE_MXFP4, [D, H, E], base, D // 32 * 17 * H * E)
    if biases:
        lw.ffn_gate_inp_bias = spt.Tensor.make("router.bias", spt.TYPE_F32, [E], base, E * 4)
        lw.ffn_gate_exps_bias = spt.Tensor.make("gate.bias", spt.TYPE_F32, [D, E], base, D * E * 4)
        lw.ffn_up_exps_bias = spt.Tensor.make("up.bias", spt.TYPE_F32, [D, E], base, D * E * 4)
        lw.ffn_down_exps_bias = spt.Tensor.make("down.bias", spt.TYPE_F32, [H, E], base, H * E * 4)
    cfg = spt.MoEConfig()
    cfg.hidden_dim, cfg.expert_hidden_dim, cfg.num_experts, cfg.num_experts_used = H, D, E, k
    return cfg, lw


def _call_moe(ctx, cfg, lw, x_ptr, x_len, out_ptr, out_len, batch):
    return spt.lib().spt_forward_moe_batch(ctx.handle if ctx else None, C.byref(cfg) if cfg else None,
                                           C.byref(lw) if lw else None, x_ptr, x_len, out_ptr, out_len, batch)


X, OUT = 0x20000000, 0x30000000


def test_moe_valid_arguments_reach_the_device(vctx):
    cfg, lw = _moe_descriptors()
    rc = _call_moe(vctx, cfg, lw, X, 64, OUT, 64, 2)
    assert rc == spt.ERR_DEVICE and b"validation-only" in spt.lib().spt_last_error()


CASES = {
    "zero hidden": lambda c, w: setattr(c, "hidden_dim", 0),
    "negative expert dimension": lambda c, w: setattr(c, "expert_hidden_dim", -1),
    "unaligned expert dimension": lambda c, w: setattr(c, "expert_hidden_dim", 63),
    "invalid topk": lambda c, w: setattr(c, "num_experts_used", 5),
    "overflow": lambda c, w: setattr(c, "hidden_dim", 2**31 - 1),
    "router type": lambda c, w: setattr(w.ffn_gate_inp, "type", 1),
    "router shape": lambda c, w: setattr(w.ffn_gate_inp, "n_dims", 0),
    "router range": lambda c, w: setattr(w.ffn_gate_inp, "nbytes", w.ffn_gate_inp.nbytes - 1),
    "router alignment": lambda c, w: setattr(w.ffn_gate_inp, "data", w.ffn_gate_inp.data + 2),
    "expert type": lambda c, w: setattr(w.ffn_up_exps, "type", 0),
    "expert shape": lambda c, w: w.ffn_gate_exps.shape.__setitem__(2, 5),
    "expert range": lambda c, w: setattr(w.ffn_down_exps, "nbytes", 0),
    "expert range overflow": lambda c, w: setattr(w.ffn_gate_exps, "nbytes", 2**64 - 8),
    "bias type": lambda c, w: setattr(w.ffn_up_exps_bias, "type", 39),
    "bias shape": lambda c, w: setattr(w.ffn_gate_exps_bias, "n_dims", 0),
    "bias range": lambda c, w: setattr(w.ffn_gate_inp_bias, "nbytes", w.ffn_gate_inp_bias.nbytes - 1),
    "unnamed bias with bytes": lambda c, w: setattr(w.ffn_down_exps_bias, "name", None),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_moe_validation(vctx, case):
    cfg, lw = _moe_descriptors()
    CASES[case](cfg, lw)
    rc = _call_moe(vctx, cfg, lw, X, 64, OUT, 64, 2)
    assert rc == spt.ERR_INVALID, (case, spt.lib().spt_last_error())


@pytest.mark.parametrize("batch", [-1, 0, 1, 2**63 - 1])
def test_moe_batch_validation(vctx, batch):
    cfg, lw = _moe_descriptors()
    assert _call_moe(vctx, cfg, lw, X, 64, OUT, 64, batch) == spt.ERR_INVALID


def test_moe_input_dimension_limit(vctx):
    """The grouped GEMV stages whole rows in LDS: MXFP4 input dimensions up to
    2880 (GPT-OSS) are accepted, larger ones rejected before any launch."""
    cfg, lw = _moe_descriptors(H=2880, D=64)
    assert _call_moe(vctx, cfg, lw, X, 2 * 2880, OUT, 2 * 2880, 2) == spt.ERR_DEVICE
    cfg, lw = _moe_descriptors(H=2912, D=64)
    assert _call_moe(vctx, cfg, lw, X, 2 * 2912, OUT, 2 * 2912, 2) == spt.ERR_INVALID
    assert b"exceeds the supported 2880" in spt.lib().spt_last_error()
    cfg, lw = _moe_descriptors(H=32, D=2912)
    assert _call_moe(vctx, cfg, lw, X, 64, OUT, 64, 2) == spt.ERR_INVALID


def test_moe_nil_and_overlap(vctx):
    cfg, lw = _moe_descriptors()
    assert _call_moe(None, cfg, lw, X, 64, OUT, 64, 2) == spt.ERR_INVALID
    assert _call_moe(vctx, None, lw, X, 64, OUT, 64, 2) == spt.ERR_INVALID
    assert _call_moe(vctx, cfg, None, X, 64, OUT, 64, 2) == spt.ERR_INVALID
    assert _call_moe(vctx, cfg, lw, X, 64, OUT, 63, 2) == spt.ERR_INVALID
    assert _call_moe(vctx, cfg, lw, X, 64, X, 64, 2) == spt.ERR_INVALID
    for xp, op in ((X, X + 4), (X + 4, X)):  # partial overlap either way
        assert _call_moe(vctx, cfg, lw, xp, 64, op, 64, 2) == spt.ERR_INVALID
        assert b"overlap" in spt.lib().spt_last_error()


def test_moe_cancellation_before_launch(vctx):
    cfg, lw = _moe_descriptors()
    flag = np.ones(1, np.int32)
    vctx.set_cancel_flag(flag)
    assert _call_moe(vctx, cfg, lw, X, 64, OUT, 64, 2) == spt.ERR_CANCELED
    flag[0] = 0
    assert _call_moe(vctx, cfg, lw, X, 64, OUT, 64, 2) == spt.ERR_DEVICE
    vctx.set_cancel_flag(None)


def _q40(inp=64, out=3, nbytes=None):
    return spt.Tensor.make("q", spt.TYPE_Q4_0, [inp, out], 0x40000000,
                           inp // 32 * 18 * out if nbytes is None else nbytes)


def _call_q40(ctx, w, x_len, y_len, batch, x=X, y=OUT):
    return spt.lib().spt_mul_q40_batch_into(ctx.handle, C.byref(w), x, x_len, y, y_len, batch)


def test_q40_validation(vctx):
    assert _call_q40(vctx, _q40(), 64, 3, 1) == spt.ERR_DEVICE
    bad = [
        (spt.Tensor.make("q", spt.TYPE_Q8_0, [64, 3], 0x40000000, 2 * 34 * 3), 64, 3, 1, b"instead of Q4_0"),
        (spt.Tensor.make("q", spt.TYPE_Q4_0, [64], 0x40000000, 36), 64, 3, 1, b"two-dimensional"),
        (spt.Tensor.make("q", spt.TYPE_Q4_0, [48, 3], 0x40000000, 36), 48, 3, 1, b"invalid Q4_0 matrix shape"),
        (_q40(nbytes=107), 64, 3, 1, b"byte range"),
        (_q40(), 63, 3, 1, b"expected 64 input and 3 output"),
        (_q40(), 64, 3, 0, b"invalid or oversized batch"),
        (_q40(), 128, 6, -2, b"invalid or oversized batch"),
    ]
    for w, xl, yl, b, msg in bad:
        assert _call_q40(vctx, w, xl, yl, b) == spt.ERR_INVALID
        assert msg in spt.lib().spt_last_error(), spt.lib().spt_last_error()
    assert _call_q40(vctx, _q40(), 64, 3, 1, x=X, y=X + 8) == spt.ERR_INVALID
    assert b"overlap" in spt.lib().spt_last_error()
    # the device GEMV's input limit (131072: one token's Q8_0 in LDS)
    wide = spt.Tensor.make("q", spt.TYPE_Q4_0, [131072, 2], 0x40000000, 131072 // 32 * 18 * 2)
    assert _call_q40(vctx, wide, 131072, 2, 1) == spt.ERR_DEVICE
    wider = spt.Tensor.make("q", spt.TYPE_Q4_0, [131104, 2], 0x40000000, 131104 // 32 * 18 * 2)
    assert _call_q40(vctx, wider, 131104, 2, 1) == spt.ERR_INVALID
    assert b"exceeds the supported 131072" in spt.lib().spt_last_error()


def _q80(inp=64, out=3, nbytes=None, shape=None, typ=None):
    return spt.Tensor.make("output.weight", spt.TYPE_Q8_0 if typ is None else typ,
                           [inp, out] if shape is None else shape, 0x40000000,
                           inp // 32 * 34 * out if nbytes is None else nbytes)


def test_q80_validation(vctx):
    """q80Shape (forward/q80.go:150-171) and the length checks of MulQ80Into
    / MulQ80Argmax (q80.go:37-39,114-116); TestQuantOptimizationQ80ShapeOverflow
    (quant_optimization_test.go:368-374)."""
    L = spt.lib()
    tok, logit = C.c_int64(), C.c_float()

    def into(w, xl, yl, x=X, y=OUT):
        return L.spt_mul_q80_into(vctx.handle, C.byref(w), x, xl, y, yl)

    def argmax(w, xl):
        return L.spt_mul_q80_argmax(vctx.handle, C.byref(w), X, xl, C.byref(tok), C.byref(logit))

    assert into(_q80(), 64, 3) == spt.ERR_DEVICE
    assert argmax(_q80(), 64) == spt.ERR_DEVICE
    bad = [
        (_q80(typ=spt.TYPE_Q4_0), b"instead of Q8_0 (8)"),
        (_q80(shape=[64]), b"expected 2D matrix"),
        (_q80(inp=48, nbytes=34 * 3), b"invalid Q8_0 shape"),
        (_q80(shape=[32, 2 ** 64 - 1], nbytes=34), b"exceed platform limits"),
        (_q80(nbytes=205), b"byte range"),
        (_q80(inp=4128, out=1), b"exceeds the supported 4096"),
    ]
    for w, msg in bad:
        xl = w.shape[0] if w.n_dims >= 1 else 64
        for rc in (into(w, xl, 3), argmax(w, xl)):
            assert rc == spt.ERR_INVALID
            assert msg in L.spt_last_error(), L.spt_last_error()
    assert into(_q80(), 63, 3) == spt.ERR_INVALID
    assert b"expected input/output lengths 64/3, got 63/3" in L.spt_last_error()
    assert into(_q80(), 64, 1) == spt.ERR_INVALID
    assert argmax(_q80(), 32) == spt.ERR_INVALID
    assert b"expected 64 input elements, got 32" in L.spt_last_error()
    assert into(_q80(), 64, 3, x=X, y=X + 8) == spt.ERR_INVALID
    assert b"overlap" in L.spt_last_error()


def test_rmsnorm_validation(vctx):
    """RMSNormInto's checks (forward/rmsnorm.go:21-58, rmsnorm_into_test.go:
    47-60) and normBatch's (layer_batch.go:141-155)."""
    L = spt.lib()

    def norm(typ=0, shape=(5,), nbytes=None):
        width = 4 if typ == 0 else 2
        return spt.Tensor.make("norm", typ, list(shape), 0x40000000, width * 5 if nbytes is None else nbytes)

    def into(w, xl, yl, eps=1e-5, x=X, y=OUT, q8=None):
        return L.spt_rmsnorm_into(vctx.handle, C.byref(w), x, xl, y, yl, eps, q8)

    def batch(w, xl, yl, b, eps=1e-5, x=X, y=OUT):
        return L.spt_rmsnorm_batch_into(vctx.handle, C.byref(w), x, xl, y, yl, b, eps, None)

    for typ in (0, 1, 28):
        assert into(norm(typ), 5, 5) == spt.ERR_DEVICE
        assert into(norm(typ), 5, 5, y=X) == spt.ERR_DEVICE  # in place
        assert batch(norm(typ), 10, 10, 2) == spt.ERR_DEVICE
    cases = [
        (lambda: into(norm(), 5, 5, eps=-1.0), b"invalid epsilon"),
        (lambda: into(norm(), 5, 5, eps=float("nan")), b"invalid epsilon"),
        (lambda: into(norm(), 5, 5, eps=float("inf")), b"invalid epsilon"),
        (lambda: into(norm(), 5, 5, y=X + 4), b"partially overlap"),
        (lambda: into(norm(), 5, 4), b"dimensions differ"),
        (lambda: into(norm(shape=(6,)), 5, 5), b"dimensions differ"),
        (lambda: into(norm(typ=30), 5, 5), b"unsupported normalization weight type 30"),
        (lambda: into(norm(nbytes=19), 5, 5), b"invalid weight data length"),
        (lambda: into(norm(), 5, 5, q8=OUT + 4096), b"multiple of 32"),
        (lambda: batch(norm(), 10, 10, 2, eps=-1.0), b"invalid epsilon"),
        (lambda: batch(norm(typ=30), 10, 10, 2), b"unsupported normalization weight type 30"),
        (lambda: batch(norm(nbytes=19), 10, 10, 2), b"invalid float vector shape or range"),
        (lambda: batch(norm(), 10, 10, 3), b"invalid batch"),
        (lambda: batch(norm(), 10, 12, 2), b"invalid batch"),
    ]
    for call, msg in cases:
        assert call() == spt.ERR_INVALID
        assert msg in L.spt_last_error(), (msg, L.spt_last_error())


def test_q40_bias_validation(vctx):
    """addBias (forward/layer.go:225-242) for one vector, biasBatch /
    readFloatVector (layer_batch.go:124-128, layer.go:279-289) for a batch."""
    L = spt.lib()

    def call(bias, batch=1, resid=None):
        b = bias if bias is not None else spt.Tensor.absent()
        return L.spt_mul_q40_batch_bias_into(vctx.handle, C.byref(_q40()), C.byref(b), X, 64 * batch, OUT,
                                             3 * batch, batch, resid)

    def bias(typ=0, shape=(3,), nbytes=None, name="attn_q.bias"):
        width = 4 if typ == 0 else 2
        return spt.Tensor.make(name, typ, list(shape), 0x50000000, width * 3 if nbytes is None else nbytes)

    assert call(None) == spt.ERR_DEVICE
    assert call(spt.Tensor.make("", 0, [3], 0, 0)) == spt.ERR_DEVICE  # unnamed and empty: absent
    for typ in (0, 1, 30):
        assert call(bias(typ)) == spt.ERR_DEVICE
        assert call(bias(typ), batch=2) == spt.ERR_DEVICE
    assert call(bias(), resid=0x60000000) == spt.ERR_DEVICE
    cases = [
        (lambda: call(bias(nbytes=0)), b"invalid bias range"),
        (lambda: call(bias(nbytes=0), batch=2), b"invalid float vector shape or range"),
        (lambda: call(bias(typ=8)), b"unsupported float tensor type 8"),
        (lambda: call(bias(shape=(4,))), b"invalid float vector shape or range"),
        (lambda: call(bias(nbytes=11)), b"invalid float vector shape or range"),
        (lambda: call(bias(), resid=X), b"residual overlaps"),
        (lambda: call(bias(), resid=OUT + 4), b"residual overlaps"),
    ]
    for fn, msg in cases:
        assert fn() == spt.ERR_INVALID
        assert msg in L.spt_last_error(), (msg, L.spt_last_error())


def test_quantize_validation(vctx):
    L = spt.lib()
    assert L.spt_quantize_q8_0(vctx.handle, X, 33, OUT) == spt.ERR_INVALID
    assert L.spt_quantize_q8_0(vctx.handle, X, 64, X + 4) == spt.ERR_INVALID
    assert L.spt_quantize_q8_0(vctx.handle, X, 64, OUT) == spt.ERR_DEVICE


def test_gemm_min_group_setting(vctx):
    L = spt.lib()
    assert L.spt_ctx_set_gemm_min_group(vctx.handle, -1) == spt.ERR_INVALID
    assert b"negative" in L.spt_last_error()
    for v in (0, 1, 9, 1 << 30):
        assert L.spt_ctx_set_gemm_min_group(vctx.handle, v) == spt.OK
    assert L.spt_ctx_set_gemm_min_group(None, 1) == spt.ERR_INVALID


def _call_moe_single(ctx, cfg, lw, x_ptr, x_len, out_ptr, out_len):
    return spt.lib().spt_forward_moe(ctx.handle, C.byref(cfg), C.byref(lw), x_ptr, x_len, out_ptr, out_len)


@pytest.mark.parametrize("which", ["ffn_gate_exps_bias", "ffn_up_exps_bias", "ffn_down_exps_bias"])
def test_forward_moe_unnamed_expert_bias_disabled(vctx, which):
    """forwardMoE (forward/moe.go:57-62) replaces an expert bias with an empty
    name by the absent tensor before validating, so an unnamed descriptor
    that still carries a byte range runs there; forwardMoEBatch rejects it
    (moe_batch.go:196-200)."""
    cfg, lw = _moe_descriptors()
    t = getattr(lw, which)
    t.name = None  # unnamed, nbytes and data left as they were
    rc = _call_moe_single(vctx, cfg, lw, X, 32, OUT, 32)
    assert rc == spt.ERR_DEVICE and b"validation-only" in spt.lib().spt_last_error()
    rc = _call_moe(vctx, cfg, lw, X, 32, OUT, 32, 1)
    assert rc == spt.ERR_INVALID and b"unnamed MoE bias has nonempty range" in spt.lib().spt_last_error()
    t.name = b""  # an empty string is unnamed too
    assert _call_moe_single(vctx, cfg, lw, X, 32, OUT, 32) == spt.ERR_DEVICE
    assert getattr(lw, which).nbytes != 0  # the caller's descriptor is not modified


def test_forward_moe_unnamed_router_bias_still_checked(vctx):
    """The router bias is not cleared by forwardMoE: an unnamed one with a
    byte range fails through both entry points."""
    cfg, lw = _moe_descriptors()
    lw.ffn_gate_inp_bias.name = None
    assert _call_moe_single(vctx, cfg, lw, X, 32, OUT, 32) == spt.ERR_INVALID
    assert b"unnamed MoE bias has nonempty range" in spt.lib().spt_last_error()


def test_moe_large_batches_run_as_slices(vctx):
    """More than 4096 selections: the plain, host and Q8_0-input forms accept
    the batch (it runs as slices of whole tokens; the validation-only
    context stops at the device), the tapped form refuses it, and the
    experts-used and expert-count limits hold."""
    H, k = 32, 2
    cfg, lw = _moe_descriptors(H=H, k=k)
    batch = 4096 // k + 1
    n = batch * H
    assert _call_moe(vctx, cfg, lw, X, n, OUT, n, batch) == spt.ERR_DEVICE
    x = np.zeros(n, np.float32)
    out = np.zeros(n, np.float32)
    rc = spt.lib().spt_forward_moe_batch_host(vctx.handle, C.byref(cfg), C.byref(lw), x.ctypes.data, n,
                                              out.ctypes.data, n, batch)
    assert rc == spt.ERR_DEVICE
    rc = spt.lib().spt_forward_moe_batch_q8(vctx.handle, C.byref(cfg), C.byref(lw), X, 0x40000000, n, OUT, n,
                                            batch)
    assert rc == spt.ERR_DEVICE
    taps = spt.MoETaps()
    rc = spt.lib().spt_forward_moe_batch_ex(vctx.handle, C.byref(cfg), C.byref(lw), X, n, OUT, n, batch,
                                            C.byref(taps))
    assert rc == spt.ERR_INVALID and b"4096" in spt.lib().spt_last_error()
    rc = spt.lib().spt_forward_moe_batch_ex(vctx.handle, C.byref(cfg), C.byref(lw), X, n - H, OUT, n - H,
                                            batch - 1, C.byref(taps))
    assert rc == spt.ERR_DEVICE
    for E, kk in ((257, 2), (32, 17)):
        cfg, lw = _moe_descriptors(H=H, E=E, k=kk)
        assert _call_moe(vctx, cfg, lw, X, 2 * H, OUT, 2 * H, 2) == spt.ERR_INVALID
        assert b"experts used <= 16, experts <= 256" in spt.lib().spt_last_error()


def test_route_router_alignment(vctx):
    """spt_route_moe_batch rejects a router whose F32 data is not 4-byte
    aligned before any launch; an aligned one reaches the device."""
    rt = spt.Tensor.make("router", spt.TYPE_F32, [32, 4], 0x10000000, 32 * 4 * 4)
    none = spt.Tensor.absent()
    lib = spt.lib()
    assert lib.spt_route_moe_batch(vctx.handle, C.byref(rt), C.byref(none), X, 1, OUT) == spt.ERR_DEVICE
    rt = spt.Tensor.make("router", spt.TYPE_F32, [32, 4], 0x10000002, 32 * 4 * 4)
    assert lib.spt_route_moe_batch(vctx.handle, C.byref(rt), C.byref(none), X, 1, OUT) == spt.ERR_INVALID
    assert b"4-byte aligned" in lib.spt_last_error()

"""Pin the oracle's MoE layer (fp32-activation restatement of
forwardMoEBatch) and the Q8_0 activation path.

Reference tests restated:
  TestForwardMoEBatchMatchesSequential  moe_batch_test.go:125-168 (bit identity)
  TestSparseMoEIndependentReference     moe_sparse_test.go:18-105 (float64, 3e-5)
  TestSparseMoESelectedWeightBytes      moe_sparse_test.go:128-181 (experts touched)
  TestSparseMoEReversedProjectionLayout moe_sparse_test.go:183-199
  TestGPTOSSExpertBiasesAndSwiGLU       inference_regression_test.go:44-103 (closed form)
The Q8_0 quantizer (no reference function; GGML's quantize_row_q8_0
reference rule) is pinned against an independent numpy statement and its
defining properties; the integer block sums against numpy int64 dots; the
Q8_0 row dot against float64 over the dequantized operands.
"""
import math

import numpy as np
import pytest

from fixtures import ROUTER_MODES, moe_batch_fixture, moe_batch_x
from helpers import tie_block

LEVELS64 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, 0, -.5, -1, -1.5, -2, -3, -4, -6], np.float64)


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    nan = np.isnan(a)
    return np.array_equal(nan, np.isnan(b)) and np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32))


@pytest.mark.parametrize("experts", [1, 4, 7])
@pytest.mark.parametrize("bias_type", [-1, 0, 1, 30])
def test_batch_matches_sequential(O, experts, bias_type):
    for topk in sorted({1, min(2, experts), experts}):
        for mode in ROUTER_MODES:
            lay = moe_batch_fixture(96, 64, experts, topk, bias_type, mode)
            for batch in (1, 5, 37):
                x = moe_batch_x(batch, 96, mode)
                got = O.forward_moe_batch(lay, x, batch, q8=False, threads=3)
                want = np.concatenate([O.forward_moe_batch(lay, x[t * 96:(t + 1) * 96], 1, q8=False)
                                       for t in range(batch)])
                assert _same(got, want), (experts, topk, bias_type, mode, batch)


def _mxfp4_matrix64(buf, expert, rows, input_dim):
    nb = input_dim // 32
    enc = buf[expert * rows * nb * 17:(expert + 1) * rows * nb * 17].reshape(rows, nb, 17)
    scale = np.ldexp(1.0, enc[:, :, 0].astype(np.int64) - 127)
    lo, hi = LEVELS64[enc[:, :, 1:] & 15], LEVELS64[enc[:, :, 1:] >> 4]
    w = np.concatenate([lo, hi], axis=2) * scale[:, :, None]
    return w.reshape(rows, input_dim)


def scalar_sparse_moe(lay, x):
    """moe_sparse_test.go:18-76 in numpy float64 (no biases)."""
    H, D, E, k = lay["hidden"], lay["expert_dim"], lay["experts"], lay["topk"]
    router = lay["router"].astype(np.float64).reshape(E, H)
    logits = router @ x.astype(np.float64)
    order = sorted(range(E), key=lambda e: -logits[e])[:k]  # stable, like sort.SliceStable
    weights = np.array([math.exp(logits[e] - logits[order[0]]) for e in order])
    total = weights.sum()
    result = np.zeros(H, np.float32)
    for rank, e in enumerate(order):
        gate = _mxfp4_matrix64(lay["gate"], e, D, H) @ x.astype(np.float64)
        up = _mxfp4_matrix64(lay["up"], e, D, H) @ x.astype(np.float64)
        g, u = np.minimum(gate, 7), np.maximum(-7, np.minimum(up, 7))
        act = g / (1 + np.exp(-1.702 * g)) * (u + 1)
        down = _mxfp4_matrix64(lay["down"], e, H, D) @ act
        result += (down * weights[rank] / total).astype(np.float32)
    return result


@pytest.mark.parametrize("mode", ["ties", "normal", "underflow"])
@pytest.mark.parametrize("k", [1, 2, 8])
def test_sparse_moe_independent_reference(O, mode, k):
    lay = moe_batch_fixture(96, 64, 8, k, -1, mode)
    batch = 19
    x = (((np.arange(batch * 96) % 13) + 1) / 16).astype(np.float32)
    out = O.forward_moe_batch(lay, x, batch, q8=False, threads=4).reshape(batch, 96)
    for t in range(batch):
        want = scalar_sparse_moe(lay, x[t * 96:(t + 1) * 96])
        assert np.all(np.abs(out[t] - want) <= 3e-5 * np.maximum(1, np.abs(want))), (t,)


@pytest.mark.parametrize("batch", [1, 23])
@pytest.mark.parametrize("mode,experts_touched", [("ties", [0, 1]), ("underflow", [7]), ("nonfinite", [0, 1])])
def test_selected_experts(O, batch, mode, experts_touched):
    lay = moe_batch_fixture(64, 64, 8, 2, -1, mode)
    x = np.full(batch * 64, 0.5, np.float32)
    _, dbg = O.forward_moe_batch(lay, x, batch, q8=False, debug=True)
    assert list(dbg["active"]) == experts_touched


def test_reversed_projection_layout(O):
    lay = moe_batch_fixture(64, 64, 8, 2, -1, "ties")
    lay["gate"], lay["up"] = lay["up"], lay["gate"]
    x = (((np.arange(64) % 7) - 3) / 16).astype(np.float32)
    out = O.forward_moe_batch(lay, x, 1, q8=False)
    want = scalar_sparse_moe(lay, x)
    assert np.all(np.abs(out - want) <= 3e-5 * np.maximum(1, np.abs(want)))


def _swiglu_fixture():
    dim, experts = 32, 2
    zero = np.zeros((experts * dim, 17), np.uint8)
    zero[:, 0] = 127
    down = zero.copy()
    down[:, 1] = 2  # first coefficient 1.0
    bias = lambda v: (np.concatenate([np.zeros(dim, np.float32), np.full(dim, v, np.float32)]), 0)
    return {"hidden": dim, "expert_dim": dim, "experts": experts, "topk": 1,
            "router": np.zeros(dim * experts, np.float32), "router_bias": (np.float32([0, 1]), 0),
            "gate": zero.reshape(-1), "up": zero.reshape(-1).copy(), "down": down.reshape(-1),
            "gate_bias": bias(10), "up_bias": bias(12), "down_bias": bias(5)}


def test_expert_biases_and_swiglu_closed_form(O):
    lay = _swiglu_fixture()
    want = 7 / (1 + math.exp(-1.702 * 7)) * 8 + 5
    out = O.forward_moe_batch(lay, np.zeros(32, np.float32), 1, q8=False)
    assert np.all(np.abs(out - want) <= 1e-5)
    out8 = O.forward_moe_batch(lay, np.zeros(32, np.float32), 1, q8=True)
    assert np.all(np.abs(out8 - want) <= 1e-3 * want)


def test_swiglu_go_semantics(O):
    # min/max propagate NaN; clamps at +-7 on up, +7 on gate
    assert np.isnan(O.swiglu(np.nan, 1.0)) and np.isnan(O.swiglu(1.0, np.nan))
    assert O.swiglu(100.0, -100.0) == np.float32(7 / (1 + math.exp(-1.702 * 7)) * -6)
    g = np.float32(0.5)
    want = np.float32(g / (np.float32(1) + np.float32(math.exp(float(np.float32(-1.702) * g))))) * np.float32(3)
    assert O.swiglu(0.5, 2.0) == want


# ---- Q8_0 path -------------------------------------------------------------------

def q8_numpy(x):
    """Independent numpy statement of GGML's quantize_row_q8_0 reference."""
    x = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.max(np.abs(x), axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    v = (x * idv[:, None]).astype(np.float32).astype(np.float64)
    q = np.sign(v) * np.floor(np.abs(v) + 0.5)
    out = np.zeros((x.shape[0], 34), np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def test_quantize_q8_0_matches_numpy_statement(O):
    from spt import synth

    for scale in (1e-3, 1.0, 3e3):
        x = synth.normal(synth.stream_key(31, int(scale * 7)), 32 * 4096) * np.float32(scale)
        assert np.array_equal(O.quantize_q8_0(x), q8_numpy(x))


def test_quantize_q8_0_properties(O):
    from spt import synth

    x = synth.normal(synth.stream_key(32, 0), 32 * 2048)
    q = O.quantize_q8_0(x).reshape(-1, 34)
    codes = q[:, 2:].view(np.int8).astype(np.int32)
    d = q[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    assert np.all(np.abs(codes) <= 127)
    assert np.all(np.max(np.abs(codes), axis=1) == 127)  # the amax element maps to +-127
    # codes come from the fp32 1/d, the stored scale is fp16(d): the
    # reconstruction error is half a step plus 127 * |fp16(d) - d|
    err = np.abs(codes * d[:, None] - x.reshape(-1, 32))
    assert np.all(err <= d[:, None] * (0.5 * (1 + 1e-3) + 127 * 2.0 ** -11) + 1e-7)
    # amax 127 gives d = 1 and id = 1 exactly, so every x * id below is an
    # exact .5 tie, where half-away-from-zero (GGML roundf) and half-even
    # (rint) disagree
    ties = tie_block()
    qt = O.quantize_q8_0(ties).reshape(34)
    assert qt[0] == 0x00 and qt[1] == 0x3C  # fp16(1.0)
    want = (np.sign(ties) * np.floor(np.abs(ties) + 0.5)).astype(np.int8)
    assert np.array_equal(qt[2:].view(np.int8), want)
    assert not np.array_equal(want, np.rint(ties).astype(np.int8))  # the rule is pinned
    z = O.quantize_q8_0(np.zeros(32, np.float32))
    assert np.all(z == 0)
    nan = np.zeros(32, np.float32)
    nan[3] = np.nan
    qn = O.quantize_q8_0(nan)
    assert qn[0] == 0x00 and qn[1] == 0x7E and np.all(qn[2:] == 0)


def test_isum_against_numpy(O):
    from spt import synth

    LUT2 = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.int64)
    w = synth.mxfp4_expert_bytes(synth.stream_key(33, 0), 0, 2000).reshape(-1, 17)
    q4 = synth.q40_bytes(synth.stream_key(34, 0), 1, 64000).reshape(-1, 18)
    rng = np.random.default_rng(1)
    q = rng.integers(-127, 128, size=(2000, 32)).astype(np.int8)
    for b in range(2000):
        wi = np.concatenate([LUT2[w[b, 1:] & 15], LUT2[w[b, 1:] >> 4]])
        assert O.isum_mxfp4_q8(w[b], q[b]) == int(np.dot(wi, q[b].astype(np.int64)))
        qi = np.concatenate([(q4[b, 2:] & 15).astype(np.int64) - 8, (q4[b, 2:] >> 4).astype(np.int64) - 8])
        assert O.isum_q40_q8(q4[b], q[b]) == int(np.dot(qi, q[b].astype(np.int64)))
    # extremes: |isum| <= 32*12*127 and 32*8*127
    big = np.full(17, 0x77, np.uint8)
    assert O.isum_mxfp4_q8(big, np.full(32, 127, np.int8)) == 32 * 12 * 127
    neg = np.zeros(18, np.uint8)
    assert O.isum_q40_q8(neg, np.full(32, 127, np.int8)) == -8 * 32 * 127


def test_q8_dots_against_float64(O):
    """The Q8_0 row dots equal float64 sums over the dequantized operands up
    to fp32 accumulation rounding (pins scale = E8M0/2 for LUT2 and d_w*d_x
    for Q4_0)."""
    from spt import synth

    for input_dim in (32, 2880, 4096):
        nb = input_dim // 32
        x = synth.normal(synth.stream_key(35, input_dim), input_dim)
        xq = O.quantize_q8_0(x).reshape(nb, 34)
        dx = xq[:, :2].copy().view(np.float16).astype(np.float64).ravel()
        codes = xq[:, 2:].view(np.int8).astype(np.float64)
        xdeq = (codes * dx[:, None]).ravel()
        mx = synth.mxfp4_expert_bytes(synth.stream_key(36, input_dim), 0, 8 * nb)
        q4 = synth.q40_bytes(synth.stream_key(37, input_dim), 8, input_dim)
        for r in range(8):
            row = mx[r * nb * 17:(r + 1) * nb * 17]
            want = _mxfp4_matrix64(row, 0, 1, input_dim)[0] @ xdeq
            got = O.dot_mxfp4_q8(row, xq.reshape(-1))
            mag = np.abs(_mxfp4_matrix64(row, 0, 1, input_dim)[0]) @ np.abs(xdeq)
            assert abs(got - want) <= 1e-6 * mag, (input_dim, r)
            row4 = q4[r * nb * 18:(r + 1) * nb * 18].reshape(nb, 18)
            dw = row4[:, :2].copy().view(np.float16).astype(np.float64).ravel()
            wq = np.concatenate([(row4[:, 2:] & 15).astype(np.int64) - 8, (row4[:, 2:] >> 4).astype(np.int64) - 8], 1)
            w64 = (wq * dw[:, None]).ravel()
            got4 = O.dot_q40_q8(row4.reshape(-1), xq.reshape(-1))
            assert abs(got4 - w64 @ xdeq) <= 1e-6 * (np.abs(w64) @ np.abs(xdeq)), (input_dim, r)


def test_q8_layer_close_to_fp32_reference(O):
    """Q8_0 activations move a GPT-OSS-shape layer by ~1% of its output
    scale: the documented deviation from the fp32-activation reference."""
    from spt import workloads as W

    shp = W.MoEShape()
    x = W.x_tokens(0, 0, 1, shp.hidden)
    small = W.host_small_tensors(0, 0, shp)
    ids, _ = O.select(O.route(small["router"], small["router_bias"], x, 1, shp.hidden, shp.experts), shp.topk)
    lay = W.host_layer(0, 0, shp, experts=ids)
    o8 = O.forward_moe_batch(lay, x, 1, q8=True, threads=8)
    of = O.forward_moe_batch(lay, x, 1, q8=False, threads=8)
    dev = np.max(np.abs(o8 - of)) / np.max(np.abs(of))
    assert 1e-4 < dev < 5e-2, dev

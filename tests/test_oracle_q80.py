"""Pin the oracle's LM-head restatement (MulQ80Into / MulQ80Argmax) against
the reference's own tests and float64 brute force.

  TestQuantOptimizationArgmaxWindowAndTies  quant_optimization_test.go:180-219
  TestQuantOptimizationNumerics (argmax)    quant_optimization_test.go:127-177
  TestMulQ80Into                            sampling_test.go:179-208
  worker-pool argmax                        worker_pool_test.go:160-200

The special-value cases (NaN, +-Inf rows) are worked out by hand from the
comparisons of forward/q80.go:64-99: a worker starts from (its first row,
-Inf) and keeps strict maxima, the windows merge into (0, -Inf) by a larger
logit or an equal one with a lower token.
"""
import numpy as np
import pytest

from fixtures import quant_optimization_fixture

WORKERS = (1, 4, 100)
WINDOWS = (1, 4, 8, 17)


def _first_max(y):
    """The reference tests' expectation: best = 0; for i: if y[i] > y[best]."""
    best = 0
    for i in range(len(y)):
        if y[i] > y[best]:
            best = i
    return best


def test_argmax_window_and_ties(O):
    data = quant_optimization_fixture(8, 32, 17)
    x = np.zeros(32, np.float32)
    for workers in WORKERS:
        for rows in WINDOWS:
            tok, logit = O.mul_q80_argmax(data, x, 32, 17, workers, rows)
            assert (tok, logit) == (0, np.float32(0.0))
    data = np.zeros(17 * 34, np.uint8)
    for row in range(17):
        data[row * 34:row * 34 + 2] = (0x00, 0x3C)
    for row in (3, 4, 8, 16):
        data[row * 34 + 2] = 1
    x[0] = 7
    for workers in WORKERS:
        for rows in WINDOWS:
            assert O.mul_q80_argmax(data, x, 32, 17, workers, rows) == (3, np.float32(7.0))


@pytest.mark.parametrize("input_dim", [32, 96, 512])
def test_argmax_matches_first_max(O, input_dim):
    data = quant_optimization_fixture(8, input_dim, 17)
    x = ((np.arange(input_dim) % 23) - 11).astype(np.float32) / 32
    y = O.mul_q80_f32(data, x, input_dim, 17)
    best = _first_max(y)
    for workers in WORKERS:
        for rows in WINDOWS:
            tok, logit = O.mul_q80_argmax(data, x, input_dim, 17, workers, rows)
            assert tok == best and logit.view(np.uint32) == y[best].view(np.uint32)


def test_mul_q80_into(O):
    data = quant_optimization_fixture(8, 96, 17)
    x = ((np.arange(96) % 7) - 3).astype(np.float32) / 8
    y = O.mul_q80_f32(data, x, 96, 17)
    enc = data.reshape(17, 3, 34)
    d = enc[:, :, 0:2].copy().view(np.uint16)[..., 0].view(np.float16).astype(np.float64)
    q = enc[:, :, 2:].view(np.int8).astype(np.float64)
    want = np.sum(d[:, :, None] * q * x.astype(np.float64).reshape(3, 32)[None], axis=(1, 2))
    assert np.all(np.abs(y - want) <= 1e-4 * (1 + np.abs(want)))
    for row in range(17):
        assert y[row].view(np.uint32) == O.dot_q80_f32(data[row * 102:(row + 1) * 102], x).view(np.uint32)


def test_mul_q80_float64_at_lm_head_width(O):
    from spt import synth

    rows, input_dim = 64, 2880
    w = synth.q80_bytes(synth.stream_key(30, 1), rows, input_dim)
    x = synth.normal(synth.stream_key(31, 1), input_dim)
    y = O.mul_q80_f32(w, x, input_dim, rows, threads=4)
    enc = w.reshape(rows, 90, 34)
    d = enc[:, :, 0:2].copy().view(np.uint16)[..., 0].view(np.float16).astype(np.float64)
    q = enc[:, :, 2:].view(np.int8).astype(np.float64)
    want = np.sum(d[:, :, None] * q * x.astype(np.float64).reshape(90, 32)[None], axis=(1, 2))
    scale = np.sum(np.abs(d[:, :, None] * q * x.astype(np.float64).reshape(90, 32)[None]), axis=(1, 2))
    assert np.all(np.abs(y - want) <= 1e-5 * scale)


def _rows_with_logits(values):
    """Q8_0 rows over 32 inputs of ones whose logits are exactly `values`:
    finite v -> scale fp16(v) (v exact in fp16) with q = (1, 0, ..., 0);
    +-Inf -> scale +-Inf with every q = 1; NaN -> a NaN scale."""
    data = np.zeros((len(values), 34), np.uint8)
    for r, v in enumerate(values):
        if np.isnan(v):
            data[r, 0:2] = np.frombuffer(np.uint16(0x7E00).tobytes(), np.uint8)
            data[r, 2:] = 1
        elif np.isinf(v):
            bits = 0x7C00 if v > 0 else 0xFC00
            data[r, 0:2] = np.frombuffer(np.uint16(bits).tobytes(), np.uint8)
            data[r, 2:] = 1
        else:
            h = np.float16(v)
            assert float(h) == v
            data[r, 0:2] = np.array([h], np.float16).view(np.uint8)
            data[r, 2] = 1
    return data.reshape(-1)


SPECIAL = [
    ([np.nan, 1, 3, 3, 2], 2, 3.0),
    ([np.nan, np.nan], 0, -np.inf),
    ([-np.inf, -np.inf, -np.inf], 0, -np.inf),
    ([np.nan, -np.inf, 5], 2, 5.0),
    ([1, np.inf, np.inf, np.nan], 1, np.inf),
    ([-np.inf, np.nan, -2], 2, -2.0),
    ([-4, -4, np.nan, -4], 0, -4.0),
]


@pytest.mark.parametrize("values,token,logit", SPECIAL)
def test_argmax_special_values(O, values, token, logit):
    data = _rows_with_logits(values)
    x = np.ones(32, np.float32)
    y = O.mul_q80_f32(data, x, 32, len(values))
    for v, got in zip(values, y):
        assert (np.isnan(v) and np.isnan(got)) or got == v
    for workers in (1, 2, 3):
        for rows in (1, 2, len(values)):
            assert O.mul_q80_argmax(data, x, 32, len(values), workers, rows) == (token, np.float32(logit))

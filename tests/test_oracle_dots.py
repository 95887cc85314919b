"""Pin the oracle's fp32-activation dot products against the reference's
known answers and float64 brute force, and the scalar lane-by-lane
restatements against the AVX2 ones (same bits).

Fixtures restate the reference tests' formulas:
  TestDotQ40 / TestDotQ40TwoBlocks      q40_test.go:12-51
  TestQ80Dot / TestMXFP4Dot             pipeline_test.go:146-201
  TestMXFP4AllScales                    mxfp4_optimization_test.go:52-78
  TestMXFP4NibbleReference              mxfp4_optimization_test.go:12-50
  TestSIMDKernelGather                  simd_kernels_test.go:13-72
  TestSIMDKernelRouter                  simd_kernels_test.go:99-153
  TestQuantOptimizationFloat16Scales    quant_optimization_test.go:69-113
  TestQuantOptimizationNumerics         quant_optimization_test.go:25-56,127-177
"""
import math

import numpy as np
import pytest

from fixtures import quant_optimization_fixture

LEVELS64 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, 0, -.5, -1, -1.5, -2, -3, -4, -6], np.float64)


def _tol(got, want, rel=3e-5):
    return abs(float(got) - float(want)) <= rel * max(1.0, abs(float(want)))


def test_dot_q40_known_answers(O):
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    blk[2] = 0x0F
    x = np.zeros(32, np.float32)
    x[0], x[16] = 2, 3
    assert O.dot_q40_f32(blk, x) == np.float32(7 * 2 - 8 * 3)
    row = np.zeros(36, np.uint8)
    for b in range(2):
        row[b * 18:b * 18 + 2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
        row[b * 18 + 2:(b + 1) * 18] = 0x88
    row[18 + 2] = 0x89
    x = np.zeros(64, np.float32)
    x[32] = 5
    assert O.dot_q40_f32(row, x) == 5


def test_dot_q80_and_mxfp4_known_answers(O):
    row = np.zeros(34, np.uint8)
    row[0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    row[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    want = float(np.sum(np.arange(32) - 16))
    assert abs(O.dot_q80_f32(row, np.ones(32, np.float32)) - want) <= 1e-4
    mx = np.full(17, 0x22, np.uint8)
    mx[0] = 127
    assert abs(O.dot_mxfp4_f32(mx, np.full(32, 2.0, np.float32)) - 64.0) <= 1e-4


def test_mxfp4_all_scales(O):
    x = np.full(32, 1.0 / 32, np.float32)
    for scale in range(256):
        row = np.full(17, 0x22, np.uint8)
        row[0] = scale
        want = np.float32(math.ldexp(1, scale - 127)) if scale < 255 else np.float32(np.inf)
        got = O.dot_mxfp4_f32(row, x)
        assert got == want, (scale, got, want)
    row = np.zeros(17, np.uint8)
    row[0] = 255
    assert np.isnan(O.dot_mxfp4_f32(row, x))


@pytest.mark.parametrize("input_dim", [32, 96, 2880])
def test_mxfp4_nibble_reference(O, input_dim):
    rows, blocks = 256, input_dim // 32
    x = ((np.arange(input_dim) % 23) - 11).astype(np.float32) / 32
    data = np.zeros((rows, blocks, 17), np.uint8)
    r = np.arange(rows)[:, None, None]
    b = np.arange(blocks)[None, :, None]
    i = np.arange(16)[None, None, :]
    data[:, :, 0] = (120 + np.arange(blocks) % 12)[None, :]
    data[:, :, 1:] = ((r + b * 7 + i * 11) & 0xFF).astype(np.uint8)
    scale = np.ldexp(1.0, data[:, :, 0].astype(np.int64) - 127)
    lo, hi = LEVELS64[data[:, :, 1:] & 15], LEVELS64[data[:, :, 1:] >> 4]
    xb = x.astype(np.float64).reshape(blocks, 32)
    want = np.sum(scale[:, :, None] * (lo * xb[None, :, :16] + hi * xb[None, :, 16:]), axis=(1, 2))
    for row in range(rows):
        enc = data[row].reshape(-1)
        got = O.dot_mxfp4_f32(enc, x)
        assert _tol(got, want[row]), (row, got, want[row])
        assert got.view(np.uint32) == O.dot_mxfp4_f32(enc, x, scalar=True).view(np.uint32)


@pytest.mark.parametrize("input_dim", [32, 96, 2880])
@pytest.mark.parametrize("count", [1, 2, 3, 16])
def test_simd_kernel_gather(O, input_dim, count):
    blocks = input_dim // 32
    row = np.zeros((blocks, 17), np.uint8)
    row[:, 0] = 123 + np.arange(blocks) % 8
    row[:, 1:] = ((np.arange(blocks)[:, None] * 37 + np.arange(16)[None, :] * 17) & 0xFF).astype(np.uint8)
    vector = ((np.arange(input_dim) % 31) - 15).astype(np.float32) / 32
    bias = np.float32([.125, -.25, .5])
    scale = np.ldexp(1.0, row[:, 0].astype(np.int64) - 127)
    for token in range(count):
        x = vector * np.float32(token + 1)
        xb = x.astype(np.float64).reshape(blocks, 32)
        want = np.sum(scale[:, None] * (LEVELS64[row[:, 1:] & 15] * xb[:, :16] + LEVELS64[row[:, 1:] >> 4] * xb[:, 16:]))
        for i, bb in enumerate(bias):
            got = O.dot_mxfp4_f32(row.reshape(-1), x) + bb
            assert _tol(got, want + float(bb)), (token, i)


@pytest.mark.parametrize("hidden", [32, 96, 2880])
@pytest.mark.parametrize("batch", [1, 2, 17])
def test_simd_kernel_router(O, hidden, batch):
    E = 5
    bias = np.float32([.125, -.25, .5, -1, 2])
    data = ((np.arange(E * hidden) % 23) - 11).astype(np.float32) / 64
    x = ((np.arange(batch * hidden) % 31) - 15).astype(np.float32) / 32
    logits = O.route(data, bias, x, batch, hidden, E).reshape(batch, E)
    want = (x.astype(np.float64).reshape(batch, hidden) @ data.astype(np.float64).reshape(E, hidden).T) + bias
    for t in range(batch):
        for e in range(E):
            assert _tol(logits[t, e], want[t, e]), (t, e)
    for t in range(batch):
        for e in range(E):
            a = O.dot_f32(data[e * hidden:(e + 1) * hidden], x[t * hidden:(t + 1) * hidden])
            s = O.dot_f32(data[e * hidden:(e + 1) * hidden], x[t * hidden:(t + 1) * hidden], scalar=True)
            assert a.view(np.uint32) == s.view(np.uint32)
    for value in (np.nan, np.inf, -np.inf):
        d = data.copy()
        d[0] = value
        xx = x.copy()
        xx[0] = 1
        got = O.route(d, bias, xx, batch, hidden, E)[0]
        if np.isnan(value):
            assert np.isnan(got)
        else:
            assert got == value


@pytest.mark.parametrize("typ", [2, 8])
def test_quant_float16_scales(O, typ):
    x = np.ones(32, np.float32)
    for s in range(65536):
        h = np.frombuffer(np.uint16(s).tobytes(), np.uint8)
        if typ == 2:
            row = np.concatenate([h, np.full(16, 0x99, np.uint8)])
            got = O.dot_q40_f32(row, x)
        else:
            row = np.concatenate([h, np.ones(32, np.uint8)])
            got = O.dot_q80_f32(row, x)
        want = np.float32(np.uint16(s).view(np.float16)) * np.float32(32)
        if np.isnan(want):
            assert np.isnan(got), hex(s)
        else:
            assert got == want, hex(s)


@pytest.mark.parametrize("typ", [2, 8])
@pytest.mark.parametrize("input_dim", [32, 96, 512])
def test_quant_numerics(O, typ, input_dim):
    output_dim = 17
    data = quant_optimization_fixture(typ, input_dim, output_dim)
    x = ((np.arange(input_dim) % 23) - 11).astype(np.float32) / 32
    bb = 18 if typ == 2 else 34
    rb = input_dim // 32 * bb
    for row in range(output_dim):
        enc = data[row * rb:(row + 1) * rb].reshape(-1, bb)
        d = enc[:, 0:2].copy().view(np.uint16).ravel().view(np.float16).astype(np.float64)
        if typ == 2:
            w = np.concatenate([(enc[:, 2:] & 15).astype(np.int64) - 8, (enc[:, 2:] >> 4).astype(np.int64) - 8], 1)
            got = O.dot_q40_f32(enc.reshape(-1), x)
        else:
            w = enc[:, 2:].view(np.int8).astype(np.int64)
            got = O.dot_q80_f32(enc.reshape(-1), x)
        want = np.sum(d[:, None] * w * x.astype(np.float64).reshape(-1, 32))
        assert abs(got - want) <= 1e-4 * (1 + abs(want)), (row, got, want)


@pytest.mark.parametrize("batch", [2, 9, 32])
def test_q40_batch_path(O, batch):
    """quantDotQ40Batch (tile of 8, one accumulator per item) against the
    batch==1 path and float64 (the reference compares them at 1e-4)."""
    from spt import synth

    input_dim, output_dim = 2880, 24
    w = synth.q40_bytes(synth.stream_key(21, 0), output_dim, input_dim)
    x = synth.normal(synth.stream_key(22, batch), batch * input_dim)
    yb = O.mul_q40_f32(w, x, input_dim, output_dim, batch).reshape(batch, output_dim)
    for t in range(batch):
        y1 = O.mul_q40_f32(w, x[t * input_dim:(t + 1) * input_dim], input_dim, output_dim, 1)
        assert np.all(np.abs(yb[t] - y1) <= 1e-4 * (1 + np.abs(y1)))


def test_exact_tables_match_oracle(O):
    """The decode tables tests/exact.py computes the bit-exact tests' expected values
    from (2 * E2M1 per nibble, low nibble = element i and high = i + 16;
    Q4_0 n - 8) against the oracle's integer block sums, over every nibble
    byte at every position and code vectors of both signs, and the E2M1
    table against the format's values (LEVELS64, the reference's table)."""
    from exact import LUT2, all_pairs_bytes, exact_dots, mx_matrix, q40_matrix

    assert np.array_equal(LUT2, (2 * LEVELS64).astype(np.int64))
    rng = np.random.default_rng(11)
    nib = all_pairs_bytes(256)
    for q in (np.full(32, 1, np.int8), np.arange(-16, 16, dtype=np.int8) * 7,
              rng.integers(-127, 128, size=32).astype(np.int8)):
        lo = LUT2[nib & 15].astype(np.int64)
        hi = LUT2[nib >> 4].astype(np.int64)
        mine = lo @ q[:16].astype(np.int64) + hi @ q[16:].astype(np.int64)
        w = mx_matrix(nib[:, None, :], np.full((256, 1), 127, np.uint8))
        assert np.array_equal(mine, [O.isum_mxfp4_q8(w[r, 0], q) for r in range(256)])
        wq = q40_matrix(nib[:, None, :], np.full((256, 1), 0x3C00, np.uint16))
        qs = (((nib & 15).astype(np.int64) - 8) @ q[:16].astype(np.int64) +
              ((nib >> 4).astype(np.int64) - 8) @ q[16:].astype(np.int64))
        assert np.array_equal(qs, [O.isum_q40_q8(wq[r, 0], q) for r in range(256)])
    # the one-block float64 form against the oracle's row dot (one block,
    # so the same single rounding), for E8M0 {4, 118, 127, 240} and d_x of
    # random fp16 values
    x = (rng.standard_normal((3, 32)) * 40).astype(np.float32)
    x[:, 0] = 127
    xq = O.quantize_q8_0(x.reshape(-1)).reshape(3, 1, 34)
    codes = xq[..., 2:].copy().view(np.int8)
    d = xq[..., :2].copy().view(np.float16)[..., 0].astype(np.float64)
    for e in (4, 118, 127, 240):
        w = mx_matrix(nib[:, None, :], np.full((256, 1), e, np.uint8))
        vals = np.concatenate([LUT2[w[..., 1:] & 15], LUT2[w[..., 1:] >> 4]], axis=-1)
        want = exact_dots(vals, np.ldexp(1.0, w[..., 0].astype(np.int64) - 128), codes, d)
        got = np.array([[O.dot_mxfp4_q8(w[r].reshape(-1), xq[t].reshape(-1)) for r in range(256)]
                        for t in range(3)], np.float32)
        assert np.array_equal(got, want), e

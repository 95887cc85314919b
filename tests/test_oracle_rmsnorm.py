"""Pin the oracle's RMSNorm restatements (RMSNormInto's and normBatch's lane
orders) against the reference's tests and float64 brute force.

  TestRMSNormFormats                   rmsnorm_test.go:17-106
  TestRMSNormInto                      rmsnorm_into_test.go:16-63
  TestRMSNormIntoWindowBoundary        rmsnorm_into_test.go:65-88
  TestPrefillBatchNormalizationFormats prefill_batch_test.go:224-262 (weights)
referenceRMSNorm (rmsnorm_test.go:191-207) is the float64 formula and
compareVectors (rmsnorm_test.go:209-224) the 1e-4 * (1 + |want|) tolerance.
"""
import numpy as np
import pytest

FORMATS = {
    0: np.array([1, 2, 0.5, -1, 1], np.float32).view(np.uint8),
    1: np.array([0x3C00, 0x4000, 0x3800, 0xBC00, 0x3C00], np.uint16).view(np.uint8),
    28: np.array([0x3F80, 0x4000, 0x3F00, 0xBF80, 0x3F80], np.uint16).view(np.uint8),
}


def reference_rmsnorm(x, w, eps):
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    factor = 1 / np.sqrt(np.sum(x64 * x64) / x.size + float(np.float32(eps)))
    return (x64 * w64 * factor).astype(np.float32)


def close(got, want):
    return np.all(np.abs(got.astype(np.float64) - want) <= 1e-4 * (1 + np.abs(want.astype(np.float64))))


@pytest.mark.parametrize("typ", [0, 1, 28])
def test_rmsnorm_formats(O, typ):
    w = O.decode_norm_weight(FORMATS[typ], typ)
    assert np.array_equal(w, np.float32([1, 2, 0.5, -1, 1]))
    x = np.float32([2, -4, 1, 3, -2])
    want = reference_rmsnorm(x, w, 1e-5)
    assert close(O.rmsnorm_f32(x, w, 1e-5), want)
    assert close(O.rmsnorm_batch_f32(x, w, 1, 1e-5), want)


def test_rmsnorm_window_boundary(O):
    count = (8 << 20) // 4 + 3  # DefaultQ40WindowBytes / 4 + 3 (q40.go:22)
    i = np.arange(count)
    w = ((i % 5 + 1) / 2).astype(np.float32)
    x = (i % 3 - 1).astype(np.float32)
    want = reference_rmsnorm(x, w, 1e-5)
    assert close(O.rmsnorm_f32(x, w, 1e-5), want)


def test_rmsnorm_batch_formats(O):
    dim, batch = 2880, 5
    for typ in (1, 28):
        bits = (0x3C00 if typ == 1 else 0x3F80) + np.arange(dim) % 7
        w = O.decode_norm_weight(bits.astype(np.uint16).view(np.uint8), typ)
        from spt import synth

        x = synth.normal(synth.stream_key(70, typ), batch * dim)
        yb = O.rmsnorm_batch_f32(x, w, batch, 1e-5).reshape(batch, dim)
        for t in range(batch):
            xt = x[t * dim:(t + 1) * dim]
            want = reference_rmsnorm(xt, w, 1e-5)
            assert close(yb[t], want)
            assert close(O.rmsnorm_f32(xt, w, 1e-5), want)


@pytest.mark.parametrize("n", [1, 7, 8, 31, 32, 33, 2880, 4097])
def test_rmsnorm_orders_against_float64(O, n):
    """Both lane orders (with their ragged tails) agree with float64 far
    inside the reference tolerance, and differ from each other only by
    rounding."""
    from spt import synth

    x = synth.normal(synth.stream_key(71, n), n) * np.float32(3)
    w = synth.normal(synth.stream_key(72, n), n)
    want = reference_rmsnorm(x, w, 1e-6)
    for got in (O.rmsnorm_f32(x, w, 1e-6), O.rmsnorm_batch_f32(x, w, 1, 1e-6)):
        rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want.astype(np.float64)), 1e-30)
        assert np.max(rel) < 2e-6, n


def test_rmsnorm_lane_order_is_the_avx2_one(O):
    """A sum of squares that depends on the order: x[0] = 4096 (square 2^24,
    where f32 spacing is 2) and ones elsewhere, n = 64.  RMSNormInto's lane 0
    is ((c0 + c8) + c16) + c24 with chain c0 = 2^24 (+1 rounds to even) and
    c8 = c16 = c24 = 2, so 2^24 + 6; lanes 1..7 = 8; sum 2^24 + 62.
    normBatch's lane 0 adds eight ones to 2^24 one at a time (each rounds
    away): 2^24; sum 2^24 + 56."""
    n = 64
    x = np.ones(n, np.float32)
    x[0] = np.float32(4096)
    w = np.ones(n, np.float32)

    def factor(total):
        return np.float32(1) / np.float32(np.sqrt(np.float64(np.float32(np.float32(total) / np.float32(n)) + np.float32(1e-5))))

    f_into, f_batch = factor(2.0 ** 24 + 62), factor(2.0 ** 24 + 56)
    assert f_into != f_batch
    assert O.rmsnorm_f32(x, w, 1e-5)[1] == f_into
    assert O.rmsnorm_batch_f32(x, w, 1, 1e-5)[1] == f_batch

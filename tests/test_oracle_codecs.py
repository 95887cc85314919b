"""Pin the oracle's block codecs against library routines and the
reference's exhaustive known-answer tests.

- fp16 -> fp32: all 65,536 encodings against numpy's float16
  (forward/q40.go:149-177, quant_portable.go:20-35; TestFloat16,
  q40_test.go:53-77).
- fp32 -> fp16 (Q8_0 scale store, round to nearest even): numpy astype.
- E8M0: all 256 exponents against math.ldexp (forward/mxfp4.go:23).
- MXFP4 decode: all 256 scales x 256 byte patterns, AVX2 and scalar
  restatements, bit-exact against factor * level computed independently
  (TestSIMDKernelMXFP4DecodeAllEncodings, simd_kernels_test.go:211-246).
"""
import math

import numpy as np

LEVELS = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6], np.float32)


def test_fp16_to_f32_all_encodings(O):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([O.fp16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_fp16_known_answers(O):
    # TestFloat16 (q40_test.go:58-63)
    assert O.fp16_to_f32(0x0000) == 0.0
    assert O.fp16_to_f32(0x3C00) == 1.0
    assert O.fp16_to_f32(0xBC00) == -1.0
    assert O.fp16_to_f32(0x0001) == 1.0 / 16777216
    assert O.fp16_to_f32(0x7C00) == math.inf


def _f16_rne(values):
    return np.asarray(values, np.float32).astype(np.float16).view(np.uint16)


def test_f32_to_fp16_round_nearest_even(O):
    rng = np.random.default_rng(0)
    exact = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    exact = exact[np.isfinite(exact)]
    # midpoints between neighbouring finite fp16 values are exact ties
    pos = np.sort(exact[exact >= 0])
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    rand = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
                           np.float32([65504, 65519.99, 65520, 1e9, 2 ** -24, 2 ** -25, 3 * 2 ** -26,
                                       2 ** -26, 5.960464477539063e-08, 6.1e-5, 6.10351e-5])])
    for vals in (exact, mids, -mids, rand.astype(np.float32)):
        got = np.array([O.f32_to_fp16(float(v)) for v in vals], np.uint16)
        assert np.array_equal(got, _f16_rne(vals)), vals[np.nonzero(got != _f16_rne(vals))[0][:5]]
    assert O.f32_to_fp16(float("nan")) == 0x7E00
    assert O.f32_to_fp16(float("inf")) == 0x7C00 and O.f32_to_fp16(float("-inf")) == 0xFC00


def test_e8m0_all_exponents(O):
    for e in range(256):
        want = np.float32(math.ldexp(1.0, e - 127)) if e < 255 else np.float32(np.inf)
        assert np.float32(O.e8m0(e)).view(np.uint32) == want.view(np.uint32), e


def test_mxfp4_decode_all_encodings(O):
    row = np.zeros((256 * 256, 17), np.uint8)
    row[:, 0] = np.repeat(np.arange(256, dtype=np.uint8), 256)
    row[:, 1:] = np.tile(np.arange(256, dtype=np.uint8), 256)[:, None]
    row = row.reshape(-1)
    for scalar in (False, True):
        got = O.mxfp4_decode_row(row, scalar=scalar).reshape(256, 256, 32)
        for scale in range(256):
            factor = np.float32(math.ldexp(1, scale - 127)) if scale < 255 else np.float32(np.inf)
            packed = np.arange(256)
            nib = np.concatenate([np.repeat((packed & 15)[:, None], 16, 1), np.repeat((packed >> 4)[:, None], 16, 1)], 1)
            with np.errstate(invalid="ignore"):
                want = factor * LEVELS[nib]
            g = got[scale]
            nan = np.isnan(want)
            assert np.array_equal(np.isnan(g), nan), scale
            assert np.array_equal(g[~nan].view(np.uint32), want[~nan].view(np.uint32)), scale


def test_mxfp4_scalar_decode_matches_avx2(O):
    from spt import synth

    row = synth.mxfp4_expert_bytes(synth.stream_key(1, 1), 0, 4096, 0, 255)
    a = O.mxfp4_decode_row(row, scalar=False)
    b = O.mxfp4_decode_row(row, scalar=True)
    nan = np.isnan(a)
    assert np.array_equal(nan, np.isnan(b))
    assert np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32))

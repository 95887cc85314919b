"""Shared test helpers."""
import numpy as np

# fp32 outputs of the Q8_0 path against the Q8_0 oracle: the per-block int32
# sums are exact, only the fp32 order of the cross-block sum differs, so the
# bar is a max relative error of 1e-3.  "Relative" is per element, with the
# denominator floored at the mean magnitude of the compared vector so that
# outputs that cancel to ~0 are judged on the vector's scale.
REL_TOL = 1e-3


def rel_err(got, want) -> float:
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    if got.size == 0:
        return 0.0
    floor = max(np.mean(np.abs(want)), 1e-30)
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), floor)))


def assert_close(got, want, tol=REL_TOL, what=""):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_g, nan_w), f"{what}: NaN positions differ"
    inf_g, inf_w = np.isinf(got), np.isinf(want)
    assert np.array_equal(inf_g, inf_w) and np.array_equal(got[inf_g], want[inf_w]), f"{what}: Inf differ"
    fin = ~(nan_g | inf_g)
    e = rel_err(got[fin], want[fin])
    assert e <= tol, f"{what}: max relative error {e:.3g} > {tol}"
    return e


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def tie_block():
    """A Q8_0 block whose amax is 127 (d = 1, id = 1) holding exact .5
    values of both signs, small and near the top of the code range."""
    v = np.array([127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 3.5, -3.5, 4.5, -4.5, 10.5, -10.5, 63.5, -63.5,
                  64.5, -64.5, 100.5, -100.5, 125.5, -125.5, 126.5, -126.5, 0.0, -0.0, 7.5, -7.5, 8.5,
                  -8.5, 31.5, -31.5, -127.0], np.float32)
    assert v.size == 32
    return v

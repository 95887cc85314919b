"""Inputs and expected values for the bit-exact kernel tests
(test_gpu_exact.py): integer tokens whose Q8_0 scale is 1, byte patterns
holding every nibble pair, and the integer form of the MXFP4 x Q8_0 and
Q4_0 x Q8_0 dots evaluated exactly in float64 and rounded once to fp32."""
import numpy as np

# 2 * E2M1 of each nibble (the integer form: contribution 2^(e-128) * isum)
LUT2 = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.int64)


def int_tokens(rng, batch, dim):
    """fp32 tokens of integers in [-127, 127] with one +-127 per 32-block, so
    each block's Q8_0 scale is 1 and its codes are the values themselves."""
    x = rng.integers(-127, 128, size=(batch, dim // 32, 32)).astype(np.float32)
    pos = rng.integers(0, 32, size=(batch, dim // 32))
    sgn = np.where(rng.integers(0, 2, size=(batch, dim // 32)) == 0, -127.0, 127.0)
    np.put_along_axis(x, pos[..., None], sgn[..., None].astype(np.float32), axis=2)
    return x.reshape(batch, dim)


def all_pairs_bytes(rows, shift=0):
    """[rows, 16] nibble bytes: byte j of row r is (r + 16 j + shift) mod 256,
    so every 256 consecutive rows hold every byte value at every position."""
    r = np.arange(rows)[:, None]
    j = np.arange(16)[None, :]
    return ((r + 16 * j + shift) & 255).astype(np.uint8)


def mx_matrix(nib, exps):
    """MXFP4 rows [rows, nb, 17] from nibble bytes [rows, nb, 16] and E8M0
    bytes [rows, nb]."""
    rows, nb = exps.shape
    w = np.empty((rows, nb, 17), np.uint8)
    w[..., 0] = exps
    w[..., 1:] = nib
    return w


def q8_codes_scales(O, x):
    """(codes [B, nb, 32] int8, d [B, nb] float64) of the oracle's Q8_0 of x."""
    B, dim = x.shape
    q = O.quantize_q8_0(x.reshape(-1)).reshape(B, dim // 32, 34)
    d = q[..., :2].copy().view(np.float16)[..., 0].astype(np.float64)
    return q[..., 2:].copy().view(np.int8), d


def exact_dots(vals, s, codes, d):
    """y[t, r] = sum_b s[r, b] * d[t, b] * isum[t, r, b], isum = sum_k
    vals[r, b, k] * codes[t, b, k], in float64 and rounded once to fp32.
    With one block the float64 value is the exact product; with several the
    family guarantees d = 1 and partial sums that are exact in any order."""
    rows, nb = s.shape
    if nb == 1:
        isum = codes[:, 0, :].astype(np.float64) @ vals[:, 0, :].astype(np.float64).T
        y = isum * s[None, :, 0] * d[:, 0, None]
    else:
        assert np.all(d == 1.0), "several blocks need d_x = 1 to be exact"
        wf = (vals.astype(np.float64) * s[..., None]).reshape(rows, -1)
        y = codes.reshape(codes.shape[0], -1).astype(np.float64) @ wf.T
    return y.astype(np.float32)


def mx_expected(w, codes, d):
    """MXFP4 rows w [rows, nb, 17]: 2 * E2M1 values against the codes, block
    scale 2^(e-128)."""
    nib = w[..., 1:]
    vals = np.concatenate([LUT2[nib & 15], LUT2[nib >> 4]], axis=-1)
    return exact_dots(vals, np.ldexp(1.0, w[..., 0].astype(np.int64) - 128), codes, d)


def q40_matrix(nib, dbits):
    """Q4_0 rows [rows, nb, 18] from nibble bytes [rows, nb, 16] and fp16
    scale bits [rows, nb]."""
    rows, nb = dbits.shape
    w = np.empty((rows, nb, 18), np.uint8)
    w[..., 0:2] = dbits.astype(np.uint16).view(np.uint8).reshape(rows, nb, 2)
    w[..., 2:] = nib
    return w


def q40_expected(w, codes, d):
    """Q4_0 rows w [rows, nb, 18]: values n - 8, block scale d_w."""
    nib = w[..., 2:].astype(np.int64)
    vals = np.concatenate([(nib & 15) - 8, (nib >> 4) - 8], axis=-1)
    dw = w[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    return exact_dots(vals, dw, codes, d)


def assert_exact(got, want, what):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, (got.shape, want.shape)
    bad = np.nonzero(got != want)
    assert bad[0].size == 0, (f"{what}: {bad[0].size} of {got.size} differ, first at {tuple(b[0] for b in bad)}: "
                              f"got {got[tuple(b[0] for b in bad)]!r}, want {want[tuple(b[0] for b in bad)]!r}")


def pow2_q40(rng, rows, nb):
    """Q4_0 rows with fp16 scales +-2^-9 or +-2^-8 per block and uniform nibbles."""
    nib = rng.integers(0, 256, size=(rows, nb, 16), dtype=np.uint8)
    mag = np.where(rng.integers(0, 2, size=(rows, nb)) == 0, 2.0 ** -9, 2.0 ** -8)
    sgn = np.where(rng.integers(0, 2, size=(rows, nb)) == 0, -1.0, 1.0)
    return q40_matrix(nib, (mag * sgn).astype(np.float16).view(np.uint16))

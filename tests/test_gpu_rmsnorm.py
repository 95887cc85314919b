"""GPU parity of the fused RMSNorm (spt_rmsnorm_into, spt_rmsnorm_batch_into)
against the oracle's restatement of RMSNormInto and normBatch: y bit-identical
in both lane orders, its Q8_0 blocks bit-identical to the oracle quantizer's,
on the reference's format fixtures, in place, ragged lengths, the
weight-window case, an order-sensitive case, special values, and a
512-token batch."""
import numpy as np
import pytest

from test_oracle_rmsnorm import FORMATS

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _weight(raw, typ, n):
    import spt

    wd = _dev(np.ascontiguousarray(raw, np.uint8))
    return wd, spt.Tensor.make("norm.weight", typ, [n], wd.data_ptr(), raw.size)


def _same_bits(got, want):
    g, w = got.view(np.uint32), want.view(np.uint32)
    bad = np.nonzero((g != w) & ~(np.isnan(got) & np.isnan(want)))[0]
    assert bad.size == 0, (bad[:8], got[bad[:4]], want[bad[:4]])


def _run(gpu_ctx, raw, typ, x, batch=None, eps=1e-5, q8=False, inplace=False):
    import torch

    n = raw.size // (4 if typ == 0 else 2)
    wd, t = _weight(raw, typ, n)
    xd = _dev(x)
    y = xd if inplace else torch.full_like(xd, 777.0)
    qb = torch.zeros(x.size // 32 * 34, dtype=torch.uint8, device="cuda") if q8 else None
    if batch is None:
        gpu_ctx.rmsnorm_into(t, xd, y, eps, qb)
    else:
        gpu_ctx.rmsnorm_batch_into(t, xd, y, batch, eps, qb)
    torch.cuda.synchronize()
    return y.cpu().numpy(), (qb.cpu().numpy() if q8 else None)


@pytest.mark.parametrize("typ", [0, 1, 28])
@pytest.mark.parametrize("inplace", [False, True])
def test_rmsnorm_formats(gpu_ctx, O, typ, inplace):
    x = np.float32([2, -4, 1, 3, -2])
    w = O.decode_norm_weight(FORMATS[typ], typ)
    y, _ = _run(gpu_ctx, FORMATS[typ], typ, x, inplace=inplace)
    _same_bits(y, O.rmsnorm_f32(x, w, 1e-5))
    y, _ = _run(gpu_ctx, FORMATS[typ], typ, x, batch=1, inplace=inplace)
    _same_bits(y, O.rmsnorm_batch_f32(x, w, 1, 1e-5))


@pytest.mark.parametrize("n", [1, 7, 8, 31, 32, 33, 96, 256, 1056, 2048, 2880, 4097, 8192, 8224])
def test_rmsnorm_ragged_lengths(gpu_ctx, O, n):
    from spt import synth

    x = synth.normal(synth.stream_key(80, n), n) * np.float32(3)
    w = synth.normal(synth.stream_key(81, n), n)
    q8 = n % 32 == 0
    y, qb = _run(gpu_ctx, w.view(np.uint8), 0, x, q8=q8)
    want = O.rmsnorm_f32(x, w, 1e-5)
    _same_bits(y, want)
    if q8:
        assert np.array_equal(qb, O.quantize_q8_0(want))
    y, qb = _run(gpu_ctx, w.view(np.uint8), 0, x, batch=1, q8=q8)
    want = O.rmsnorm_batch_f32(x, w, 1, 1e-5)
    _same_bits(y, want)
    if q8:
        assert np.array_equal(qb, O.quantize_q8_0(want))


def test_rmsnorm_weight_window(gpu_ctx, O):
    """TestRMSNormIntoWindowBoundary's vector (2^21 + 3 elements)."""
    count = (8 << 20) // 4 + 3
    i = np.arange(count)
    w = ((i % 5 + 1) / 2).astype(np.float32)
    x = (i % 3 - 1).astype(np.float32)
    y, _ = _run(gpu_ctx, w.view(np.uint8), 0, x)
    _same_bits(y, O.rmsnorm_f32(x, w, 1e-5))


def test_rmsnorm_order_sensitive(gpu_ctx, O):
    """x[0] = 4096 and ones: the two lane orders give different factors."""
    x = np.ones(64, np.float32)
    x[0] = 4096
    w = np.ones(64, np.float32)
    y1, _ = _run(gpu_ctx, w.view(np.uint8), 0, x)
    yb, _ = _run(gpu_ctx, w.view(np.uint8), 0, x, batch=1)
    _same_bits(y1, O.rmsnorm_f32(x, w, 1e-5))
    _same_bits(yb, O.rmsnorm_batch_f32(x, w, 1, 1e-5))
    assert y1[1] != yb[1]


@pytest.mark.parametrize("case", ["zeros", "zeros_eps0", "nan", "inf", "huge", "tiny"])
def test_rmsnorm_special_values(gpu_ctx, O, case):
    from spt import synth

    n = 96
    x = synth.normal(synth.stream_key(82, 0), n)
    eps = 1e-5
    if case == "zeros":
        x[:] = 0
    elif case == "zeros_eps0":
        x[:] = 0
        eps = 0.0
    elif case == "nan":
        x[17] = np.nan
    elif case == "inf":
        x[40] = np.inf
    elif case == "huge":
        x *= np.float32(1e30)
    elif case == "tiny":
        x *= np.float32(1e-30)
    w = synth.normal(synth.stream_key(83, 0), n)
    for batch in (None, 1):
        y, qb = _run(gpu_ctx, w.view(np.uint8), 0, x, batch=batch, eps=eps, q8=True)
        want = O.rmsnorm_f32(x, w, eps) if batch is None else O.rmsnorm_batch_f32(x, w, 1, eps)
        _same_bits(y, want)
        assert np.array_equal(qb, O.quantize_q8_0(want))


@pytest.mark.parametrize("typ", [0, 1, 28])
def test_rmsnorm_prefill_batch(gpu_ctx, O, typ):
    """512 tokens of 2880 (the hot_b512 prefill batch), normBatch order,
    with the Q8_0 of every row; TestPrefillBatchNormalizationFormats'
    weights for F16 / BF16."""
    from spt import synth

    dim, batch = 2880, 512
    if typ == 0:
        raw = synth.normal(synth.stream_key(84, 0), dim).view(np.uint8)
    else:
        bits = (0x3C00 if typ == 1 else 0x3F80) + np.arange(dim) % 7
        raw = bits.astype(np.uint16).view(np.uint8)
    w = O.decode_norm_weight(raw, typ)
    x = synth.normal(synth.stream_key(85, typ), batch * dim) * np.float32(2)
    y, qb = _run(gpu_ctx, raw, typ, x, batch=batch, q8=True)
    want = O.rmsnorm_batch_f32(x, w, batch, 1e-5)
    _same_bits(y, want)
    assert np.array_equal(qb, O.quantize_q8_0(want))

"""GPU parity of the Q8_0 LM head (spt_mul_q80_into, spt_mul_q80_argmax)
against the oracle's restatement of MulQ80Into / MulQ80Argmax: logits
bit-identical (the kernel keeps the reference's 32 chains per row and its
reduction), argmax token and logit bits identical, including ties, NaN and
infinite rows, and the full 201088 x 2880 GPT-OSS LM head."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _tensor(wd, input_dim, output_dim):
    import spt

    return spt.Tensor.make("output.weight", spt.TYPE_Q8_0, [input_dim, output_dim], wd.data_ptr(),
                           input_dim // 32 * 34 * output_dim)


def _same_bits(got, want):
    g, w = got.view(np.uint32), want.view(np.uint32)
    nan = np.isnan(got) & np.isnan(want)
    bad = np.nonzero((g != w) & ~nan)[0]
    assert bad.size == 0, (bad[:10], got[bad[:5]], want[bad[:5]])


def _same_argmax(got, want):
    assert got[0] == want[0] and np.float32(got[1]).view(np.uint32) == np.float32(want[1]).view(np.uint32), (got, want)


def _run(gpu_ctx, w, x, input_dim, output_dim):
    import torch

    wd, xd = _dev(w), _dev(x)
    t = _tensor(wd, input_dim, output_dim)
    y = torch.full((output_dim,), 12345.0, dtype=torch.float32, device="cuda")
    gpu_ctx.mul_q80_into(t, xd, y)
    tok, logit = gpu_ctx.mul_q80_argmax(t, xd)
    torch.cuda.synchronize()
    return y.cpu().numpy(), tok, np.float32(logit)


SHAPES = [(32, 17), (96, 17), (512, 17), (2880, 1), (2880, 2), (2880, 3), (2880, 4099),
          (4096, 1001), (4096, 2), (64, 70001), (2880, 100000)]


@pytest.mark.parametrize("input_dim,output_dim", SHAPES)
def test_q80_rows_bit_exact(gpu_ctx, O, input_dim, output_dim):
    from spt import synth

    print(f"q80 rows {input_dim}x{output_dim}", flush=True)
    w = synth.q80_bytes(synth.stream_key(40, input_dim), output_dim, input_dim)
    x = synth.normal(synth.stream_key(41, output_dim), input_dim)
    y, tok, logit = _run(gpu_ctx, w, x, input_dim, output_dim)
    want = O.mul_q80_f32(w, x, input_dim, output_dim, threads=8)
    _same_bits(y, want)
    _same_argmax((tok, logit), O.mul_q80_argmax(w, x, input_dim, output_dim))


def test_q80_host_forms(gpu_ctx, O):
    """The host-slice entry points give the device forms' results."""
    from spt import synth

    input_dim, rows = 2880, 3001
    w = synth.q80_bytes(synth.stream_key(46, 0), rows, input_dim)
    x = synth.normal(synth.stream_key(47, 0), input_dim)
    wd = _dev(w)
    t = _tensor(wd, input_dim, rows)
    y = np.zeros(rows, np.float32)
    gpu_ctx.mul_q80_into_host(t, x, y)
    _same_bits(y, O.mul_q80_f32(w, x, input_dim, rows))
    tok, logit = gpu_ctx.mul_q80_argmax_host(t, x)
    _same_argmax((tok, np.float32(logit)), O.mul_q80_argmax(w, x, input_dim, rows))


@pytest.mark.parametrize("input_dim", [32, 2880])
def test_q80_reference_fixture(gpu_ctx, O, input_dim):
    """quantOptimizationFixture rows (scales 1, -0.5, subnormal, the largest
    finite, -0, ...) as in TestQuantOptimizationNumerics."""
    from fixtures import quant_optimization_fixture

    w = quant_optimization_fixture(8, input_dim, 17)
    x = ((np.arange(input_dim) % 23) - 11).astype(np.float32) / 32
    y, tok, logit = _run(gpu_ctx, w, x, input_dim, 17)
    _same_bits(y, O.mul_q80_f32(w, x, input_dim, 17))
    _same_argmax((tok, logit), O.mul_q80_argmax(w, x, input_dim, 17))


def test_q80_all_fp16_scales(gpu_ctx, O):
    """Every fp16 scale (v_fma_mix_f32 reads it as fp16): one row per scale."""
    rows = 65536
    w = np.zeros((rows, 34), np.uint8)
    w[:, 0:2] = np.arange(rows, dtype=np.uint16).view(np.uint8).reshape(rows, 2)
    w[:, 2:] = ((np.arange(32) * 37 + 11) & 0xFF).astype(np.uint8)[None, :]
    w = w.reshape(-1)
    x = ((np.arange(32) % 9) - 4).astype(np.float32) / 4
    y, tok, logit = _run(gpu_ctx, w, x, 32, rows)
    _same_bits(y, O.mul_q80_f32(w, x, 32, rows))
    _same_argmax((tok, logit), O.mul_q80_argmax(w, x, 32, rows))


def _plant(w, nb, row, src):
    rb = nb * 34
    w[row * rb:(row + 1) * rb] = w[src * rb:(src + 1) * rb]


def test_q80_argmax_ties_and_specials(gpu_ctx, O):
    from spt import synth

    input_dim, rows = 2880, 50021
    nb = input_dim // 32
    w = synth.q80_bytes(synth.stream_key(42, 0), rows, input_dim)
    x = np.abs(synth.normal(synth.stream_key(43, 0), input_dim)) + np.float32(0.125)
    y = O.mul_q80_f32(w, x, input_dim, rows, threads=8)
    m = int(np.argmax(y))
    # the maximum row copied to a later and an earlier row (across waves and chunks)
    for r in (rows - 1, 7, 40000):
        _plant(w, nb, r, m)
    yg, tok, logit = _run(gpu_ctx, w, x, input_dim, rows)
    _same_argmax((tok, logit), O.mul_q80_argmax(w, x, input_dim, rows))
    assert tok == min(7, m)
    _same_bits(yg, O.mul_q80_f32(w, x, input_dim, rows, threads=8))
    # NaN rows (a NaN scale) never win; a +Inf row (+Inf scale, all codes 1, x > 0) does
    rb = nb * 34
    wn = w.copy()
    for r in (0, 5, 20000):
        wn[r * rb:r * rb + 2] = (0x00, 0x7E)
    _, tok, logit = _run(gpu_ctx, wn, x, input_dim, rows)
    _same_argmax((tok, logit), O.mul_q80_argmax(wn, x, input_dim, rows))
    assert tok == min(7, m)
    wi = wn.copy()
    for r in (33333, 44444):
        wi[r * rb:r * rb + 2] = (0x00, 0x7C)
        wi[r * rb + 2:r * rb + 34] = 1
    _, tok, logit = _run(gpu_ctx, wi, x, input_dim, rows)
    assert (tok, logit) == (33333, np.float32(np.inf))
    # all rows NaN: row 0 with -Inf
    wa = w.copy().reshape(rows, nb, 34)
    wa[:, 0, 0:2] = (0x00, 0x7E)
    wa = wa.reshape(-1)
    yg, tok, logit = _run(gpu_ctx, wa, x, input_dim, rows)
    assert np.all(np.isnan(yg))
    _same_argmax((tok, logit), (0, -np.inf))
    _same_argmax((tok, logit), O.mul_q80_argmax(wa, x, input_dim, rows))


def test_q80_lm_head_full(gpu_ctx, O):
    """The GPT-OSS LM head: 201088 x 2880 Q8_0 (615 MB), every logit."""
    from spt import synth

    input_dim, rows = 2880, 201088
    print("q80 LM head 2880x201088", flush=True)
    w = synth.q80_bytes(synth.stream_key(44, 0), rows, input_dim)
    x = synth.normal(synth.stream_key(45, 0), input_dim)
    y, tok, logit = _run(gpu_ctx, w, x, input_dim, rows)
    _same_bits(y, O.mul_q80_f32(w, x, input_dim, rows, threads=16))
    _same_argmax((tok, logit), O.mul_q80_argmax(w, x, input_dim, rows))


@pytest.mark.parametrize("off", [2, 6, 14])
@pytest.mark.parametrize("input_dim,output_dim", [(2880, 4099), (96, 17)])
def test_q80_unaligned_base(gpu_ctx, O, off, input_dim, output_dim):
    """A Q8_0 matrix whose base is 2, 6 or 14 bytes past a 16-byte boundary
    (the C ABI requires only 2-byte alignment): logits and argmax bits equal
    to the oracle's, as on an aligned base."""
    import torch

    import spt
    from spt import synth

    print(f"q80 base +{off} {input_dim}x{output_dim}", flush=True)
    w = synth.q80_bytes(synth.stream_key(42, input_dim + off), output_dim, input_dim)
    x = synth.normal(synth.stream_key(43, output_dim + off), input_dim)
    buf = torch.zeros(w.size + 64, dtype=torch.uint8, device="cuda")
    buf[off:off + w.size].copy_(torch.from_numpy(np.ascontiguousarray(w)))
    t = spt.Tensor.make("output.weight", spt.TYPE_Q8_0, [input_dim, output_dim], buf.data_ptr() + off, w.size)
    xd = _dev(x)
    y = torch.full((output_dim,), 12345.0, dtype=torch.float32, device="cuda")
    gpu_ctx.mul_q80_into(t, xd, y)
    tok, logit = gpu_ctx.mul_q80_argmax(t, xd)
    torch.cuda.synchronize()
    _same_bits(y.cpu().numpy(), O.mul_q80_f32(w, x, input_dim, output_dim, threads=8))
    _same_argmax((tok, np.float32(logit)), O.mul_q80_argmax(w, x, input_dim, output_dim))

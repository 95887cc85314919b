"""GPU parity of the individual kernels against the CPU oracle, through the
C ABI.  Integer and byte outputs are compared bit-exactly; fp32 dot products
within helpers.REL_TOL."""
import numpy as np
import pytest

from helpers import assert_close, tie_block

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _mx_tensor(buf, input_dim, output_dim, experts, name="w"):
    import spt

    return spt.Tensor.make(name, spt.TYPE_MXFP4, [input_dim, output_dim, experts], buf.data_ptr(),
                           buf.numel())


def test_synth_matches_host(gpu_ctx):
    import torch

    from spt import synth

    key = synth.stream_key(7, 3)
    first, n = 12345, 4099
    d = torch.zeros(n * 17, dtype=torch.uint8, device="cuda")
    gpu_ctx.synth_mxfp4(d, key, first, n)
    torch.cuda.synchronize()
    assert np.array_equal(d.cpu().numpy(), synth.mxfp4_expert_bytes(key, first, n))


@pytest.mark.parametrize("case", ["normal", "edge"])
def test_quantize_q8_0_bit_exact(gpu_ctx, O, case):
    import torch

    from spt import synth

    n = 32 * 1024
    x = synth.normal(synth.stream_key(1, 2), n) * 3.0
    if case == "edge":
        x = x.reshape(-1, 32)
        x[0] = 0.0                         # all-zero block: d = 0, id = 0
        x[1, 5] = np.nan                   # NaN block
        x[2, 7] = np.inf                   # Inf block
        x[3] = np.float32(1e-30)           # subnormal fp16 scale
        x[4] = np.float32(6e4) * np.sign(x[4])   # scale overflows fp16
        x[5] = tie_block()                 # amax 127: d = id = 1, exact .5 ties
        x[6] = -0.0
        x[7, :] = np.arange(32, dtype=np.float32) * 4 - 62  # amax 62: codes 127*x/62, no ties
        x[8] = tie_block() * np.float32(0.5)  # amax 63.5: id = 2, the same ties
        x = x.reshape(-1)
    xd = _dev(x.astype(np.float32))
    out = torch.zeros(n // 32 * 34, dtype=torch.uint8, device="cuda")
    gpu_ctx.quantize_q8_0(xd, out)
    torch.cuda.synchronize()
    want = O.quantize_q8_0(x)
    got = out.cpu().numpy()
    assert np.array_equal(got, want), np.nonzero(got != want)[0][:10]
    if case == "edge":
        # the tie rows against half-away-from-zero worked out directly
        for row in (5, 8):
            t = tie_block()
            codes = got.reshape(-1, 34)[row, 2:].view(np.int8)
            assert np.array_equal(codes, (np.sign(t) * np.floor(np.abs(t) + 0.5)).astype(np.int8)), row


def _q8_of(O, x):
    return O.quantize_q8_0(np.ascontiguousarray(x, np.float32))


@pytest.mark.parametrize("input_dim", [32, 96, 2880])
def test_mxfp4_block_sums_exact(gpu_ctx, O, input_dim):
    import torch

    from spt import synth

    rows, E = 64, 3
    nb = input_dim // 32
    w = synth.mxfp4_expert_bytes(synth.stream_key(3, input_dim), 0, rows * nb * E)
    x = synth.normal(synth.stream_key(4, input_dim), input_dim)
    xq = _q8_of(O, x)
    wd = _dev(w)
    t = _mx_tensor(wd, input_dim, rows, E)
    sums = torch.zeros(rows * nb, dtype=torch.int32, device="cuda")
    for expert in range(E):
        gpu_ctx.block_sums(t, expert, _dev(xq), rows, sums)
        torch.cuda.synchronize()
        got = sums.cpu().numpy().reshape(rows, nb)
        base = expert * rows * nb * 17
        for r in range(rows):
            for b in range(nb):
                blk = w[base + (r * nb + b) * 17: base + (r * nb + b + 1) * 17]
                q = xq[b * 34 + 2: b * 34 + 34].view(np.int8)
                assert got[r, b] == O.isum_mxfp4_q8(blk, q), (expert, r, b)


def test_mxfp4_block_sums_all_encodings(gpu_ctx, O):
    """Every nibble byte with every sign/magnitude against all-ones and
    signed ramp activations (TestSIMDKernelMXFP4DecodeAllEncodings shape)."""
    import torch

    nb = 256
    w = np.zeros((nb, 17), np.uint8)
    w[:, 0] = 127
    w[:, 1:] = np.arange(256, dtype=np.uint8)[:, None]
    w = w.reshape(-1)
    wd = _dev(w)  # keep the device copy alive while the descriptor is used
    t = _mx_tensor(wd, 32 * nb, 1, 1)
    for x in (np.ones(32 * nb, np.float32), (np.arange(32 * nb) % 64 - 31.5).astype(np.float32)):
        xq = _q8_of(O, x)
        sums = torch.zeros(nb, dtype=torch.int32, device="cuda")
        gpu_ctx.block_sums(t, 0, _dev(xq), 1, sums)
        torch.cuda.synchronize()
        got = sums.cpu().numpy()
        want = [O.isum_mxfp4_q8(w[b * 17:(b + 1) * 17], xq[b * 34 + 2:b * 34 + 34].view(np.int8))
                for b in range(nb)]
        assert np.array_equal(got, np.array(want, np.int32))


@pytest.mark.parametrize("input_dim,output_dim,batch", [(2880, 2880, 1), (2880, 2880, 3), (96, 64, 5),
                                                       (32, 257, 1)])
def test_mxfp4_expert_gemv(gpu_ctx, O, input_dim, output_dim, batch):
    import torch

    import spt
    from spt import synth

    E, expert = 2, 1
    nb = input_dim // 32
    w = synth.mxfp4_expert_bytes(synth.stream_key(5, input_dim + output_dim), 0, E * output_dim * nb)
    bias = synth.normal(synth.stream_key(6, 1), E * output_dim, 0.0, 0.02)
    x = synth.normal(synth.stream_key(7, batch), batch * input_dim)
    wd, bd, xd = _dev(w), _dev(bias), _dev(x)
    y = torch.zeros(batch * output_dim, dtype=torch.float32, device="cuda")
    bt = spt.Tensor.make("b", spt.TYPE_F32, [output_dim, E], bd.data_ptr(), bd.numel() * 4)
    gpu_ctx.mul_mxfp4_expert(_mx_tensor(wd, input_dim, output_dim, E), bt, expert, xd, y, batch)
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(batch, output_dim)
    ew = w[expert * output_dim * nb * 17:(expert + 1) * output_dim * nb * 17]
    for t in range(batch):
        xq = _q8_of(O, x[t * input_dim:(t + 1) * input_dim])
        want = O.mul_mxfp4_q8(ew, xq, bias[expert * output_dim:(expert + 1) * output_dim], input_dim,
                              output_dim)
        assert_close(got[t], want, what=f"token {t}")


@pytest.mark.parametrize("bias_type", [1, 30])
def test_mxfp4_expert_gemv_odd_half_bias(gpu_ctx, O, bias_type):
    """One expert of 257 rows with a 2-byte bias: the last bias element sits
    in a dword that crosses the tensor's end, and the matrix (257 * 17
    bytes) ends inside a 16-byte load."""
    import torch

    import spt
    from spt import synth

    input_dim, output_dim = 64, 257
    nb = input_dim // 32
    w = synth.mxfp4_expert_bytes(synth.stream_key(8, 1), 0, output_dim * nb)
    b32 = synth.normal(synth.stream_key(9, 1), output_dim, 0.0, 0.5)
    if bias_type == 1:
        bh = b32.astype(np.float16).view(np.uint16)
        bias = bh.view(np.float16).astype(np.float32)
    else:
        bh = (b32.view(np.uint32) >> 16).astype(np.uint16)
        bias = (bh.astype(np.uint32) << 16).view(np.float32)
    x = synth.normal(synth.stream_key(10, 1), input_dim)
    wd, bd, xd = _dev(w), _dev(bh), _dev(x)
    y = torch.zeros(output_dim, dtype=torch.float32, device="cuda")
    bt = spt.Tensor.make("b", bias_type, [output_dim, 1], bd.data_ptr(), output_dim * 2)
    gpu_ctx.mul_mxfp4_expert(_mx_tensor(wd, input_dim, output_dim, 1), bt, 0, xd, y, 1)
    torch.cuda.synchronize()
    want = O.mul_mxfp4_q8(w, _q8_of(O, x), bias, input_dim, output_dim)
    assert_close(y.cpu().numpy(), want, what="odd-count 2-byte bias")


@pytest.mark.parametrize("input_dim,output_dim,batch", [
    (2880, 4096, 1), (2880, 512, 1), (4096, 2880, 1), (32, 17, 1),
    # up to four tokens: one launch quantizing its input itself, every
    # weight-block count per lane (inputs of 1 to 128 blocks)
    (2880, 4096, 2), (2880, 512, 3), (4096, 2880, 4), (96, 70, 2), (160, 33, 4), (1024, 100, 3),
    (2048, 64, 1),
    (2880, 4096, 32), (2880, 512, 32), (4096, 2880, 32), (32, 17, 32),
    # the int8-MFMA GEMM (64 tokens and up): full and ragged token tiles,
    # row counts off the 64-row tile and the 4-row stores, inputs shorter
    # than one 8-block segment and off its multiple
    (2880, 4096, 100), (2880, 512, 64), (4096, 2880, 70), (32, 17, 64), (96, 70, 129),
    (288, 4, 65), (2880, 512, 512), (4096, 2880, 512),
    # narrow projections of 256 tokens and up: the GEMM with K split four
    # ways (fewer ways when the input has fewer blocks)
    (96, 70, 300), (32, 17, 256), (4096, 512, 257),
    # wide inputs: the GEMV's activation staging above 64 KB of LDS (eight
    # tokens per pass at 8192 inputs, two at 40960)
    (8192, 300, 1), (8192, 300, 9), (40960, 40, 3),
])
def test_q40_gemv(gpu_ctx, O, input_dim, output_dim, batch):
    import torch

    import spt
    from spt import synth

    w = synth.q40_bytes(synth.stream_key(8, output_dim), output_dim, input_dim)
    x = synth.normal(synth.stream_key(9, batch), batch * input_dim)
    wd, xd = _dev(w), _dev(x)
    y = torch.zeros(batch * output_dim, dtype=torch.float32, device="cuda")
    t = spt.Tensor.make("attn", spt.TYPE_Q4_0, [input_dim, output_dim], wd.data_ptr(), w.size)
    gpu_ctx.mul_q40_batch_into(t, xd, y, batch)
    torch.cuda.synchronize()
    want = O.mul_q40_q8(w, x, input_dim, output_dim, batch)
    assert_close(y.cpu().numpy(), want, what="q40")
    # exact int32 block sums of the first rows against token 0
    nb = input_dim // 32
    xq = _q8_of(O, x[:input_dim])
    rows = min(output_dim, 16)
    sums = torch.zeros(rows * nb, dtype=torch.int32, device="cuda")
    gpu_ctx.block_sums(t, 0, _dev(xq), rows, sums)
    torch.cuda.synchronize()
    got = sums.cpu().numpy().reshape(rows, nb)
    for r in range(rows):
        for b in range(nb):
            blk = w[(r * nb + b) * 18:(r * nb + b + 1) * 18]
            assert got[r, b] == O.isum_q40_q8(blk, xq[b * 34 + 2:b * 34 + 34].view(np.int8))


@pytest.mark.parametrize("input_dim,output_dim,batch", [(2880, 4096, 1), (2880, 512, 32), (2880, 4096, 512),
                                                       (4096, 2880, 70), (32, 17, 3), (2880, 512, 300)])
@pytest.mark.parametrize("btype", [0, 1, 30])
def test_q40_bias_residual(gpu_ctx, O, input_dim, output_dim, batch, btype):
    """The projection epilogue (addBias / biasBatch, then the residual
    addVector): y = (W x) + bias with one f32 add of the decoded bias, and
    resid + y with one more, on the GEMV and on the GEMM (B = 512, 70)."""
    import torch

    import spt
    from spt import synth

    w = synth.q40_bytes(synth.stream_key(8, output_dim), output_dim, input_dim)
    x = synth.normal(synth.stream_key(9, batch), batch * input_dim)
    bf = synth.normal(synth.stream_key(10, output_dim), output_dim)
    if btype == 0:
        braw = bf.view(np.uint8)
        bdec = bf
    elif btype == 1:
        h = bf.astype(np.float16)
        braw, bdec = h.view(np.uint8), h.astype(np.float32)
    else:
        hb = (bf.view(np.uint32) >> 16).astype(np.uint16)
        braw, bdec = hb.view(np.uint8), (hb.astype(np.uint32) << 16).view(np.float32)
    r0 = synth.normal(synth.stream_key(11, batch), batch * output_dim)
    wd, xd, bd, rd = _dev(w), _dev(x), _dev(braw), _dev(r0)
    t = spt.Tensor.make("attn", spt.TYPE_Q4_0, [input_dim, output_dim], wd.data_ptr(), w.size)
    bt = spt.Tensor.make("attn.bias", btype, [output_dim], bd.data_ptr(), braw.size)
    y0 = torch.zeros(batch * output_dim, dtype=torch.float32, device="cuda")
    y1 = torch.zeros_like(y0)
    gpu_ctx.mul_q40_batch_into(t, xd, y0, batch)
    gpu_ctx.mul_q40_batch_bias_into(t, bt, xd, y1, batch, rd)
    torch.cuda.synchronize()
    plain, got, resid = y0.cpu().numpy(), y1.cpu().numpy(), rd.cpu().numpy()
    want = (plain.reshape(batch, output_dim) + bdec[None, :]).astype(np.float32).reshape(-1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(resid.view(np.uint32), (r0 + got).astype(np.float32).view(np.uint32))
    ref = O.mul_q40_q8(w, x, input_dim, output_dim, batch).reshape(batch, output_dim) + bdec[None, :]
    assert_close(got, ref.reshape(-1), what="q40+bias")


@pytest.mark.parametrize("hidden,batch", [(2880, 1), (2880, 19), (2880, 40), (2880, 64), (2880, 80), (2880, 200),
                                          (2880, 300), (96, 3), (32, 2), (96, 17), (32, 70), (160, 37), (96, 255),
                                          (160, 513)])
def test_router_logits_bit_exact(gpu_ctx, O, hidden, batch):
    import torch

    import spt
    from spt import synth

    E = 128 if hidden == 2880 else 5
    W = synth.normal(synth.stream_key(10, hidden), E * hidden, 0.0, 0.02)
    b = synth.normal(synth.stream_key(11, hidden), E, 0.0, 0.02)
    x = synth.normal(synth.stream_key(12, batch), batch * hidden)
    Wd, bd, xd = _dev(W), _dev(b), _dev(x)
    logits = torch.zeros(batch * E, dtype=torch.float32, device="cuda")
    rt = spt.Tensor.make("router", spt.TYPE_F32, [hidden, E], Wd.data_ptr(), W.size * 4)
    bt = spt.Tensor.make("router.bias", spt.TYPE_F32, [E], bd.data_ptr(), E * 4)
    gpu_ctx.route_moe_batch(rt, bt, xd, batch, logits)
    torch.cuda.synchronize()
    want = O.route(W, b, x, batch, hidden, E)
    got = logits.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), np.nonzero(got != want)[0][:8]


def test_mxfp4_all_scales(gpu_ctx, O):
    """TestMXFP4AllScales (mxfp4_optimization_test.go:52-78) through the Q8_0
    path: one block per row, every E8M0 exponent, nibbles 0x22 (1.0),
    x = 1/32; exponent 255 with zero nibbles must give NaN.  Row tiles
    holding exponents outside [4, 240] take the integer-decode fallback."""
    import math

    import torch

    import spt

    rows = 257
    data = np.zeros((rows, 17), np.uint8)
    data[:256, 0] = np.arange(256)
    data[:256, 1:] = 0x22
    data[256, 0] = 255
    data = data.reshape(-1)
    x = np.full(32, 1.0 / 32, np.float32)
    wd, xd = _dev(data), _dev(x)
    y = torch.zeros(rows, dtype=torch.float32, device="cuda")
    t = spt.Tensor.make("w", spt.TYPE_MXFP4, [32, rows, 1], wd.data_ptr(), data.size)
    gpu_ctx.mul_mxfp4_expert(t, None, 0, xd, y, 1)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = O.mul_mxfp4_q8(data, _q8_of(O, x), None, 32, rows)
    assert_close(got, want, what="all scales vs Q8_0 oracle")
    assert np.isnan(got[256]) and np.isinf(got[255])
    ref = np.array([math.ldexp(1, s - 127) for s in range(255)], np.float64)
    assert np.all(np.abs(got[:255] - ref) <= 1e-3 * ref), "closed form 2^(s-127)"


def test_mxfp4_large_scales_stay_finite(gpu_ctx, O):
    """One 16-row tile with exponents 239..254 and the largest Q8_0 codes
    (nibbles 0x22, x = 1/32, so q = 127 everywhere): the result 2^(e-127)
    is finite for every row, although the unscaled block sums times
    2^(e-127) exceed the fp32 range for e above 240."""
    import math

    import torch

    import spt

    rows = 16
    data = np.zeros((rows, 17), np.uint8)
    data[:, 0] = np.arange(239, 255)
    data[:, 1:] = 0x22
    data = data.reshape(-1)
    x = np.full(32, 1.0 / 32, np.float32)
    wd, xd = _dev(data), _dev(x)
    y = torch.zeros(rows, dtype=torch.float32, device="cuda")
    t = spt.Tensor.make("w", spt.TYPE_MXFP4, [32, rows, 1], wd.data_ptr(), data.size)
    gpu_ctx.mul_mxfp4_expert(t, None, 0, xd, y, 1)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = O.mul_mxfp4_q8(data, _q8_of(O, x), None, 32, rows)
    assert np.all(np.isfinite(want)) and np.all(np.isfinite(got)), got
    assert_close(got, want, what="large scales vs Q8_0 oracle")
    ref = np.array([math.ldexp(1, s - 127) for s in range(239, 255)], np.float64)
    assert np.all(np.abs(got - ref) <= 1e-3 * ref), "closed form 2^(s-127)"


def test_q40_split_batch_dependence(gpu_ctx, O):
    """The split-K GEMM adds its four K ranges' partial sums in range order,
    so a token's projection may differ in the last bits from the same token
    in a batch large enough for the unsplit GEMM: the O projection
    (4096 -> 2880) of 70 tokens alone (45 x 2 tiles: split) and as the first
    70 of 512 (45 x 8 tiles: unsplit) agree within the oracle's tolerance,
    each against the oracle too.  (With exactly representable sums the two
    agree bit for bit: test_gpu_exact.py.)"""
    import torch

    import spt
    from spt import synth

    din, dout = 4096, 2880
    w = synth.q40_bytes(synth.stream_key(8, dout), dout, din)
    x = synth.normal(synth.stream_key(12, 512), 512 * din)
    wd, xd = _dev(w), _dev(x)
    t = spt.Tensor.make("attn_output", spt.TYPE_Q4_0, [din, dout], wd.data_ptr(), w.size)
    assert spt_split(dout, 70) and not spt_split(dout, 512)
    y70 = torch.zeros(70 * dout, dtype=torch.float32, device="cuda")
    y512 = torch.zeros(512 * dout, dtype=torch.float32, device="cuda")
    gpu_ctx.mul_q40_batch_into(t, xd[:70 * din], y70, 70)
    gpu_ctx.mul_q40_batch_into(t, xd, y512, 512)
    torch.cuda.synchronize()
    a, b = y70.cpu().numpy(), y512.cpu().numpy()[:70 * dout]
    want = O.mul_q40_q8(w, x[:70 * din], din, dout, 70)
    assert_close(a, want, what="split")
    assert_close(b, want, what="unsplit")
    e = assert_close(a, b, what="split vs unsplit")
    ulps = np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))
    print(f"split vs unsplit: {np.count_nonzero(ulps)} of {a.size} differ, max {ulps.max()} ulp, rel {e:.2e}")


def spt_split(rows, ntok):
    """The library's split rule (kQ40SplitMaxTiles = 256 tiles of 64 x 64,
    narrow projections below 1024 rows always)."""
    tiles = ((rows + 63) // 64) * ((ntok + 63) // 64)
    return ntok >= 32 and (rows < 1024 or tiles < 256)


def _at_offset(raw, off):
    """raw's bytes on the device starting `off` bytes past a 256-byte
    aligned allocation (with room past the end): the tensor base the C ABI
    accepts for Q4_0 and Q8_0 data (2-byte aligned) without being 16-byte
    aligned."""
    import torch

    buf = torch.zeros(raw.size + 64, dtype=torch.uint8, device="cuda")
    buf[off:off + raw.size].copy_(torch.from_numpy(np.ascontiguousarray(raw)))
    return buf, buf.data_ptr() + off


@pytest.mark.parametrize("off", [2, 6, 14])
@pytest.mark.parametrize("batch", [1, 8, 70, 300])
def test_q40_unaligned_base(gpu_ctx, O, off, batch):
    """Every Q4_0 launch form (1 token: the few-token launch, 8: the tiled
    MFMA form, 70 and 300: the GEMM) on a weight base 2, 6 or 14 bytes past
    a 16-byte boundary gives the same bits as on an aligned base, and stays
    within tolerance of the oracle."""
    import torch

    import spt
    from spt import synth

    din, dout = 2880, 512
    print(f"q40 base +{off} batch {batch}", flush=True)
    w = synth.q40_bytes(synth.stream_key(8, dout + off), dout, din)
    x = synth.normal(synth.stream_key(9, batch + off), batch * din)
    xd = _dev(x)
    outs = []
    for o in (0, off):
        buf, ptr = _at_offset(w, o)
        t = spt.Tensor.make("attn", spt.TYPE_Q4_0, [din, dout], ptr, w.size)
        y = torch.full((batch * dout,), 12345.0, dtype=torch.float32, device="cuda")
        gpu_ctx.mul_q40_batch_into(t, xd, y, batch)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
        del buf
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert_close(outs[1], O.mul_q40_q8(w, x, din, dout, batch), what="q40 unaligned base")


@pytest.mark.parametrize("off", [1, 3, 10])
@pytest.mark.parametrize("batch", [1, 5])
def test_mxfp4_expert_unaligned_base(gpu_ctx, O, off, batch):
    """MXFP4 expert weights (17-byte blocks, accepted at any byte address)
    whose base is 1, 3 or 10 bytes past a 16-byte boundary give the same
    bits as on an aligned base."""
    import torch

    import spt
    from spt import synth

    din, dout, E, expert = 2880, 2880, 2, 1
    print(f"mxfp4 base +{off} batch {batch}", flush=True)
    w = synth.mxfp4_expert_bytes(synth.stream_key(5, din + off), 0, E * dout * (din // 32))
    x = synth.normal(synth.stream_key(7, batch + off), batch * din)
    xd = _dev(x)
    outs = []
    for o in (0, off):
        buf, ptr = _at_offset(w, o)
        t = spt.Tensor.make("w", spt.TYPE_MXFP4, [din, dout, E], ptr, w.size)
        y = torch.full((batch * dout,), 12345.0, dtype=torch.float32, device="cuda")
        gpu_ctx.mul_mxfp4_expert(t, None, expert, xd, y, batch)
        torch.cuda.synchronize()
        outs.append(y.cpu().numpy())
        del buf
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))

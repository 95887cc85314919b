"""GPU tests of the boundary's other forms against the device forms already
pinned to the oracle:
  - the host-slice entry points a cgo caller binds (spt_forward_moe_batch_host,
    spt_mul_q40_batch_into_host), forwardMoE (spt_forward_moe) and
    spt_tensor_upload: bit-equal to the device forms;
  - the Q8_0-input forms (spt_mul_q40_batch_q8_into, spt_forward_moe_batch_q8)
    and the fused Q/K/V call (spt_mul_q40_qkv_batch_into): bit-equal to the
    fp32-input forms on the input their Q8_0 blocks come from, including the
    blocks the fused RMSNorm writes;
  - the Q8_0-input Q4_0 forms also against the oracle directly."""
import numpy as np
import pytest

from helpers import assert_close, bits

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _zeros(n, dtype=None):
    import torch

    return torch.zeros(n, dtype=dtype or torch.float32, device="cuda")


def _q8(ctx, xd):
    import torch

    q = torch.zeros(xd.numel() // 32 * 34, dtype=torch.uint8, device="cuda")
    ctx.quantize_q8_0(xd, q)
    return q


def _q40(name, din, dout, key):
    import spt
    from spt import synth

    w = synth.q40_bytes(synth.stream_key(key, dout), dout, din)
    wd = _dev(w)
    return w, wd, spt.Tensor.make(name, spt.TYPE_Q4_0, [din, dout], wd.data_ptr(), w.size)


def _f32_bias(name, dout, key):
    import spt
    from spt import synth

    b = synth.normal(synth.stream_key(key, dout), dout)
    bd = _dev(b)
    return b, bd, spt.Tensor.make(name, spt.TYPE_F32, [dout], bd.data_ptr(), dout * 4)


@pytest.mark.parametrize("din,dout,batch", [(2880, 4096, 1), (2880, 512, 32), (4096, 2880, 1), (2880, 4096, 100),
                                            (2880, 512, 300), (96, 70, 5), (8192, 300, 9)])
def test_q40_q8_input_equals_fp32_input(gpu_ctx, O, din, dout, batch):
    """MulQ40BatchInto + bias + residual on GGML Q8_0 blocks: bit-equal to
    the fp32-input call on the x they quantize (GEMV reading the blocks in
    place, GEMM and split-K GEMM on unpacked blocks), and within the Q8_0
    oracle's tolerance."""
    import torch

    from spt import synth

    w, wd, t = _q40("attn_output", din, dout, 21)
    b, bd, bt = _f32_bias("attn_output.bias", dout, 22)
    x = synth.normal(synth.stream_key(23, batch), batch * din)
    xd = _dev(x)
    xq = _q8(gpu_ctx, xd)
    r0 = synth.normal(synth.stream_key(24, batch), batch * dout)
    ra, rb = _dev(r0), _dev(r0)
    ya, yb = _zeros(batch * dout), _zeros(batch * dout)
    gpu_ctx.mul_q40_batch_bias_into(t, bt, xd, ya, batch, ra)
    gpu_ctx.mul_q40_batch_q8_into(t, bt, xq, yb, batch, rb)
    torch.cuda.synchronize()
    assert np.array_equal(bits(ya.cpu().numpy()), bits(yb.cpu().numpy()))
    assert np.array_equal(bits(ra.cpu().numpy()), bits(rb.cpu().numpy()))
    want = O.mul_q40_q8(w, x, din, dout, batch).reshape(batch, dout) + b[None, :]
    assert_close(yb.cpu().numpy(), want.reshape(-1), what="q8-input projection")


@pytest.mark.parametrize("batch", [1, 2, 3, 4])
def test_q40_few_tokens_quantize_in_launch(gpu_ctx, O, batch):
    """Up to four tokens run as one launch that quantizes the fp32 input
    itself: bit-equal to the same call on the input's Q8_0 blocks from the
    quantizer (pinned to the oracle bit for bit), on blocks that exercise
    every rule of the quantization -- all-zero, NaN, Inf, subnormal fp16
    scale, exact .5 ties, -0 -- in the last token, normal blocks before."""
    import torch

    from helpers import tie_block
    from spt import synth

    din, dout = 2880, 512
    w, wd, t = _q40("attn_k", din, dout, 70)
    x = synth.normal(synth.stream_key(71, batch), batch * din) * np.float32(3)
    last = x.reshape(batch, -1, 32)[batch - 1]
    last[0] = 0.0
    last[1, 5] = np.nan
    last[2, 7] = np.inf
    last[3] = np.float32(1e-30)
    last[4] = tie_block()
    last[5] = -0.0
    last[6] = tie_block() * np.float32(0.5)
    xd = _dev(x)
    xq = _q8(gpu_ctx, xd)
    ya, yb = _zeros(batch * dout), _zeros(batch * dout)
    gpu_ctx.mul_q40_batch_into(t, xd, ya, batch)
    gpu_ctx.mul_q40_batch_q8_into(t, None, xq, yb, batch)
    torch.cuda.synchronize()
    assert np.array_equal(xq.cpu().numpy(), O.quantize_q8_0(x))
    assert np.array_equal(bits(ya.cpu().numpy()), bits(yb.cpu().numpy()))
    if batch > 1:  # the tokens of normal blocks against the oracle
        want = O.mul_q40_q8(w, x[:(batch - 1) * din], din, dout, batch - 1)
        assert_close(ya.cpu().numpy()[:(batch - 1) * dout], want, what="few-token projection")


@pytest.mark.parametrize("batch", [1, 3, 32, 300, 512])
@pytest.mark.parametrize("form", ["fp32", "q8"])
def test_q40_qkv_fused(gpu_ctx, O, batch, form):
    """The Q, K, V projections of one normed input in one call (one
    quantization or none, one GEMV launch for all three below the GEMM batch
    sizes): each output bit-equal to its own MulQ40BatchInto + bias call,
    and each against the oracle (at 512 tokens: the long-prompt chunk)."""
    import torch

    from spt import synth

    din = 2880
    mats = [_q40(n, din, d, 30 + i) for i, (n, d) in enumerate((("attn_q", 4096), ("attn_k", 512), ("attn_v", 512)))]
    biases = [_f32_bias(n + ".bias", d, 40 + i) for i, (n, d) in enumerate((("attn_q", 4096), ("attn_k", 512),
                                                                             ("attn_v", 512)))]
    biases[1] = None  # K has no bias: the absent tensor
    x = synth.normal(synth.stream_key(25, batch), batch * din)
    xd = _dev(x)
    want = []
    for (w, wd, t), bb in zip(mats, biases):
        y = _zeros(batch * int(t.shape[1]))
        gpu_ctx.mul_q40_batch_bias_into(t, bb[2] if bb else None, xd, y, batch)
        want.append(y)
    ys = [_zeros(batch * int(t.shape[1])) for _, _, t in mats]
    ws = [t for _, _, t in mats]
    bs = [bb[2] if bb else None for bb in biases]
    if form == "fp32":
        gpu_ctx.mul_q40_qkv_batch_into(ws, bs, xd, ys, batch)
    else:
        gpu_ctx.mul_q40_qkv_batch_into(ws, bs, None, ys, batch, xq=_q8(gpu_ctx, xd), x_len=batch * din)
    torch.cuda.synchronize()
    for i in range(3):
        assert np.array_equal(bits(ys[i].cpu().numpy()), bits(want[i].cpu().numpy())), f"projection {i}"
    for i, name in enumerate("QKV"):
        w, _, t = mats[i]
        dout = int(t.shape[1])
        want_i = O.mul_q40_q8(w, x, din, dout, batch).reshape(batch, dout)
        if biases[i] is not None:
            want_i = want_i + biases[i][0][None, :]
        assert_close(ys[i].cpu().numpy(), want_i.reshape(-1), what=f"fused {name}")


@pytest.mark.parametrize("douts", [(1088, 320, 200), (576, 128, 72), (200, 1100, 90)])
def test_q40_qkv_fused_split_group(gpu_ctx, O, douts):
    """The fused call at 300 tokens with narrow projections of ragged widths:
    those under 1024 rows share one split-K GEMM launch (their partial sums
    side by side in the arena, then one reduce over all of them), each
    output bit-equal to its own call, the last also against the oracle.
    65 blocks per row: the four K ranges end in partial segments."""
    import torch

    from spt import synth

    din, batch = 2080, 300
    names = ("attn_q", "attn_k", "attn_v")
    mats = [_q40(n, din, d, 50 + i) for i, (n, d) in enumerate(zip(names, douts))]
    biases = [_f32_bias(n + ".bias", d, 60 + i) for i, (n, d) in enumerate(zip(names, douts))]
    biases[0] = None
    x = synth.normal(synth.stream_key(26, batch), batch * din)
    xd = _dev(x)
    want = []
    for (w, wd, t), bb in zip(mats, biases):
        y = _zeros(batch * int(t.shape[1]))
        gpu_ctx.mul_q40_batch_bias_into(t, bb[2] if bb else None, xd, y, batch)
        want.append(y)
    ys = [_zeros(batch * d) for d in douts]
    gpu_ctx.mul_q40_qkv_batch_into([t for _, _, t in mats], [bb[2] if bb else None for bb in biases], xd, ys,
                                   batch)
    torch.cuda.synchronize()
    for i in range(3):
        assert np.array_equal(bits(ys[i].cpu().numpy()), bits(want[i].cpu().numpy())), f"projection {i}"
    w, _, _ = mats[2]
    wv = O.mul_q40_q8(w, x, din, douts[2], batch).reshape(batch, douts[2]) + biases[2][0][None, :]
    assert_close(ys[2].cpu().numpy(), wv.reshape(-1), what="fused V")


def test_rmsnorm_q8_feeds_qkv_and_moe(gpu_ctx, O):
    """The fused RMSNorm's Q8_0 output consumed as is: normBatch of 8 rows
    with its GGML blocks, then the fused Q/K/V call and the MoE layer on those
    blocks, each bit-equal to the same calls on the normed fp32 rows."""
    import torch

    import spt
    from spt import synth
    from spt import workloads as W

    batch, dim = 8, 2880
    nw = synth.normal(synth.stream_key(26, 0), dim)
    nwd = _dev(nw)
    nt = spt.Tensor.make("ffn_norm.weight", spt.TYPE_F32, [dim], nwd.data_ptr(), dim * 4)
    h = _dev(synth.normal(synth.stream_key(27, 0), batch * dim) * np.float32(3))
    y = _zeros(batch * dim)
    q8 = _zeros(batch * dim // 32 * 34, torch.uint8)
    gpu_ctx.rmsnorm_batch_into(nt, h, y, batch, 1e-5, q8)
    mats = [_q40(n, dim, d, 50 + i) for i, (n, d) in enumerate((("q", 4096), ("k", 512), ("v", 512)))]
    ws = [t for _, _, t in mats]
    ya = [_zeros(batch * int(t.shape[1])) for t in ws]
    yb = [_zeros(batch * int(t.shape[1])) for t in ws]
    gpu_ctx.mul_q40_qkv_batch_into(ws, None, y, ya, batch)
    gpu_ctx.mul_q40_qkv_batch_into(ws, None, None, yb, batch, xq=q8, x_len=batch * dim)
    shp = W.MoEShape()
    dl = W.device_layer(gpu_ctx, seed=5, layer=0, shp=shp)
    oa, ob = _zeros(batch * dim), _zeros(batch * dim)
    gpu_ctx.forward_moe_batch(dl.config, dl.layer, y, oa, batch)
    gpu_ctx.forward_moe_batch_q8(dl.config, dl.layer, y, q8, ob, batch)
    torch.cuda.synchronize()
    assert np.array_equal(q8.cpu().numpy(), O.quantize_q8_0(y.cpu().numpy()))
    for i in range(3):
        assert np.array_equal(bits(ya[i].cpu().numpy()), bits(yb[i].cpu().numpy())), f"projection {i}"
    assert np.array_equal(bits(oa.cpu().numpy()), bits(ob.cpu().numpy())), "MoE on the RMSNorm's Q8_0"


@pytest.mark.parametrize("batch", [1, 64])
def test_forward_moe_q8_and_host_forms(gpu_ctx, O, batch):
    """One GPT-OSS-shape MoE layer: forwardMoEBatch on device buffers, with
    the Q8_0 of x supplied, through the host-slice form, and (batch 1)
    forwardMoE: the same bits (the device form is pinned to the oracle stage
    by stage in test_gpu_moe.py)."""
    import torch

    from spt import workloads as W

    shp = W.MoEShape()
    dl = W.device_layer(gpu_ctx, seed=6, layer=0, shp=shp)
    x = W.x_tokens(6, 0, batch, shp.hidden)
    xd = _dev(x)
    H = shp.hidden
    o_dev, o_q8 = _zeros(batch * H), _zeros(batch * H)
    gpu_ctx.forward_moe_batch(dl.config, dl.layer, xd, o_dev, batch)
    gpu_ctx.forward_moe_batch_q8(dl.config, dl.layer, xd, _q8(gpu_ctx, xd), o_q8, batch)
    torch.cuda.synchronize()
    o_host = np.full(batch * H, 7.0, np.float32)
    for _ in range(2):  # the second call reuses the grown staging and arena
        gpu_ctx.forward_moe_batch_host(dl.config, dl.layer, x, o_host, batch)
        assert np.array_equal(bits(o_host), bits(o_dev.cpu().numpy()))
    assert np.array_equal(bits(o_q8.cpu().numpy()), bits(o_dev.cpu().numpy()))
    if batch == 1:
        o1 = _zeros(H)
        gpu_ctx.forward_moe(dl.config, dl.layer, xd, o1)
        torch.cuda.synchronize()
        assert np.array_equal(bits(o1.cpu().numpy()), bits(o_dev.cpu().numpy()))


@pytest.mark.parametrize("din,dout,batch", [(2880, 4096, 1), (2880, 512, 32), (2880, 512, 300)])
def test_q40_host_form(gpu_ctx, O, din, dout, batch):
    import torch

    from spt import synth

    w, wd, t = _q40("attn_q", din, dout, 60)
    x = synth.normal(synth.stream_key(61, batch), batch * din)
    yd = _zeros(batch * dout)
    gpu_ctx.mul_q40_batch_into(t, _dev(x), yd, batch)
    torch.cuda.synchronize()
    for _ in range(2):
        yh = np.zeros(batch * dout, np.float32)
        gpu_ctx.mul_q40_batch_into_host(t, x, yh, batch)
        assert np.array_equal(bits(yh), bits(yd.cpu().numpy()))


def test_tensor_upload_round_trip(gpu_ctx, O):
    """spt_tensor_upload copies a tensor's bytes to HBM unchanged; a
    projection through the uploaded tensor matches the one through a copy
    made by torch, bit for bit."""
    import ctypes as C

    import torch

    import spt
    from spt import synth

    din, dout = 2880, 512
    w = synth.q40_bytes(synth.stream_key(62, dout), dout, din)
    t = spt.Tensor.make("blk.0.attn_k.weight", spt.TYPE_Q4_0, [din, dout], None, w.size)
    spt._check(spt.lib().spt_tensor_upload(gpu_ctx.handle, C.byref(t), w.ctypes.data))
    back = np.zeros(w.size, np.uint8)
    spt._check(spt.lib().spt_copy_d2h(gpu_ctx.handle, back.ctypes.data, t.data, w.size))
    assert np.array_equal(back, w)
    x = _dev(synth.normal(synth.stream_key(63, 0), din))
    ya, yb = _zeros(dout), _zeros(dout)
    _, wd, t2 = _q40("blk.0.attn_k.weight", din, dout, 62)
    gpu_ctx.mul_q40_into(t, x, ya)
    gpu_ctx.mul_q40_into(t2, x, yb)
    torch.cuda.synchronize()
    assert np.array_equal(bits(ya.cpu().numpy()), bits(yb.cpu().numpy()))
    spt._check(spt.lib().spt_free(gpu_ctx.handle, t.data))

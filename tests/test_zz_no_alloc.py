"""spt_forward_moe_batch_noalloc, the forwardMoEBatch form that allocates
nothing (its scratch is a fixed device array per GPU): through the C ABI,
called first on a freshly created context, whose arena and staging stay
empty (spt_ctx_memory) through every call; two calls in a row, the second
with a smaller batch, each bit-equal to spt_forward_moe_batch of another
context on the same inputs; a 260-token GPT-OSS batch (1,040 selections)
that takes the grouped GEMM on the context's second stream; and a batch
beyond its array rejected before any launch."""
import ctypes as C

import numpy as np
import pytest

from fixtures import device_moe_layer, moe_batch_fixture, moe_batch_x
from helpers import bits

pytestmark = pytest.mark.gpu


def _noalloc(ctx, cfg, lw, x, out, batch):
    import spt

    return spt.lib().spt_forward_moe_batch_noalloc(ctx.handle, C.byref(cfg), C.byref(lw), x.data_ptr(), x.numel(),
                                                   out.data_ptr(), out.numel(), batch)


@pytest.fixture()
def fresh_ctx():
    """A new context on torch's current stream: nothing allocated yet."""
    import torch

    import spt

    ctx = spt.Context(0, torch.cuda.current_stream().cuda_stream)
    assert ctx.memory() == (0, 0)
    yield ctx
    ctx.close()


def _check_calls(fresh, ref_ctx, cfg, lw, xs, H):
    """The no-allocation calls on `fresh` first, then the allocating form on
    ref_ctx, each batch compared bit for bit; `fresh` never allocates."""
    import torch

    import spt

    gots = []
    for x, batch in xs:
        got = torch.full((batch * H,), -5.0, dtype=torch.float32, device="cuda")
        rc = _noalloc(fresh, cfg, lw, x, got, batch)
        assert rc == spt.OK, spt.lib().spt_last_error()
        gots.append(got)
    torch.cuda.synchronize()
    assert fresh.memory() == (0, 0), "the no-allocation form grew the context's arena or staging"
    for (x, batch), got in zip(xs, gots):
        ref = torch.full((batch * H,), 5.0, dtype=torch.float32, device="cuda")
        ref_ctx.forward_moe_batch(cfg, lw, x, ref, batch)
        torch.cuda.synchronize()
        assert np.array_equal(bits(got.cpu().numpy()), bits(ref.cpu().numpy())), f"batch {batch}"


def test_noalloc_gpt_oss_layer(gpu_ctx, fresh_ctx):
    """GPT-OSS-120B layer: 260 tokens (grouped GEMM for the groups of nine or
    more, on the second stream), then 64 and 8 (grouped GEMV): the array
    keeps the previous call's contents between calls."""
    import torch

    import spt
    from spt import workloads as W

    shp = W.MoEShape()
    dl = W.device_layer(gpu_ctx, seed=7, layer=0, shp=shp)
    xs = [(torch.from_numpy(W.x_tokens(7, 0, b, shp.hidden)).cuda(), b) for b in (260, 64, 8)]
    # the 260-token batch does reach the GEMM: at least n_cu / 23 experts
    # hold nine or more selections (23 row units of 128 per expert)
    n = 260 * shp.topk
    counts = torch.zeros(shp.experts, dtype=torch.int32, device="cuda")
    out = torch.empty(260 * shp.hidden, dtype=torch.float32, device="cuda")
    gpu_ctx.forward_moe_batch(dl.config, dl.layer, xs[0][0], out, 260, spt.make_taps(counts=counts))
    torch.cuda.synchronize()
    assert n >= 1024 and int((counts >= 9).sum()) * 23 >= 256
    _check_calls(fresh_ctx, gpu_ctx, dl.config, dl.layer, xs, shp.hidden)


def test_noalloc_reference_fixture(gpu_ctx, fresh_ctx):
    lay = moe_batch_fixture(96, 64, 8, 2, 0, "mixed-nan")
    keep, cfg, lw = device_moe_layer(lay)
    import torch

    xs = [(torch.from_numpy(moe_batch_x(b, 96, "mixed-nan")).cuda(), b) for b in (37, 5)]
    _check_calls(fresh_ctx, gpu_ctx, cfg, lw, xs, 96)


def test_noalloc_rejects_oversized_batch(gpu_ctx, fresh_ctx):
    import torch

    import spt
    from spt import workloads as W

    shp = W.MoEShape()
    dl = W.device_layer(gpu_ctx, seed=7, layer=0, shp=shp)
    batch = 300
    x = torch.zeros(batch * shp.hidden, dtype=torch.float32, device="cuda")
    out = torch.full((batch * shp.hidden,), 3.0, dtype=torch.float32, device="cuda")
    rc = _noalloc(fresh_ctx, dl.config, dl.layer, x, out, batch)
    torch.cuda.synchronize()
    assert rc == spt.ERR_INVALID and b"no-allocation form holds" in spt.lib().spt_last_error()
    assert bool(torch.all(out == 3.0))  # nothing was launched
    assert fresh_ctx.memory() == (0, 0)

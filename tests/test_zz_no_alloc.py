"""spt_forward_moe_batch_noalloc, the forwardMoEBatch form that allocates
nothing (its scratch is a fixed device array per GPU): through the C ABI,
two calls in a row, the second with a smaller batch, each bit-equal to
spt_forward_moe_batch on the same inputs; and a batch beyond its array
rejected before any launch."""
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


def _check_pair(ctx, cfg, lw, x, batch, H):
    import torch

    import spt

    ref = torch.full((batch * H,), 5.0, dtype=torch.float32, device="cuda")
    got = torch.full((batch * H,), -5.0, dtype=torch.float32, device="cuda")
    ctx.forward_moe_batch(cfg, lw, x, ref, batch)
    rc = _noalloc(ctx, cfg, lw, x, got, batch)
    assert rc == spt.OK, spt.lib().spt_last_error()
    torch.cuda.synchronize()
    assert np.array_equal(bits(got.cpu().numpy()), bits(ref.cpu().numpy())), f"batch {batch}"


def test_noalloc_gpt_oss_layer(gpu_ctx):
    import torch

    from spt import workloads as W

    shp = W.MoEShape()
    dl = W.device_layer(gpu_ctx, seed=7, layer=0, shp=shp)
    for batch in (64, 8):  # the second call smaller: the array keeps the first call's contents
        x = torch.from_numpy(W.x_tokens(7, 0, batch, shp.hidden)).cuda()
        _check_pair(gpu_ctx, dl.config, dl.layer, x, batch, shp.hidden)


def test_noalloc_reference_fixture(gpu_ctx):
    import torch

    lay = moe_batch_fixture(96, 64, 8, 2, 0, "mixed-nan")
    keep, cfg, lw = device_moe_layer(lay)
    for batch in (37, 5):
        x = torch.from_numpy(moe_batch_x(batch, 96, "mixed-nan")).cuda()
        _check_pair(gpu_ctx, cfg, lw, x, batch, 96)


def test_noalloc_rejects_oversized_batch(gpu_ctx):
    import torch

    import spt
    from spt import workloads as W

    shp = W.MoEShape()
    dl = W.device_layer(gpu_ctx, seed=7, layer=0, shp=shp)
    batch = 300
    x = torch.zeros(batch * shp.hidden, dtype=torch.float32, device="cuda")
    out = torch.full((batch * shp.hidden,), 3.0, dtype=torch.float32, device="cuda")
    rc = _noalloc(gpu_ctx, dl.config, dl.layer, x, out, batch)
    torch.cuda.synchronize()
    assert rc == spt.ERR_INVALID and b"no-allocation form holds" in spt.lib().spt_last_error()
    assert bool(torch.all(out == 3.0))  # nothing was launched

"""GPU tests of the GGUF residency loader: a model file written by the test
(one MoE layer of moeBatchFixture, a Q4_0 projection, a shared Q8_0 head
and a tensor larger than the loader's staging) opened with spt_gguf_open,
its tensors uploaded with spt_gguf_upload / spt_gguf_upload_moe_layer:
every uploaded byte equal to the file's, and the MoE layer and projection
computed through the uploaded tensors bit-equal to the same computation on
copies made by torch (pinned to the oracle in test_gpu_moe.py and
test_gpu_kernels.py), and within the oracle's tolerance."""
import numpy as np
import pytest

from fixtures import device_moe_layer, moe_batch_fixture, moe_batch_x
from gguf_file import F32, STRING, U32, gstr, u32, write
from helpers import assert_close, bits

pytestmark = pytest.mark.gpu

H, D, E, K = 96, 64, 4, 2


def _layer_tensors(lay, prefix="blk.0."):
    """The fixture's layer as GGUF tensors (names of forward/layer.go:40-85,
    shapes [in, out, experts])."""
    ts = [(prefix + "ffn_gate_inp.weight", 0, [H, E], lay["router"].tobytes()),
          (prefix + "ffn_gate_exps.weight", 39, [H, D, E], lay["gate"].tobytes()),
          (prefix + "ffn_up_exps.weight", 39, [H, D, E], lay["up"].tobytes()),
          (prefix + "ffn_down_exps.weight", 39, [D, H, E], lay["down"].tobytes())]
    for name, key, shape in (("ffn_gate_inp.bias", "router_bias", [E]), ("ffn_gate_exps.bias", "gate_bias", [D, E]),
                             ("ffn_up_exps.bias", "up_bias", [D, E]), ("ffn_down_exps.bias", "down_bias", [H, E])):
        if lay.get(key) is not None:
            arr, typ = lay[key]
            ts.append((prefix + name, typ, shape, np.ascontiguousarray(arr).tobytes()))
    return ts


def _read_back(ctx, t):
    import spt

    out = np.zeros(int(t.nbytes), np.uint8)
    spt._check(spt.lib().spt_copy_d2h(ctx.handle, out.ctypes.data, t.data, int(t.nbytes)))
    return out.tobytes()


def _free(ctx, t):
    import spt

    if t.data:
        spt._check(spt.lib().spt_free(ctx.handle, t.data))


@pytest.mark.parametrize("bias_type", [-1, 0, 1])
def test_gguf_moe_layer_upload_and_forward(gpu_ctx, O, tmp_path, bias_type):
    import torch

    import spt
    from spt import synth

    lay = moe_batch_fixture(H, D, E, K, bias_type, "normal")
    q40 = synth.q40_bytes(synth.stream_key(80, 128), 128, H)
    head = np.frombuffer(synth.normal(synth.stream_key(81, 0), 64 * 34 // 4).tobytes(), np.uint8).copy()
    head[0::34] = 0x10   # finite fp16 scales
    head[1::34] = 0x20
    big = synth.normal(synth.stream_key(82, 0), 5_000_003)  # > two 8 MiB staging chunks, odd size
    tensors = _layer_tensors(lay) + [
        ("blk.0.attn_q.weight", 2, [H, 128], q40.tobytes()),
        ("output.weight", 8, [64, 32], head[:64 * 32 // 32 * 34].tobytes()),
        ("token_embd.weight", 0, [5_000_003], big.tobytes()),
    ]
    path = tmp_path / "model.gguf"
    data, ranges = write(path, [("general.architecture", STRING, gstr("gpt-oss")),
                                ("gpt_oss.block_count", U32, u32(1))], tensors)
    with spt.Gguf(str(path)) as g:
        lw = g.upload_moe_layer(gpu_ctx, 0)
        uploaded = []
        try:
            # every field: the file's bytes, name, type and shape
            want = {t[0]: (t, r) for t, r in zip(tensors, ranges)}
            for field, _ in spt.MoELayer._fields_:
                t = getattr(lw, field)
                if not t.name:
                    assert bias_type == -1 and field.endswith("_bias") and not t.data and t.nbytes == 0
                    continue
                (name, typ, shape, blob), (a, b) = want[t.name.decode()]
                suffix = field[:-5] + ".bias" if field.endswith("_bias") else field + ".weight"
                assert name == "blk.0." + suffix
                assert (t.type, t.n_dims, [int(t.shape[i]) for i in range(t.n_dims)], t.nbytes) == \
                    (typ, len(shape), shape, b - a)
                assert _read_back(gpu_ctx, t) == blob == data[a:b]
            qt = g.upload(gpu_ctx, "blk.0.attn_q.weight")
            uploaded.append(qt)
            ht = g.upload(gpu_ctx, "output.weight")
            uploaded.append(ht)
            bt = g.upload(gpu_ctx, "token_embd.weight")
            uploaded.append(bt)
            for t in uploaded:
                (name, typ, shape, blob), _ = want[t.name.decode()]
                assert _read_back(gpu_ctx, t) == blob
            with pytest.raises(spt.SptError) as e:
                g.upload(gpu_ctx, "absent.weight")
            assert e.value.code == spt.ERR_NOT_FOUND

            # the MoE layer through the uploaded tensors: bit-equal to the
            # layer uploaded by torch, and the oracle's result within tolerance
            keep, cfg, lw_ref = device_moe_layer(lay)
            for batch in (1, 5, 37):
                x = moe_batch_x(batch, H, "normal")
                xd = torch.from_numpy(x).cuda()
                oa = torch.zeros(batch * H, dtype=torch.float32, device="cuda")
                ob = torch.zeros_like(oa)
                gpu_ctx.forward_moe_batch(cfg, lw, xd, oa, batch)
                gpu_ctx.forward_moe_batch(cfg, lw_ref, xd, ob, batch)
                torch.cuda.synchronize()
                assert np.array_equal(bits(oa.cpu().numpy()), bits(ob.cpu().numpy())), batch
                assert_close(oa.cpu().numpy(), O.forward_moe_batch(lay, x, batch, q8=True), what=f"batch {batch}")
            # the Q4_0 projection and the Q8_0 head likewise
            xq = synth.normal(synth.stream_key(83, 0), 3 * H)
            xd = torch.from_numpy(xq).cuda()
            wd = torch.from_numpy(q40).cuda()
            tq = spt.Tensor.make("blk.0.attn_q.weight", spt.TYPE_Q4_0, [H, 128], wd.data_ptr(), q40.size)
            ya = torch.zeros(3 * 128, dtype=torch.float32, device="cuda")
            yb = torch.zeros_like(ya)
            gpu_ctx.mul_q40_batch_into(qt, xd, ya, 3)
            gpu_ctx.mul_q40_batch_into(tq, xd, yb, 3)
            torch.cuda.synchronize()
            assert np.array_equal(bits(ya.cpu().numpy()), bits(yb.cpu().numpy()))
            assert_close(ya.cpu().numpy(), O.mul_q40_q8(q40, xq, H, 128, 3), what="q40 from GGUF")
            hb = head[:64 * 32 // 32 * 34].copy()
            hd = torch.from_numpy(hb).cuda()
            th = spt.Tensor.make("output.weight", spt.TYPE_Q8_0, [64, 32], hd.data_ptr(), hb.size)
            xh = torch.from_numpy(synth.normal(synth.stream_key(84, 0), 64)).cuda()
            za = torch.zeros(32, dtype=torch.float32, device="cuda")
            zb = torch.zeros_like(za)
            gpu_ctx.mul_q80_into(ht, xh, za)
            gpu_ctx.mul_q80_into(th, xh, zb)
            torch.cuda.synchronize()
            assert np.array_equal(bits(za.cpu().numpy()), bits(zb.cpu().numpy()))
        finally:
            for f, _ in spt.MoELayer._fields_:
                _free(gpu_ctx, getattr(lw, f))
            for t in uploaded:
                _free(gpu_ctx, t)


def test_gguf_upload_refuses_wide_tensors(gpu_ctx, tmp_path):
    """spt_tensor holds four dimensions: a five-dimensional tensor is
    refused, with nothing left allocated."""
    import spt

    path = tmp_path / "five.gguf"
    write(path, [], [("w", F32, [2, 2, 2, 2, 2], bytes(128))])
    with spt.Gguf(str(path)) as g:
        assert g.find("w").n_dims == 5
        with pytest.raises(spt.SptError) as e:
            g.upload(gpu_ctx, "w")
        assert e.value.code == spt.ERR_INVALID and "dimensions" in e.value.message

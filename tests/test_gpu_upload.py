"""GPU tests of residency from the model files (spt_upload_range): tensors
written at 32-byte-aligned offsets of a file, as a GGUF file's data section
holds them (one MoE layer of moeBatchFixture, a Q4_0 projection, a Q8_0 head
and a tensor larger than the two 8 MiB staging halves), each uploaded from
its (path, start, end) range with the descriptor a ggufindex.Tensor gives:
every uploaded byte equal to the file's, and the MoE layer, the projection
and the head computed through the uploaded tensors bit-equal to the same on
copies made by torch (those are pinned to the oracle in test_gpu_moe.py,
test_gpu_kernels.py and test_gpu_q80.py) and within the oracle's tolerance.
The range's refusals: a missing file, a range past the end of the file, a
reversed range, a size that does not match the type and shape, and more
than four dimensions."""
import numpy as np
import pytest

from fixtures import device_moe_layer, moe_batch_fixture, moe_batch_x
from helpers import assert_close, bits

pytestmark = pytest.mark.gpu

H, D, E, K = 96, 64, 4, 2


def _write(path, tensors, lead=1000):
    """Tensors (name, type, shape, bytes) at 32-byte-aligned offsets after
    `lead` bytes of other content; returns the file bytes and each range."""
    rng = np.random.default_rng(5)
    blob = bytearray(rng.integers(0, 256, size=lead, dtype=np.uint8).tobytes())
    ranges = []
    for _, _, _, b in tensors:
        blob += bytes((-len(blob)) % 32)
        ranges.append((len(blob), len(blob) + len(b)))
        blob += b
    blob += b"trailing"
    path.write_bytes(bytes(blob))
    return bytes(blob), ranges


def _layer_tensors(lay):
    """The fixture's layer under the names and shapes of forward/layer.go:40-85
    ([in, out, experts])."""
    ts = [("blk.0.ffn_gate_inp.weight", 0, [H, E], lay["router"].tobytes()),
          ("blk.0.ffn_gate_exps.weight", 39, [H, D, E], lay["gate"].tobytes()),
          ("blk.0.ffn_up_exps.weight", 39, [H, D, E], lay["up"].tobytes()),
          ("blk.0.ffn_down_exps.weight", 39, [D, H, E], lay["down"].tobytes())]
    for name, key, shape in (("ffn_gate_inp.bias", "router_bias", [E]), ("ffn_gate_exps.bias", "gate_bias", [D, E]),
                             ("ffn_up_exps.bias", "up_bias", [D, E]), ("ffn_down_exps.bias", "down_bias", [H, E])):
        if lay.get(key) is not None:
            arr, typ = lay[key]
            ts.append(("blk.0." + name, typ, shape, np.ascontiguousarray(arr).tobytes()))
    return ts


FIELDS = {"ffn_gate_inp.weight": "ffn_gate_inp", "ffn_gate_inp.bias": "ffn_gate_inp_bias",
          "ffn_gate_exps.weight": "ffn_gate_exps", "ffn_gate_exps.bias": "ffn_gate_exps_bias",
          "ffn_up_exps.weight": "ffn_up_exps", "ffn_up_exps.bias": "ffn_up_exps_bias",
          "ffn_down_exps.weight": "ffn_down_exps", "ffn_down_exps.bias": "ffn_down_exps_bias"}


def _read_back(ctx, t):
    import spt

    out = np.zeros(int(t.nbytes), np.uint8)
    spt._check(spt.lib().spt_copy_d2h(ctx.handle, out.ctypes.data, t.data, int(t.nbytes)))
    return out.tobytes()


@pytest.mark.parametrize("bias_type", [-1, 0, 1])
def test_upload_range_moe_layer_and_forward(gpu_ctx, O, tmp_path, bias_type):
    import torch

    import spt
    from spt import synth

    lay = moe_batch_fixture(H, D, E, K, bias_type, "normal")
    q40 = synth.q40_bytes(synth.stream_key(80, 128), 128, H)
    head = np.frombuffer(synth.normal(synth.stream_key(81, 0), 64 * 34 // 4).tobytes(), np.uint8).copy()
    head[0::34] = 0x10   # finite fp16 scales
    head[1::34] = 0x20
    head = head[:64 * 32 // 32 * 34]
    big = synth.normal(synth.stream_key(82, 0), 5_000_003)  # > two 8 MiB staging chunks, odd size
    tensors = _layer_tensors(lay) + [
        ("blk.0.attn_q.weight", 2, [H, 128], q40.tobytes()),
        ("output.weight", 8, [64, 32], head.tobytes()),
        ("token_embd.weight", 0, [5_000_003], big.tobytes()),
    ]
    path = tmp_path / "model.bin"
    data, ranges = _write(path, tensors)
    up = {}
    try:
        for (name, typ, shape, blob), (a, b) in zip(tensors, ranges):
            t = gpu_ctx.upload_range(path, a, b, name, typ, shape)
            up[name] = t
            assert (t.name.decode(), t.type, t.n_dims, [int(t.shape[i]) for i in range(t.n_dims)], t.nbytes) == \
                (name, typ, len(shape), shape, b - a)
            assert _read_back(gpu_ctx, t) == blob == data[a:b]
        assert gpu_ctx.memory()[1] >= 2 * (8 << 20)  # the two staging halves
        lw = spt.MoELayer()
        for name, field in FIELDS.items():
            if "blk.0." + name in up:
                setattr(lw, field, up["blk.0." + name])
        # the MoE layer through the uploaded tensors: bit-equal to the layer
        # uploaded by torch, and the oracle's result within tolerance
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
        gpu_ctx.mul_q40_batch_into(up["blk.0.attn_q.weight"], xd, ya, 3)
        gpu_ctx.mul_q40_batch_into(tq, xd, yb, 3)
        torch.cuda.synchronize()
        assert np.array_equal(bits(ya.cpu().numpy()), bits(yb.cpu().numpy()))
        assert_close(ya.cpu().numpy(), O.mul_q40_q8(q40, xq, H, 128, 3), what="q40 from the file")
        hd = torch.from_numpy(head).cuda()
        th = spt.Tensor.make("output.weight", spt.TYPE_Q8_0, [64, 32], hd.data_ptr(), head.size)
        xh = torch.from_numpy(synth.normal(synth.stream_key(84, 0), 64)).cuda()
        za = torch.zeros(32, dtype=torch.float32, device="cuda")
        zb = torch.zeros_like(za)
        gpu_ctx.mul_q80_into(up["output.weight"], xh, za)
        gpu_ctx.mul_q80_into(th, xh, zb)
        torch.cuda.synchronize()
        assert np.array_equal(bits(za.cpu().numpy()), bits(zb.cpu().numpy()))
        assert_close(za.cpu().numpy(), O.mul_q80_f32(head, xh.cpu().numpy(), 64, 32), what="q80 from the file")
    finally:
        for t in up.values():
            gpu_ctx.free(t.data)


def test_upload_range_refusals(gpu_ctx, tmp_path):
    import spt

    path = tmp_path / "small.bin"
    _, ((a, b),) = _write(path, [("w", 0, [8], np.arange(8, dtype=np.float32).tobytes())], lead=40)
    cases = [
        (str(tmp_path / "absent.bin"), a, b, [8], 0, spt.ERR_IO, "open"),
        (path, a, b + 4096, [8 + 1024], 0, spt.ERR_IO, "end of file"),
        (path, b, a, [8], 0, spt.ERR_INVALID, "invalid byte range"),
        (path, a, b, [9], 0, spt.ERR_INVALID, "does not match"),
        (path, a, b, [16], 1, spt.ERR_INVALID, "does not match"),   # F16: 32 bytes hold 16, shape says so: ok below
        (path, a, b, [33, 1], 2, spt.ERR_INVALID, "does not match"),  # not a whole number of Q4_0 blocks
    ]
    for p, s, e, shape, typ, code, msg in cases:
        if typ == 1:  # the F16 reading of the same 32 bytes is valid
            t = gpu_ctx.upload_range(p, s, e, "w16", typ, shape)
            gpu_ctx.free(t.data)
            continue
        with pytest.raises(spt.SptError) as err:
            gpu_ctx.upload_range(p, s, e, "w", typ, shape)
        assert err.value.code == code and msg in err.value.message, (shape, err.value.message)
    t = spt.Tensor.make("w5", spt.TYPE_F32, [2, 2, 2, 1], None, 0)
    t.n_dims = 5
    rc = spt.lib().spt_upload_range(gpu_ctx.handle, str(path).encode(), a, b, t)
    assert rc == spt.ERR_INVALID and b"dimensions" in spt.lib().spt_last_error()

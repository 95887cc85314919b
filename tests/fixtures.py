"""Deterministic fixtures of the reference's own tests, regenerated from their
formulas (the reference writes them to a temp file; here they are arrays).

moe_batch_fixture: tests/testdata/forward/moe_batch_test.go:20-111
moe_batch_x:       tests/testdata/forward/moe_batch_test.go:134-139
quant_optimization_fixture:
                   tests/testdata/forward/quant_optimization_test.go:25-56
"""
import numpy as np

def quant_optimization_fixture(typ, input_dim, output_dim):
    """Q4_0 (typ 2) or Q8_0 (typ 8) [input, output] bytes: block g's fp16
    scale cycles through eight values (normal, negative, subnormal, the
    largest finite, -0), byte j of its payload is (13g + 7(j+2)) & 0xFF."""
    bb = 18 if typ == 2 else 34
    nblk = input_dim // 32 * output_dim
    scales = np.array([0x3C00, 0xB800, 0x3400, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0x8000], np.uint16)
    data = np.zeros((nblk, bb), np.uint8)
    data[:, 0:2] = scales[np.arange(nblk) % 8].view(np.uint8).reshape(nblk, 2)
    data[:, 2:] = ((np.arange(nblk)[:, None] * 13 + np.arange(2, bb)[None, :] * 7) & 0xFF).astype(np.uint8)
    return data.reshape(-1)


ROUTER_MODES = ("normal", "ties", "nonfinite", "mixed-nan", "infinite", "underflow", "clamp")


def _quantized(input_dim, output_dim, experts, salt):
    n = input_dim // 32 * 17 * output_dim * experts
    block = np.arange(n // 17, dtype=np.int64)
    enc = np.empty((n // 17, 17), np.uint8)
    enc[:, 0] = (120 + (block + salt) % 4).astype(np.uint8)
    i = np.arange(1, 17, dtype=np.int64)
    enc[:, 1:] = ((block[:, None] * 13 + i[None, :] * 7 + salt) & 0xFF).astype(np.uint8)
    return enc.reshape(-1)


def _bias(dim, count, bias_type):
    i = np.arange(dim * count)
    value = ((i % 5) - 2).astype(np.float32) / 4
    if bias_type == 0:
        return value.astype(np.float32)
    if bias_type == 30:
        return (value.view(np.uint32) >> 16).astype(np.uint16)
    bits = np.array([0xB800, 0xB400, 0, 0x3400, 0x3800], np.uint16)
    return bits[i % 5]


def moe_batch_fixture(hidden, expert_dim, experts, topk, bias_type, mode):
    """Layer dict in oracle.forward_moe_batch format (bias_type -1: none)."""
    e = np.arange(experts)[:, None]
    i = np.arange(hidden)[None, :]
    router = (((e * 7 + i * 3) % 19) - 9).astype(np.float32) / 32
    if mode == "ties":
        router[:] = 0
    elif mode == "nonfinite":
        router[:] = np.nan
    elif mode == "mixed-nan":
        router[:] = np.nan
        if experts > 1:
            router[1] = 0
    elif mode == "infinite":
        router[:] = np.inf
    elif mode == "underflow":
        router = np.broadcast_to((e * 1000).astype(np.float32), (experts, hidden)).copy()
    lay = {"hidden": hidden, "expert_dim": expert_dim, "experts": experts, "topk": topk,
           "router": router.reshape(-1).astype(np.float32),
           "gate": _quantized(hidden, expert_dim, experts, 1),
           "up": _quantized(hidden, expert_dim, experts, 7),
           "down": _quantized(expert_dim, hidden, experts, 17)}
    if bias_type >= 0:
        lay["router_bias"] = (_bias(experts, 1, bias_type), bias_type)
        lay["gate_bias"] = (_bias(expert_dim, experts, bias_type), bias_type)
        lay["up_bias"] = (_bias(expert_dim, experts, bias_type), bias_type)
        lay["down_bias"] = (_bias(hidden, experts, bias_type), bias_type)
    return lay


def moe_batch_x(batch, hidden, mode):
    i = np.arange(batch * hidden)
    x = (((i * 17 + i // hidden) % 31) - 15).astype(np.float32) / 16
    if mode == "clamp":
        x = x * 1000
    return x.astype(np.float32)


def device_moe_layer(lay):
    """Upload an oracle-format layer; returns (keepalive, MoEConfig, MoELayer)."""
    import torch

    import spt

    H, D, E, k = lay["hidden"], lay["expert_dim"], lay["experts"], lay["topk"]
    keep = {}

    def up(name, arr):
        keep[name] = torch.from_numpy(np.ascontiguousarray(arr)).cuda()
        return keep[name]

    lw = spt.MoELayer()
    r = up("router", lay["router"])
    lw.ffn_gate_inp = spt.Tensor.make("router", spt.TYPE_F32, [H, E], r.data_ptr(), H * E * 4)
    for field, name, shape in (("ffn_gate_exps", "gate", [H, D, E]), ("ffn_up_exps", "up", [H, D, E]),
                               ("ffn_down_exps", "down", [D, H, E])):
        t = up(name, lay[name])
        setattr(lw, field, spt.Tensor.make(name, spt.TYPE_MXFP4, shape, t.data_ptr(), t.numel()))
    for field, name, shape in (("ffn_gate_inp_bias", "router_bias", [E]),
                               ("ffn_gate_exps_bias", "gate_bias", [D, E]),
                               ("ffn_up_exps_bias", "up_bias", [D, E]),
                               ("ffn_down_exps_bias", "down_bias", [H, E])):
        if lay.get(name) is None:
            continue
        arr, typ = lay[name]
        t = up(name, arr)
        setattr(lw, field, spt.Tensor.make(name, typ, shape, t.data_ptr(), t.numel() * t.element_size()))
    cfg = spt.MoEConfig()
    cfg.hidden_dim, cfg.expert_hidden_dim, cfg.num_experts, cfg.num_experts_used = H, D, E, k
    return keep, cfg, lw

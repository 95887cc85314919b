"""Synthetic GPT-OSS-120B-shape MoE layers and Q4_0 projections.

Shapes (forward/config.go:57-75): hidden 2880, expert hidden 2880, 128
experts, 4 used.  Every tensor comes from spt.synth keyed by (seed, stream),
so the host (oracle) and the device hold identical bytes; MXFP4 expert
tensors are generated directly in HBM by spt_synth_mxfp4 and the host
regenerates only the experts it needs.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import synth

HIDDEN, EXPERT_DIM, EXPERTS, TOPK = 2880, 2880, 128, 4

# stream ids inside one layer
S_ROUTER, S_ROUTER_BIAS, S_GATE, S_GATE_BIAS, S_UP, S_UP_BIAS, S_DOWN, S_DOWN_BIAS, S_X = range(1, 10)
S_Q, S_K, S_V, S_O = 11, 12, 13, 14


def key(seed: int, layer: int, stream: int) -> int:
    return synth.stream_key(seed, layer * 64 + stream)


@dataclass
class MoEShape:
    hidden: int = HIDDEN
    expert_dim: int = EXPERT_DIM
    experts: int = EXPERTS
    topk: int = TOPK
    biases: bool = True

    @property
    def gate_bytes(self) -> int:  # one expert's gate (or up) matrix
        return self.hidden // 32 * 17 * self.expert_dim

    @property
    def down_bytes(self) -> int:
        return self.expert_dim // 32 * 17 * self.hidden


def x_tokens(seed: int, layer: int, batch: int, hidden: int) -> np.ndarray:
    """x ~ N(0,1), RMS-normalised per token, float32 [batch*hidden]."""
    x = synth.normal(key(seed, layer, S_X), batch * hidden).reshape(batch, hidden)
    return synth.rms_normalize(x).reshape(-1)


def host_small_tensors(seed: int, layer: int, shp: MoEShape) -> dict:
    """Router, router bias and expert biases (all N(0, 0.02)) on the host."""
    H, D, E = shp.hidden, shp.expert_dim, shp.experts
    out = {"router": synth.normal(key(seed, layer, S_ROUTER), E * H, 0.0, 0.02)}
    if shp.biases:
        out["router_bias"] = synth.normal(key(seed, layer, S_ROUTER_BIAS), E, 0.0, 0.02)
        out["gate_bias"] = synth.normal(key(seed, layer, S_GATE_BIAS), E * D, 0.0, 0.02)
        out["up_bias"] = synth.normal(key(seed, layer, S_UP_BIAS), E * D, 0.0, 0.02)
        out["down_bias"] = synth.normal(key(seed, layer, S_DOWN_BIAS), E * H, 0.0, 0.02)
    return out


def host_expert(seed: int, layer: int, shp: MoEShape, which: str, expert: int) -> np.ndarray:
    """Bytes of one expert matrix of gate/up/down, as generated in HBM."""
    stream = {"gate": S_GATE, "up": S_UP, "down": S_DOWN}[which]
    nbytes = shp.down_bytes if which == "down" else shp.gate_bytes
    nblocks = nbytes // 17
    return synth.mxfp4_expert_bytes(key(seed, layer, stream), expert * nblocks, nblocks)


def host_layer(seed: int, layer: int, shp: MoEShape, experts=None) -> dict:
    """Oracle-side layer dict (oracle.forward_moe_batch format).  Experts not
    listed in `experts` are left as zeros (they are never read when the
    routing does not select them)."""
    small = host_small_tensors(seed, layer, shp)
    E = shp.experts
    sel = range(E) if experts is None else sorted(set(int(e) for e in experts))
    lay = {"hidden": shp.hidden, "expert_dim": shp.expert_dim, "experts": E, "topk": shp.topk,
           "router": small["router"]}
    for which, nbytes in (("gate", shp.gate_bytes), ("up", shp.gate_bytes), ("down", shp.down_bytes)):
        buf = np.zeros(E * nbytes, np.uint8)
        for e in sel:
            buf[e * nbytes:(e + 1) * nbytes] = host_expert(seed, layer, shp, which, e)
        lay[which] = buf
    if shp.biases:
        for n in ("router_bias", "gate_bias", "up_bias", "down_bias"):
            lay[n] = (small[n], 0)
    return lay


@dataclass
class DeviceMoELayer:
    """Device tensors of one MoE layer plus the C descriptors."""
    shape: MoEShape
    tensors: dict = field(default_factory=dict)
    layer: object = None
    config: object = None


def device_layer(ctx, seed: int, layer: int, shp: MoEShape, device="cuda") -> DeviceMoELayer:
    import torch

    from . import MoEConfig, MoELayer, Tensor, TYPE_F32, TYPE_MXFP4

    H, D, E = shp.hidden, shp.expert_dim, shp.experts
    small = host_small_tensors(seed, layer, shp)
    dl = DeviceMoELayer(shape=shp)
    t = dl.tensors
    t["router"] = torch.from_numpy(small["router"]).to(device)
    for which, stream, nbytes in (("gate", S_GATE, shp.gate_bytes), ("up", S_UP, shp.gate_bytes),
                                  ("down", S_DOWN, shp.down_bytes)):
        buf = torch.empty(E * nbytes, dtype=torch.uint8, device=device)
        ctx.synth_mxfp4(buf, key(seed, layer, stream), 0, E * nbytes // 17)
        t[which] = buf
    lw = MoELayer()
    lw.ffn_gate_inp = Tensor.make("blk.ffn_gate_inp.weight", TYPE_F32, [H, E], t["router"].data_ptr(), H * E * 4)
    lw.ffn_gate_exps = Tensor.make("blk.ffn_gate_exps.weight", TYPE_MXFP4, [H, D, E], t["gate"].data_ptr(),
                                   E * shp.gate_bytes)
    lw.ffn_up_exps = Tensor.make("blk.ffn_up_exps.weight", TYPE_MXFP4, [H, D, E], t["up"].data_ptr(),
                                 E * shp.gate_bytes)
    lw.ffn_down_exps = Tensor.make("blk.ffn_down_exps.weight", TYPE_MXFP4, [D, H, E], t["down"].data_ptr(),
                                   E * shp.down_bytes)
    if shp.biases:
        for n in ("router_bias", "gate_bias", "up_bias", "down_bias"):
            t[n] = torch.from_numpy(small[n]).to(device)
        lw.ffn_gate_inp_bias = Tensor.make("blk.ffn_gate_inp.bias", TYPE_F32, [E], t["router_bias"].data_ptr(), E * 4)
        lw.ffn_gate_exps_bias = Tensor.make("blk.ffn_gate_exps.bias", TYPE_F32, [D, E], t["gate_bias"].data_ptr(),
                                            D * E * 4)
        lw.ffn_up_exps_bias = Tensor.make("blk.ffn_up_exps.bias", TYPE_F32, [D, E], t["up_bias"].data_ptr(),
                                          D * E * 4)
        lw.ffn_down_exps_bias = Tensor.make("blk.ffn_down_exps.bias", TYPE_F32, [H, E], t["down_bias"].data_ptr(),
                                            H * E * 4)
    cfg = MoEConfig()
    cfg.hidden_dim, cfg.expert_hidden_dim, cfg.num_experts, cfg.num_experts_used = H, D, E, shp.topk
    dl.layer, dl.config = lw, cfg
    return dl


def moe_algorithmic_bytes(shp: MoEShape, batch: int, distinct_experts: int) -> int:
    """Bytes a perfect implementation must move for one MoE layer call:
    router weights + bias, each touched expert's gate/up/down matrices and
    biases once, the token activations in and the outputs out."""
    H, D, E = shp.hidden, shp.expert_dim, shp.experts
    router = H * E * 4 + (E * 4 if shp.biases else 0)
    per_expert = 2 * shp.gate_bytes + shp.down_bytes + ((2 * D + H) * 4 if shp.biases else 0)
    return router + distinct_experts * per_expert + 2 * batch * H * 4


def q40_projection_shapes():
    """GPT-OSS-120B attention projections: (name, input, output)."""
    return [("q", HIDDEN, 4096), ("k", HIDDEN, 512), ("v", HIDDEN, 512), ("o", 4096, HIDDEN)]

#!/usr/bin/env python3
"""MoE-layer throughput of the quantized MoE hot path on one MI355X.

Workload: continuous-batching decode over all 36 GPT-OSS-120B MoE layers
(hidden 2880, 128 experts, top-4, MXFP4 gate/up/down 2880x2880 per expert,
~60.9 GB of expert weights resident in HBM).  One step = B tokens (one per
sequence) through the 36 layers; routing is independent per token (router
N(0,0.02) over RMS-normalised N(0,1) tokens, logits ~N(0,1)).

Timed region: K steps bracketed by torch.cuda.synchronize(); value =
MoE-layer tokens/s = B * 36 / step time.  The step's launches are captured
once into a HIP graph and the K steps are graph replays (every kernel of
every layer runs each step; the eager time is reported beside it, and the
replayed outputs are checked against the eager step's).  A second, event-instrumented pass
of the same steps measures the average duration of each kernel launch on the
library's stream; the roofline object is computed for the dominant kernel
(grouped gate/up GEMV) from its algorithmic bytes per launch.  The CPU
baseline is the reference-algorithm layer (fp32 activations, AVX2/FMA lane
order, row-parallel threads) timed on this host on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "stream-pt_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBPS = 8000.0
BF16_DENSE_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
INT8_DENSE_TOPS = 5000.0     # MI355X dense int8 MFMA
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "k_mx_mfma_decode_b64_36layers.md")
MFMA_PROFILE = os.path.join(ROOT, "profiles", "k_mx_gemm_prefill_b512_hot.md")
# grouped-GEMM policy of the library's default (spt_abi.hip: kGemmMinGroup,
# kGemmMinSelections; select: items must fill half the device)
GEMM_MIN_GROUP, GEMM_MIN_SELECTIONS = 9, 384
# selections per grouped-GEMV weight pass (spt_kernels.h: kGemvTokens)
GEMV_TOKENS = 4
# host threads for the CPU baseline: the host's CPU share per GPU
CPU_SHARE = 16


def measured_traffic(batch, layers, seed):
    """HBM bytes per gate/up launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (scaled by a copy kernel of known size); only for the
    workload those passes ran (B=64, 36 layers, seed 3), else None."""
    if (batch, layers, seed) != (64, 36, 3):
        return None
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch k_mx_mfma<0> B=64:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def measured_mfma_util(workload):
    """MFMA busy fraction of the grouped GEMM kernels from the committed
    rocprofv3 counter pass (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x
    SIMDs)), for the workload that pass ran, else None."""
    try:
        with open(MFMA_PROFILE) as f:
            for line in f:
                if line.startswith(f"mfma_util {workload}:"):
                    return json.loads(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=64, help="tokens per decode step (headline)")
    ap.add_argument("--extra-batches", default="1,8", help="other batch sizes reported beside it")
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--seed", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill workloads")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the prefill workloads (one layer resident; for counter passes)")
    ap.add_argument("--prefill-workloads", default="zipf_b32,hot_b512",
                    help="which prefill workloads run (comma-separated; for counter passes)")
    ap.add_argument("--no-lm-head", action="store_true", help="skip the Q8_0 LM head")
    ap.add_argument("--q40-only", action="store_true", help="only the Q4_0 attention projections (for profiles)")
    ap.add_argument("--no-graph", action="store_true",
                    help="time the decode step with eager launches only (no HIP graph replay)")
    ap.add_argument("--decode-max-selections", type=int, default=0,
                    help="decode-path limit of the library (0: its default, negative: off)")
    ap.add_argument("--lm-head-only", action="store_true", help="only the Q8_0 LM head (for profiles)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a 1 GiB elementwise copy kernel three times (known "
                         "traffic for scaling hardware byte counters)")
    return ap.parse_args()


def gate_up_bytes(shp, batch, n_distinct, n_valid):
    """Algorithmic HBM bytes of one grouped gate/up launch: both matrices and
    biases of every distinct expert once, the Q8_0 token rows in, the SwiGLU
    rows out."""
    H, D = shp.hidden, shp.expert_dim
    w = n_distinct * (2 * shp.gate_bytes + (2 * D * 4 if shp.biases else 0))
    return w + batch * (H + H // 32 * 4) + n_valid * D * 4


def down_bytes(shp, n_distinct, n_valid):
    H, D = shp.hidden, shp.expert_dim
    w = n_distinct * (shp.down_bytes + (H * 4 if shp.biases else 0))
    return w + n_valid * (D + D // 32 * 4) + n_valid * H * 4


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the expert-parallel "
              "sharding across GPUs is not built.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import spt
    from spt import workloads as W

    torch.cuda.set_device(0)
    # a stream of its own (graph capture cannot use the device's null stream),
    # made current so torch's own work is ordered with the library's
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)  # elementwise kernel: 1 GiB read, 1 GiB written
        torch.cuda.synchronize()
        log("copy calibration: 3 x 1 GiB elementwise copies done")
        del src, dst
    ctx = spt.Context(0, stream.cuda_stream)
    ctx.set_decode_max_selections(args.decode_max_selections)
    shp = W.MoEShape()
    if args.lm_head_only:
        print(json.dumps({"lm_head": lm_head(ctx, stream), "rmsnorm_q8": rmsnorm_rows(ctx, stream)}), flush=True)
        ctx.close()
        return
    if args.q40_only:
        print(json.dumps({str(B): q40_projections(ctx, B, W, stream, 20) for B in (1, 32)}), flush=True)
        ctx.close()
        return
    if args.prefill_only:
        layer0 = W.device_layer(ctx, args.seed, 0, shp)
        print(json.dumps({"prefill": prefill(args, ctx, layer0, shp, W, stream)}), flush=True)
        ctx.close()
        return
    L = args.layers
    t0 = time.time()
    layers = [W.device_layer(ctx, args.seed, l, shp) for l in range(L)]
    torch.cuda.synchronize()
    resident = sum(t.numel() * t.element_size() for dl in layers for t in dl.tensors.values())
    log(f"{L} layers resident: {resident / 1e9:.2f} GB in {time.time() - t0:.1f}s")

    results = {}
    batches = [args.batch] + [int(b) for b in args.extra_batches.split(",") if b and int(b) != args.batch]
    for B in batches:
        xs = [torch.from_numpy(W.x_tokens(args.seed, l, B, shp.hidden)).cuda() for l in range(L)]
        outs = [torch.empty(B * shp.hidden, dtype=torch.float32, device="cuda") for _ in range(L)]

        def step():
            for l in range(L):
                ctx.forward_moe_batch(layers[l].config, layers[l].layer, xs[l], outs[l], B)

        # routing statistics per layer (deterministic: same tokens every step)
        n_active = torch.zeros(1, dtype=torch.int32, device="cuda")
        weights = torch.zeros(B * shp.topk, dtype=torch.float32, device="cuda")
        distinct, valid = [], []
        for l in range(L):
            taps = spt.make_taps(n_active=n_active, weights=weights)
            ctx.forward_moe_batch(layers[l].config, layers[l].layer, xs[l], outs[l], B, taps)
            torch.cuda.synchronize()
            distinct.append(int(n_active.item()))
            valid.append(int((weights > 0).sum().item()))
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        log(f"B={B}: warmup done; distinct experts/layer mean {np.mean(distinct):.1f}")
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        wall0 = time.perf_counter()
        start.record(stream)
        for _ in range(args.steps):
            step()
        end.record(stream)
        torch.cuda.synchronize()
        eager_ms = start.elapsed_time(end) / args.steps
        eager_wall = time.perf_counter() - wall0
        ms_step, wall = eager_ms, eager_wall
        graph_ok = None
        if not args.no_graph:
            # the step's launches captured once into a HIP graph and replayed:
            # the same kernels, without the host's per-launch cost
            ref = [o.clone() for o in outs]
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                step()
            for _ in range(args.warmup):
                g.replay()
            torch.cuda.synchronize()
            graph_ok = all(bool(torch.equal(a_, b_)) for a_, b_ in zip(outs, ref))
            wall0 = time.perf_counter()
            start.record(stream)
            for _ in range(args.steps):
                g.replay()
            end.record(stream)
            torch.cuda.synchronize()
            wall = time.perf_counter() - wall0
            ms_step = start.elapsed_time(end) / args.steps
            del g
            if not graph_ok:
                log(f"B={B}: graph replay output differs from the eager step")
        # instrumented pass: per-kernel durations from HIP events
        ctx.enable_timing(True)
        ctx.read_timing()
        for _ in range(args.steps):
            step()
        kt = ctx.read_timing()
        ctx.enable_timing(False)
        gu_ms, gu_n = kt["gate_up"]
        dn_ms, dn_n = kt["down"]
        gu_bytes = np.mean([gate_up_bytes(shp, B, d, v) for d, v in zip(distinct, valid)])
        dn_bytes = np.mean([down_bytes(shp, d, v) for d, v in zip(distinct, valid)])
        layer_bytes = np.mean([W.moe_algorithmic_bytes(shp, B, d) for d in distinct])
        res = {
            "batch": B,
            "ms_per_step": ms_step,
            "wall_ms_per_step": wall * 1e3 / args.steps,
            "launch": "hip graph replay" if graph_ok is not None else "eager",
            "graph_matches_eager": graph_ok,
            "eager_ms_per_step": eager_ms,
            "moe_layer_tokens_per_s": B * L / (ms_step / 1e3),
            "decode_tokens_per_s": B / (ms_step / 1e3),
            "distinct_experts_per_layer": float(np.mean(distinct)),
            "step_algorithmic_gb": float(layer_bytes * L / 1e9),
            "step_gbps": float(layer_bytes * L / (ms_step / 1e3) / 1e9),
            "gate_up_avg_us": gu_ms / gu_n * 1e3,
            "gate_up_gbps": float(gu_bytes / (gu_ms / gu_n / 1e3) / 1e9),
            "gate_up_bytes_per_launch": float(gu_bytes),
            "down_avg_us": dn_ms / dn_n * 1e3,
            "down_gbps": float(dn_bytes / (dn_ms / dn_n / 1e3) / 1e9),
            "kernel_ms_per_step": {k: v[0] / args.steps for k, v in kt.items() if v[1]},
        }
        res["step_hbm_frac"] = res["step_gbps"] / HBM_PEAK_GBPS
        res["gate_up_hbm_frac"] = res["gate_up_gbps"] / HBM_PEAK_GBPS
        res["down_hbm_frac"] = res["down_gbps"] / HBM_PEAK_GBPS
        res["host_entry_us_per_layer"] = host_entry_us(ctx, layers, xs, B)
        results[B] = res
        log(f"B={B}: {json.dumps(res)}")
        del xs, outs

    head = results[args.batch]
    roofline = {
        "kernel": "grouped MXFP4xQ8_0 gate/up GEMV + bias + SwiGLU (k_mx_mfma<kGateUp>)",
        "bound": "hbm",
        "achieved": round(head["gate_up_gbps"], 1),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(head["gate_up_gbps"] / HBM_PEAK_GBPS, 4),
        "traffic": measured_traffic(args.batch, L, args.seed),
        "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT),
        "bytes_per_launch": head["gate_up_bytes_per_launch"],
        "avg_launch_us": round(head["gate_up_avg_us"], 2),
    }
    pre = None if args.no_prefill else prefill(args, ctx, layers[0], shp, W, stream)
    lmh = None if args.no_lm_head else lm_head(ctx, stream)
    rms = None if args.no_lm_head else rmsnorm_rows(ctx, stream)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args, shp, W)
    line = {
        "metric": "MoE-layer tokens/s; decode HBM GB/s vs peak; prefill int8 MFMA util",
        "value": round(head["moe_layer_tokens_per_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded MXFP4 experts generated in HBM, N(0,0.02) router/biases, N(0,1) tokens)",
        "config": {
            "workload": f"continuous-batching decode step: B={args.batch} tokens through {L} GPT-OSS-120B MoE "
                        f"layers (hidden 2880, 128 experts, top-4, MXFP4 experts resident in HBM)",
            "batch": args.batch, "layers": L, "hidden": shp.hidden, "expert_dim": shp.expert_dim,
            "experts": shp.experts, "topk": shp.topk, "activations": "Q8_0 (int8 dot, fp32 accumulate)",
            "resident_gb": round(resident / 1e9, 2),
        },
        "decode_tokens_per_s": round(head["decode_tokens_per_s"], 1),
        "step_gbps": round(head["step_gbps"], 1),
        "by_batch": {str(b): {k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()
                              if k != "kernel_ms_per_step"} for b, r in results.items()},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "prefill": pre,
        "lm_head": lmh,
        "rmsnorm_q8": rms,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


def host_entry_us(ctx, layers, xs, B, reps=3):
    """The host-slice entry point a cgo caller binds
    (spt_forward_moe_batch_host): x copied in from pageable host memory and
    out copied back, synchronised, per layer call -- microseconds per layer,
    PCIe included (never the bench value)."""
    import numpy as np

    hx = [x.cpu().numpy() for x in xs]
    ho = np.empty_like(hx[0])
    for l in range(len(layers)):
        ctx.forward_moe_batch_host(layers[l].config, layers[l].layer, hx[l], ho, B)
    t0 = time.perf_counter()
    for _ in range(reps):
        for l in range(len(layers)):
            ctx.forward_moe_batch_host(layers[l].config, layers[l].layer, hx[l], ho, B)
    return round((time.perf_counter() - t0) / (reps * len(layers)) * 1e6, 1)


def prefill(args, ctx, dl, shp, W, stream, reps=20):
    """The batched-prefill workloads, one MoE layer each (router logits
    injected so expert popularity follows Zipf(1.1)):
      zipf_b32:  32 positions per weight pass;
      hot_b512:  a 512-token prompt chunk, 25% of the tokens forced to one
                 hot expert, plus the layer's Q4_0 attention projections
                 (Q, K, V, O) at B = 512.
    Per workload: tokens/s of the layer, per-kernel durations (HIP events on
    the library's stream), the weight bytes of the touched experts over the
    layer time, and for the grouped GEMM its algorithmic multiply-adds
    (selections of GEMM experts x 3 x hidden x expert dim) over its kernel
    time against the dense bf16 MFMA peak it runs on (it issues bf16 MFMAs
    only); at 512 tokens, the Q4_0 projections' int8 MFMA rate (the int8
    MFMA kernel of this path) against the dense int8 peak."""
    import numpy as np
    import torch

    import spt
    from spt import synth

    H, D, E, k = shp.hidden, shp.expert_dim, shp.experts, shp.topk
    out = {}
    wanted = set(args.prefill_workloads.split(","))
    for name, B, hot, seed in (("zipf_b32", 32, 0.0, 2), ("hot_b512", 512, 0.25, 4)):
        if name not in wanted:
            continue
        logits = torch.from_numpy(synth.zipf_logits(synth.stream_key(seed, 99), B, E, 1.1,
                                                    hot_fraction=hot, hot_expert=17)).cuda()
        x = torch.from_numpy(W.x_tokens(seed, 0, B, H)).cuda()
        y = torch.empty(B * H, dtype=torch.float32, device="cuda")
        counts = torch.zeros(E, dtype=torch.int32, device="cuda")
        taps = spt.make_taps(logits_in=logits, counts=counts)
        ctx.forward_moe_batch(dl.config, dl.layer, x, y, B, taps)
        torch.cuda.synchronize()
        c = counts.cpu().numpy()
        distinct = int(np.count_nonzero(c))
        n = B * k
        big = c[c >= GEMM_MIN_GROUP]
        gemm_on = n >= GEMM_MIN_SELECTIONS and int(np.sum((big + 63) // 64)) * ((D + 127) // 128) >= 128
        gemm_sel = int(big.sum()) if gemm_on else 0
        # warm for at least 60 ms of back-to-back layers: a few calls after
        # the host-side set-up above the 512-token layer still runs about
        # 10 % slower than in steady state (measured: 650 against 595 us
        # over the first 23 calls)
        t_warm = time.perf_counter() + 0.06
        nw = 0
        while nw < 3 or time.perf_counter() < t_warm:
            ctx.forward_moe_batch(dl.config, dl.layer, x, y, B, taps)
            nw += 1
            if nw % 4 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            ctx.forward_moe_batch(dl.config, dl.layer, x, y, B, taps)
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        ctx.enable_timing(True)
        ctx.read_timing()
        for _ in range(reps):
            ctx.forward_moe_batch(dl.config, dl.layer, x, y, B, taps)
        kt = ctx.read_timing()
        ctx.enable_timing(False)
        kus = {kk: round(v[0] / reps * 1e3, 1) for kk, v in kt.items() if v[1]}
        wbytes = distinct * (2 * shp.gate_bytes + shp.down_bytes)
        # the grouped GEMV streams each of its experts once per pass of
        # GEMV_TOKENS selections: its weight bytes once, and as streamed
        gv = c[(c > 0) & ~((c >= GEMM_MIN_GROUP) & gemm_on)]
        gv_passes = int(np.sum((gv + GEMV_TOKENS - 1) // GEMV_TOKENS))
        res = {
            "batch": B, "ms_per_layer": round(ms, 4), "tokens_per_s": round(B / (ms / 1e3), 1),
            "distinct_experts": distinct, "largest_group": int(c.max()),
            "weight_gb": round(wbytes / 1e9, 4), "weight_gbps": round(wbytes / (ms / 1e3) / 1e9, 1),
            "gemv_experts": int(gv.size), "gemv_passes": gv_passes,
            "gemv_gate_up_bytes_once": int(gv.size * 2 * shp.gate_bytes),
            "gemv_gate_up_bytes_streamed": int(gv_passes * 2 * shp.gate_bytes),
            "kernel_us": kus, "gemm_experts": int(len(big)) if gemm_on else 0, "gemm_selections": gemm_sel,
        }
        gemm_us = kus.get("gate_up_gemm", 0.0) + kus.get("down_gemm", 0.0)
        if gemm_sel and gemm_us > 0:
            macs = gemm_sel * 3 * H * D
            tops = 2 * macs / (gemm_us * 1e-6) / 1e12
            res["gemm"] = {"mfma": "bf16 (v_mfma_f32_16x16x32_bf16)", "macs": macs, "us": round(gemm_us, 1),
                           "tflops_bf16": round(tops, 2), "frac_bf16_dense": round(tops / BF16_DENSE_TFLOPS, 4),
                           "mfma_util_measured": measured_mfma_util(name)}
        if name == "hot_b512":
            qa = q40_projections(ctx, B, W, stream, reps)
            # the four projections' int8 multiply-adds (k_q40_gemm, int8 MFMA)
            ops = 2 * B * sum(din * dout for _, din, dout in W.q40_projection_shapes())
            q_us = qa["fused_qkv_o_us"]
            qa["int8_mfma"] = {"mfma": "int8 (v_mfma_i32_16x16x32_i8)", "ops": ops,
                               "tops": round(ops / (q_us * 1e-6) / 1e12, 2),
                               "frac_int8_dense": round(ops / (q_us * 1e-6) / 1e12 / INT8_DENSE_TOPS, 4),
                               "mfma_util_measured_pct": (measured_mfma_util(name) or {}).get("q40_gemm_pct")}
            res["q40_attention"] = qa
        out[name] = res
        log(f"prefill {name}: {json.dumps(res)}")
    # the dense Q4_0 projections alone (GEMV at B=1, small GEMM at B=32)
    out["q40_attention"] = {str(B): q40_projections(ctx, B, W, stream, reps) for B in (1, 32)}
    log(f"prefill q40: {json.dumps(out['q40_attention'])}")
    return out


def warm(fn, seconds=0.03, min_calls=3, sync_every=16):
    """Calls fn back to back for at least `seconds` of wall time (and at
    least min_calls times), so that the timed calls after it run in steady
    state rather than right after host-side set-up."""
    import torch

    t_end = time.perf_counter() + seconds
    n = 0
    while n < min_calls or time.perf_counter() < t_end:
        fn()
        n += 1
        if n % sync_every == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def q40_projections(ctx, B, W, stream, reps):
    """Q4_0 x Q8_0 attention projections of one layer (Q 2880->4096,
    K/V 2880->512, O 4096->2880; fp16 scales |N(0,0.01)|, uniform nibbles)
    for B tokens: microseconds per projection and in total."""
    import torch

    import spt
    from spt import synth

    res, total = {}, 0.0
    for i, (name, din, dout) in enumerate(W.q40_projection_shapes()):
        wb = torch.from_numpy(synth.q40_bytes(synth.stream_key(40 + i, dout), dout, din)).cuda()
        t = spt.Tensor.make(name, spt.TYPE_Q4_0, [din, dout], wb.data_ptr(), wb.numel())
        xq = torch.from_numpy(synth.normal(synth.stream_key(50 + i, B), B * din)).cuda()
        yq = torch.empty(B * dout, dtype=torch.float32, device="cuda")
        warm(lambda: ctx.mul_q40_batch_into(t, xq, yq, B))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            ctx.mul_q40_batch_into(t, xq, yq, B)
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / reps * 1e3
        res[name] = round(us, 1)
        total += us
    res["total_us"] = round(total, 1)
    res.update(q40_fused(ctx, B, W, stream, reps))
    return res


def q40_fused(ctx, B, W, stream, reps):
    """The same four projections as a layer runs them on the device: Q, K
    and V in one call on the GGML Q8_0 blocks of the normed input (as the
    fused RMSNorm writes them), then O on the fp32 attention context (the
    call quantizes it), microseconds for the whole sequence, and the weight
    bytes it moves over that time."""
    import torch

    import spt
    from spt import synth

    shapes = W.q40_projection_shapes()
    ts, keep = [], []
    for i, (name, din, dout) in enumerate(shapes):
        wb = torch.from_numpy(synth.q40_bytes(synth.stream_key(40 + i, dout), dout, din)).cuda()
        keep.append(wb)
        ts.append(spt.Tensor.make(name, spt.TYPE_Q4_0, [din, dout], wb.data_ptr(), wb.numel()))
    H, QD = shapes[0][1], shapes[3][1]
    x = torch.from_numpy(synth.normal(synth.stream_key(50, B), B * H)).cuda()
    ctxv = torch.from_numpy(synth.normal(synth.stream_key(53, B), B * QD)).cuda()
    xq = torch.empty(B * H // 32 * 34, dtype=torch.uint8, device="cuda")
    ctx.quantize_q8_0(x, xq)
    ys = [torch.empty(B * d, dtype=torch.float32, device="cuda") for _, _, d in shapes[:3]]
    yo = torch.empty(B * shapes[3][2], dtype=torch.float32, device="cuda")

    def run():
        ctx.mul_q40_qkv_batch_into(ts[:3], None, None, ys, B, xq=xq, x_len=B * H)
        ctx.mul_q40_batch_into(ts[3], ctxv, yo, B)

    warm(run)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / reps * 1e3
    wbytes = sum(t.nbytes for t in ts)
    # the two launches of each of the 36 layers captured into a HIP graph
    # and replayed, as a decode step replays them
    layers = 36
    ref = [y.clone() for y in ys + [yo]]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(layers):
            run()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    same = all(bool(torch.equal(a, b)) for a, b in zip(ys + [yo], ref))
    greps = max(1, reps // 10)
    e0.record(stream)
    for _ in range(greps):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    gus = e0.elapsed_time(e1) / (greps * layers) * 1e3
    del g
    return {"fused_qkv_o_us": round(us, 1), "fused_weights_gbps": round(wbytes / (us * 1e-6) / 1e9, 1),
            "fused_qkv_o_graph_us": round(gus, 1), "graph_matches_eager": same}


def lm_head(ctx, stream, reps=20, rows=201088, input_dim=2880):
    """The GPT-OSS LM head, 201088 x 2880 Q8_0 (615 MB; fp16 scales
    |N(0,0.01)|, uniform int8 codes) times one fp32 token: MulQ80Into (all
    logits) and MulQ80Argmax (best token only).  Kernel microseconds from HIP
    events on the library's stream; algorithmic bytes = the matrix once + x
    (+ the fp32 logits for MulQ80Into), over 8 TB/s."""
    import torch

    import spt
    from spt import synth

    wb = torch.from_numpy(synth.q80_bytes(synth.stream_key(60, 0), rows, input_dim)).cuda()
    t = spt.Tensor.make("output.weight", spt.TYPE_Q8_0, [input_dim, rows], wb.data_ptr(), wb.numel())
    x = torch.from_numpy(synth.normal(synth.stream_key(61, 0), input_dim)).cuda()
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    def both():
        ctx.mul_q80_into(t, x, y)
        ctx.mul_q80_argmax(t, x)

    warm(both, sync_every=2)
    res = {"rows": rows, "input": input_dim, "matrix_bytes": wb.numel()}
    for name, call, extra in (("into", lambda: ctx.mul_q80_into(t, x, y), rows * 4),
                              ("argmax", lambda: ctx.mul_q80_argmax(t, x), 0)):
        ctx.enable_timing(True)
        ctx.read_timing()
        for _ in range(reps):
            call()
        kt = ctx.read_timing()
        ctx.enable_timing(False)
        us = kt["q80"][0] / kt["q80"][1] * 1e3
        nbytes = wb.numel() + input_dim * 4 + extra
        gbps = nbytes / (us * 1e-6) / 1e9
        res[name] = {"us": round(us, 1), "gbps": round(gbps, 1), "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4)}
    log(f"lm_head: {json.dumps(res)}")
    del wb
    return res


def rmsnorm_rows(ctx, stream, reps=50, dim=2880):
    """The fused RMSNorm + Q8_0 of B rows of 2880 (normBatch order; F32
    weights), B = 1, 64, 512: microseconds per call (HIP events on the
    library's stream) and the bytes moved (x, y, Q8_0 and the weights) per
    microsecond."""
    import torch

    import spt
    from spt import synth

    w = torch.from_numpy(synth.normal(synth.stream_key(90, 0), dim)).cuda()
    t = spt.Tensor.make("norm.weight", spt.TYPE_F32, [dim], w.data_ptr(), dim * 4)
    res = {}
    for B in (1, 64, 512):
        x = torch.from_numpy(synth.normal(synth.stream_key(91, B), B * dim)).cuda()
        y = torch.empty_like(x)
        q = torch.empty(B * dim // 32 * 34, dtype=torch.uint8, device="cuda")
        warm(lambda: ctx.rmsnorm_batch_into(t, x, y, B, 1e-5, q))
        ctx.enable_timing(True)
        ctx.read_timing()
        for _ in range(reps):
            ctx.rmsnorm_batch_into(t, x, y, B, 1e-5, q)
        kt = ctx.read_timing()
        ctx.enable_timing(False)
        us = kt["rmsnorm"][0] / kt["rmsnorm"][1] * 1e3
        nbytes = B * dim * 8 + B * dim // 32 * 34 + dim * 4
        res[str(B)] = {"us": round(us, 2), "gbps": round(nbytes / (us * 1e-6) / 1e9, 1)}
    log(f"rmsnorm_q8: {json.dumps(res)}")
    return res


def cpu_baseline(args, shp, W):
    """Reference-algorithm layer on the host: fp32 activations in the
    reference's AVX2/FMA order, rows split over threads like the Go worker
    pool (forward/workers_quant.go:42-52), weights pre-faulted in RAM (1.4 GB
    for layer 0's ~108 experts, far beyond the last-level cache).  Timed with
    the host's CPU share of threads (16 per GPU, capped by the affinity mask)
    and with one thread."""
    import numpy as np

    from oracle import oracle as O

    B = args.batch
    host_cpus = len(os.sched_getaffinity(0))
    threads = max(1, min(host_cpus, CPU_SHARE))
    x = W.x_tokens(args.seed, 0, B, shp.hidden)
    small = W.host_small_tensors(args.seed, 0, shp)
    logits = O.route(small["router"], small.get("router_bias"), x, B, shp.hidden, shp.experts)
    ids = np.concatenate([O.select(logits[t * shp.experts:(t + 1) * shp.experts], shp.topk)[0] for t in range(B)])
    t0 = time.time()
    lay = W.host_layer(args.seed, 0, shp, experts=np.unique(ids))
    log(f"cpu baseline: layer 0 weights for {len(np.unique(ids))} experts generated in {time.time() - t0:.1f}s")

    def timed(n_threads, seconds):
        O.forward_moe_batch(lay, x, B, q8=False, threads=n_threads)  # warm (page in)
        reps, t1 = 0, time.perf_counter()
        while True:
            O.forward_moe_batch(lay, x, B, q8=False, threads=n_threads)
            reps += 1
            el = time.perf_counter() - t1
            if el >= seconds or reps >= 400:
                return reps, el

    reps, el = timed(threads, args.cpu_seconds)
    reps1, el1 = timed(1, args.cpu_seconds)
    per_layer, per_layer1 = el / reps, el1 / reps1
    log(f"cpu baseline: {threads} threads {per_layer * 1e3:.1f} ms/layer, 1 thread {per_layer1 * 1e3:.1f} ms/layer")
    return {
        "value": round(B / per_layer, 2),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"layer 0 of the same workload, B={B} tokens, {len(np.unique(ids))} distinct experts: "
                  f"{reps} repetitions in {el:.1f}s on {threads} threads ({per_layer * 1e3:.1f} ms/layer), "
                  f"{reps1} in {el1:.1f}s on 1 thread ({per_layer1 * 1e3:.1f} ms/layer); MoE-layer tokens/s",
        "value_1core": round(B / per_layer1, 2),
        "host_cpus": host_cpus,
        "cpu": _cpu_model(),
    }


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    main()

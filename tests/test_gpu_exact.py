"""Bit-exact parity of the kernels that produce the outputs, through the C ABI.

The per-block integer sums of the MXFP4 x Q8_0 and Q4_0 x Q8_0 dots are exact
in every kernel; what may differ from the oracle is only the fp32 order in
which blocks (and, in the block-scaled MFMA, the two E4M3 digit halves of a
block) are added.  Two input families make that order irrelevant, so every
kernel's output must equal the integer form exactly:

* one block per row (input dimension 32): the result is the single rounding
  of isum * 2^(e-128) * d_x (MXFP4) or isum * (d_w * d_x) (Q4_0).  In the
  block-scaled MFMA each digit half's product D * d_x is exact (at most 13
  significant bits times the 11 of an fp16 scale), so the one rounding is
  the add of the two halves; in the other kernels it is the FMA.  Rows of
  256 cover every nibble byte at every byte position, and the E8M0 set
  {4, 118, 127, 240} spans the range the MFMA path takes (outside it the
  integer-decode fallback runs, tested against the oracle elsewhere).
* full input rows whose every partial sum is an exact fp32: d_x = 1 (each
  Q8_0 block's amax is 127, so the codes are the integers of x) and block
  scales of two adjacent powers of two, so every partial sum is a multiple
  of the smaller one below 2^24 of them.

The expected values (tests/exact.py) are the integer form evaluated in
float64 from the E2M1 / Q4_0 decode tables, which
tests/test_oracle_dots.py::test_exact_tables_match_oracle pins to the
oracle's integer block sums, and rounded once to fp32.  Equality is of
values (so +0 and -0 compare equal).
"""
import numpy as np
import pytest
from exact import (all_pairs_bytes, assert_exact, int_tokens, mx_expected, mx_matrix, pow2_q40, q8_codes_scales,
                   q40_expected, q40_matrix)

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


# ---- MXFP4: the grouped GEMV's kRows form (mulMoEBatchExpert) ---------------------------

@pytest.mark.parametrize("batch", [1, 4, 5, 9])
def test_mxfp4_one_block_all_pairs(gpu_ctx, O, batch):
    """Input 32: 1,024 rows of expert 1 (every nibble byte at every position
    under each E8M0 of {4, 118, 127, 240}); tokens alternately with d_x = 1
    and with a general d_x (amax 40..127)."""
    import torch

    import spt

    rng = np.random.default_rng(100 + batch)
    rows, E = 1024, 2
    exps_set = np.array([4, 118, 127, 240], np.uint8)
    mats = []
    for e in range(E):
        nib = all_pairs_bytes(rows, shift=37 * e)[:, None, :]
        ex = exps_set[(np.arange(rows) + e) % 4][:, None]
        mats.append(mx_matrix(nib, ex))
    w = np.stack(mats)  # [E, rows, 1, 17]
    x = int_tokens(rng, batch, 32)
    for t in range(1, batch, 2):  # general scales: amax well above 31.75 keeps 2^-124 * d_x normal
        x[t] = (rng.standard_normal(32) * 40).astype(np.float32)
        x[t, 0] = 127.0 * (0.4 + 0.6 * rng.random())
    wd, xd = _dev(w.reshape(-1)), _dev(x.reshape(-1))
    y = torch.zeros(batch * rows, dtype=torch.float32, device="cuda")
    t = spt.Tensor.make("ffn_down_exps", spt.TYPE_MXFP4, [32, rows, E], wd.data_ptr(), w.size)
    gpu_ctx.mul_mxfp4_expert(t, None, 1, xd, y, batch)
    torch.cuda.synchronize()
    codes, d = q8_codes_scales(O, x)
    assert_exact(y.cpu().numpy().reshape(batch, rows), mx_expected(w[1], codes, d), "kRows one block")


@pytest.mark.parametrize("e0", [4, 118, 127, 200])
@pytest.mark.parametrize("batch", [1, 5])
def test_mxfp4_full_row_exact(gpu_ctx, O, e0, batch):
    """Input 2880 (GPT-OSS), 512 rows, E8M0 in {e0, e0 + 1} per block, d_x = 1:
    every partial sum is exact, so each output equals the integer form."""
    import torch

    import spt

    rng = np.random.default_rng(e0 * 7 + batch)
    rows, nb = 512, 90
    nib = rng.integers(0, 256, size=(rows, nb, 16), dtype=np.uint8)
    w = mx_matrix(nib, (e0 + rng.integers(0, 2, size=(rows, nb))).astype(np.uint8))
    x = int_tokens(rng, batch, 32 * nb)
    wd, xd = _dev(w.reshape(-1)), _dev(x.reshape(-1))
    y = torch.zeros(batch * rows, dtype=torch.float32, device="cuda")
    t = spt.Tensor.make("ffn_gate_exps", spt.TYPE_MXFP4, [32 * nb, rows, 1], wd.data_ptr(), w.size)
    gpu_ctx.mul_mxfp4_expert(t, None, 0, xd, y, batch)
    torch.cuda.synchronize()
    codes, d = q8_codes_scales(O, x)
    assert np.all(d == 1.0)
    assert_exact(y.cpu().numpy().reshape(batch, rows), mx_expected(w, codes, d), "kRows full row")


# ---- MXFP4: the MoE layer's gate/up and down kernels on every path ----------------------

def exact_moe_layer(seed):
    """GPT-OSS hidden 2880, expert dim 32, 8 experts, top-4, no biases.
    gate/up: E8M0 in {116, 117} per block (full-row exact with d_x = 1);
    down: one block per row, every nibble byte at every position, E8M0
    cycling over {16, 118, 127, 240} (products stay normal and finite for
    act scales above 2^-10)."""
    rng = np.random.default_rng(seed)
    H, D, E, k = 2880, 32, 8, 4
    nbh = H // 32

    def gu():
        nib = rng.integers(0, 256, size=(E * D, nbh, 16), dtype=np.uint8)
        return mx_matrix(nib, (116 + rng.integers(0, 2, size=(E * D, nbh))).astype(np.uint8)).reshape(-1)

    exps_set = np.array([16, 118, 127, 240], np.uint8)
    down = np.stack([mx_matrix(all_pairs_bytes(H, shift=53 * e)[:, None, :],
                               exps_set[(np.arange(H) + e) % 4][:, None]) for e in range(E)])
    router = (rng.standard_normal(E * H) * 2.5e-4).astype(np.float32)
    return {"hidden": H, "expert_dim": D, "experts": E, "topk": k, "router": router,
            "gate": gu(), "up": gu(), "down": down.reshape(-1)}


@pytest.fixture(scope="module")
def exact_layer():
    from fixtures import device_moe_layer

    lay = exact_moe_layer(7)
    keep, cfg, lw = device_moe_layer(lay)
    yield lay, cfg, lw
    del keep


@pytest.mark.parametrize("path,batch", [("default", 1), ("default", 2), ("decode", 3), ("default", 3), ("grouped", 1),
                                        ("grouped", 5), ("gemm", 5), ("gemm", 37), ("default", 64)])
def test_moe_kernels_exact(gpu_ctx, O, exact_layer, path, batch):
    """Decode kernels (k_dec_gate_up / k_dec_down: up to 8 selections on the
    default path, 12 when forced), the grouped GEMV (k_mx_mfma kGateUp / kDown) and the
    grouped GEMM (k_mx_gemm, every group forced onto it): the gate and up
    taps equal the integer form over the full 2,880-input rows, every
    selection's down result the single rounding of its one block, and the
    usual stage-wise checks hold (ids, packing, SwiGLU, act Q8_0, combine)."""
    from test_gpu_moe import _run, check_stagewise, gemm_path

    lay, cfg, lw = exact_layer
    H, D, E, k = lay["hidden"], lay["expert_dim"], lay["experts"], lay["topk"]
    rng = np.random.default_rng(batch * 31 + len(path))
    x = int_tokens(rng, batch, H).reshape(-1)
    with gemm_path(gpu_ctx, path):
        g = _run(gpu_ctx, cfg, lw, x, batch)
    check_stagewise(O, lay, x, batch, g)
    n = batch * k
    codes, d = q8_codes_scales(O, x.reshape(batch, H))
    assert np.all(d == 1.0)
    gate_w = lay["gate"].reshape(E, D, H // 32, 17)
    up_w = lay["up"].reshape(E, D, H // 32, 17)
    down_w = lay["down"].reshape(E, H, 1, 17)
    actq = g["actq"].reshape(n, 34)
    acodes = actq[:, 2:].copy().view(np.int8).reshape(n, 1, 32)
    ad = actq[:, :2].copy().view(np.float16)[:, 0].astype(np.float64).reshape(n, 1)
    checked = 0
    for idx in range(n):
        if g["weights"][idx] <= 0:
            continue
        e, t = int(g["ids"][idx]), idx // k
        assert_exact(g["gate"].reshape(n, D)[idx], mx_expected(gate_w[e], codes[t:t + 1], d[t:t + 1])[0],
                     f"gate idx {idx}")
        assert_exact(g["up"].reshape(n, D)[idx], mx_expected(up_w[e], codes[t:t + 1], d[t:t + 1])[0],
                     f"up idx {idx}")
        assert ad[idx, 0] > 2.0 ** -10, "act scale too small for exact products"
        assert_exact(g["results"].reshape(n, H)[idx],
                     mx_expected(down_w[e], acodes[idx:idx + 1], ad[idx:idx + 1])[0], f"down idx {idx}")
        checked += 1
    assert checked >= batch


# ---- Q4_0 x Q8_0: k_q40_dec, k_q40_gemv, k_q40_gemm (split and unsplit) ------------------

def _q40_tensor(w, din, dout, name="attn_q"):
    import spt

    wd = _dev(w.reshape(-1))
    return wd, spt.Tensor.make(name, spt.TYPE_Q4_0, [din, dout], wd.data_ptr(), w.size)


@pytest.mark.parametrize("rows,batch", [(4096, 1), (4096, 2), (4096, 4), (4096, 5), (4096, 17), (4096, 32),
                                        (4096, 512), (512, 3), (512, 32), (512, 300)])
def test_q40_one_block_all_pairs(gpu_ctx, O, rows, batch):
    """Input 32: every nibble byte at every position, fp16 scales of both
    signs including subnormals; tokens with d_x = 1 and with general d_x.
    Covers the few-token launch (<= 4 tokens), the GEMV, the split-K GEMM
    (narrow, or too few tiles) and the unsplit GEMM (4,096 rows x 512
    tokens)."""
    import torch

    rng = np.random.default_rng(rows + batch)
    nib = all_pairs_bytes(rows)[:, None, :]
    dh = (rng.standard_normal(rows) * 0.01).astype(np.float16).view(np.uint16)
    dh[::37] = rng.integers(1, 1024, size=dh[::37].size).astype(np.uint16) | np.uint16(0x8000)  # subnormal, negative
    w = q40_matrix(nib, dh[:, None])
    x = int_tokens(rng, batch, 32)
    for t in range(1, batch, 2):
        x[t] = (rng.standard_normal(32) * 3).astype(np.float32)
    wd, t = _q40_tensor(w, 32, rows)
    y = torch.zeros(batch * rows, dtype=torch.float32, device="cuda")
    gpu_ctx.mul_q40_batch_into(t, _dev(x.reshape(-1)), y, batch)
    torch.cuda.synchronize()
    codes, d = q8_codes_scales(O, x)
    assert_exact(y.cpu().numpy().reshape(batch, rows), q40_expected(w, codes, d), "Q4_0 one block")


@pytest.mark.parametrize("din,dout,batch", [(2880, 4096, 1), (2880, 4096, 4), (2880, 4096, 5), (2880, 4096, 32),
                                            (2880, 4096, 64), (2880, 4096, 512), (2880, 512, 1), (2880, 512, 32),
                                            (2880, 512, 300), (4096, 2880, 1), (4096, 2880, 4), (4096, 2880, 70),
                                            (4096, 2880, 512)])
def test_q40_full_row_exact(gpu_ctx, O, din, dout, batch):
    """Config-1/4 shapes (Q 2880->4096, K/V 2880->512, O 4096->2880) at 1 to
    512 tokens with power-of-two block scales and d_x = 1: every kernel's
    output equals the integer form exactly."""
    import torch

    rng = np.random.default_rng(din + dout + batch)
    w = pow2_q40(rng, dout, din // 32)
    x = int_tokens(rng, batch, din)
    wd, t = _q40_tensor(w, din, dout)
    y = torch.zeros(batch * dout, dtype=torch.float32, device="cuda")
    gpu_ctx.mul_q40_batch_into(t, _dev(x.reshape(-1)), y, batch)
    torch.cuda.synchronize()
    codes, d = q8_codes_scales(O, x)
    assert np.all(d == 1.0)
    assert_exact(y.cpu().numpy().reshape(batch, dout), q40_expected(w, codes, d), "Q4_0 full row")


@pytest.mark.parametrize("batch", [1, 32, 512])
def test_q40_qkv_o_exact(gpu_ctx, O, batch):
    """The fused Q/K/V call on the input's GGML Q8_0 blocks, then O on an
    fp32 context, at 1, 32 and 512 tokens (config 1 and config 4's
    projections): all four outputs equal the integer form exactly."""
    import torch

    rng = np.random.default_rng(900 + batch)
    din = 2880
    mats = [pow2_q40(rng, dout, din // 32) for dout in (4096, 512, 512)]
    ts = [_q40_tensor(w, din, w.shape[0], n) for w, n in zip(mats, ("attn_q", "attn_k", "attn_v"))]
    x = int_tokens(rng, batch, din)
    xd = _dev(x.reshape(-1))
    xq = torch.zeros(batch * din // 32 * 34, dtype=torch.uint8, device="cuda")
    gpu_ctx.quantize_q8_0(xd, xq)
    ys = [torch.zeros(batch * w.shape[0], dtype=torch.float32, device="cuda") for w in mats]
    gpu_ctx.mul_q40_qkv_batch_into([t for _, t in ts], None, None, ys, batch, xq=xq, x_len=batch * din)
    wo = pow2_q40(rng, 2880, 4096 // 32)
    od, ot = _q40_tensor(wo, 4096, 2880, "attn_output")
    ctx_in = int_tokens(rng, batch, 4096)
    yo = torch.zeros(batch * 2880, dtype=torch.float32, device="cuda")
    gpu_ctx.mul_q40_batch_into(ot, _dev(ctx_in.reshape(-1)), yo, batch)
    torch.cuda.synchronize()
    codes, d = q8_codes_scales(O, x)
    for w, y, name in zip(mats, ys, "QKV"):
        assert_exact(y.cpu().numpy().reshape(batch, -1), q40_expected(w, codes, d), f"fused {name}")
    oc, odd = q8_codes_scales(O, ctx_in)
    assert_exact(yo.cpu().numpy().reshape(batch, 2880), q40_expected(wo, oc, odd), "O projection")

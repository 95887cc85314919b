"""Seeded, position-addressable synthetic inputs for the MoE hot path.

Every value is a pure function of (seed, stream, index), so any slice of a
tensor can be produced on its own: the device kernel ``spt_synth_mxfp4``
writes the same MXFP4 bytes as :func:`mxfp4_expert_bytes` for any expert
range, which lets a 60 GB weight set be generated in HBM while the CPU checks
only the experts a step touched.

Hash: SplitMix64's finaliser over ``key + i * 0x9E3779B97F4A7C15``.
Normals: Box-Muller in float64, rounded to float32 (host only).
"""
from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15


def _mix64(z: np.ndarray) -> np.ndarray:
    z = z + np.uint64(GOLDEN)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def stream_key(seed: int, stream: int) -> int:
    """64-bit key of one named stream (one tensor) under one seed."""
    z = np.array([((seed * 0x100000001B3) ^ (stream * 0xD1B54A32D192ED03)) & M64], np.uint64)
    with np.errstate(over="ignore"):
        return int(_mix64(z)[0])


def rand_u64(key: int, start: int, count: int) -> np.ndarray:
    i = np.arange(start, start + count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(np.uint64(key) + i * np.uint64(GOLDEN))


def normal(key: int, count: int, mean: float = 0.0, std: float = 1.0, start: int = 0) -> np.ndarray:
    """float32 N(mean, std) values; element i uses hashes 2i and 2i+1."""
    r = rand_u64(key, 2 * start, 2 * count).reshape(count, 2)
    u1 = ((r[:, 0] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (r[:, 1] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (mean + std * z).astype(np.float32)


def rms_normalize(x: np.ndarray) -> np.ndarray:
    """Unit-weight RMS normalisation in float64, rounded to float32."""
    x64 = x.astype(np.float64)
    r = np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True))
    return (x64 / r).astype(np.float32)


def mxfp4_expert_bytes(key: int, first_block: int, nblocks: int,
                       scale_lo: int = 118, scale_hi: int = 124) -> np.ndarray:
    """MXFP4 blocks [first_block, first_block+nblocks) of a tensor.

    Block g: E8M0 byte = scale_lo + hash(3g) mod (scale_hi-scale_lo+1);
    nibble bytes 0..7 = little-endian bytes of hash(3g+1), 8..15 of hash(3g+2),
    so all 16 E2M1 codes are uniform.
    """
    h = rand_u64(key, 3 * first_block, 3 * nblocks).reshape(nblocks, 3)
    out = np.empty((nblocks, 17), np.uint8)
    span = np.uint64(scale_hi - scale_lo + 1)
    out[:, 0] = (np.uint64(scale_lo) + h[:, 0] % span).astype(np.uint8)
    out[:, 1:9] = h[:, 1].copy().view(np.uint8).reshape(nblocks, 8)
    out[:, 9:17] = h[:, 2].copy().view(np.uint8).reshape(nblocks, 8)
    return out.reshape(-1)


def q40_bytes(key: int, rows: int, input_dim: int, scale_std: float = 0.01) -> np.ndarray:
    """Q4_0 matrix [rows][input/32 blocks of 18 B]: fp16 scale |N(0, std)|,
    uniform nibbles (hashes of the same key after the scale stream)."""
    nb = rows * (input_dim // 32)
    scales = np.abs(normal(key, nb, 0.0, scale_std)).astype(np.float16)
    h = rand_u64(key ^ 0x5A5A5A5A5A5A5A5A, 0, 2 * nb).reshape(nb, 2)
    out = np.empty((nb, 18), np.uint8)
    out[:, 0:2] = scales.view(np.uint8).reshape(nb, 2)
    out[:, 2:10] = h[:, 0].copy().view(np.uint8).reshape(nb, 8)
    out[:, 10:18] = h[:, 1].copy().view(np.uint8).reshape(nb, 8)
    return out.reshape(-1)


def q80_bytes(key: int, rows: int, input_dim: int, scale_std: float = 0.01) -> np.ndarray:
    """Q8_0 matrix [rows][input/32 blocks of 34 B]: fp16 scale |N(0, std)|,
    uniform int8 codes.  Drawn from numpy's PCG64 seeded with the key (fast
    enough for a 615 MB LM head), so also a pure function of the key."""
    nb = rows * (input_dim // 32)
    rng = np.random.Generator(np.random.PCG64(key))
    out = np.empty((nb, 34), np.uint8)
    step = 1 << 22
    for b0 in range(0, nb, step):
        n = min(step, nb - b0)
        d = np.abs(rng.standard_normal(n, dtype=np.float32) * np.float32(scale_std)).astype(np.float16)
        out[b0:b0 + n, 0:2] = d.view(np.uint8).reshape(n, 2)
        out[b0:b0 + n, 2:] = rng.integers(0, 256, size=(n, 32), dtype=np.uint8)
    return out.reshape(-1)


def zipf_logits(key: int, batch: int, experts: int, s: float = 1.1,
                hot_fraction: float = 0.0, hot_expert: int = 0) -> np.ndarray:
    """Router logits under which top-k selection samples experts without
    replacement with Zipf(s) popularity (Gumbel-top-k: logit = log p + G).
    Expert popularity ranks follow a hashed permutation of the expert ids.
    The first round(batch*hot_fraction) tokens get hot_expert forced to the
    top."""
    ranks = np.arange(1, experts + 1, dtype=np.float64)
    logp = -s * np.log(ranks)
    perm = np.argsort(rand_u64(key ^ 0x1234567, 0, experts), kind="stable")
    logp_by_expert = np.empty(experts)
    logp_by_expert[perm] = logp
    r = rand_u64(key, 0, batch * experts).reshape(batch, experts)
    u = ((r >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)
    logits = logp_by_expert[None, :] - np.log(-np.log(u))
    if hot_fraction > 0:
        n_hot = int(round(batch * hot_fraction))
        logits[:n_hot, hot_expert] = 64.0
    return np.ascontiguousarray(logits, dtype=np.float32)

"""Seeded synthetic k-quant tensors with the BASELINE distributions.

Q4_K block (144 B): fp16 d, dmin ~ f16(U(0.001, 0.02)); 12 packed bytes of six-bit
scales/mins ~ U{0..63}; 128 bytes of nibbles ~ U{0..15}. Packing independent
uniform six-bit scales and mins with GGML's layout yields 12 independent uniform
bytes, so those bytes are drawn uniformly.
Q5_K (176 B) adds 32 bytes of high bits ~ U{0,1}. Q6_K (210 B): 128 B low
nibbles, 64 B high 2-bit pairs (uniform bytes), 16 int8 scales ~ U{-32..31}, fp16 d.

Two generators with the same distributions: numpy (host, for parity fixtures) and
torch (device, for the bandwidth benchmark, where gigabytes of distinct weights
are needed to defeat the 256 MB Infinity Cache).
"""
from __future__ import annotations

import numpy as np

BLOCK_BYTES = {12: 144, 13: 176, 14: 210}
Q4_K, Q5_K, Q6_K = 12, 13, 14


def _f16_bits(values: np.ndarray) -> np.ndarray:
    return values.astype(np.float16).view(np.uint16)  # round-to-nearest-even


def kquant_numpy(value_type: int, k: int, n: int, seed: int, centered: bool = False) -> np.ndarray:
    """[n rows x k/256 blocks] encoded tensor as a flat uint8 array (numpy
    generator). centered: as kquant_torch's (zero-mean Q4_K / Q5_K weights)."""
    if k % 256:
        raise ValueError("k must be a multiple of 256")
    rng = np.random.default_rng(seed)
    nb = (k // 256) * n
    bb = BLOCK_BYTES[value_type]
    blocks = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    if value_type in (Q4_K, Q5_K):
        d = _f16_bits(rng.uniform(0.001, 0.02, size=nb))
        dmin = _f16_bits(rng.uniform(0.001, 0.02, size=nb))
        if centered:
            dmin = _f16_bits(d.view(np.float16).astype(np.float32) * _MEAN_Q[value_type])
        blocks[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        blocks[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    else:
        scales = rng.integers(-32, 32, size=(nb, 16), dtype=np.int8)
        blocks[:, 192:208] = scales.view(np.uint8)
        d = _f16_bits(rng.uniform(0.001, 0.02, size=nb))
        blocks[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return blocks.reshape(-1)


def activations_numpy(k: int, members: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.standard_normal((members, k)).astype(np.float32)


def gamma_numpy(k: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (1.0 + 0.02 * rng.standard_normal(k)).astype(np.float32)


# Mean quant of a uniform Q4_K nibble / Q5_K 5-bit value.
_MEAN_Q = {Q4_K: 7.5, Q5_K: 15.5}


def kquant_torch(value_type: int, k: int, n: int, generator, device, centered: bool = False):
    """Device-side generator (same distributions) returning a flat uint8 tensor.

    centered=True (Q4_K / Q5_K): dmin = f16(d * mean quant) instead of an
    independent draw, so the minimum term cancels the quants' mean on average
    (d*sc*q - dmin*m has mean 0 over independent uniform sc, m, q). Weights of
    the BASELINE distribution all share a positive mean, which makes every
    output of a random-weight decoder nearly a multiple of sum(x); a decoder
    built on centered weights produces varied greedy tokens. Block layout and
    sizes are unchanged."""
    import torch

    if k % 256:
        raise ValueError("k must be a multiple of 256")
    nb = (k // 256) * n
    bb = BLOCK_BYTES[value_type]
    blocks = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, device=device, generator=generator)

    def f16_vals(count):
        return torch.empty(count, dtype=torch.float32, device=device).uniform_(0.001, 0.02, generator=generator)

    def f16_bytes(count, vals=None):
        vals = f16_vals(count) if vals is None else vals
        return vals.to(torch.float16).view(torch.uint8).view(count, 2)

    if value_type in (Q4_K, Q5_K):
        d = f16_vals(nb).to(torch.float16).to(torch.float32)
        blocks[:, 0:2] = f16_bytes(nb, d)
        blocks[:, 2:4] = f16_bytes(nb, d * _MEAN_Q[value_type] if centered else None)
    else:
        sc = torch.randint(-32, 32, (nb, 16), dtype=torch.int8, device=device, generator=generator)
        blocks[:, 192:208] = sc.view(torch.uint8)
        blocks[:, 208:210] = f16_bytes(nb)
    return blocks.reshape(-1)

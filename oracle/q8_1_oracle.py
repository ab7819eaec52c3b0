"""Q8_1 activation packing and the integer-dot reference arithmetic -- TEST
INFRASTRUCTURE ONLY (tests/, never the product path).

pack_q8_1 restates the reference's packer (crates/nvidia/src/activation.cu:1-28,
and the host restatement in crates/nvidia/tests/q4_q8_1.rs:95-138): per
32-value block, d = max|x| / 127 in f32, q = round(x / d) half away from
zero (x / d in f32), the block sum formed by the xor butterfly over offsets
16, 8, 4, 2, 1 (lane 0's value), and the header half(d) | half(sum) << 16
with round-to-nearest-even conversions.

q8_1_reference restates the f64 reference of the reference's integer-dot
tests (q4_q8_1.rs:140-205 for Q4_K, the same form for Q5_K, q6_q8_1.rs:156-206
for Q6_K): per row the packed-arithmetic output, the float output of the
unpacked activations, the packing error bound and the arithmetic magnitude
that scales the f32 rounding allowance.
"""
from __future__ import annotations

import numpy as np

from . import kquant_np

F32 = np.float32
BLOCK_BYTES = {12: 144, 13: 176, 14: 210}


def _round_half_away(v: np.ndarray) -> np.ndarray:
    """roundf: nearest integer, ties away from zero (v exact in float64)."""
    v = v.astype(np.float64)
    return np.trunc(v + np.copysign(0.5, v))


def pack_q8_1(x: np.ndarray) -> np.ndarray:
    """float32 [n * 32] -> uint32 [n * 9]."""
    x = np.ascontiguousarray(x, F32).reshape(-1, 32)
    lanes = np.arange(32)
    maximum = np.abs(x).max(axis=1)
    sums = x.copy()
    for off in (16, 8, 4, 2, 1):
        sums = (sums + sums[:, lanes ^ off]).astype(F32)
    total = sums[:, 0]
    d = (maximum / F32(127.0)).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        quot = (x / d[:, None]).astype(F32)
    q = np.where(maximum[:, None] == 0, 0.0, _round_half_away(quot)).astype(np.int64)
    qb = (q & 0xFF).astype(np.uint8).reshape(-1, 8, 4)
    words = qb.view("<u4").reshape(-1, 8).astype(np.uint32)
    dh = d.astype(np.float16).view(np.uint16).astype(np.uint32)
    sh = total.astype(np.float16).view(np.uint16).astype(np.uint32)
    out = np.empty((x.shape[0], 9), np.uint32)
    out[:, 0] = dh | (sh << 16)
    out[:, 1:] = words
    return out.reshape(-1)


def unpack_q8_1(words: np.ndarray):
    """uint32 [n * 9] -> (scale f64 [n], sum f64 [n], q int32 [n, 32])."""
    w = np.ascontiguousarray(words, np.uint32).reshape(-1, 9)
    scale = (w[:, 0] & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    total = (w[:, 0] >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
    q = w[:, 1:].copy().view(np.int8).reshape(-1, 32).astype(np.int32)
    return scale, total, q


def block_fields(value_type: int, encoded: np.ndarray, k: int, n: int):
    """Per [row, block]: Q4_K / Q5_K -> (d, dmin, sc[8], mn[8], q[256] unsigned);
    Q6_K -> (d, scales[16], q[256] signed), all f64 / int64."""
    nbk = k // 256
    blocks = np.frombuffer(np.ascontiguousarray(encoded, np.uint8).tobytes(), np.uint8).reshape(
        -1, BLOCK_BYTES[value_type])
    if value_type in (12, 13):
        d = kquant_np._half(blocks, 0).astype(np.float64)
        dmin = kquant_np._half(blocks, 2).astype(np.float64)
        sc, mn = kquant_np.scale_min_k4(blocks[:, 4:16])
        ql = blocks[:, 16:144] if value_type == 12 else blocks[:, 48:176]
        q = np.empty((blocks.shape[0], 256), np.int64)
        for g in range(8):
            nib = (ql[:, 32 * (g // 2):32 * (g // 2) + 32] >> (4 * (g % 2))) & 0xF
            q[:, 32 * g:32 * g + 32] = nib
            if value_type == 13:
                q[:, 32 * g:32 * g + 32] += ((blocks[:, 16:48] >> g) & 1).astype(np.int64) << 4
        shape = (n, nbk)
        return (d.reshape(shape), dmin.reshape(shape), sc.astype(np.int64).reshape(shape + (8,)),
                mn.astype(np.int64).reshape(shape + (8,)), q.reshape(shape + (256,)))
    d = kquant_np._half(blocks, 208).astype(np.float64)
    scales = blocks[:, 192:208].view(np.int8).astype(np.int64)
    q = np.empty((blocks.shape[0], 256), np.int64)
    for g in range(8):
        hf, c = g // 4, g % 4
        lo = (blocks[:, 64 * hf + 32 * (c & 1):64 * hf + 32 * (c & 1) + 32] >> (4 * (c >> 1))) & 0xF
        hi = (blocks[:, 128 + 32 * hf:128 + 32 * hf + 32] >> (2 * c)) & 3
        q[:, 32 * g:32 * g + 32] = (lo.astype(np.int64) | (hi.astype(np.int64) << 4)) - 32
    shape = (n, nbk)
    return d.reshape(shape), scales.reshape(shape + (16,)), q.reshape(shape + (256,))


def q8_1_reference(value_type: int, encoded: np.ndarray, k: int, n: int, x: np.ndarray, packed: np.ndarray):
    """For one member: dict of f64 [n] arrays packed_output, float_output,
    packing_error_bound, arithmetic_magnitude."""
    nbk = k // 256
    x = np.asarray(x, F32).astype(np.float64).reshape(nbk, 8, 32)
    scale, total, qa = unpack_q8_1(packed)
    scale = scale.reshape(nbk, 8)
    total = total.reshape(nbk, 8)
    qa = qa.reshape(nbk, 8, 32).astype(np.int64)
    out = {name: np.zeros(n) for name in ("packed_output", "float_output", "packing_error_bound",
                                          "arithmetic_magnitude")}
    err_x = np.abs(scale[:, :, None] * qa - x)  # [nbk, 8, 32]
    if value_type in (12, 13):
        d, dmin, sc, mn, q = block_fields(value_type, encoded, k, n)
        q = q.reshape(n, nbk, 8, 32)
        a = d[:, :, None] * sc  # [n, nbk, 8]
        b = dmin[:, :, None] * mn
        dot = (q * qa[None]).sum(axis=3)
        out["packed_output"] = (a * scale[None] * dot - b * total[None]).sum(axis=(1, 2))
        out["float_output"] = ((a[..., None] * q - b[..., None]) * x[None]).sum(axis=(1, 2, 3))
        out["packing_error_bound"] = ((np.abs(a)[..., None] * q * err_x[None]).sum(axis=(1, 2, 3))
                                      + (np.abs(b) * np.abs(total[None] - x.sum(axis=2)[None])).sum(axis=(1, 2)))
        out["arithmetic_magnitude"] = (np.abs(a[..., None] * q * scale[None, :, :, None] * qa[None]).sum(axis=(1, 2, 3))
                                       + np.abs(b * total[None]).sum(axis=(1, 2)))
        return out
    d, scales, q = block_fields(14, encoded, k, n)
    q = q.reshape(n, nbk, 8, 2, 16)
    a = d[:, :, None, None] * scales.reshape(n, nbk, 8, 2)  # [n, nbk, 8, 2]
    qa2 = qa.reshape(nbk, 8, 2, 16)
    x2 = x.reshape(nbk, 8, 2, 16)
    dot = ((q + 32) * qa2[None]).sum(axis=4) - 32 * qa2.sum(axis=3)[None]
    s2 = scale[None, :, :, None]
    out["packed_output"] = (a * s2 * dot).sum(axis=(1, 2, 3))
    out["float_output"] = (a[..., None] * q * x2[None]).sum(axis=(1, 2, 3, 4))
    out["packing_error_bound"] = (np.abs(a)[..., None] * np.abs(q) * err_x.reshape(nbk, 8, 2, 16)[None]).sum(
        axis=(1, 2, 3, 4))
    out["arithmetic_magnitude"] = (np.abs(a[..., None] * q * s2[..., None] * qa2[None]).sum(axis=(1, 2, 3, 4))
                                   + np.abs(a * s2 * dot).sum(axis=(1, 2, 3)))
    return out


def rounding_allowance(ref: dict) -> np.ndarray:
    """The reference tests' f32 rounding allowance: magnitude * eps * 32 + 1e-5."""
    return ref["arithmetic_magnitude"] * float(np.finfo(np.float32).eps) * 32.0 + 1e-5

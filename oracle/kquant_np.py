"""Independent vectorised numpy k-quant decoder -- TEST INFRASTRUCTURE ONLY.

A second implementation written from GGML's published block definitions
(llama.cpp ggml-quants.c dequantize_row_q4_K / q5_K / q6_K and
get_scale_min_k4, at the commit the reference names in
crates/nvidia/src/qwen_reference.rs:1-3), vectorised over blocks instead of
looping like the C oracle. It is used only to cross-check the C oracle
bit-for-bit; it keeps the reference's f32 op order (d*sc)*q - (dmin*m).
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def _half(block_bytes: np.ndarray, offset: int) -> np.ndarray:
    """Little-endian binary16 field -> float32 via numpy's IEEE conversion."""
    raw = block_bytes[:, offset:offset + 2].copy().view(np.float16).reshape(-1)
    return raw.astype(F32)


def scale_min_k4(scale_bytes: np.ndarray):
    """get_scale_min_k4 for j = 0..7 over [nb, 12] packed bytes -> ([nb, 8], [nb, 8])."""
    q = scale_bytes.astype(np.uint32)
    sc = np.empty((q.shape[0], 8), np.uint32)
    mn = np.empty((q.shape[0], 8), np.uint32)
    for j in range(8):
        if j < 4:
            sc[:, j] = q[:, j] & 63
            mn[:, j] = q[:, j + 4] & 63
        else:
            sc[:, j] = (q[:, j + 4] & 0xF) | ((q[:, j - 4] >> 6) << 4)
            mn[:, j] = (q[:, j + 4] >> 4) | ((q[:, j] >> 6) << 4)
    return sc, mn


def dequantize_q4_k(blocks: np.ndarray) -> np.ndarray:
    """[nb, 144] uint8 -> [nb, 256] float32 (dequantize_row_q4_K)."""
    nb = blocks.shape[0]
    d = _half(blocks, 0)
    dmin = _half(blocks, 2)
    sc, mn = scale_min_k4(blocks[:, 4:16])
    qs = blocks[:, 16:144].reshape(nb, 4, 32)  # 64-element chunks: low nibbles, then high
    out = np.empty((nb, 256), F32)
    for j in range(4):
        for half, shift in ((0, 0), (1, 4)):
            g = 2 * j + half
            d1 = d * sc[:, g].astype(F32)
            m1 = dmin * mn[:, g].astype(F32)
            q = ((qs[:, j, :] >> shift) & 0xF).astype(F32)
            out[:, g * 32:(g + 1) * 32] = d1[:, None] * q - m1[:, None]
    return out


def dequantize_q5_k(blocks: np.ndarray) -> np.ndarray:
    """[nb, 176] uint8 -> [nb, 256] float32 (dequantize_row_q5_K)."""
    nb = blocks.shape[0]
    d = _half(blocks, 0)
    dmin = _half(blocks, 2)
    sc, mn = scale_min_k4(blocks[:, 4:16])
    qh = blocks[:, 16:48]
    ql = blocks[:, 48:176].reshape(nb, 4, 32)
    out = np.empty((nb, 256), F32)
    for j in range(4):
        for half, shift in ((0, 0), (1, 4)):
            g = 2 * j + half
            u = np.uint8(1 << g)
            d1 = d * sc[:, g].astype(F32)
            m1 = dmin * mn[:, g].astype(F32)
            q = ((ql[:, j, :] >> shift) & 0xF) + np.where((qh & u) != 0, 16, 0)
            out[:, g * 32:(g + 1) * 32] = d1[:, None] * q.astype(F32) - m1[:, None]
    return out


def dequantize_q6_k(blocks: np.ndarray) -> np.ndarray:
    """[nb, 210] uint8 -> [nb, 256] float32 (dequantize_row_q6_K)."""
    nb = blocks.shape[0]
    ql_all = blocks[:, 0:128]
    qh_all = blocks[:, 128:192]
    scales = blocks[:, 192:208].view(np.int8).astype(F32)
    d = _half(blocks, 208)
    out = np.empty((nb, 256), F32)
    for n in range(2):  # two 128-element halves
        ql = ql_all[:, 64 * n:64 * n + 64].astype(np.int32)
        qh = qh_all[:, 32 * n:32 * n + 32].astype(np.int32)
        sc = scales[:, 8 * n:8 * n + 8]
        lidx = np.arange(32)
        is_ = lidx // 16
        q1 = ((ql[:, 0:32] & 0xF) | (((qh >> 0) & 3) << 4)) - 32
        q2 = ((ql[:, 32:64] & 0xF) | (((qh >> 2) & 3) << 4)) - 32
        q3 = ((ql[:, 0:32] >> 4) | (((qh >> 4) & 3) << 4)) - 32
        q4 = ((ql[:, 32:64] >> 4) | (((qh >> 6) & 3) << 4)) - 32
        base = 128 * n
        for k, q in enumerate((q1, q2, q3, q4)):
            s = sc[:, is_ + 2 * k]  # [nb, 32]
            out[:, base + 32 * k:base + 32 * k + 32] = (d[:, None] * s) * q.astype(F32)
    return out


DECODERS = {12: (144, dequantize_q4_k), 13: (176, dequantize_q5_k), 14: (210, dequantize_q6_k)}


def dequantize(value_type: int, encoded: np.ndarray) -> np.ndarray:
    block_bytes, fn = DECODERS[value_type]
    blocks = np.ascontiguousarray(encoded, dtype=np.uint8).reshape(-1, block_bytes)
    return fn(blocks).reshape(-1)

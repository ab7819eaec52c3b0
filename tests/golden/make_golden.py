"""Writes the committed golden fixtures under tests/golden/.

Inputs are (a) the byte patterns of the reference's own device-test fixtures
(crates/nvidia/tests/cuda_reference.rs:312-409, q{4,5,6}_k_fixture: four blocks,
GGML dims [512, 2], input (i % 17) * 0.125 - 1), restated here as generators, and
(b) small seeded BASELINE-distributed tensors. Expected outputs come from the
CPU oracle (oracle/kquant_oracle.c), which tests/test_oracle.py pins against the
reference's KATs and closed forms. Run from the repo root:

    make -C oracle && python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from engine_amd import synth  # noqa: E402
from oracle import kquant_oracle as O  # noqa: E402


def q4_k_fixture_block(seed: int) -> bytes:
    """cuda_reference.rs:312-330 q4_k_fixture_block."""
    block = bytearray(144)
    block[0:2] = (0x3C00).to_bytes(2, "little")
    block[2:4] = (0x3800).to_bytes(2, "little")
    for index in range(4):
        block[4 + index] = ((1 + seed + index) | ((index & 3) << 6)) & 0xFF
        block[8 + index] = ((1 + index) | (((index + 1) & 3) << 6)) & 0xFF
        block[12 + index] = ((5 + seed + index) | ((2 + index) << 4)) & 0xFF
    for index in range(128):
        pattern = (index + seed * 5) % 16
        low = (pattern * 3) & 0x0F
        high = (15 - pattern * 3) & 0x0F
        block[16 + index] = low | (high << 4)
    return bytes(block)


def rotl8(value: int, amount: int) -> int:
    amount %= 8
    return ((value << amount) | (value >> (8 - amount))) & 0xFF


def q5_k_fixture_block(seed: int) -> bytes:
    """cuda_reference.rs:336-352 q5_k_fixture_block."""
    block = bytearray(q4_k_fixture_block(seed)) + bytearray(32)
    for i in range(16, 48):
        block[i] = rotl8(0x55, seed)
    for index in range(128):
        pattern = (index + seed * 7) % 16
        low = (pattern * 5) & 0x0F
        high = (15 - pattern * 5) & 0x0F
        block[48 + index] = low | (high << 4)
    return bytes(block)


def q6_k_fixture_block(seed: int) -> bytes:
    """cuda_reference.rs:388-405 q6_k_fixture_block."""
    block = bytearray(210)
    for index in range(128):
        block[index] = (index * 7 + seed * 11) % 256
    for index in range(64):
        block[128 + index] = (index * 13 + seed * 5) % 256
    for index in range(16):
        pattern = (index + seed * 3) % 17
        block[192 + index] = (pattern - 8) & 0xFF
    block[208:210] = (0x3C00).to_bytes(2, "little")
    return bytes(block)


FIXTURE_BLOCKS = {12: q4_k_fixture_block, 13: q5_k_fixture_block, 14: q6_k_fixture_block}


def reference_fixture(value_type: int) -> np.ndarray:
    return np.frombuffer(b"".join(FIXTURE_BLOCKS[value_type](s) for s in range(4)), np.uint8)


def reference_input(k: int) -> np.ndarray:
    """cuda_reference.rs:872-877: f32::from(index % 17) * 0.125 - 1.0."""
    return np.array([(i % 17) * 0.125 - 1.0 for i in range(k)], dtype=np.float32)


RANDOM_CASES = [
    # (value_type, K, N, members, seed)
    (12, 512, 48, 1, 101),
    (12, 1024, 40, 3, 102),
    (13, 768, 36, 2, 103),
    (13, 512, 24, 1, 104),
    (14, 512, 40, 1, 105),
    (14, 1280, 20, 4, 106),
]


def sha256_f32(values: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(values, np.float32).tobytes()).hexdigest()


def main() -> None:
    out = {}
    for t in (12, 13, 14):
        enc = reference_fixture(t)
        x = reference_input(512)
        out[f"fixture_{t}_encoded"] = enc
        out[f"fixture_{t}_input"] = x
        out[f"fixture_{t}_dequant"] = O.dequantize_tensor(t, enc)
        out[f"fixture_{t}_output"] = O.quant_gemv(t, enc, 512, 2, x)
    for i, (t, k, n, m, seed) in enumerate(RANDOM_CASES):
        enc = synth.kquant_numpy(t, k, n, seed)
        x = synth.activations_numpy(k, m, seed + 1000)
        out[f"random_{i}_meta"] = np.array([t, k, n, m, seed], np.int64)
        out[f"random_{i}_encoded"] = enc
        out[f"random_{i}_input"] = x
        out[f"random_{i}_output"] = O.quant_gemv(t, enc, k, n, x, members=m).reshape(m, n)
        out[f"random_{i}_dequant_sha256"] = np.frombuffer(
            sha256_f32(O.dequantize_tensor(t, enc)).encode(), np.uint8)
    # RMSNorm: the reference's elementwise fixture (cuda_reference.rs:970-988) and a
    # Qwen3-8B-width vector.
    out["rms_small_input"] = np.array([1.0, -2.0, 3.0, -4.0], np.float32)
    out["rms_small_weight"] = np.array([1.0, 0.5, 2.0, -1.0], np.float32)
    out["rms_small_output"] = O.rms_norm_raw(out["rms_small_input"], out["rms_small_weight"], 1e-5)
    x = synth.activations_numpy(4096, 1, 7)[0]
    g = synth.gamma_numpy(4096, 8)
    out["rms_4096_input"] = x
    out["rms_4096_weight"] = g
    out["rms_4096_output"] = O.rms_norm_raw(x, g, 1e-6)
    path = os.path.join(HERE, "kquant_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()

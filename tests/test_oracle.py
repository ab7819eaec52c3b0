"""Pins the CPU oracle (oracle/kquant_oracle.c) to the reference and to mathematics.

Each check is chosen so that a plausible restatement mistake (a wrong shift,
group index, scale byte, sign or op order) fails it:
  * the reference's KATs (crates/gguf/src/lib.rs:1369-1514);
  * the reference's fixture encoders with their exact float64 closed forms
    (crates/nvidia/tests/q{4,5,6}_q8_1.rs fixture() +
    exact_activations_and_fixture_metadata_match_float_arithmetic);
  * all 65536 binary16 patterns against numpy's IEEE conversion;
  * the scale packing inverse over every (scale, min) pair at every group;
  * an independent vectorised decoder (oracle/kquant_np.py) bit-for-bit;
  * a float64 error bound on the sequential f32 dot and closed forms for RMSNorm.
"""
import math
import struct

import numpy as np
import pytest

from engine_amd import synth
from oracle import kquant_np as NP
from oracle import kquant_oracle as O


def f32_bits(v):
    return struct.unpack("<I", struct.pack("<f", v))[0]


# --------------------------------------------------------------- KATs (lib.rs:1369-1514)

def test_kat_scalar_and_q8_0():
    assert f32_bits(O.dequantize_block(0, struct.pack("<f", 1.5))[0]) == f32_bits(1.5)
    assert f32_bits(O.dequantize_block(1, (0x3C00).to_bytes(2, "little"))[0]) == f32_bits(1.0)
    q8 = bytearray(34)
    q8[0:2] = (0x3C00).to_bytes(2, "little")
    q8[2] = 0x80
    q8[3] = 0x7F
    out = O.dequantize_block(8, q8)
    assert out.size == 32
    assert f32_bits(out[0]) == f32_bits(-128.0)
    assert f32_bits(out[1]) == f32_bits(127.0)


def test_kat_q4_k():
    q4 = bytearray(144)
    q4[0:2] = (0x3C00).to_bytes(2, "little")
    q4[4:8] = b"\x01" * 4
    q4[16] = 0x10
    out = O.dequantize_block(12, q4)
    assert out.size == 256
    assert f32_bits(out[0]) == f32_bits(0.0)
    assert f32_bits(out[32]) == f32_bits(1.0)


def test_kat_q5_k():
    q5 = bytearray(176)
    q5[0:2] = (0x3C00).to_bytes(2, "little")
    q5[4:8] = b"\x01" * 4
    q5[16] = 1
    q5[48] = 0x10
    out = O.dequantize_block(13, q5)
    assert out.size == 256
    assert f32_bits(out[0]) == f32_bits(16.0)
    assert f32_bits(out[32]) == f32_bits(1.0)


def test_kat_q6_k():
    q6 = bytearray(210)
    q6[192:208] = b"\x01" * 16
    q6[208:210] = (0x3C00).to_bytes(2, "little")
    out = O.dequantize_block(14, q6)
    assert out.size == 256
    assert all(f32_bits(v) == f32_bits(-32.0) for v in out)


def test_kat_out_of_path_types_are_reported():
    # Q3_K / IQ4_NL / IQ3_S / IQ4_XS decode in the reference but are not on this path.
    for t, n in ((11, 110), (20, 18), (21, 110), (23, 136)):
        with pytest.raises(O.OracleError) as e:
            O.dequantize_block(t, bytes(n))
        assert e.value.status == O.OUT_OF_SCOPE


def test_kat_invalid_blocks():
    with pytest.raises(O.OracleError) as e:
        O.dequantize_block(12, bytes(143))
    assert e.value.status == O.INVALID_BLOCK_LENGTH
    assert e.value.expected == 144
    with pytest.raises(O.OracleError) as e:
        O.dequantize_block(22, bytes(82))
    assert e.value.status == O.UNSUPPORTED_TYPE


def test_kat_byte_len():
    assert O.byte_len([256], 12) == 144
    with pytest.raises(O.OracleError) as e:
        O.byte_len([128, 2], 12)
    assert e.value.status == O.DIMENSION_MISMATCH
    assert O.byte_len([256], 23) == 136
    assert O.byte_len([256], 21) == 110
    assert O.byte_len([4096, 4096], 12) == 9_437_184
    assert O.byte_len([12288, 4096], 13) == 34_603_008
    assert O.byte_len([4096, 151936], 14) == 510_504_960


# ---------------------------------------------------------- binary16 (lib.rs:551-563)

def test_f16_to_f32_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(expected)
    assert np.array_equal(got[~nan].view(np.uint32), expected[~nan].view(np.uint32))
    # f32::NAN for every NaN payload and sign
    assert np.all(got[nan].view(np.uint32) == 0x7FC00000)


# ---------------------------------------- scale packing (lib.rs:573-587 and its inverse)

def pack_scales(scales, minima):
    """The reference's encoder (crates/nvidia/examples/int_dot_bench.rs:540-549,
    crates/nvidia/tests/q4_q8_1.rs:25-29)."""
    enc = bytearray(12)
    for g in range(4):
        enc[g] = scales[g] | ((scales[g + 4] >> 4) << 6)
        enc[4 + g] = minima[g] | ((minima[g + 4] >> 4) << 6)
        enc[8 + g] = (scales[g + 4] & 15) | ((minima[g + 4] & 15) << 4)
    return bytes(enc)


def test_scale_packing_round_trip_every_value_every_group():
    rng = np.random.default_rng(5)
    for g in range(8):
        for s in range(64):
            scales = list(rng.integers(0, 64, 8))
            minima = list(rng.integers(0, 64, 8))
            scales[g] = s
            minima[g] = 63 - s
            sc, mn = O.q4_k_scales(pack_scales(scales, minima))
            assert list(sc) == scales and list(mn) == minima


# -------------- reference fixtures with exact f64 closed forms (q{4,5,6}_q8_1.rs fixture())

def decode_half64(bits):
    exponent = (bits >> 10) & 31
    fraction = float(bits & 1023)
    mag = fraction * 2.0 ** -24 if exponent == 0 else (1.0 + fraction / 1024.0) * 2.0 ** (exponent - 15)
    return -mag if bits & 0x8000 else mag


def q45_fixture(value_type, seed):
    scales = [1, 17, 33, 63, 32, 47, 62, 48]
    minima = [63, 32, 17, 1, 47, 48, 33, 62]
    d_bits = [0x2C00, 0x3000, 0x3400][seed % 3]
    m_bits = [0x2800, 0x2C00, 0x3000][seed % 3]
    nbytes = 144 if value_type == 12 else 176
    enc = bytearray(nbytes)
    enc[0:2] = d_bits.to_bytes(2, "little")
    enc[2:4] = m_bits.to_bytes(2, "little")
    enc[4:16] = pack_scales(scales, minima)
    mod = 16 if value_type == 12 else 32
    quants = [(i * 7 + seed * 3 + i // 32) % mod for i in range(256)]
    for g in range(8):
        for i in range(32):
            q = quants[g * 32 + i]
            if value_type == 12:
                enc[16 + (g // 2) * 32 + i] |= q << ((g % 2) * 4)
            else:
                enc[48 + (g // 2) * 32 + i] |= (q & 15) << ((g % 2) * 4)
                enc[16 + i] |= ((q >> 4) & 1) << g
    expected = [decode_half64(d_bits) * scales[e // 32] * quants[e]
                - decode_half64(m_bits) * minima[e // 32] for e in range(256)]
    return bytes(enc), expected


def q6_fixture(seed):
    scales = [3, -5, 11, -13, 19, -23, 29, -31, 7, -9, 15, -17, 21, -25, 27, -2]
    d_bits = [0x2C00, 0x3000, 0x3400][seed % 3]
    enc = bytearray(210)
    quants = [(i * 7 + seed * 3 + i // 32) % 64 - 32 for i in range(256)]
    for g in range(8):
        low_base = (g // 4) * 64 + (g % 2) * 32
        low_shift = 0 if g % 4 < 2 else 4
        high_base = 128 + (g // 4) * 32
        high_shift = (g % 4) * 2
        for i in range(32):
            u = quants[g * 32 + i] + 32
            enc[low_base + i] |= (u & 15) << low_shift
            enc[high_base + i] |= ((u >> 4) & 3) << high_shift
    for i, s in enumerate(scales):
        enc[192 + i] = s & 0xFF
    enc[208:210] = d_bits.to_bytes(2, "little")
    expected = [decode_half64(d_bits) * scales[(e // 32) * 2 + (e % 32) // 16] * quants[e]
                for e in range(256)]
    return bytes(enc), expected


@pytest.mark.parametrize("value_type", [12, 13, 14])
def test_reference_fixture_closed_forms(value_type):
    # ROWS * INPUTS / 256 = 5 * 3 = 15 seeds, as in the reference fixtures
    for seed in range(15):
        enc, expected = q6_fixture(seed) if value_type == 14 else q45_fixture(value_type, seed)
        got = O.dequantize_block(value_type, enc)
        assert [float(v) for v in got] == expected


# ------------------------------------------------ independent decoder (bit-for-bit)

@pytest.mark.parametrize("value_type", [12, 13, 14])
def test_numpy_decoder_agrees_bitwise(value_type):
    enc = synth.kquant_numpy(value_type, 2048, 96, seed=40 + value_type)
    a = O.dequantize_tensor(value_type, enc)
    b = NP.dequantize(value_type, enc)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_dequant_products_are_exact_in_f32():
    # Fact: (d*sc)*q and dmin*m are exact in f32, so the decoded value equals the
    # f64 closed form rounded once to f32 (fused or unfused).
    enc = synth.kquant_numpy(12, 1024, 16, seed=3).reshape(-1, 144)
    got = O.dequantize_tensor(12, enc)
    for b in range(0, enc.shape[0], 7):
        blk = enc[b]
        d = decode_half64(int(blk[0]) | int(blk[1]) << 8)
        dm = decode_half64(int(blk[2]) | int(blk[3]) << 8)
        sc, mn = O.q4_k_scales(bytes(blk[4:16]))
        for e in range(0, 256, 5):
            g = e // 32
            q = (blk[16 + (g // 2) * 32 + e % 32] >> (4 * (g % 2))) & 15
            exact = d * int(sc[g]) * int(q) - dm * int(mn[g])
            assert float(got[b * 256 + e]) == float(np.float32(exact))


# ----------------------------------------------------- GEMV (qwen_reference.rs:31-40)

def test_gguf_gemv_sequential_sum_within_f64_bound():
    rng = np.random.default_rng(11)
    k, n = 4096, 8
    w = rng.standard_normal((n, k)).astype(np.float32)
    x = rng.standard_normal(k).astype(np.float32)
    y = O.gguf_gemv(w, k, x)
    exact = (w.astype(np.float64) * x.astype(np.float64)).sum(axis=1)
    bound = k * 2.0 ** -24 * np.abs(w.astype(np.float64) * x).sum(axis=1) * 1.01
    assert np.all(np.abs(y - exact) <= bound)
    # exact sequential order: a permuted summation generally differs in the last bits
    seq = np.array([math.fsum([0.0])] * n)
    for r in range(n):
        acc = np.float32(-0.0)
        for i in range(k):
            acc = np.float32(acc + np.float32(x[i] * w[r, i]))
        seq[r] = acc
    assert np.array_equal(y, seq.astype(np.float32))


def test_quant_gemv_equals_dequant_then_gemv():
    enc = synth.kquant_numpy(13, 768, 12, seed=9)
    x = synth.activations_numpy(768, 1, 10)[0]
    y = O.quant_gemv(13, enc, 768, 12, x)
    w = O.dequantize_tensor(13, enc)
    assert np.array_equal(y, O.gguf_gemv(w, 768, x))


def test_quant_gemv_constant_block_reduces_to_scaled_sum():
    # all q = c, all scales s, all mins m: y = (d*s*c - dmin*m) * sum(x) (to f32 rounding)
    k, n = 1024, 3
    blk = bytearray(144)
    blk[0:2] = np.float16(0.015625).view(np.uint16).tobytes()
    blk[2:4] = np.float16(0.0078125).view(np.uint16).tobytes()
    blk[4:16] = pack_scales([5] * 8, [3] * 8)
    blk[16:] = bytes([0x77]) * 128  # every nibble = 7
    enc = np.frombuffer(bytes(blk) * (n * k // 256), np.uint8)
    x = synth.activations_numpy(k, 1, 12)[0]
    y = O.quant_gemv(12, enc, k, n, x)
    w = 0.015625 * 5 * 7 - 0.0078125 * 3
    expected = w * x.astype(np.float64).sum()
    assert np.allclose(y, expected, rtol=0, atol=k * 2 ** -23 * w * np.abs(x).sum())


def test_quant_gemv_members_are_independent_rows():
    enc = synth.kquant_numpy(14, 512, 9, seed=2)
    x = synth.activations_numpy(512, 3, 4)
    y = O.quant_gemv(14, enc, 512, 9, x, members=3)
    for m in range(3):
        assert np.array_equal(y[m], O.quant_gemv(14, enc, 512, 9, x[m]))


def test_quant_gemv_threaded_is_identical():
    enc = synth.kquant_numpy(12, 1024, 64, seed=6)
    x = synth.activations_numpy(1024, 1, 7)[0]
    assert np.array_equal(O.quant_gemv(12, enc, 1024, 64, x),
                          O.quant_gemv(12, enc, 1024, 64, x, threads=4))


# --------------------------------------------------- RMSNorm (qwen_reference.rs:550-556)

def test_rms_norm_reference_elementwise_case():
    x = np.array([1.0, -2.0, 3.0, -4.0], np.float32)
    w = np.array([1.0, 0.5, 2.0, -1.0], np.float32)
    got = O.rms_norm_raw(x, w, 1e-5)
    inv = 1.0 / math.sqrt((1 + 4 + 9 + 16) / 4.0 + 1e-5)
    assert np.allclose(got, x * inv * w, rtol=1e-6, atol=0)


def test_rms_norm_invariants():
    x = synth.activations_numpy(4096, 1, 1)[0]
    ones = np.ones(4096, np.float32)
    y = O.rms_norm_raw(x, ones, 1e-6)
    assert abs(float(np.sqrt((y.astype(np.float64) ** 2).mean())) - 1.0) < 1e-5
    # scale invariance once eps is negligible
    y2 = O.rms_norm_raw(x * np.float32(8.0), ones, 1e-6)
    assert np.allclose(y, y2, rtol=1e-5, atol=1e-6)
    # the reference rejects vectors longer than u16
    with pytest.raises(O.OracleError):
        O.rms_norm_raw(np.ones(65536, np.float32), np.ones(65536, np.float32), 1e-6)


# --------------------------------------------------------------- golden fixtures

def test_golden_fixtures_reproduce():
    import os
    import hashlib
    here = os.path.join(os.path.dirname(__file__), "golden", "kquant_golden.npz")
    g = np.load(here)
    for t in (12, 13, 14):
        enc = g[f"fixture_{t}_encoded"]
        assert np.array_equal(O.dequantize_tensor(t, enc), g[f"fixture_{t}_dequant"])
        assert np.array_equal(O.quant_gemv(t, enc, 512, 2, g[f"fixture_{t}_input"]),
                              g[f"fixture_{t}_output"])
    i = 0
    while f"random_{i}_meta" in g:
        t, k, n, m, seed = (int(v) for v in g[f"random_{i}_meta"])
        enc = g[f"random_{i}_encoded"]
        assert np.array_equal(enc, synth.kquant_numpy(t, k, n, seed))
        y = O.quant_gemv(t, enc, k, n, g[f"random_{i}_input"], members=m).reshape(m, n)
        assert np.array_equal(y, g[f"random_{i}_output"])
        digest = hashlib.sha256(O.dequantize_tensor(t, enc).tobytes()).hexdigest()
        assert digest == bytes(g[f"random_{i}_dequant_sha256"]).decode()
        i += 1
    assert i >= 6

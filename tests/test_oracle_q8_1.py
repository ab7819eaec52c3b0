"""Pins of the Q8_1 oracle (oracle/q8_1_oracle.py) on the CPU.

- The packer reproduces the reference's known-answer words
  (crates/nvidia/tests/cuda_activation.rs:14-40) and its rounding rule
  (ties away from zero).
- The f64 reference arithmetic reproduces the reference tests' own checks:
  with dyadic activations packing is exact, and the packed output equals the
  float output exactly (q4_q8_1.rs:207-230, q6_q8_1.rs:214-235); with lossy
  activations the difference stays within the packing error bound and is
  non-trivial (q4_q8_1.rs:232-246, q6_q8_1.rs:237-250).
- The restated fixture encoders decode (through the independent numpy
  decoder) to the closed forms the reference tests assert.
- A planted mistake (a dropped minimum term) breaks the exact equality.
"""
import numpy as np

from oracle import kquant_np
from oracle import q8_1_oracle as Q

from . import q8_1_fixtures as F


def test_pack_known_answer_words():
    got = Q.pack_q8_1(F.pack_kat_input())
    assert np.array_equal(got, F.pack_kat_words())


def test_pack_rounds_ties_away_from_zero_and_zero_blocks():
    x = np.zeros(64, np.float32)
    x[0] = 127.0           # d = 1
    x[1:5] = [0.5, -0.5, 2.5, -2.5]
    w = Q.pack_q8_1(x)
    b = w[1:9].view(np.int8)
    assert list(b[:5]) == [127, 1, -1, 3, -3]
    assert np.all(w[9:] == 0)   # the all-zero block packs to zero words


def test_pack_matches_a_direct_elementwise_evaluation():
    # a second, scalar evaluation of the same definition on random blocks
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(32 * 40) * 3).astype(np.float32)
    words = Q.pack_q8_1(x).reshape(-1, 9)
    for blk in range(40):
        v = x[32 * blk:32 * blk + 32]
        m = np.float32(max(abs(float(t)) for t in v))
        d = np.float32(m / np.float32(127))
        lanes = [np.float32(t) for t in v]
        for off in (16, 8, 4, 2, 1):
            lanes = [np.float32(lanes[i] + lanes[i ^ off]) for i in range(32)]
        head = int(np.float16(d).view(np.uint16)) | (int(np.float16(lanes[0]).view(np.uint16)) << 16)
        assert int(words[blk, 0]) == head
        for i in range(32):
            r = float(np.float32(v[i] / d))
            q = int(np.floor(abs(r) + 0.5)) * (1 if r >= 0 else -1)
            assert int(words[blk, 1:].view(np.int8)[i]) == q


def _rows(fixture):
    return F.encoded_rows(fixture)


def test_fixture_encoders_decode_to_the_stated_closed_forms():
    for enc, quants, scales, minima, d, dmin in F.q4k_fixture():
        got = kquant_np.dequantize(12, enc).astype(np.float64)
        want = np.array([d * scales[i // 32] * quants[i] - dmin * minima[i // 32] for i in range(256)])
        assert np.array_equal(got, want)
    for enc, quants, scales, d in F.q6k_fixture():
        got = kquant_np.dequantize(14, enc).astype(np.float64)
        want = np.array([d * scales[(i // 32) * 2 + (i % 32) // 16] * quants[i] for i in range(256)])
        assert np.array_equal(got, want)


def test_exact_activations_pack_exactly_and_match_float_arithmetic():
    x = F.activations(True)
    packed = Q.pack_q8_1(x)
    for t, fx in ((12, F.q4k_fixture()), (14, F.q6k_fixture())):
        ref = Q.q8_1_reference(t, _rows(fx), F.INPUTS, F.ROWS, x, packed)
        assert np.all(ref["packing_error_bound"] == 0.0), t
        assert np.array_equal(ref["packed_output"], ref["float_output"]), t


def test_lossy_activations_stay_within_the_packing_bound():
    x = F.activations(False)
    packed = Q.pack_q8_1(x)
    for t, fx in ((12, F.q4k_fixture()), (14, F.q6k_fixture())):
        ref = Q.q8_1_reference(t, _rows(fx), F.INPUTS, F.ROWS, x, packed)
        err = np.abs(ref["packed_output"] - ref["float_output"])
        assert np.all(err <= ref["packing_error_bound"] + 1e-10), t
        assert np.all(ref["packing_error_bound"] > 0), t
        assert np.any(err > 1e-4), t


def test_q5k_reference_equals_float_output_on_exact_inputs():
    # Q5_K: random blocks with the high bit set; dyadic activations are packed
    # exactly, so packed and float outputs agree exactly
    from engine_amd import synth
    enc = synth.kquant_numpy(13, F.INPUTS, 7, seed=3)
    x = F.activations(True)
    ref = Q.q8_1_reference(13, enc, F.INPUTS, 7, x, Q.pack_q8_1(x))
    assert np.all(ref["packing_error_bound"] == 0.0)
    assert np.allclose(ref["packed_output"], ref["float_output"], rtol=0, atol=1e-9 * np.abs(ref["float_output"]).max())


def test_planted_dropped_minimum_term_is_caught():
    x = F.activations(True)
    packed = Q.pack_q8_1(x)
    enc = _rows(F.q4k_fixture())
    ref = Q.q8_1_reference(12, enc, F.INPUTS, F.ROWS, x, packed)
    d, dmin, sc, mn, q = Q.block_fields(12, enc, F.INPUTS, F.ROWS)
    scale, total, qa = Q.unpack_q8_1(packed)
    a = d[:, :, None] * sc
    dot = (q.reshape(F.ROWS, 3, 8, 32) * qa.reshape(3, 8, 32)[None]).sum(axis=3)
    wrong = (a * scale.reshape(3, 8)[None] * dot).sum(axis=(1, 2))  # minimum term left out
    assert not np.array_equal(wrong, ref["float_output"])

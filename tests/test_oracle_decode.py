"""Pins the CPU oracle's decode-step functions (oracle/kquant_oracle.c,
oracle/qwen3_oracle.py) to mathematics and to independent implementations.

  * f32 -> binary16 (model_ops.rs:1211-1250): bit-exact against numpy's IEEE
    conversion over every exponent, ties and specials;
  * NEOX rope (qwen_reference.rs:403-419): identity at position 0, pair norms
    kept, the rotation group law, and a float64 evaluation of the formula;
  * attention (qwen_reference.rs:368-455): one token returns f16(v) exactly,
    equal keys give the mean of the values, the GQA head mapping, and a float64
    evaluation;
  * argmax (model_ops.rs:201-258): first maximum, NaN never chosen, -0 < +0;
  * the decode-step composition (decode.rs:544-631): against a float64 numpy
    forward written separately from the oracle (its own vectorised dequantiser,
    matmuls and softmax), so a wrong norm, residual or step order fails.
"""
import numpy as np
import pytest

from engine_amd import synth
from oracle import kquant_np as NP
from oracle import kquant_oracle as O
from oracle.qwen3_oracle import OracleQwen3

from .decode_helpers import SMALL, small_weights

# ------------------------------------------------------------------ f16


def test_f32_to_f16_matches_ieee_round_to_nearest_even():
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    # every f32 exponent that maps near the binary16 range, with random mantissas
    exps = rng.integers(100, 150, size=200_000).astype(np.uint32)
    near = (bits & 0x807FFFFF) | (exps << 23)
    # exact ties: the 13 dropped mantissa bits are 1000...0 (normal) and the
    # subnormal-range halfway points
    ties = ((rng.integers(0, 2**10, size=4096).astype(np.uint32) << 13) | 0x1000
            | (rng.integers(113, 143, size=4096).astype(np.uint32) << 23))
    sub_ties = (np.arange(1, 2048, dtype=np.float64) * 2.0**-25).astype(np.float32).view(np.uint32)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x477FE000, 0x477FF000,
                        0x477FEFFF, 0x38800000, 0x387FFFFF, 0x33000000, 0x33000001, 0x32FFFFFF, 1],
                       np.uint32)
    allb = np.concatenate([bits, near, ties, sub_ties, special])
    vals = allb.view(np.float32)
    got = np.array([O.f32_to_f16_bits(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    nan = np.isnan(vals)
    assert np.array_equal(got[~nan], ref[~nan])
    # NaN: quiet NaN 0x7e00 with the input's sign (model_ops.rs:1217-1220)
    assert np.all((got[nan] & 0x7FFF) == 0x7E00)
    assert np.array_equal(got[nan] >> 15, (allb[nan] >> 31).astype(np.uint16))


# ------------------------------------------------------------------ rope


def _rope64(x, heads, head_dim, rot, pos, base):
    out = x.astype(np.float64).reshape(heads, head_dim).copy()
    half = rot // 2
    p = np.arange(half)
    theta = pos * np.power(np.float64(base), -2.0 * p / rot)
    c, s = np.cos(theta), np.sin(theta)
    x0, x1 = out[:, :half].copy(), out[:, half:rot].copy()
    out[:, :half] = x0 * c - x1 * s
    out[:, half:rot] = x0 * s + x1 * c
    return out.reshape(-1)


@pytest.mark.parametrize("pos", [0, 1, 7, 2047])
def test_rope_matches_float64_formula(pos):
    rng = np.random.default_rng(pos)
    x = rng.standard_normal(4 * 128).astype(np.float32)
    got = O.rope_neox(x, 4, 128, 128, pos, 1.0e6)
    ref = _rope64(x, 4, 128, 128, pos, 1.0e6)
    # theta = pos * base^(-2p/128) is formed in f32; at pos ~2^11 its rounding
    # (and the f32 pow) move the angle by up to ~1e-4 rad
    assert np.abs(got - ref).max() <= 1e-6 + 2e-7 * pos * np.abs(x).max() * 4
    if pos == 0:
        assert np.array_equal(got, x)


def test_rope_keeps_pair_norms_and_composes():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(2 * 128).astype(np.float32)
    y = O.rope_neox(x, 2, 128, 128, 9, 1.0e6)
    n0 = np.hypot(x.reshape(2, 2, 64)[:, 0], x.reshape(2, 2, 64)[:, 1])
    n1 = np.hypot(y.reshape(2, 2, 64)[:, 0], y.reshape(2, 2, 64)[:, 1])
    np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-6)
    # rotations compose: rope(rope(x, 4), 5) == rope(x, 9) up to rounding
    z = O.rope_neox(O.rope_neox(x, 2, 128, 128, 4, 1.0e6), 2, 128, 128, 5, 1.0e6)
    np.testing.assert_allclose(z, y, rtol=0, atol=5e-5)
    # dims past rot_dims pass through; partial rope pairs (p, p + rot/2)
    w = O.rope_neox(x, 1, 256, 64, 3, 1.0e7)
    assert np.array_equal(w[64:], x[64:])
    np.testing.assert_allclose(w, _rope64(x, 1, 256, 64, 3, 1.0e7), atol=1e-5)


# ------------------------------------------------------------- attention


def _attention64(q, k, v, qn, kn, eps, base, qh, kvh, hd, pos, keys, values):
    """float64 restatement: f16-rounded K/V like the cache, softmax in float64."""
    q = q.astype(np.float64).reshape(qh, hd)
    k = k.astype(np.float64).reshape(kvh, hd)

    def norm(a, w):
        return a / np.sqrt((a * a).mean(axis=1, keepdims=True) + eps) * w.astype(np.float64)

    qr = _rope64(norm(q, qn), qh, hd, hd, pos, base).reshape(qh, hd)
    kr = _rope64(norm(k, kn), kvh, hd, hd, pos, base).reshape(kvh, hd)
    K = keys.view(np.float16).astype(np.float64).copy()
    V = values.view(np.float16).astype(np.float64).copy()
    K[pos] = kr.astype(np.float16)
    V[pos] = v.reshape(kvh, hd).astype(np.float16)
    out = np.zeros((qh, hd))
    for h in range(qh):
        g = h // (qh // kvh)
        s = K[:pos + 1, g] @ qr[h] / np.sqrt(hd)
        e = np.exp(s - s.max())
        out[h] = (e / e.sum()) @ V[:pos + 1, g]
    return out.reshape(-1)


def _attn_case(qh, kvh, pos, seed, cap=None):
    rng = np.random.default_rng(seed)
    hd = 128
    cap = cap or pos + 1
    q = rng.standard_normal(qh * hd).astype(np.float32)
    k = rng.standard_normal(kvh * hd).astype(np.float32)
    v = rng.standard_normal(kvh * hd).astype(np.float32)
    qn = synth.gamma_numpy(hd, seed + 1)
    kn = synth.gamma_numpy(hd, seed + 2)
    keys = rng.standard_normal((cap, kvh, hd)).astype(np.float16).view(np.uint16)
    values = rng.standard_normal((cap, kvh, hd)).astype(np.float16).view(np.uint16)
    return q, k, v, qn, kn, keys, values


@pytest.mark.parametrize("qh,kvh,pos", [(4, 1, 0), (8, 2, 5), (32, 8, 300)])
def test_attention_matches_float64(qh, kvh, pos):
    q, k, v, qn, kn, keys, values = _attn_case(qh, kvh, pos, 3 + pos)
    ref = _attention64(q, k, v, qn, kn, 1e-6, 1e6, qh, kvh, 128, pos, keys.copy(), values.copy())
    kk, vv = keys.copy(), values.copy()
    got = O.qwen3_attention(q, k, v, qn, kn, 1e-6, 1e6, qh, kvh, 128, pos, kk.reshape(pos + 1, -1),
                            vv.reshape(pos + 1, -1))
    assert np.abs(got - ref).max() <= 2e-5 * np.abs(ref).max()
    # the append wrote f16(v) at pos and left older slots alone
    assert np.array_equal(vv[pos].reshape(-1), v.astype(np.float16).view(np.uint16))
    assert np.array_equal(kk[:pos], keys[:pos]) and np.array_equal(vv[:pos], values[:pos])


def test_attention_single_token_returns_value_exactly():
    q, k, v, qn, kn, keys, values = _attn_case(8, 2, 0, 21)
    out = O.qwen3_attention(q, k, v, qn, kn, 1e-6, 1e6, 8, 2, 128, 0, keys.reshape(1, -1), values.reshape(1, -1))
    vf16 = v.astype(np.float16).astype(np.float32).reshape(2, 128)
    # softmax over one token is exactly 1: every q head returns its KV head's f16(v)
    for h in range(8):
        assert np.array_equal(out.reshape(8, 128)[h], vf16[h // 4])


def test_attention_equal_keys_average_values_and_gqa_mapping():
    qh, kvh, hd, pos = 8, 4, 128, 6
    rng = np.random.default_rng(8)
    q = rng.standard_normal(qh * hd).astype(np.float32)
    # k == 0: after the norm the new key is 0 and so are the cached keys below,
    # so every score is 0 and the weights are uniform
    k = np.zeros(kvh * hd, np.float32)
    v = rng.standard_normal(kvh * hd).astype(np.float32)
    keys = np.zeros((pos + 1, kvh, hd), np.uint16)
    # KV head g holds the constant value g + t/8 at token t
    vals = np.stack([np.stack([np.full(hd, g + t / 8, np.float16) for g in range(kvh)]) for t in range(pos + 1)])
    values = vals.view(np.uint16).copy()
    out = O.qwen3_attention(q, k, v, np.ones(hd, np.float32), np.ones(hd, np.float32), 1e-6, 1e6, qh, kvh, hd,
                            pos, keys.reshape(pos + 1, -1), values.reshape(pos + 1, -1)).reshape(qh, hd)
    vnew = v.astype(np.float16).astype(np.float64).reshape(kvh, hd)
    for h in range(qh):
        g = h // (qh // kvh)
        expect = (sum(g + t / 8 for t in range(pos)) + vnew[g]) / (pos + 1)
        np.testing.assert_allclose(out[h], expect, rtol=1e-6, atol=1e-6)


# ------------------------------------------------------------------ argmax


def test_argmax_first_max_nan_and_signed_zero():
    assert O.argmax(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1
    assert O.argmax(np.array([np.nan, -5.0, np.nan, -4.0], np.float32)) == 3
    assert O.argmax(np.array([-0.0, 0.0], np.float32)) == 1
    assert O.argmax(np.array([0.0, -0.0], np.float32)) == 0
    assert O.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    rng = np.random.default_rng(2)
    x = rng.standard_normal(151936).astype(np.float32)
    assert O.argmax(x) == int(np.argmax(x))


# ------------------------------------------------------- step composition

def _deq64(entry):
    t, k, n, enc = entry
    blocks = enc.reshape(-1, O.BLOCK_BYTES[t])
    return NP.dequantize(t, blocks).reshape(n, k).astype(np.float64)


def _forward64(cfg, w, tokens):
    """float64 numpy forward of `tokens` at positions 0.. (a separate implementation)."""
    eps, hd = cfg["epsilon"], 128
    qh, kvh = cfg["q_heads"], cfg["kv_heads"]
    W = {k: _deq64(v) for k, v in w.items() if isinstance(v, tuple)}

    def rms(x, g):
        return x / np.sqrt((x * x).mean() + eps) * g.astype(np.float64)

    def rms_heads(x, g, heads):
        x = x.reshape(heads, hd)
        return (x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * g.astype(np.float64)).reshape(-1)

    K = [[] for _ in range(cfg["layers"])]
    V = [[] for _ in range(cfg["layers"])]
    logits = []
    for pos, tok in enumerate(tokens):
        x = W["token_embd"][tok].copy()
        for l in range(cfg["layers"]):
            p = f"blk.{l}."
            n = rms(x, w[p + "attn_norm"])
            q = _rope64(rms_heads(W[p + "attn_q"] @ n, w[p + "attn_q_norm"], qh), qh, hd, hd, pos, 1e6)
            k = _rope64(rms_heads(W[p + "attn_k"] @ n, w[p + "attn_k_norm"], kvh), kvh, hd, hd, pos, 1e6)
            v = W[p + "attn_v"] @ n
            K[l].append(k.astype(np.float16).astype(np.float64).reshape(kvh, hd))
            V[l].append(v.astype(np.float16).astype(np.float64).reshape(kvh, hd))
            Ks, Vs = np.stack(K[l]), np.stack(V[l])
            att = np.zeros((qh, hd))
            for h in range(qh):
                g = h // (qh // kvh)
                s = Ks[:, g] @ q.reshape(qh, hd)[h] / np.sqrt(hd)
                e = np.exp(s - s.max())
                att[h] = (e / e.sum()) @ Vs[:, g]
            x = x + W[p + "attn_output"] @ att.reshape(-1)
            n = rms(x, w[p + "ffn_norm"])
            gt, up = W[p + "ffn_gate"] @ n, W[p + "ffn_up"] @ n
            x = x + W[p + "ffn_down"] @ (gt / (1 + np.exp(-gt)) * up)
        logits.append(W["output"] @ rms(x, w["output_norm"]))
    return logits


def test_decode_composition_matches_float64_forward():
    w = small_weights(SMALL, 40)
    orc = OracleQwen3(SMALL, w, capacity=8)
    tokens = [5, 299, 0, 17, 17, 123]
    ref = _forward64(SMALL, w, tokens)
    for pos, tok in enumerate(tokens):
        sel = orc.step(tok, pos)
        err = np.abs(orc.logits - ref[pos]).max() / np.abs(ref[pos]).max()
        assert err < 1e-4, (pos, err)
        assert sel == int(np.argmax(orc.logits))

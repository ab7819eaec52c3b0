"""GPU parity tests of the decode step, through the C ABI.

Bars (the oracle is oracle/kquant_oracle.c + oracle/qwen3_oracle.py):
  * fused GEMV forms (SwiGLU prologue, residual accumulate) within RTOL
    (normwise 1e-3) of the oracle; accumulate bit-equal to store + f32 add;
  * attention within RTOL of the oracle at positions across chunk boundaries
    and GQA groups 1..8; the appended f16 V bit-exact, K within RTOL;
  * argmax bit-exact (first maximum, NaN skipped);
  * the whole decoder: logits within 1e-3 normwise of the oracle over a
    prompt and greedy steps (the k-quant GEMV, the f16 cache and the online
    softmax each round differently from the sequential f32 oracle), greedy
    tokens equal wherever the oracle's top-2 margin exceeds the error;
  * graph replays bit-identical to direct launches (one capture replayed for
    every cache), batch members of up to 8 equal to single-sequence steps bit
    for bit (GEMV_WARP), batched steps of 5 and 8 members within 1e-3 of the
    oracle, generate() equal to stepping;
  * a prefill chunk equal to serial prefill steps bit for bit in GEMV_WARP
    (chunks of 3, 4, 8 and 12), within the GEMV bar in GEMV_FIXED16.
"""
import ctypes

import numpy as np
import pytest

from engine_amd import synth
from oracle import kquant_oracle as O
from oracle.qwen3_oracle import OracleQwen3

from .decode_helpers import small_weights
from .gpu_helpers import RTOL, max_rel_err, to_dev, to_host

pytestmark = pytest.mark.gpu

TINY = dict(layers=2, hidden=1024, q_heads=8, kv_heads=2, head_dim=128, ffn=4608, vocab=2048,
            rope_base=1.0e6, epsilon=1.0e-6)
WIDE = dict(layers=1, hidden=4096, q_heads=32, kv_heads=8, head_dim=128, ffn=12288, vocab=4096,
            rope_base=1.0e6, epsilon=1.0e-6)


def print_case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@pytest.fixture(scope="module")
def env():
    import torch
    import engine_amd as E
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    ctx = E.AmdContext(0)
    return {"E": E, "ctx": ctx, "store": E.AmdWeightStore(ctx), "n": [0],
            "k": {t: E.QwenGemvKernel.from_value_type(ctx, t) for t in (12, 13, 14)}}


def upload(env, t, k, n, enc):
    env["n"][0] += 1
    name = f"d{env['n'][0]}"
    env["store"].materialize_quantized(name, [k, n], t, enc)
    return env["store"].quantized_tensor(name)


def config(env, cfg):
    return env["E"].AmdQwen3Config(**cfg)


def build_decoder(env, cfg, w, max_members=1):
    E = env["E"]
    handles = {}
    for name, val in w.items():
        if isinstance(val, tuple):
            t, k, n, enc = val
            handles[name] = upload(env, t, k, n, enc)
        else:
            handles[name] = to_dev(val)
    layers = []
    for l in range(cfg["layers"]):
        p = f"blk.{l}."
        layers.append({f: handles[p + f] for f in
                       ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down",
                        "attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm")})
    dec = E.AmdQwen3Decode(env["ctx"], config(env, cfg), handles["token_embd"], handles["output"],
                           handles["output_norm"], layers, max_members)
    return dec


# ------------------------------------------------------------ fused GEMV


@pytest.mark.parametrize("t,k,n,members", [(13, 12288, 4096, 1), (13, 12288, 4096, 3), (12, 1024, 768, 2),
                                           (14, 4608, 512, 1)])
def test_swiglu_prologue_matches_oracle(env, t, k, n, members):
    print_case(test="swiglu", t=t, k=k, n=n, members=members)
    enc = synth.kquant_numpy(t, k, n, 100 + k + members)
    w = upload(env, t, k, n, enc)
    rng = np.random.default_rng(k + n)
    g = rng.standard_normal((members, k)).astype(np.float32) * 3
    u = rng.standard_normal((members, k)).astype(np.float32)
    y = to_dev(np.full(members * n, np.nan, np.float32))
    env["k"][t].execute_fused(w, to_dev(g), y, members, up=to_dev(u))
    got = to_host(y, env["ctx"]).reshape(members, n)
    for m in range(members):
        ref = O.quant_gemv(t, enc, k, n, O.swiglu(g[m], u[m]))
        assert max_rel_err(got[m], ref) <= RTOL, m


@pytest.mark.parametrize("t,k,n,members", [(12, 4096, 1024, 1), (12, 4096, 1024, 5), (13, 12288, 2048, 2)])
def test_accumulate_equals_store_plus_add(env, t, k, n, members):
    print_case(test="accumulate", t=t, k=k, n=n, members=members)
    enc = synth.kquant_numpy(t, k, n, 7 + members)
    w = upload(env, t, k, n, enc)
    rng = np.random.default_rng(members)
    x = to_dev(rng.standard_normal((members, k)).astype(np.float32))
    base = rng.standard_normal(members * n).astype(np.float32) * 100
    plain = to_dev(np.zeros(members * n, np.float32))
    env["k"][t].execute_warp_batch(w, x, plain, members)
    acc = to_dev(base)
    env["k"][t].execute_fused(w, x, acc, members, accumulate=True)
    got = to_host(acc, env["ctx"])
    assert np.array_equal(got.view(np.uint32), (base + to_host(plain)).view(np.uint32))
    if t == 13:
        u = to_dev(rng.standard_normal((members, k)).astype(np.float32))
        s = to_dev(np.zeros(members * n, np.float32))
        env["k"][t].execute_fused(w, x, s, members, up=u)
        a2 = to_dev(base)
        env["k"][t].execute_fused(w, x, a2, members, up=u, accumulate=True)
        assert np.array_equal(to_host(a2, env["ctx"]).view(np.uint32), (base + to_host(s)).view(np.uint32))


@pytest.mark.parametrize("t,n,members", [(12, 3072, 1), (12, 3072, 3), (12, 3072, 8), (13, 2048, 2), (14, 2048, 5),
                                         (12, 16384, 1), (14, 16384, 1)])
def test_gate_up_swiglu_pairs_match_oracle(env, t, n, members):
    print_case(test="gate_up_pairs", t=t, n=n, members=members)
    k = 4096
    ge, ue = synth.kquant_numpy(t, k, n, 300 + n), synth.kquant_numpy(t, k, n, 301 + n)
    gw, uw = upload(env, t, k, n, ge), upload(env, t, k, n, ue)
    x = synth.activations_numpy(k, members, seed=n + members)
    gamma = synth.gamma_numpy(k, seed=5)
    out = to_dev(np.full(members * n, np.nan, np.float32))
    env["k"][t].execute_gate_up_swiglu(gw, uw, to_dev(x), out, members, gamma=to_dev(gamma))
    got = to_host(out, env["ctx"]).reshape(members, n)
    for m in range(members):
        normed = O.rms_norm_raw(x[m], gamma, 1e-6)
        ref = O.swiglu(O.quant_gemv(t, ge, k, n, normed), O.quant_gemv(t, ue, k, n, normed))
        assert max_rel_err(got[m], ref) <= RTOL, m
    if members > 1:
        # GEMV_WARP batches: rows bit-identical to the single-member launch
        one = to_dev(np.full(n, np.nan, np.float32))
        env["k"][t].execute_gate_up_swiglu(gw, uw, to_dev(x[members - 1]), one, 1, gamma=to_dev(gamma))
        assert np.array_equal(to_host(one, env["ctx"]).view(np.uint32), got[members - 1].view(np.uint32))


def test_fused_rejects_swiglu_with_norm(env):
    E = env["E"]
    enc = synth.kquant_numpy(12, 256, 4, 1)
    w = upload(env, 12, 256, 4, enc)
    x = to_dev(np.zeros(256, np.float32))
    with pytest.raises(E.AmdKernelError) as err:
        env["k"][12].execute_fused(w, x, to_dev(np.zeros(4, np.float32)), 1, up=x, gamma=x)
    assert err.value.kind == "InvalidArgument"


# ------------------------------------------------------------- attention


def _fill_cache(env, cache, layer, keys_tok_major, values_tok_major):
    """Writes oracle-layout [tokens][kv_heads][128] f16 bits into the device's
    [kv_heads][capacity][128] layer cache."""
    lib, ctx = env["ctx"]._lib, env["ctx"]
    kptr, vptr = cache.layer(layer)
    cap = cache.capacity()
    for ptr, arr in ((kptr, keys_tok_major), (vptr, values_tok_major)):
        dev = np.zeros((arr.shape[1], cap, 128), np.uint16)
        dev[:, :arr.shape[0]] = arr.transpose(1, 0, 2)
        dev = np.ascontiguousarray(dev)
        assert lib.ribn_amd_memcpy_htod(ctx.handle, ctypes.c_void_p(ptr), dev.ctypes.data_as(ctypes.c_void_p),
                                        dev.nbytes) == 0


def _read_cache_row(env, cache, layer, pos, kv_heads):
    lib, ctx = env["ctx"]._lib, env["ctx"]
    kptr, vptr = cache.layer(layer)
    cap = cache.capacity()
    rows = []
    for ptr in (kptr, vptr):
        full = np.zeros((kv_heads, cap, 128), np.uint16)
        assert lib.ribn_amd_memcpy_dtoh(ctx.handle, full.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(ptr),
                                        full.nbytes) == 0
        rows.append(full[:, pos].copy())
    return rows


def _f16_err(a_bits, b_bits):
    a = a_bits.view(np.float16).astype(np.float64)
    b = b_bits.view(np.float16).astype(np.float64)
    return np.abs(a - b).max() / np.abs(b).max()


@pytest.mark.parametrize("qh,kvh", [(32, 8), (8, 2), (4, 4), (16, 2)])
def test_attention_matches_oracle(env, qh, kvh):
    positions = [0, 1, 15, 16, 33, 300, 2047, 2100]
    for i0 in range(0, len(positions), 3):
        _check_attention(env, qh, kvh, positions[i0:i0 + 3], i0)


@pytest.mark.parametrize("qh,kvh", [(32, 8), (8, 8)])
def test_attention_eight_members_long_chunks(env, qh, kvh):
    """Eight members over 8 KV heads fill the chip, so the launch splits each
    context into at most 8 chunks (272 tokens at position 2100) instead of
    64-token ones."""
    _check_attention(env, qh, kvh, [2100, 0, 511, 512, 1000, 63, 2047, 64], 99)


@pytest.mark.parametrize("qh,kvh", [(32, 8), (8, 2)])
def test_attention_wide_batch_chunks(env, qh, kvh):
    """From 9 members a chunk spans at least 128 tokens (at most 8 members: 64),
    so 12 and 16 members over contexts up to 2,101 tokens (every chunk edge
    from one to 17 chunks) run the wide chunking, against the oracle."""
    _check_attention(env, qh, kvh, [2100, 0, 127, 128, 129, 255, 256, 511, 1000, 63, 2047, 64], 7)
    _check_attention(env, qh, kvh, [1, 2, 130, 300, 383, 384, 700, 900, 1023, 1024, 1500, 1800, 2000, 2099, 5, 77],
                     8)


def _check_attention(env, qh, kvh, pos_list, seed):
    E = env["E"]
    cfg = dict(layers=1, hidden=qh * 128, q_heads=qh, kv_heads=kvh, head_dim=128, ffn=256, vocab=1,
               rope_base=1.0e6, epsilon=1.0e-6)
    cap = 2200
    members = len(pos_list)
    print_case(test="attention", qh=qh, kvh=kvh, positions=pos_list)
    caches, orc = [], []
    qs, ks, vs = [], [], []
    rng = np.random.default_rng(qh * 1000 + seed)
    qn = synth.gamma_numpy(128, qh + 1)
    kn = synth.gamma_numpy(128, qh + 2)
    for m, pos in enumerate(pos_list):
        c = E.AmdKvCache(env["ctx"], config(env, cfg), cap)
        keys = rng.standard_normal((cap, kvh, 128)).astype(np.float16).view(np.uint16)
        values = rng.standard_normal((cap, kvh, 128)).astype(np.float16).view(np.uint16)
        _fill_cache(env, c, 0, keys[:pos], values[:pos])
        caches.append(c)
        orc.append((keys, values))
        qs.append(rng.standard_normal(qh * 128).astype(np.float32))
        ks.append(rng.standard_normal(kvh * 128).astype(np.float32))
        vs.append(rng.standard_normal(kvh * 128).astype(np.float32) * 4)
    out = to_dev(np.full(members * qh * 128, np.nan, np.float32))
    posd = to_dev(np.array(pos_list, np.int32))
    args = (to_dev(np.concatenate(qs)), to_dev(np.concatenate(ks)), to_dev(np.concatenate(vs)), to_dev(qn),
            to_dev(kn), posd)
    E.attention_decode(env["ctx"], config(env, cfg), caches, 0, *args, out)
    got = to_host(out, env["ctx"]).reshape(members, -1)
    # a second launch at the same positions repeats the result bit for bit
    out2 = to_dev(np.full(members * qh * 128, np.nan, np.float32))
    E.attention_decode(env["ctx"], config(env, cfg), caches, 0, *args, out2)
    assert np.array_equal(to_host(out2, env["ctx"]).reshape(members, -1).view(np.uint32), got.view(np.uint32))
    for m, pos in enumerate(pos_list):
        keys, values = orc[m]
        kk = np.ascontiguousarray(keys[:pos + 1]).reshape(pos + 1, -1)
        vv = np.ascontiguousarray(values[:pos + 1]).reshape(pos + 1, -1)
        ref = O.qwen3_attention(qs[m], ks[m], vs[m], qn, kn, 1e-6, 1e6, qh, kvh, 128, pos, kk, vv)
        bad = ~np.isfinite(got[m].reshape(qh, 128))
        assert max_rel_err(got[m], ref) <= RTOL, (m, pos, int(bad.sum()), sorted(set(np.where(bad)[0].tolist())),
                                                 sorted(set(np.where(bad)[1].tolist()))[:16])
        krow, vrow = _read_cache_row(env, caches[m], 0, pos, kvh)
        # V is stored as f16(v) of the same input: bit-exact. K passes
        # through the norm and the rope, whose angle pos * base^(-2p/128)
        # moves by an f32 ulp (1.2e-4 rad near pos 2048) between pow
        # implementations: normwise bound, as for the outputs.
        assert np.array_equal(vrow.reshape(-1), vv[pos])
        assert _f16_err(krow.reshape(-1), kk[pos]) <= RTOL, pos


# ---------------------------------------------------------------- argmax


def test_argmax_matches_oracle(env):
    E = env["E"]
    rng = np.random.default_rng(3)
    vocab = 151936
    logits = rng.standard_normal((3, vocab)).astype(np.float32)
    logits[0, 17] = logits[0, 99999] = 9.0         # tie: first index wins
    logits[1, 5] = np.nan
    logits[1, 6] = 50.0
    logits[1, 7] = np.nan                           # NaN never selected
    logits[2, :] = -0.0
    logits[2, 151935] = 0.0                         # +0 ranks above -0
    sel = to_dev(np.zeros(3, np.int32))
    ops = E.AmdQwenOps(env["ctx"])
    ops.argmax_into_batch(to_dev(logits.reshape(-1)), vocab, sel)
    got = to_host(sel, env["ctx"])
    assert list(got) == [O.argmax(logits[m]) for m in range(3)] == [17, 6, 151935]


@pytest.mark.parametrize("vocab", [300, 1024, 4097, 65537])
def test_argmax_slices_match_oracle(env, vocab):
    """Row lengths that give one slice, an exact slice, ragged slices and rows
    that are not whole float4s; ties across slices, NaN runs, an all-NaN row."""
    E = env["E"]
    rng = np.random.default_rng(vocab)
    logits = rng.standard_normal((5, vocab)).astype(np.float32)
    logits[0, 3] = logits[0, vocab - 2] = 7.5          # first index wins across slices
    logits[1, : vocab // 2] = np.nan
    logits[1, vocab - 1] = -np.inf                      # every other value beats -inf
    logits[2, :] = np.nan                               # all NaN: index 0
    logits[3, :] = -np.inf
    logits[3, vocab // 3] = -1e30
    logits[4, :] = 1.0                                  # all equal: index 0
    sel = to_dev(np.zeros(5, np.int32))
    ops = E.AmdQwenOps(env["ctx"])
    ops.argmax_into_batch(to_dev(logits.reshape(-1)), vocab, sel)
    got = to_host(sel, env["ctx"])
    assert list(got) == [O.argmax(logits[m]) for m in range(5)]


# ------------------------------------------------------------- decoder


def _run_prompt(dec, cache, orc, tokens, gen_steps, env, tol):
    """Prefill `tokens`, then greedy steps; compares every step with the oracle."""
    pos = 0
    for tok in tokens[:-1]:
        dec.prefill_step(cache, tok, pos)
        orc.step(tok, pos, head=False)
        pos += 1
    tok = tokens[-1]
    picked = []
    for _ in range(gen_steps + 1):
        sel = dec.decode_step(cache, tok, pos)
        ref_sel = orc.step(tok, pos)
        logits = dec.copy_logits(0)
        err = max_rel_err(logits, orc.logits)
        assert err <= tol, (pos, err)
        assert max_rel_err(dec.copy_hidden(0), orc.hidden) <= tol
        top2 = np.sort(orc.logits.astype(np.float64))[-2:]
        margin = (top2[1] - top2[0]) / np.abs(orc.logits).max()
        if margin > 4 * max(err, 1e-7):
            assert sel == ref_sel, (pos, sel, ref_sel, margin, err)
        picked.append(sel)
        # teacher forcing on the oracle's choice keeps both on one sequence
        tok = ref_sel
        pos += 1
    return picked


@pytest.mark.parametrize("graphs", [True, False])
def test_decoder_matches_oracle_tiny(env, graphs):
    print_case(test="decoder_tiny", graphs=graphs)
    w = small_weights(TINY, 500)
    dec = build_decoder(env, TINY, w)
    dec.set_graphs(graphs)
    cache = env["E"].AmdKvCache(env["ctx"], config(env, TINY), 64)
    orc = OracleQwen3(TINY, w, 64)
    _run_prompt(dec, cache, orc, [3, 1500, 77, 2047, 9], 6, env, RTOL)


def test_decoder_matches_oracle_qwen3_8b_geometry(env):
    print_case(test="decoder_wide")
    w = small_weights(WIDE, 900, types={"attn_v": 14, "ffn_down": 13, "output": 14})
    dec = build_decoder(env, WIDE, w)
    cache = env["E"].AmdKvCache(env["ctx"], config(env, WIDE), 16)
    orc = OracleQwen3(WIDE, w, 16)
    _run_prompt(dec, cache, orc, [11, 4000], 2, env, RTOL)


def test_graph_replays_equal_direct_launches(env):
    print_case(test="graph_vs_direct")
    E = env["E"]
    w = small_weights(TINY, 77)
    dec = build_decoder(env, TINY, w)
    a = E.AmdKvCache(env["ctx"], config(env, TINY), 32)
    b = E.AmdKvCache(env["ctx"], config(env, TINY), 32)
    tok_a = tok_b = 42
    for pos in range(8):
        dec.set_graphs(True)
        tok_a = dec.decode_step(a, tok_a, pos)
        la = dec.copy_logits(0)
        dec.set_graphs(False)
        tok_b = dec.decode_step(b, tok_b, pos)
        lb = dec.copy_logits(0)
        assert tok_a == tok_b
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), pos


@pytest.mark.parametrize("members", [3, 5, 8])
def test_batch_members_equal_single_sequences(env, members):
    """decode_step_batch against decode_step per member: with the default
    GEMV_WARP arithmetic every member's logits and token equal its
    single-sequence step bit for bit, up to the reference's 8 batch members
    (cuda_reference.rs:5322-5334; up to 8 members the attention chunks
    depend on the caches' capacity only)."""
    print_case(test="batch_vs_single", members=members)
    E = env["E"]
    w = small_weights(TINY, 31)
    dec = build_decoder(env, TINY, w, max_members=members)
    prompts = [[1 + 97 * m + i for i in range(2 + (5 * m) % 7)] for m in range(members)]
    batch_caches = [E.AmdKvCache(env["ctx"], config(env, TINY), 64) for _ in range(members)]
    single_caches = [E.AmdKvCache(env["ctx"], config(env, TINY), 64) for _ in range(members)]
    nxt_b, nxt_s, pos = [], [], []
    for m, p in enumerate(prompts):
        for i, t in enumerate(p[:-1]):
            dec.prefill_step(batch_caches[m], t, i)
            dec.prefill_step(single_caches[m], t, i)
        nxt_b.append(p[-1])
        nxt_s.append(p[-1])
        pos.append(len(p) - 1)
    for _ in range(4):
        sel_b = dec.decode_step_batch(batch_caches, nxt_b, pos)
        logits_b = [dec.copy_logits(m) for m in range(members)]
        for m in range(members):
            sel = dec.decode_step(single_caches[m], nxt_s[m], pos[m])
            single = dec.copy_logits(0)
            assert np.array_equal(single.view(np.uint32), logits_b[m].view(np.uint32)), m
            assert sel == sel_b[m]
            nxt_s[m] = sel_b[m]
        nxt_b = sel_b
        pos = [p + 1 for p in pos]


@pytest.mark.parametrize("members", [5, 8, 12, 16, 33])
def test_batch_step_matches_oracle(env, members):
    """A batched decode step of 5 and 8 members (the f32 wave GEMV) and of
    12, 16 and 33 members (projections on the f32-faithful matrix-core GEMV)
    against the CPU oracle's decode step per member, teacher-forced, at the
    1e-3 bar."""
    print_case(test="batch_vs_oracle", members=members)
    E = env["E"]
    w = small_weights(TINY, 41 + members)
    dec = build_decoder(env, TINY, w, max_members=members)
    prompts = [[(211 * m + 13 * i + 5) % TINY["vocab"] for i in range(1 + m % 3)] for m in range(members)]
    caches = [E.AmdKvCache(env["ctx"], config(env, TINY), 16) for _ in range(members)]
    orcs = [OracleQwen3(TINY, w, 16) for _ in range(members)]
    nxt, pos = [], []
    for m, p in enumerate(prompts):
        for i, t in enumerate(p[:-1]):
            dec.prefill_step(caches[m], t, i)
            orcs[m].step(t, i, head=False)
        nxt.append(p[-1])
        pos.append(len(p) - 1)
    for _ in range(3):
        sel = dec.decode_step_batch(caches, nxt, pos)
        ref = [orcs[m].step(nxt[m], pos[m]) for m in range(members)]
        for m in range(members):
            logits = dec.copy_logits(m)
            err = max_rel_err(logits, orcs[m].logits)
            assert err <= RTOL, (m, err)
            assert max_rel_err(dec.copy_hidden(m), orcs[m].hidden) <= RTOL
            top2 = np.sort(orcs[m].logits.astype(np.float64))[-2:]
            if (top2[1] - top2[0]) / np.abs(orcs[m].logits).max() > 4 * max(err, 1e-7):
                assert sel[m] == ref[m], (m, sel[m], ref[m])
        nxt = ref  # teacher forcing on the oracle's choices
        pos = [p + 1 for p in pos]


def test_wide_batch_member_bits_independent_of_batch(env):
    """From 9 members (projections on the f32-faithful matrix-core GEMV,
    attention chunks of at least 128 tokens) over contexts of several chunks:
    every member's step against the
    oracle's at the decoder bar, and a member's logits independent of the batch
    it runs in (the same caches and tokens at 16 and at 9 members give the same
    bits for the shared members)."""
    print_case(test="wide_batch_bits")
    E = env["E"]
    w = small_weights(TINY, 77)
    dec = build_decoder(env, TINY, w, max_members=16)
    rng = np.random.default_rng(5)
    cap = 640
    caches, pos, orcs = [], [], []
    for m in range(16):
        c = E.AmdKvCache(env["ctx"], config(env, TINY), cap)
        orc = OracleQwen3(TINY, w, cap)
        p = int(rng.integers(100, cap - 8))
        for layer in range(TINY["layers"]):
            keys = rng.standard_normal((p, TINY["kv_heads"], 128)).astype(np.float16).view(np.uint16)
            values = rng.standard_normal((p, TINY["kv_heads"], 128)).astype(np.float16).view(np.uint16)
            _fill_cache(env, c, layer, keys, values)
            orc.keys[layer][:p] = keys
            orc.values[layer][:p] = values
        caches.append(c)
        orcs.append(orc)
        pos.append(p)
    toks = [int(t) for t in rng.integers(0, TINY["vocab"], 16)]
    sel16 = dec.decode_step_batch(caches, toks, pos)
    l16 = [dec.copy_logits(m) for m in range(9)]
    for m in range(16):
        orcs[m].step(toks[m], pos[m])
        err = max_rel_err(dec.copy_logits(m), orcs[m].logits)
        assert err <= RTOL, (m, pos[m], err)
    sel9 = dec.decode_step_batch(caches[:9], toks[:9], pos[:9])
    for m in range(9):
        assert np.array_equal(dec.copy_logits(m).view(np.uint32), l16[m].view(np.uint32)), m
        assert sel9[m] == sel16[m]


LONG_FFN = dict(layers=2, hidden=1024, q_heads=8, kv_heads=2, head_dim=128, ffn=16640, vocab=2048,
                rope_base=1.0e6, epsilon=1.0e-6)
WIDE_LONG_FFN = dict(layers=1, hidden=4352, q_heads=8, kv_heads=2, head_dim=128, ffn=17408, vocab=512,
                     rope_base=1.0e6, epsilon=1.0e-6)


@pytest.mark.parametrize("cfg_name,members", [("long", 1), ("long", 3), ("long", 12), ("wide", 1), ("wide", 2)])
def test_decoder_ffn_beyond_staging(env, cfg_name, members):
    """An FFN wider than one GEMV launch stages (16640 and 17408, the latter the
    reference's 27B down projection): the down projection runs the slice-split
    GEMV, after the gate/up pairs (hidden 1024) or after separate gate and up
    launches and an elementwise SwiGLU (hidden 4352). Teacher-forced steps
    against the oracle at the decoder bar, and up to 8 members every member's
    logits bit-identical to its single-sequence step."""
    print_case(test="ffn_beyond_staging", cfg=cfg_name, members=members)
    E = env["E"]
    cfg = LONG_FFN if cfg_name == "long" else WIDE_LONG_FFN
    w = small_weights(cfg, 91 + members, centered=True)
    dec = build_decoder(env, cfg, w, max_members=members)
    prompts = [[(131 * m + 17 * i + 3) % cfg["vocab"] for i in range(2 + m % 2)] for m in range(members)]
    caches = [E.AmdKvCache(env["ctx"], config(env, cfg), 16) for _ in range(members)]
    orcs = [OracleQwen3(cfg, w, 16) for _ in range(members)]
    nxt, pos = [], []
    for m, p in enumerate(prompts):
        for i, t in enumerate(p[:-1]):
            dec.prefill_step(caches[m], t, i)
            orcs[m].step(t, i, head=False)
        nxt.append(p[-1])
        pos.append(len(p) - 1)
    for step in range(2):
        dec.decode_step_batch(caches, nxt, pos)
        logits = [dec.copy_logits(m) for m in range(members)]
        ref = [orcs[m].step(nxt[m], pos[m]) for m in range(members)]
        for m in range(members):
            assert max_rel_err(logits[m], orcs[m].logits) <= RTOL, (step, m)
        if step == 0 and 1 < members <= 8:
            for m in range(members):
                single = E.AmdKvCache(env["ctx"], config(env, cfg), 16)
                for i, t in enumerate(prompts[m][:-1]):
                    dec.prefill_step(single, t, i)
                dec.decode_step(single, nxt[m], pos[m])
                assert np.array_equal(dec.copy_logits(0).view(np.uint32), logits[m].view(np.uint32)), m
        nxt = ref  # teacher forcing on the oracle's choices
        pos = [p + 1 for p in pos]


def _cache_bytes(env, cache, layers, kv_heads):
    lib, ctx = env["ctx"]._lib, env["ctx"]
    out = []
    for layer in range(layers):
        for ptr in cache.layer(layer):
            full = np.zeros((kv_heads, cache.capacity(), 128), np.uint16)
            assert lib.ribn_amd_memcpy_dtoh(ctx.handle, full.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(ptr),
                                            full.nbytes) == 0
            out.append(full)
    return out


@pytest.mark.parametrize("chunk,mode", [(3, "warp"), (4, "warp"), (8, "warp"), (12, "warp"), (4, "fixed16"),
                                        (8, "fixed16")])
def test_prefill_chunk_equals_serial_prefill(env, chunk, mode):
    """A prefill chunk (consecutive tokens of one sequence as one step's
    members, K/V appended before attention) against serial prefill_step.
    GEMV_WARP (default): bit-equal caches and next-step logits at every chunk
    up to 8, the reference's default chunk (serving.rs:357-371;
    cuda_reference.rs:5322-5334: batched rows equal batch-1 rows bit for bit);
    a chunk of 12 runs the f32-faithful matrix-core GEMV, so its caches and
    logits agree with serial prefill to f32 rounding (f16 cache values within
    one rounding step, logits within 1e-4 normwise). GEMV_FIXED16: within the
    GEMV bar where the matrix cores serve the FFN down (4) or every GEMV (8)."""
    print_case(test="prefill_chunk", chunk=chunk, mode=mode)
    E = env["E"]
    w = small_weights(TINY, 310)
    dec = build_decoder(env, TINY, w, max_members=chunk)
    if mode == "fixed16":
        dec.set_gemv_mode(E.GEMV_FIXED16)
    prompt = [(37 * i + 5) % TINY["vocab"] for i in range(2 * chunk + 3)]
    a = E.AmdKvCache(env["ctx"], config(env, TINY), 96)
    b = E.AmdKvCache(env["ctx"], config(env, TINY), 96)
    # chunked: two whole chunks, then the remainder serially
    for c0 in (0, chunk):
        dec.prefill_chunk(a, prompt[c0:c0 + chunk], c0)
    for i in range(2 * chunk, len(prompt) - 1):
        dec.prefill_step(a, prompt[i], i)
    for i in range(len(prompt) - 1):
        dec.prefill_step(b, prompt[i], i)
    last = len(prompt) - 1
    sel_a = dec.decode_step(a, prompt[-1], last)
    la = dec.copy_logits(0)
    sel_b = dec.decode_step(b, prompt[-1], last)
    lb = dec.copy_logits(0)
    ca = _cache_bytes(env, a, TINY["layers"], TINY["kv_heads"])
    cb = _cache_bytes(env, b, TINY["layers"], TINY["kv_heads"])
    if mode == "warp" and chunk <= 8:
        for x, y in zip(ca, cb):
            assert np.array_equal(x[:, :len(prompt)], y[:, :len(prompt)])
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
        assert sel_a == sel_b
    elif mode == "warp":
        for x, y in zip(ca, cb):
            assert _f16_err(x[:, :len(prompt)], y[:, :len(prompt)]) <= 1e-3
        assert max_rel_err(la, lb) <= 1e-4
        top = np.sort(lb)[-2:]
        if top[1] - top[0] > 4e-4 * np.abs(lb).max():
            assert sel_a == sel_b
    else:
        for x, y in zip(ca, cb):
            assert _f16_err(x[:, :len(prompt)], y[:, :len(prompt)]) <= 4e-3
        assert max_rel_err(la, lb) <= 2e-3
        top = np.sort(lb)[-2:]
        if top[1] - top[0] > 4e-3 * np.abs(lb).max():
            assert sel_a == sel_b


def test_prefill_chunk_rejects_bad_chunks(env):
    print_case(test="prefill_chunk_errors")
    E = env["E"]
    w = small_weights(TINY, 311)
    dec = build_decoder(env, TINY, w, max_members=4)
    cache = E.AmdKvCache(env["ctx"], config(env, TINY), 8)
    for tokens, pos, kind in (([1], 0, "InputLength"), ([1, 2, 3, 4, 5], 0, "InvalidPlan"),
                              ([1, 2, 3, 4], 5, "PositionOverflow"), ([1, TINY["vocab"]], 0, "InvalidPlan")):
        with pytest.raises(E.AmdKernelError) as err:
            dec.prefill_chunk(cache, tokens, pos)
        assert err.value.kind == kind, (tokens, pos)


def test_one_graph_serves_every_cache(env):
    """Captured steps hold no cache addresses: stepping several caches with
    graphs (one capture, replayed for each cache) equals direct launches."""
    print_case(test="graph_across_caches")
    E = env["E"]
    w = small_weights(TINY, 78)
    dec = build_decoder(env, TINY, w, max_members=2)
    g = [E.AmdKvCache(env["ctx"], config(env, TINY), 48 + 16 * i) for i in range(3)]
    d = [E.AmdKvCache(env["ctx"], config(env, TINY), 48 + 16 * i) for i in range(3)]
    tg, td = [5, 600, 1999], [5, 600, 1999]
    for pos in range(5):
        for i in range(3):
            dec.set_graphs(True)
            tg[i] = dec.decode_step(g[i], tg[i], pos)
            lg = dec.copy_logits(0)
            dec.set_graphs(False)
            td[i] = dec.decode_step(d[i], td[i], pos)
            ld = dec.copy_logits(0)
            assert np.array_equal(lg.view(np.uint32), ld.view(np.uint32)), (pos, i)
        dec.set_graphs(True)
        pair = dec.decode_step_batch([g[2], g[0]], [tg[2], tg[0]], [pos + 1, pos + 1])
        dec.set_graphs(False)
        assert dec.decode_step_batch([d[2], d[0]], [td[2], td[0]], [pos + 1, pos + 1]) == pair
    assert tg == td


def test_generate_equals_stepping(env):
    print_case(test="generate")
    E = env["E"]
    w = small_weights(TINY, 64)
    dec = build_decoder(env, TINY, w, max_members=2)
    ca = [E.AmdKvCache(env["ctx"], config(env, TINY), 320) for _ in range(2)]
    cb = [E.AmdKvCache(env["ctx"], config(env, TINY), 320) for _ in range(2)]
    for m in range(2):
        for i in range(3 + m):
            dec.prefill_step(ca[m], 10 * m + i, i)
            dec.prefill_step(cb[m], 10 * m + i, i)
    start_tok, start_pos = [100, 200], [3, 4]
    got = dec.generate(ca, start_tok, start_pos, 7)
    tok, pos = list(start_tok), list(start_pos)
    for s in range(7):
        tok = dec.decode_step_batch(cb, tok, pos)
        assert list(got[:, s]) == tok, s
        pos = [p + 1 for p in pos]
    # a longer run grows the history and recaptures
    got2 = dec.generate(ca, [1, 2], [10, 11], 300)
    assert got2.shape == (2, 300) and got2.max() < TINY["vocab"]


def test_decoder_errors(env):
    E = env["E"]
    w = small_weights(TINY, 5)
    dec = build_decoder(env, TINY, w, max_members=2)
    cache = E.AmdKvCache(env["ctx"], config(env, TINY), 4)
    with pytest.raises(E.AmdKernelError) as err:
        dec.decode_step(cache, 1, 4)
    assert err.value.kind == "PositionOverflow" and err.value.expected == 4
    with pytest.raises(E.AmdKernelError) as err:
        dec.decode_step(cache, TINY["vocab"], 0)
    assert err.value.kind == "InvalidPlan"
    with pytest.raises(E.AmdKernelError) as err:
        dec.decode_step_batch([cache, cache], [1, 2], [0, 1])
    assert err.value.kind == "InvalidPlan"
    with pytest.raises(E.AmdKernelError) as err:
        dec.generate([cache], [1], [2], 3)
    assert err.value.kind == "PositionOverflow"
    other = dict(TINY, layers=1)
    with pytest.raises(E.AmdKernelError) as err:
        dec.decode_step(E.AmdKvCache(env["ctx"], config(env, other), 8), 1, 0)
    assert err.value.kind == "InvalidPlan"
    with pytest.raises(E.AmdKernelError) as err:
        E.AmdKvCache(env["ctx"], config(env, dict(TINY, head_dim=64)), 8)
    assert err.value.kind == "InvalidPlan"
    # hidden up to 16384, ffn up to 65536 (its down projection on the slice-split GEMV)
    for bad_cfg, limit in ((dict(TINY, hidden=16640), 16384), (dict(TINY, ffn=65536 + 256), 65536)):
        with pytest.raises(E.AmdKernelError) as err:
            E.AmdKvCache(env["ctx"], config(env, bad_cfg), 8)
        assert err.value.kind == "InvalidPlan" and err.value.expected == limit
    long_dec = build_decoder(env, LONG_FFN, small_weights(LONG_FFN, 6))
    with pytest.raises(E.AmdKernelError) as err:
        long_dec.prefill_prompt(E.AmdKvCache(env["ctx"], config(env, LONG_FFN), 8), [1, 2], 0)
    assert err.value.kind == "InvalidPlan"  # the prefill matmul takes K <= 16384
    bad = dict(w)
    bad["blk.1.ffn_up"] = (12, 1024, 4352, synth.kquant_numpy(12, 1024, 4352, 3))
    with pytest.raises(E.AmdKernelError) as err:
        build_decoder(env, TINY, bad)
    assert err.value.kind == "InvalidPlan"


def _random_positions(seed):
    import random
    rng = random.Random(seed)
    members = rng.choice((1, 2, 3, 5, 8))
    edges = [0, 1, 62, 63, 64, 65, 127, 128, 255, 256, 1023, 1024, 2047, 2048, 2175, 2199]
    return [rng.choice(edges) if rng.random() < 0.5 else rng.randrange(2200) for _ in range(members)]


@pytest.mark.parametrize("seed", range(6))
def test_attention_random_positions(env, seed):
    """Seeded random member counts and positions (chunk edges at multiples of
    64 among them) against the oracle's attention, with the K/V append."""
    qh, kvh = ((32, 8), (16, 4), (8, 2))[seed % 3]
    _check_attention(env, qh, kvh, _random_positions(seed), 500 + seed)

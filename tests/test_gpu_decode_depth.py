"""Decoder parity at BASELINE config 4's shapes and context depth, through the
C ABI: four layers at the full Qwen3-8B geometry (hidden 4096, 32 query / 8 KV
heads of 128, SwiGLU 12288; q/k/v/o/gate/up Q4_K, down Q5_K), the full
Q4_K token_embd and Q6_K lm_head over the 151,936-token vocabulary, and KV
caches holding 2,048 cached tokens before the steps checked.

The caches are filled through the ABI's cache addresses with seeded random
f16 keys and values, and the CPU oracle (oracle/qwen3_oracle.py; its GEMVs on
16 host threads, the same sequential per-row arithmetic) gets the same f16
bytes. Then teacher-forced decode steps at positions 2048.. run at batch 1
and at batch 8 (eight caches with different contents), each member against
its own oracle sequence: logits and the final hidden state within 1e-3
normwise (the decoder bar of tests/test_gpu_decode.py), greedy tokens equal
wherever the oracle's top-2 margin exceeds the error. The reference
qualifies whole-model greedy replays against llama.cpp on its 27B artifact
(crates/nvidia/tests/cuda_reference.rs:4558,4769), which is not available
here: at model level this test pins the composition against the oracle, not
against llama.cpp.
"""
import ctypes

import numpy as np
import pytest

from engine_amd import synth
from oracle import kquant_oracle as O
from oracle.qwen3_oracle import OracleQwen3

from .gpu_helpers import RTOL, max_rel_err, to_dev

pytestmark = pytest.mark.gpu

DEPTH = dict(layers=4, hidden=4096, q_heads=32, kv_heads=8, head_dim=128, ffn=12288, vocab=151936,
             rope_base=1.0e6, epsilon=1.0e-6)
CONTEXT = 2048
CAPACITY = CONTEXT + 8


class ThreadedOracle(OracleQwen3):
    """The oracle step with its GEMVs split by rows over 16 host threads
    (each row's sequential f32 sum unchanged)."""

    def _gemv(self, name, x):
        t, k, n, enc = self.w[name]
        return O.quant_gemv(t, enc, k, n, x, threads=16)


def case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@pytest.fixture(scope="module")
def model():
    """Device handles and host copies of a seeded 4-layer Qwen3-8B-shaped model."""
    import torch
    import engine_amd as E
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    ctx = E.AmdContext(0)
    store = E.AmdWeightStore(ctx)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(4040)
    dev = torch.device("cuda:0")
    c = DEPTH
    h, f, q, kv = c["hidden"], c["ffn"], c["q_heads"] * 128, c["kv_heads"] * 128
    host, handles = {}, {}

    def add(name, t, k, n):
        # centered (zero-mean) weights: greedy tokens vary from step to step
        enc = synth.kquant_torch(t, k, n, gen, dev, centered=True)
        store.materialize_quantized(name, [k, n], t, enc)
        handles[name] = store.quantized_tensor(name)
        host[name] = (t, k, n, enc.cpu().numpy())

    def norm(name, n, seed):
        g = synth.gamma_numpy(n, seed)
        host[name] = g
        handles[name] = to_dev(g)

    add("token_embd", 12, h, c["vocab"])
    add("output", 14, h, c["vocab"])
    norm("output_norm", h, 1)
    layers = []
    for l in range(c["layers"]):
        p = f"blk.{l}."
        for name, t, k, n in (("attn_q", 12, h, q), ("attn_k", 12, h, kv), ("attn_v", 12, h, kv),
                              ("attn_output", 12, q, h), ("ffn_gate", 12, h, f), ("ffn_up", 12, h, f),
                              ("ffn_down", 13, f, h)):
            add(p + name, t, k, n)
        for j, nm in enumerate(("attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm")):
            norm(p + nm, 128 if nm in ("attn_q_norm", "attn_k_norm") else h, 100 + 10 * l + j)
        layers.append({nm: handles[p + nm] for nm in
                       ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down",
                        "attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm")})
    cfg = E.AmdQwen3Config(**c)
    dec = E.AmdQwen3Decode(ctx, cfg, handles["token_embd"], handles["output"], handles["output_norm"], layers, 8)
    torch.cuda.synchronize()
    return {"E": E, "ctx": ctx, "store": store, "dec": dec, "cfg": cfg, "host": host, "handles": handles}


def filled_cache(model, seed):
    """A device cache and an oracle sequence holding the same seeded f16
    keys and values at positions 0..CONTEXT-1 of every layer."""
    E, ctx = model["E"], model["ctx"]
    cache = E.AmdKvCache(ctx, model["cfg"], CAPACITY)
    orc = ThreadedOracle(DEPTH, model["host"], CAPACITY)
    rng = np.random.default_rng(seed)
    kvh = DEPTH["kv_heads"]
    for l in range(DEPTH["layers"]):
        for ptr, dst in zip(cache.layer(l), (orc.keys[l], orc.values[l])):
            full = np.zeros((kvh, CAPACITY, 128), np.float16)  # the cache's [kv_head][token][dim] layout
            full[:, :CONTEXT] = rng.standard_normal((kvh, CONTEXT, 128)).astype(np.float16)
            bits = full.view(np.uint16)
            assert ctx._lib.ribn_amd_memcpy_htod(ctx.handle, ctypes.c_void_p(ptr),
                                                 bits.ctypes.data_as(ctypes.c_void_p), bits.nbytes) == 0
            dst[:] = bits.transpose(1, 0, 2)  # the oracle's [token][kv_head][dim]
    return cache, orc


def check_member(model, m, orc, sel, ref):
    dec = model["dec"]
    logits = dec.copy_logits(m)
    err = max_rel_err(logits, orc.logits)
    herr = max_rel_err(dec.copy_hidden(m), orc.hidden)
    print(f"member {m}: logits {err:.2e}, hidden {herr:.2e}, token {sel} (oracle {ref})", flush=True)
    assert err <= RTOL, (m, err)
    assert herr <= RTOL, m
    top2 = np.sort(orc.logits.astype(np.float64))[-2:]
    if (top2[1] - top2[0]) / np.abs(orc.logits).max() > 4 * max(err, 1e-7):
        assert sel == ref, (m, sel, ref)


def test_batch1_steps_after_2048_context(model):
    """Three teacher-forced batch-1 steps at positions 2048, 2049, 2050."""
    case(test="depth batch1", layers=DEPTH["layers"], context=CONTEXT)
    cache, orc = filled_cache(model, 11)
    rng = np.random.default_rng(12)
    token = int(rng.integers(DEPTH["vocab"]))
    for s in range(3):
        pos = CONTEXT + s
        sel = model["dec"].decode_step(cache, token, pos)
        ref = orc.step(token, pos)
        check_member(model, 0, orc, sel, ref)
        token = ref  # teacher forcing on the oracle's choice


def test_batch8_steps_after_2048_context(model):
    """Two teacher-forced steps of eight members, each on its own filled
    cache, every member against its own oracle sequence."""
    case(test="depth batch8", layers=DEPTH["layers"], context=CONTEXT)
    pairs = [filled_cache(model, 100 + m) for m in range(8)]
    caches = [p[0] for p in pairs]
    orcs = [p[1] for p in pairs]
    rng = np.random.default_rng(13)
    tokens = [int(t) for t in rng.integers(DEPTH["vocab"], size=8)]
    for s in range(2):
        positions = [CONTEXT + s] * 8
        sel = model["dec"].decode_step_batch(caches, tokens, positions)
        refs = [orcs[m].step(tokens[m], positions[m]) for m in range(8)]
        for m in range(8):
            check_member(model, m, orcs[m], sel[m], refs[m])
        tokens = refs

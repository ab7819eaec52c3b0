"""Model-building helpers shared by the decode-step tests (CPU and GPU)."""
import numpy as np

from engine_amd import synth

SMALL = dict(layers=2, hidden=512, q_heads=4, kv_heads=2, head_dim=128, ffn=768, vocab=300,
             rope_base=1.0e6, epsilon=1.0e-6)


def small_weights(cfg, seed, types=None, centered=False):
    """Seeded model tensors; types maps tensor kind -> GGML type; centered:
    zero-mean Q4_K / Q5_K weights (synth.kquant_numpy)."""
    types = types or {}
    h, f, q, kv = cfg["hidden"], cfg["ffn"], cfg["q_heads"] * 128, cfg["kv_heads"] * 128
    w = {}
    s = seed

    def add(name, t, k, n):
        nonlocal s
        s += 1
        w[name] = (t, k, n, synth.kquant_numpy(t, k, n, s, centered))

    add("token_embd", types.get("token_embd", 12), h, cfg["vocab"])
    add("output", types.get("output", 14), h, cfg["vocab"])
    w["output_norm"] = synth.gamma_numpy(h, seed + 1000)
    for l in range(cfg["layers"]):
        p = f"blk.{l}."
        add(p + "attn_q", types.get("attn_q", 12), h, q)
        add(p + "attn_k", types.get("attn_k", 12), h, kv)
        add(p + "attn_v", types.get("attn_v", 12), h, kv)
        add(p + "attn_output", types.get("attn_output", 12), q, h)
        add(p + "ffn_gate", types.get("ffn_gate", 12), h, f)
        add(p + "ffn_up", types.get("ffn_up", 12), h, f)
        add(p + "ffn_down", types.get("ffn_down", 13), f, h)
        for j, nm in enumerate(("attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm")):
            w[p + nm] = synth.gamma_numpy(128 if "q_norm" in nm or "k_norm" in nm else h, seed + 2000 + 10 * l + j)
    return w

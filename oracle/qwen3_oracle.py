"""CPU oracle of the Qwen3 decode step -- TEST INFRASTRUCTURE ONLY.

Composes the C oracle's restatements (kquant_oracle) in the reference's
decode-step order (crates/nvidia/src/decode.rs:544-631 run_step, 929-1034
full_attention_layer, 655-677 run_output_head):

    hidden = dequantised token_embd row                    (q4_k_embedding)
    per layer:
      normed = rms_norm_raw(hidden, attn_norm)             (decode.rs:582-587)
      q, k, v = gguf GEMV of normed                        (cuda_reference.rs:889-902)
      attn = qwen3_attention(q, k, v, ...)                 (qwen_reference.rs:368-455, F16 cache)
      hidden += gemv(attn_output, attn)                    (residual_add)
      normed = rms_norm_raw(hidden, ffn_norm)              (decode.rs:601-606)
      hidden += gemv(ffn_down, swiglu(gemv(gate), gemv(up)))  (qwen_reference.rs:529-539)
    logits = gemv(output, rms_norm_raw(hidden, output_norm)); token = argmax(logits)

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
"""
from __future__ import annotations

import numpy as np

from . import kquant_oracle as O


class OracleQwen3:
    """Host state of one sequence: weights (encoded bytes and f32 norms) and
    the per-layer F16 KV caches [capacity][kv_heads][head_dim]."""

    def __init__(self, cfg: dict, weights: dict, capacity: int):
        self.cfg = cfg
        self.w = weights
        self.capacity = capacity
        kvh, hd = cfg["kv_heads"], cfg["head_dim"]
        self.keys = [np.zeros((capacity, kvh, hd), np.uint16) for _ in range(cfg["layers"])]
        self.values = [np.zeros((capacity, kvh, hd), np.uint16) for _ in range(cfg["layers"])]
        self.hidden = None
        self.logits = None

    def _gemv(self, name, x):
        t, k, n, enc = self.w[name]
        return O.quant_gemv(t, enc, k, n, x)

    def embed(self, token: int) -> np.ndarray:
        t, hidden, vocab, enc = self.w["token_embd"]
        bb = O.BLOCK_BYTES[t]
        row = hidden // 256 * bb
        return O.dequantize_tensor(t, enc[token * row:(token + 1) * row])

    def step(self, token: int, pos: int, head: bool = True):
        c = self.cfg
        eps = c["epsilon"]
        h = self.embed(token)
        for l in range(c["layers"]):
            p = f"blk.{l}."
            normed = O.rms_norm_raw(h, self.w[p + "attn_norm"], eps)
            q = self._gemv(p + "attn_q", normed)
            k = self._gemv(p + "attn_k", normed)
            v = self._gemv(p + "attn_v", normed)
            attn = O.qwen3_attention(q, k, v, self.w[p + "attn_q_norm"], self.w[p + "attn_k_norm"], eps,
                                     c["rope_base"], c["q_heads"], c["kv_heads"], c["head_dim"], pos,
                                     self.keys[l].reshape(self.capacity, -1), self.values[l].reshape(self.capacity, -1))
            h = (h + self._gemv(p + "attn_output", attn)).astype(np.float32)
            normed = O.rms_norm_raw(h, self.w[p + "ffn_norm"], eps)
            act = O.swiglu(self._gemv(p + "ffn_gate", normed), self._gemv(p + "ffn_up", normed))
            h = (h + self._gemv(p + "ffn_down", act)).astype(np.float32)
        self.hidden = h
        if not head:
            return None
        self.logits = self._gemv("output", O.rms_norm_raw(h, self.w["output_norm"], eps))
        return O.argmax(self.logits)

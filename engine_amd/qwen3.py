"""Host-side mirror of the reference's decode executor over the C ABI.

  AmdQwen3Config   <- the Qwen3 geometry (decode.rs keeps it in constants)
  AmdKvCache       <- CudaKvState, the KV part of CudaHybridState (state.rs:99-254, 529-660)
  AmdQwen3Decode   <- CudaQwen35Decode (decode.rs:236-800) and CudaQwen35BatchDecode
                      (decode.rs:1626-1960): new, prefill_step, decode_step,
                      decode_step_batch, copy_hidden, copy_logits
  attention_decode <- the per-layer sequence q/k norm + rope + kv_append_f16 +
                      attn_score_gqa (decode.rs:929-1034)

Every computation runs in libribn_amd.so; weights are AmdQuantizedWeight
handles and norm vectors are f32 device tensors (torch is only the allocator).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .kquant import RANK_CACHE, RANK_DECODER, AmdModelKernelError, _check, _live, _own, _ptr


@dataclass(frozen=True)
class AmdQwen3Config:
    layers: int = 36
    hidden: int = 4096
    q_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 12288
    vocab: int = 151936
    rope_base: float = 1.0e6
    epsilon: float = 1.0e-6

    def to_c(self) -> _lib.Qwen3Config:
        return _lib.Qwen3Config(self.layers, self.hidden, self.q_heads, self.kv_heads, self.head_dim, self.ffn,
                                self.vocab, self.rope_base, self.epsilon)


QWEN3_8B = AmdQwen3Config()


class AmdKvCache:
    """One sequence's f16 KV cache for every layer ([layer][kv_head][token][head_dim])."""

    def __init__(self, ctx, config: AmdQwen3Config, capacity: int):
        self.ctx = ctx
        self.config = config
        self._cfg = config.to_c()
        self.handle = ctypes.c_void_p()
        _check(ctx._lib.ribn_amd_kv_cache_create(ctx.handle, ctypes.byref(self._cfg), capacity,
                                                 ctypes.byref(self.handle)), AmdModelKernelError)
        _own(self, RANK_CACHE)

    def capacity(self) -> int:
        return int(self.ctx._lib.ribn_amd_kv_cache_capacity(self.handle))

    def layer(self, layer: int):
        """Device addresses of one layer's key and value caches."""
        k = ctypes.c_void_p()
        v = ctypes.c_void_p()
        _check(self.ctx._lib.ribn_amd_kv_cache_layer(self.handle, layer, ctypes.byref(k), ctypes.byref(v)),
               AmdModelKernelError)
        return k.value, v.value

    def close(self):
        if self.handle and _live():
            self.ctx._lib.ribn_amd_kv_cache_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _handles(caches):
    return (ctypes.c_void_p * len(caches))(*[c.handle.value for c in caches])


def attention_decode(ctx, config: AmdQwen3Config, caches, layer: int, q, k, v, q_norm, k_norm, positions, output):
    """One layer's decode attention for len(caches) members (positions: device int32)."""
    cfg = config.to_c()
    _check(ctx._lib.ribn_amd_attention_decode(ctx.handle, ctypes.byref(cfg), _handles(caches), len(caches), layer,
                                              _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm), _ptr(positions),
                                              _ptr(output), output.numel()), AmdModelKernelError)


def attention_prefill(ctx, config: AmdQwen3Config, cache, layer: int, q, k, v, q_norm, k_norm, tokens: int,
                      position: int, output):
    """One layer's causal attention for a prompt chunk of `tokens` tokens at
    `position` (the K/V appended first)."""
    cfg = config.to_c()
    _check(ctx._lib.ribn_amd_attention_prefill(ctx.handle, ctypes.byref(cfg), cache.handle, layer, _ptr(q), _ptr(k),
                                               _ptr(v), _ptr(q_norm), _ptr(k_norm), tokens, position, _ptr(output),
                                               output.numel()), AmdModelKernelError)


class AmdQwen3Decode:
    """Decode-step executor (CudaQwen35Decode + CudaQwen35BatchDecode).

    `layers` is a list of dicts with the weight handles attn_q, attn_k, attn_v,
    attn_output, ffn_gate, ffn_up, ffn_down and the f32 device tensors
    attn_norm, attn_q_norm, attn_k_norm, ffn_norm."""

    def __init__(self, ctx, config: AmdQwen3Config, token_embd, output, output_norm, layers, max_members: int = 1):
        self.ctx = ctx
        self.config = config
        self._cfg = config.to_c()
        # The decoder reads these every step: weight handles and norm tensors
        # stay referenced for its lifetime (the C side does not own them).
        self._keep = [output_norm, token_embd, output]
        arr = (_lib.Qwen3Layer * len(layers))()
        for i, lw in enumerate(layers):
            for name in _lib.QWEN3_LAYER_FIELDS:
                obj = lw[name]
                if hasattr(obj, "handle"):
                    setattr(arr[i], name, obj.handle.value)
                else:
                    setattr(arr[i], name, obj.data_ptr())
                self._keep.append(obj)
        self.handle = ctypes.c_void_p()
        _check(ctx._lib.ribn_amd_qwen3_decode_create(ctx.handle, ctypes.byref(self._cfg), token_embd.handle,
                                                     output.handle, _ptr(output_norm), arr, max_members,
                                                     ctypes.byref(self.handle)), AmdModelKernelError)
        _own(self, RANK_DECODER)

    def set_graphs(self, enabled: bool):
        _check(self.ctx._lib.ribn_amd_qwen3_decode_set_graphs(self.handle, 1 if enabled else 0))

    def set_gemv_mode(self, mode: int):
        """CudaQwen35Decode::set_gemv_mode (decode.rs:738-741): GEMV_WARP (f32
        activations, default) or GEMV_FIXED16 (opt-in block fixed point)."""
        _check(self.ctx._lib.ribn_amd_qwen3_decode_set_gemv_mode(self.handle, mode))

    def gemv_mode(self) -> int:
        return int(self.ctx._lib.ribn_amd_qwen3_decode_gemv_mode(self.handle))

    def prefill_step(self, cache: AmdKvCache, token: int, position: int):
        _check(self.ctx._lib.ribn_amd_qwen3_prefill_step(self.handle, cache.handle, token, position),
               AmdModelKernelError)

    def prefill_chunk(self, cache: AmdKvCache, tokens, position: int):
        """Consecutive prompt tokens of one sequence as one step's members."""
        n = len(tokens)
        tok = (ctypes.c_uint32 * n)(*[int(t) for t in tokens])
        _check(self.ctx._lib.ribn_amd_qwen3_prefill_chunk(self.handle, cache.handle, tok, n, position),
               AmdModelKernelError)

    def prefill_prompt(self, cache: AmdKvCache, tokens, position: int, chunk_tokens: int = 0):
        """A whole prompt (consecutive tokens of one sequence from `position`)
        on the prefill matmul, in chunks of `chunk_tokens` (0: 2048): the
        projections as matmuls over the chunk, causal chunk attention on the
        matrix cores, K/V written to the cache, no output head. Stands where
        the reference runs run_prefill_chunk (decode.rs:2149-2267)."""
        import numpy as np
        tok = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32).reshape(-1))
        ptr = tok.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))
        _check(self.ctx._lib.ribn_amd_qwen3_prefill_prompt(self.handle, cache.handle, ptr, tok.size, position,
                                                           chunk_tokens), AmdModelKernelError)

    def reserve_prompt(self, chunk_tokens: int = 0):
        """Allocates the prompt workspace for chunks of `chunk_tokens` tokens ahead of prefill_prompt."""
        _check(self.ctx._lib.ribn_amd_qwen3_reserve_prompt(self.handle, chunk_tokens), AmdModelKernelError)

    def decode_step(self, cache: AmdKvCache, token: int, position: int) -> int:
        out = ctypes.c_uint32()
        _check(self.ctx._lib.ribn_amd_qwen3_decode_step(self.handle, cache.handle, token, position,
                                                        ctypes.byref(out)), AmdModelKernelError)
        return out.value

    def decode_step_batch(self, caches, tokens, positions) -> list[int]:
        m = len(caches)
        tok = (ctypes.c_uint32 * m)(*[int(t) for t in tokens])
        pos = (ctypes.c_uint32 * m)(*[int(p) for p in positions])
        out = (ctypes.c_uint32 * m)()
        _check(self.ctx._lib.ribn_amd_qwen3_decode_step_batch(self.handle, _handles(caches), tok, pos, m, out),
               AmdModelKernelError)
        return list(out)

    def generate(self, caches, tokens, positions, steps: int) -> np.ndarray:
        """Greedy tokens [members][steps], looping on the device."""
        m = len(caches)
        tok = (ctypes.c_uint32 * m)(*[int(t) for t in tokens])
        pos = (ctypes.c_uint32 * m)(*[int(p) for p in positions])
        out = np.zeros((m, steps), np.uint32)
        _check(self.ctx._lib.ribn_amd_qwen3_generate(self.handle, _handles(caches), tok, pos, m, steps,
                                                     out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))),
               AmdModelKernelError)
        return out

    def copy_hidden(self, member: int = 0) -> np.ndarray:
        out = np.zeros(self.config.hidden, np.float32)
        _check(self.ctx._lib.ribn_amd_qwen3_copy_hidden(self.handle, member, out.ctypes.data_as(ctypes.c_void_p),
                                                        out.size))
        return out

    def copy_logits(self, member: int = 0) -> np.ndarray:
        out = np.zeros(self.config.vocab, np.float32)
        _check(self.ctx._lib.ribn_amd_qwen3_copy_logits(self.handle, member, out.ctypes.data_as(ctypes.c_void_p),
                                                        out.size))
        return out

    def close(self):
        if self.handle and _live():
            self.ctx._lib.ribn_amd_qwen3_decode_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

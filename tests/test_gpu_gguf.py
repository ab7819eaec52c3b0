"""GPU tests of GGUF staging (engine_amd/csrc/gguf.cpp ribn_amd_gguf_stage) and the
Qwen3 GGUF loader (engine_amd/gguf.py).

Bars: staged device bytes equal the file's tensor bytes exactly (the
reference's copy_quantized_to_host round trip, cuda_reference.rs:282-310),
for tensors spanning several staging chunks too; a GEMV over a staged weight
is within 1e-3 of the oracle; an over-budget request fails with
BudgetExceeded before any upload (staging.rs:246-258); a decoder loaded from
a Qwen3 GGUF matches the CPU oracle's decode step (logits within 1e-3
normwise, the oracle's greedy tokens).
"""
import ctypes

import numpy as np
import pytest

from engine_amd import synth
from oracle import kquant_oracle as O

from engine_amd import gguf_writer as W
from .gpu_helpers import RTOL, max_rel_err, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    import engine_amd as E
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return {"E": E, "ctx": E.AmdContext(0)}


def print_case(**kw):
    print("case", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def device_bytes(env, w) -> bytes:
    lib = env["ctx"]._lib
    n = int(lib.ribn_amd_weight_encoded_bytes(w.handle))
    buf = (ctypes.c_uint8 * n)()
    assert lib.ribn_amd_weight_copy_to_host(env["ctx"].handle, w.handle, buf, n) == 0
    return bytes(buf)


def test_stage_round_trips_bytes(env, tmp_path):
    print_case(test="gguf_stage")
    from engine_amd.gguf import GgufFile, stage
    rng = np.random.default_rng(3)
    specs = [("big.q4", 12, 4096, 12288), ("q5", 13, 12288, 40), ("q6", 14, 4096, 70)]
    tensors = [(n, [k, m], t, synth.kquant_numpy(t, k, m, seed=k + m).tobytes()) for n, t, k, m in specs]
    tensors += [("norm", [4096], 0, W.f32_payload(rng.standard_normal(4096))),
                ("table", [32, 4], 1, rng.integers(0, 256, 256, dtype=np.uint8).tobytes())]
    path = tmp_path / "stage.gguf"
    path.write_bytes(W.build([("general.architecture", W.STRING, "x")], tensors, alignment=64))
    g = GgufFile.open(str(path))
    staged = stage(env["ctx"], g, [t[0] for t in tensors])
    for name, dims, t, payload in tensors:
        obj = staged[name]
        w = obj if t in (12, 13, 14) else obj.weight
        assert device_bytes(env, w) == payload, name
    # a GEMV over a staged weight
    enc = np.frombuffer(tensors[1][3], np.uint8)
    x = synth.activations_numpy(12288, 1, seed=9)[0]
    y = to_dev(np.full(40, np.nan, np.float32))
    env["E"].AmdQ5KGemv.from_context(env["ctx"]).execute_warp(staged["q5"], to_dev(x), y)
    assert max_rel_err(to_host(y, env["ctx"]), O.quant_gemv(13, enc, 12288, 40, x)) <= RTOL


def test_stage_budget_and_missing(env, tmp_path):
    print_case(test="gguf_budget")
    from engine_amd.gguf import GgufError, GgufFile, stage
    payload = synth.kquant_numpy(12, 256, 8, seed=1).tobytes()
    path = tmp_path / "b.gguf"
    path.write_bytes(W.build([], [("w", [256, 8], 12, payload)]))
    g = GgufFile.open(str(path))
    with pytest.raises(GgufError) as e:
        stage(env["ctx"], g, ["w"], budget_bytes=len(payload) - 1)
    assert e.value.kind == "BudgetExceeded" and e.value.actual == len(payload)
    with pytest.raises(GgufError) as e:
        stage(env["ctx"], g, ["w", "absent"])
    assert e.value.kind == "MissingTensor"
    assert device_bytes(env, stage(env["ctx"], g, ["w"], budget_bytes=len(payload))["w"]) == payload


def test_qwen3_gguf_decodes_like_the_oracle(env, tmp_path):
    print_case(test="gguf_qwen3")
    from engine_amd.gguf import load_qwen3_decode
    from oracle.qwen3_oracle import OracleQwen3

    h, f, qd, kvd, vocab = 512, 768, 512, 256, 300
    cfg = dict(layers=2, hidden=h, q_heads=4, kv_heads=2, head_dim=128, ffn=f, vocab=vocab, rope_base=1.0e6,
               epsilon=1.0e-6)
    md = [("general.architecture", W.STRING, "qwen3"), ("qwen3.block_count", W.U32, 2),
          ("qwen3.embedding_length", W.U32, h), ("qwen3.feed_forward_length", W.U32, f),
          ("qwen3.attention.head_count", W.U32, 4), ("qwen3.attention.head_count_kv", W.U32, 2),
          ("qwen3.attention.key_length", W.U32, 128), ("qwen3.rope.freq_base", W.F32, 1.0e6),
          ("qwen3.attention.layer_norm_rms_epsilon", W.F32, 1.0e-6), ("qwen3.context_length", W.U32, 4096)]
    w, tensors = {}, []
    shapes = {"token_embd": (12, h, vocab), "output": (14, h, vocab)}
    for li in range(2):
        shapes.update({f"blk.{li}.attn_q": (12, h, qd), f"blk.{li}.attn_k": (12, h, kvd),
                       f"blk.{li}.attn_v": (13, h, kvd), f"blk.{li}.attn_output": (12, qd, h),
                       f"blk.{li}.ffn_gate": (12, h, f), f"blk.{li}.ffn_up": (12, h, f),
                       f"blk.{li}.ffn_down": (14, f, h)})
    for i, (name, (t, k, n)) in enumerate(shapes.items()):
        enc = synth.kquant_numpy(t, k, n, seed=70 + i)
        w[name] = (t, k, n, enc)
        tensors.append((f"{name}.weight", [k, n], t, enc.tobytes()))
    norms = {"output_norm": h}
    for li in range(2):
        norms.update({f"blk.{li}.attn_norm": h, f"blk.{li}.ffn_norm": h, f"blk.{li}.attn_q_norm": 128,
                      f"blk.{li}.attn_k_norm": 128})
    for i, (name, size) in enumerate(norms.items()):
        w[name] = synth.gamma_numpy(size, seed=90 + i)
        tensors.append((f"{name}.weight", [size], 0, W.f32_payload(w[name])))
    path = tmp_path / "qwen3.gguf"
    path.write_bytes(W.build(md, tensors))
    dec, got_cfg, _, _ = load_qwen3_decode(env["ctx"], str(path))
    assert (got_cfg.layers, got_cfg.hidden, got_cfg.q_heads, got_cfg.kv_heads, got_cfg.ffn, got_cfg.vocab) == \
        (2, h, 4, 2, f, vocab)
    cache = env["E"].AmdKvCache(env["ctx"], got_cfg, 16)
    orc = OracleQwen3(cfg, w, 16)
    tok = 11
    for pos in range(4):
        sel = dec.decode_step(cache, tok, pos)
        ref = orc.step(tok, pos)
        err = max_rel_err(dec.copy_logits(0), orc.logits)
        assert err <= 1e-3, (pos, err)
        top = np.sort(orc.logits)[-2:]
        if top[1] - top[0] > 4e-3 * np.abs(orc.logits).max():
            assert sel == ref, pos
        tok = ref

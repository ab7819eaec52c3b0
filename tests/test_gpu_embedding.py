"""GPU tests of the k-quant embedding gather (row a13), through the C ABI.

Bar: every gathered row is bit-identical to the oracle's dequantisation of
that row (the reference test `executes_q4_k_embedding_against_the_gguf_decoder`,
crates/nvidia/tests/cuda_reference.rs:2163-2207, uses the Q4_K device fixture
[512, 2] with a 1e-3 tolerance; the decoder arithmetic makes it exact).
"""
import os

import numpy as np
import pytest

from engine_amd import synth
from oracle import kquant_oracle as O

from .gpu_helpers import empty_dev, to_dev, to_host

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "kquant_golden.npz")
BLOCK_BYTES = {12: 144, 13: 176, 14: 210}


@pytest.fixture(scope="module")
def env():
    import torch
    import engine_amd as E
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    ctx = E.AmdContext(0)
    store = E.AmdWeightStore(ctx)
    return {"E": E, "ctx": ctx, "store": store, "n": [0]}


def upload(env, t, hidden, vocab, enc):
    env["n"][0] += 1
    name = f"emb{env['n'][0]}"
    env["store"].materialize_quantized(name, [hidden, vocab], t, enc)
    return env["store"].quantized_tensor(name)


def oracle_row(t, enc, hidden, token):
    per = hidden // 256 * BLOCK_BYTES[t]
    return O.dequantize_tensor(t, np.frombuffer(enc, np.uint8)[token * per:(token + 1) * per])


def test_reference_fixture_rows_bit_exact(env):
    g = np.load(GOLDEN)
    enc = g["fixture_12_encoded"]  # four Q4_K fixture blocks: [512, 2]
    w = upload(env, 12, 512, 2, enc)
    emb = env["E"].AmdQ4KEmbedding.from_context(env["ctx"])
    for token in (0, 1):
        print("CASE embedding fixture token", token, flush=True)
        out = empty_dev(512)
        emb.execute(w, token, out)
        got = to_host(out, env["ctx"])
        expected = oracle_row(12, enc.tobytes(), 512, token)
        assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))
        # the fixture's dequantised tensor holds the same rows
        assert np.array_equal(got.view(np.uint32), g["fixture_12_dequant"][token * 512:(token + 1) * 512]
                              .view(np.uint32))


@pytest.mark.parametrize("t", (12, 13, 14))
def test_batch_rows_bit_exact_with_duplicates(env, t):
    import torch
    hidden, vocab = 1024, 300
    print("CASE embedding batch", t, hidden, vocab, flush=True)
    enc = synth.kquant_numpy(t, hidden, vocab, seed=40 + t)
    w = upload(env, t, hidden, vocab, enc)
    emb = env["E"].AmdKQuantEmbedding.from_value_type(env["ctx"], t)
    tokens = np.array([0, 299, 17, 17, 150, 1], np.int32)
    out = empty_dev(len(tokens) * hidden)
    emb.execute_batch(w, to_dev(tokens), out)
    got = to_host(out, env["ctx"]).reshape(len(tokens), hidden)
    for m, tok in enumerate(tokens):
        expected = oracle_row(t, enc.tobytes(), hidden, int(tok))
        assert np.array_equal(got[m].view(np.uint32), expected.view(np.uint32)), (m, tok)
    # single-token calls agree with the batch bit for bit
    one = empty_dev(hidden)
    emb.execute(w, 150, one)
    assert np.array_equal(to_host(one, env["ctx"]).view(np.uint32), got[4].view(np.uint32))
    del torch


def test_batch_out_of_vocabulary_rows_are_left_unwritten(env):
    hidden, vocab = 512, 10
    print("CASE embedding out-of-vocabulary batch", flush=True)
    enc = synth.kquant_numpy(12, hidden, vocab, seed=7)
    w = upload(env, 12, hidden, vocab, enc)
    emb = env["E"].AmdQ4KEmbedding.from_context(env["ctx"])
    tokens = np.array([3, 10, 9, 4000000000 - 2**32], np.int32)  # ids 10 and 4e9 (as u32) are outside
    out = empty_dev(len(tokens) * hidden)  # NaN-filled
    emb.execute_batch(w, to_dev(tokens), out)
    got = to_host(out, env["ctx"]).reshape(len(tokens), hidden)
    assert np.array_equal(got[0].view(np.uint32), oracle_row(12, enc.tobytes(), hidden, 3).view(np.uint32))
    assert np.array_equal(got[2].view(np.uint32), oracle_row(12, enc.tobytes(), hidden, 9).view(np.uint32))
    assert np.all(np.isnan(got[1])) and np.all(np.isnan(got[3]))


def test_full_size_token_embd_rows(env):
    # Qwen3-8B token_embd shape [4096, 151936] Q4_K (311 MB), rows at both ends
    hidden, vocab = 4096, 151936
    print("CASE embedding token_embd full size", flush=True)
    import torch
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(5)
    enc_dev = synth.kquant_torch(12, hidden, vocab, gen, torch.device("cuda:0"))
    w = upload(env, 12, hidden, vocab, enc_dev)
    emb = env["E"].AmdQ4KEmbedding.from_context(env["ctx"])
    tokens = np.array([0, 151935, 77777], np.int32)
    out = empty_dev(len(tokens) * hidden)
    emb.execute_batch(w, to_dev(tokens), out)
    got = to_host(out, env["ctx"]).reshape(len(tokens), hidden)
    per = hidden // 256 * 144
    for m, tok in enumerate(tokens):
        row = enc_dev[int(tok) * per:(int(tok) + 1) * per].cpu().numpy()
        expected = O.dequantize_tensor(12, row)
        assert np.array_equal(got[m].view(np.uint32), expected.view(np.uint32)), tok


def test_validation_errors(env):
    E = env["E"]
    hidden, vocab = 512, 4
    enc = synth.kquant_numpy(12, hidden, vocab, seed=3)
    w = upload(env, 12, hidden, vocab, enc)
    emb = E.AmdQ4KEmbedding.from_context(env["ctx"])
    out = empty_dev(hidden)
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        emb.execute(w, 4, out)  # quantized.rs:1007-1012
    assert e.value.kind == "InvalidWeight" and (e.value.expected, e.value.actual) == (4, 4)
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        emb.execute(w, 0, empty_dev(hidden * 2))
    assert e.value.kind == "OutputLength" and (e.value.expected, e.value.actual) == (512, 1024)
    w6 = upload(env, 14, hidden, vocab, synth.kquant_numpy(14, hidden, vocab, seed=4))
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        emb.execute(w6, 0, out)
    assert e.value.kind == "UnsupportedValueType" and (e.value.expected, e.value.actual) == (12, 14)
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        emb.execute_batch(w, to_dev(np.zeros(0, np.int32)), out)
    assert e.value.kind == "InputLength" and (e.value.expected, e.value.actual) == (1, 0)
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        emb.execute_batch(w, to_dev(np.zeros(3, np.int32)), out)
    assert e.value.kind == "OutputLength" and (e.value.expected, e.value.actual) == (3 * 512, 512)

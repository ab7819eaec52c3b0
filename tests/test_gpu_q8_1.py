"""GPU parity tests of the Q8_1 path (engine_amd/csrc/q8_1.hip) through the C ABI.

Bars (the reference's own, crates/nvidia/tests/cuda_activation.rs and
q{4,6}_q8_1.rs GPU tests): packed words bit-identical to the oracle packer
and to the known-answer words; every GEMV output within
magnitude * eps_f32 * 32 + 1e-5 of the f64 packed arithmetic and within
packing bound + that allowance of the float output; batched rows
bit-identical to single-member launches; invalid storage rejected with the
reference's error kinds and outputs left untouched.
"""
import numpy as np
import pytest

from engine_amd import synth
from oracle import q8_1_oracle as Q

from . import q8_1_fixtures as F
from .gpu_helpers import to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    import engine_amd as E
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    ctx = E.AmdContext(0)
    store = E.AmdWeightStore(ctx)
    gemv = {12: E.AmdQ4KQ8_1Gemv(ctx), 13: E.AmdQ5KQ8_1Gemv(ctx), 14: E.AmdQ6KQ8_1Gemv(ctx)}
    return {"E": E, "ctx": ctx, "store": store, "q": E.AmdQ8_1Quantizer(ctx), "g": gemv, "n": [0]}


def print_case(**kw):
    print("case", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def upload(env, t, k, n, enc):
    env["n"][0] += 1
    name = f"q8w{env['n'][0]}"
    env["store"].materialize_quantized(name, [k, n], t, enc)
    return env["store"].quantized_tensor(name)


def words_dev(n, fill=0xFFFFFFFF):
    return to_dev(np.full(n, fill, np.uint32).view(np.int32))


def words_host(t, ctx):
    return to_host(t, ctx).view(np.uint32)


def pack_dev(env, x):
    out = words_dev(x.size // 32 * 9)
    env["q"].execute(to_dev(x), out)
    return out


def test_packer_known_answer_words(env):
    print_case(test="q8_pack_kat")
    x = to_dev(F.pack_kat_input())
    out = words_dev(45)
    env["q"].execute(x, out)
    got = words_host(out, env["ctx"])
    assert np.array_equal(got, F.pack_kat_words())
    env["q"].execute(x, out)  # caller-owned storage reused on the same stream
    assert np.array_equal(words_host(out, env["ctx"]), got)


@pytest.mark.parametrize("blocks", [1, 3, 8, 9, 257, 1024])
def test_packer_bit_identical_to_oracle(env, blocks):
    print_case(test="q8_pack", blocks=blocks)
    rng = np.random.default_rng(blocks)
    x = (rng.standard_normal(blocks * 32) * rng.uniform(0.01, 10)).astype(np.float32)
    x[:32] *= 0  # an all-zero block
    got = words_host(pack_dev(env, x), env["ctx"])
    assert np.array_equal(got, Q.pack_q8_1(x))


def test_packer_rejects_invalid_storage(env):
    E = env["E"]
    print_case(test="q8_pack_invalid")
    out = words_dev(9)
    for n, n_out, kind in ((31, 9, "InputLength"), (0, 9, "InputLength"), (32, 8, "OutputLength")):
        x = to_dev(np.zeros(max(n, 1), np.float32))[:n]
        o = words_dev(n_out)
        with pytest.raises(E.AmdQuantizedKernelError) as e:
            env["q"].execute(x, o)
        assert e.value.kind == kind
    assert np.all(words_host(out, env["ctx"]) == 0xFFFFFFFF)


def _check_rows(actual, ref):
    rounding = Q.rounding_allowance(ref)
    a = np.asarray(actual, np.float64)
    assert np.all(np.abs(a - ref["packed_output"]) <= rounding), np.abs(a - ref["packed_output"]).max()
    assert np.all(np.abs(a - ref["float_output"]) <= ref["packing_error_bound"] + rounding)


@pytest.mark.parametrize("t", [12, 14])
@pytest.mark.parametrize("kind", ["exact", "lossy", "zero"])
def test_fixture_gemv_matches_reference_arithmetic(env, t, kind):
    print_case(test="q8_fixture", t=t, kind=kind)
    fx = F.q4k_fixture() if t == 12 else F.q6k_fixture()
    enc = F.encoded_rows(fx)
    w = upload(env, t, F.INPUTS, F.ROWS, enc)
    x = {"exact": F.activations(True), "lossy": F.activations(False), "zero": np.zeros(F.INPUTS, np.float32)}[kind]
    packed = pack_dev(env, x)
    host_packed = words_host(packed, env["ctx"])
    assert np.array_equal(host_packed, Q.pack_q8_1(x))
    y = to_dev(np.full(F.ROWS, np.nan, np.float32))
    env["g"][t].execute(w, packed, y)
    _check_rows(to_host(y, env["ctx"]), Q.q8_1_reference(t, enc, F.INPUTS, F.ROWS, x, host_packed))


@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("k,n,members", [(4096, 512, 1), (4096, 512, 8), (12288, 64, 3), (768, 33, 5)])
def test_batched_gemv_matches_reference_and_single(env, t, k, n, members):
    print_case(test="q8_batch", t=t, k=k, n=n, members=members)
    enc = synth.kquant_numpy(t, k, n, seed=t + k + n)
    w = upload(env, t, k, n, enc)
    x = synth.activations_numpy(k, members, seed=members + 50)
    packed = pack_dev(env, x.reshape(-1))
    host_packed = words_host(packed, env["ctx"]).reshape(members, -1)
    y = to_dev(np.full(members * n, np.nan, np.float32))
    if members == 1:
        env["g"][t].execute(w, packed, y)
    else:
        env["g"][t].execute_batch(w, packed, y, members)
    got = to_host(y, env["ctx"]).reshape(members, n)
    for m in range(members):
        _check_rows(got[m], Q.q8_1_reference(t, enc, k, n, x[m], host_packed[m]))
    # each member's row is bit-identical to a single-member launch
    m = members - 1
    one = to_dev(np.full(n, np.nan, np.float32))
    env["g"][t].execute(w, to_dev(host_packed[m].view(np.int32)), one)
    assert np.array_equal(to_host(one, env["ctx"]).view(np.uint32), got[m].view(np.uint32))


def test_gemv_rejects_invalid_storage(env):
    E = env["E"]
    print_case(test="q8_invalid")
    enc = F.q4k_fixture()[0][0]
    w = upload(env, 12, 256, 1, enc)
    good = words_dev(72, 0)
    out = to_dev(np.array([123.0], np.float32))
    g = env["g"][12]
    cases = [
        (lambda: g.execute(w, words_dev(71, 0), out), "InputLength"),
        (lambda: g.execute(w, good, to_dev(np.zeros(2, np.float32))), "OutputLength"),
        (lambda: env["g"][14].execute(w, good, out), None),
        (lambda: g.execute_batch(w, good, out, 0), "InputLength"),
        (lambda: g.execute_batch(w, words_dev(144 * 5, 0), to_dev(np.zeros(9, np.float32)), 9), "InvalidWeight"),
        (lambda: g.execute_batch(w, words_dev(143, 0), to_dev(np.zeros(2, np.float32)), 2), "InputLength"),
    ]
    for call, kind in cases:
        with pytest.raises(E.AmdQuantizedKernelError) as e:
            call()
        if kind is not None:
            assert e.value.kind == kind
        else:
            assert e.value.kind in ("InvalidWeight", "UnsupportedValueType")
    assert to_host(out, env["ctx"])[0] == 123.0

"""GPU parity tests for the k-quant path, called through the C ABI.

Bars: dequantised weights bit-exact against the oracle; the exact-order GEMV
bit-exact against the oracle's sequential f32 dot; the wave GEMV (default
decode path), batched and RMSNorm-fused variants within max relative error
1e-3 (normwise, gpu_helpers.RTOL) of the oracle. Full BASELINE shapes are
checked against the oracle too (the C oracle runs them in well under a second
each) and through size-independent properties (linearity, batch/single
bit identity).
"""
import hashlib
import os

import numpy as np
import pytest

from engine_amd import synth
from oracle import kquant_oracle as O

from .gpu_helpers import (F32_BITWISE_MEMBERS, F32_RTOL, RTOL, empty_dev, max_rel_err, to_dev, to_host,
                          wide_range_activations)

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "kquant_golden.npz")
TYPES = (12, 13, 14)


@pytest.fixture(scope="module")
def env():
    import torch
    import engine_amd as E
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    ctx = E.AmdContext(0)
    store = E.AmdWeightStore(ctx)
    kernels = {t: E.QwenGemvKernel.from_value_type(ctx, t) for t in TYPES}
    return {"E": E, "ctx": ctx, "store": store, "k": kernels, "n": [0]}


def upload(env, t, k, n, enc):
    env["n"][0] += 1
    name = f"w{env['n'][0]}"
    env["store"].materialize_quantized(name, [k, n], t, enc)
    return env["store"].quantized_tensor(name)


def print_case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


# ------------------------------------------------------------------ dequant

@pytest.mark.parametrize("t", TYPES)
def test_dequant_reference_fixture_bit_exact(env, t):
    g = np.load(GOLDEN)
    enc = g[f"fixture_{t}_encoded"]
    w = upload(env, t, 512, 2, enc)
    out = empty_dev(1024)
    env["k"][t].dequantize(w, out)
    got = to_host(out, env["ctx"])
    assert np.array_equal(got.view(np.uint32), g[f"fixture_{t}_dequant"].view(np.uint32))


@pytest.mark.parametrize("t,k,n", [(12, 4096, 4096), (13, 12288, 512), (14, 4096, 1024), (14, 512, 33),
                                   (12, 256, 1), (13, 768, 7)])
def test_dequant_bit_exact_random(env, t, k, n):
    print_case(test="dequant", t=t, k=k, n=n)
    enc = synth.kquant_numpy(t, k, n, seed=1000 + t + k + n)
    w = upload(env, t, k, n, enc)
    out = empty_dev(k * n)
    env["k"][t].dequantize(w, out)
    got = to_host(out, env["ctx"])
    ref = O.dequantize_tensor(t, enc)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_golden_checksums(env):
    g = np.load(GOLDEN)
    i = 0
    while f"random_{i}_meta" in g:
        t, k, n, m, seed = (int(v) for v in g[f"random_{i}_meta"])
        w = upload(env, t, k, n, g[f"random_{i}_encoded"])
        out = empty_dev(k * n)
        env["k"][t].dequantize(w, out)
        got = to_host(out, env["ctx"])
        assert hashlib.sha256(got.tobytes()).hexdigest() == bytes(g[f"random_{i}_dequant_sha256"]).decode()
        i += 1


# ------------------------------------------------------- reference fixtures

@pytest.mark.parametrize("t", TYPES)
def test_reference_device_fixture(env, t):
    # cuda_reference.rs:858-960 (and the Q6_K twin): [512, 2], input (i%17)*0.125-1, |d| < 1e-3
    g = np.load(GOLDEN)
    w = upload(env, t, 512, 2, g[f"fixture_{t}_encoded"])
    x = to_dev(g[f"fixture_{t}_input"])
    expected = g[f"fixture_{t}_output"]
    for variant in ("execute", "execute_warp"):
        y = empty_dev(2)
        getattr(env["k"][t], variant)(w, x, y)
        got = to_host(y, env["ctx"])
        assert np.all(np.abs(got - expected) < 1e-3), (variant, got, expected)
    y = empty_dev(2)
    env["k"][t].execute(w, x, y)
    assert np.array_equal(to_host(y, env["ctx"]), expected)


# ------------------------------------------------------------- exact GEMV

@pytest.mark.parametrize("t,k,n", [(12, 1024, 64), (13, 768, 40), (14, 1280, 24), (12, 4096, 256)])
def test_exact_gemv_bit_identical_to_oracle(env, t, k, n):
    print_case(test="exact", t=t, k=k, n=n)
    enc = synth.kquant_numpy(t, k, n, seed=7 * k + n + t)
    x = synth.activations_numpy(k, 1, seed=n)[0]
    w = upload(env, t, k, n, enc)
    y = empty_dev(n)
    env["k"][t].execute(w, to_dev(x), y)
    got = to_host(y, env["ctx"])
    ref = O.quant_gemv(t, enc, k, n, x)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


# --------------------------------------------------------------- wave GEMV

def test_golden_random_cases_wave_and_batch(env):
    g = np.load(GOLDEN)
    i = 0
    while f"random_{i}_meta" in g:
        t, k, n, m, seed = (int(v) for v in g[f"random_{i}_meta"])
        print_case(test="golden", i=i, t=t, k=k, n=n, m=m)
        w = upload(env, t, k, n, g[f"random_{i}_encoded"])
        x = to_dev(g[f"random_{i}_input"].reshape(-1))
        y = empty_dev(m * n)
        env["k"][t].execute_warp_batch(w, x, y, m)
        got = to_host(y, env["ctx"]).reshape(m, n)
        assert max_rel_err(got, g[f"random_{i}_output"]) <= RTOL
        i += 1


# Qwen3-8B projection shapes plus ragged / small edges.
SHAPES = [
    (12, 4096, 4096), (12, 4096, 1024), (12, 4096, 12288), (13, 12288, 4096), (14, 4096, 4096),
    (14, 12288, 4096), (12, 256, 1), (13, 256, 3), (14, 256, 5), (12, 768, 333), (14, 2304, 77),
    (12, 5120, 100), (13, 4352, 64),
]


@pytest.mark.parametrize("t,k,n", SHAPES)
def test_wave_gemv_against_oracle(env, t, k, n):
    print_case(test="wave", t=t, k=k, n=n)
    enc = synth.kquant_numpy(t, k, n, seed=k + 3 * n + t)
    x = synth.activations_numpy(k, 1, seed=n + 5)[0]
    w = upload(env, t, k, n, enc)
    y = empty_dev(n)
    env["k"][t].execute_warp(w, to_dev(x), y)
    got = to_host(y, env["ctx"])
    ref = O.quant_gemv(t, enc, k, n, x, threads=8)
    err = max_rel_err(got, ref)
    print(f"max_rel_err={err:.3e}", flush=True)
    assert err <= RTOL


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("members", [1, 2, 3, 4, 5, 8, 13])
def test_batch_matches_oracle_and_single_bitwise(env, t, members):
    k, n = 1024, 96
    print_case(test="batch", t=t, members=members)
    enc = synth.kquant_numpy(t, k, n, seed=members + 31 * t)
    x = synth.activations_numpy(k, members, seed=members)
    w = upload(env, t, k, n, enc)
    xd = to_dev(x.reshape(-1))
    y = empty_dev(members * n)
    env["k"][t].execute_warp_batch(w, xd, y, members)
    got = to_host(y, env["ctx"]).reshape(members, n)
    ref = O.quant_gemv(t, enc, k, n, x.reshape(-1), members=members).reshape(members, n)
    assert max_rel_err(got, ref) <= RTOL
    if members > F32_BITWISE_MEMBERS:
        # 9..64 members: the f32-faithful matrix-core GEMV
        assert max_rel_err(got, ref) <= F32_RTOL
        return
    # GEMV_WARP batching (weights read once for up to 8 members) keeps every
    # row bit-identical to the single path (cuda_reference.rs:5322-5334)
    for m in range(members):
        ys = empty_dev(n)
        env["k"][t].execute_warp(w, to_dev(x[m]), ys)
        assert np.array_equal(to_host(ys, env["ctx"]).view(np.uint32), got[m].view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("k,n", [(5120, 5120), (5120, 17408), (17408, 5120)])
def test_reference_bench_shapes(env, t, k, n):
    """The shapes of the reference's own GEMV bench (int_dot_bench.rs:24, Qwen3.x-27B
    projections; K = 17408 leaves a 4-block last slice): execute_warp within 1e-3 of the
    oracle, and 8 members through execute_warp_batch bit-identical to their single
    launches (cuda_reference.rs:5322-5334)."""
    print_case(test="reference_bench_shape", t=t, k=k, n=n)
    enc = synth.kquant_numpy(t, k, n, seed=k + 7 * n + t)
    x = synth.activations_numpy(k, 8, seed=abs(k - n) + t)
    w = upload(env, t, k, n, enc)
    y = empty_dev(8 * n)
    env["k"][t].execute_warp_batch(w, to_dev(x.reshape(-1)), y, 8)
    got = to_host(y, env["ctx"]).reshape(8, n)
    for m in (0, 5):
        assert max_rel_err(got[m], O.quant_gemv(t, enc, k, n, x[m], threads=8)) <= RTOL
    for m in range(8):
        ys = empty_dev(n)
        env["k"][t].execute_warp(w, to_dev(x[m]), ys)
        assert np.array_equal(to_host(ys, env["ctx"]).view(np.uint32), got[m].view(np.uint32))


@pytest.mark.parametrize("t,k,n,members", [(13, 256 * 130, 75, 3), (14, 65536, 64, 1), (12, 65536, 40, 8),
                                           (12, 16640, 333, 2)])
def test_long_k_slice_split(env, t, k, n, members):
    """K beyond one workgroup's staging (16384) runs the f32 GEMV's slice-split form
    (one slice staged per workgroup, slice totals added in order): a grouped launch of
    two weights against the oracle, members bit-identical to their single launches, and
    the accumulating form (output += W x) equal to a store plus a host add."""
    print_case(test="long_k", t=t, k=k, n=n, members=members)
    encs = [synth.kquant_numpy(t, k, n, seed=k + n + j) for j in range(2)]
    x = synth.activations_numpy(k, members, seed=n + members)
    ws = [upload(env, t, k, n, e) for e in encs]
    ys = [empty_dev(members * n) for _ in ws]
    env["k"][t].execute_group(ws, to_dev(x.reshape(-1)), ys, members)
    for j in range(2):
        got = to_host(ys[j], env["ctx"]).reshape(members, n)
        ref = O.quant_gemv(t, encs[j], k, n, x.reshape(-1), members=members).reshape(members, n)
        assert max_rel_err(got, ref) <= RTOL
        for m in range(members):
            y1 = empty_dev(n)
            env["k"][t].execute_warp(ws[j], to_dev(x[m]), y1)
            assert np.array_equal(to_host(y1, env["ctx"]).view(np.uint32), got[m].view(np.uint32))
    base = synth.activations_numpy(n, members, seed=7).reshape(-1)
    acc = to_dev(base)
    env["k"][t].execute_fused(ws[0], to_dev(x.reshape(-1)), acc, members, accumulate=True)
    want = base + to_host(ys[0], env["ctx"])
    assert np.array_equal(to_host(acc, env["ctx"]).view(np.uint32), want.view(np.uint32))


def test_long_k_modes_and_exact_fallback(env):
    """The opt-in fixed-point mode takes the same slice-split f32 form beyond K = 16384
    (same bits as the default mode); past the split form's largest K (65536) a plain
    product still runs on the exact-order kernel, bit-identical to the oracle's
    sequential dot (qwen_reference.rs:31-40)."""
    E = env["E"]
    t, k, n = 12, 17408, 96
    enc = synth.kquant_numpy(t, k, n, seed=5)
    x = synth.activations_numpy(k, 1, seed=6)[0]
    w = upload(env, t, k, n, enc)
    outs = []
    for mode in (E.GEMV_WARP, E.GEMV_FIXED16):
        env["k"][t].set_mode(mode)
        y = empty_dev(n)
        env["k"][t].execute_warp(w, to_dev(x), y)
        outs.append(to_host(y, env["ctx"]))
    env["k"][t].set_mode(E.GEMV_WARP)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    k2, n2 = 65536 + 256, 24
    enc2 = synth.kquant_numpy(t, k2, n2, seed=8)
    x2 = synth.activations_numpy(k2, 1, seed=9)[0]
    w2 = upload(env, t, k2, n2, enc2)
    y2 = empty_dev(n2)
    env["k"][t].execute_warp(w2, to_dev(x2), y2)
    ref = O.quant_gemv(t, enc2, k2, n2, x2)
    assert np.array_equal(to_host(y2, env["ctx"]).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("t,k,n", [(12, 4096, 12288), (13, 12288, 4096), (14, 4096, 4096)])
def test_linearity_full_size(env, t, k, n):
    # W(a x1 + b x2) = a W x1 + b W x2 (size-independent property)
    enc = synth.kquant_numpy(t, k, n, seed=99 + t)
    x = synth.activations_numpy(k, 2, seed=17)
    a, b = np.float32(0.75), np.float32(-1.25)
    w = upload(env, t, k, n, enc)
    outs = []
    for v in (x[0], x[1], a * x[0] + b * x[1]):
        y = empty_dev(n)
        env["k"][t].execute_warp(w, to_dev(v.astype(np.float32)), y)
        outs.append(to_host(y, env["ctx"]).astype(np.float64))
    assert max_rel_err(outs[2], a * outs[0] + b * outs[1]) <= RTOL


# -------------------------------------------------------------- RMSNorm

def test_rms_norm_against_oracle(env):
    import torch
    g = np.load(GOLDEN)
    ops = env["E"].AmdQwenOps.from_context(env["ctx"])
    for name, eps in (("rms_small", 1e-5), ("rms_4096", 1e-6)):
        x = to_dev(g[f"{name}_input"])
        w = to_dev(g[f"{name}_weight"])
        y = torch.empty_like(x)
        ops.rms_norm(x, w, y, eps)
        got = to_host(y, env["ctx"])
        assert np.allclose(got, g[f"{name}_output"], rtol=1e-5, atol=1e-6)
    xb = synth.activations_numpy(4096, 3, seed=2)
    gam = synth.gamma_numpy(4096, seed=3)
    yb = empty_dev(3 * 4096)
    ops.rms_norm_batch(to_dev(xb.reshape(-1)), to_dev(gam), yb, 4096, 1e-6)
    got = to_host(yb, env["ctx"]).reshape(3, 4096)
    for m in range(3):
        assert np.allclose(got[m], O.rms_norm_raw(xb[m], gam, 1e-6), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("t,k,n,members", [(12, 4096, 4096, 1), (12, 4096, 12288, 1), (12, 4096, 1024, 4),
                                           (14, 4096, 512, 2), (13, 4096, 256, 3)])
def test_fused_rms_norm_gemv(env, t, k, n, members):
    print_case(test="fused", t=t, k=k, n=n, m=members)
    enc = synth.kquant_numpy(t, k, n, seed=5 + n)
    x = synth.activations_numpy(k, members, seed=6)
    gam = synth.gamma_numpy(k, seed=7)
    w = upload(env, t, k, n, enc)
    y = empty_dev(members * n)
    env["k"][t].execute_rms_norm(w, to_dev(x.reshape(-1)), to_dev(gam), 1e-6, y, members)
    got = to_host(y, env["ctx"]).reshape(members, n)
    for m in range(members):
        normed = O.rms_norm_raw(x[m], gam, 1e-6)
        ref = O.quant_gemv(t, enc, k, n, normed, threads=8)
        assert max_rel_err(got[m], ref) <= RTOL


# ------------------------------------------------------ boundary behaviour

def test_weight_bytes_round_trip(env):
    # cuda_reference.rs:282-310: encoded bytes come back unchanged
    import io
    store = env["store"]
    for t in TYPES:
        enc = synth.kquant_numpy(t, 512, 9, seed=t)
        store.materialize_quantized(f"rt{t}", [512, 9], t, enc)
        assert store.copy_quantized_to_host(f"rt{t}") == enc.tobytes()
        store.materialize_quantized_reader(f"rr{t}", [512, 9], t, enc.nbytes, io.BytesIO(enc.tobytes()))
        assert store.copy_quantized_to_host(f"rr{t}") == enc.tobytes()
    E = env["E"]
    with pytest.raises(E.AmdWeightError) as e:
        store.materialize_quantized_reader("short", [512, 9], 12, 144 * 18, io.BytesIO(b"\0" * 100))
    assert e.value.kind == "SourceIncomplete" and e.value.actual == 100


def test_validation_errors(env):
    import torch
    E = env["E"]
    enc = synth.kquant_numpy(12, 512, 4, seed=1)
    w = upload(env, 12, 512, 4, enc)
    x = torch.zeros(512, device="cuda:0")
    y = torch.zeros(4, device="cuda:0")
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        env["k"][13].execute_warp(w, x, y)
    assert e.value.kind == "UnsupportedValueType" and (e.value.expected, e.value.actual) == (13, 12)
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        env["k"][12].execute_warp(w, torch.zeros(256, device="cuda:0"), y)
    assert e.value.kind == "InputLength" and (e.value.expected, e.value.actual) == (512, 256)
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        env["k"][12].execute_warp(w, x, torch.zeros(8, device="cuda:0"))
    assert e.value.kind == "OutputLength" and (e.value.expected, e.value.actual) == (4, 8)
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        env["k"][12].execute_warp_batch(w, x, y, 0)
    assert e.value.kind == "InputLength" and (e.value.expected, e.value.actual) == (1, 0)
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        env["k"][12].execute_warp_batch(w, x, y, 65)
    assert e.value.kind == "InvalidWeight"
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        env["k"][12].execute_warp(w, torch.zeros(520, device="cuda:0")[1:513], y)
    assert e.value.kind == "InvalidArgument"  # misaligned device pointer
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        env["k"][12].execute_warp(w, torch.zeros(512), y)
    assert e.value.kind == "InvalidArgument"  # host memory
    bad = upload(env, 12, 512, 3, synth.kquant_numpy(12, 512, 4, seed=1))  # 4 rows of bytes for 3
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        env["k"][12].execute_warp(bad, x, torch.zeros(3, device="cuda:0"))
    assert e.value.kind == "InvalidWeight" and e.value.expected == 3 * 2 * 144
    ops = E.AmdQwenOps.from_context(env["ctx"])
    with pytest.raises(E.AmdModelKernelError) as e:
        ops.rms_norm(x, torch.zeros(511, device="cuda:0"), torch.zeros(512, device="cuda:0"), 1e-6)
    assert e.value.kind == "WeightLength"
    with pytest.raises(E.AmdModelKernelError) as e:
        ops.rms_norm(x, x, torch.zeros(512, device="cuda:0"), 0.0)
    assert e.value.kind == "InvalidEpsilon"
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        E.QwenGemvKernel.from_value_type(env["ctx"], 11)
    assert e.value.kind == "UnsupportedValueType" and e.value.actual == 11


@pytest.mark.parametrize("t,k,ns,members,norm", [(12, 4096, (4096, 1024, 1024), 1, True),
                                                 (12, 4096, (12288, 12288), 1, True),
                                                 (12, 4096, (512, 96, 33), 3, True),
                                                 (13, 12288, (256, 100), 2, False),
                                                 (12, 4096, (512, 96), 6, True),
                                                 (14, 4096, (300, 40), 7, True),
                                                 (13, 2048, (130,), 8, False),
                                                 (14, 2304, (77, 5, 64, 9), 1, False)])
def test_grouped_launch_matches_separate(env, t, k, ns, members, norm):
    # one launch over weights sharing the input equals the per-weight launches bit for bit
    import torch
    print_case(test="group", t=t, k=k, ns=ns, m=members, norm=norm)
    encs = [synth.kquant_numpy(t, k, n, seed=n + i) for i, n in enumerate(ns)]
    ws = [upload(env, t, k, n, e) for n, e in zip(ns, encs)]
    x = synth.activations_numpy(k, members, seed=3)
    gam = synth.gamma_numpy(k, seed=4)
    xd, gd = to_dev(x.reshape(-1)), to_dev(gam)
    outs = [empty_dev(members * n) for n in ns]
    env["k"][t].execute_group(ws, xd, outs, members, gd if norm else None, 1e-6)
    for w, n, o, e in zip(ws, ns, outs, encs):
        single = empty_dev(members * n)
        if norm:
            env["k"][t].execute_rms_norm(w, xd, gd, 1e-6, single, members)
        else:
            env["k"][t].execute_warp_batch(w, xd, single, members)
        got = to_host(o, env["ctx"])
        assert np.array_equal(got.view(np.uint32), to_host(single, env["ctx"]).view(np.uint32))
        for m in range(members):
            src = O.rms_norm_raw(x[m], gam, 1e-6) if norm else x[m]
            ref = O.quant_gemv(t, e, k, n, src, threads=8)
            assert max_rel_err(got.reshape(members, n)[m], ref) <= RTOL


# ------------------------------------------- shapes the decode step runs

def _row_sample(n, count, seed):
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([[0, 1, n // 2, n - 2, n - 1], rng.integers(0, n, count)]))
    return rows[rows < n]


def _oracle_rows(t, enc, k, n, x, rows):
    row_bytes = k // 256 * O.BLOCK_BYTES[t]
    sub = enc.reshape(n, row_bytes)[rows].reshape(-1)
    return O.quant_gemv(t, sub, k, len(rows), x, threads=8)


@pytest.mark.parametrize("t,n,norm", [(14, 151936, True), (12, 32768, True), (13, 32768, False),
                                      (14, 32768, False)])
def test_long_stream_launch_shape(env, t, n, norm):
    """The batch-1 launch shape of long one-slice streams (>= 128 rows per CU):
    the Qwen3-8B lm_head (Q6_K 4096 -> 151936, RMSNorm fused) that every decode
    step runs, and Q4_K / Q5_K / Q6_K at 32768 rows; checked on a row sample."""
    k = 4096
    print_case(test="long_stream", t=t, n=n, norm=norm)
    enc = synth.kquant_numpy(t, k, n, seed=77 + t)
    x = synth.activations_numpy(k, 1, seed=t)[0]
    gam = synth.gamma_numpy(k, seed=5)
    w = upload(env, t, k, n, enc)
    y = empty_dev(n)
    if norm:
        env["k"][t].execute_rms_norm(w, to_dev(x), to_dev(gam), 1e-6, y, 1)
        src = O.rms_norm_raw(x, gam, 1e-6)
    else:
        env["k"][t].execute_warp(w, to_dev(x), y)
        src = x
    got = to_host(y, env["ctx"])
    rows = _row_sample(n, 3000, seed=n)
    ref = _oracle_rows(t, enc, k, n, src, rows)
    err = max_rel_err(got[rows], ref)
    print(f"max_rel_err={err:.3e}", flush=True)
    assert err <= RTOL
    assert np.all(np.isfinite(got))
    del w, y


@pytest.mark.parametrize("mode", ["warp", "fixed16"])
@pytest.mark.parametrize("t,k,n,members,norm", [(12, 4096, 1024, 1, True), (13, 12288, 512, 1, False),
                                                (14, 4096, 512, 1, False), (12, 4096, 512, 3, False),
                                                (12, 4096, 512, 8, True), (13, 4096, 256, 6, False),
                                                (14, 4096, 256, 16, True)])
def test_wide_dynamic_range_activations(env, mode, t, k, n, members, norm):
    """Outlier channels and wide dynamic range inside scale groups and blocks,
    the case where block fixed point drops the small values. GEMV_WARP holds
    f32-level agreement with the oracle (normwise 5e-5); GEMV_FIXED16 (wave
    kernel below 5 members, matrix cores from 5) the 1e-3 bar. (The f32
    paths differ from the oracle only in summation order; Q6_K's (q - 32)
    offset enters as S - 32 X per 16-element group, which cancels more.)"""
    print_case(test="wide_range", mode=mode, t=t, k=k, n=n, m=members, norm=norm)
    E = env["E"]
    kern = env["k"][t]
    enc = synth.kquant_numpy(t, k, n, seed=3 * k + n + t)
    x = np.stack([wide_range_activations(k, seed=m + 10 * t) for m in range(members)])
    gam = synth.gamma_numpy(k, seed=9)
    w = upload(env, t, k, n, enc)
    y = empty_dev(members * n)
    kern.set_mode(E.GEMV_FIXED16 if mode == "fixed16" else E.GEMV_WARP)
    try:
        if norm:
            kern.execute_rms_norm(w, to_dev(x.reshape(-1)), to_dev(gam), 1e-6, y, members)
        else:
            kern.execute_warp_batch(w, to_dev(x.reshape(-1)), y, members)
    finally:
        kern.set_mode(E.GEMV_WARP)
    got = to_host(y, env["ctx"]).reshape(members, n)
    for m in range(members):
        src = O.rms_norm_raw(x[m], gam, 1e-6) if norm else x[m]
        ref = O.quant_gemv(t, enc, k, n, src, threads=8)
        err = max_rel_err(got[m], ref)
        print(f"member {m} max_rel_err={err:.3e}", flush=True)
        assert err <= (5e-5 if mode == "warp" else RTOL), (m, err)


@pytest.mark.parametrize("t,k,members,norm", [(12, 4096, 1, False), (13, 12288, 1, True), (14, 4096, 3, False),
                                            (12, 4096, 8, True)])
def test_nan_activation_propagates(env, t, k, members, norm):
    """GEMV_WARP: one NaN activation makes every output row of its member NaN,
    as the oracle's sequential f32 sum does; the other members stay finite
    and within 1e-3."""
    print_case(test="nan_activation", t=t, k=k, m=members, norm=norm)
    kern = env["k"][t]
    n = 256
    enc = synth.kquant_numpy(t, k, n, seed=11 * k + t)
    x = synth.activations_numpy(k, members, seed=t + members)
    x[0, k // 3] = np.nan
    gam = synth.gamma_numpy(k, seed=4)
    w = upload(env, t, k, n, enc)
    y = empty_dev(members * n)
    if norm:
        kern.execute_rms_norm(w, to_dev(x.reshape(-1)), to_dev(gam), 1e-6, y, members)
    else:
        kern.execute_warp_batch(w, to_dev(x.reshape(-1)), y, members)
    got = to_host(y, env["ctx"]).reshape(members, n)
    for m in range(members):
        src = O.rms_norm_raw(x[m], gam, 1e-6) if norm else x[m]
        ref = O.quant_gemv(t, enc, k, n, src, threads=8)
        if m == 0:
            assert np.isnan(ref).all() and np.isnan(got[m]).all()
        else:
            assert np.isfinite(got[m]).all() and max_rel_err(got[m], ref) <= RTOL, m


@pytest.mark.parametrize("t,k,ns,members,norm", [(12, 4096, (4096, 1024, 1024), 8, True), (12, 4096, (12288,), 8, True),
                                                  (13, 12288, (4096,), 8, True), (13, 12288, (4096,), 8, False),
                                                  (13, 12288, (4096, 100), 5, False), (12, 8192, (700,), 3, False),
                                                  (14, 4096, (151936,), 8, True)])
def test_eight_members_bit_identical_at_qwen3_shapes(env, t, k, ns, members, norm):
    """Up to eight members (the reference's batch cap) at the decode step's
    shapes: every row bit-identical to its single-member call (q/k/v group,
    gate or up, the 12288-wide down projection with and without RMSNorm --
    plain long-K batches split by slice -- the lm_head), and a row sample
    within the bar of the oracle."""
    print_case(test="eight_members", t=t, k=k, ns=ns, m=members, norm=norm)
    encs = [synth.kquant_numpy(t, k, n, seed=n + 3) for n in ns]
    ws = [upload(env, t, k, n, e) for n, e in zip(ns, encs)]
    x = synth.activations_numpy(k, members, seed=11)
    gam = synth.gamma_numpy(k, seed=12)
    xd, gd = to_dev(x.reshape(-1)), to_dev(gam)
    outs = [empty_dev(members * n) for n in ns]
    env["k"][t].execute_group(ws, xd, outs, members, gd if norm else None, 1e-6)
    for w, n, o, e in zip(ws, ns, outs, encs):
        got = to_host(o, env["ctx"]).reshape(members, n)
        rows = _row_sample(n, 400, seed=n)
        for m in (0, members - 1):
            single = empty_dev(n)
            if norm:
                env["k"][t].execute_rms_norm(w, to_dev(x[m]), gd, 1e-6, single, 1)
            else:
                env["k"][t].execute_warp(w, to_dev(x[m]), single)
            assert np.array_equal(to_host(single, env["ctx"]).view(np.uint32), got[m].view(np.uint32)), m
            src = O.rms_norm_raw(x[m], gam, 1e-6) if norm else x[m]
            ref = _oracle_rows(t, e, k, n, src, rows)
            assert max_rel_err(got[m][rows], ref) <= RTOL


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n", [10247, 14341])
def test_eight_member_last_passes_bit_identical(env, t, n):
    """Eight members over 4096-wide rows: the workgroups' 2048 waves (256 CUs)
    take 5-6 (n = 10247) or 7-8 (n = 14341) rows each, so a wave's last pass
    over its ring (4 rows for Q4_K / Q5_K, 3 for Q6_K) reduces 1, 2, 3 or all
    of its rows. Every row of members 0 and 7 bit-identical to the
    single-member call, and a row sample within the bar of the oracle."""
    k, members = 4096, 8
    print_case(test="last_passes", t=t, n=n)
    enc = synth.kquant_numpy(t, k, n, seed=n + t)
    w = upload(env, t, k, n, enc)
    x = synth.activations_numpy(k, members, seed=n)
    y = empty_dev(members * n)
    env["k"][t].execute_warp_batch(w, to_dev(x.reshape(-1)), y, members)
    got = to_host(y, env["ctx"]).reshape(members, n)
    rows = _row_sample(n, 300, seed=t)
    for m in (0, members - 1):
        single = empty_dev(n)
        env["k"][t].execute_warp(w, to_dev(x[m]), single)
        assert np.array_equal(to_host(single, env["ctx"]).view(np.uint32), got[m].view(np.uint32)), m
        assert max_rel_err(got[m][rows], _oracle_rows(t, enc, k, n, x[m], rows)) <= RTOL
    del w, y


@pytest.mark.parametrize("t,k,n,members", [(12, 4096, 4096, 1), (13, 12288, 4096, 2), (14, 4096, 1024, 4),
                                           (12, 2048, 333, 3)])
def test_fixed16_wave_gemv_against_oracle(env, t, k, n, members):
    """The opt-in GEMV_FIXED16 mode on its wave kernel (below the matrix-core
    member counts): within the bar of the oracle, rows bit-identical to the
    single-member call."""
    E = env["E"]
    kern = env["k"][t]
    print_case(test="fixed16_wave", t=t, k=k, n=n, m=members)
    enc = synth.kquant_numpy(t, k, n, seed=k + n)
    x = synth.activations_numpy(k, members, seed=2)
    w = upload(env, t, k, n, enc)
    y = empty_dev(members * n)
    one = empty_dev(n)
    kern.set_mode(E.GEMV_FIXED16)
    try:
        assert kern.mode() == E.GEMV_FIXED16
        kern.execute_warp_batch(w, to_dev(x.reshape(-1)), y, members)
        kern.execute_warp(w, to_dev(x[members - 1]), one)
    finally:
        kern.set_mode(E.GEMV_WARP)
    got = to_host(y, env["ctx"]).reshape(members, n)
    assert np.array_equal(to_host(one, env["ctx"]).view(np.uint32), got[members - 1].view(np.uint32))
    for m in range(members):
        assert max_rel_err(got[m], O.quant_gemv(t, enc, k, n, x[m], threads=8)) <= RTOL


def test_gemv_mode_errors(env):
    E = env["E"]
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        env["k"][12].set_mode(7)
    assert e.value.kind == "InvalidArgument" and e.value.actual == 7
    assert env["k"][12].mode() == E.GEMV_WARP


def _random_gemv_shapes(count, seed):
    import random
    rng = random.Random(seed)
    shapes = []
    for _ in range(count):
        t = rng.choice(TYPES)
        k = 256 * rng.choice((1, 2, 3, 5, 8, 12, 16, 17, 24, 48, 64))
        n = rng.choice((1, 7, 64, 75, 300, 1000, 2050, 4096, 6000, 12288, 32768))
        members = rng.choice((1, 2, 3, 4, 5, 6, 7, 8, 9, 13, 16, 24, 33, 64))
        shapes.append((t, k, n, members))
    return shapes


@pytest.mark.parametrize("i,t,k,n,members", [(i, *s) for i, s in enumerate(_random_gemv_shapes(24, 11))])
def test_random_shapes_batch_matches_oracle_and_single_bitwise(env, i, t, k, n, members):
    """Seeded random (type, K, N, members) through the default f32 GEMV: the
    batch within 1e-3 of the oracle on sampled members; up to 8 members every
    sampled member's row bit-identical to its single-member launch
    (cuda_reference.rs:5322-5334), from 9 (the matrix-core f32 path) within
    5e-5 of the oracle."""
    print_case(test="random gemv", i=i, t=t, k=k, n=n, members=members)
    enc = synth.kquant_numpy(t, k, n, seed=300 + i)
    x = synth.activations_numpy(k, members, seed=400 + i)
    w = upload(env, t, k, n, enc)
    y = empty_dev(members * n)
    env["k"][t].execute_warp_batch(w, to_dev(x.reshape(-1)), y, members)
    got = to_host(y, env["ctx"]).reshape(members, n)
    assert np.all(np.isfinite(got))
    sample = sorted({0, members // 2, members - 1})
    ref = np.stack([O.quant_gemv(t, enc, k, n, x[m], threads=16) for m in sample])
    assert max_rel_err(got[sample], ref) <= RTOL
    if members > F32_BITWISE_MEMBERS:
        assert max_rel_err(got[sample], ref) <= F32_RTOL
        return
    for m in sample:
        ys = empty_dev(n)
        env["k"][t].execute_warp(w, to_dev(x[m]), ys)
        assert np.array_equal(to_host(ys, env["ctx"]).view(np.uint32), got[m].view(np.uint32))


@pytest.mark.parametrize("mode", ("warp", "fixed16"))
@pytest.mark.parametrize("i,t,k,n,members", [(i, *s) for i, s in enumerate(_random_gemv_shapes(12, 23))])
def test_random_shapes_fused_rms_norm(env, mode, i, t, k, n, members):
    """Seeded random shapes through the RMSNorm-fused GEMV in the default f32
    mode and the opt-in fixed-point mode: sampled members within 1e-3 of the
    oracle's RMSNorm followed by its GEMV."""
    E = env["E"]
    kern = env["k"][t]
    print_case(test="random fused", mode=mode, i=i, t=t, k=k, n=n, members=members)
    enc = synth.kquant_numpy(t, k, n, seed=500 + i)
    x = synth.activations_numpy(k, members, seed=600 + i) * 2.0
    gam = synth.gamma_numpy(k, seed=700 + i)
    w = upload(env, t, k, n, enc)
    y = empty_dev(members * n)
    kern.set_mode(E.GEMV_FIXED16 if mode == "fixed16" else E.GEMV_WARP)
    try:
        kern.execute_rms_norm(w, to_dev(x.reshape(-1)), to_dev(gam), 1e-6, y, members)
    finally:
        kern.set_mode(E.GEMV_WARP)
    got = to_host(y, env["ctx"]).reshape(members, n)
    assert np.all(np.isfinite(got))
    for m in sorted({0, members // 2, members - 1}):
        normed = O.rms_norm_raw(x[m], gam, 1e-6)
        assert max_rel_err(got[m], O.quant_gemv(t, enc, k, n, normed, threads=16)) <= RTOL

"""GPU parity tests of the f32-faithful batched GEMV on the bf16 matrix cores
(engine_amd/csrc/gemv_f32mma.hip): the default GEMV_WARP arithmetic for 9..64
members, called through the C ABI.

Activations are split exactly into three bf16 pieces and the quants are exact
in bf16, so the products are exact and only the f32 accumulation rounds; the
bar is therefore the f32 wave GEMV's own: normwise max relative error
<= 5e-5 (gpu_helpers.F32_RTOL) against the oracle's sequential f32 GEMV
(crates/nvidia/src/qwen_reference.rs:31-40 over lib.rs:596-661 dequantised
weights), on N(0,1) and on wide-dynamic-range activations. A member's output
depends only on its own activations, so its bits do not change with the batch
it runs in (from 9 members on). Below 9 members the wave GEMV's bit identity
with the single call holds (tests/test_gpu_kquant.py).
"""
import numpy as np
import pytest

from engine_amd import synth
from oracle import kquant_oracle as O

from .gpu_helpers import F32_RTOL, empty_dev, max_rel_err, to_dev, to_host, wide_range_activations

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    import engine_amd as E
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    ctx = E.AmdContext(0)
    store = E.AmdWeightStore(ctx)
    kernels = {t: E.QwenGemvKernel.from_value_type(ctx, t) for t in (12, 13, 14)}
    return {"E": E, "ctx": ctx, "store": store, "k": kernels, "n": [0]}


def upload(env, t, k, n, enc):
    env["n"][0] += 1
    name = f"f{env['n'][0]}"
    env["store"].materialize_quantized(name, [k, n], t, enc)
    return env["store"].quantized_tensor(name)


def case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def oracle_rows(t, enc, k, n, x):
    """The oracle's GEMV of every member (row of x), 16 host threads each."""
    return np.stack([O.quant_gemv(t, enc, k, n, row, threads=16) for row in x])


def batch(env, t, w, x, n, members):
    y = empty_dev(members * n)
    env["k"][t].execute_warp_batch(w, to_dev(x.reshape(-1)), y, members)
    return to_host(y, env["ctx"]).reshape(members, n)


@pytest.mark.parametrize("members", [9, 16, 17, 33, 64])
@pytest.mark.parametrize("t,k,n", [(12, 4096, 1000), (13, 12288, 300), (14, 4096, 1000), (12, 256, 75),
                                   (14, 12288, 64), (13, 1280, 2050)])
def test_batch_matches_oracle(env, t, k, n, members):
    """Every member's row against the oracle, N(0,1) activations; N not a
    multiple of 16 (ragged last tile), K from one super-block to 48."""
    case(test="f32mma oracle", t=t, k=k, n=n, members=members)
    enc = synth.kquant_numpy(t, k, n, seed=7 * members + t)
    x = synth.activations_numpy(k, members, seed=members + k)
    w = upload(env, t, k, n, enc)
    got = batch(env, t, w, x, n, members)
    assert np.all(np.isfinite(got))
    ref = oracle_rows(t, enc, k, n, x.reshape(members, k))
    for m in range(members):
        assert max_rel_err(got[m], ref[m]) <= F32_RTOL, m


@pytest.mark.parametrize("members", [16, 64])
@pytest.mark.parametrize("t,k,n", [(12, 4096, 512), (13, 12288, 256), (14, 4096, 512)])
def test_wide_dynamic_range(env, t, k, n, members):
    """Activations with x3000 outlier channels, groups at 2^-20 and groups
    spread over 2^-16..1: the split into bf16 pieces keeps every bit, so the
    f32 bar holds as for the wave GEMV."""
    case(test="f32mma wide", t=t, k=k, n=n, members=members)
    enc = synth.kquant_numpy(t, k, n, seed=91 + t)
    x = np.stack([wide_range_activations(k, seed=1000 + m) for m in range(members)])
    w = upload(env, t, k, n, enc)
    got = batch(env, t, w, x, n, members)
    ref = oracle_rows(t, enc, k, n, x)
    for m in range(members):
        assert max_rel_err(got[m], ref[m]) <= F32_RTOL, m


@pytest.mark.parametrize("t", [12, 13, 14])
def test_member_bits_independent_of_batch(env, t):
    """A member's row is the same bits at 64, 16 and 9 members and at any
    position in the batch (the MFMA C rows are independent dot products)."""
    k, n = (12288 if t == 13 else 4096), 384
    case(test="f32mma batch invariance", t=t, k=k, n=n)
    enc = synth.kquant_numpy(t, k, n, seed=33 + t)
    x = synth.activations_numpy(k, 64, seed=5).reshape(64, k)
    w = upload(env, t, k, n, enc)
    full = batch(env, t, w, x, n, 64)
    first16 = batch(env, t, w, x[:16], n, 16)
    assert np.array_equal(first16.view(np.uint32), full[:16].view(np.uint32))
    mid9 = batch(env, t, w, x[37:46], n, 9)  # members 37..45 moved to tile 0
    assert np.array_equal(mid9.view(np.uint32), full[37:46].view(np.uint32))


@pytest.mark.parametrize("t,k,n", [(12, 4096, 12288), (13, 12288, 4096), (12, 4096, 4096), (13, 12288, 4000)])
def test_member_bits_independent_of_batch_ffn_shapes(env, t, k, n):
    """The same at the Qwen3-8B FFN and o shapes (and a ragged row count),
    where launches of 16 and 64 members differ in member tiles per launch and
    waves per workgroup: the K split follows the weight shape alone, so a
    member's sums are added in the same order (a split that followed the
    member count would change the last bits here)."""
    case(test="f32mma batch invariance ffn", t=t, k=k, n=n)
    enc = synth.kquant_numpy(t, k, n, seed=60 + t)
    x = synth.activations_numpy(k, 64, seed=61).reshape(64, k)
    w = upload(env, t, k, n, enc)
    full = batch(env, t, w, x, n, 64)
    assert np.all(np.isfinite(full))
    for lo, hi in ((0, 16), (40, 49), (48, 64)):
        part = batch(env, t, w, x[lo:hi], n, hi - lo)
        assert np.array_equal(part.view(np.uint32), full[lo:hi].view(np.uint32)), (lo, hi)


def test_fused_rms_norm(env):
    """RMSNorm fused into the pack stage (x * gamma packed, 1/rms applied per
    member at the output) against the oracle's RMSNorm then GEMV."""
    t, k, n, members = 12, 4096, 1024, 24
    case(test="f32mma rmsnorm", t=t, k=k, n=n, members=members)
    enc = synth.kquant_numpy(t, k, n, seed=3)
    x = synth.activations_numpy(k, members, seed=4).reshape(members, k) * 3.0
    gam = synth.gamma_numpy(k, seed=5)
    w = upload(env, t, k, n, enc)
    y = empty_dev(members * n)
    env["k"][t].execute_rms_norm(w, to_dev(x.reshape(-1)), to_dev(gam), 1e-6, y, members)
    got = to_host(y, env["ctx"]).reshape(members, n)
    for m in range(members):
        ref = O.quant_gemv(t, enc, k, n, O.rms_norm_raw(x[m], gam, 1e-6), threads=16)
        assert max_rel_err(got[m], ref) <= F32_RTOL, m


def test_group_and_gate_up_pair(env):
    """q/k/v as one grouped launch equal to three separate calls bit for bit
    (a row's arithmetic does not depend on its neighbours); the gate/up pair
    equals silu(gate) * up of the separate calls."""
    t, k, members = 12, 4096, 12
    case(test="f32mma group pair", t=t, k=k, members=members)
    x = synth.activations_numpy(k, members, seed=8)
    xd = to_dev(x.reshape(-1))
    ws = [upload(env, t, k, n, synth.kquant_numpy(t, k, n, seed=20 + i)) for i, n in enumerate((1024, 256, 256))]
    outs = [empty_dev(members * n) for n in (1024, 256, 256)]
    env["k"][t].execute_group(ws, xd, outs, members)
    for w, o, n in zip(ws, outs, (1024, 256, 256)):
        single = empty_dev(members * n)
        env["k"][t].execute_warp_batch(w, xd, single, members)
        assert np.array_equal(to_host(o, env["ctx"]).view(np.uint32), to_host(single, env["ctx"]).view(np.uint32))
    ffn = 2048
    gate = upload(env, t, k, ffn, synth.kquant_numpy(t, k, ffn, seed=30))
    up = upload(env, t, k, ffn, synth.kquant_numpy(t, k, ffn, seed=31))
    act = empty_dev(members * ffn)
    env["k"][t].execute_gate_up_swiglu(gate, up, xd, act, members)
    g, u = empty_dev(members * ffn), empty_dev(members * ffn)
    env["k"][t].execute_warp_batch(gate, xd, g, members)
    env["k"][t].execute_warp_batch(up, xd, u, members)
    gh, uh = to_host(g, env["ctx"]), to_host(u, env["ctx"])
    want = (gh / (np.float32(1) + np.exp(-gh))) * uh
    assert max_rel_err(to_host(act, env["ctx"]), want) <= 1e-6


def test_swiglu_prologue_and_accumulate(env):
    """The down projection's form: silu(gate) * up packed from two inputs,
    the product added into the output (residual)."""
    t, k, n, members = 13, 4608, 1024, 10
    case(test="f32mma swiglu accumulate", t=t, k=k, n=n, members=members)
    enc = synth.kquant_numpy(t, k, n, seed=12)
    g = synth.activations_numpy(k, members, seed=13).reshape(members, k)
    u = synth.activations_numpy(k, members, seed=14).reshape(members, k)
    base = synth.activations_numpy(n, members, seed=15).reshape(members, n)
    w = upload(env, t, k, n, enc)
    y = to_dev(base.reshape(-1))
    env["k"][t].execute_fused(w, to_dev(g.reshape(-1)), y, members, up=to_dev(u.reshape(-1)), accumulate=True)
    got = to_host(y, env["ctx"]).reshape(members, n)
    for m in range(members):
        a = (g[m] / (np.float32(1) + np.exp(-g[m]))) * u[m]
        ref = base[m].astype(np.float64) + O.quant_gemv(t, enc, k, n, a.astype(np.float32), threads=16)
        assert max_rel_err(got[m], ref) <= F32_RTOL, m


def test_nan_activation_stays_in_its_member(env):
    """A NaN in one member's activations makes that member's outputs NaN (as
    the oracle's sequential sum does) and leaves the others finite."""
    t, k, n, members = 12, 4096, 256, 20
    case(test="f32mma nan", t=t, k=k, n=n, members=members)
    enc = synth.kquant_numpy(t, k, n, seed=40)
    x = synth.activations_numpy(k, members, seed=41).reshape(members, k)
    x[5, 1234] = np.nan
    w = upload(env, t, k, n, enc)
    got = batch(env, t, w, x, n, members)
    assert np.all(np.isnan(got[5]))
    others = np.delete(got, 5, axis=0)
    assert np.all(np.isfinite(others))


@pytest.mark.parametrize("members", [4, 16, 64])
def test_config2_ffn_shapes(env, members):
    """BASELINE config 2 at its exact shapes and batch sizes: the Qwen3-8B FFN
    (gate/up Q4_K 4096 -> 12288 as one grouped launch, down Q5_K 12288 ->
    4096) with f32 activations ~N(0,1). M = 4 runs the f32 wave GEMV (rows
    bit-identical to the single call), M = 16 and 64 the matrix-core f32
    path; sampled members against the oracle at the f32 bar."""
    import torch
    case(test="config2 ffn", members=members)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(2000 + members)
    dev = torch.device("cuda:0")
    shapes = {"gate": (12, 4096, 12288), "up": (12, 4096, 12288), "down": (13, 12288, 4096)}
    enc = {nm: synth.kquant_torch(t, k, n, gen, dev) for nm, (t, k, n) in shapes.items()}
    w = {nm: upload(env, t, k, n, enc[nm]) for nm, (t, k, n) in shapes.items()}
    x = synth.activations_numpy(4096, members, seed=members).reshape(members, 4096)
    h = synth.activations_numpy(12288, members, seed=members + 1).reshape(members, 12288)
    g, u, d = empty_dev(members * 12288), empty_dev(members * 12288), empty_dev(members * 4096)
    env["k"][12].execute_group([w["gate"], w["up"]], to_dev(x.reshape(-1)), [g, u], members)
    env["k"][13].execute_warp_batch(w["down"], to_dev(h.reshape(-1)), d, members)
    got = {"gate": to_host(g, env["ctx"]).reshape(members, -1), "up": to_host(u, env["ctx"]).reshape(members, -1),
           "down": to_host(d, env["ctx"]).reshape(members, -1)}
    sample = sorted({0, members // 2, members - 1})
    for nm, (t, k, n) in shapes.items():
        e = enc[nm].cpu().numpy()
        src = h if nm == "down" else x
        assert np.all(np.isfinite(got[nm]))
        for m in sample:
            assert max_rel_err(got[nm][m], O.quant_gemv(t, e, k, n, src[m], threads=16)) <= F32_RTOL, (nm, m)

"""GPU tests of the prefill matmul (bf16 MFMA-class path),
called through the C ABI.

Bar (north star): outputs within max relative error 1e-3 (normwise,
gpu_helpers.RTOL) of the f32-accumulated oracle on the same inputs. bf16
inputs are generated as bf16 values and handed to the oracle as the same
values in f32, so the comparison isolates the kernel's own rounding.
"""
import random

import numpy as np
import pytest

from engine_amd import synth
from oracle import kquant_oracle as O

from .gpu_helpers import (F32_BITWISE_MEMBERS, F32_RTOL, RTOL, empty_dev, max_rel_err, to_dev, to_host,
                          wide_range_activations)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    import engine_amd as E
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    ctx = E.AmdContext(0)
    ctx.reserve_prefill(512, 12288, 12288)
    store = E.AmdWeightStore(ctx)
    kernels = {t: E.QwenGemvKernel.from_value_type(ctx, t) for t in (12, 13, 14)}
    return {"E": E, "ctx": ctx, "store": store, "k": kernels, "n": [0]}


def upload(env, t, k, n, enc):
    env["n"][0] += 1
    name = f"p{env['n'][0]}"
    env["store"].materialize_quantized(name, [k, n], t, enc)
    return env["store"].quantized_tensor(name)


def bf16_values(x):
    """Round f32 to bf16 (RNE) and return both the device bf16 tensor and the exact f32 values."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16)
    return t.to("cuda:0"), t.to(torch.float32).numpy()


def oracle_rows(t, enc, k, n, x, threads=1):
    return np.stack([O.quant_gemv(t, enc, k, n, x[m], threads=threads) for m in range(x.shape[0])])


@pytest.mark.parametrize("t", (12, 13, 14))
@pytest.mark.parametrize("k,n,m", [(256, 32, 1), (512, 96, 40), (1024, 200, 130), (2304, 128, 257), (1024, 75, 40)])
@pytest.mark.parametrize("dtype", ("f32", "bf16"))
def test_prefill_against_oracle(env, t, k, n, m, dtype):
    print("CASE prefill", t, k, n, m, dtype, flush=True)
    enc = synth.kquant_numpy(t, k, n, seed=k + n + t)
    w = upload(env, t, k, n, enc)
    x = synth.activations_numpy(k, m, seed=m + 3)
    if dtype == "bf16":
        xd, x = bf16_values(x)
    else:
        xd = to_dev(x)
    y = empty_dev(m * n)
    env["k"][t].gemm_prefill(w, xd, y, m)
    got = to_host(y, env["ctx"]).reshape(m, n)
    ref = oracle_rows(t, enc, k, n, x)
    assert max_rel_err(got, ref) <= RTOL


@pytest.mark.parametrize("t", (12, 14))
def test_prefill_fused_rms_norm(env, t):
    k, n, m = 1024, 160, 48
    print("CASE prefill rmsnorm", t, flush=True)
    enc = synth.kquant_numpy(t, k, n, seed=77 + t)
    w = upload(env, t, k, n, enc)
    x = synth.activations_numpy(k, m, seed=5) * 3.0
    gamma = synth.gamma_numpy(k, seed=6)
    y = empty_dev(m * n)
    env["k"][t].gemm_prefill(w, to_dev(x), y, m, gamma=to_dev(gamma), epsilon=1e-6)
    got = to_host(y, env["ctx"]).reshape(m, n)
    normed = np.stack([O.rms_norm_raw(x[i], gamma, 1e-6) for i in range(m)])
    ref = oracle_rows(t, enc, k, n, normed)
    assert max_rel_err(got, ref) <= RTOL


@pytest.mark.parametrize("t,k,n", [(12, 4096, 12288), (14, 12288, 4096)])
def test_prefill_config3_full_size(env, t, k, n):
    # M = 512 bf16 tokens; the oracle checks a token sample
    import torch
    m = 512
    print("CASE prefill config3", t, k, n, flush=True)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(31 + t)
    enc_dev = synth.kquant_torch(t, k, n, gen, torch.device("cuda:0"))
    w = upload(env, t, k, n, enc_dev)
    x = synth.activations_numpy(k, m, seed=9)
    xd, x = bf16_values(x)
    y = empty_dev(m * n)
    env["k"][t].gemm_prefill(w, xd, y, m)
    got = to_host(y, env["ctx"]).reshape(m, n)
    enc = enc_dev.cpu().numpy()
    sample = [0, 1, 127, 128, 255, 300, 511]
    ref = np.stack([O.quant_gemv(t, enc, k, n, x[i], threads=16) for i in sample])
    assert max_rel_err(got[sample], ref) <= RTOL
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("t,k,n,m,dtype", [
    (12, 1024, 11000, 450, "bf16"),   # last row tile 56 of 192 rows, last token tile 66 of 128
    (13, 768, 12288, 512, "f32"),     # three super-blocks: one pair of steps and the odd one
    (14, 256, 11520, 400, "bf16"),    # one super-block (the odd step alone), 2-byte aligned rows
    (14, 2048, 12288, 500, "f32"),
    (12, 4096, 12288, 128, "bf16"),   # 64 x 1 tiles of 128 tokens, K split in 4 (partials reduced in order)
    (14, 4096, 12288, 48, "f32"),     # 64 x 1 tiles of 64 tokens, K split in 4, last token tile 48 of 64
    (14, 4096, 4096, 100, "bf16"),    # 32-row waves: 32 x 2 tiles of 64 tokens, K split in 4
    (13, 12288, 4096, 64, "f32"),     # 32 x 1 tiles of 64 tokens, K split in 8
    (14, 12288, 4096, 384, "bf16"),   # Q6_K 256-row tiles: 16 x 3, K split in 5 (10, 10, 10, 10, 8 blocks)
    (14, 6144, 4000, 200, "f32"),     # Q6_K 256-row tiles: 16 x 2, K split in 8 (3 blocks each), last row tile 160 of 256
    (12, 4096, 12288, 256, "bf16"),   # 64 x 2 tiles, K split in 2 (one round)
    (12, 4096, 12288, 384, "f32"),    # 64 x 3 tiles, no split (three quarters of the CUs)
    (13, 12288, 4096, 256, "bf16"),   # Q5_K 256-row tiles: 16 x 2, K split in 8
    (13, 12288, 4096, 640, "f32"),    # Q5_K 256-row tiles: 16 x 5, K split in 3 (one round, 94%)
    (13, 4096, 4000, 300, "bf16"),    # Q5_K 256-row tiles: 16 x 3, K split in 5; last row tile 160, last token tile 44
    (12, 2048, 6000, 160, "f32"),     # 32 x 2 tiles, K split in 4; last row tile 48 of 192, last token tile 32 of 128
    (12, 4096, 12288, 768, "bf16"),   # 64 x 6 tiles, no split: two rounds, the second three quarters full
    (14, 12288, 4096, 768, "f32"),    # Q6_K 256-row tiles: 16 x 6, K split in 2
    (14, 12288, 4094, 384, "bf16"),   # as (14, 12288, 4096, 384) with N not a multiple of 4: one-wide split reduce
    (12, 4096, 12288, 129, "f32"),    # 64 x 2 tiles, K split in 2; the last token tile holds one token
    (12, 4096, 12288, 640, "bf16"),   # 320 tiles: two rounds, the second a quarter full, and no split fits: the 32x32 kernel
    (12, 4096, 12288, 2047, "f32"),   # many tokens: 256-row tiles, 48 x 16 (three whole rounds), last token tile 127
    (12, 4096, 4096, 2000, "bf16"),   # many tokens: 256-row tiles, 16 x 16, last token tile 80 of 128
    (13, 12288, 4096, 2047, "f32"),   # many tokens: Q5_K 256-row tiles without a split
])
def test_prefill_wide_tiles(env, t, k, n, m, dtype):
    """Shapes whose wide-tile grid fills a 256-CU MI355X (the wide-tile
    matmul with packed-f16 dequantisation, with K split for 32 < M <= 128):
    rows of a token sample against the oracle, every output finite."""
    import torch
    print("CASE prefill wide", t, k, n, m, dtype, flush=True)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(k + n + t)
    enc_dev = synth.kquant_torch(t, k, n, gen, torch.device("cuda:0"))
    w = upload(env, t, k, n, enc_dev)
    x = synth.activations_numpy(k, m, seed=m + 11)
    if dtype == "bf16":
        xd, x = bf16_values(x)
    else:
        xd = to_dev(x)
    y = empty_dev(m * n)
    env["k"][t].gemm_prefill(w, xd, y, m)
    got = to_host(y, env["ctx"]).reshape(m, n)
    enc = enc_dev.cpu().numpy()
    sample = sorted(i for i in {0, 1, 15, 16, 127, 128, m // 2, m - 1} if i < m)
    ref = np.stack([O.quant_gemv(t, enc, k, n, x[i], threads=16) for i in sample])
    assert max_rel_err(got[sample], ref) <= RTOL
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("t,k,n,m,dtype,norm", [
    (12, 4096, 1024, 40, "f32", False),     # 32x32 kernel, 2 token blocks
    (13, 4096, 12288, 128, "bf16", False),  # wide tiles, K split
    (14, 4096, 512, 200, "f32", True),      # 32x32 kernel, 4 token blocks x 8 waves
    (12, 4096, 12288, 256, "bf16", True),   # wide tiles, one round
    (14, 12288, 4096, 256, "f32", True),    # Q6_K 256-row tiles, K split in 8
])
def test_prefill_wide_dynamic_range(env, t, k, n, m, dtype, norm):
    """Outlier channels (x3000), whole scale groups at 2^-20 and groups spread
    over 2^-16..1: the per-token power-of-two scale maps each token's maximum
    just below 2^15 before the f16 conversion, so small values keep their
    relative precision down to f16's subnormal step (2^-24 of 2^15). Token
    sample against the oracle at the 1e-3 bar, every output finite."""
    import torch
    print("CASE prefill wide range", t, k, n, m, dtype, norm, flush=True)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(7 * k + n + t)
    enc_dev = synth.kquant_torch(t, k, n, gen, torch.device("cuda:0"))
    w = upload(env, t, k, n, enc_dev)
    x = np.stack([wide_range_activations(k, seed=1000 + i) for i in range(m)])
    if dtype == "bf16":
        xd, x = bf16_values(x)
    else:
        xd = to_dev(x)
    gamma = synth.gamma_numpy(k, seed=17) if norm else None
    y = empty_dev(m * n)
    env["k"][t].gemm_prefill(w, xd, y, m, gamma=to_dev(gamma) if norm else None, epsilon=1e-6)
    got = to_host(y, env["ctx"]).reshape(m, n)
    enc = enc_dev.cpu().numpy()
    for i in sorted({0, 1, 31, m // 2, m - 1}):
        src = O.rms_norm_raw(x[i], gamma, 1e-6) if norm else x[i]
        ref = O.quant_gemv(t, enc, k, n, src, threads=16)
        err = max_rel_err(got[i], ref)
        print(f"token {i} max_rel_err={err:.3e}", flush=True)
        assert err <= RTOL, (i, err)
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("t,k,n", [(12, 4096, 12288), (13, 12288, 4096)])
def test_batched_ffn_m64_full_size(env, t, k, n):
    """BASELINE config 2 at M = 64 on the Qwen3-8B FFN shapes (gate/up Q4_K
    4096 -> 12288, down Q5_K 12288 -> 4096, f32 activations, RMSNorm fused on
    gate/up): the f16 matrix-core matmul and the batched GEMV (GEMV_WARP,
    which runs 64 members on the f32-faithful matrix-core GEMV) against the
    oracle on a token sample, and batched rows within F32_RTOL of
    single-member calls (bit-identical only up to F32_BITWISE_MEMBERS)."""
    m = 64
    print("CASE batched m64", t, k, n, flush=True)
    enc = synth.kquant_numpy(t, k, n, seed=640 + t)
    w = upload(env, t, k, n, enc)
    x = synth.activations_numpy(k, m, seed=64)
    gamma = synth.gamma_numpy(k, seed=65) if t == 12 else None
    xd = to_dev(x)
    y = empty_dev(m * n)
    env["k"][t].gemm_prefill(w, xd, y, m, gamma=to_dev(gamma) if gamma is not None else None, epsilon=1e-6)
    got = to_host(y, env["ctx"]).reshape(m, n)
    yb = empty_dev(m * n)
    if gamma is not None:
        env["k"][t].execute_rms_norm(w, xd, to_dev(gamma), 1e-6, yb, m)
    else:
        env["k"][t].execute_warp_batch(w, xd, yb, m)
    batched = to_host(yb, env["ctx"]).reshape(m, n)
    sample = [0, 1, 7, 8, 31, 40, 63]
    for i in sample:
        src = O.rms_norm_raw(x[i], gamma, 1e-6) if gamma is not None else x[i]
        ref = O.quant_gemv(t, enc, k, n, src, threads=16)
        assert max_rel_err(got[i], ref) <= RTOL, ("matmul", i)
        assert max_rel_err(batched[i], ref) <= RTOL, ("batched", i)
    for i in (0, 63):
        one = empty_dev(n)
        if gamma is not None:
            env["k"][t].execute_rms_norm(w, to_dev(x[i]), to_dev(gamma), 1e-6, one, 1)
        else:
            env["k"][t].execute_warp(w, to_dev(x[i]), one)
        assert m > F32_BITWISE_MEMBERS
        assert max_rel_err(batched[i], to_host(one, env["ctx"])) <= F32_RTOL, i


def test_prefill_matches_wave_gemv_rows(env):
    # the two paths agree on the same tokens (both within tolerance of f32)
    k, n, m = 4096, 512, 8
    print("CASE prefill vs wave", flush=True)
    enc = synth.kquant_numpy(12, k, n, seed=123)
    w = upload(env, 12, k, n, enc)
    x = synth.activations_numpy(k, m, seed=124)
    y1 = empty_dev(m * n)
    env["k"][12].gemm_prefill(w, to_dev(x), y1, m)
    y2 = empty_dev(m * n)
    env["k"][12].execute_warp_batch(w, to_dev(x), y2, m)
    a = to_host(y1, env["ctx"])
    b = to_host(y2, env["ctx"])
    assert max_rel_err(a, b) <= 2 * RTOL


def test_prefill_validation(env):
    E = env["E"]
    k, n = 512, 64
    enc = synth.kquant_numpy(12, k, n, seed=1)
    w = upload(env, 12, k, n, enc)
    kern = env["k"][12]
    x = to_dev(synth.activations_numpy(k, 4, seed=2))
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        kern.gemm_prefill(w, x, empty_dev(4 * n + 1), 4)
    assert e.value.kind == "OutputLength" and (e.value.expected, e.value.actual) == (4 * n, 4 * n + 1)
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        kern.gemm_prefill(w, x, empty_dev(4 * n), 4, gamma=to_dev(np.ones(k - 256, np.float32)))
    assert e.value.kind == "WeightLength" and (e.value.expected, e.value.actual) == (k, k - 256)
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        kern.gemm_prefill(w, x, empty_dev(4 * n), 4, gamma=to_dev(np.ones(k, np.float32)), epsilon=0.0)
    assert e.value.kind == "InvalidEpsilon"
    # a context without a reserved workspace reports the bytes it needs
    ctx2 = E.AmdContext(0)
    kern2 = E.QwenGemvKernel.from_value_type(ctx2, 12)
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        kern2.gemm_prefill(w, x, empty_dev(4 * n), 4)
    assert e.value.kind == "WorkspaceTooSmall" and e.value.actual == 0
    assert e.value.expected == E._lib.load().ribn_amd_gemm_workspace_bytes(4, k, 0)


def _random_prefill_shapes(count, seed):
    rng = random.Random(seed)
    shapes = []
    while len(shapes) < count:
        t = rng.choice((12, 13, 14))
        k = rng.choice((256, 1024, 2048, 4096, 6144, 12288))
        n = rng.choice((75, 1000, 2050, 4096, 6000, 11000, 12288))
        m = rng.choice((33, 48, 64, 100, 128, 129, 160, 200, 256, 300, 384, 511, 512))
        shapes.append((t, k, n, m))
    return shapes


@pytest.mark.parametrize("i,t,k,n,m", [(i, *s) for i, s in enumerate(_random_prefill_shapes(24, 7))])
def test_prefill_random_shapes(env, i, t, k, n, m):
    """Seeded random shapes across every route (32x32 kernel, small-M tiles,
    wide tiles with and without split K, ragged row and token tiles, N not a
    multiple of 4): sampled rows against the oracle (the first and last token
    and one seeded token inside every 128-token tile), every output finite."""
    import torch
    print("CASE prefill random", i, t, k, n, m, flush=True)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(1000 + i)
    enc_dev = synth.kquant_torch(t, k, n, gen, torch.device("cuda:0"))
    w = upload(env, t, k, n, enc_dev)
    xd, x = bf16_values(synth.activations_numpy(k, m, seed=2000 + i))
    y = empty_dev(m * n)
    env["k"][t].gemm_prefill(w, xd, y, m)
    got = to_host(y, env["ctx"]).reshape(m, n)
    enc = enc_dev.cpu().numpy()
    rng = random.Random(3000 + i)
    sample = sorted({0, m - 1} | {t0 + rng.randrange(min(128, m - t0)) for t0 in range(0, m, 128)})
    ref = np.stack([O.quant_gemv(t, enc, k, n, x[r], threads=16) for r in sample])
    assert max_rel_err(got[sample], ref) <= RTOL
    assert np.all(np.isfinite(got))

"""GPU parity tests of the batched matrix-core GEMV (engine_amd/csrc/gemv_mfma.hip),
which, in the opt-in GEMV_FIXED16 mode, serves Q4_K / Q5_K / Q6_K batches of 5..16 members (4..16 when K spans more
than one 4096 slice) through the same C-ABI entry points as the wave GEMV
(execute_warp_batch, execute_rms_norm, execute_group, execute_fused,
execute_gate_up_swiglu). Every case asserts that it takes that path. Up to 8
members use the packed digit-plane layout (high digits in rows 0-7, low
digits in rows 8-15 of one fragment); 9..16 the two-plane layout.

Bars: every member's rows within max relative error 1e-3 (normwise,
gpu_helpers.RTOL) of the f32-accumulated oracle; within a layout, a member's
output bits do not depend on the other members of the batch (checked by
permuting and sub-setting batches); the residual form equals store-then-add
bit for bit.
"""
import numpy as np
import pytest

from engine_amd import synth
from oracle import kquant_oracle as O

from .gpu_helpers import RTOL, empty_dev, max_rel_err, mfma_path, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    import engine_amd as E
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    ctx = E.AmdContext(0)
    store = E.AmdWeightStore(ctx)
    kernels = {t: E.QwenGemvKernel.from_value_type(ctx, t) for t in (12, 13, 14)}
    for kern in kernels.values():
        kern.set_mode(E.GEMV_FIXED16)  # the matrix cores serve the opt-in fixed-point mode
    return {"E": E, "ctx": ctx, "store": store, "k": kernels, "n": [0]}


def upload(env, t, k, n, enc):
    env["n"][0] += 1
    name = f"mfma{env['n'][0]}"
    env["store"].materialize_quantized(name, [k, n], t, enc)
    return env["store"].quantized_tensor(name)


def print_case(**kw):
    print("case", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def oracle_rows(t, enc, k, n, x, gamma=None):
    rows = []
    for xm in x:
        src = O.rms_norm_raw(xm, gamma, 1e-6) if gamma is not None else xm
        rows.append(O.quant_gemv(t, enc, k, n, src, threads=8))
    return np.stack(rows)


@pytest.mark.parametrize("t,k,n,members,norm", [
    (12, 256, 16, 9, False),       # one super-block, one tile
    (12, 1024, 33, 10, True),      # partial tile (rows 32..32 live)
    (12, 4096, 1024, 12, True),
    (12, 4096, 4096, 16, False),   # a full member tile
    (13, 12288, 4096, 8, False),   # down projection at batch 8 (48 blocks, 4-way K split, packed digits)
    (13, 12288, 300, 6, True),
    (13, 12288, 4096, 4, False),   # four members, long K
    (12, 4096, 6144, 5, True),     # q/k/v-sized at five members
    (12, 4096, 4096, 8, True),     # batch 8, packed digits
    (12, 256, 16, 7, False),       # one super-block, packed digits
    (14, 4096, 1024, 8, True),     # Q6_K lm_head-shaped at batch 8, packed digits
    (14, 4096, 300, 12, False),    # Q6_K, two planes, partial last tile
    (14, 256, 16, 5, True),        # Q6_K, one super-block
    (13, 2048, 100, 13, True),
    (12, 16384, 48, 7, False),     # the largest K
    (12, 4096, 12288, 9, True),    # four-tile row groups (>= 2048 tiles)
])
def test_batched_matches_oracle(env, t, k, n, members, norm):
    print_case(test="mfma_batch", t=t, k=k, n=n, members=members, norm=norm)
    assert mfma_path(t, k, members)
    enc = synth.kquant_numpy(t, k, n, seed=k + n + members)
    w = upload(env, t, k, n, enc)
    x = synth.activations_numpy(k, members, seed=members + 7)
    gamma = synth.gamma_numpy(k, seed=11) if norm else None
    y = empty_dev(members * n)
    if norm:
        env["k"][t].execute_rms_norm(w, to_dev(x.reshape(-1)), to_dev(gamma), 1e-6, y, members)
    else:
        env["k"][t].execute_warp_batch(w, to_dev(x.reshape(-1)), y, members)
    got = to_host(y, env["ctx"]).reshape(members, n)
    ref = oracle_rows(t, enc, k, n, x, gamma)
    for m in range(members):
        assert max_rel_err(got[m], ref[m]) <= RTOL, m


@pytest.mark.parametrize("t", (12, 13, 14))
def test_packed_digit_members_do_not_depend_on_the_batch(env, t):
    """Up to 8 members (packed digit planes): reversed order and a 5-member
    subset give the same bits per member."""
    print_case(test="mfma_hl_independence", t=t)
    k, n, members = 4096, 512, 8
    enc = synth.kquant_numpy(t, k, n, seed=190 + t)
    w = upload(env, t, k, n, enc)
    x = synth.activations_numpy(k, members, seed=33)
    y = empty_dev(members * n)
    env["k"][t].execute_warp_batch(w, to_dev(x.reshape(-1)), y, members)
    full = to_host(y, env["ctx"]).reshape(members, n)
    rev = empty_dev(members * n)
    env["k"][t].execute_warp_batch(w, to_dev(x[::-1].reshape(-1)), rev, members)
    assert np.array_equal(to_host(rev, env["ctx"]).reshape(members, n)[::-1].view(np.uint32), full.view(np.uint32))
    pick = [6, 0, 3, 7, 2]
    assert mfma_path(t, k, members) and mfma_path(t, k, len(pick))
    sub = empty_dev(len(pick) * n)
    env["k"][t].execute_warp_batch(w, to_dev(x[pick].reshape(-1)), sub, len(pick))
    assert np.array_equal(to_host(sub, env["ctx"]).reshape(len(pick), n).view(np.uint32), full[pick].view(np.uint32))
    for m in range(members):
        assert max_rel_err(full[m], O.quant_gemv(t, enc, k, n, x[m], threads=8)) <= RTOL, m


@pytest.mark.parametrize("t", (12, 13))
def test_member_outputs_do_not_depend_on_the_batch(env, t):
    print_case(test="mfma_independence", t=t)
    k, n, members = 4096, 512, 13
    enc = synth.kquant_numpy(t, k, n, seed=90 + t)
    w = upload(env, t, k, n, enc)
    x = synth.activations_numpy(k, members, seed=3)
    y = empty_dev(members * n)
    env["k"][t].execute_warp_batch(w, to_dev(x.reshape(-1)), y, members)
    full = to_host(y, env["ctx"]).reshape(members, n)
    # reversed order, and a 9-member subset at other positions
    rev = empty_dev(members * n)
    env["k"][t].execute_warp_batch(w, to_dev(x[::-1].reshape(-1)), rev, members)
    assert np.array_equal(to_host(rev, env["ctx"]).reshape(members, n)[::-1].view(np.uint32), full.view(np.uint32))
    pick = [9, 0, 4, 7, 12, 1, 11, 3, 5]
    assert mfma_path(t, k, members) and mfma_path(t, k, len(pick))
    sub = empty_dev(len(pick) * n)
    env["k"][t].execute_warp_batch(w, to_dev(x[pick].reshape(-1)), sub, len(pick))
    assert np.array_equal(to_host(sub, env["ctx"]).reshape(len(pick), n).view(np.uint32), full[pick].view(np.uint32))


def test_grouped_qkv_at_batch_12(env):
    print_case(test="mfma_group_qkv")
    k, ns, members = 4096, (4096, 1024, 1024), 12
    assert mfma_path(12, k, members)
    encs = [synth.kquant_numpy(12, k, n, seed=200 + i) for i, n in enumerate(ns)]
    ws = [upload(env, 12, k, n, e) for n, e in zip(ns, encs)]
    x = synth.activations_numpy(k, members, seed=21)
    gamma = synth.gamma_numpy(k, seed=22)
    outs = [empty_dev(members * n) for n in ns]
    env["k"][12].execute_group(ws, to_dev(x.reshape(-1)), outs, members, to_dev(gamma), 1e-6)
    for o, n, e in zip(outs, ns, encs):
        got = to_host(o, env["ctx"]).reshape(members, n)
        ref = oracle_rows(12, e, k, n, x, gamma)
        for m in range(members):
            assert max_rel_err(got[m], ref[m]) <= RTOL, (n, m)


@pytest.mark.parametrize("t,n,members", [(12, 12288, 12), (13, 2048, 9), (12, 48, 16)])
def test_gate_up_pairs_at_batch(env, t, n, members):
    print_case(test="mfma_pairs", t=t, n=n, members=members)
    k = 4096
    assert mfma_path(t, k, members)
    ge, ue = synth.kquant_numpy(t, k, n, 400 + n), synth.kquant_numpy(t, k, n, 401 + n)
    gw, uw = upload(env, t, k, n, ge), upload(env, t, k, n, ue)
    x = synth.activations_numpy(k, members, seed=n + members)
    gamma = synth.gamma_numpy(k, seed=5)
    out = empty_dev(members * n)
    env["k"][t].execute_gate_up_swiglu(gw, uw, to_dev(x), out, members, gamma=to_dev(gamma))
    got = to_host(out, env["ctx"]).reshape(members, n)
    for m in range(members):
        normed = O.rms_norm_raw(x[m], gamma, 1e-6)
        ref = O.swiglu(O.quant_gemv(t, ge, k, n, normed, threads=8), O.quant_gemv(t, ue, k, n, normed, threads=8))
        assert max_rel_err(got[m], ref) <= RTOL, m


@pytest.mark.parametrize("t,k,n,members", [(13, 12288, 4096, 8), (12, 4096, 4096, 11)])
def test_residual_accumulate_equals_store_plus_add(env, t, k, n, members):
    print_case(test="mfma_accumulate", t=t, k=k, n=n, members=members)
    assert mfma_path(t, k, members)
    enc = synth.kquant_numpy(t, k, n, seed=61)
    w = upload(env, t, k, n, enc)
    rng = np.random.default_rng(5)
    x = to_dev(rng.standard_normal((members, k)).astype(np.float32))
    base = rng.standard_normal(members * n).astype(np.float32) * 50
    plain = empty_dev(members * n)
    env["k"][t].execute_warp_batch(w, x, plain, members)
    acc = to_dev(base)
    env["k"][t].execute_fused(w, x, acc, members, accumulate=True)
    assert np.array_equal(to_host(acc, env["ctx"]).view(np.uint32), (base + to_host(plain)).view(np.uint32))

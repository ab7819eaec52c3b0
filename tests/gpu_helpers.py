"""Shared helpers for the GPU parity tests (device buffers via torch)."""
import numpy as np

# Max relative error bound for GEMV/GEMM outputs against the f32-accumulated
# oracle, measured normwise: max|y - ref| <= RTOL * max|ref|.
RTOL = 1e-3
# The bar of the f32 GEMV arithmetic on its own (the f32 wave GEMV on
# wide-dynamic-range activations, and the f32-faithful matrix-core GEMV for
# 9..64 members): normwise as RTOL.
F32_RTOL = 5e-5
# Batches up to this many members run the f32 wave GEMV, whose rows are
# bit-identical to the single-member call (cuda_reference.rs:5322-5334);
# larger ones run the f32-faithful matrix-core GEMV (within F32_RTOL).
F32_BITWISE_MEMBERS = 8


def mfma_path(t, k, members):
    """Whether a batched GEMV of this shape runs on the matrix cores in the
    opt-in GEMV_FIXED16 mode (engine_amd/csrc/gemv_mfma.hip launch_gemv):
    Q4_K / Q5_K / Q6_K with 5..16 members, or 4..16 members when K spans more
    than one 4096 slice. The default GEMV_WARP mode never takes that path:
    every batched row is bit-identical to its single-member call."""
    return t in (12, 13, 14) and members <= 16 and (members >= 5 or (k > 4096 and members >= 4))


def wide_range_activations(k, seed):
    """N(0,1) activations with a few x3000 outlier channels, whole scale groups
    at 2^-20, and groups whose elements spread over 2^-16..1 in magnitude."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(k)
    x[rng.choice(k, 8, replace=False)] *= 3000.0
    groups = k // 32
    for g in rng.choice(groups, groups // 8, replace=False):
        x[32 * g:32 * g + 32] *= 2.0 ** -20
    for g in rng.choice(groups, groups // 8, replace=False):
        x[32 * g:32 * g + 32] *= 2.0 ** rng.uniform(-16, 0, 32)
    return x.astype(np.float32)


def max_rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(float(np.abs(ref).max()), 1e-30)
    return float(np.abs(got - ref).max()) / scale


def to_dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to("cuda:0")


def empty_dev(n, dtype=None):
    import torch
    return torch.full((n,), float("nan"), dtype=dtype or torch.float32, device="cuda:0")


def to_host(t, ctx=None):
    import torch
    if ctx is not None:
        ctx.synchronize()
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()

"""GPU test of the allocation-free prefill entry point (ribn_amd_gemm_prefill_static),
called through the C ABI.

It runs the same kernels as ribn_amd_gemm_prefill on a static per-device
scratch array instead of the context's reserved workspace. Bar: two calls in
a row (the second smaller) each within max relative error 1e-3 (normwise,
gpu_helpers.RTOL) of ribn_amd_gemm_prefill on the same inputs and of the f32
oracle; requests beyond the scratch are rejected before any launch.
"""
import ctypes

import numpy as np
import pytest

from engine_amd import synth
from oracle import kquant_oracle as O

from .gpu_helpers import RTOL, empty_dev, max_rel_err, to_dev, to_host

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 8 << 20  # the documented maximum


def static_prefill(lib, kern, w, x, y, members, gamma=None, epsilon=1e-6):
    fn = lib.ribn_amd_gemm_prefill_static  # typed by engine_amd._lib from include/ribn_amd.h
    return fn(kern.handle, w.handle, ctypes.c_void_p(x.data_ptr()), 0, x.numel(), members,
              ctypes.c_void_p(gamma.data_ptr()) if gamma is not None else None,
              gamma.numel() if gamma is not None else 0, epsilon, ctypes.c_void_p(y.data_ptr()), y.numel())


def test_static_prefill_matches_reserved_workspace_prefill():
    import torch
    import engine_amd as E
    from engine_amd import _lib
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    ctx = E.AmdContext(0)
    ctx.reserve_prefill(128, 12288, 2048)
    store = E.AmdWeightStore(ctx)
    lib = _lib.load()
    cases = [(14, 12288, 1024, 96, True), (12, 4096, 512, 8, False)]  # the second call is smaller
    for i, (t, k, n, m, norm) in enumerate(cases):
        print("CASE static_prefill", t, k, n, m, norm, flush=True)
        kern = E.QwenGemvKernel.from_value_type(ctx, t)
        enc = synth.kquant_numpy(t, k, n, seed=90 + i)
        store.materialize_quantized(f"na{i}", [k, n], t, enc)
        w = store.quantized_tensor(f"na{i}")
        x = synth.activations_numpy(k, m, seed=91 + i)
        gamma = synth.gamma_numpy(k, seed=92) if norm else None
        xd, gd = to_dev(x), (to_dev(gamma) if norm else None)
        want = empty_dev(m * n)
        kern.gemm_prefill(w, xd, want, m, gamma=gd, epsilon=1e-6)
        got = empty_dev(m * n)
        assert static_prefill(lib, kern, w, xd, got, m, gd) == 0, _lib.last_error().message
        a = to_host(got, ctx).reshape(m, n)
        b = to_host(want, ctx).reshape(m, n)
        assert np.all(np.isfinite(a))
        assert max_rel_err(a, b) <= RTOL
        for j in (0, m - 1):
            src = O.rms_norm_raw(x[j], gamma, 1e-6) if norm else x[j]
            assert max_rel_err(a[j], O.quant_gemv(t, enc, k, n, src, threads=8)) <= RTOL
    # beyond the static scratch: rejected with the sizes, nothing launched
    kern = E.QwenGemvKernel.from_value_type(ctx, 12)
    m, k = 1024, 8192
    store.materialize_quantized("na_big", [k, 4], 12, synth.kquant_numpy(12, k, 4, seed=1))
    w = store.quantized_tensor("na_big")
    x = torch.zeros(m * k, device="cuda:0")
    y = torch.zeros(m * 4, device="cuda:0")
    assert static_prefill(lib, kern, w, x, y, m) == 15  # WorkspaceTooSmall
    err = _lib.last_error()
    assert err.expected == SCRATCH_BYTES and err.actual > SCRATCH_BYTES

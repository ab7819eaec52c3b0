"""CPU checks of the C-ABI boundary: the library loads, exports every symbol the
header declares, and its host-only validation mirrors the reference's
validate_quantized_geometry (crates/nvidia/src/quantized.rs:1755-1804).
No kernel is launched here."""
import ctypes
import subprocess

import pytest

import engine_amd as E
from engine_amd import _lib


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _lib.declared_functions()
    assert len(declared) >= 30
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing, missing
    # the ctypes binding types every declared function
    assert sorted(_lib.SIGNATURES) == declared
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(declared) <= exported


def test_abi_version_and_status_names():
    lib = _lib.load()
    assert lib.ribn_amd_abi_version() == 2
    for code, name in _lib.STATUS_NAMES.items():
        assert lib.ribn_amd_status_name(code).decode() == name


@pytest.mark.parametrize("t,k,n,nbytes", [(12, 4096, 4096, 9_437_184), (13, 12288, 4096, 34_603_008),
                                          (14, 4096, 151936, 510_504_960), (12, 256, 1, 144)])
def test_geometry_accepts_exact_shapes(t, k, n, nbytes):
    assert E.validate_quantized_geometry(t, t, [k, n], nbytes) == (k, n)


def expect(kind, fn, expected=None, actual=None):
    with pytest.raises(E.AmdQuantizedKernelError) as e:
        fn()
    assert e.value.kind == kind, str(e.value)
    if expected is not None:
        assert e.value.expected == expected
    if actual is not None:
        assert e.value.actual == actual
    return e.value


def test_geometry_errors_in_reference_order():
    v = E.validate_quantized_geometry
    expect("UnsupportedValueType", lambda: v(12, 13, [256, 1], 176), 12, 13)
    expect("UnsupportedValueType", lambda: v(11, 11, [256, 1], 110), 12, 11)
    expect("InvalidWeight", lambda: v(12, 12, [256], 144), 2, 1)
    expect("InvalidWeight", lambda: v(12, 12, [256, 1, 1], 144), 2, 3)
    expect("InvalidWeight", lambda: v(12, 12, [128, 2], 144), 256, 128)
    expect("InvalidWeight", lambda: v(12, 12, [0, 2], 0))
    expect("InvalidWeight", lambda: v(12, 12, [256, 0], 0))
    expect("InvalidWeight", lambda: v(12, 12, [512, 2], 575), 576, 575)
    # i32 launch limits (quantized.rs:1795-1800)
    big_n = 2**31 // 144 + 10
    expect("ShapeOverflow", lambda: v(12, 12, [256, big_n], 144 * big_n))
    expect("ShapeOverflow", lambda: v(12, 12, [256 * 2**40, 2**40], 1))


def test_null_handles_are_rejected_without_a_device():
    lib = _lib.load()
    st = lib.ribn_amd_gemv_execute(None, None, None, 0, None, 0)
    assert _lib.STATUS_NAMES[st] == "InvalidArgument"
    st = lib.ribn_amd_gemv_execute_warp_batch(None, None, None, 0, None, 0, 0)
    assert _lib.STATUS_NAMES[st] == "InputLength"  # members == 0 is checked first (quantized.rs:458-463)
    err = _lib.last_error()
    assert (err.expected, err.actual) == (1, 0)
    assert _lib.STATUS_NAMES[lib.ribn_amd_last_error(None)] == "InvalidArgument"


def test_package_fails_loudly_without_library(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.load()


def test_decoder_keeps_its_weights_and_norms_alive():
    """AmdQwen3Decode holds every weight handle and norm tensor it is given:
    the C decoder reads them at every step and does not own them, so dropping
    the caller's references must not free them while the decoder lives, and
    dropping the decoder releases them. (A stand-in library answers the
    create call; nothing reaches the device.)"""
    import gc
    import weakref

    from engine_amd import qwen3

    class FakeLib:
        def ribn_amd_qwen3_decode_create(self, *args):
            return 0

    class FakeCtx:
        def __init__(self):
            self._lib = FakeLib()
            self.handle = ctypes.c_void_p(1)

    class Weight:
        def __init__(self):
            self.handle = ctypes.c_void_p(0x1000)

    class Tensor:
        def data_ptr(self):
            return 0x2000

    weights = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"}
    layers = [{n: (Weight() if n in weights else Tensor()) for n in _lib.QWEN3_LAYER_FIELDS} for _ in range(2)]
    emb, out, norm = Weight(), Weight(), Tensor()
    refs = [weakref.ref(o) for lw in layers for o in lw.values()] + [weakref.ref(o) for o in (emb, out, norm)]
    dec = qwen3.AmdQwen3Decode(FakeCtx(), qwen3.AmdQwen3Config(layers=2), emb, out, norm, layers)
    del layers, emb, out, norm
    gc.collect()
    assert all(r() is not None for r in refs)
    del dec
    gc.collect()
    assert all(r() is None for r in refs)

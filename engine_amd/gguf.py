"""GGUF reader and device weight staging over the C ABI (engine_amd/csrc/gguf.cpp).

Mirrors the reference's format boundary:
  GgufFile / TensorInfo / MetadataValue   <- crates/gguf/src/lib.rs:29-345
  stage()                                 <- CudaQwen35Weights::stage (crates/nvidia/src/staging.rs:238-292)
  qwen3_config_from_gguf()                <- config_from_gguf (crates/qwen/src/gguf.rs:14-56), for the
                                             dense Qwen3 architecture ("qwen3.*" keys)
  load_qwen3_decode()                     <- staging + CudaQwen35Decode construction for a GGUF checkpoint
Parsing runs on the host inside libribn_amd.so; staging copies the encoded
bytes unchanged to device memory.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from . import _lib
from .kquant import RANK_RESOURCE, AmdContext, AmdKernelError, AmdQuantizedWeight, _check, _own

DEFAULT_BUDGET = 1 << 62


class GgufError(AmdKernelError):
    """GgufError (lib.rs:741-805): `kind` carries the variant name."""


@dataclass(frozen=True)
class TensorInfo:
    """TensorInfo (lib.rs:87-163)."""
    name: str
    dimensions: tuple
    value_type: int
    offset: int

    def element_count(self) -> int:
        n = 1
        for d in self.dimensions:
            n *= d
        return n


def _value(v: _lib.GgufValue, g, key: str, path: tuple = ()):
    t = v.type
    if t in (0, 2, 4, 10):
        return int(v.u)
    if t in (1, 3, 5, 11):
        return int(v.i)
    if t in (6, 12):
        return float(v.f)
    if t == 7:
        return bool(v.u)
    if t == 8:
        return ctypes.string_at(v.str, v.str_len).decode("utf-8")
    if t == 9:
        items = []
        lib = _lib.load()
        for i in range(v.array_len):
            sub = path + (i,)
            arr = (ctypes.c_uint64 * len(sub))(*sub)
            item = _lib.GgufValue()
            _check(lib.ribn_amd_gguf_metadata_item(g, key.encode(), arr, len(sub), ctypes.byref(item)), GgufError)
            items.append(_value(item, g, key, sub))
        return items
    raise GgufError(23, 12, t, f"InvalidValueType: {t}")


class GgufFile:
    """GgufFile (lib.rs:165-345): header, metadata and tensor directory."""

    def __init__(self, handle, path: str):
        self._lib = _lib.load()
        self.handle = handle
        self._path = path
        _own(self, RANK_RESOURCE)

    @classmethod
    def open(cls, path: str) -> "GgufFile":
        lib = _lib.load()
        h = ctypes.c_void_p()
        _check(lib.ribn_amd_gguf_open(str(path).encode(), ctypes.byref(h)), GgufError)
        return cls(h, str(path))

    def path(self) -> str:
        return self._path

    def version(self) -> int:
        return int(self._lib.ribn_amd_gguf_version(self.handle))

    def tensor_count(self) -> int:
        return int(self._lib.ribn_amd_gguf_tensor_count(self.handle))

    def tensor_data_offset(self) -> int:
        return int(self._lib.ribn_amd_gguf_tensor_data_offset(self.handle))

    def metadata(self, key: str):
        """The value of `key` as a Python value, or None when absent."""
        v = _lib.GgufValue()
        st = self._lib.ribn_amd_gguf_metadata_get(self.handle, key.encode(), ctypes.byref(v))
        if st == 35:  # MissingMetadata
            return None
        _check(st, GgufError)
        return _value(v, self.handle, key)

    def metadata_map(self) -> dict:
        n = int(self._lib.ribn_amd_gguf_metadata_count(self.handle))
        keys = [self._lib.ribn_amd_gguf_metadata_key(self.handle, i).decode("utf-8") for i in range(n)]
        return {k: self.metadata(k) for k in keys}

    def tensors(self) -> list:
        out = []
        for i in range(self.tensor_count()):
            t = _lib.GgufTensor()
            _check(self._lib.ribn_amd_gguf_tensor_info(self.handle, i, ctypes.byref(t)), GgufError)
            out.append(TensorInfo(t.name.decode("utf-8"), tuple(int(t.dims[d]) for d in range(t.n_dims)),
                                  int(t.value_type), int(t.offset)))
        return out

    def tensor(self, name: str):
        idx = ctypes.c_uint64()
        st = self._lib.ribn_amd_gguf_find_tensor(self.handle, name.encode(), ctypes.byref(idx))
        if st == 18:  # MissingTensor
            return None
        _check(st, GgufError)
        t = _lib.GgufTensor()
        _check(self._lib.ribn_amd_gguf_tensor_info(self.handle, idx.value, ctypes.byref(t)), GgufError)
        return TensorInfo(t.name.decode("utf-8"), tuple(int(t.dims[d]) for d in range(t.n_dims)),
                          int(t.value_type), int(t.offset))

    def tensor_data_range(self, name: str) -> range:
        s, e = ctypes.c_uint64(), ctypes.c_uint64()
        _check(self._lib.ribn_amd_gguf_tensor_data_range(self.handle, name.encode(), ctypes.byref(s),
                                                         ctypes.byref(e)), GgufError)
        return range(s.value, e.value)

    def close(self):
        if self.handle:
            self._lib.ribn_amd_gguf_close(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class AmdDeviceTensor:
    """A staged non-k-quant tensor (e.g. an F32 norm vector): its device bytes
    through `data_ptr()`, for the decoder's norm arguments."""

    def __init__(self, weight: AmdQuantizedWeight):
        self.weight = weight

    def data_ptr(self) -> int:
        return self.weight.device_ptr()


def stage(ctx: AmdContext, file: GgufFile, names, budget_bytes: int = DEFAULT_BUDGET) -> dict:
    """CudaQwen35Weights::stage: checks the encoded total against the budget,
    then uploads every named tensor unchanged. Returns name -> weight (k-quant
    types) or AmdDeviceTensor (other types)."""
    names = list(names)
    arr = (ctypes.c_char_p * len(names))(*[n.encode() for n in names])
    out = (ctypes.c_void_p * len(names))()
    _check(ctx._lib.ribn_amd_gguf_stage(ctx.handle, file.handle, arr, len(names), budget_bytes, out), GgufError)
    staged = {}
    for name, h in zip(names, out):
        info = file.tensor(name)
        w = AmdQuantizedWeight(ctx, ctypes.c_void_p(h), name, info.dimensions, info.value_type)
        staged[name] = w if info.value_type in (12, 13, 14) else AmdDeviceTensor(w)
    return staged


def _required_u64(file: GgufFile, key: str) -> int:
    lib = _lib.load()
    v = _lib.GgufValue()
    st = lib.ribn_amd_gguf_metadata_get(file.handle, key.encode(), ctypes.byref(v))
    if st == 35:
        raise GgufError(35, 0, 0, f"MissingMetadata: {key}")
    _check(st, GgufError)
    if v.type not in (0, 2, 4, 10):  # MetadataValue::as_u64
        raise GgufError(36, 0, v.type, f"MetadataTypeMismatch: {key}")
    return int(v.u)


def _required_u32(file: GgufFile, key: str) -> int:
    v = _required_u64(file, key)
    if v > 0xFFFFFFFF:
        raise GgufError(36, 0xFFFFFFFF, v, f"MetadataTypeMismatch: {key}")
    return v


def _optional_f32(file: GgufFile, key: str, default: float) -> float:
    v = file.metadata(key)
    return default if v is None else float(v)


def qwen3_config_from_gguf(file: GgufFile):
    """Qwen3 dense geometry from "qwen3.*" metadata (the reference's
    config_from_gguf reads "qwen35.*" for its hybrid model the same way)."""
    from .qwen3 import AmdQwen3Config

    arch = file.metadata("general.architecture")
    if arch is None:
        raise GgufError(35, 0, 0, "MissingMetadata: general.architecture")
    if arch != "qwen3":
        raise GgufError(36, 0, 0, f"UnsupportedArchitecture: {arch}")
    hidden = _required_u32(file, "qwen3.embedding_length")
    heads = _required_u32(file, "qwen3.attention.head_count")
    head_dim = file.metadata("qwen3.attention.key_length")
    head_dim = int(head_dim) if head_dim is not None else hidden // heads
    embd = file.tensor("token_embd.weight")
    if embd is None:
        raise GgufError(18, 0, 0, "MissingTensor: token_embd.weight")
    return AmdQwen3Config(layers=_required_u32(file, "qwen3.block_count"), hidden=hidden, q_heads=heads,
                          kv_heads=_required_u32(file, "qwen3.attention.head_count_kv"), head_dim=head_dim,
                          ffn=_required_u32(file, "qwen3.feed_forward_length"), vocab=int(embd.dimensions[1]),
                          rope_base=_optional_f32(file, "qwen3.rope.freq_base", 1.0e6),
                          epsilon=_optional_f32(file, "qwen3.attention.layer_norm_rms_epsilon", 1.0e-6))


LAYER_TENSORS = {"attn_q": "attn_q.weight", "attn_k": "attn_k.weight", "attn_v": "attn_v.weight",
                 "attn_output": "attn_output.weight", "ffn_gate": "ffn_gate.weight", "ffn_up": "ffn_up.weight",
                 "ffn_down": "ffn_down.weight", "attn_norm": "attn_norm.weight",
                 "attn_q_norm": "attn_q_norm.weight", "attn_k_norm": "attn_k_norm.weight",
                 "ffn_norm": "ffn_norm.weight"}


def qwen3_tensor_names(layers: int) -> list:
    names = ["token_embd.weight", "output_norm.weight"]
    for i in range(layers):
        names += [f"blk.{i}.{v}" for v in LAYER_TENSORS.values()]
    return names


def load_qwen3_decode(ctx: AmdContext, path: str, max_members: int = 1, budget_bytes: int = DEFAULT_BUDGET):
    """Stages a Qwen3 GGUF checkpoint and builds the decoder over it. A file
    without "output.weight" ties the lm_head to token_embd (as Qwen3 files
    with tied embeddings do). Returns (decoder, config, file, staged)."""
    from .qwen3 import AmdQwen3Decode

    file = GgufFile.open(path)
    cfg = qwen3_config_from_gguf(file)
    names = qwen3_tensor_names(cfg.layers)
    tied = file.tensor("output.weight") is None
    if not tied:
        names.append("output.weight")
    staged = stage(ctx, file, names, budget_bytes)
    layers = [{k: staged[f"blk.{i}.{v}"] for k, v in LAYER_TENSORS.items()} for i in range(cfg.layers)]
    output = staged["token_embd.weight"] if tied else staged["output.weight"]
    dec = AmdQwen3Decode(ctx, cfg, staged["token_embd.weight"], output, staged["output_norm.weight"], layers,
                         max_members)
    return dec, cfg, file, staged

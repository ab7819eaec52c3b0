"""ctypes binding of libribn_amd.so (the C ABI in include/ribn_amd.h).

The library is built in-tree by `python -m engine_amd.build` (or
__graft_entry__.build()). Loading fails loudly when it is missing: there is no
CPU fallback for any operation of this package.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
# RIBN_AMD_LIBRARY names another build of the same ABI (the host-sanitized
# test library of `python -m engine_amd.build --sanitize`); default: the
# in-tree product library.
LIB_PATH = os.environ.get("RIBN_AMD_LIBRARY") or os.path.join(HERE, "libribn_amd.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "ribn_amd.h")

STATUS_NAMES = {
    0: "Ok", 1: "Driver", 2: "Module", 3: "InvalidWeight", 4: "UnsupportedValueType",
    5: "ShapeOverflow", 6: "InputLength", 7: "OutputLength", 8: "ContextMismatch",
    9: "EmptyInput", 10: "WeightLength", 11: "InvalidEpsilon", 12: "InvalidArgument",
    13: "EmptyEncoding", 14: "SourceIncomplete", 15: "WorkspaceTooSmall", 16: "InvalidPlan",
    17: "PositionOverflow", 18: "MissingTensor", 19: "Io", 20: "InvalidMagic", 21: "UnsupportedVersion",
    22: "InvalidUtf8", 23: "InvalidValueType", 24: "InvalidBool", 25: "InvalidLength", 26: "ArrayNestingTooDeep",
    27: "DuplicateMetadata", 28: "InvalidDimensionCount", 29: "InvalidAlignment", 30: "Truncated",
    31: "TensorOffsetOutOfBounds", 32: "UnsupportedTensorType", 33: "TensorByteLengthOverflow",
    34: "QuantizationMismatch", 35: "MissingMetadata", 36: "MetadataTypeMismatch", 37: "BudgetExceeded",
    38: "Unsupported", 39: "ExecutionFailed", 40: "UnknownSubmission", 41: "DeviceFaulted", 42: "StatePosition",
}


class RibnAmdError(ctypes.Structure):
    _fields_ = [("status", ctypes.c_int32), ("expected", ctypes.c_uint64),
                ("actual", ctypes.c_uint64), ("message", ctypes.c_char * 512)]


class Qwen3Config(ctypes.Structure):
    """ribn_amd_qwen3_config."""
    _fields_ = [("layers", ctypes.c_uint32), ("hidden", ctypes.c_uint32), ("q_heads", ctypes.c_uint32),
                ("kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32), ("ffn", ctypes.c_uint32),
                ("vocab", ctypes.c_uint32), ("rope_base", ctypes.c_float), ("epsilon", ctypes.c_float)]


QWEN3_LAYER_FIELDS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down",
                      "attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm")


class Qwen3Layer(ctypes.Structure):
    """ribn_amd_qwen3_layer: seven weight handles, then four device norm vectors."""
    _fields_ = [(name, ctypes.c_void_p) for name in QWEN3_LAYER_FIELDS]


class GgufValue(ctypes.Structure):
    """ribn_amd_gguf_value."""
    _fields_ = [("type", ctypes.c_uint32), ("array_type", ctypes.c_uint32), ("array_len", ctypes.c_uint64),
                ("u", ctypes.c_uint64), ("i", ctypes.c_int64), ("f", ctypes.c_double),
                ("str", ctypes.c_void_p), ("str_len", ctypes.c_uint64)]


class GgufTensor(ctypes.Structure):
    """ribn_amd_gguf_tensor."""
    _fields_ = [("name", ctypes.c_char_p), ("n_dims", ctypes.c_uint32), ("dims", ctypes.c_uint64 * 16),
                ("value_type", ctypes.c_uint32), ("offset", ctypes.c_uint64)]


class ServingRow(ctypes.Structure):
    """ribn_amd_serving_row."""
    _fields_ = [("request", ctypes.c_uint64), ("state", ctypes.c_uint64), ("phase", ctypes.c_uint32),
                ("state_position", ctypes.c_uint32), ("tokens", ctypes.POINTER(ctypes.c_uint32)),
                ("token_count", ctypes.c_uint32), ("requests_sampling", ctypes.c_uint32),
                ("temperature", ctypes.c_float), ("kv_tokens", ctypes.c_uint32),
                ("logical_position", ctypes.c_uint32)]


class ServingOutcome(ctypes.Structure):
    """ribn_amd_serving_outcome."""
    _fields_ = [("elapsed_nanos", ctypes.c_uint64), ("has_token", ctypes.c_uint32), ("token", ctypes.c_uint32)]


class MemoryPlan(ctypes.Structure):
    """ribn_amd_memory_plan."""
    _fields_ = [("free_before_preparation_bytes", ctypes.c_uint64), ("weight_budget_bytes", ctypes.c_uint64),
                ("reserved_sequence_bytes", ctypes.c_uint64)]


READ_FN = ctypes.CFUNCTYPE(ctypes.c_int64, ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint8), ctypes.c_size_t)

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_pvp = ctypes.POINTER(ctypes.c_void_p)

SIGNATURES = {
    "ribn_amd_last_error": (_i32, [ctypes.POINTER(RibnAmdError)]),
    "ribn_amd_status_name": (ctypes.c_char_p, [_i32]),
    "ribn_amd_abi_version": (_i32, []),
    "ribn_amd_context_create": (_i32, [_i32, _pvp]),
    "ribn_amd_context_wrap_stream": (_i32, [_i32, _vp, _pvp]),
    "ribn_amd_context_destroy": (None, [_vp]),
    "ribn_amd_context_synchronize": (_i32, [_vp]),
    "ribn_amd_context_stream": (_vp, [_vp]),
    "ribn_amd_context_device": (_i32, [_vp]),
    "ribn_amd_alloc": (_i32, [_vp, _sz, _pvp]),
    "ribn_amd_free": (_i32, [_vp, _vp]),
    "ribn_amd_memcpy_htod": (_i32, [_vp, _vp, _vp, _sz]),
    "ribn_amd_memcpy_dtoh": (_i32, [_vp, _vp, _vp, _sz]),
    "ribn_amd_weight_materialize": (_i32, [_vp, _u32, _u64, _u64, _vp, _u64, _pvp]),
    "ribn_amd_weight_materialize_reader": (_i32, [_vp, _u32, _u64, _u64, _u64, READ_FN, _vp, _pvp]),
    "ribn_amd_weight_wrap_device": (_i32, [_vp, _u32, _u64, _u64, _vp, _u64, _pvp]),
    "ribn_amd_weight_copy_to_host": (_i32, [_vp, _vp, _vp, _u64]),
    "ribn_amd_weight_destroy": (None, [_vp]),
    "ribn_amd_weight_value_type": (_u32, [_vp]),
    "ribn_amd_weight_encoded_bytes": (_u64, [_vp]),
    "ribn_amd_weight_input_size": (_u64, [_vp]),
    "ribn_amd_weight_output_size": (_u64, [_vp]),
    "ribn_amd_weight_device_ptr": (_vp, [_vp]),
    "ribn_amd_validate_quantized_geometry": (_i32, [_u32, _u32, ctypes.POINTER(_u64), _sz, _u64,
                                                    ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "ribn_amd_gemv_create": (_i32, [_vp, _u32, _pvp]),
    "ribn_amd_gemv_destroy": (None, [_vp]),
    "ribn_amd_gemv_value_type": (_u32, [_vp]),
    "ribn_amd_gemv_set_mode": (_i32, [_vp, _u32]),
    "ribn_amd_gemv_mode": (_u32, [_vp]),
    "ribn_amd_gemv_execute": (_i32, [_vp, _vp, _vp, _sz, _vp, _sz]),
    "ribn_amd_gemv_execute_warp": (_i32, [_vp, _vp, _vp, _sz, _vp, _sz]),
    "ribn_amd_gemv_execute_warp_batch": (_i32, [_vp, _vp, _vp, _sz, _vp, _sz, _sz]),
    "ribn_amd_gemv_execute_rms_norm": (_i32, [_vp, _vp, _vp, _sz, _vp, _sz, _f32, _vp, _sz, _sz]),
    "ribn_amd_gemv_execute_group": (_i32, [_vp, _pvp, _sz, _vp, _sz, _vp, _sz, _f32, _pvp,
                                           ctypes.POINTER(_sz), _sz]),
    "ribn_amd_dequantize": (_i32, [_vp, _vp, _vp, _sz]),
    "ribn_amd_gemm_workspace_bytes": (_sz, [_sz, _sz, _sz]),
    "ribn_amd_context_reserve_prefill": (_i32, [_vp, _sz, _sz, _sz]),
    "ribn_amd_gemm_prefill": (_i32, [_vp, _vp, _vp, _u32, _sz, _sz, _vp, _sz, _f32, _vp, _sz]),
    "ribn_amd_gemm_prefill_static": (_i32, [_vp, _vp, _vp, _u32, _sz, _sz, _vp, _sz, _f32, _vp, _sz]),
    "ribn_amd_embedding_create": (_i32, [_vp, _u32, _pvp]),
    "ribn_amd_embedding_destroy": (None, [_vp]),
    "ribn_amd_embedding_execute": (_i32, [_vp, _vp, _u32, _vp, _sz]),
    "ribn_amd_embedding_execute_batch": (_i32, [_vp, _vp, _vp, _sz, _vp, _sz]),
    "ribn_amd_rms_norm": (_i32, [_vp, _vp, _sz, _vp, _sz, _vp, _sz, _f32]),
    "ribn_amd_rms_norm_batch": (_i32, [_vp, _vp, _sz, _vp, _sz, _vp, _sz, _sz, _f32]),
    "ribn_amd_gemv_execute_fused": (_i32, [_vp, _vp, _vp, _vp, _sz, _vp, _sz, _f32, _vp, _sz, _sz, _u32]),
    "ribn_amd_gemv_execute_gate_up_swiglu": (_i32, [_vp, _vp, _vp, _vp, _sz, _vp, _sz, _f32, _vp, _sz, _sz]),
    "ribn_amd_q8_1_quantize": (_i32, [_vp, _vp, _sz, _vp, _sz]),
    "ribn_amd_gemv_execute_q8_1": (_i32, [_vp, _vp, _vp, _sz, _vp, _sz]),
    "ribn_amd_gemv_execute_q8_1_batch": (_i32, [_vp, _vp, _vp, _sz, _vp, _sz, _sz]),
    "ribn_amd_gguf_open": (_i32, [ctypes.c_char_p, _pvp]),
    "ribn_amd_gguf_close": (None, [_vp]),
    "ribn_amd_gguf_version": (_u32, [_vp]),
    "ribn_amd_gguf_tensor_count": (_u64, [_vp]),
    "ribn_amd_gguf_tensor_data_offset": (_u64, [_vp]),
    "ribn_amd_gguf_metadata_count": (_u64, [_vp]),
    "ribn_amd_gguf_metadata_key": (ctypes.c_char_p, [_vp, _u64]),
    "ribn_amd_gguf_metadata_get": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(GgufValue)]),
    "ribn_amd_gguf_metadata_array_get": (_i32, [_vp, ctypes.c_char_p, _u64, ctypes.POINTER(GgufValue)]),
    "ribn_amd_gguf_metadata_item": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(_u64), _sz, ctypes.POINTER(GgufValue)]),
    "ribn_amd_gguf_tensor_info": (_i32, [_vp, _u64, ctypes.POINTER(GgufTensor)]),
    "ribn_amd_gguf_find_tensor": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(_u64)]),
    "ribn_amd_gguf_tensor_data_range": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "ribn_amd_gguf_stage": (_i32, [_vp, _vp, ctypes.POINTER(ctypes.c_char_p), _sz, _u64, _pvp]),
    "ribn_amd_kv_cache_create": (_i32, [_vp, ctypes.POINTER(Qwen3Config), _u32, _pvp]),
    "ribn_amd_kv_cache_destroy": (None, [_vp]),
    "ribn_amd_kv_cache_capacity": (_u32, [_vp]),
    "ribn_amd_kv_cache_layer": (_i32, [_vp, _u32, _pvp, _pvp]),
    "ribn_amd_attention_decode": (_i32, [_vp, ctypes.POINTER(Qwen3Config), _pvp, _sz, _u32, _vp, _vp, _vp, _vp,
                                         _vp, _vp, _vp, _sz]),
    "ribn_amd_argmax": (_i32, [_vp, _vp, _sz, _sz, _vp]),
    "ribn_amd_qwen3_decode_create": (_i32, [_vp, ctypes.POINTER(Qwen3Config), _vp, _vp, _vp,
                                            ctypes.POINTER(Qwen3Layer), _u32, _pvp]),
    "ribn_amd_qwen3_decode_destroy": (None, [_vp]),
    "ribn_amd_qwen3_decode_set_graphs": (_i32, [_vp, _i32]),
    "ribn_amd_qwen3_decode_set_gemv_mode": (_i32, [_vp, _u32]),
    "ribn_amd_qwen3_decode_gemv_mode": (_u32, [_vp]),
    "ribn_amd_qwen3_prefill_step": (_i32, [_vp, _vp, _u32, _u32]),
    "ribn_amd_qwen3_prefill_chunk": (_i32, [_vp, _vp, ctypes.POINTER(_u32), _sz, _u32]),
    "ribn_amd_attention_prefill": (_i32, [_vp, ctypes.POINTER(Qwen3Config), _vp, _u32, _vp, _vp, _vp, _vp, _vp, _sz,
                                       _u32, _vp, _sz]),
    "ribn_amd_probe_mfma_peak": (_i32, [_vp, _u32, _u32, ctypes.POINTER(ctypes.c_double)]),
    "ribn_amd_qwen3_prefill_prompt": (_i32, [_vp, _vp, ctypes.POINTER(_u32), _sz, _u32, _u32]),
    "ribn_amd_qwen3_reserve_prompt": (_i32, [_vp, _u32]),
    "ribn_amd_qwen3_decode_step": (_i32, [_vp, _vp, _u32, _u32, ctypes.POINTER(_u32)]),
    "ribn_amd_qwen3_decode_step_batch": (_i32, [_vp, _pvp, ctypes.POINTER(_u32), ctypes.POINTER(_u32), _sz,
                                                ctypes.POINTER(_u32)]),
    "ribn_amd_qwen3_generate": (_i32, [_vp, _pvp, ctypes.POINTER(_u32), ctypes.POINTER(_u32), _sz, _u32,
                                       ctypes.POINTER(_u32)]),
    "ribn_amd_qwen3_copy_hidden": (_i32, [_vp, _sz, _vp, _sz]),
    "ribn_amd_qwen3_copy_logits": (_i32, [_vp, _sz, _vp, _sz]),
    "ribn_amd_serving_create": (_i32, [_vp, _u32, _u64, _pvp]),
    "ribn_amd_serving_destroy": (None, [_vp]),
    "ribn_amd_serving_set_prefill_chunk": (_i32, [_vp, _u32]),
    "ribn_amd_serving_set_prompt_prefill": (_i32, [_vp, _u32]),
    "ribn_amd_serving_set_grouped_decode": (_i32, [_vp, _i32]),
    "ribn_amd_serving_dispatch_batch": (_i32, [_vp, ctypes.POINTER(ServingRow), _sz, ctypes.POINTER(ServingOutcome)]),
    "ribn_amd_serving_submit_batch": (_i32, [_vp, _u64, ctypes.POINTER(ServingRow), _sz]),
    "ribn_amd_serving_poll_batch": (_i32, [_vp, _u64, ctypes.POINTER(ServingOutcome), _sz,
                                           ctypes.POINTER(_i32)]),
    "ribn_amd_serving_release_state": (_i32, [_vp, _u64]),
    "ribn_amd_serving_pending": (_sz, [_vp]),
    "ribn_amd_serving_state_count": (_sz, [_vp]),
    "ribn_amd_serving_state_bytes": (_u64, [_vp, ctypes.POINTER(_u64)]),
    "ribn_amd_serving_state_position": (_i32, [_vp, _u64, ctypes.POINTER(_u32)]),
    "ribn_amd_serving_chunked_prefix_len": (_u32, [_u32, _u32, _i32]),
    "ribn_amd_serving_decode_group": (_sz, [ctypes.POINTER(ServingRow), _sz, ctypes.POINTER(ctypes.c_uint8), _sz,
                                            _sz, ctypes.POINTER(_sz)]),
    "ribn_amd_plan_memory": (_i32, [_vp, _u64, _u64, _u64, _u64, _u64, ctypes.POINTER(MemoryPlan)]),
    "ribn_amd_qwen3_kv_bytes": (_u64, [ctypes.POINTER(Qwen3Config), _u32]),
}

_lib = None


def declared_functions() -> list[str]:
    """Function names declared in include/ribn_amd.h (typedefs excluded)."""
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(ribn_amd_[a-z0-9_]+)\s*\(", text))
    typedefs = set(re.findall(r"\(\s*\*\s*(ribn_amd_[a-z0-9_]+)\s*\)", text))
    return sorted(names - typedefs)


def load():
    """Loads and types the library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m engine_amd.build` "
            "(the k-quant path has no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error():
    err = RibnAmdError()
    load().ribn_amd_last_error(ctypes.byref(err))
    return err

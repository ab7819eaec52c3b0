"""engine_amd: MI355X-native (gfx950) k-quant decode path behind a C ABI.

The product is libribn_amd.so (HIP kernels + C ABI, include/ribn_amd.h); this
package holds its sources (csrc/), the build script, a ctypes binding and a
host-side mirror of the reference's operator API (kquant.py).
"""
from . import _lib  # noqa: F401
from .kquant import (  # noqa: F401
    AmdQ4KQ8_1Gemv, AmdQ5KQ8_1Gemv, AmdQ6KQ8_1Gemv, AmdQ8_1Quantizer,
    Q4_K, Q5_K, Q6_K, BLOCK_BYTES, GEMV_WARP, GEMV_FIXED16,
    AmdContext, AmdWeightStore, AmdQuantizedWeight,
    AmdQ4KGemv, AmdQ5KGemv, AmdQ6KGemv, QwenGemvKernel, AmdQwenOps,
    AmdQ4KEmbedding, AmdKQuantEmbedding,
    AmdKernelError, AmdQuantizedKernelError, AmdModelKernelError, AmdWeightError,
    validate_quantized_geometry,
)
from .gguf import GgufError, GgufFile, TensorInfo, load_qwen3_decode, qwen3_config_from_gguf  # noqa: F401
from .qwen3 import AmdKvCache, AmdQwen3Config, AmdQwen3Decode, QWEN3_8B, attention_decode, attention_prefill  # noqa: F401
from .serving import AmdBackend, AmdDispatcher, AmdServingDispatcher, BackendError, plan_memory  # noqa: F401

__all__ = [
    "Q4_K", "Q5_K", "Q6_K", "BLOCK_BYTES", "GEMV_WARP", "GEMV_FIXED16", "AmdContext", "AmdWeightStore", "AmdQuantizedWeight",
    "AmdQ4KGemv", "AmdQ5KGemv", "AmdQ6KGemv", "QwenGemvKernel", "AmdQwenOps", "AmdQ4KEmbedding",
    "AmdKQuantEmbedding", "AmdKernelError",
    "AmdQuantizedKernelError", "AmdModelKernelError", "AmdWeightError", "validate_quantized_geometry",
    "AmdKvCache", "AmdQwen3Config", "AmdQwen3Decode", "QWEN3_8B", "attention_decode",
    "AmdQ8_1Quantizer", "AmdQ4KQ8_1Gemv", "AmdQ5KQ8_1Gemv", "AmdQ6KQ8_1Gemv",
    "GgufError", "GgufFile", "TensorInfo", "load_qwen3_decode", "qwen3_config_from_gguf",
    "AmdBackend", "AmdDispatcher", "AmdServingDispatcher", "BackendError", "plan_memory",
]

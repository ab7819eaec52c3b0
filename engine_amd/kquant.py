"""Host-side mirror of the reference's k-quant operator API over the C ABI.

Same names, argument meaning and error behaviour as crates/nvidia:
  AmdQuantizedKernelError   <- CudaQuantizedKernelError (quantized.rs:91-134)
  AmdModelKernelError       <- CudaModelKernelError (model_ops.rs:12-22)
  AmdWeightStore            <- CudaWeightStore (cuda.rs:192-459)
  AmdQ4KGemv/AmdQ5KGemv/AmdQ6KGemv <- CudaQ4KGemv/... (quantized.rs:1465-1753)
  AmdQ8_1Quantizer          <- CudaQ8_1Quantizer (activation.rs:8-88)
  AmdQ4KQ8_1Gemv/...        <- CudaQ4KQ8_1Gemv/... (q4_q8_1.rs, q5_q8_1.rs, q6_q8_1.rs)
  QwenGemvKernel            <- QwenGemvKernel (staging.rs:90-217)
  AmdQwenOps                <- CudaQwen35Ops::{rms_norm, rms_norm_batch} (model_ops.rs:1714-1824)

Device buffers are torch tensors on the context's device (torch is only the
allocator and stream provider here); every computation runs in
libribn_amd.so. Launches are asynchronous on the context stream, which by
default is torch's current stream so torch-side copies order after them.
"""
from __future__ import annotations

import atexit
import ctypes
import gc
import weakref

from . import _lib

Q4_K, Q5_K, Q6_K = 12, 13, 14
BLOCK_BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210}
# GEMV arithmetic (the reference's GemvMode, decode.rs:285-307): GEMV_WARP is
# f32 activations (default); GEMV_FIXED16 the opt-in block fixed-point mode.
GEMV_WARP, GEMV_FIXED16 = 0, 1


class AmdKernelError(Exception):
    """A non-Ok status of the C ABI with its expected/actual fields."""

    def __init__(self, status: int, expected: int, actual: int, message: str):
        self.status = status
        self.kind = _lib.STATUS_NAMES.get(status, f"Status{status}")
        self.expected = expected
        self.actual = actual
        super().__init__(f"{self.kind}: {message}")


class AmdQuantizedKernelError(AmdKernelError):
    pass


class AmdModelKernelError(AmdKernelError):
    pass


class AmdWeightError(AmdKernelError):
    pass


_SHUTTING_DOWN = [False]

# Live owners of library handles, released in rank order at exit: serving
# dispatchers, then decoders, KV caches, weights / kernels / GGUF files, and
# contexts last (each destroy may synchronise its context's stream).
RANK_DISPATCHER, RANK_DECODER, RANK_CACHE, RANK_RESOURCE, RANK_CONTEXT = range(5)
_OWNERS = weakref.WeakSet()


def _own(obj, rank: int):
    obj._release_rank = rank
    _OWNERS.add(obj)


def _release_all():
    """Runs at exit before interpreter finalization, while torch and the HIP
    runtime are whole. Owners held only by reference cycles (a frame kept by
    an exception's traceback, say) would otherwise survive to the runtime's
    own teardown with live graphs, events, streams and pinned memory, which is
    not ordered against this library's code objects. The collection finalizes
    those; every owner still referenced is then released in rank order. After
    this, finalizers no longer call into the library."""
    gc.collect()
    for obj in sorted(list(_OWNERS), key=lambda o: o._release_rank):
        try:
            obj.close()
        except Exception:
            pass
    _SHUTTING_DOWN[0] = True


atexit.register(_release_all)


def _live() -> bool:
    return not _SHUTTING_DOWN[0]


def _check(status: int, cls=AmdQuantizedKernelError):
    if status != 0:
        err = _lib.last_error()
        raise cls(status, int(err.expected), int(err.actual), err.message.decode(errors="replace"))


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


class AmdContext:
    """A device plus the stream every launch of this context is ordered on."""

    def __init__(self, device: int = 0, stream=None, own_stream: bool = False):
        lib = _lib.load()
        handle = ctypes.c_void_p()
        if own_stream:
            _check(lib.ribn_amd_context_create(device, ctypes.byref(handle)))
        else:
            if stream is None:
                import torch
                stream = torch.cuda.current_stream(device)
            raw = getattr(stream, "cuda_stream", stream)
            _check(lib.ribn_amd_context_wrap_stream(device, ctypes.c_void_p(raw), ctypes.byref(handle)))
        self._lib = lib
        self.handle = handle
        self.device = device
        _own(self, RANK_CONTEXT)

    def synchronize(self):
        _check(self._lib.ribn_amd_context_synchronize(self.handle))

    def reserve_prefill(self, max_tokens: int, max_k: int, max_n: int = 0):
        """Set-up call: device workspace for prefill of up to max_tokens x max_k
        activations and split-K room for [max_tokens][max_n] outputs."""
        _check(self._lib.ribn_amd_context_reserve_prefill(self.handle, max_tokens, max_k, max_n))

    def close(self):
        if self.handle and _live():
            self._lib.ribn_amd_context_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class AmdQuantizedWeight:
    """One opaque block-encoded tensor in device memory (CudaQuantizedWeight)."""

    def __init__(self, ctx: AmdContext, handle, name: str, dims, value_type: int):
        self.ctx = ctx
        self.handle = handle
        _own(self, RANK_RESOURCE)
        self.name = name
        self.dims = tuple(dims)
        self._value_type = value_type

    def value_type(self) -> int:
        return self._value_type

    def encoded_bytes(self) -> int:
        return int(self.ctx._lib.ribn_amd_weight_encoded_bytes(self.handle))

    def device_ptr(self) -> int:
        return int(self.ctx._lib.ribn_amd_weight_device_ptr(self.handle) or 0)

    def close(self):
        if self.handle and _live():
            self.ctx._lib.ribn_amd_weight_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class AmdWeightStore:
    """Backend-owned store of opaque encoded tensors (CudaWeightStore)."""

    def __init__(self, ctx: AmdContext):
        self.ctx = ctx
        self.quantized_tensors: dict[str, AmdQuantizedWeight] = {}

    def materialize_quantized(self, name: str, dims, value_type: int, encoded) -> tuple:
        """Uploads `encoded` (bytes / numpy uint8 / CUDA uint8 tensor) for GGML dims [K, N]."""
        if name in self.quantized_tensors:
            raise AmdWeightError(0, 0, 0, f"DuplicateTensor: {name}")
        if len(dims) != 2:
            raise AmdQuantizedKernelError(3, 2, len(dims), f"expected rank-2 tensor, got rank {len(dims)}")
        k, n = int(dims[0]), int(dims[1])
        lib = self.ctx._lib
        handle = ctypes.c_void_p()
        if hasattr(encoded, "is_cuda") and encoded.is_cuda:
            nbytes = encoded.numel() * encoded.element_size()
            st = lib.ribn_amd_weight_wrap_device(self.ctx.handle, value_type, k, n, _ptr(encoded), nbytes,
                                                 ctypes.byref(handle))
            keep = encoded
        else:
            import numpy as np
            arr = np.ascontiguousarray(np.frombuffer(bytes(encoded), np.uint8) if isinstance(
                encoded, (bytes, bytearray)) else encoded, dtype=np.uint8)
            st = lib.ribn_amd_weight_materialize(self.ctx.handle, value_type, k, n,
                                                 arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes,
                                                 ctypes.byref(handle))
            keep = None
        _check(st, AmdWeightError)
        w = AmdQuantizedWeight(self.ctx, handle, name, dims, value_type)
        w._keep = keep
        self.quantized_tensors[name] = w
        return (name, tuple(dims))

    def materialize_quantized_reader(self, name: str, dims, value_type: int, encoded_bytes: int, reader):
        """Streams from a file-like `reader` (the reference's `&mut impl Read`)."""
        lib = self.ctx._lib

        def read(_user, buf, cap):
            try:
                data = reader.read(cap)
            except Exception:
                return -1
            ctypes.memmove(buf, data, len(data))
            return len(data)

        cb = _lib.READ_FN(read)
        handle = ctypes.c_void_p()
        st = lib.ribn_amd_weight_materialize_reader(self.ctx.handle, value_type, int(dims[0]), int(dims[1]),
                                                    encoded_bytes, cb, None, ctypes.byref(handle))
        _check(st, AmdWeightError)
        w = AmdQuantizedWeight(self.ctx, handle, name, dims, value_type)
        self.quantized_tensors[name] = w
        return (name, tuple(dims))

    def quantized_tensor(self, name: str):
        return self.quantized_tensors.get(name)

    def copy_quantized_to_host(self, name: str) -> bytes:
        w = self.quantized_tensors.get(name)
        if w is None:
            raise AmdWeightError(0, 0, 0, f"MissingTensor: {name}")
        n = w.encoded_bytes()
        buf = (ctypes.c_uint8 * n)()
        _check(self.ctx._lib.ribn_amd_weight_copy_to_host(self.ctx.handle, w.handle, buf, n), AmdWeightError)
        return bytes(buf)


class _AmdQuantizedGemv:
    VALUE_TYPE = 0

    def __init__(self, ctx: AmdContext, value_type: int):
        self.ctx = ctx
        self._lib = ctx._lib
        self.handle = ctypes.c_void_p()
        _check(self._lib.ribn_amd_gemv_create(ctx.handle, value_type, ctypes.byref(self.handle)))
        _own(self, RANK_RESOURCE)

    @classmethod
    def from_context(cls, ctx: AmdContext):
        return cls(ctx, cls.VALUE_TYPE)

    @classmethod
    def new(cls, device: int = 0):
        return cls(AmdContext(device), cls.VALUE_TYPE)

    def value_type(self) -> int:
        return int(self._lib.ribn_amd_gemv_value_type(self.handle))

    def set_mode(self, mode: int):
        """GEMV_WARP (f32 activations, default) or GEMV_FIXED16 (opt-in, lossy)."""
        _check(self._lib.ribn_amd_gemv_set_mode(self.handle, mode))

    def mode(self) -> int:
        return int(self._lib.ribn_amd_gemv_mode(self.handle))

    def execute(self, weight, input, output):
        _check(self._lib.ribn_amd_gemv_execute(self.handle, weight.handle, _ptr(input), input.numel(),
                                               _ptr(output), output.numel()))

    def execute_warp(self, weight, input, output):
        _check(self._lib.ribn_amd_gemv_execute_warp(self.handle, weight.handle, _ptr(input), input.numel(),
                                                    _ptr(output), output.numel()))

    def execute_warp_batch(self, weight, input, output, members: int):
        _check(self._lib.ribn_amd_gemv_execute_warp_batch(self.handle, weight.handle, _ptr(input), input.numel(),
                                                          _ptr(output), output.numel(), members))

    def execute_rms_norm(self, weight, input, gamma, epsilon: float, output, members: int = 1):
        _check(self._lib.ribn_amd_gemv_execute_rms_norm(self.handle, weight.handle, _ptr(input), input.numel(),
                                                        _ptr(gamma), gamma.numel(), epsilon, _ptr(output),
                                                        output.numel(), members))

    def execute_group(self, weights, input, outputs, members: int = 1, gamma=None, epsilon: float = 1e-6):
        """One launch over weights sharing `input` (optionally RMSNorm-fused)."""
        n = len(weights)
        wh = (ctypes.c_void_p * n)(*[w.handle.value for w in weights])
        oh = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outputs])
        ol = (ctypes.c_size_t * n)(*[o.numel() for o in outputs])
        g = _ptr(gamma) if gamma is not None else None
        gl = gamma.numel() if gamma is not None else 0
        _check(self._lib.ribn_amd_gemv_execute_group(self.handle, wh, n, _ptr(input), input.numel(), g, gl,
                                                     epsilon, oh, ol, members))

    def execute_fused(self, weight, input, output, members: int = 1, up=None, gamma=None, epsilon: float = 1e-6,
                      accumulate: bool = False):
        """execute_warp_batch with the decode step's neighbours fused: `up` given,
        the activation is silu(input) * up; `accumulate`, output += W x; `gamma`
        given, the RMSNorm prologue."""
        flags = (1 if up is not None else 0) | (2 if accumulate else 0)
        g = _ptr(gamma) if gamma is not None else None
        gl = gamma.numel() if gamma is not None else 0
        u = _ptr(up) if up is not None else None
        _check(self._lib.ribn_amd_gemv_execute_fused(self.handle, weight.handle, _ptr(input), u, input.numel(), g,
                                                     gl, epsilon, _ptr(output), output.numel(), members, flags))

    def execute_gate_up_swiglu(self, gate, up, input, output, members: int = 1, gamma=None, epsilon: float = 1e-6):
        """output = silu(gate x') * (up x') in one launch (x' = RMSNorm(input) when gamma is given)."""
        g = _ptr(gamma) if gamma is not None else None
        gl = gamma.numel() if gamma is not None else 0
        _check(self._lib.ribn_amd_gemv_execute_gate_up_swiglu(self.handle, gate.handle, up.handle, _ptr(input),
                                                              input.numel(), g, gl, epsilon, _ptr(output),
                                                              output.numel(), members))

    def gemm_prefill(self, weight, input, output, members: int, gamma=None, epsilon: float = 1e-6):
        """y[members][N] = x[members][K] W^T on the matrix cores; x is f32 or bf16.
        Needs AmdContext.reserve_prefill(members, K) beforehand."""
        import torch
        dtype = {torch.float32: 0, torch.bfloat16: 1}.get(input.dtype)
        if dtype is None:
            raise TypeError(f"prefill input must be float32 or bfloat16, got {input.dtype}")
        g = _ptr(gamma) if gamma is not None else None
        gl = gamma.numel() if gamma is not None else 0
        _check(self._lib.ribn_amd_gemm_prefill(self.handle, weight.handle, _ptr(input), dtype, input.numel(), members,
                                               g, gl, epsilon, _ptr(output), output.numel()))

    def dequantize(self, weight, output):
        _check(self._lib.ribn_amd_dequantize(self.handle, weight.handle, _ptr(output), output.numel()))

    def close(self):
        if self.handle and _live():
            self._lib.ribn_amd_gemv_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class AmdQ8_1Quantizer:
    """CudaQ8_1Quantizer (crates/nvidia/src/activation.rs:8-88): packs f32
    activations into Q8_1 blocks (nine uint32 words per 32 values) on the
    context stream, into caller-owned storage."""

    def __init__(self, ctx: AmdContext):
        self.ctx = ctx
        self._lib = ctx._lib

    @classmethod
    def new(cls, ctx: AmdContext):
        return cls(ctx)

    def execute(self, input, output):
        _check(self._lib.ribn_amd_q8_1_quantize(self.ctx.handle, _ptr(input), input.numel(), _ptr(output),
                                                output.numel()))


class _AmdQ8_1Gemv:
    """CudaQ4KQ8_1Gemv / CudaQ5KQ8_1Gemv / CudaQ6KQ8_1Gemv (q{4,5,6}_q8_1.rs):
    the integer-dot GEMV over Q8_1-packed activations (uint32 tensors)."""
    VALUE_TYPE = 0

    def __init__(self, ctx: AmdContext):
        self._gemv = _AmdQuantizedGemv(ctx, self.VALUE_TYPE)
        self.ctx = ctx
        self._lib = ctx._lib

    @classmethod
    def new(cls, ctx: AmdContext):
        return cls(ctx)

    def execute(self, weight, input, output):
        _check(self._lib.ribn_amd_gemv_execute_q8_1(self._gemv.handle, weight.handle, _ptr(input), input.numel(),
                                                    _ptr(output), output.numel()))

    def execute_batch(self, weight, input, output, members: int):
        _check(self._lib.ribn_amd_gemv_execute_q8_1_batch(self._gemv.handle, weight.handle, _ptr(input),
                                                          input.numel(), _ptr(output), output.numel(), members))


class AmdQ4KQ8_1Gemv(_AmdQ8_1Gemv):
    VALUE_TYPE = Q4_K


class AmdQ5KQ8_1Gemv(_AmdQ8_1Gemv):
    VALUE_TYPE = Q5_K


class AmdQ6KQ8_1Gemv(_AmdQ8_1Gemv):
    VALUE_TYPE = Q6_K


class AmdQ4KGemv(_AmdQuantizedGemv):
    VALUE_TYPE = Q4_K


class AmdQ5KGemv(_AmdQuantizedGemv):
    VALUE_TYPE = Q5_K


class AmdQ6KGemv(_AmdQuantizedGemv):
    VALUE_TYPE = Q6_K


class _AmdEmbedding:
    """Gather of dequantised table rows (CudaQ4KEmbedding, quantized.rs:913-1160)."""

    VALUE_TYPE = Q4_K

    def __init__(self, ctx: AmdContext, value_type: int):
        self.ctx = ctx
        self._lib = ctx._lib
        self.handle = ctypes.c_void_p()
        _check(self._lib.ribn_amd_embedding_create(ctx.handle, value_type, ctypes.byref(self.handle)))
        _own(self, RANK_RESOURCE)

    @classmethod
    def from_context(cls, ctx: AmdContext):
        return cls(ctx, cls.VALUE_TYPE)

    @classmethod
    def new(cls, device: int = 0):
        return cls(AmdContext(device), cls.VALUE_TYPE)

    def execute(self, weight, token_index: int, output):
        _check(self._lib.ribn_amd_embedding_execute(self.handle, weight.handle, int(token_index), _ptr(output),
                                                    output.numel()))

    def execute_batch(self, weight, token_indices, output):
        """token_indices: device tensor of 32-bit token ids, one per member."""
        members = token_indices.numel()
        tok = _ptr(token_indices) if members else None
        _check(self._lib.ribn_amd_embedding_execute_batch(self.handle, weight.handle, tok, members, _ptr(output),
                                                          output.numel()))

    def close(self):
        if self.handle and _live():
            self._lib.ribn_amd_embedding_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class AmdQ4KEmbedding(_AmdEmbedding):
    VALUE_TYPE = Q4_K


class AmdKQuantEmbedding(_AmdEmbedding):
    """Embedding gather for any served k-quant type (Q4_K / Q5_K / Q6_K tables)."""

    @classmethod
    def from_value_type(cls, ctx: AmdContext, value_type: int):
        return cls(ctx, value_type)


class QwenGemvKernel:
    """Per-GGML-type kernel selection (staging.rs:90-217)."""

    _FAMILIES = {Q4_K: AmdQ4KGemv, Q5_K: AmdQ5KGemv, Q6_K: AmdQ6KGemv}

    @classmethod
    def from_value_type(cls, ctx: AmdContext, value_type: int) -> _AmdQuantizedGemv:
        fam = cls._FAMILIES.get(value_type)
        if fam is None:
            # the C ABI reports UnsupportedValueType with expected/actual
            return _AmdQuantizedGemv(ctx, value_type)
        return fam.from_context(ctx)


class AmdQwenOps:
    """RMSNorm operators of CudaQwen35Ops (model_ops.rs:1714-1824)."""

    def __init__(self, ctx: AmdContext):
        self.ctx = ctx
        self._lib = ctx._lib

    @classmethod
    def from_context(cls, ctx: AmdContext):
        return cls(ctx)

    def rms_norm(self, input, weight, output, epsilon: float):
        _check(self._lib.ribn_amd_rms_norm(self.ctx.handle, _ptr(input), input.numel(), _ptr(weight),
                                           weight.numel(), _ptr(output), output.numel(), epsilon),
               AmdModelKernelError)

    def rms_norm_batch(self, input, weight, output, length: int, epsilon: float):
        _check(self._lib.ribn_amd_rms_norm_batch(self.ctx.handle, _ptr(input), input.numel(), _ptr(weight),
                                                 weight.numel(), _ptr(output), output.numel(), length,
                                                 epsilon), AmdModelKernelError)

    def argmax_into(self, logits, selected):
        """argmax_into (model_ops.rs:1583-1620): selected[0] = greedy index of logits."""
        _check(self._lib.ribn_amd_argmax(self.ctx.handle, _ptr(logits), logits.numel(), logits.numel(),
                                         _ptr(selected)), AmdModelKernelError)

    def argmax_into_batch(self, logits, length: int, selected):
        """argmax_into_batch (model_ops.rs:1634-1674): one selection per row of `length`."""
        _check(self._lib.ribn_amd_argmax(self.ctx.handle, _ptr(logits), logits.numel(), length, _ptr(selected)),
               AmdModelKernelError)


def validate_quantized_geometry(kernel_value_type: int, weight_value_type: int, dims, encoded_bytes: int):
    """Host-only geometry check (quantized.rs:1755-1804); returns (K, N) or raises."""
    lib = _lib.load()
    arr = (ctypes.c_uint64 * max(1, len(dims)))(*[int(d) for d in dims])
    k = ctypes.c_uint64()
    n = ctypes.c_uint64()
    _check(lib.ribn_amd_validate_quantized_geometry(kernel_value_type, weight_value_type, arr, len(dims),
                                                    encoded_bytes, ctypes.byref(k), ctypes.byref(n)))
    return k.value, n.value

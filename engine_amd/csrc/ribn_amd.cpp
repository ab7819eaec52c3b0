// Host side of the C ABI declared in include/ribn_amd.h: contexts, the opaque
// weight store, validation that mirrors the reference's operator wrappers
// (crates/nvidia/src/quantized.rs, model_ops.rs, cuda.rs) and kernel dispatch.
#include "ribn_amd.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <limits>
#include <functional>
#include <mutex>
#include <new>
#include <vector>

#include "abi_internal.hpp"
#include "decode_launch.hpp"
#include "kquant_launch.hpp"

namespace ribn_amd_abi {

thread_local ribn_amd_error g_last_error = {RIBN_AMD_OK, 0, 0, {0}};

ribn_amd_status fail(ribn_amd_status status, uint64_t expected, uint64_t actual, const char* fmt, ...) {
    g_last_error.status = status;
    g_last_error.expected = expected;
    g_last_error.actual = actual;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error.message, sizeof g_last_error.message, fmt, ap);
    va_end(ap);
    return status;
}

ribn_amd_status ok() {
    g_last_error.status = RIBN_AMD_OK;
    g_last_error.expected = 0;
    g_last_error.actual = 0;
    g_last_error.message[0] = 0;
    return RIBN_AMD_OK;
}

ribn_amd_status driver(hipError_t e, const char* what) {
    if (e == hipErrorNoBinaryForGpu || e == hipErrorInvalidImage || e == hipErrorInvalidDeviceFunction) {
        return fail(RIBN_AMD_MODULE, 0, 0, "%s: no gfx950 code object for this device (%s)", what,
                    hipGetErrorString(e));
    }
    return fail(RIBN_AMD_DRIVER, 0, 0, "%s: %s", what, hipGetErrorString(e));
}

const char* type_label(uint32_t t) {
    switch (t) {
    case RIBN_AMD_Q4_K: return "Q4_K";
    case RIBN_AMD_Q5_K: return "Q5_K";
    case RIBN_AMD_Q6_K: return "Q6_K";
    default: return "unsupported";
    }
}

uint64_t block_bytes(uint32_t t) {
    switch (t) {
    case RIBN_AMD_Q4_K: return 144;
    case RIBN_AMD_Q5_K: return 176;
    case RIBN_AMD_Q6_K: return 210;
    default: return 0;
    }
}

bool supported(uint32_t t) { return block_bytes(t) != 0; }

// The ContextMismatch check of quantized.rs:260-266 for raw device pointers:
// the buffer must be device (or managed) memory of the context's device.
ribn_amd_status check_device_ptr(const ribn_amd_context* ctx, const void* ptr, const char* what, uintptr_t align) {
    if (ptr == nullptr) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "%s is null", what);
    if ((reinterpret_cast<uintptr_t>(ptr) & (align - 1)) != 0) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, align, reinterpret_cast<uintptr_t>(ptr) & (align - 1),
                    "%s must be %u-byte aligned", what, (unsigned)align);
    }
    hipPointerAttribute_t attr;
    hipError_t e = hipPointerGetAttributes(&attr, ptr);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "%s is not a device allocation (%s)", what,
                    hipGetErrorString(e));
    }
    if (attr.type != hipMemoryTypeDevice && attr.type != hipMemoryTypeManaged) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "%s is not device memory", what);
    }
    if (attr.device != ctx->device) {
        return fail(RIBN_AMD_CONTEXT_MISMATCH, (uint64_t)ctx->device, (uint64_t)attr.device,
                    "%s belongs to device %d, the context to device %d", what, attr.device, ctx->device);
    }
    return RIBN_AMD_OK;
}

ribn_amd_status validate_geometry(uint32_t kernel_type, const ribn_amd_quantized_weight* w, uint64_t* k,
                                  uint64_t* n) {
    const uint64_t dims[2] = {w->input_size, w->output_size};
    return ribn_amd_validate_quantized_geometry(kernel_type, w->value_type, dims, 2, w->encoded_bytes, k, n);
}

// quantized.rs:252-355 validate / validate_batch, in the reference's order:
// contexts, geometry, input length, output length.
ribn_amd_status validate_launch(const ribn_amd_gemv* g, const ribn_amd_quantized_weight* w, const float* in,
                                size_t in_len, const float* out, size_t out_len, size_t members, uint64_t* k,
                                uint64_t* n) {
    if (g == nullptr || w == nullptr) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null kernel or weight handle");
    if (w->ctx->device != g->ctx->device) {
        return fail(RIBN_AMD_CONTEXT_MISMATCH, (uint64_t)g->ctx->device, (uint64_t)w->ctx->device,
                    "weight and kernel belong to different devices");
    }
    ribn_amd_status st = check_device_ptr(g->ctx, in, "input");
    if (st != RIBN_AMD_OK) return st;
    st = check_device_ptr(g->ctx, out, "output");
    if (st != RIBN_AMD_OK) return st;
    st = validate_geometry(g->value_type, w, k, n);
    if (st != RIBN_AMD_OK) return st;
    if (members != 0 && *k > std::numeric_limits<size_t>::max() / members) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "input size overflows");
    }
    if (members != 0 && *n > std::numeric_limits<size_t>::max() / members) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "output size overflows");
    }
    const uint64_t expected_in = *k * members;
    const uint64_t expected_out = *n * members;
    if (in_len != expected_in) {
        return fail(RIBN_AMD_INPUT_LENGTH, expected_in, in_len,
                    "quantized GEMV input has %zu values, expected %llu", in_len,
                    (unsigned long long)expected_in);
    }
    if (out_len != expected_out) {
        return fail(RIBN_AMD_OUTPUT_LENGTH, expected_out, out_len,
                    "quantized GEMV output has %zu values, expected %llu", out_len,
                    (unsigned long long)expected_out);
    }
    if (members > (size_t)std::numeric_limits<int>::max()) return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "members overflow");
    return RIBN_AMD_OK;
}

ribn_amd_status validate_members(const ribn_amd_gemv* g, size_t members) {
    // quantized.rs:458-469: zero members is an input-length error, too many an
    // invalid-weight error naming the family.
    if (members == 0) return fail(RIBN_AMD_INPUT_LENGTH, 1, 0, "batched GEMV needs at least one member");
    if (members > RIBN_AMD_MAX_BATCH_MEMBERS) {
        return fail(RIBN_AMD_INVALID_WEIGHT, RIBN_AMD_MAX_BATCH_MEMBERS, members,
                    "%s batched GEMV supports at most %u members", g ? type_label(g->value_type) : "?",
                    RIBN_AMD_MAX_BATCH_MEMBERS);
    }
    return RIBN_AMD_OK;
}

// Runs a (grouped) wave GEMV over `count` weights sharing one activation
// vector. Members are split into launch groups that fit the LDS staging of K.
ribn_amd_status launch_wave_group(ribn_amd_gemv* g, const ribn_amd_quantized_weight* const* ws, size_t count,
                                  const float* in, const float* gamma, float eps, float* const* outs, uint64_t k,
                                  size_t members, const float* up = nullptr, bool accumulate = false) {
    DeviceGuard guard(g->ctx->device);
    int per_launch = std::min(ribn_amd::wave_max_members((int)k), ribn_amd::kWaveMaxMembers);
    if (up != nullptr) per_launch = std::min(per_launch, ribn_amd::kSwigluMaxMembers);
    int arith = arith_of_mode(g->mode);
    uint64_t total_rows = 0;
    for (size_t i = 0; i < count; ++i) total_rows += ws[i]->output_size;
    if (per_launch <= 0 && gamma == nullptr && up == nullptr && total_rows <= (uint64_t)INT32_MAX &&
        ribn_amd::f32_long_k_members((int)k, (int)total_rows) > 0) {
        // K beyond what one workgroup stages (e.g. the 17408-wide down
        // projection of the reference's 27B shapes): the f32 GEMV's
        // slice-split form, in either mode
        arith = ribn_amd::kArithF32;
        per_launch = 1;
    }
    if (per_launch <= 0) {
        // K too large for every staged form: the exact-order kernel still serves it.
        if (gamma != nullptr || up != nullptr || accumulate) {
            return fail(RIBN_AMD_SHAPE_OVERFLOW, (uint64_t)ribn_amd::kWaveMaxK, k, "fused GEMV forms support K up to %d",
                        ribn_amd::kWaveMaxK);
        }
        for (size_t i = 0; i < count; ++i) {
            hipError_t e = ribn_amd::launch_gemv_exact((int)g->value_type, ws[i]->data,
                                                       (uint32_t)ws[i]->encoded_bytes, in, outs[i], (int)k,
                                                       (int)ws[i]->output_size, (int)members, g->ctx->stream);
            if (e != hipSuccess) return driver(e, "launch exact GEMV");
        }
        return ok();
    }
    per_launch = ribn_amd::gemv_launch_members((int)g->value_type, (int)k, up != nullptr, arith);
    if (per_launch <= 0) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, (uint64_t)ribn_amd::kWaveMaxK, k, "no GEMV form serves K = %llu",
                    (unsigned long long)k);
    }
    for (size_t m0 = 0; m0 < members; m0 += (size_t)per_launch) {
        const size_t mc = std::min<size_t>((size_t)per_launch, members - m0);
        ribn_amd::WaveGemvArgs a{};
        int rows = 0;
        for (size_t i = 0; i < count; ++i) {
            const uint64_t n = ws[i]->output_size;
            a.w[i] = ws[i]->data;
            a.wbytes[i] = (uint32_t)ws[i]->encoded_bytes;
            a.y[i] = outs[i] + m0 * n;
            rows += (int)n;
            a.rows_end[i] = rows;
        }
        a.count = (int)count;
        a.total_rows = rows;
        a.x = in + m0 * k;
        a.x2 = up != nullptr ? up + m0 * k : nullptr;
        a.accumulate = accumulate ? 1 : 0;
        a.gamma = gamma;
        a.eps = eps;
        a.K = (int)k;
        a.members = (int)mc;
        a.arith = arith;
        hipError_t e = ribn_amd::launch_gemv((int)g->value_type, a, g->ctx->act_scratch, g->ctx->cu_count,
                                             g->ctx->stream);
        if (e != hipSuccess) return driver(e, "launch GEMV");
    }
    return ok();
}

ribn_amd_status launch_batched(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w, const float* in,
                               const float* gamma, float eps, float* out, uint64_t k, uint64_t /*n*/,
                               size_t members) {
    const ribn_amd_quantized_weight* ws[1] = {w};
    float* outs[1] = {out};
    return launch_wave_group(g, ws, 1, in, gamma, eps, outs, k, members);
}

ribn_amd_status check_epsilon(float epsilon) {
    if (!(epsilon > 0.f) || epsilon == std::numeric_limits<float>::infinity()) {
        return fail(RIBN_AMD_INVALID_EPSILON, 0, 0, "RMSNorm epsilon must be finite and positive");
    }
    return RIBN_AMD_OK;
}

// ---- device scratch of the allocation-free prefill (ribn_amd_gemm_prefill_static)
//
// One file-scope array per device, resolved to its device address once per
// device (when a context is created there, else on the entry point's first
// call). Every call on a device shares it; calls on different streams are
// ordered through a per-device event (see order_static_call).
constexpr size_t kStaticScratchBytes = (size_t)8 << 20;
constexpr int kStaticScratchDevices = 64;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
static std::mutex g_scratch_mutex;
static void* g_scratch_ptr[kStaticScratchDevices];  // device address of `scratch` per device
static hipEvent_t g_scratch_done[kStaticScratchDevices];  // the last uncaptured call's completion per device

// With `device` current: looks up the device address of `scratch` (once).
ribn_amd_status resolve_static_scratch(int device) {
    if (device < 0 || device >= kStaticScratchDevices) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, kStaticScratchDevices, (uint64_t)device,
                    "device %d is beyond the %d devices the static scratch table covers", device,
                    kStaticScratchDevices);
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[device] != nullptr) return RIBN_AMD_OK;
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return driver(e, "hipGetSymbolAddress(scratch)");
    if (ptr == nullptr) return fail(RIBN_AMD_DRIVER, 0, 0, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_ptr[device] = ptr;
    return RIBN_AMD_OK;
}

void* static_scratch(int device) {
    if (device < 0 || device >= kStaticScratchDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    return g_scratch_ptr[device];
}

// With `device` current, ahead of a call's launches on `stream`: makes the
// stream wait for the previous uncaptured call on this device (whatever its
// stream), then records this call's completion after `launch` has enqueued
// its kernels, so calls from several streams or contexts take the array in
// turn. A stream under graph capture is left alone: the graph's own order
// (and the caller's order of its replays against other calls) decides.
// The event wait and record allocate nothing.
ribn_amd_status order_static_call(int device, hipStream_t stream, const std::function<hipError_t()>& launch) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(stream, &cap);
    if (e != hipSuccess) return driver(e, "hipStreamIsCapturing");
    if (cap != hipStreamCaptureStatusNone) {
        e = launch();
        return e == hipSuccess ? RIBN_AMD_OK : driver(e, "launch allocation-free prefill");
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    hipEvent_t& done = g_scratch_done[device];
    if (done == nullptr) {
        e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
        if (e != hipSuccess) {
            done = nullptr;
            return driver(e, "hipEventCreateWithFlags");
        }
    } else {
        e = hipStreamWaitEvent(stream, done, 0);
        if (e != hipSuccess) return driver(e, "hipStreamWaitEvent");
    }
    e = launch();
    if (e != hipSuccess) return driver(e, "launch allocation-free prefill");
    e = hipEventRecord(done, stream);
    return e == hipSuccess ? RIBN_AMD_OK : driver(e, "hipEventRecord");
}

ribn_amd_status new_context(int device, hipStream_t stream, bool owns, ribn_amd_context** out) {
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return driver(e, "hipGetDeviceProperties");
    void* ctx_scratch = nullptr;
    const size_t act_bytes = (ribn_amd::gemv_act_scratch_bytes() + 255) / 256 * 256;
    {
        DeviceGuard guard(device);
        // Resolved here when it can be; a failure only concerns the
        // allocation-free entry point, which tries again and reports it.
        (void)resolve_static_scratch(device);
        e = hipMalloc(&ctx_scratch, act_bytes + RIBN_AMD_MAX_BATCH_MEMBERS * sizeof(ribn_amd::AttnMember));
        if (e != hipSuccess) return driver(e, "hipMalloc context scratch");
    }
    auto* ctx = new (std::nothrow) ribn_amd_context{device,  stream,  owns, prop.multiProcessorCount,
                                                    nullptr, 0,       ctx_scratch,
                                                    static_cast<char*>(ctx_scratch) + act_bytes};
    if (!ctx) {
        DeviceGuard guard(device);
        hipFree(ctx_scratch);
        return fail(RIBN_AMD_DRIVER, 0, 0, "host allocation failed");
    }
    *out = ctx;
    return ok();
}

}  // namespace ribn_amd_abi

using namespace ribn_amd_abi;

namespace {

// Argument checks of the prefill entry points, in the order of the other
// execute calls (quantized.rs:1755-1804), then the prefill limits.
ribn_amd_status validate_prefill(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w, const void* input,
                                 uint32_t input_dtype, size_t input_len, size_t members, const float* gamma,
                                 size_t gamma_len, float epsilon, float* output, size_t output_len, uint64_t* k_out,
                                 uint64_t* n_out) {
    if (input_dtype != RIBN_AMD_F32 && input_dtype != RIBN_AMD_BF16) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, RIBN_AMD_BF16, input_dtype, "input dtype %u is neither f32 nor bf16",
                    input_dtype);
    }
    uint64_t k, n;
    // Pointer checks take f32 alignment for either dtype; rows of bf16 input
    // are read one element at a time.
    ribn_amd_status st = validate_launch(g, w, static_cast<const float*>(input), input_len, output, output_len,
                                         members, &k, &n);
    if (st != RIBN_AMD_OK) return st;
    if (members == 0) return fail(RIBN_AMD_INPUT_LENGTH, 1, 0, "prefill needs at least one token");
    if (gamma != nullptr) {
        st = check_device_ptr(g->ctx, gamma, "gamma");
        if (st != RIBN_AMD_OK) return st;
        if (gamma_len != k) {
            return fail(RIBN_AMD_WEIGHT_LENGTH, k, gamma_len, "RMSNorm weight has %zu values, expected %llu",
                        gamma_len, (unsigned long long)k);
        }
        st = check_epsilon(epsilon);
        if (st != RIBN_AMD_OK) return st;
    }
    if (k > (uint64_t)ribn_amd::kGemmMaxK || members > (size_t)std::numeric_limits<int>::max() / k ||
        n > (uint64_t)std::numeric_limits<int>::max() || w->encoded_bytes > 0xffffffffull) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, (uint64_t)ribn_amd::kGemmMaxK, k,
                    "prefill supports K up to %d and tokens*K < 2^31", ribn_amd::kGemmMaxK);
    }
    *k_out = k;
    *n_out = n;
    return RIBN_AMD_OK;
}

}  // namespace

extern "C" {

ribn_amd_status ribn_amd_last_error(ribn_amd_error* out) {
    if (!out) return RIBN_AMD_INVALID_ARGUMENT;
    *out = g_last_error;
    return RIBN_AMD_OK;
}

const char* ribn_amd_status_name(int32_t status) {
    switch (status) {
    case RIBN_AMD_OK: return "Ok";
    case RIBN_AMD_DRIVER: return "Driver";
    case RIBN_AMD_MODULE: return "Module";
    case RIBN_AMD_INVALID_WEIGHT: return "InvalidWeight";
    case RIBN_AMD_UNSUPPORTED_VALUE_TYPE: return "UnsupportedValueType";
    case RIBN_AMD_SHAPE_OVERFLOW: return "ShapeOverflow";
    case RIBN_AMD_INPUT_LENGTH: return "InputLength";
    case RIBN_AMD_OUTPUT_LENGTH: return "OutputLength";
    case RIBN_AMD_CONTEXT_MISMATCH: return "ContextMismatch";
    case RIBN_AMD_EMPTY_INPUT: return "EmptyInput";
    case RIBN_AMD_WEIGHT_LENGTH: return "WeightLength";
    case RIBN_AMD_INVALID_EPSILON: return "InvalidEpsilon";
    case RIBN_AMD_INVALID_ARGUMENT: return "InvalidArgument";
    case RIBN_AMD_EMPTY_ENCODING: return "EmptyEncoding";
    case RIBN_AMD_SOURCE_INCOMPLETE: return "SourceIncomplete";
    case RIBN_AMD_WORKSPACE_TOO_SMALL: return "WorkspaceTooSmall";
    case RIBN_AMD_INVALID_PLAN: return "InvalidPlan";
    case RIBN_AMD_POSITION_OVERFLOW: return "PositionOverflow";
    case RIBN_AMD_MISSING_TENSOR: return "MissingTensor";
    case RIBN_AMD_GGUF_IO: return "Io";
    case RIBN_AMD_GGUF_INVALID_MAGIC: return "InvalidMagic";
    case RIBN_AMD_GGUF_UNSUPPORTED_VERSION: return "UnsupportedVersion";
    case RIBN_AMD_GGUF_INVALID_UTF8: return "InvalidUtf8";
    case RIBN_AMD_GGUF_INVALID_VALUE_TYPE: return "InvalidValueType";
    case RIBN_AMD_GGUF_INVALID_BOOL: return "InvalidBool";
    case RIBN_AMD_GGUF_INVALID_LENGTH: return "InvalidLength";
    case RIBN_AMD_GGUF_ARRAY_NESTING_TOO_DEEP: return "ArrayNestingTooDeep";
    case RIBN_AMD_GGUF_DUPLICATE_METADATA: return "DuplicateMetadata";
    case RIBN_AMD_GGUF_INVALID_DIMENSION_COUNT: return "InvalidDimensionCount";
    case RIBN_AMD_GGUF_INVALID_ALIGNMENT: return "InvalidAlignment";
    case RIBN_AMD_GGUF_TRUNCATED: return "Truncated";
    case RIBN_AMD_GGUF_TENSOR_OFFSET_OUT_OF_BOUNDS: return "TensorOffsetOutOfBounds";
    case RIBN_AMD_GGUF_UNSUPPORTED_TENSOR_TYPE: return "UnsupportedTensorType";
    case RIBN_AMD_GGUF_BYTE_LENGTH_OVERFLOW: return "TensorByteLengthOverflow";
    case RIBN_AMD_GGUF_QUANTIZATION_MISMATCH: return "QuantizationMismatch";
    case RIBN_AMD_GGUF_MISSING_METADATA: return "MissingMetadata";
    case RIBN_AMD_GGUF_METADATA_TYPE_MISMATCH: return "MetadataTypeMismatch";
    case RIBN_AMD_BUDGET_EXCEEDED: return "BudgetExceeded";
    case RIBN_AMD_UNSUPPORTED: return "Unsupported";
    case RIBN_AMD_EXECUTION_FAILED: return "ExecutionFailed";
    case RIBN_AMD_UNKNOWN_SUBMISSION: return "UnknownSubmission";
    case RIBN_AMD_DEVICE_FAULTED: return "DeviceFaulted";
    case RIBN_AMD_STATE_POSITION: return "StatePosition";
    default: return "Unknown";
    }
}

int32_t ribn_amd_abi_version(void) { return RIBN_AMD_ABI_VERSION; }

ribn_amd_status ribn_amd_context_create(int32_t device, ribn_amd_context** out) {
    if (!out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "out is null");
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return driver(e, "hipGetDeviceCount");
    if (device < 0 || device >= count) {
        return fail(RIBN_AMD_DRIVER, (uint64_t)count, (uint64_t)device, "device %d out of range (%d devices)",
                    device, count);
    }
    DeviceGuard guard(device);
    hipStream_t stream;
    e = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
    if (e != hipSuccess) return driver(e, "hipStreamCreateWithFlags");
    ribn_amd_status st = new_context(device, stream, true, out);
    if (st != RIBN_AMD_OK) hipStreamDestroy(stream);
    return st;
}

ribn_amd_status ribn_amd_context_wrap_stream(int32_t device, void* hip_stream, ribn_amd_context** out) {
    if (!out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "out is null");
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return driver(e, "hipGetDeviceCount");
    if (device < 0 || device >= count) {
        return fail(RIBN_AMD_DRIVER, (uint64_t)count, (uint64_t)device, "device %d out of range", device);
    }
    hipStream_t stream = static_cast<hipStream_t>(hip_stream);
    if (stream != nullptr) {
        hipDevice_t sdev;
        e = hipStreamGetDevice(stream, &sdev);
        if (e == hipSuccess && sdev != device) {
            return fail(RIBN_AMD_CONTEXT_MISMATCH, (uint64_t)device, (uint64_t)sdev,
                        "stream belongs to device %d, not %d", sdev, device);
        }
    }
    return new_context(device, stream, false, out);
}

void ribn_amd_context_destroy(ribn_amd_context* ctx) {
    if (!ctx) return;
    context_release(ctx);
}

extern "C++" {
namespace ribn_amd_abi {

void context_retain(ribn_amd_context* ctx) { ctx->refs.fetch_add(1, std::memory_order_relaxed); }

void context_release(ribn_amd_context* ctx) {
    if (ctx->refs.fetch_sub(1, std::memory_order_acq_rel) != 1) return;
    DeviceGuard guard(ctx->device);
    if (ctx->workspace || ctx->act_scratch) hipStreamSynchronize(ctx->stream);
    if (ctx->workspace) hipFree(ctx->workspace);
    if (ctx->act_scratch) hipFree(ctx->act_scratch);
    if (ctx->owns_stream) {
        hipStreamSynchronize(ctx->stream);
        hipStreamDestroy(ctx->stream);
    }
    delete ctx;
}

}  // namespace ribn_amd_abi
}  // extern "C++"

size_t ribn_amd_gemm_workspace_bytes(size_t tokens, size_t k, size_t n) {
    return ribn_amd::gemm_workspace_bytes(tokens, k, n);
}

ribn_amd_status ribn_amd_context_reserve_prefill(ribn_amd_context* ctx, size_t max_tokens, size_t max_k,
                                                 size_t max_n) {
    if (!ctx) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null context");
    if (max_n > (size_t)std::numeric_limits<int>::max()) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, (uint64_t)std::numeric_limits<int>::max(), max_n, "max_n overflows");
    }
    if (max_tokens == 0 || max_k == 0 || max_k > (size_t)ribn_amd::kGemmMaxK || max_k % 256 != 0 ||
        max_tokens > (size_t)std::numeric_limits<int>::max() / max_k) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, (uint64_t)ribn_amd::kGemmMaxK, max_k,
                    "prefill workspace needs 1 <= tokens, K a multiple of 256 up to %d, tokens*K < 2^31",
                    ribn_amd::kGemmMaxK);
    }
    const size_t need = ribn_amd::gemm_workspace_bytes(max_tokens, max_k, max_n);
    if (need <= ctx->workspace_bytes) return ok();
    DeviceGuard guard(ctx->device);
    if (ctx->workspace) {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) return driver(e, "hipStreamSynchronize");
        hipFree(ctx->workspace);
        ctx->workspace = nullptr;
        ctx->workspace_bytes = 0;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, need);
    if (e != hipSuccess) return driver(e, "hipMalloc prefill workspace");
    ctx->workspace = p;
    ctx->workspace_bytes = need;
    return ok();
}

ribn_amd_status ribn_amd_context_synchronize(ribn_amd_context* ctx) {
    if (!ctx) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null context");
    DeviceGuard guard(ctx->device);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return driver(e, "hipStreamSynchronize");
    return ok();
}

void* ribn_amd_context_stream(const ribn_amd_context* ctx) { return ctx ? (void*)ctx->stream : nullptr; }
int32_t ribn_amd_context_device(const ribn_amd_context* ctx) { return ctx ? ctx->device : -1; }

ribn_amd_status ribn_amd_alloc(ribn_amd_context* ctx, size_t bytes, void** out) {
    if (!ctx || !out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    DeviceGuard guard(ctx->device);
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) return driver(e, "hipMalloc");
    e = hipMemsetAsync(p, 0, bytes ? bytes : 1, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        hipFree(p);
        return driver(e, "zero-fill");
    }
    *out = p;
    return ok();
}

ribn_amd_status ribn_amd_free(ribn_amd_context* ctx, void* ptr) {
    if (!ctx) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null context");
    DeviceGuard guard(ctx->device);
    hipError_t e = hipFree(ptr);
    if (e != hipSuccess) return driver(e, "hipFree");
    return ok();
}

ribn_amd_status ribn_amd_memcpy_htod(ribn_amd_context* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    DeviceGuard guard(ctx->device);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return driver(e, "host-to-device copy");
    return ok();
}

ribn_amd_status ribn_amd_memcpy_dtoh(ribn_amd_context* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    DeviceGuard guard(ctx->device);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return driver(e, "device-to-host copy");
    return ok();
}

ribn_amd_status ribn_amd_validate_quantized_geometry(uint32_t kernel_value_type, uint32_t weight_value_type,
                                                     const uint64_t* dims, size_t rank, uint64_t encoded_bytes,
                                                     uint64_t* input_size, uint64_t* output_size) {
    if (weight_value_type != kernel_value_type) {
        return fail(RIBN_AMD_UNSUPPORTED_VALUE_TYPE, kernel_value_type, weight_value_type,
                    "quantized GEMV requires GGML value type %u, got %u", kernel_value_type, weight_value_type);
    }
    if (!supported(kernel_value_type)) {
        return fail(RIBN_AMD_UNSUPPORTED_VALUE_TYPE, RIBN_AMD_Q4_K, kernel_value_type,
                    "GGML value type %u has no MI355X kernel", kernel_value_type);
    }
    if (rank != 2 || dims == nullptr) {
        return fail(RIBN_AMD_INVALID_WEIGHT, 2, rank, "expected rank-2 tensor, got rank %zu", rank);
    }
    const uint64_t k = dims[0], n = dims[1];
    const uint64_t bb = block_bytes(kernel_value_type);
    if (k == 0 || n == 0 || k % 256 != 0) {
        return fail(RIBN_AMD_INVALID_WEIGHT, 256, k,
                    "%s shape is %llux%llu; input size must be a positive multiple of 256",
                    type_label(kernel_value_type), (unsigned long long)k, (unsigned long long)n);
    }
    const uint64_t per_row = k / 256;
    if (per_row > std::numeric_limits<uint64_t>::max() / n) return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "block count overflows");
    const uint64_t blocks = per_row * n;
    if (blocks > std::numeric_limits<uint64_t>::max() / bb) return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "byte count overflows");
    const uint64_t expected = blocks * bb;
    if (encoded_bytes != expected) {
        return fail(RIBN_AMD_INVALID_WEIGHT, expected, encoded_bytes, "encoded length is %llu, expected %llu",
                    (unsigned long long)encoded_bytes, (unsigned long long)expected);
    }
    // quantized.rs:1795-1800: every byte offset and dimension must fit i32.
    // (Offsets are additionally bounded by the buffer resource's 32-bit range.)
    if (blocks > (uint64_t)std::numeric_limits<int32_t>::max() / bb) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "encoded tensor exceeds the i32 byte-offset range");
    }
    if (k > (uint64_t)std::numeric_limits<int32_t>::max() || n > (uint64_t)std::numeric_limits<int32_t>::max()) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "dimension exceeds i32");
    }
    if (input_size) *input_size = k;
    if (output_size) *output_size = n;
    return ok();
}

static ribn_amd_status new_weight(ribn_amd_context* ctx, uint32_t value_type, uint64_t k, uint64_t n,
                                  uint64_t encoded_bytes, ribn_amd_quantized_weight** out) {
    if (!ctx || !out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (encoded_bytes == 0) return fail(RIBN_AMD_EMPTY_ENCODING, 1, 0, "tensor has an empty encoding");
    if (encoded_bytes > (uint64_t)std::numeric_limits<size_t>::max()) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "encoded length does not fit the host");
    }
    auto* w = new (std::nothrow)
        ribn_amd_quantized_weight{ctx, ctx->device, value_type, k, n, encoded_bytes, nullptr, true};
    if (!w) return fail(RIBN_AMD_DRIVER, 0, 0, "host allocation failed");
    DeviceGuard guard(ctx->device);
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&w->data), encoded_bytes);
    if (e != hipSuccess) {
        delete w;
        return driver(e, "hipMalloc weight");
    }
    context_retain(ctx);  // released by ribn_amd_weight_destroy
    *out = w;
    return RIBN_AMD_OK;
}

ribn_amd_status ribn_amd_weight_materialize(ribn_amd_context* ctx, uint32_t value_type, uint64_t input_size,
                                            uint64_t output_size, const uint8_t* encoded, uint64_t encoded_bytes,
                                            ribn_amd_quantized_weight** out) {
    if (!encoded && encoded_bytes) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "encoded is null");
    ribn_amd_quantized_weight* w = nullptr;
    ribn_amd_status st = new_weight(ctx, value_type, input_size, output_size, encoded_bytes, &w);
    if (st != RIBN_AMD_OK) return st;
    DeviceGuard guard(ctx->device);
    hipError_t e = hipMemcpyAsync(w->data, encoded, encoded_bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        ribn_amd_weight_destroy(w);
        return driver(e, "upload weight");
    }
    *out = w;
    return ok();
}

ribn_amd_status ribn_amd_weight_materialize_reader(ribn_amd_context* ctx, uint32_t value_type,
                                                   uint64_t input_size, uint64_t output_size,
                                                   uint64_t encoded_bytes, ribn_amd_read_fn read, void* user,
                                                   ribn_amd_quantized_weight** out) {
    if (!read) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "read callback is null");
    ribn_amd_quantized_weight* w = nullptr;
    ribn_amd_status st = new_weight(ctx, value_type, input_size, output_size, encoded_bytes, &w);
    if (st != RIBN_AMD_OK) return st;
    DeviceGuard guard(ctx->device);
    const size_t chunk = (size_t)std::min<uint64_t>(encoded_bytes, 1u << 20);
    std::vector<uint8_t> host(chunk);
    uint64_t offset = 0;
    while (offset < encoded_bytes) {
        const size_t requested = (size_t)std::min<uint64_t>(encoded_bytes - offset, chunk);
        size_t filled = 0;
        while (filled < requested) {
            const int64_t got = read(user, host.data() + filled, requested - filled);
            if (got < 0) {
                ribn_amd_weight_destroy(w);
                return fail(RIBN_AMD_SOURCE_INCOMPLETE, encoded_bytes, offset + filled, "source read failed");
            }
            if (got == 0) {
                ribn_amd_weight_destroy(w);
                return fail(RIBN_AMD_SOURCE_INCOMPLETE, encoded_bytes, offset + filled,
                            "source ended after %llu of %llu bytes", (unsigned long long)(offset + filled),
                            (unsigned long long)encoded_bytes);
            }
            filled += (size_t)got;
        }
        hipError_t e = hipMemcpyAsync(w->data + offset, host.data(), requested, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            ribn_amd_weight_destroy(w);
            return driver(e, "upload weight chunk");
        }
        offset += requested;
    }
    *out = w;
    return ok();
}

ribn_amd_status ribn_amd_weight_wrap_device(ribn_amd_context* ctx, uint32_t value_type, uint64_t input_size,
                                            uint64_t output_size, const void* device_bytes, uint64_t encoded_bytes,
                                            ribn_amd_quantized_weight** out) {
    if (!ctx || !out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (encoded_bytes == 0) return fail(RIBN_AMD_EMPTY_ENCODING, 1, 0, "tensor has an empty encoding");
    ribn_amd_status st = check_device_ptr(ctx, device_bytes, "weight bytes");
    if (st != RIBN_AMD_OK) return st;
    auto* w = new (std::nothrow) ribn_amd_quantized_weight{
        ctx, ctx->device, value_type, input_size, output_size, encoded_bytes,
        const_cast<uint8_t*>(static_cast<const uint8_t*>(device_bytes)), false};
    if (!w) return fail(RIBN_AMD_DRIVER, 0, 0, "host allocation failed");
    context_retain(ctx);
    *out = w;
    return ok();
}

ribn_amd_status ribn_amd_weight_copy_to_host(ribn_amd_context* ctx, const ribn_amd_quantized_weight* weight,
                                             uint8_t* host, uint64_t capacity) {
    if (!ctx || !weight || !host) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (capacity != weight->encoded_bytes) {
        return fail(RIBN_AMD_OUTPUT_LENGTH, weight->encoded_bytes, capacity, "host buffer holds %llu bytes, need %llu",
                    (unsigned long long)capacity, (unsigned long long)weight->encoded_bytes);
    }
    return ribn_amd_memcpy_dtoh(ctx, host, weight->data, (size_t)capacity);
}

void ribn_amd_weight_destroy(ribn_amd_quantized_weight* weight) {
    if (!weight) return;
    if (weight->owns_data && weight->data) {
        DeviceGuard guard(weight->device);
        hipFree(weight->data);  // synchronises with outstanding work on the device
    }
    ribn_amd_context* ctx = weight->ctx;
    delete weight;
    context_release(ctx);
}

uint32_t ribn_amd_weight_value_type(const ribn_amd_quantized_weight* w) { return w ? w->value_type : 0; }
uint64_t ribn_amd_weight_encoded_bytes(const ribn_amd_quantized_weight* w) { return w ? w->encoded_bytes : 0; }
uint64_t ribn_amd_weight_input_size(const ribn_amd_quantized_weight* w) { return w ? w->input_size : 0; }
uint64_t ribn_amd_weight_output_size(const ribn_amd_quantized_weight* w) { return w ? w->output_size : 0; }
const void* ribn_amd_weight_device_ptr(const ribn_amd_quantized_weight* w) { return w ? w->data : nullptr; }

ribn_amd_status ribn_amd_gemv_create(ribn_amd_context* ctx, uint32_t value_type, ribn_amd_gemv** out) {
    if (!ctx || !out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (!supported(value_type)) {
        return fail(RIBN_AMD_UNSUPPORTED_VALUE_TYPE, RIBN_AMD_Q4_K, value_type,
                    "GGML value type %u has no MI355X GEMV kernel", value_type);
    }
    auto* g = new (std::nothrow) ribn_amd_gemv{ctx, value_type, RIBN_AMD_GEMV_WARP};
    if (!g) return fail(RIBN_AMD_DRIVER, 0, 0, "host allocation failed");
    context_retain(ctx);
    *out = g;
    return ok();
}

void ribn_amd_gemv_destroy(ribn_amd_gemv* gemv) {
    if (!gemv) return;
    ribn_amd_context* ctx = gemv->ctx;
    delete gemv;
    context_release(ctx);
}
uint32_t ribn_amd_gemv_value_type(const ribn_amd_gemv* gemv) { return gemv ? gemv->value_type : 0; }

ribn_amd_status ribn_amd_gemv_set_mode(ribn_amd_gemv* gemv, uint32_t mode) {
    if (!gemv) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null GEMV");
    if (mode != RIBN_AMD_GEMV_WARP && mode != RIBN_AMD_GEMV_FIXED16) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, RIBN_AMD_GEMV_FIXED16, mode, "unknown GEMV mode %u", mode);
    }
    gemv->mode = mode;
    return ok();
}

uint32_t ribn_amd_gemv_mode(const ribn_amd_gemv* gemv) { return gemv ? gemv->mode : RIBN_AMD_GEMV_WARP; }

ribn_amd_status ribn_amd_gemv_execute(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w, const float* input,
                                      size_t input_len, float* output, size_t output_len) {
    uint64_t k, n;
    ribn_amd_status st = validate_launch(g, w, input, input_len, output, output_len, 1, &k, &n);
    if (st != RIBN_AMD_OK) return st;
    DeviceGuard guard(g->ctx->device);
    hipError_t e = ribn_amd::launch_gemv_exact((int)g->value_type, w->data, (uint32_t)w->encoded_bytes, input,
                                               output, (int)k, (int)n, 1, g->ctx->stream);
    if (e != hipSuccess) return driver(e, "launch exact GEMV");
    return ok();
}

ribn_amd_status ribn_amd_gemv_execute_warp(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w,
                                           const float* input, size_t input_len, float* output,
                                           size_t output_len) {
    uint64_t k, n;
    ribn_amd_status st = validate_launch(g, w, input, input_len, output, output_len, 1, &k, &n);
    if (st != RIBN_AMD_OK) return st;
    return launch_batched(g, w, input, nullptr, 0.f, output, k, n, 1);
}

ribn_amd_status ribn_amd_gemv_execute_warp_batch(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w,
                                                 const float* input, size_t input_len, float* output,
                                                 size_t output_len, size_t members) {
    ribn_amd_status st = validate_members(g, members);
    if (st != RIBN_AMD_OK) return st;
    uint64_t k, n;
    st = validate_launch(g, w, input, input_len, output, output_len, members, &k, &n);
    if (st != RIBN_AMD_OK) return st;
    return launch_batched(g, w, input, nullptr, 0.f, output, k, n, members);
}

ribn_amd_status ribn_amd_gemv_execute_rms_norm(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w,
                                               const float* input, size_t input_len, const float* gamma,
                                               size_t gamma_len, float epsilon, float* output,
                                               size_t output_len, size_t members) {
    ribn_amd_status st = validate_members(g, members);
    if (st != RIBN_AMD_OK) return st;
    uint64_t k, n;
    st = validate_launch(g, w, input, input_len, output, output_len, members, &k, &n);
    if (st != RIBN_AMD_OK) return st;
    st = check_device_ptr(g->ctx, gamma, "gamma");
    if (st != RIBN_AMD_OK) return st;
    if (gamma_len != k) {
        return fail(RIBN_AMD_WEIGHT_LENGTH, k, gamma_len, "RMSNorm weight has %zu values, expected %llu", gamma_len,
                    (unsigned long long)k);
    }
    st = check_epsilon(epsilon);
    if (st != RIBN_AMD_OK) return st;
    return launch_batched(g, w, input, gamma, epsilon, output, k, n, members);
}

ribn_amd_status ribn_amd_gemv_execute_group(ribn_amd_gemv* g, const ribn_amd_quantized_weight* const* weights,
                                            size_t count, const float* input, size_t input_len,
                                            const float* gamma, size_t gamma_len, float epsilon,
                                            float* const* outputs, const size_t* output_lens, size_t members) {
    ribn_amd_status st = validate_members(g, members);
    if (st != RIBN_AMD_OK) return st;
    if (!weights || !outputs || !output_lens) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null array argument");
    if (count == 0 || count > (size_t)ribn_amd::kMaxGroup) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, ribn_amd::kMaxGroup, count, "a group holds 1..%d weights",
                    ribn_amd::kMaxGroup);
    }
    uint64_t k0 = 0;
    uint64_t total_rows = 0;
    for (size_t i = 0; i < count; ++i) {
        uint64_t k, n;
        st = validate_launch(g, weights[i], input, input_len, outputs[i], output_lens[i], members, &k, &n);
        if (st != RIBN_AMD_OK) return st;
        if (i == 0) k0 = k;
        total_rows += n;
    }
    if (total_rows > (uint64_t)std::numeric_limits<int32_t>::max()) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "grouped rows exceed i32");
    }
    if (gamma != nullptr) {
        st = check_device_ptr(g->ctx, gamma, "gamma");
        if (st != RIBN_AMD_OK) return st;
        if (gamma_len != k0) {
            return fail(RIBN_AMD_WEIGHT_LENGTH, k0, gamma_len, "RMSNorm weight has %zu values, expected %llu",
                        gamma_len, (unsigned long long)k0);
        }
        st = check_epsilon(epsilon);
        if (st != RIBN_AMD_OK) return st;
    }
    return launch_wave_group(g, weights, count, input, gamma, epsilon, outputs, k0, members);
}

ribn_amd_status ribn_amd_gemv_execute_fused(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w,
                                           const float* input, const float* up, size_t input_len, const float* gamma,
                                           size_t gamma_len, float epsilon, float* output, size_t output_len,
                                           size_t members, uint32_t flags) {
    ribn_amd_status st = validate_members(g, members);
    if (st != RIBN_AMD_OK) return st;
    if ((flags & ~(RIBN_AMD_FUSE_SWIGLU | RIBN_AMD_FUSE_ACCUMULATE)) != 0) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, 0, flags, "unknown fusion flags 0x%x", flags);
    }
    const bool swiglu = (flags & RIBN_AMD_FUSE_SWIGLU) != 0;
    if (swiglu && gamma != nullptr) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "the SwiGLU and RMSNorm prologues do not combine");
    }
    uint64_t k, n;
    st = validate_launch(g, w, input, input_len, output, output_len, members, &k, &n);
    if (st != RIBN_AMD_OK) return st;
    if (swiglu) {
        st = check_device_ptr(g->ctx, up, "up");
        if (st != RIBN_AMD_OK) return st;
    }
    if (gamma != nullptr) {
        st = check_device_ptr(g->ctx, gamma, "gamma");
        if (st != RIBN_AMD_OK) return st;
        if (gamma_len != k) {
            return fail(RIBN_AMD_WEIGHT_LENGTH, k, gamma_len, "RMSNorm weight has %zu values, expected %llu", gamma_len,
                        (unsigned long long)k);
        }
        st = check_epsilon(epsilon);
        if (st != RIBN_AMD_OK) return st;
    }
    const ribn_amd_quantized_weight* ws[1] = {w};
    float* outs[1] = {output};
    return launch_wave_group(g, ws, 1, input, gamma, epsilon, outs, k, members, swiglu ? up : nullptr,
                             (flags & RIBN_AMD_FUSE_ACCUMULATE) != 0);
}

ribn_amd_status ribn_amd_gemv_execute_gate_up_swiglu(ribn_amd_gemv* g, const ribn_amd_quantized_weight* gate,
                                                     const ribn_amd_quantized_weight* up, const float* input,
                                                     size_t input_len, const float* gamma, size_t gamma_len,
                                                     float epsilon, float* output, size_t output_len,
                                                     size_t members) {
    ribn_amd_status st = validate_members(g, members);
    if (st != RIBN_AMD_OK) return st;
    uint64_t k, n, k2, n2;
    st = validate_launch(g, gate, input, input_len, output, output_len, members, &k, &n);
    if (st != RIBN_AMD_OK) return st;
    st = validate_launch(g, up, input, input_len, output, output_len, members, &k2, &n2);
    if (st != RIBN_AMD_OK) return st;
    if (k > (uint64_t)ribn_amd::kSliceK) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, ribn_amd::kSliceK, k, "the gate/up pair epilogue supports K up to %d",
                    ribn_amd::kSliceK);
    }
    if (2 * n > (uint64_t)std::numeric_limits<int32_t>::max()) return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "rows exceed i32");
    if (gamma != nullptr) {
        st = check_device_ptr(g->ctx, gamma, "gamma");
        if (st != RIBN_AMD_OK) return st;
        if (gamma_len != k) {
            return fail(RIBN_AMD_WEIGHT_LENGTH, k, gamma_len, "RMSNorm weight has %zu values, expected %llu", gamma_len,
                        (unsigned long long)k);
        }
        st = check_epsilon(epsilon);
        if (st != RIBN_AMD_OK) return st;
    }
    DeviceGuard guard(g->ctx->device);
    const int per_launch = ribn_amd::gemv_launch_members((int)g->value_type, (int)k, false, arith_of_mode(g->mode));
    for (size_t m0 = 0; m0 < members; m0 += (size_t)per_launch) {
        const size_t mc = std::min<size_t>((size_t)per_launch, members - m0);
        ribn_amd::WaveGemvArgs a{};
        a.w[0] = gate->data;
        a.wbytes[0] = (uint32_t)gate->encoded_bytes;
        a.w[1] = up->data;
        a.wbytes[1] = (uint32_t)up->encoded_bytes;
        a.y[0] = output + m0 * n;
        a.y[1] = output + m0 * n;
        a.rows_end[0] = (int)n;
        a.rows_end[1] = (int)(2 * n);
        a.count = 2;
        a.total_rows = (int)(2 * n);
        a.x = input + m0 * k;
        a.gamma = gamma;
        a.eps = epsilon;
        a.K = (int)k;
        a.members = (int)mc;
        a.pair_swiglu = 1;
        a.arith = arith_of_mode(g->mode);
        hipError_t e = ribn_amd::launch_gemv((int)g->value_type, a, g->ctx->act_scratch, g->ctx->cu_count,
                                             g->ctx->stream);
        if (e != hipSuccess) return driver(e, "launch gate/up GEMV");
    }
    return ok();
}

ribn_amd_status ribn_amd_q8_1_quantize(ribn_amd_context* ctx, const float* input, size_t input_len, uint32_t* output,
                                       size_t output_len) {
    if (!ctx) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null context");
    // activation.rs:52-73: whole, non-empty blocks; nine words per block
    // (lengths first: an empty input is an InputLength error whatever its pointer)
    if (input_len == 0 || input_len % 32 != 0) {
        const size_t want = (std::max<size_t>(input_len, 1) + 31) / 32 * 32;
        return fail(RIBN_AMD_INPUT_LENGTH, want, input_len, "Q8_1 packing needs whole 32-value blocks, got %zu values",
                    input_len);
    }
    const size_t blocks = input_len / 32;
    if (output_len != blocks * 9) {
        return fail(RIBN_AMD_OUTPUT_LENGTH, blocks * 9, output_len, "Q8_1 output has %zu words, expected %zu",
                    output_len, blocks * 9);
    }
    ribn_amd_status st = check_device_ptr(ctx, input, "input", 4);
    if (st != RIBN_AMD_OK) return st;
    st = check_device_ptr(ctx, output, "output", 4);
    if (st != RIBN_AMD_OK) return st;
    if (input_len > std::numeric_limits<uint32_t>::max()) return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "input exceeds u32");
    DeviceGuard guard(ctx->device);
    hipError_t e = ribn_amd::launch_quantize_q8_1(input, output, (uint32_t)blocks, ctx->stream);
    if (e != hipSuccess) return driver(e, "launch Q8_1 packing");
    return ok();
}

static ribn_amd_status q8_1_gemv(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w, const uint32_t* input,
                                 size_t input_len, float* output, size_t output_len, size_t members) {
    if (g == nullptr || w == nullptr) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null kernel or weight handle");
    if (w->ctx->device != g->ctx->device) {
        return fail(RIBN_AMD_CONTEXT_MISMATCH, (uint64_t)g->ctx->device, (uint64_t)w->ctx->device,
                    "weight and kernel belong to different devices");
    }
    ribn_amd_status st = check_device_ptr(g->ctx, input, "input", 4);
    if (st != RIBN_AMD_OK) return st;
    st = check_device_ptr(g->ctx, output, "output", 4);
    if (st != RIBN_AMD_OK) return st;
    uint64_t k, n;
    st = validate_geometry(g->value_type, w, &k, &n);
    if (st != RIBN_AMD_OK) return st;
    // q4_q8_1.rs:95-112 / 176-200: K / 32 * 9 words and N outputs per member
    const uint64_t expected_in = k / 32 * 9 * members;
    const uint64_t expected_out = n * members;
    if (input_len != expected_in) {
        return fail(RIBN_AMD_INPUT_LENGTH, expected_in, input_len, "Q8_1 input has %zu words, expected %llu",
                    input_len, (unsigned long long)expected_in);
    }
    if (output_len != expected_out) {
        return fail(RIBN_AMD_OUTPUT_LENGTH, expected_out, output_len, "output has %zu values, expected %llu",
                    output_len, (unsigned long long)expected_out);
    }
    if (expected_in * 4 > std::numeric_limits<uint32_t>::max() || expected_out * 4 > std::numeric_limits<uint32_t>::max()) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "geometry exceeds u32");
    }
    DeviceGuard guard(g->ctx->device);
    hipError_t e = ribn_amd::launch_gemv_q8_1((int)g->value_type, w->data, (uint32_t)w->encoded_bytes, input, output,
                                              (int)k, (int)n, (int)members, g->ctx->stream);
    if (e != hipSuccess) return driver(e, "launch Q8_1 GEMV");
    return ok();
}

ribn_amd_status ribn_amd_gemv_execute_q8_1(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w, const uint32_t* input,
                                           size_t input_len, float* output, size_t output_len) {
    return q8_1_gemv(g, w, input, input_len, output, output_len, 1);
}

ribn_amd_status ribn_amd_gemv_execute_q8_1_batch(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w,
                                                 const uint32_t* input, size_t input_len, float* output,
                                                 size_t output_len, size_t members) {
    // q4_q8_1.rs:149-159: zero members is an input-length error, more than
    // eight an invalid-weight error naming the family
    if (members == 0) return fail(RIBN_AMD_INPUT_LENGTH, 1, 0, "batched GEMV needs at least one member");
    if (members > (size_t)ribn_amd::kQ8MaxMembers) {
        return fail(RIBN_AMD_INVALID_WEIGHT, (uint64_t)ribn_amd::kQ8MaxMembers, members,
                    "%s integer-dot batch variant supports at most %d members", g ? type_label(g->value_type) : "?",
                    ribn_amd::kQ8MaxMembers);
    }
    return q8_1_gemv(g, w, input, input_len, output, output_len, members);
}

ribn_amd_status ribn_amd_dequantize(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w, float* output,
                                    size_t output_len) {
    if (!g || !w) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null kernel or weight handle");
    ribn_amd_status st = check_device_ptr(g->ctx, output, "output");
    if (st != RIBN_AMD_OK) return st;
    uint64_t k, n;
    st = validate_geometry(g->value_type, w, &k, &n);
    if (st != RIBN_AMD_OK) return st;
    if (output_len != k * n) {
        return fail(RIBN_AMD_OUTPUT_LENGTH, k * n, output_len, "dequantized output has %zu values, expected %llu",
                    output_len, (unsigned long long)(k * n));
    }
    DeviceGuard guard(g->ctx->device);
    hipError_t e = ribn_amd::launch_dequant((int)g->value_type, w->data, (uint32_t)w->encoded_bytes, output,
                                            (uint32_t)(k / 256 * n), g->ctx->stream);
    if (e != hipSuccess) return driver(e, "launch dequantize");
    return ok();
}

// ------------------------------------------------------------ prefill GEMM

ribn_amd_status ribn_amd_gemm_prefill(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w, const void* input,
                                      uint32_t input_dtype, size_t input_len, size_t members, const float* gamma,
                                      size_t gamma_len, float epsilon, float* output, size_t output_len) {
    uint64_t k, n;
    ribn_amd_status st = validate_prefill(g, w, input, input_dtype, input_len, members, gamma, gamma_len, epsilon,
                                          output, output_len, &k, &n);
    if (st != RIBN_AMD_OK) return st;
    // the activation stage's part is required; split-K room is used as far as reserved
    const size_t need = ribn_amd::gemm_workspace_bytes(members, k, 0);
    if (need > g->ctx->workspace_bytes) {
        return fail(RIBN_AMD_WORKSPACE_TOO_SMALL, need, g->ctx->workspace_bytes,
                    "prefill of %zu tokens x K=%llu needs %zu workspace bytes; reserve them with "
                    "ribn_amd_context_reserve_prefill",
                    members, (unsigned long long)k, need);
    }
    DeviceGuard guard(g->ctx->device);
    hipError_t e = ribn_amd::launch_act_f16(input_dtype == RIBN_AMD_BF16, input, gamma, epsilon, (int)members, (int)k,
                                            g->ctx->workspace, g->ctx->stream);
    if (e != hipSuccess) return driver(e, "launch prefill activation stage");
    e = ribn_amd::launch_qgemm((int)g->value_type, w->data, (uint32_t)w->encoded_bytes, g->ctx->workspace,
                               g->ctx->workspace_bytes, output, (int)members, (int)n, (int)k, g->ctx->cu_count,
                               g->ctx->stream);
    if (e != hipSuccess) return driver(e, "launch prefill matmul");
    return ok();
}

ribn_amd_status ribn_amd_gemm_prefill_static(ribn_amd_gemv* g, const ribn_amd_quantized_weight* w, const void* input,
                                             uint32_t input_dtype, size_t input_len, size_t members,
                                             const float* gamma, size_t gamma_len, float epsilon, float* output,
                                             size_t output_len) {
    uint64_t k, n;
    ribn_amd_status st = validate_prefill(g, w, input, input_dtype, input_len, members, gamma, gamma_len, epsilon,
                                          output, output_len, &k, &n);
    if (st != RIBN_AMD_OK) return st;
    // the f16 activations and per-token unscales must fit; split-K partials use what is left
    const size_t need = ribn_amd::gemm_workspace_bytes(members, k, 0);
    if (need > kStaticScratchBytes) {
        return fail(RIBN_AMD_WORKSPACE_TOO_SMALL, kStaticScratchBytes, need,
                    "allocation-free prefill of %zu tokens x K=%llu needs %zu scratch bytes; the static scratch "
                    "holds %zu (use ribn_amd_gemm_prefill with a reserved workspace)",
                    members, (unsigned long long)k, need, kStaticScratchBytes);
    }
    const int device = g->ctx->device;
    DeviceGuard guard(device);
    void* ptr = static_scratch(device);
    if (ptr == nullptr) {
        st = resolve_static_scratch(device);  // with the device current
        if (st != RIBN_AMD_OK) return st;
        ptr = static_scratch(device);
    }
    hipStream_t stream = g->ctx->stream;
    st = order_static_call(device, stream, [&]() {
        hipError_t e = ribn_amd::launch_act_f16(input_dtype == RIBN_AMD_BF16, input, gamma, epsilon, (int)members,
                                                (int)k, ptr, stream);
        if (e != hipSuccess) return e;
        return ribn_amd::launch_qgemm((int)g->value_type, w->data, (uint32_t)w->encoded_bytes, ptr,
                                      kStaticScratchBytes, output, (int)members, (int)n, (int)k, g->ctx->cu_count,
                                      stream);
    });
    return st == RIBN_AMD_OK ? ok() : st;
}

// ------------------------------------------------------------ embedding

ribn_amd_status ribn_amd_embedding_create(ribn_amd_context* ctx, uint32_t value_type, ribn_amd_embedding** out) {
    if (!ctx || !out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (!supported(value_type)) {
        return fail(RIBN_AMD_UNSUPPORTED_VALUE_TYPE, RIBN_AMD_Q4_K, value_type,
                    "GGML value type %u has no MI355X embedding kernel", value_type);
    }
    auto* e = new (std::nothrow) ribn_amd_embedding{ctx, value_type};
    if (!e) return fail(RIBN_AMD_DRIVER, 0, 0, "host allocation failed");
    context_retain(ctx);
    *out = e;
    return ok();
}

void ribn_amd_embedding_destroy(ribn_amd_embedding* e) {
    if (!e) return;
    ribn_amd_context* ctx = e->ctx;
    delete e;
    context_release(ctx);
}

namespace {

// quantized.rs:961-1057 (execute) and 1058-1160 (execute_batch), in order:
// contexts, value type, shape, encoded length.
ribn_amd_status validate_embedding(const ribn_amd_embedding* e, const ribn_amd_quantized_weight* w,
                                   const float* output, uint64_t* hidden, uint64_t* vocab) {
    if (!e || !w) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null embedding or weight handle");
    if (w->ctx->device != e->ctx->device) {
        return fail(RIBN_AMD_CONTEXT_MISMATCH, (uint64_t)e->ctx->device, (uint64_t)w->ctx->device,
                    "weight and embedding kernel belong to different devices");
    }
    ribn_amd_status st = check_device_ptr(e->ctx, output, "output");
    if (st != RIBN_AMD_OK) return st;
    if (w->value_type != e->value_type) {
        return fail(RIBN_AMD_UNSUPPORTED_VALUE_TYPE, e->value_type, w->value_type,
                    "%s embedding got a weight of GGML value type %u", type_label(e->value_type), w->value_type);
    }
    *hidden = w->input_size;
    *vocab = w->output_size;
    if (*hidden == 0 || *vocab == 0 || *hidden % 256 != 0) {
        return fail(RIBN_AMD_INVALID_WEIGHT, 0, 0,
                    "%s embedding shape is %llux%llu; hidden size must be a positive multiple of 256",
                    type_label(e->value_type), (unsigned long long)*hidden, (unsigned long long)*vocab);
    }
    const uint64_t per_token = *hidden / 256;
    if (*vocab > std::numeric_limits<uint64_t>::max() / per_token) return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "shape overflows");
    const uint64_t blocks = per_token * *vocab;
    const uint64_t bb = block_bytes(e->value_type);
    if (blocks > std::numeric_limits<uint64_t>::max() / bb) return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "shape overflows");
    if (w->encoded_bytes != blocks * bb) {
        return fail(RIBN_AMD_INVALID_WEIGHT, blocks * bb, w->encoded_bytes, "encoded length is %llu, expected %llu",
                    (unsigned long long)w->encoded_bytes, (unsigned long long)(blocks * bb));
    }
    return RIBN_AMD_OK;
}

}  // namespace

ribn_amd_status ribn_amd_embedding_execute(ribn_amd_embedding* e, const ribn_amd_quantized_weight* w, uint32_t token,
                                           float* output, size_t output_len) {
    uint64_t hidden, vocab;
    ribn_amd_status st = validate_embedding(e, w, output, &hidden, &vocab);
    if (st != RIBN_AMD_OK) return st;
    if (token >= vocab) {
        return fail(RIBN_AMD_INVALID_WEIGHT, vocab, token, "token index %u is outside vocabulary size %llu", token,
                    (unsigned long long)vocab);
    }
    if (hidden > (uint64_t)std::numeric_limits<int>::max() || vocab > (uint64_t)std::numeric_limits<int>::max() ||
        w->encoded_bytes > 0xffffffffull) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "embedding table exceeds the kernel's index range");
    }
    if (output_len != hidden) {
        return fail(RIBN_AMD_OUTPUT_LENGTH, hidden, output_len, "embedding output has %zu values, expected %llu",
                    output_len, (unsigned long long)hidden);
    }
    DeviceGuard guard(e->ctx->device);
    hipError_t he = ribn_amd::launch_embedding((int)e->value_type, w->data, (uint32_t)w->encoded_bytes, nullptr, token,
                                               output, (uint32_t)(hidden / 256), (uint32_t)vocab, 1, e->ctx->stream);
    if (he != hipSuccess) return driver(he, "launch embedding");
    return ok();
}

ribn_amd_status ribn_amd_embedding_execute_batch(ribn_amd_embedding* e, const ribn_amd_quantized_weight* w,
                                                 const uint32_t* tokens, size_t members, float* output,
                                                 size_t output_len) {
    uint64_t hidden, vocab;
    ribn_amd_status st = validate_embedding(e, w, output, &hidden, &vocab);
    if (st != RIBN_AMD_OK) return st;
    if (members != 0) {
        st = check_device_ptr(e->ctx, tokens, "token indices", 4);
        if (st != RIBN_AMD_OK) return st;
    }
    if (hidden > (uint64_t)std::numeric_limits<int>::max() || vocab > (uint64_t)std::numeric_limits<int>::max() ||
        w->encoded_bytes > 0xffffffffull) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "embedding table exceeds the kernel's index range");
    }
    if (members == 0) return fail(RIBN_AMD_INPUT_LENGTH, 1, 0, "embedding batch needs at least one token");
    if (members > 65535) return fail(RIBN_AMD_SHAPE_OVERFLOW, 65535, members, "embedding batch exceeds 65535 tokens");
    if (output_len / members != hidden || output_len % members != 0) {
        return fail(RIBN_AMD_OUTPUT_LENGTH, members * hidden, output_len,
                    "embedding output has %zu values, expected %llu", output_len,
                    (unsigned long long)(members * hidden));
    }
    DeviceGuard guard(e->ctx->device);
    hipError_t he = ribn_amd::launch_embedding((int)e->value_type, w->data, (uint32_t)w->encoded_bytes, tokens, 0,
                                               output, (uint32_t)(hidden / 256), (uint32_t)vocab, (uint32_t)members,
                                               e->ctx->stream);
    if (he != hipSuccess) return driver(he, "launch embedding batch");
    return ok();
}

static ribn_amd_status rms_common(ribn_amd_context* ctx, const float* input, size_t input_len, const float* weight,
                                  size_t weight_len, float* output, size_t output_len, size_t length,
                                  float epsilon) {
    if (!ctx) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null context");
    ribn_amd_status st = check_device_ptr(ctx, input, "input");
    if (st == RIBN_AMD_OK) st = check_device_ptr(ctx, weight, "weight");
    if (st == RIBN_AMD_OK) st = check_device_ptr(ctx, output, "output");
    if (st != RIBN_AMD_OK) return st;
    // model_ops.rs:1780-1806 order: empty, divisibility, weight, output, epsilon.
    if (input_len == 0 || length == 0) return fail(RIBN_AMD_EMPTY_INPUT, 1, 0, "RMSNorm input is empty");
    if (input_len % length != 0) {
        return fail(RIBN_AMD_INPUT_LENGTH, input_len, length, "input of %zu values is not a multiple of %zu",
                    input_len, length);
    }
    if (weight_len != length) {
        return fail(RIBN_AMD_WEIGHT_LENGTH, length, weight_len, "RMSNorm weight has %zu values, expected %zu",
                    weight_len, length);
    }
    if (output_len != input_len) {
        return fail(RIBN_AMD_OUTPUT_LENGTH, input_len, output_len, "RMSNorm output has %zu values, expected %zu",
                    output_len, input_len);
    }
    st = check_epsilon(epsilon);
    if (st != RIBN_AMD_OK) return st;
    const size_t members = input_len / length;
    if (length > (size_t)std::numeric_limits<int>::max() || members > (size_t)std::numeric_limits<int>::max()) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "RMSNorm shape exceeds launch limits");
    }
    DeviceGuard guard(ctx->device);
    hipError_t e = ribn_amd::launch_rms_norm(input, weight, output, (int)length, (int)members, epsilon, ctx->stream);
    if (e != hipSuccess) return driver(e, "launch RMSNorm");
    return ok();
}

ribn_amd_status ribn_amd_rms_norm(ribn_amd_context* ctx, const float* input, size_t input_len, const float* weight,
                                  size_t weight_len, float* output, size_t output_len, float epsilon) {
    // model_ops.rs:1714-1760: one vector; weight and output lengths equal the input's.
    return rms_common(ctx, input, input_len, weight, weight_len, output, output_len, input_len, epsilon);
}

ribn_amd_status ribn_amd_rms_norm_batch(ribn_amd_context* ctx, const float* input, size_t input_len,
                                        const float* weight, size_t weight_len, float* output, size_t output_len,
                                        size_t length, float epsilon) {
    return rms_common(ctx, input, input_len, weight, weight_len, output, output_len, length, epsilon);
}

}  // extern "C"

// Internal declarations shared by the C-ABI translation units (ribn_amd.cpp,
// qwen3_decode.cpp): the opaque handle types and the validation / error helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include <atomic>
#include <stdint.h>

#include "ribn_amd.h"

struct ribn_amd_context {
    int device;
    hipStream_t stream;
    bool owns_stream;
    int cu_count;
    void* workspace;  // prefill activation workspace (ribn_amd_context_reserve_prefill)
    size_t workspace_bytes;
    void* act_scratch;  // packed activations of the matrix-core batched GEMV, reserved at creation
    void* attn_members; // cache descriptors of the standalone attention call (same allocation)
    // Owner handle plus every decoder and dispatcher built on the context: the
    // device resources are released when the last of them lets go, so handles
    // may be destroyed in any order (e.g. by a garbage collector).
    std::atomic<int> refs{1};
};

struct ribn_amd_quantized_weight {
    ribn_amd_context* ctx;
    int device;  // kept so destruction never touches the (possibly destroyed) context
    uint32_t value_type;
    uint64_t input_size;
    uint64_t output_size;
    uint64_t encoded_bytes;
    uint8_t* data;
    bool owns_data;
};

struct ribn_amd_gemv {
    ribn_amd_context* ctx;
    uint32_t value_type;
    uint32_t mode;  // RIBN_AMD_GEMV_WARP or RIBN_AMD_GEMV_FIXED16
};

namespace ribn_amd_abi {
// Launch arithmetic (ribn_amd::kArith*) of a GEMV mode.
inline int arith_of_mode(uint32_t mode) { return mode == RIBN_AMD_GEMV_FIXED16 ? 1 : 0; }
}  // namespace ribn_amd_abi

struct ribn_amd_embedding {
    ribn_amd_context* ctx;
    uint32_t value_type;
};

namespace ribn_amd_abi {

// Records the calling thread's last error and returns `status`.
ribn_amd_status fail(ribn_amd_status status, uint64_t expected, uint64_t actual, const char* fmt, ...);
// Clears the last error and returns RIBN_AMD_OK.
ribn_amd_status ok();
// Maps a HIP error onto Driver (or Module for a missing code object).
ribn_amd_status driver(hipError_t e, const char* what);
const char* type_label(uint32_t t);
uint64_t block_bytes(uint32_t t);
bool supported(uint32_t t);
// ContextMismatch / InvalidArgument checks of a raw device pointer.
ribn_amd_status check_device_ptr(const ribn_amd_context* ctx, const void* ptr, const char* what,
                                 uintptr_t align = 16);
ribn_amd_status validate_geometry(uint32_t kernel_type, const ribn_amd_quantized_weight* w, uint64_t* k,
                                  uint64_t* n);
ribn_amd_status check_epsilon(float epsilon);

// Context lifetime: dependents retain the context they use and release it
// when destroyed; the last release frees the stream, scratch and workspace.
void context_retain(ribn_amd_context* ctx);
void context_release(ribn_amd_context* ctx);

struct DeviceGuard {
    int previous = -1;
    explicit DeviceGuard(int device) {
        if (hipGetDevice(&previous) != hipSuccess) previous = -1;
        if (previous != device) hipSetDevice(device);
    }
    ~DeviceGuard() {
        if (previous >= 0) hipSetDevice(previous);
    }
};

}  // namespace ribn_amd_abi

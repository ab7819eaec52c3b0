/*
 * ribn_amd.h -- C ABI of the MI355X (gfx950) k-quant decode path.
 *
 * This is the drop-in boundary a Rust `crates/amd` backend binds in place of
 * the reference's `crates/nvidia` operators. Every entry point below names the
 * reference interface it replaces (paths relative to nijaru/engine). Device
 * buffers are plain pointers plus element counts (the reference passes
 * `CudaSlice<T>`, whose `len()` the C side receives explicitly); no torch or
 * HIP C++ types appear in signatures. HIP streams are passed as `void*`.
 *
 * Conventions
 *  - GGML dims are [K, N]: K is the contiguous input size, N the output rows
 *    (crates/nvidia/src/quantized.rs:136-142). Encoded weights stay in GGML's
 *    array-of-blocks layout on the device; nothing is repacked.
 *  - Activations are f32 batch-major [members][K]; outputs [members][N].
 *  - Launches are asynchronous on the context's stream; completion is observed
 *    by ribn_amd_context_synchronize or a later stream-ordered copy
 *    (quantized.rs:357-363). Execute calls never allocate device memory.
 *  - Every call validates before launching and returns a status; details
 *    (expected/actual values, message) are kept per thread and read with
 *    ribn_amd_last_error (mirrors CudaQuantizedKernelError, quantized.rs:91-134,
 *    and CudaModelKernelError, model_ops.rs:12-22).
 *  - Device pointers handed to kernels must be 16-byte aligned (hipMalloc and
 *    ribn_amd_alloc return 256-byte-aligned memory).
 *  - Thread compatibility: a context and its kernel objects may be used from
 *    one thread at a time; distinct contexts are independent.
 */
#ifndef RIBN_AMD_H
#define RIBN_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RIBN_AMD_ABI_VERSION 2

/* GGML value types served by this library (quantized.rs:25-27). */
#define RIBN_AMD_Q4_K 12u
#define RIBN_AMD_Q5_K 13u
#define RIBN_AMD_Q6_K 14u

/* Members one batched call accepts. The reference caps its weights-read-once
 * kernels at 8 (quantized.rs:12); this library serves decode batches up to 64. */
#define RIBN_AMD_MAX_BATCH_MEMBERS 64u

/* Activation element types accepted by ribn_amd_gemm_prefill. */
#define RIBN_AMD_F32 0u
#define RIBN_AMD_BF16 1u

typedef enum ribn_amd_status {
    RIBN_AMD_OK = 0,
    RIBN_AMD_DRIVER = 1,                 /* Driver(String): a HIP runtime call failed */
    RIBN_AMD_MODULE = 2,                 /* Nvrtc(String): no gfx950 code object for this device */
    RIBN_AMD_INVALID_WEIGHT = 3,         /* InvalidWeight(String) */
    RIBN_AMD_UNSUPPORTED_VALUE_TYPE = 4, /* UnsupportedValueType { expected, actual } */
    RIBN_AMD_SHAPE_OVERFLOW = 5,         /* ShapeOverflow */
    RIBN_AMD_INPUT_LENGTH = 6,           /* InputLength { expected, actual } */
    RIBN_AMD_OUTPUT_LENGTH = 7,          /* OutputLength { expected, actual } */
    RIBN_AMD_CONTEXT_MISMATCH = 8,       /* ContextMismatch: buffer on another device */
    RIBN_AMD_EMPTY_INPUT = 9,            /* CudaModelKernelError::EmptyInput */
    RIBN_AMD_WEIGHT_LENGTH = 10,         /* CudaModelKernelError::WeightLength { expected, actual } */
    RIBN_AMD_INVALID_EPSILON = 11,       /* CudaModelKernelError::InvalidEpsilon */
    RIBN_AMD_INVALID_ARGUMENT = 12,      /* null handle / misaligned pointer (no reference twin) */
    RIBN_AMD_EMPTY_ENCODING = 13,        /* CudaWeightError::EmptyEncoding (cuda.rs:335-337) */
    RIBN_AMD_SOURCE_INCOMPLETE = 14,     /* CudaWeightError::SourceIncomplete (cuda.rs:350-356) */
    RIBN_AMD_WORKSPACE_TOO_SMALL = 15,   /* prefill workspace not reserved (no reference twin) */
    RIBN_AMD_INVALID_PLAN = 16,          /* CudaDecodeError::InvalidPlan (decode.rs:91-93) */
    RIBN_AMD_POSITION_OVERFLOW = 17,     /* CudaDecodeError::PositionOverflow { position, capacity } */
    RIBN_AMD_MISSING_TENSOR = 18,        /* CudaDecodeError::MissingTensor (decode.rs:86-87); GgufError::MissingTensor */
    /* GgufError (crates/gguf/src/lib.rs:741-805) */
    RIBN_AMD_GGUF_IO = 19,                        /* Io { path, message } (open, read, unexpected end of file) */
    RIBN_AMD_GGUF_INVALID_MAGIC = 20,             /* InvalidMagic(u32): actual = the magic read */
    RIBN_AMD_GGUF_UNSUPPORTED_VERSION = 21,       /* UnsupportedVersion(u32) */
    RIBN_AMD_GGUF_INVALID_UTF8 = 22,              /* InvalidUtf8 */
    RIBN_AMD_GGUF_INVALID_VALUE_TYPE = 23,        /* InvalidValueType(u32) */
    RIBN_AMD_GGUF_INVALID_BOOL = 24,              /* InvalidBool(u8) */
    RIBN_AMD_GGUF_INVALID_LENGTH = 25,            /* InvalidLength { kind, value } */
    RIBN_AMD_GGUF_ARRAY_NESTING_TOO_DEEP = 26,    /* ArrayNestingTooDeep */
    RIBN_AMD_GGUF_DUPLICATE_METADATA = 27,        /* DuplicateMetadata(key) */
    RIBN_AMD_GGUF_INVALID_DIMENSION_COUNT = 28,   /* InvalidDimensionCount(u32) */
    RIBN_AMD_GGUF_INVALID_ALIGNMENT = 29,         /* InvalidAlignment(u64) */
    RIBN_AMD_GGUF_TRUNCATED = 30,                 /* Truncated */
    RIBN_AMD_GGUF_TENSOR_OFFSET_OUT_OF_BOUNDS = 31, /* TensorOffsetOutOfBounds { name, offset } */
    RIBN_AMD_GGUF_UNSUPPORTED_TENSOR_TYPE = 32,   /* UnsupportedTensorType(u32) */
    RIBN_AMD_GGUF_BYTE_LENGTH_OVERFLOW = 33,      /* ElementCountOverflow / TensorByteLengthOverflow */
    RIBN_AMD_GGUF_QUANTIZATION_MISMATCH = 34,     /* QuantizationDimensionMismatch / QuantizationBlockMismatch */
    RIBN_AMD_GGUF_MISSING_METADATA = 35,          /* MissingMetadata(key) */
    RIBN_AMD_GGUF_METADATA_TYPE_MISMATCH = 36,    /* MetadataTypeMismatch { key } */
    RIBN_AMD_BUDGET_EXCEEDED = 37,                /* CudaWeightStagingError::BudgetExceeded (staging.rs:255-258);
                                                     also a KV materialization past the serving budget */
    /* serving dispatcher (BackendError, crates/core/src/backend.rs:188-196; CudaStateError, state.rs:905-956) */
    RIBN_AMD_UNSUPPORTED = 38,                    /* BackendError::Unsupported (non-greedy sampling, other phases) */
    RIBN_AMD_EXECUTION_FAILED = 39,               /* BackendError::ExecutionFailed (row input, slots, duplicates) */
    RIBN_AMD_UNKNOWN_SUBMISSION = 40,             /* BackendError::UnknownSubmission */
    RIBN_AMD_DEVICE_FAULTED = 41,                 /* ExecutionFailed after a device failure: terminal */
    RIBN_AMD_STATE_POSITION = 42,                 /* UnmaterializedPrefix / PositionMismatch / PositionRegression */
} ribn_amd_status;

typedef struct ribn_amd_error {
    int32_t status;
    uint64_t expected;
    uint64_t actual;
    char message[512];
} ribn_amd_error;

typedef struct ribn_amd_context ribn_amd_context;
typedef struct ribn_amd_quantized_weight ribn_amd_quantized_weight;
typedef struct ribn_amd_gemv ribn_amd_gemv;
typedef struct ribn_amd_embedding ribn_amd_embedding;

/* ---------------------------------------------------------------- errors */

/* Copies the calling thread's last error record (status RIBN_AMD_OK if none). */
ribn_amd_status ribn_amd_last_error(ribn_amd_error *out);
/* Static, NUL-terminated name of a status ("InputLength", ...). */
const char *ribn_amd_status_name(int32_t status);
int32_t ribn_amd_abi_version(void);

/* ------------------------------------------------------------- lifecycle */

/* CudaQ4KGemv::new (quantized.rs:1575-1580; the same in every family):
 * CudaContext::new(device) + default_stream(). Here: a context owning a fresh
 * non-blocking stream on `device`. Every context (created or wrapping a stream)
 * reserves about 0.56 MB of device scratch for the packed activations of
 * batched GEMV launches (calls on one context share it in stream order), so
 * execute calls allocate nothing. */
ribn_amd_status ribn_amd_context_create(int32_t device, ribn_amd_context **out);
/* CudaQ4KGemv::from_context(&ctx, stream) (quantized.rs:1588-1610): wraps a
 * caller-owned HIP stream; the caller keeps ownership and must outlive the context. */
ribn_amd_status ribn_amd_context_wrap_stream(int32_t device, void *hip_stream, ribn_amd_context **out);
/* Releases the caller's reference. Weights, kernel objects, decoders and
 * serving dispatchers built on the context hold references of their own (as
 * the reference's operators hold an Arc<CudaContext>), so handles may be
 * destroyed in any order: the stream (when owned), scratch and workspace go
 * with the last reference. */
void ribn_amd_context_destroy(ribn_amd_context *ctx);
/* CudaStream::synchronize. */
ribn_amd_status ribn_amd_context_synchronize(ribn_amd_context *ctx);
void *ribn_amd_context_stream(const ribn_amd_context *ctx);
int32_t ribn_amd_context_device(const ribn_amd_context *ctx);

/* ---------------------------------------------------- device memory helpers */

/* CudaStream::alloc_zeros::<u8>(bytes): zero-filled, 256-byte aligned. */
ribn_amd_status ribn_amd_alloc(ribn_amd_context *ctx, size_t bytes, void **out);
ribn_amd_status ribn_amd_free(ribn_amd_context *ctx, void *device_ptr);
/* clone_htod / clone_dtoh: stream-ordered copies that return after completion. */
ribn_amd_status ribn_amd_memcpy_htod(ribn_amd_context *ctx, void *dst, const void *src, size_t bytes);
ribn_amd_status ribn_amd_memcpy_dtoh(ribn_amd_context *ctx, void *dst, const void *src, size_t bytes);

/* ----------------------------------------------------------- weight store */

/* Pull-style source for ribn_amd_weight_materialize_reader, mirroring
 * `&mut impl Read`: returns bytes written to buf (0 = end of source), or a
 * negative value on a source error. */
typedef int64_t (*ribn_amd_read_fn)(void *user, uint8_t *buf, size_t capacity);

/* CudaWeightStore::materialize_quantized (crates/nvidia/src/cuda.rs:321-387):
 * uploads `encoded_bytes` opaque GGML bytes of a [input_size=K, output_size=N]
 * tensor of `value_type`. The bytes are not interpreted or repacked; geometry
 * is checked when a kernel uses the weight (validate_quantized_geometry). */
ribn_amd_status ribn_amd_weight_materialize(ribn_amd_context *ctx, uint32_t value_type, uint64_t input_size,
                                            uint64_t output_size, const uint8_t *encoded, uint64_t encoded_bytes,
                                            ribn_amd_quantized_weight **out);
/* Same, streaming from `read` in 1 MiB chunks (cuda.rs:340-377). */
ribn_amd_status ribn_amd_weight_materialize_reader(ribn_amd_context *ctx, uint32_t value_type,
                                                   uint64_t input_size, uint64_t output_size,
                                                   uint64_t encoded_bytes, ribn_amd_read_fn read, void *user,
                                                   ribn_amd_quantized_weight **out);
/* Adopts `encoded_bytes` already resident on the context's device (no copy;
 * the caller keeps ownership of the memory). */
ribn_amd_status ribn_amd_weight_wrap_device(ribn_amd_context *ctx, uint32_t value_type, uint64_t input_size,
                                            uint64_t output_size, const void *device_bytes, uint64_t encoded_bytes,
                                            ribn_amd_quantized_weight **out);
/* CudaWeightStore::copy_quantized_to_host (cuda.rs:451-458): exact bytes back. */
ribn_amd_status ribn_amd_weight_copy_to_host(ribn_amd_context *ctx, const ribn_amd_quantized_weight *weight,
                                             uint8_t *host, uint64_t capacity);
void ribn_amd_weight_destroy(ribn_amd_quantized_weight *weight);
/* CudaQuantizedWeight accessors (cuda.rs:164-183). */
uint32_t ribn_amd_weight_value_type(const ribn_amd_quantized_weight *weight);
uint64_t ribn_amd_weight_encoded_bytes(const ribn_amd_quantized_weight *weight);
uint64_t ribn_amd_weight_input_size(const ribn_amd_quantized_weight *weight);
uint64_t ribn_amd_weight_output_size(const ribn_amd_quantized_weight *weight);
const void *ribn_amd_weight_device_ptr(const ribn_amd_quantized_weight *weight);

/* validate_quantized_geometry (quantized.rs:1755-1804), host-only: checks the
 * value type against the kernel's, rank 2, K a positive multiple of 256, the
 * exact encoded length and i32 launch limits. Writes (K, N) on success. */
ribn_amd_status ribn_amd_validate_quantized_geometry(uint32_t kernel_value_type, uint32_t weight_value_type,
                                                     const uint64_t *dims, size_t rank, uint64_t encoded_bytes,
                                                     uint64_t *input_size, uint64_t *output_size);

/* ----------------------------------------------------------- GEMV kernels */

/* CudaQ4KGemv / CudaQ5KGemv / CudaQ6KGemv ::from_context (quantized.rs:1465-1753),
 * i.e. QwenGemvKernel::from_value_type (staging.rs:108-127): a kernel object
 * for one GGML value type on a context. Unsupported types return
 * UnsupportedValueType { expected: 12, actual }. */
ribn_amd_status ribn_amd_gemv_create(ribn_amd_context *ctx, uint32_t value_type, ribn_amd_gemv **out);
void ribn_amd_gemv_destroy(ribn_amd_gemv *gemv);
uint32_t ribn_amd_gemv_value_type(const ribn_amd_gemv *gemv);

/* GEMV arithmetic of the warp-family calls below (execute_warp, _warp_batch,
 * _rms_norm, _group, _fused, _gate_up_swiglu); the reference's GemvMode
 * (crates/nvidia/src/decode.rs:285-307).
 *   RIBN_AMD_GEMV_WARP (default; GemvMode::Warp): f32 activations against
 *     weights dequantised in registers, f32 accumulation. Up to 8 members
 *     (the reference's batch cap) share one weight stream (from 3 members,
 *     K > 4096 is split by 4096-wide slice and the slice totals added in
 *     order); every row is bit-identical to the single-member call. From 9
 *     to 64 members the products run on the matrix cores at f32 precision
 *     (Q4_K / Q5_K: quants times group scale exact in f16, activations in
 *     two f16 pieces; Q6_K: activations in three bf16 pieces; f32
 *     accumulation) with the weights read once per 64 members (32 for
 *     Q6_K): rows agree with the single call to f32 rounding (within 5e-5
 *     normwise of the sequential f32 GEMV), and a member's bits do not
 *     depend on the rest of the batch.
 *   RIBN_AMD_GEMV_FIXED16 (opt-in, lossy; no reference twin, used like
 *     GemvMode::IntegerDot for throughput comparison): activations rounded to
 *     block fixed point (16-bit per scale group in the wave kernel, 15-bit per
 *     super-block on the int8 matrix cores from 5 members) with integer dot
 *     products. Never bit-identical to WARP.
 * The reference's third mode, GemvMode::Scalar (one thread per row, its
 * decode correctness oracle), is not a mode here: its per-operator form is
 * ribn_amd_gemv_execute (bit-identical to the host decoder + sequential
 * dot), and decoder-level correctness is checked against a CPU oracle of the
 * whole step instead. Mapping GemvMode::Scalar to a decoder mode is
 * therefore InvalidArgument by design. */
#define RIBN_AMD_GEMV_WARP 0u
#define RIBN_AMD_GEMV_FIXED16 1u
/* set_gemv_mode / gemv_mode (decode.rs:711-741) at the operator level: an
 * unknown mode is InvalidArgument. */
ribn_amd_status ribn_amd_gemv_set_mode(ribn_amd_gemv *gemv, uint32_t mode);
uint32_t ribn_amd_gemv_mode(const ribn_amd_gemv *gemv);

/* execute (quantized.rs:368-388): y[N] = W x[K]. Exact-order kernel: per row,
 * elements in K order, each product and sum rounded separately, so results
 * equal the host decoder + sequential f32 dot bit for bit. Correctness oracle;
 * slow. */
ribn_amd_status ribn_amd_gemv_execute(ribn_amd_gemv *gemv, const ribn_amd_quantized_weight *weight,
                                      const float *input, size_t input_len, float *output, size_t output_len);
/* execute_warp (quantized.rs:401-435): the wave64 bandwidth kernel (default
 * decode path), in the kernel object's GEMV mode. K up to 16384 stages in one
 * launch; a K of 16640..65536 (e.g. the 17408-wide down projection of the
 * reference's 27B shapes) runs the f32 slice-split form in either mode (one
 * 4096-wide slice per workgroup, slice totals added in order by a second
 * launch; plain, grouped and accumulating products); a larger K runs the
 * exact-order kernel. */
ribn_amd_status ribn_amd_gemv_execute_warp(ribn_amd_gemv *gemv, const ribn_amd_quantized_weight *weight,
                                           const float *input, size_t input_len, float *output,
                                           size_t output_len);
/* execute_warp_batch (quantized.rs:445-487): `members` batch-major rows,
 * weights read once per launch group. input_len == members*K,
 * output_len == members*N, 1 <= members <= RIBN_AMD_MAX_BATCH_MEMBERS.
 * Every row is bit-identical to execute_warp on that member alone. */
ribn_amd_status ribn_amd_gemv_execute_warp_batch(ribn_amd_gemv *gemv, const ribn_amd_quantized_weight *weight,
                                                 const float *input, size_t input_len, float *output,
                                                 size_t output_len, size_t members);
/* RMSNorm fused into the activation load of execute_warp_batch: replaces the
 * pair rms_norm_batch (model_ops.rs:1770-1824) + gemv_batch (decode.rs:1516-1558)
 * with one launch computing y_m = W * (x_m * inv_rms(x_m) * gamma),
 * inv_rms = 1/sqrt(sum(x^2)/K + eps). gamma has K values. */
ribn_amd_status ribn_amd_gemv_execute_rms_norm(ribn_amd_gemv *gemv, const ribn_amd_quantized_weight *weight,
                                               const float *input, size_t input_len, const float *gamma,
                                               size_t gamma_len, float epsilon, float *output,
                                               size_t output_len, size_t members);
/* Grouped form of execute_rms_norm / execute_warp_batch with no reference
 * counterpart (the reference launches each projection separately,
 * decode.rs:582-617): streams `count` (1..4) weights of this kernel's type and
 * equal K that share one input in a single launch, e.g. q/k/v or gate/up of a
 * decoder layer. outputs[i] holds members*N_i values (output_lens[i]).
 * gamma == NULL skips the RMSNorm prologue (gamma_len and epsilon ignored). */
ribn_amd_status ribn_amd_gemv_execute_group(ribn_amd_gemv *gemv, const ribn_amd_quantized_weight *const *weights,
                                            size_t count, const float *input, size_t input_len,
                                            const float *gamma, size_t gamma_len, float epsilon,
                                            float *const *outputs, const size_t *output_lens, size_t members);
/* Fusion flags of ribn_amd_gemv_execute_fused. */
#define RIBN_AMD_FUSE_SWIGLU 1u     /* activation = silu(input) * up */
#define RIBN_AMD_FUSE_ACCUMULATE 2u /* output += W activation (residual add) */
/* execute_warp_batch with the decode step's elementwise neighbours fused in;
 * no single reference counterpart. The reference runs them as separate
 * launches around gemv (decode.rs:596-631,1021-1031):
 *   RIBN_AMD_FUSE_SWIGLU: the activation is silu(input) * up, the
 *     reference's silu_mul (model_ops.rs:316-328, 1888-1929); `up` holds
 *     input_len values (members <= RIBN_AMD_MAX_BATCH_MEMBERS, launched in
 *     pairs).
 *   RIBN_AMD_FUSE_ACCUMULATE: output += W x (residual_add, model_ops.rs:600-611,
 *     2314-2350); each output element is added exactly once.
 *   gamma != NULL: the RMSNorm prologue of execute_rms_norm (not with SWIGLU).
 * Every row is computed as execute_warp_batch computes it. */
ribn_amd_status ribn_amd_gemv_execute_fused(ribn_amd_gemv *gemv, const ribn_amd_quantized_weight *weight,
                                            const float *input, const float *up, size_t input_len,
                                            const float *gamma, size_t gamma_len, float epsilon, float *output,
                                            size_t output_len, size_t members, uint32_t flags);
/* Gate/up projection pair with the SwiGLU activation fused into the epilogue:
 * output_m = silu(gate . x'_m) * (up . x'_m), x' = input or its RMSNorm
 * (gamma != NULL). It replaces the reference's gemv(ffn_gate) + gemv(ffn_up) +
 * silu_mul (decode.rs:608-631, model_ops.rs:316-328): one wave reduces row n
 * of both weights back to back and stores only the product, so the gate and
 * up vectors never reach memory. gate and up are this kernel's type, equal
 * [K, N] shapes, K <= 4096; output holds members*N values. */
ribn_amd_status ribn_amd_gemv_execute_gate_up_swiglu(ribn_amd_gemv *gemv, const ribn_amd_quantized_weight *gate,
                                                     const ribn_amd_quantized_weight *up, const float *input,
                                                     size_t input_len, const float *gamma, size_t gamma_len,
                                                     float epsilon, float *output, size_t output_len,
                                                     size_t members);
/* ------------------------------------------- GGUF reader and staging */

/* GgufFile (crates/gguf/src/lib.rs:165-345). Parsed at open; bulk tensor data
 * is not read until staged. */
typedef struct ribn_amd_gguf ribn_amd_gguf;

/* One metadata value (MetadataValue, lib.rs:29-46). `type` is the GGUF value
 * type: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string,
 * 9 array, 10 u64, 11 i64, 12 f64. Unsigned types and bool fill `u`, signed
 * types `i`, f32/f64 `f` (with the raw bits in `u`), strings `str`/`str_len`
 * (owned by the file handle, not NUL-terminated by contract), arrays
 * `array_type`/`array_len` (items via ribn_amd_gguf_metadata_array_get). */
typedef struct ribn_amd_gguf_value {
    uint32_t type;
    uint32_t array_type;
    uint64_t array_len;
    uint64_t u;
    int64_t i;
    double f;
    const char *str;
    uint64_t str_len;
} ribn_amd_gguf_value;

/* TensorInfo (lib.rs:87-163): name (owned by the file handle), GGUF
 * dimensions (dims[0] is the innermost, K for a weight), GGML type id, and
 * offset relative to the aligned tensor data. */
typedef struct ribn_amd_gguf_tensor {
    const char *name;
    uint32_t n_dims;
    uint64_t dims[16];
    uint32_t value_type;
    uint64_t offset;
} ribn_amd_gguf_tensor;

/* GgufFile::open (lib.rs:178-272): header, metadata and tensor directory,
 * with the reference's limits and errors (GGUF_* statuses). */
ribn_amd_status ribn_amd_gguf_open(const char *path, ribn_amd_gguf **out);
void ribn_amd_gguf_close(ribn_amd_gguf *g);
/* GgufFile::{version, tensor_count, tensor_data_offset} (lib.rs:279-289, 374-377) */
uint32_t ribn_amd_gguf_version(const ribn_amd_gguf *g);
uint64_t ribn_amd_gguf_tensor_count(const ribn_amd_gguf *g);
uint64_t ribn_amd_gguf_tensor_data_offset(const ribn_amd_gguf *g);
/* GgufFile::metadata_map (lib.rs:291-299): keys in sorted order, as the
 * reference's BTreeMap iterates. */
uint64_t ribn_amd_gguf_metadata_count(const ribn_amd_gguf *g);
const char *ribn_amd_gguf_metadata_key(const ribn_amd_gguf *g, uint64_t index);
/* GgufFile::metadata (lib.rs:291-294): GGUF_MISSING_METADATA when absent. */
ribn_amd_status ribn_amd_gguf_metadata_get(const ribn_amd_gguf *g, const char *key, ribn_amd_gguf_value *out);
ribn_amd_status ribn_amd_gguf_metadata_array_get(const ribn_amd_gguf *g, const char *key, uint64_t index,
                                                 ribn_amd_gguf_value *out);
/* The item at `path` (depth indices) inside nested arrays of `key`
 * (MetadataValue::Array nesting, lib.rs:1111-1120); depth 0 is the value itself. */
ribn_amd_status ribn_amd_gguf_metadata_item(const ribn_amd_gguf *g, const char *key, const uint64_t *path,
                                            size_t depth, ribn_amd_gguf_value *out);
/* GgufFile::{tensors, tensor} (lib.rs:301-309) */
ribn_amd_status ribn_amd_gguf_tensor_info(const ribn_amd_gguf *g, uint64_t index, ribn_amd_gguf_tensor *out);
ribn_amd_status ribn_amd_gguf_find_tensor(const ribn_amd_gguf *g, const char *name, uint64_t *index);
/* GgufFile::tensor_data_range (lib.rs:311-339): absolute [start, end) of a
 * tensor's encoded bytes; MissingTensor, UnsupportedTensorType, the byte_len
 * errors, or TensorOffsetOutOfBounds. */
ribn_amd_status ribn_amd_gguf_tensor_data_range(const ribn_amd_gguf *g, const char *name, uint64_t *start,
                                                uint64_t *end);
/* CudaQwen35Weights::stage (staging.rs:238-292) over GgufFile::open_tensor
 * readers and CudaWeightStore::materialize_quantized (cuda.rs:321-387):
 * checks the summed encoded sizes against budget_bytes (BudgetExceeded,
 * nothing allocated), then copies each tensor's bytes unchanged into device
 * memory through pinned double buffers on the context stream, returning one
 * weight handle per name (Q4_K/Q5_K/Q6_K with [K, N] geometry checks; other
 * types as plain device bytes whose pointer ribn_amd_weight_device_ptr
 * gives). Returns after the copies complete; on error no handle is left. */
ribn_amd_status ribn_amd_gguf_stage(ribn_amd_context *ctx, const ribn_amd_gguf *g, const char *const *names,
                                    size_t count, uint64_t budget_bytes, ribn_amd_quantized_weight **out);

/* ------------------------------------------------- Q8_1 integer-dot path */

/* CudaQ8_1Quantizer::execute (crates/nvidia/src/activation.rs:52-88,
 * kernel activation.cu:1-28): packs `input_len` (a non-zero multiple of 32)
 * values into input_len / 32 blocks of nine words, half(d) | half(sum) << 16
 * then 32 int8 q = round(x / d), d = max|x| / 127. Bit-identical to the
 * reference's packer. Errors: InputLength (empty or partial block),
 * OutputLength (output_len != blocks * 9), ShapeOverflow. Lossy; the default
 * decode path does not use it. */
ribn_amd_status ribn_amd_q8_1_quantize(ribn_amd_context *ctx, const float *input, size_t input_len, uint32_t *output,
                                       size_t output_len);
/* CudaQ4KQ8_1Gemv / CudaQ5KQ8_1Gemv / CudaQ6KQ8_1Gemv::execute
 * (q4_q8_1.rs:74-133, q5_q8_1.rs, q6_q8_1.rs): y[N] from packed input of
 * K / 32 * 9 words, for the gemv handle's value type (Q4_K, Q5_K, Q6_K).
 * Errors as ribn_amd_gemv_execute, with InputLength counted in words. */
ribn_amd_status ribn_amd_gemv_execute_q8_1(ribn_amd_gemv *g, const ribn_amd_quantized_weight *w, const uint32_t *input,
                                           size_t input_len, float *output, size_t output_len);
/* ...::execute_batch (q4_q8_1.rs:135-219): `members` (1..8) batch-major packed
 * rows, weights read once, output [members][N]. members == 0: InputLength;
 * members > 8: InvalidWeight. */
ribn_amd_status ribn_amd_gemv_execute_q8_1_batch(ribn_amd_gemv *g, const ribn_amd_quantized_weight *w,
                                                 const uint32_t *input, size_t input_len, float *output,
                                                 size_t output_len, size_t members);

/* Bit-exact device dequantisation to f32 [N][K] (twin of lib.rs:596-661;
 * the reference's device equivalent is the q4_k_embedding gather, q4_k.cu:1-67). */
ribn_amd_status ribn_amd_dequantize(ribn_amd_gemv *gemv, const ribn_amd_quantized_weight *weight, float *output,
                                    size_t output_len);

/* ----------------------------------------------------------- prefill GEMM */

/* Bytes of device workspace for `tokens` x K activations plus split-K room for
 * [tokens][n] outputs (n = 0: the minimum, no split-K room). */
size_t ribn_amd_gemm_workspace_bytes(size_t tokens, size_t k, size_t n);
/* Reserves (grows, never shrinks) the context's prefill workspace for up to
 * `max_tokens` tokens of K <= max_k and N <= max_n. This is the only allocating
 * call of the prefill path, made once at set-up like the reference's decode
 * scratch (alloc_scratch / BatchScratch, decode.rs:1188-1216,1582-1617).
 * Execute calls whose activations do not fit return WorkspaceTooSmall
 * { expected: bytes needed, actual: bytes reserved }; split-K uses the rest of
 * the reservation. Synchronises the context's stream if it replaces a buffer. */
ribn_amd_status ribn_amd_context_reserve_prefill(ribn_amd_context *ctx, size_t max_tokens, size_t max_k,
                                                 size_t max_n);
/* Prefill matmul (north-star prefill path, M >= 128; the reference runs
 * prefill through gemv_batch, decode.rs:1516-1558): y[members][N] =
 * x[members][K] W^T for a Q4_K/Q5_K/Q6_K weight, x in f32 or bf16
 * (input_dtype), RMSNorm fused into the activation stage when gamma is not
 * NULL. Weights are dequantised in registers and multiplied with f16 MFMA,
 * accumulating in f32; within 1e-3 normwise relative error of the f32
 * reference. K <= 16384. */
ribn_amd_status ribn_amd_gemm_prefill(ribn_amd_gemv *gemv, const ribn_amd_quantized_weight *weight,
                                      const void *input, uint32_t input_dtype, size_t input_len, size_t members,
                                      const float *gamma, size_t gamma_len, float epsilon, float *output,
                                      size_t output_len);
/* Allocation-free variant of ribn_amd_gemm_prefill. It has no counterpart in
 * the reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, validation and kernels, but the f16 activations
 * and split-K partials live in a static 8 MiB device array per GPU instead of
 * the context's reserved workspace (no reserve call is needed). Limit: the
 * activation stage, align256(members * K * 2) + align256(members * 4) bytes,
 * must fit 8 MiB (e.g. 1024 tokens at K = 4096, 256 at K = 16384); larger
 * calls return WorkspaceTooSmall { expected: 8 MiB, actual: bytes needed }
 * before any launch. Split K uses what is left. Every call on a GPU shares
 * that GPU's array (whatever the context or stream). Calls made outside graph
 * capture are ordered through a per-GPU event: each call's stream waits for
 * the previous such call on that GPU, from any stream or context. Under
 * capture nothing is added to the graph: replays of a captured call race
 * with other calls on the GPU unless the caller orders them (one stream, or
 * a synchronisation between them). The array's address is resolved at
 * context creation, or on the first call if that failed; a GPU index past
 * 63 is InvalidArgument here only. */
ribn_amd_status ribn_amd_gemm_prefill_static(ribn_amd_gemv *gemv, const ribn_amd_quantized_weight *weight,
                                             const void *input, uint32_t input_dtype, size_t input_len,
                                             size_t members, const float *gamma, size_t gamma_len, float epsilon,
                                             float *output, size_t output_len);

/* ----------------------------------------------------------- measurement */

/* Matrix-core peak probe (no reference counterpart; it confirms the MFMA peak
 * the prefill roofline is priced against): a grid of four waves per SIMD
 * issuing independent MFMAs on register operands for `iterations` rounds,
 * timed with events on the context stream (blocking). kind 0
 * v_mfma_f32_16x16x32_f16, 1 v_mfma_f32_32x32x16_f16, 2
 * v_mfma_f32_16x16x32_bf16, 3 v_mfma_f32_16x16x4_f32. Writes the achieved
 * dense TFLOP/s. */
ribn_amd_status ribn_amd_probe_mfma_peak(ribn_amd_context *ctx, uint32_t kind, uint32_t iterations,
                                         double *tflops);

/* ------------------------------------------------------------- embedding */

/* CudaQ4KEmbedding::from_context (quantized.rs:913-960): gather kernel for a
 * [hidden, vocab] k-quant table (token_embd). The reference serves Q4_K; Q5_K
 * and Q6_K tables use the same kernel. */
ribn_amd_status ribn_amd_embedding_create(ribn_amd_context *ctx, uint32_t value_type, ribn_amd_embedding **out);
void ribn_amd_embedding_destroy(ribn_amd_embedding *embedding);
/* CudaQ4KEmbedding::execute (quantized.rs:961-1057): output[hidden] = the
 * bit-exact dequantised row `token`. token >= vocab is InvalidWeight. */
ribn_amd_status ribn_amd_embedding_execute(ribn_amd_embedding *embedding, const ribn_amd_quantized_weight *weight,
                                           uint32_t token, float *output, size_t output_len);
/* CudaQ4KEmbedding::execute_batch (quantized.rs:1058-1160): `members` token ids
 * in device memory, output [members][hidden]. Ids outside the vocabulary leave
 * their output row unwritten, as the reference kernel does (q4_k.cu:30-67). */
ribn_amd_status ribn_amd_embedding_execute_batch(ribn_amd_embedding *embedding,
                                                 const ribn_amd_quantized_weight *weight, const uint32_t *tokens,
                                                 size_t members, float *output, size_t output_len);

/* ------------------------------------------------------------- model ops */

/* CudaQwen35Ops::rms_norm (model_ops.rs:1714-1760). */
ribn_amd_status ribn_amd_rms_norm(ribn_amd_context *ctx, const float *input, size_t input_len,
                                  const float *weight, size_t weight_len, float *output, size_t output_len,
                                  float epsilon);
/* CudaQwen35Ops::rms_norm_batch (model_ops.rs:1770-1824): [members][length]. */
ribn_amd_status ribn_amd_rms_norm_batch(ribn_amd_context *ctx, const float *input, size_t input_len,
                                        const float *weight, size_t weight_len, float *output,
                                        size_t output_len, size_t length, float epsilon);

/* ------------------------------------------------------ Qwen3 decode step */

typedef struct ribn_amd_kv_cache ribn_amd_kv_cache;
typedef struct ribn_amd_qwen3_decode ribn_amd_qwen3_decode;

/* Decoder geometry. Qwen3-8B: 36 layers, hidden 4096, 32 query / 8 KV heads
 * of 128, FFN 12288, vocab 151936, rope base 1e6, RMSNorm eps 1e-6. hidden
 * and q_heads * head_dim are multiples of 256 up to 16384; ffn a multiple of
 * 256 up to 65536 (beyond 16384 the down projection runs the slice-split
 * GEMV, as for the reference's 17408-wide FFN; the prompt prefill matmul
 * still needs every K <= 16384). */
typedef struct ribn_amd_qwen3_config {
    uint32_t layers;
    uint32_t hidden;
    uint32_t q_heads;
    uint32_t kv_heads;
    uint32_t head_dim; /* 128 */
    uint32_t ffn;
    uint32_t vocab;
    float rope_base;
    float epsilon;
} ribn_amd_qwen3_config;

/* One layer's tensors: the reference's full-attention layer
 * (FULL_ATTENTION_LAYER_TENSORS, decode.rs:62-74) without a q gate, as Qwen3
 * has none. Weights are GGML [K, N] k-quant tensors; norm weights are device
 * f32 vectors, used as stored (GGUF keeps them already +1'd,
 * qwen_reference.rs:383). */
typedef struct ribn_amd_qwen3_layer {
    const ribn_amd_quantized_weight *attn_q;      /* [hidden, q_heads*head_dim] */
    const ribn_amd_quantized_weight *attn_k;      /* [hidden, kv_heads*head_dim] */
    const ribn_amd_quantized_weight *attn_v;      /* [hidden, kv_heads*head_dim] */
    const ribn_amd_quantized_weight *attn_output; /* [q_heads*head_dim, hidden] */
    const ribn_amd_quantized_weight *ffn_gate;    /* [hidden, ffn] */
    const ribn_amd_quantized_weight *ffn_up;      /* [hidden, ffn] */
    const ribn_amd_quantized_weight *ffn_down;    /* [ffn, hidden] */
    const float *attn_norm;                       /* [hidden] */
    const float *attn_q_norm;                     /* [head_dim] */
    const float *attn_k_norm;                     /* [head_dim] */
    const float *ffn_norm;                        /* [hidden] (post_attention_norm) */
} ribn_amd_qwen3_layer;

/* The KV part of the reference's per-sequence state (CudaKvState,
 * state.rs:99-254, inside CudaHybridState 529-660; F16 caches as
 * decode.rs:1000-1011 requires): f16 keys and
 * values of every layer for `capacity` tokens, laid out
 * [layer][kv_head][token][head_dim] so a KV head's tokens are contiguous, plus
 * the sequence's attention scratch. The one allocating call of a sequence. */
ribn_amd_status ribn_amd_kv_cache_create(ribn_amd_context *ctx, const ribn_amd_qwen3_config *config,
                                         uint32_t capacity, ribn_amd_kv_cache **out);
void ribn_amd_kv_cache_destroy(ribn_amd_kv_cache *cache);
uint32_t ribn_amd_kv_cache_capacity(const ribn_amd_kv_cache *cache);
/* Device views of one layer's f16 caches, [kv_heads][capacity][head_dim]
 * each (for staging a context or inspecting the cache). */
ribn_amd_status ribn_amd_kv_cache_layer(ribn_amd_kv_cache *cache, uint32_t layer, uint16_t **keys,
                                        uint16_t **values);

/* One layer's decode attention for `members` sequences, fusing the
 * reference's per-layer sequence (decode.rs:944-1020): per-head q/k RMSNorm
 * (q_gate_norm / strided_rms_norm, model_ops.rs:3784-3839, 2475-2529), NEOX
 * rope of q and k (rope_neox, 2012-2070), the f16 append of the new K/V at
 * `positions[m]` (kv_append_f16, 3854-3922) and GQA attention over tokens
 * 0..positions[m] (attn_score_gqa, 2135-2220). q is [members][q_heads*128],
 * k and v [members][kv_heads*128] (raw projections), positions a device
 * int32 array, output [members][q_heads*128]. */
ribn_amd_status ribn_amd_attention_decode(ribn_amd_context *ctx, const ribn_amd_qwen3_config *config,
                                          ribn_amd_kv_cache *const *caches, size_t members, uint32_t layer,
                                          const float *q, const float *k, const float *v, const float *q_norm,
                                          const float *k_norm, const int32_t *positions, float *output,
                                          size_t output_len);

/* One layer's attention for a prompt chunk of one sequence, as the reference's
 * full_attention_layer_prefill_chunk runs it (decode.rs:2508-2640): the K
 * (per-head RMSNorm + NEOX rope) and V of `tokens` consecutive tokens stored
 * as f16 at positions position .. position + tokens - 1 first, then token t
 * attends positions 0 .. position + t. q is [tokens][q_heads*128], k and v
 * [tokens][kv_heads*128] (raw projections), output [tokens][q_heads*128].
 * The attention runs on the matrix cores, q and the probabilities each as
 * two f16 pieces (22 significant bits), K / V f16, f32 sums; the prompt
 * prefill's attention. */
ribn_amd_status ribn_amd_attention_prefill(ribn_amd_context *ctx, const ribn_amd_qwen3_config *config,
                                           ribn_amd_kv_cache *cache, uint32_t layer, const float *q, const float *k,
                                           const float *v, const float *q_norm, const float *k_norm, size_t tokens,
                                           uint32_t position, float *output, size_t output_len);

/* CudaQwen35Ops::argmax_into / argmax_into_batch (model_ops.rs:1583-1674):
 * selected[m] = the first index of the largest non-NaN value of
 * logits[m*length .. (m+1)*length) (device u32 array), 0 when every value is
 * NaN. Its slice results use the context's scratch, in stream order. */
ribn_amd_status ribn_amd_argmax(ribn_amd_context *ctx, const float *logits, size_t logits_len, size_t length,
                                uint32_t *selected);

/* CudaQwen35Decode::new (decode.rs:412-475) and CudaQwen35BatchDecode::new
 * (1660-1690) in one: validates the plan (geometry of every tensor, non-null
 * norms) and allocates the step's device buffers for up to `max_members`
 * sequences (<= 64). Weights stay owned by the caller. `layers` is a host
 * array of config->layers entries, copied. */
ribn_amd_status ribn_amd_qwen3_decode_create(ribn_amd_context *ctx, const ribn_amd_qwen3_config *config,
                                             const ribn_amd_quantized_weight *token_embd,
                                             const ribn_amd_quantized_weight *output, const float *output_norm,
                                             const ribn_amd_qwen3_layer *layers, uint32_t max_members,
                                             ribn_amd_qwen3_decode **out);
void ribn_amd_qwen3_decode_destroy(ribn_amd_qwen3_decode *decode);
/* Steps are captured once per shape (members, caches, head or not) as HIP
 * graphs and replayed (default); disabled, every step launches its kernels
 * directly. Both run the same kernels with the same arguments. */
ribn_amd_status ribn_amd_qwen3_decode_set_graphs(ribn_amd_qwen3_decode *decode, int32_t enabled);
/* CudaQwen35Decode::set_gemv_mode / gemv_mode (decode.rs:711-741): the
 * arithmetic of every projection of later steps (RIBN_AMD_GEMV_WARP by
 * default, or RIBN_AMD_GEMV_FIXED16); an unknown mode, GemvMode::Scalar's
 * included (see the GEMV modes above), is InvalidArgument. Captured graphs
 * of the other mode are dropped. */
ribn_amd_status ribn_amd_qwen3_decode_set_gemv_mode(ribn_amd_qwen3_decode *decode, uint32_t mode);
uint32_t ribn_amd_qwen3_decode_gemv_mode(const ribn_amd_qwen3_decode *decode);
/* CudaQwen35Decode::prefill_step (decode.rs:489-499): advances `cache` by
 * `token` at `position` without the output head. Stream-ordered, not
 * blocking: a later step or copy on the context stream observes it. */
ribn_amd_status ribn_amd_qwen3_prefill_step(ribn_amd_qwen3_decode *decode, ribn_amd_kv_cache *cache,
                                            uint32_t token, uint32_t position);
/* CudaQwen35BatchDecode::prefill_chunk (decode.rs:1953-1977): `count`
 * consecutive prompt tokens of one sequence (positions position ..
 * position + count - 1, 2 <= count <= max_members) as the members of one
 * step without the output head, so the weights are read once for the chunk.
 * Every attention input equals the serial prefill_step sequence's; GEMV
 * results are the batched GEMV's: bit-equal to serial in
 * RIBN_AMD_GEMV_WARP, within the GEMV tolerance in RIBN_AMD_GEMV_FIXED16
 * from 5 members (matrix cores). Stream-ordered. */
ribn_amd_status ribn_amd_qwen3_prefill_chunk(ribn_amd_qwen3_decode *decode, ribn_amd_kv_cache *cache,
                                             const uint32_t *tokens, size_t count, uint32_t position);
/* Prompt prefill on the prefill matmul. It stands where the reference runs
 * run_prefill_chunk (decode.rs:2149-2267: the prompt's projections through
 * gemv_batch, `members` tokens at a time) and takes whole prompts: `count`
 * consecutive tokens of one sequence at positions position ..
 * position + count - 1, in chunks of up to `chunk_tokens` (16..2048; 0 means
 * 2048). Per chunk every projection runs on ribn_amd_gemm_prefill's kernels
 * over all its tokens (f16 MFMA, f32 accumulation), attention is causal over
 * the cache on the matrix cores (ribn_amd_attention_prefill's arithmetic),
 * and the chunk's K/V are written to the cache; no
 * output head. The cache then matches the serial prefill_step sequence's
 * within the prefill matmul's tolerance (not bit for bit). Needs K <= 16384
 * for every projection. The workspace for `chunk_tokens` is allocated on the
 * first call (or by ribn_amd_qwen3_reserve_prompt) and grown when a call
 * needs more, synchronising the context stream then; otherwise
 * stream-ordered (tokens travel in kernel arguments: the host array is read
 * before the call returns, and nothing waits for the stream). */
ribn_amd_status ribn_amd_qwen3_prefill_prompt(ribn_amd_qwen3_decode *decode, ribn_amd_kv_cache *cache,
                                              const uint32_t *tokens, size_t count, uint32_t position,
                                              uint32_t chunk_tokens);
/* Allocates (grows) the prompt workspace for chunks of `chunk_tokens` tokens
 * (0 means 2048) ahead of ribn_amd_qwen3_prefill_prompt. No reference
 * counterpart (the reference sizes its batch scratch at construction,
 * decode.rs:1582-1617). */
ribn_amd_status ribn_amd_qwen3_reserve_prompt(ribn_amd_qwen3_decode *decode, uint32_t chunk_tokens);
/* CudaQwen35Decode::decode_step (decode.rs:508-516): one forward pass and the
 * greedy token (blocking, as the reference). */
ribn_amd_status ribn_amd_qwen3_decode_step(ribn_amd_qwen3_decode *decode, ribn_amd_kv_cache *cache,
                                           uint32_t token, uint32_t position, uint32_t *selected);
/* CudaQwen35BatchDecode::decode_step_batch (decode.rs:1859-1872): one step for
 * `members` sequences (distinct caches); selected[m] per member. Every
 * member's result equals its single-sequence decode_step bit for bit. */
ribn_amd_status ribn_amd_qwen3_decode_step_batch(ribn_amd_qwen3_decode *decode, ribn_amd_kv_cache *const *caches,
                                                 const uint32_t *tokens, const uint32_t *positions, size_t members,
                                                 uint32_t *selected);
/* Greedy generation of `steps` tokens per member with no host round trip
 * between steps (no reference counterpart: the reference's driver calls
 * decode_step per token). Member m starts from tokens[m] at positions[m];
 * out_tokens is a host [members][steps] array. Equal to `steps` calls of
 * decode_step_batch feeding each selection back. */
ribn_amd_status ribn_amd_qwen3_generate(ribn_amd_qwen3_decode *decode, ribn_amd_kv_cache *const *caches,
                                        const uint32_t *tokens, const uint32_t *positions, size_t members,
                                        uint32_t steps, uint32_t *out_tokens);
/* copy_hidden / copy_logits (decode.rs:764-784, 1924-1930): a member's
 * residual stream [hidden] or logits [vocab] after the last step, to host. */
ribn_amd_status ribn_amd_qwen3_copy_hidden(ribn_amd_qwen3_decode *decode, size_t member, float *host, size_t len);
ribn_amd_status ribn_amd_qwen3_copy_logits(ribn_amd_qwen3_decode *decode, size_t member, float *host, size_t len);

/* ------------------------------------------------------ serving dispatcher */

/* The asynchronous serving dispatcher over one decoder
 * (CudaQwen35ServingDispatcher, crates/nvidia/src/serving.rs:81-1038) with its
 * physical state registry (CudaStateRegistry / CudaHybridState, state.rs:411-725;
 * KV family only: Qwen3 has no recurrent state) and submission ownership
 * (submissions.rs:1-47). An engine-core adapter maps ExecutionSegment /
 * InferenceStateSet onto ribn_amd_serving_row and BackendError onto the
 * statuses 38-42. One dispatcher per decoder; calls on one dispatcher must
 * not overlap (the reference takes &mut self). */
typedef struct ribn_amd_serving ribn_amd_serving;

/* ExecutionPhase (crates/core/src/execution.rs); only prefill and decode run. */
typedef enum ribn_amd_phase {
    RIBN_AMD_PHASE_PREFILL = 0,
    RIBN_AMD_PHASE_DECODE = 1,
    RIBN_AMD_PHASE_SPEC_DRAFT = 2,
    RIBN_AMD_PHASE_SPEC_VERIFY = 3,
    RIBN_AMD_PHASE_ENCODER = 4,
    RIBN_AMD_PHASE_MOE_EXPERT = 5
} ribn_amd_phase;

#define RIBN_AMD_NO_POSITION 0xffffffffu

/* One scheduler row: an ExecutionSegment with its InferenceStateSet. */
typedef struct ribn_amd_serving_row {
    uint64_t request;           /* RequestId, for messages */
    uint64_t state;             /* logical state identity (CudaStateKey::from_state_set), nonzero */
    uint32_t phase;             /* ribn_amd_phase */
    uint32_t state_position;    /* ExecutionSegment::state_position: the row's first position */
    const uint32_t *tokens;     /* host: the prompt slice (prefill) or the one decode token; null = none */
    uint32_t token_count;       /* ExecutionSegment::token_count */
    uint32_t requests_sampling; /* nonzero: the row returns a token (sampling parameters present) */
    float temperature;          /* SamplingParams temperature: only 0 (greedy) runs */
    uint32_t kv_tokens;         /* the state's KvStateSpec block tokens (KV capacity); 0: no KV state */
    uint32_t logical_position;  /* InferenceStateSet::token_position, RIBN_AMD_NO_POSITION when absent */
} ribn_amd_serving_row;

/* ExecutionOutcome: the row's wall time spent queueing and its token. */
typedef struct ribn_amd_serving_outcome {
    uint64_t elapsed_nanos;
    uint32_t has_token;
    uint32_t token;
} ribn_amd_serving_outcome;

/* CudaQwen35ServingDispatcher::new (serving.rs:281-329): `max_pending_rows`
 * (>= 1) pinned one-token output slots (hipHostMalloc) bound the sampling
 * rows in flight; decode rows run together in lanes of 2 ..
 * min(max_pending_rows, the decoder's max_members) members. KV state is
 * materialized on a state's first row, `kv_budget_bytes` bounding the
 * device bytes held by states (0: unbounded); a released state's cache is
 * kept for reuse by a later state of the same capacity (freed when the
 * budget needs the room), so release never waits on the device. The decoder
 * must outlive the dispatcher and is used on its context's stream. */
ribn_amd_status ribn_amd_serving_create(ribn_amd_qwen3_decode *decode, uint32_t max_pending_rows,
                                        uint64_t kv_budget_bytes, ribn_amd_serving **out);
/* Drains the stream and frees every state, slot and event, quarantined ones
 * included (teardown). */
void ribn_amd_serving_destroy(ribn_amd_serving *serving);
/* with_prefill_chunk (serving.rs:357-371): leading whole chunks of `members`
 * prompt tokens run as one prefill-chunk step (2 <= members <= the decoder's
 * max_members); 0 restores serial prefill. */
ribn_amd_status ribn_amd_serving_set_prefill_chunk(ribn_amd_serving *serving, uint32_t members);
/* No reference counterpart (the reference prefills through prefill_chunk
 * and prefill_step, serving.rs:136-160,357-371): with chunk_tokens != 0 a
 * prefill segment's tokens other than the sampling one, when at least 16,
 * run as one ribn_amd_qwen3_prefill_prompt call in chunks of chunk_tokens
 * (16..2048); shorter prefixes keep the prefill-chunk / serial path. Results
 * are within the prefill matmul's tolerance of serial prefill, not bit-equal.
 * Allocates the decoder's prompt workspace now (synchronising its stream),
 * so submissions neither allocate nor wait. 0 turns the lane off. */
ribn_amd_status ribn_amd_serving_set_prompt_prefill(ribn_amd_serving *serving, uint32_t chunk_tokens);
/* with_grouped_decode (serving.rs:337-341): compatible decode rows of mixed
 * batches are gathered into lanes (opt-in, as in the reference). */
ribn_amd_status ribn_amd_serving_set_grouped_decode(ribn_amd_serving *serving, int32_t enabled);

/* NvidiaDispatcher::dispatch_batch (serving.rs:854-882): eager execution of
 * every row in order; returns after the stream drained. outcomes[count]. */
ribn_amd_status ribn_amd_serving_dispatch_batch(ribn_amd_serving *serving, const ribn_amd_serving_row *rows,
                                                size_t count, ribn_amd_serving_outcome *outcomes);
/* NvidiaDispatcher::submit_batch (serving.rs:884-958): queues the batch
 * without blocking (all-decode batches as one batched step unless grouped
 * decode is on, otherwise rows in order with grouped lanes) and records one
 * completion event. `submission` is a nonzero id, unique among pending ones.
 * An error means nothing of the batch stays queued (or, after a device
 * fault, its resources are quarantined). */
ribn_amd_status ribn_amd_serving_submit_batch(ribn_amd_serving *serving, uint64_t submission,
                                              const ribn_amd_serving_row *rows, size_t count);
/* NvidiaDispatcher::poll_batch (serving.rs:960-1016): *ready = 0 while the
 * completion event is pending; once complete, writes outcomes[count] (count =
 * the submitted row count) and forgets the submission. A device fault poisons
 * the dispatcher (RIBN_AMD_DEVICE_FAULTED on every later call). */
ribn_amd_status ribn_amd_serving_poll_batch(ribn_amd_serving *serving, uint64_t submission,
                                            ribn_amd_serving_outcome *outcomes, size_t count, int32_t *ready);
/* release_inference_state (serving.rs:1018-1038): frees the state's physical
 * KV now, or when the last pending submission using it completes. Missing
 * state is a no-op; refused while a failed drain keeps ownership uncertain. */
ribn_amd_status ribn_amd_serving_release_state(ribn_amd_serving *serving, uint64_t state);

/* Introspection: pending submissions, materialized states, device bytes held
 * by states (in use and kept for reuse), a state's physical position. */
size_t ribn_amd_serving_pending(const ribn_amd_serving *serving);
size_t ribn_amd_serving_state_count(const ribn_amd_serving *serving);
uint64_t ribn_amd_serving_state_bytes(const ribn_amd_serving *serving, uint64_t *reusable_bytes);
ribn_amd_status ribn_amd_serving_state_position(const ribn_amd_serving *serving, uint64_t state,
                                                uint32_t *position);

/* Host-only scheduling rules (no device access).
 * chunked_prefix_len (serving.rs:111-118): the leading tokens of a prefill of
 * `token_count` tokens that run as whole chunks of `members`; a sampling
 * prefill keeps its last token serial. */
uint32_t ribn_amd_serving_chunked_prefix_len(uint32_t token_count, uint32_t members, int32_t requests_sampling);
/* decode_group (serving.rs:520-550): the rows, from `first` on, that run as one
 * decode lane with row `first` (single-token sampling decode rows with a
 * token, a logical position and a KV state of the same spec as `first`'s,
 * not yet scheduled, at most `max_members`), in row order; just `first` when
 * it is not eligible. Writes indices to out (capacity count), returns how
 * many. */
size_t ribn_amd_serving_decode_group(const ribn_amd_serving_row *rows, size_t count, const uint8_t *scheduled,
                                     size_t first, size_t max_members, size_t *out);

/* Loading-time memory plan (crates/qwen/src/loading.rs:117-132, 200-213):
 * continuation = per_sequence_state_bytes * max_sequences (or the given
 * override when nonzero); available = free - continuation - headroom;
 * the weight budget is `requested_weight_budget` (0: all available), and it
 * must be nonzero and within the available bytes. */
typedef struct ribn_amd_memory_plan {
    uint64_t free_before_preparation_bytes;
    uint64_t weight_budget_bytes;
    uint64_t reserved_sequence_bytes;
} ribn_amd_memory_plan;
ribn_amd_status ribn_amd_plan_memory(ribn_amd_context *ctx, uint64_t per_sequence_state_bytes,
                                     uint64_t max_sequences, uint64_t continuation_override,
                                     uint64_t headroom_bytes, uint64_t requested_weight_budget,
                                     ribn_amd_memory_plan *out);
/* KvStateSpec::byte_size (crates/core/src/state.rs:112-119) of a Qwen3
 * sequence of `tokens`: layers * kv_heads * head_dim * tokens * 2 (K and V)
 * * 2 bytes (f16). 147,456 bytes per token at Qwen3-8B geometry. */
uint64_t ribn_amd_qwen3_kv_bytes(const ribn_amd_qwen3_config *config, uint32_t tokens);

#ifdef __cplusplus
}
#endif

#endif /* RIBN_AMD_H */

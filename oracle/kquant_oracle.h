/*
 * CPU oracle for the k-quant decode path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's host k-quant decoder and its host
 * GEMV / RMSNorm equations. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker or as the
 * timed CPU baseline; the product library (engine_amd) never links or calls it.
 *
 * The reference is Rust (nijaru/engine crates/gguf, crates/nvidia); there is no
 * Rust toolchain in this image, so the reference itself cannot be built and the
 * functions below restate it statement by statement, citing file:line.
 * Compile with -O2 -ffp-contract=off and without -ffast-math: the op order and
 * rounding of every f32 operation below is part of the contract.
 *
 * Pins (tests/test_oracle.py): the reference's KATs (crates/gguf/src/lib.rs
 * :1369-1514), the reference's fixture encoders with their exact f64 closed
 * forms (crates/nvidia/tests/q{4,5,6}_q8_1.rs fixture()), all 65536 binary16
 * patterns against numpy's IEEE conversion, the GGML scale packing round trip
 * over all 64x64 (scale, min) pairs, an independent vectorised numpy decoder,
 * and a float64 bound on the sequential f32 dot.
 */
#ifndef KQUANT_ORACLE_H
#define KQUANT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML value types on the path (crates/gguf/src/lib.rs:1051-1083). */
enum {
    ORACLE_TYPE_F32 = 0,
    ORACLE_TYPE_F16 = 1,
    ORACLE_TYPE_Q8_0 = 8,
    ORACLE_TYPE_Q4_K = 12,
    ORACLE_TYPE_Q5_K = 13,
    ORACLE_TYPE_Q6_K = 14,
};

/* Status codes mirroring engine_gguf::GgufError variants used on this path. */
enum {
    ORACLE_OK = 0,
    ORACLE_UNSUPPORTED_TYPE = 1,        /* GgufError::UnsupportedTensorType */
    ORACLE_INVALID_BLOCK_LENGTH = 2,    /* GgufError::InvalidTensorBlockLength */
    ORACLE_DIMENSION_MISMATCH = 3,      /* GgufError::QuantizationDimensionMismatch */
    ORACLE_BLOCK_MISMATCH = 4,          /* GgufError::QuantizationBlockMismatch */
    ORACLE_OVERFLOW = 5,                /* GgufError::TensorByteLengthOverflow */
    ORACLE_INVALID_DIMENSION_COUNT = 6, /* GgufError::InvalidDimensionCount */
    ORACLE_OUT_OF_SCOPE = 7,            /* decodable by the reference, not restated here */
    ORACLE_BAD_ARGUMENT = 8,            /* shape / length misuse of the oracle itself */
};

/* lib.rs:551-563 f16_to_f32 (NaN -> canonical f32 NaN 0x7fc00000). */
float oracle_f16_to_f32(uint16_t bits);

/* lib.rs:1051-1083 tensor_layout: (block elements, block bytes) per type. */
int oracle_tensor_layout(uint32_t value_type, uint64_t *block_elements, uint64_t *block_bytes);

/* lib.rs:138-163 TensorInfo::byte_len. */
int oracle_byte_len(const uint64_t *dims, size_t ndims, uint32_t value_type, uint64_t *out_bytes);

/* lib.rs:573-587 q4_k_scales: 12 packed bytes -> 8 six-bit scales, 8 six-bit mins. */
void oracle_q4_k_scales(const uint8_t *packed12, uint8_t scales[8], uint8_t minima[8]);

/*
 * lib.rs:520-547 dequantize_block. Writes the decoded values of exactly one
 * block to out (capacity out_cap). *expected_len receives the block length the
 * type requires (the `expected` field of InvalidTensorBlockLength).
 */
int oracle_dequantize_block(uint32_t value_type, const uint8_t *encoded, size_t len,
                            float *out, size_t out_cap, size_t *expected_len);

/* Block-by-block dequantisation of a whole tensor (n_blocks consecutive blocks). */
int oracle_dequantize_tensor(uint32_t value_type, const uint8_t *encoded, size_t len,
                             float *out, size_t out_len);

/* crates/nvidia/src/qwen_reference.rs:31-40 gguf_gemv on dequantised f32 weights. */
int oracle_gguf_gemv(const float *weight, size_t weight_len, size_t in_dim,
                     const float *x, float *y);

/*
 * Quantised GEMV exactly as the reference's device tests compose it
 * (crates/nvidia/tests/cuda_reference.rs:889-902): per row, dequantize_block per
 * block, then one sequential f32 sum over all K products. Batch-major members:
 * x is [members][K], y is [members][N].
 */
int oracle_quant_gemv(uint32_t value_type, const uint8_t *encoded, size_t len,
                      size_t k, size_t n, const float *x, float *y, size_t members);

/* Same arithmetic, rows split over `threads` OpenMP threads (CPU baseline variant ii). */
int oracle_quant_gemv_threads(uint32_t value_type, const uint8_t *encoded, size_t len,
                              size_t k, size_t n, const float *x, float *y, int threads);

/* qwen_reference.rs:550-556 rms_norm_raw. */
int oracle_rms_norm_raw(const float *input, const float *weight, size_t len, float eps,
                        float *out);

/* qwen_reference.rs:529-539 SwiGLU composition g/(1+exp(-g))*u. */
void oracle_swiglu(const float *gate, const float *up, size_t len, float *out);

/* model_ops.rs:1211-1250 f32_to_f16_bits: IEEE binary16, round to nearest even. */
uint16_t oracle_f32_to_f16_bits(float value);

/* qwen_reference.rs:403-419 NEOX rope (pair stride rot_dims/2, theta_p = pos*base^(-2p/rot_dims)). */
void oracle_rope_neox(float *values, size_t heads, size_t head_dim, size_t rot_dims, size_t pos,
                      float base);

/*
 * qwen_reference.rs:368-455 one attention step, Qwen3 geometry (no q gate), F16
 * cache as the device decode keeps it (decode.rs:997-1033). Caches are
 * [capacity][kv_heads][head_dim] binary16 bits; the step writes slot `pos` and
 * attends over 0..pos. out is [q_heads][head_dim].
 */
int oracle_qwen3_attention(const float *q_raw, const float *k_raw, const float *v_raw,
                           const float *q_norm, const float *k_norm, float eps, float rope_base,
                           size_t q_heads, size_t kv_heads, size_t head_dim, size_t pos,
                           uint16_t *kv_keys, uint16_t *kv_values, size_t capacity,
                           float *out);

/* model_ops.rs:201-258 argmax: first index of the largest non-NaN value. */
size_t oracle_argmax(const float *logits, size_t len);

/*
 * Times the CPU baseline (dequantize_block + sequential f32 dot per row) with
 * steady-clock timing: `warmup` untimed runs, then `iters` timed runs. Writes
 * median and minimum seconds per run. threads == 1 is the faithful
 * single-threaded reference path; threads > 1 splits rows with OpenMP.
 */
int oracle_time_quant_gemv(uint32_t value_type, const uint8_t *encoded, size_t len,
                           size_t k, size_t n, const float *x, float *y, int threads,
                           int warmup, int iters, double *median_s, double *min_s);

#ifdef __cplusplus
}
#endif

#endif /* KQUANT_ORACLE_H */

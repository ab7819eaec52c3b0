/*
 * CPU oracle for the k-quant decode path -- TEST INFRASTRUCTURE ONLY.
 * See kquant_oracle.h for scope, pins and build flags (-O2 -ffp-contract=off).
 *
 * Every function restates the cited reference source statement by statement;
 * f32 expressions keep the reference's evaluation order so results are
 * bit-identical to the Rust code (Rust never contracts a*b-c into an FMA).
 */
#include "kquant_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK_K 256

/* crates/gguf/src/lib.rs:551-563 */
float oracle_f16_to_f32(uint16_t bits)
{
    const float sign = (bits & 0x8000u) == 0 ? 1.0f : -1.0f;
    const unsigned exponent = (bits >> 10) & 0x1fu;
    const unsigned fraction = bits & 0x03ffu;
    if (exponent == 0) {
        /* sign * f32::from(fraction) * 2_f32.powi(-24) */
        return sign * (float)fraction * 5.9604644775390625e-08f;
    }
    if (exponent == 0x1f) {
        if (fraction == 0) {
            return sign * INFINITY;
        }
        /* f32::NAN: the canonical quiet NaN regardless of payload and sign */
        uint32_t canonical = 0x7fc00000u;
        float nan_value;
        memcpy(&nan_value, &canonical, sizeof nan_value);
        return nan_value;
    }
    /* sign * (1.0 + f32::from(fraction) / 1024.0) * 2_f32.powi(exponent - 15) */
    return sign * (1.0f + (float)fraction / 1024.0f) * ldexpf(1.0f, (int)exponent - 15);
}

/* lib.rs:565-567 read_f16: little-endian binary16 at `offset`. */
static float read_f16(const uint8_t *encoded, size_t offset)
{
    return oracle_f16_to_f32((uint16_t)(encoded[offset] | (encoded[offset + 1] << 8)));
}

/* lib.rs:1051-1083 tensor_layout */
int oracle_tensor_layout(uint32_t value_type, uint64_t *block_elements, uint64_t *block_bytes)
{
    uint64_t e, b;
    switch (value_type) {
    case 0: case 26: e = 1; b = 4; break;
    case 1: case 25: case 30: e = 1; b = 2; break;
    case 2: case 20: e = 32; b = 18; break;
    case 3: e = 32; b = 20; break;
    case 6: e = 32; b = 22; break;
    case 7: e = 32; b = 24; break;
    case 8: e = 32; b = 34; break;
    case 9: e = 32; b = 36; break;
    case 10: e = 256; b = 84; break;
    case 11: case 21: e = 256; b = 110; break;
    case 12: e = 256; b = 144; break;
    case 13: e = 256; b = 176; break;
    case 14: e = 256; b = 210; break;
    case 15: e = 256; b = 292; break;
    case 16: case 35: e = 256; b = 66; break;
    case 17: e = 256; b = 74; break;
    case 18: e = 256; b = 98; break;
    case 19: e = 256; b = 50; break;
    case 22: e = 256; b = 82; break;
    case 23: e = 256; b = 136; break;
    case 24: e = 1; b = 1; break;
    case 27: case 28: e = 1; b = 8; break;
    case 29: e = 256; b = 56; break;
    case 34: e = 256; b = 54; break;
    case 39: e = 32; b = 17; break;
    case 40: e = 64; b = 36; break;
    case 41: e = 128; b = 18; break;
    case 42: e = 64; b = 18; break;
    default: return ORACLE_UNSUPPORTED_TYPE;
    }
    if (block_elements) *block_elements = e;
    if (block_bytes) *block_bytes = b;
    return ORACLE_OK;
}

/* lib.rs:138-163 TensorInfo::byte_len (element_count: product of dims, checked). */
int oracle_byte_len(const uint64_t *dims, size_t ndims, uint32_t value_type, uint64_t *out_bytes)
{
    uint64_t block_elements, block_bytes;
    int status = oracle_tensor_layout(value_type, &block_elements, &block_bytes);
    if (status != ORACLE_OK) return status;
    if (ndims == 0) return ORACLE_INVALID_DIMENSION_COUNT;
    if (dims[0] % block_elements != 0) return ORACLE_DIMENSION_MISMATCH;
    uint64_t elements = 1;
    for (size_t i = 0; i < ndims; ++i) {
        if (dims[i] != 0 && elements > UINT64_MAX / dims[i]) return ORACLE_OVERFLOW;
        elements *= dims[i];
    }
    if (elements % block_elements != 0) return ORACLE_BLOCK_MISMATCH;
    uint64_t blocks = elements / block_elements;
    if (block_bytes != 0 && blocks > UINT64_MAX / block_bytes) return ORACLE_OVERFLOW;
    *out_bytes = blocks * block_bytes;
    return ORACLE_OK;
}

/* lib.rs:573-587 q4_k_scales */
void oracle_q4_k_scales(const uint8_t *encoded, uint8_t scales[8], uint8_t minima[8])
{
    for (int index = 0; index < 4; ++index) {
        const uint8_t low_scale = encoded[index] & 0x3f;
        const uint8_t high_scale = (uint8_t)((encoded[8 + index] & 0x0f) | ((encoded[index] >> 2) & 0x30));
        const uint8_t low_min = encoded[4 + index] & 0x3f;
        const uint8_t high_min = (uint8_t)((encoded[8 + index] >> 4) | ((encoded[4 + index] >> 2) & 0x30));
        scales[index] = low_scale;
        scales[index + 4] = high_scale;
        minima[index] = low_min;
        minima[index + 4] = high_min;
    }
}

/* lib.rs:589-594 dequantize_q8_0 */
static void dequantize_q8_0(const uint8_t *encoded, float *output)
{
    const float scale = read_f16(encoded, 0);
    for (int index = 0; index < 32; ++index) {
        output[index] = scale * (float)(int8_t)encoded[2 + index];
    }
}

/* lib.rs:596-612 dequantize_q4_k */
static void dequantize_q4_k(const uint8_t *encoded, float *output)
{
    const float scale = read_f16(encoded, 0);
    const float minimum_scale = read_f16(encoded, 2);
    uint8_t scales[8], minima[8];
    oracle_q4_k_scales(encoded + 4, scales, minima);
    size_t out = 0;
    for (int group = 0; group < 8; ++group) {
        const int data_offset = 16 + (group / 2) * 32;
        const int shift = (group % 2) * 4;
        const float group_scale = scale * (float)scales[group];
        const float group_minimum = minimum_scale * (float)minima[group];
        for (int index = 0; index < 32; ++index) {
            const uint8_t quantized = (encoded[data_offset + index] >> shift) & 0x0f;
            output[out++] = group_scale * (float)quantized - group_minimum;
        }
    }
}

/* lib.rs:614-633 dequantize_q5_k */
static void dequantize_q5_k(const uint8_t *encoded, float *output)
{
    const float scale = read_f16(encoded, 0);
    const float minimum_scale = read_f16(encoded, 2);
    uint8_t scales[8], minima[8];
    oracle_q4_k_scales(encoded + 4, scales, minima);
    const uint8_t *high_bits = encoded + 16;
    const uint8_t *low_bits = encoded + 48;
    size_t out = 0;
    for (int group = 0; group < 8; ++group) {
        const int data_offset = (group / 2) * 32;
        const int shift = (group % 2) * 4;
        const float group_scale = scale * (float)scales[group];
        const float group_minimum = minimum_scale * (float)minima[group];
        for (int index = 0; index < 32; ++index) {
            const uint8_t low = (low_bits[data_offset + index] >> shift) & 0x0f;
            const uint8_t high = (high_bits[index] >> group) & 1;
            output[out++] = group_scale * (float)(uint8_t)(low | (high << 4)) - group_minimum;
        }
    }
}

/* lib.rs:635-661 dequantize_q6_k */
static void dequantize_q6_k(const uint8_t *encoded, float *output)
{
    const uint8_t *low_bits = encoded;
    const uint8_t *high_bits = encoded + 128;
    const uint8_t *scales = encoded + 192;
    const float scale = read_f16(encoded, 208);
    size_t out = 0;
    for (int group = 0; group < 8; ++group) {
        const int chunk = group / 4;
        const int variant = group % 4;
        const int low_offset = chunk * 64 + (variant % 2) * 32;
        const int low_shift = variant < 2 ? 0 : 4;
        const int high_offset = chunk * 32;
        const int high_shift = variant % 4;
        for (int half = 0; half < 2; ++half) {
            const int scale_index = group * 2 + half;
            const float group_scale = scale * (float)(int8_t)scales[scale_index];
            for (int index = 0; index < 16; ++index) {
                const int position = half * 16 + index;
                const uint8_t low = (low_bits[low_offset + position] >> low_shift) & 0x0f;
                const uint8_t high = (high_bits[high_offset + position] >> (high_shift * 2)) & 0x03;
                const int16_t quantized = (int16_t)((int16_t)(low | (high << 4)) - 32);
                output[out++] = group_scale * (float)quantized;
            }
        }
    }
}

/* lib.rs:520-547 dequantize_block */
int oracle_dequantize_block(uint32_t value_type, const uint8_t *encoded, size_t len,
                            float *out, size_t out_cap, size_t *expected_len)
{
    uint64_t block_elements, block_bytes;
    int status = oracle_tensor_layout(value_type, &block_elements, &block_bytes);
    if (status != ORACLE_OK) return status;
    if (expected_len) *expected_len = (size_t)block_bytes;
    if (len != block_bytes) return ORACLE_INVALID_BLOCK_LENGTH;
    switch (value_type) {
    case 0:
    case 1:
    case 8:
    case 12:
    case 13:
    case 14:
        break;
    case 11: case 20: case 21: case 23:
        /* Q3_K / IQ4_NL / IQ3_S / IQ4_XS: decodable by the reference, not on this path. */
        return ORACLE_OUT_OF_SCOPE;
    default:
        return ORACLE_UNSUPPORTED_TYPE;
    }
    if (out_cap < block_elements) return ORACLE_BAD_ARGUMENT;
    switch (value_type) {
    case 0: {
        float value;
        memcpy(&value, encoded, sizeof value); /* f32::from_le_bytes on a little-endian host */
        out[0] = value;
        break;
    }
    case 1: out[0] = read_f16(encoded, 0); break;
    case 8: dequantize_q8_0(encoded, out); break;
    case 12: dequantize_q4_k(encoded, out); break;
    case 13: dequantize_q5_k(encoded, out); break;
    case 14: dequantize_q6_k(encoded, out); break;
    }
    return ORACLE_OK;
}

int oracle_dequantize_tensor(uint32_t value_type, const uint8_t *encoded, size_t len,
                             float *out, size_t out_len)
{
    uint64_t block_elements, block_bytes;
    int status = oracle_tensor_layout(value_type, &block_elements, &block_bytes);
    if (status != ORACLE_OK) return status;
    if (len % block_bytes != 0) return ORACLE_INVALID_BLOCK_LENGTH;
    const size_t blocks = len / block_bytes;
    if (out_len != blocks * block_elements) return ORACLE_BAD_ARGUMENT;
    for (size_t b = 0; b < blocks; ++b) {
        status = oracle_dequantize_block(value_type, encoded + b * block_bytes, (size_t)block_bytes,
                                         out + b * block_elements, (size_t)block_elements, NULL);
        if (status != ORACLE_OK) return status;
    }
    return ORACLE_OK;
}

/*
 * qwen_reference.rs:31-40 gguf_gemv: y[n] = sum_k x[k] * W[n*K + k], a sequential
 * f32 fold. Rust's float Sum starts from -0.0, which only changes the sign of an
 * exactly-zero result.
 */
int oracle_gguf_gemv(const float *weight, size_t weight_len, size_t in_dim,
                     const float *x, float *y)
{
    if (in_dim == 0 || weight_len % in_dim != 0) return ORACLE_BAD_ARGUMENT;
    const size_t rows = weight_len / in_dim;
    for (size_t n = 0; n < rows; ++n) {
        const float *column = weight + n * in_dim;
        float sum = -0.0f;
        for (size_t k = 0; k < in_dim; ++k) {
            sum += x[k] * column[k];
        }
        y[n] = sum;
    }
    return ORACLE_OK;
}

static int quant_geometry(uint32_t value_type, size_t len, size_t k, size_t n,
                          size_t *blocks_per_row, size_t *block_bytes_out)
{
    uint64_t block_elements, block_bytes;
    int status = oracle_tensor_layout(value_type, &block_elements, &block_bytes);
    if (status != ORACLE_OK) return status;
    if (value_type != 12 && value_type != 13 && value_type != 14) return ORACLE_OUT_OF_SCOPE;
    if (k == 0 || n == 0 || k % block_elements != 0) return ORACLE_BAD_ARGUMENT;
    if (len != (k / block_elements) * n * block_bytes) return ORACLE_BAD_ARGUMENT;
    *blocks_per_row = k / block_elements;
    *block_bytes_out = (size_t)block_bytes;
    return ORACLE_OK;
}

/* One output row: dequantize_block per block, one sequential sum over K
 * (cuda_reference.rs:889-902: flat_map over blocks, zip with x, .sum()). */
static float quant_row(uint32_t value_type, const uint8_t *row, size_t blocks_per_row,
                       size_t block_bytes, const float *x)
{
    float decoded[QK_K];
    float sum = -0.0f;
    for (size_t b = 0; b < blocks_per_row; ++b) {
        oracle_dequantize_block(value_type, row + b * block_bytes, block_bytes, decoded, QK_K, NULL);
        const float *xb = x + b * QK_K;
        for (int i = 0; i < QK_K; ++i) {
            sum += decoded[i] * xb[i];
        }
    }
    return sum;
}

int oracle_quant_gemv(uint32_t value_type, const uint8_t *encoded, size_t len,
                      size_t k, size_t n, const float *x, float *y, size_t members)
{
    size_t blocks_per_row, block_bytes;
    int status = quant_geometry(value_type, len, k, n, &blocks_per_row, &block_bytes);
    if (status != ORACLE_OK) return status;
    if (members == 0) return ORACLE_BAD_ARGUMENT;
    for (size_t m = 0; m < members; ++m) {
        for (size_t row = 0; row < n; ++row) {
            y[m * n + row] = quant_row(value_type, encoded + row * blocks_per_row * block_bytes,
                                       blocks_per_row, block_bytes, x + m * k);
        }
    }
    return ORACLE_OK;
}

int oracle_quant_gemv_threads(uint32_t value_type, const uint8_t *encoded, size_t len,
                              size_t k, size_t n, const float *x, float *y, int threads)
{
    size_t blocks_per_row, block_bytes;
    int status = quant_geometry(value_type, len, k, n, &blocks_per_row, &block_bytes);
    if (status != ORACLE_OK) return status;
    if (threads < 1) return ORACLE_BAD_ARGUMENT;
    long rows = (long)n;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (long row = 0; row < rows; ++row) {
        y[row] = quant_row(value_type, encoded + (size_t)row * blocks_per_row * block_bytes,
                           blocks_per_row, block_bytes, x);
    }
    return ORACLE_OK;
}

/* qwen_reference.rs:550-556 rms_norm_raw */
int oracle_rms_norm_raw(const float *input, const float *weight, size_t len, float eps,
                        float *out)
{
    /* u16::try_from(input.len()).expect(..): the reference panics above 65535 */
    if (len == 0 || len > 65535) return ORACLE_BAD_ARGUMENT;
    float sum = -0.0f;
    for (size_t i = 0; i < len; ++i) {
        sum += input[i] * input[i];
    }
    const float count = (float)len;
    const float inv = 1.0f / sqrtf(sum / count + eps);
    for (size_t i = 0; i < len; ++i) {
        out[i] = input[i] * inv * weight[i];
    }
    return ORACLE_OK;
}

/* qwen_reference.rs:529-539: g / (1 + exp(-g)) * u */
void oracle_swiglu(const float *gate, const float *up, size_t len, float *out)
{
    for (size_t i = 0; i < len; ++i) {
        const float g = gate[i];
        out[i] = g / (1.0f + expf(-g)) * up[i];
    }
}

/*
 * f32 -> IEEE binary16 bits, round to nearest even: the conversion the
 * reference's device KV append applies (crates/nvidia/src/model_ops.rs
 * :1211-1250 f32_to_f16_bits). Restated from the IEEE 754 definition; NaN
 * keeps its sign and becomes the quiet NaN 0x7e00 as in the reference.
 */
uint16_t oracle_f32_to_f16_bits(float value)
{
    uint32_t bits;
    memcpy(&bits, &value, sizeof bits);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const uint32_t biased = (bits >> 23) & 0xffu;
    const uint32_t frac = bits & 0x7fffffu;
    if (biased == 0xffu) return (uint16_t)(sign | 0x7c00u | (frac ? 0x0200u : 0u));
    const int e = (int)biased - 127; /* unbiased exponent of a normal f32 */
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    /* the value's magnitude is m * 2^(e-23) with m the 24-bit significand */
    const uint32_t m = biased ? (frac | 0x800000u) : frac;
    /* target unit: 2^-24 for subnormal halves (e < -14), else 2^(e-10) */
    const int unit_exp = e < -14 ? -24 : e - 10;
    const int shift = (biased ? e - 23 : -149) - unit_exp; /* m * 2^shift units */
    uint32_t q;
    if (shift >= 0) {
        q = m << shift;
    } else if (shift < -25) {
        q = 0;
    } else {
        const int r = -shift;
        q = m >> r;
        const uint32_t rem = m & ((1u << r) - 1u);
        const uint32_t half = 1u << (r - 1);
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
    }
    if (e < -14) {
        /* subnormal half: q counts 2^-24; q == 1024 rounds up into the normals */
        return (uint16_t)(sign | q);
    }
    /* normal half: q in [1024, 2048]; 2048 carries into the exponent */
    int he = e + 15;
    if (q >= 2048u) {
        q >>= 1;
        he += 1;
    }
    if (he >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)he << 10) | (q & 0x3ffu));
}

/*
 * NEOX rope over `heads` heads of head_dim values: pair (p, p + rot_dims/2)
 * of the first rot_dims dims rotates by theta_p = pos * base^(-2p/rot_dims)
 * (crates/nvidia/src/qwen_reference.rs:403-419 apply_rope, with the pair stride
 * rot_dims/2 that rope_neox uses for any rot_dims, model_ops.rs:393-425).
 */
void oracle_rope_neox(float *values, size_t heads, size_t head_dim, size_t rot_dims, size_t pos,
                      float base)
{
    const size_t half = rot_dims / 2;
    for (size_t head = 0; head < heads; ++head) {
        const size_t b = head * head_dim;
        for (size_t pair = 0; pair < half; ++pair) {
            const float theta = (float)pos * powf(base, -(2.0f * (float)pair) / (float)rot_dims);
            const float sn = sinf(theta), cs = cosf(theta);
            const float x0 = values[b + pair];
            const float x1 = values[b + half + pair];
            values[b + pair] = x0 * cs - x1 * sn;
            values[b + half + pair] = x0 * sn + x1 * cs;
        }
    }
}

/*
 * One decode step's attention for a Qwen3 layer:
 * crates/nvidia/src/qwen_reference.rs:368-455 host_full_attn_ar_step_traced with
 * Qwen3's geometry (no q gate: q_raw is [q_heads][head_dim]; full-width rope)
 * and the device decode's F16 cache (decode.rs:997-1033: kv_append_f16 then
 * attention over the F16 cache).
 *   per-head RMSNorm of q and k (rms_norm_raw with the shared head weight),
 *   rope of q and k at `pos`,
 *   kv_keys/kv_values[pos] = f16(k), f16(v)    ([capacity][kv_heads][head_dim]),
 *   out[h] = softmax(q_h . K_t * scale) . V_t over t = 0..pos, KV head h / (q_heads / kv_heads).
 * q_scratch and k_scratch hold q_heads*head_dim and kv_heads*head_dim floats.
 */
int oracle_qwen3_attention(const float *q_raw, const float *k_raw, const float *v_raw,
                           const float *q_norm, const float *k_norm, float eps, float rope_base,
                           size_t q_heads, size_t kv_heads, size_t head_dim, size_t pos,
                           uint16_t *kv_keys, uint16_t *kv_values, size_t capacity,
                           float *out)
{
    if (q_heads == 0 || kv_heads == 0 || q_heads % kv_heads || head_dim == 0 || head_dim > 65535 ||
        pos >= capacity) {
        return ORACLE_BAD_ARGUMENT;
    }
    float *q = malloc(q_heads * head_dim * sizeof *q);
    float *k = malloc(kv_heads * head_dim * sizeof *k);
    float *scores = malloc((pos + 1) * sizeof *scores);
    float *exps = malloc((pos + 1) * sizeof *exps);
    if (!q || !k || !scores || !exps) {
        free(q); free(k); free(scores); free(exps);
        return ORACLE_BAD_ARGUMENT;
    }
    for (size_t h = 0; h < q_heads; ++h) {
        oracle_rms_norm_raw(q_raw + h * head_dim, q_norm, head_dim, eps, q + h * head_dim);
    }
    for (size_t h = 0; h < kv_heads; ++h) {
        oracle_rms_norm_raw(k_raw + h * head_dim, k_norm, head_dim, eps, k + h * head_dim);
    }
    oracle_rope_neox(q, q_heads, head_dim, head_dim, pos, rope_base);
    oracle_rope_neox(k, kv_heads, head_dim, head_dim, pos, rope_base);
    const size_t row = kv_heads * head_dim;
    for (size_t i = 0; i < row; ++i) {
        kv_keys[pos * row + i] = oracle_f32_to_f16_bits(k[i]);
        kv_values[pos * row + i] = oracle_f32_to_f16_bits(v_raw[i]);
    }
    const size_t tokens = pos + 1;
    const size_t q_per_kv = q_heads / kv_heads;
    /* 1.0 / f32::sqrt(f32::from(head_dim)) */
    const float scale = 1.0f / sqrtf((float)head_dim);
    for (size_t qh = 0; qh < q_heads; ++qh) {
        const size_t kvh = qh / q_per_kv;
        const float *qv = q + qh * head_dim;
        for (size_t t = 0; t < tokens; ++t) {
            const uint16_t *key = kv_keys + (t * kv_heads + kvh) * head_dim;
            float dot = -0.0f;
            for (size_t d = 0; d < head_dim; ++d) dot += qv[d] * oracle_f16_to_f32(key[d]);
            scores[t] = dot * scale;
        }
        float mx = -INFINITY;
        for (size_t t = 0; t < tokens; ++t) mx = fmaxf(mx, scores[t]);
        float total = -0.0f;
        for (size_t t = 0; t < tokens; ++t) {
            exps[t] = expf(scores[t] - mx);
            total += exps[t];
        }
        float *o = out + qh * head_dim;
        for (size_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
        for (size_t t = 0; t < tokens; ++t) {
            const uint16_t *value = kv_values + (t * kv_heads + kvh) * head_dim;
            const float weight = exps[t] / total;
            for (size_t d = 0; d < head_dim; ++d) o[d] += weight * oracle_f16_to_f32(value[d]);
        }
    }
    free(q); free(k); free(scores); free(exps);
    return ORACLE_OK;
}

/* decode.rs:655-677 argmax_into: first index of the largest non-NaN value
 * (model_ops.rs:201-258 key order: -0.0 ranks below +0.0). */
size_t oracle_argmax(const float *logits, size_t len)
{
    uint32_t best_key = 0;
    size_t best = 0;
    for (size_t i = 0; i < len; ++i) {
        const float v = logits[i];
        if (v != v) continue;
        uint32_t bits;
        memcpy(&bits, &v, sizeof bits);
        const uint32_t key = (bits >> 31) ? ~bits : (bits ^ 0x80000000u);
        if (key > best_key) {
            best_key = key;
            best = i;
        }
    }
    return best;
}

static double now_seconds(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static int compare_double(const void *a, const void *b)
{
    const double x = *(const double *)a, y = *(const double *)b;
    return (x > y) - (x < y);
}

int oracle_time_quant_gemv(uint32_t value_type, const uint8_t *encoded, size_t len,
                           size_t k, size_t n, const float *x, float *y, int threads,
                           int warmup, int iters, double *median_s, double *min_s)
{
    if (iters < 1 || warmup < 0) return ORACLE_BAD_ARGUMENT;
    double *samples = (double *)malloc(sizeof(double) * (size_t)iters);
    if (!samples) return ORACLE_BAD_ARGUMENT;
    int status = ORACLE_OK;
    for (int i = 0; i < warmup + iters && status == ORACLE_OK; ++i) {
        const double start = now_seconds();
        status = threads == 1
                     ? oracle_quant_gemv(value_type, encoded, len, k, n, x, y, 1)
                     : oracle_quant_gemv_threads(value_type, encoded, len, k, n, x, y, threads);
        const double elapsed = now_seconds() - start;
        if (i >= warmup) samples[i - warmup] = elapsed;
    }
    if (status == ORACLE_OK) {
        qsort(samples, (size_t)iters, sizeof(double), compare_double);
        *median_s = (iters % 2) ? samples[iters / 2]
                                : 0.5 * (samples[iters / 2 - 1] + samples[iters / 2]);
        *min_s = samples[0];
    }
    free(samples);
    return status;
}

// k-quant kernels for gfx950 (CDNA4, wave64): bit-exact dequantisation, the
// exact-order per-row GEMV (the device twin of the host oracle) and the
// standalone RMSNorm. The bandwidth GEMV lives in gemv_wave.hip.
//
// Weight layout in HBM: the encoded GGML array-of-blocks exactly as uploaded.
// Row n of a [K, N] tensor is K/256 consecutive super-blocks
// (crates/nvidia/src/quantized.rs:136-142). Activations are f32 batch-major
// [members][K]; outputs f32 batch-major [members][N].
#include "kquant_device.hpp"
#include "kquant_launch.hpp"

namespace ribn_amd {

// ---------------------------------------------------------------------------
// Bit-exact dequantisation: one workgroup of 256 threads per super-block,
// one element per thread. Products are exact in f32, so the single rounding of
// the final subtraction reproduces lib.rs:596-661 bit for bit.
// ---------------------------------------------------------------------------
template <int T>
__device__ __forceinline__ float dequant_element(const uint8_t* blk, int e) {
#pragma clang fp contract(off)
    if constexpr (T == kQ4K || T == kQ5K) {
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
        const float dmin = half_bits_to_float(blk[2] | (blk[3] << 8));
        const int g = e >> 5, i = e & 31;
        uint32_t sc, mn;
        const uint32_t s0 = blk[4] | (blk[5] << 8) | (blk[6] << 16) | ((uint32_t)blk[7] << 24);
        const uint32_t s1 = blk[8] | (blk[9] << 8) | (blk[10] << 16) | ((uint32_t)blk[11] << 24);
        const uint32_t s2 = blk[12] | (blk[13] << 8) | (blk[14] << 16) | ((uint32_t)blk[15] << 24);
        q4k_scale_min(s0, s1, s2, g, sc, mn);
        uint32_t q;
        if constexpr (T == kQ4K) {
            q = (blk[16 + (g >> 1) * 32 + i] >> (4 * (g & 1))) & 15u;
        } else {
            const uint32_t low = (blk[48 + (g >> 1) * 32 + i] >> (4 * (g & 1))) & 15u;
            const uint32_t high = (blk[16 + i] >> g) & 1u;
            q = low | (high << 4);
        }
        const float group_scale = d * (float)sc;
        const float group_minimum = dmin * (float)mn;
        return group_scale * (float)q - group_minimum;
    } else {
        const float d = half_bits_to_float(blk[208] | (blk[209] << 8));
        const int g = e >> 5, pos = e & 31;
        const int chunk = g >> 2, variant = g & 3;
        const int low_offset = chunk * 64 + (variant & 1) * 32;
        const int low_shift = variant < 2 ? 0 : 4;
        const uint32_t low = (blk[low_offset + pos] >> low_shift) & 15u;
        const uint32_t high = (blk[128 + chunk * 32 + pos] >> (2 * variant)) & 3u;
        const int q = (int)(low | (high << 4)) - 32;
        const float group_scale = d * (float)(int8_t)blk[192 + (e >> 4)];
        return group_scale * (float)q;
    }
}

template <int T>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w, uint32_t wbytes,
                                                      float* __restrict__ out, uint32_t nblocks) {
    constexpr int BB = BlockTraits<T>::bytes;
    __shared__ uint8_t blk[256];
    const __amdgpu_buffer_rsrc_t r = make_rsrc(w, wbytes);
    for (uint32_t b = blockIdx.x; b < nblocks; b += gridDim.x) {
        if (threadIdx.x < BB) {
            blk[threadIdx.x] = (uint8_t)__builtin_amdgcn_raw_buffer_load_b8(
                r, (int)(b * BB + threadIdx.x), 0, 0);
        }
        __syncthreads();
        out[(size_t)b * 256 + threadIdx.x] = dequant_element<T>(blk, threadIdx.x);
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Exact-order GEMV: one thread per output row, elements in K order, each
// product and sum rounded separately (no contraction), accumulator starting
// at -0.0. This is the arithmetic of cuda_reference.rs:889-902 /
// qwen_reference.rs:31-40, so results equal the host oracle bit for bit. It
// is the device correctness oracle, not a fast path.
// ---------------------------------------------------------------------------
template <int T>
__global__ __launch_bounds__(256) void gemv_exact_kernel(const uint8_t* __restrict__ w, uint32_t wbytes,
                                                         const float* __restrict__ x, float* __restrict__ y,
                                                         int K, int N, int members) {
    // Separate roundings for every product and sum, as in the host reference:
    // no FMA contraction in this kernel.
#pragma clang fp contract(off)
    constexpr int BB = BlockTraits<T>::bytes;
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    const int m = blockIdx.y;
    if (row >= N || m >= members) return;
    const int nb = K >> 8;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(w, wbytes);
    const float* xm = x + (size_t)m * K;
    uint8_t blk[BB];
    float sum = -0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint32_t off = (uint32_t)(row * nb + b) * BB;
        for (int i = 0; i < BB; ++i) {
            blk[i] = (uint8_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)(off + i), 0, 0);
        }
        for (int e = 0; e < 256; ++e) {
            const float product = dequant_element<T>(blk, e) * xm[b * 256 + e];
            sum = sum + product;
        }
    }
    y[(size_t)m * N + row] = sum;
}

// ---------------------------------------------------------------------------
// Standalone RMSNorm over batch-major vectors (model_ops.rs:106-199 semantics):
// one workgroup per member vector.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                       float* __restrict__ y, int length, float eps) {
    __shared__ float partial[4];
    const float* xm = x + (size_t)blockIdx.x * length;
    float* ym = y + (size_t)blockIdx.x * length;
    float ssq = 0.f;
    for (int i = threadIdx.x; i < length; i += 256) ssq += xm[i] * xm[i];
    ssq = wave_sum(ssq);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ssq;
    __syncthreads();
    const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    const float inv = 1.0f / sqrtf(total / (float)length + eps);
    for (int i = threadIdx.x; i < length; i += 256) ym[i] = xm[i] * inv * w[i];
}

// ---------------------------------------------------------------------------
// Embedding gather (q4_k.cu:1-67 q4_k_embedding / _batch): row `token` of a
// [hidden, vocab] k-quant table, dequantised bit-exactly. One workgroup per
// (member, super-block); tokens come from a device array (batch) or a value.
// Batch ids outside the vocabulary leave their output row unwritten, as the
// reference kernel does (the single-token call validates on the host).
// ---------------------------------------------------------------------------
template <int T>
__global__ __launch_bounds__(256) void embedding_kernel(const uint8_t* __restrict__ w, uint32_t wbytes,
                                                        const uint32_t* __restrict__ tokens, uint32_t token,
                                                        float* __restrict__ out, uint32_t blocks_per_token,
                                                        uint32_t vocab) {
    constexpr int BB = BlockTraits<T>::bytes;
    __shared__ uint8_t blk[256];
    const uint32_t member = blockIdx.y;
    const uint32_t tok = tokens ? tokens[member] : token;
    if (tok >= vocab) return;  // uniform across the workgroup
    const uint32_t block = (uint32_t)tok * blocks_per_token + blockIdx.x;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(w, wbytes);
    if (threadIdx.x < BB) {
        blk[threadIdx.x] = (uint8_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)(block * BB + threadIdx.x), 0, 0);
    }
    __syncthreads();
    out[((size_t)member * blocks_per_token + blockIdx.x) * 256 + threadIdx.x] = dequant_element<T>(blk, threadIdx.x);
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
template <int T>
static hipError_t launch_dequant_t(const uint8_t* w, uint32_t wbytes, float* out, uint32_t nblocks,
                                   hipStream_t stream) {
    const uint32_t grid = nblocks < 65536u ? nblocks : 65536u;
    hipLaunchKernelGGL(dequant_kernel<T>, dim3(grid), dim3(256), 0, stream, w, wbytes, out, nblocks);
    return hipGetLastError();
}

hipError_t launch_dequant(int value_type, const uint8_t* w, uint32_t wbytes, float* out, uint32_t nblocks,
                          hipStream_t stream) {
    switch (value_type) {
    case kQ4K: return launch_dequant_t<kQ4K>(w, wbytes, out, nblocks, stream);
    case kQ5K: return launch_dequant_t<kQ5K>(w, wbytes, out, nblocks, stream);
    case kQ6K: return launch_dequant_t<kQ6K>(w, wbytes, out, nblocks, stream);
    default: return hipErrorInvalidValue;
    }
}

template <int T>
static hipError_t launch_exact_t(const uint8_t* w, uint32_t wbytes, const float* x, float* y, int K, int N,
                                 int members, hipStream_t stream) {
    hipLaunchKernelGGL(gemv_exact_kernel<T>, dim3((N + 255) / 256, members), dim3(256), 0, stream, w, wbytes,
                       x, y, K, N, members);
    return hipGetLastError();
}

hipError_t launch_gemv_exact(int value_type, const uint8_t* w, uint32_t wbytes, const float* x, float* y,
                             int K, int N, int members, hipStream_t stream) {
    switch (value_type) {
    case kQ4K: return launch_exact_t<kQ4K>(w, wbytes, x, y, K, N, members, stream);
    case kQ5K: return launch_exact_t<kQ5K>(w, wbytes, x, y, K, N, members, stream);
    case kQ6K: return launch_exact_t<kQ6K>(w, wbytes, x, y, K, N, members, stream);
    default: return hipErrorInvalidValue;
    }
}

template <int T>
static hipError_t launch_embedding_t(const uint8_t* w, uint32_t wbytes, const uint32_t* tokens, uint32_t token,
                                     float* out, uint32_t blocks_per_token, uint32_t vocab, uint32_t members,
                                     hipStream_t stream) {
    hipLaunchKernelGGL(embedding_kernel<T>, dim3(blocks_per_token, members), dim3(256), 0, stream, w, wbytes, tokens,
                       token, out, blocks_per_token, vocab);
    return hipGetLastError();
}

hipError_t launch_embedding(int value_type, const uint8_t* w, uint32_t wbytes, const uint32_t* tokens,
                            uint32_t token, float* out, uint32_t blocks_per_token, uint32_t vocab, uint32_t members,
                            hipStream_t stream) {
    switch (value_type) {
    case kQ4K: return launch_embedding_t<kQ4K>(w, wbytes, tokens, token, out, blocks_per_token, vocab, members, stream);
    case kQ5K: return launch_embedding_t<kQ5K>(w, wbytes, tokens, token, out, blocks_per_token, vocab, members, stream);
    case kQ6K: return launch_embedding_t<kQ6K>(w, wbytes, tokens, token, out, blocks_per_token, vocab, members, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_rms_norm(const float* x, const float* w, float* y, int length, int members, float eps,
                           hipStream_t stream) {
    hipLaunchKernelGGL(rms_norm_kernel, dim3(members), dim3(256), 0, stream, x, w, y, length, eps);
    return hipGetLastError();
}

}  // namespace ribn_amd

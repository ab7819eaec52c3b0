// k-quant kernels for gfx950 (CDNA4, wave64): bit-exact dequantisation, the
// exact-order per-row GEMV (the device twin of the host oracle), and the
// bandwidth-oriented wave GEMV with an optional fused RMSNorm prologue.
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
        const float group_scale = __fmul_rn(d, (float)sc);
        const float group_minimum = __fmul_rn(dmin, (float)mn);
        return __fsub_rn(__fmul_rn(group_scale, (float)q), group_minimum);
    } else {
        const float d = half_bits_to_float(blk[208] | (blk[209] << 8));
        const int g = e >> 5, pos = e & 31;
        const int chunk = g >> 2, variant = g & 3;
        const int low_offset = chunk * 64 + (variant & 1) * 32;
        const int low_shift = variant < 2 ? 0 : 4;
        const uint32_t low = (blk[low_offset + pos] >> low_shift) & 15u;
        const uint32_t high = (blk[128 + chunk * 32 + pos] >> (2 * variant)) & 3u;
        const int q = (int)(low | (high << 4)) - 32;
        const float group_scale = __fmul_rn(d, (float)(int8_t)blk[192 + (e >> 4)]);
        return __fmul_rn(group_scale, (float)q);
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
            sum = __fadd_rn(sum, __fmul_rn(dequant_element<T>(blk, e), xm[b * 256 + e]));
        }
    }
    y[(size_t)m * N + row] = sum;
}

// ---------------------------------------------------------------------------
// Wave GEMV.
//
// A wave covers 16 consecutive super-blocks of a row per "slice"; lane l owns
// block (l >> 2) of the slice and quarter p = (l & 3) of that block, i.e. 64
// of its 256 elements:
//   Q4_K / Q5_K: groups 2p and 2p+1 (qs bytes 32p..32p+31, low / high nibbles);
//   Q6_K:        groups 4c..4c+3 at positions 16s..16s+15 (c = p >> 1, s = p & 1).
// Per row the lane issues 128-bit buffer loads for its payload and the block
// header, sums q * x per scale group in f32, and applies the group's scale and
// minimum once: sum_g (d*sc_g) * sum(q*x) - (dmin*m_g) * sum(x). The lane's 64
// activations (normalised in the fused-RMSNorm variant) stay in registers
// across rows when a row is one slice (K <= 4096).
// ---------------------------------------------------------------------------
constexpr int kWaveRows = 2;  // rows per pass of a wave

template <int T, int MT>
struct LaneActivations {
    float v[MT][64];
    float gsum[MT][4];
};

__device__ __forceinline__ float4 ld_f4(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}

// Offset (within a block's 256 elements) of lane-local activation j.
template <int T>
__device__ __forceinline__ int lane_x_offset(int p, int j) {
    if constexpr (T == kQ6K) {
        const int c = p >> 1, s = p & 1;
        return 128 * c + 32 * (j >> 4) + 16 * s + (j & 15);
    } else {
        return 64 * p + j;
    }
}

template <int T, int MT, bool NORM>
__device__ __forceinline__ void load_lane_activations(LaneActivations<T, MT>& xa, const float* __restrict__ x,
                                                      int K, int members, int b, int p, bool valid,
                                                      const float* inv, const float* __restrict__ gamma) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const bool live = valid && m < members;
        const float* xm = x + (size_t)m * K + (size_t)b * 256;
#pragma unroll
        for (int j = 0; j < 64; j += 4) {
            const int o = lane_x_offset<T>(p, j);
            float4 v = live ? ld_f4(xm + o) : make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (NORM) {
                if (live) {
                    const float4 g = ld_f4(gamma + (size_t)b * 256 + o);
                    v.x = v.x * inv[m] * g.x;
                    v.y = v.y * inv[m] * g.y;
                    v.z = v.z * inv[m] * g.z;
                    v.w = v.w * inv[m] * g.w;
                }
            }
            xa.v[m][j] = v.x;
            xa.v[m][j + 1] = v.y;
            xa.v[m][j + 2] = v.z;
            xa.v[m][j + 3] = v.w;
        }
        constexpr int NG = (T == kQ6K) ? 4 : 2;
        constexpr int GS = 64 / NG;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < GS; ++j) s += xa.v[m][g * GS + j];
            xa.gsum[m][g] = s;
        }
    }
}

__device__ __forceinline__ float ubyte_f(uint32_t w, int t) {
    return (float)((w >> (8 * t)) & 0xffu);
}

// Adds this lane's share of one row's dot products (block at byte offset off).
template <int T, int MT>
__device__ __forceinline__ void lane_block_dot(__amdgpu_buffer_rsrc_t r, uint32_t off, int p,
                                               const LaneActivations<T, MT>& xa, float (&acc)[MT]) {
    if constexpr (T == kQ4K || T == kQ5K) {
        const uint4 h = load_b128(r, off);
        uint32_t qw[8];
        uint32_t hw[8];
        if constexpr (T == kQ4K) {
            const uint4 qa = load_b128(r, off + 16 + 32 * p);
            const uint4 qb = load_b128(r, off + 32 + 32 * p);
            qw[0] = qa.x; qw[1] = qa.y; qw[2] = qa.z; qw[3] = qa.w;
            qw[4] = qb.x; qw[5] = qb.y; qw[6] = qb.z; qw[7] = qb.w;
        } else {
            const uint4 ha = load_b128(r, off + 16);
            const uint4 hb = load_b128(r, off + 32);
            const uint4 qa = load_b128(r, off + 48 + 32 * p);
            const uint4 qb = load_b128(r, off + 64 + 32 * p);
            qw[0] = qa.x; qw[1] = qa.y; qw[2] = qa.z; qw[3] = qa.w;
            qw[4] = qb.x; qw[5] = qb.y; qw[6] = qb.z; qw[7] = qb.w;
            hw[0] = ha.x; hw[1] = ha.y; hw[2] = ha.z; hw[3] = ha.w;
            hw[4] = hb.x; hw[5] = hb.y; hw[6] = hb.z; hw[7] = hb.w;
        }
        const float d = half_bits_to_float(h.x & 0xffffu);
        const float dmin = half_bits_to_float(h.x >> 16);
        // six-bit scales/minima of all 8 groups, four per word (lib.rs:573-587)
        const uint32_t lo_sc = h.y & 0x3f3f3f3fu;
        const uint32_t lo_mn = h.z & 0x3f3f3f3fu;
        const uint32_t hi_sc = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
        const uint32_t hi_mn = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
        const uint32_t scw = (p < 2) ? lo_sc : hi_sc;
        const uint32_t mnw = (p < 2) ? lo_mn : hi_mn;
        const int sh = (p & 1) * 16;
        const float a0 = d * (float)((scw >> sh) & 0xffu);
        const float a1 = d * (float)((scw >> (sh + 8)) & 0xffu);
        const float b0 = dmin * (float)((mnw >> sh) & 0xffu);
        const float b1 = dmin * (float)((mnw >> (sh + 8)) & 0xffu);
        float q0[32], q1[32];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t lo = qw[j] & 0x0f0f0f0fu;
            uint32_t hi = (qw[j] >> 4) & 0x0f0f0f0fu;
            if constexpr (T == kQ5K) {
                lo |= ((hw[j] >> (2 * p)) & 0x01010101u) << 4;
                hi |= ((hw[j] >> (2 * p + 1)) & 0x01010101u) << 4;
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                q0[4 * j + t] = ubyte_f(lo, t);
                q1[4 * j + t] = ubyte_f(hi, t);
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float s0 = 0.f, s1 = 0.f;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                s0 = __builtin_fmaf(q0[i], xa.v[m][i], s0);
                s1 = __builtin_fmaf(q1[i], xa.v[m][32 + i], s1);
            }
            float a = acc[m];
            a = __builtin_fmaf(a0, s0, a);
            a = __builtin_fmaf(-b0, xa.gsum[m][0], a);
            a = __builtin_fmaf(a1, s1, a);
            a = __builtin_fmaf(-b1, xa.gsum[m][1], a);
            acc[m] = a;
        }
    } else {
        const int c = p >> 1, s = p & 1;
        const uint4 la = load_16_at_half_aligned(r, off + 64 * c + 16 * s);
        const uint4 lb = load_16_at_half_aligned(r, off + 64 * c + 32 + 16 * s);
        const uint4 qh = load_16_at_half_aligned(r, off + 128 + 32 * c + 16 * s);
        // scales 192..207 and d at 208..209 from five dword-aligned words
        const uint32_t hoff = off + 192;
        const uint32_t hbase = hoff & ~3u;
        const uint32_t hsh = (hoff & 3u) * 8u;
        const uint4 ha = load_b128(r, hbase);
        const uint32_t he = load_b32(r, hbase + 16);
        const uint32_t sc_lo = __builtin_amdgcn_alignbit(ha.y, ha.x, hsh);   // scales 0..3
        const uint32_t sc_1 = __builtin_amdgcn_alignbit(ha.z, ha.y, hsh);    // scales 4..7
        const uint32_t sc_2 = __builtin_amdgcn_alignbit(ha.w, ha.z, hsh);    // scales 8..11
        const uint32_t sc_3 = __builtin_amdgcn_alignbit(he, ha.w, hsh);      // scales 12..15
        const float d = half_bits_to_float((he >> hsh) & 0xffffu);
        // lane scales: sc[8c + 2v + s], v = 0..3
        const uint32_t w0 = c ? sc_2 : sc_lo;   // scales 8c+0..8c+3
        const uint32_t w1 = c ? sc_3 : sc_1;    // scales 8c+4..8c+7
        float a[4];
        a[0] = d * (float)(int8_t)((w0 >> (8 * s)) & 0xffu);
        a[1] = d * (float)(int8_t)((w0 >> (8 * (2 + s))) & 0xffu);
        a[2] = d * (float)(int8_t)((w1 >> (8 * s)) & 0xffu);
        a[3] = d * (float)(int8_t)((w1 >> (8 * (2 + s))) & 0xffu);
        const uint32_t law[4] = {la.x, la.y, la.z, la.w};
        const uint32_t lbw[4] = {lb.x, lb.y, lb.z, lb.w};
        const uint32_t qhw[4] = {qh.x, qh.y, qh.z, qh.w};
        float q[4][16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t v0 = (law[j] & 0x0f0f0f0fu) | ((qhw[j] << 4) & 0x30303030u);
            const uint32_t v1 = (lbw[j] & 0x0f0f0f0fu) | ((qhw[j] << 2) & 0x30303030u);
            const uint32_t v2 = ((law[j] >> 4) & 0x0f0f0f0fu) | (qhw[j] & 0x30303030u);
            const uint32_t v3 = ((lbw[j] >> 4) & 0x0f0f0f0fu) | ((qhw[j] >> 2) & 0x30303030u);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                q[0][4 * j + t] = ubyte_f(v0, t);
                q[1][4 * j + t] = ubyte_f(v1, t);
                q[2][4 * j + t] = ubyte_f(v2, t);
                q[3][4 * j + t] = ubyte_f(v3, t);
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float accm = acc[m];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                float sv = 0.f;
#pragma unroll
                for (int i = 0; i < 16; ++i) sv = __builtin_fmaf(q[v][i], xa.v[m][16 * v + i], sv);
                // (q - 32) * x summed: sum(q*x) - 32 * sum(x)
                accm = __builtin_fmaf(a[v], sv, accm);
                accm = __builtin_fmaf(-32.f * a[v], xa.gsum[m][v], accm);
            }
            acc[m] = accm;
        }
    }
}

template <int T, int MT, bool NORM, bool ONE_SLICE>
__global__ __launch_bounds__(256) void gemv_wave_kernel(const uint8_t* __restrict__ w, uint32_t wbytes,
                                                        const float* __restrict__ x, float* __restrict__ y,
                                                        int K, int N, int members,
                                                        const float* __restrict__ gamma, float eps) {
    constexpr int BB = BlockTraits<T>::bytes;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nb = K >> 8;
    const int slices = (nb + 15) >> 4;
    const uint32_t row_bytes = (uint32_t)nb * BB;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(w, wbytes);

    float inv[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) inv[m] = 1.f;
    if constexpr (NORM) {
        // Fused RMSNorm prologue: inverse RMS of each member vector,
        // 1 / sqrt(sum(x^2) / K + eps) (qwen_reference.rs:550-556).
        __shared__ float partial[MT][4];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float ssq = 0.f;
            if (m < members) {
                const float* xm = x + (size_t)m * K;
                for (int k = threadIdx.x * 4; k < K; k += 1024) {
                    const float4 v = ld_f4(xm + k);
                    ssq += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                }
            }
            ssq = wave_sum(ssq);
            if (lane == 0) partial[m][wave] = ssq;
        }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float total = (partial[m][0] + partial[m][1]) + (partial[m][2] + partial[m][3]);
            inv[m] = 1.0f / sqrtf(total / (float)K + eps);
        }
    }

    const int p = lane & 3;
    const int bs = lane >> 2;
    const int total_waves = gridDim.x * 4;
    const int wave_global = blockIdx.x * 4 + wave;

    LaneActivations<T, MT> xa;
    if constexpr (ONE_SLICE) {
        load_lane_activations<T, MT, NORM>(xa, x, K, members, bs, p, bs < nb, inv, gamma);
    }
    for (int row0 = wave_global * kWaveRows; row0 < N; row0 += total_waves * kWaveRows) {
        float acc[kWaveRows][MT];
#pragma unroll
        for (int rr = 0; rr < kWaveRows; ++rr)
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[rr][m] = 0.f;
        for (int s = 0; s < slices; ++s) {
            const int b = s * 16 + bs;
            const bool valid = b < nb;
            if constexpr (!ONE_SLICE) {
                load_lane_activations<T, MT, NORM>(xa, x, K, members, b, p, valid, inv, gamma);
            }
            if (valid) {
#pragma unroll
                for (int rr = 0; rr < kWaveRows; ++rr) {
                    const int row = row0 + rr;
                    if (row < N) {
                        lane_block_dot<T, MT>(r, (uint32_t)row * row_bytes + (uint32_t)b * BB, p, xa, acc[rr]);
                    }
                }
            }
        }
#pragma unroll
        for (int rr = 0; rr < kWaveRows; ++rr) {
            const int row = row0 + rr;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float total = wave_sum(acc[rr][m]);
                if (lane == 0 && row < N && m < members) y[(size_t)m * N + row] = total;
            }
        }
    }
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

template <int T, int MT, bool NORM>
static hipError_t launch_wave_tm(const uint8_t* w, uint32_t wbytes, const float* x, float* y, int K, int N,
                                 int members, const float* gamma, float eps, int cu_count, hipStream_t stream) {
    const int pairs = (N + kWaveRows - 1) / kWaveRows;
    const int max_waves = cu_count * 16;
    const int waves = pairs < max_waves ? pairs : max_waves;
    const int grid = (waves + 3) / 4;
    if ((K >> 8) <= 16) {
        hipLaunchKernelGGL((gemv_wave_kernel<T, MT, NORM, true>), dim3(grid), dim3(256), 0, stream, w, wbytes, x,
                           y, K, N, members, gamma, eps);
    } else {
        hipLaunchKernelGGL((gemv_wave_kernel<T, MT, NORM, false>), dim3(grid), dim3(256), 0, stream, w, wbytes,
                           x, y, K, N, members, gamma, eps);
    }
    return hipGetLastError();
}

template <int T, bool NORM>
static hipError_t launch_wave_t(const uint8_t* w, uint32_t wbytes, const float* x, float* y, int K, int N,
                                int members, const float* gamma, float eps, int cu_count, hipStream_t stream) {
    // members <= kWaveMaxMembers per launch (the host splits larger batches)
    if (members <= 1) return launch_wave_tm<T, 1, NORM>(w, wbytes, x, y, K, N, members, gamma, eps, cu_count, stream);
    if (members <= 2) return launch_wave_tm<T, 2, NORM>(w, wbytes, x, y, K, N, members, gamma, eps, cu_count, stream);
    return launch_wave_tm<T, 4, NORM>(w, wbytes, x, y, K, N, members, gamma, eps, cu_count, stream);
}

hipError_t launch_gemv_wave(int value_type, const uint8_t* w, uint32_t wbytes, const float* x, float* y, int K,
                            int N, int members, const float* gamma, float eps, int cu_count,
                            hipStream_t stream) {
    const bool norm = gamma != nullptr;
    switch (value_type) {
    case kQ4K:
        return norm ? launch_wave_t<kQ4K, true>(w, wbytes, x, y, K, N, members, gamma, eps, cu_count, stream)
                    : launch_wave_t<kQ4K, false>(w, wbytes, x, y, K, N, members, gamma, eps, cu_count, stream);
    case kQ5K:
        return norm ? launch_wave_t<kQ5K, true>(w, wbytes, x, y, K, N, members, gamma, eps, cu_count, stream)
                    : launch_wave_t<kQ5K, false>(w, wbytes, x, y, K, N, members, gamma, eps, cu_count, stream);
    case kQ6K:
        return norm ? launch_wave_t<kQ6K, true>(w, wbytes, x, y, K, N, members, gamma, eps, cu_count, stream)
                    : launch_wave_t<kQ6K, false>(w, wbytes, x, y, K, N, members, gamma, eps, cu_count, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_rms_norm(const float* x, const float* w, float* y, int length, int members, float eps,
                           hipStream_t stream) {
    hipLaunchKernelGGL(rms_norm_kernel, dim3(members), dim3(256), 0, stream, x, w, y, length, eps);
    return hipGetLastError();
}

}  // namespace ribn_amd

// Prefill / large-batch matmul for Q4_K / Q5_K / Q6_K on gfx950: y[M][N] =
// x[M][K] . W^T with the weights dequantised in registers straight into MFMA
// operand layout and multiplied on the matrix cores (v_mfma_f32_32x32x16_f16),
// accumulating in f32.
//
// Two kernels:
//  - act_f16_kernel: one workgroup per token. Optional RMSNorm
//    (x * 1/sqrt(sum(x^2)/K + eps) * gamma, qwen_reference.rs:550-556), then
//    conversion to f16 after a power-of-two scale that maps the token's
//    largest |x| just below 2^15. bf16 inputs convert exactly (8-bit into
//    11-bit significands) down to 2^-24 of the token maximum; f32 inputs round
//    once (RNE, 2^-11 relative). The per-token unscale goes to a side array.
//  - qgemm_kernel: a workgroup of WAVES waves owns 32*WAVES weight rows and
//    32*CB tokens; wave w owns rows [32w, 32w+32) of the tile. K advances in
//    half super-blocks (128 elements): the x tile [32*CB][128] f16 is staged
//    in LDS (padded rows, double-buffered; a step's tile is loaded into
//    registers two steps ahead and written to LDS one step ahead), weights are
//    loaded per lane straight from HBM (three steps ahead) and dequantised in
//    f32, (d*sc)*q - dmin*m, then rounded once to f16 (RNE) in the A-operand
//    layout. Each A fragment feeds CB MFMAs.
//
// MFMA 32x32x16 operand layout (measured on gfx950): lane l holds
// A[l%32][8*(l/32)+j], B[8*(l/32)+j][l%32] (j = 0..7) and
// C[8*(i/4)+4*(l/32)+(i%4)][l%32] (i = 0..15). Here A = W rows, B = x^T, so
// C[n][m]. A dot product does not depend on the order of its k terms, so
// each 16-wide MFMA k-chunk is a set of 16 block elements chosen to make the
// lane's 8 elements come from 8 consecutive payload bytes; the B fragment
// reads the same 8 activations, consecutive in k.
#include "kquant_device.hpp"
#include "kquant_launch.hpp"

#include <algorithm>
#include <type_traits>

namespace ribn_amd {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_v __attribute__((ext_vector_type(2)));
typedef float float2_v __attribute__((ext_vector_type(2)));
typedef float float16_v __attribute__((ext_vector_type(16)));

constexpr int kActThreads = 256;
constexpr int kStepK = 128;                                // K per pipeline step (half a super-block)
constexpr int kXRow = kStepK + 8;                          // padded LDS row (halfs): 272 B, bank-conflict free
constexpr uint32_t kGemmOutOfRange = 0xffffff00u;

// ------------------------------------------------------------ activations

__device__ __forceinline__ float block_sum_256(float v, float* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float t = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return t;
}

__device__ __forceinline__ float block_max_256(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float t = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return t;
}

template <bool BF16_IN, bool NORM>
__global__ __launch_bounds__(kActThreads) void act_f16_kernel(const void* __restrict__ xin,
                                                               const float* __restrict__ gamma, float eps, int K,
                                                               _Float16* __restrict__ xh, float* __restrict__ unscale) {
    // Thread t owns chunks of 8 consecutive elements, 8*(t + 256c): one
    // 16-byte load (bf16) or two (f32) in, one 16-byte f16 store out.
    constexpr int kChunks = kGemmMaxK / 8 / kActThreads;  // 8
    __shared__ float red[4];
    const int m = blockIdx.x;
    float v[kChunks][8];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const int e = 8 * ((int)threadIdx.x + kActThreads * c);
        if (e < K) {
            if constexpr (BF16_IN) {
                const uint4 raw = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(xin) + (size_t)m * K + e);
                const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    v[c][2 * j] = __builtin_bit_cast(float, wv[j] << 16);
                    v[c][2 * j + 1] = __builtin_bit_cast(float, wv[j] & 0xffff0000u);
                }
            } else {
                const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(xin) + (size_t)m * K + e);
                const float4 a = src[0], b = src[1];
                v[c][0] = a.x; v[c][1] = a.y; v[c][2] = a.z; v[c][3] = a.w;
                v[c][4] = b.x; v[c][5] = b.y; v[c][6] = b.z; v[c][7] = b.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[c][j] = 0.f;
        }
    }
    if constexpr (NORM) {
        float ssq = 0.f;
#pragma unroll
        for (int c = 0; c < kChunks; ++c)
#pragma unroll
            for (int j = 0; j < 8; ++j) ssq += v[c][j] * v[c][j];
        const float inv = 1.0f / sqrtf(block_sum_256(ssq, red) / (float)K + eps);
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
            const int e = 8 * ((int)threadIdx.x + kActThreads * c);
            if (e < K) {
                const float4 g0 = *reinterpret_cast<const float4*>(gamma + e);
                const float4 g1 = *reinterpret_cast<const float4*>(gamma + e + 4);
                const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
                for (int j = 0; j < 8; ++j) v[c][j] = v[c][j] * inv * g[j];
            }
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[c][j]));
    amax = block_max_256(amax, red);
    int ex = amax > 0.f ? __builtin_amdgcn_frexp_expf(amax) : 0;  // amax < 2^ex
    ex = ex < -100 ? -100 : ex;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const int e = 8 * ((int)threadIdx.x + kActThreads * c);
        if (e < K) {
            half8_t h;
#pragma unroll
            for (int j = 0; j < 8; j += 2) {
                const float2_v f = {__builtin_amdgcn_ldexpf(v[c][j], 15 - ex),
                                    __builtin_amdgcn_ldexpf(v[c][j + 1], 15 - ex)};
                const half2_v p = __builtin_convertvector(f, half2_v);
                h[j] = p[0];
                h[j + 1] = p[1];
            }
            *reinterpret_cast<half8_t*>(xh + (size_t)m * K + e) = h;
        }
    }
    if (threadIdx.x == 0) unscale[m] = __builtin_amdgcn_ldexpf(1.0f, ex - 15);
}

// ------------------------------------------------------------ weight fragments

// Per-lane weight bytes for one pipeline step (half super-block `half`).
template <int T> struct StepW;
template <> struct StepW<kQ4K> { uint4 h, q0, q1; };        // header; qs bytes 32t+16hl.. for t = 2*half, 2*half+1
template <> struct StepW<kQ5K> { uint4 h, qh, q0, q1; };    // + qh bytes 16hl..16hl+15
template <> struct StepW<kQ6K> {
    uint4 l0, l1, qh, sc;             // dword-aligned-down windows of ql (two), qh, scales
    uint32_t l0t, l1t, qht, sct;      // the dword after each window
    uint32_t d16, shift;
};

template <int T>
__device__ __forceinline__ void load_step(StepW<T>& s, __amdgpu_buffer_rsrc_t r, uint32_t blk, int half, int hl) {
    if constexpr (T == kQ4K) {
        s.h = load_b128(r, blk);
        s.q0 = load_b128(r, blk + 16 + 32 * (2 * half) + 16 * hl);
        s.q1 = load_b128(r, blk + 16 + 32 * (2 * half + 1) + 16 * hl);
    } else if constexpr (T == kQ5K) {
        s.h = load_b128(r, blk);
        s.qh = load_b128(r, blk + 16 + 16 * hl);
        s.q0 = load_b128(r, blk + 48 + 32 * (2 * half) + 16 * hl);
        s.q1 = load_b128(r, blk + 48 + 32 * (2 * half + 1) + 16 * hl);
    } else {
        const uint32_t base = blk & ~3u;
        s.shift = (blk & 3u) * 8u;
        const uint32_t l0 = base + 64 * half + 16 * hl;
        const uint32_t l1 = l0 + 32;
        const uint32_t qh = base + 128 + 32 * half + 16 * hl;
        s.l0 = load_b128(r, l0);
        s.l0t = load_b32(r, l0 + 16);
        s.l1 = load_b128(r, l1);
        s.l1t = load_b32(r, l1 + 16);
        s.qh = load_b128(r, qh);
        s.qht = load_b32(r, qh + 16);
        s.sc = load_b128(r, base + 192);
        s.sct = load_b32(r, base + 208);
        s.d16 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)(blk + 208), 0, kStreamPolicy);
    }
}

__device__ __forceinline__ uint4 funnel4(uint4 a, uint32_t t, uint32_t sh) {
    uint4 o;
    o.x = __builtin_amdgcn_alignbit(a.y, a.x, sh);
    o.y = __builtin_amdgcn_alignbit(a.z, a.y, sh);
    o.z = __builtin_amdgcn_alignbit(a.w, a.z, sh);
    o.w = __builtin_amdgcn_alignbit(t, a.w, sh);
    return o;
}

// Eight f16 weights (a*q_j - b), q_j = byte j of (lo, hi) after masking
// (byte-to-float converts are single v_cvt_f32_ubyteN instructions).
__device__ __forceinline__ half8_t dequant8(uint32_t lo, uint32_t hi, float a, float b) {
    // Opaque to the optimiser, so each byte converts with one v_cvt_f32_ubyteN
    // instead of a bit-field extract plus a convert.
    asm volatile("" : "+v"(lo), "+v"(hi));
    float w[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        w[j] = __builtin_fmaf(a, (float)((lo >> (8 * j)) & 0xffu), -b);
        w[4 + j] = __builtin_fmaf(a, (float)((hi >> (8 * j)) & 0xffu), -b);
    }
    half8_t h;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        const float2_v f = {w[j], w[j + 1]};
        const half2_v p = __builtin_convertvector(f, half2_v);
        h[j] = p[0];
        h[j + 1] = p[1];
    }
    return h;
}

// A step's weights decoded once: scale and offset of each scale group the
// lane touches, and (Q6_K) the payload windows realigned.
template <int T> struct StepDec;
template <> struct StepDec<kQ4K> { float a[4], b[4]; };
template <> struct StepDec<kQ5K> { float a[4], b[4]; };
template <> struct StepDec<kQ6K> { float a[4]; uint4 l0, l1, qh; };

template <int T, int HALF>
__device__ __forceinline__ void decode_step(const StepW<T>& s, int hl, StepDec<T>& o) {
    if constexpr (T == kQ4K || T == kQ5K) {
        // groups 4*HALF + i, i = 2t' + p; six-bit scales/minima (lib.rs:573-587)
        const float d = half_bits_to_float(s.h.x & 0xffffu);
        const float dmin = half_bits_to_float(s.h.x >> 16);
        const uint32_t scw = HALF ? ((s.h.w & 0x0f0f0f0fu) | ((s.h.y >> 2) & 0x30303030u)) : (s.h.y & 0x3f3f3f3fu);
        const uint32_t mnw = HALF ? (((s.h.w >> 4) & 0x0f0f0f0fu) | ((s.h.z >> 2) & 0x30303030u))
                                  : (s.h.z & 0x3f3f3f3fu);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o.a[i] = d * (float)((scw >> (8 * i)) & 0xffu);
            o.b[i] = dmin * (float)((mnw >> (8 * i)) & 0xffu);
        }
    } else {
        o.l0 = funnel4(s.l0, s.l0t, s.shift);
        o.l1 = funnel4(s.l1, s.l1t, s.shift);
        o.qh = funnel4(s.qh, s.qht, s.shift);
        const uint4 scw = funnel4(s.sc, s.sct, s.shift);
        const float d = half_bits_to_float(s.d16);
        // scale 8*HALF + 2v + hl: bytes hl and hl+2 of dwords 2*HALF (v = 0, 1) and 2*HALF+1 (v = 2, 3)
        const uint32_t w0 = (HALF ? scw.z : scw.x) >> (8 * hl);
        const uint32_t w1 = (HALF ? scw.w : scw.y) >> (8 * hl);
        o.a[0] = d * (float)(int8_t)(w0 & 0xffu);
        o.a[1] = d * (float)(int8_t)((w0 >> 16) & 0xffu);
        o.a[2] = d * (float)(int8_t)(w1 & 0xffu);
        o.a[3] = d * (float)(int8_t)((w1 >> 16) & 0xffu);
    }
}

// Chunk C (0..7) of a step: the lane's 8 f16 weights and the k offset
// (within the 128-element step) of the 8 activations they multiply.
//   Q4_K/Q5_K: C = (t', p, s): payload bytes 32t+16hl+8s+j, nibble p, group 2t+p;
//              element 64t' + 32p + 16hl + 8s + j of the step (t = 2*HALF + t').
//   Q6_K:      C = (v, s): element 32v + 16hl + 8s + j of the step, scale 8*HALF + 2v + hl.
template <int T, int HALF, int C>
__device__ __forceinline__ half8_t chunk_weights(const StepW<T>& s, const StepDec<T>& dec, int hl, int& koff) {
    if constexpr (T == kQ4K || T == kQ5K) {
        constexpr int tp = C >> 2, p = (C >> 1) & 1, ss = C & 1;
        constexpr int g = 4 * HALF + 2 * tp + p;
        koff = 64 * tp + 32 * p + 16 * hl + 8 * ss;
        const uint4 q = tp ? s.q1 : s.q0;
        uint32_t lo = ((ss ? q.z : q.x) >> (4 * p)) & 0x0f0f0f0fu;
        uint32_t hi = ((ss ? q.w : q.y) >> (4 * p)) & 0x0f0f0f0fu;
        if constexpr (T == kQ5K) {
            lo |= (((ss ? s.qh.z : s.qh.x) >> g) & 0x01010101u) << 4;
            hi |= (((ss ? s.qh.w : s.qh.y) >> g) & 0x01010101u) << 4;
        }
        return dequant8(lo, hi, dec.a[2 * tp + p], dec.b[2 * tp + p]);
    } else {
        constexpr int v = C >> 1, ss = C & 1;
        koff = 32 * v + 16 * hl + 8 * ss;
        const uint4 lw = (v & 1) ? dec.l1 : dec.l0;
        uint32_t lo = ss ? lw.z : lw.x;
        uint32_t hi = ss ? lw.w : lw.y;
        const uint32_t hlo = ss ? dec.qh.z : dec.qh.x;
        const uint32_t hhi = ss ? dec.qh.w : dec.qh.y;
        lo = ((lo >> (4 * (v >> 1))) & 0x0f0f0f0fu) | (((hlo >> (2 * v)) & 0x03030303u) << 4);
        hi = ((hi >> (4 * (v >> 1))) & 0x0f0f0f0fu) | (((hhi >> (2 * v)) & 0x03030303u) << 4);
        return dequant8(lo, hi, dec.a[v], 32.f * dec.a[v]);
    }
}

// ------------------------------------------------------------------- GEMM

constexpr int kRing = 4;  // weight steps in flight per lane (the current one + three ahead)

// Split K: workgroup z covers steps [z*split_steps, (z+1)*split_steps) (a
// multiple of the four-step unroll); with partial != null it writes its raw
// tile to partial[z][M][N] and qgemm_reduce_kernel adds the splits in order.
template <int T, int CB, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void qgemm_kernel(const uint8_t* __restrict__ w, uint32_t wbytes,
                                                           const _Float16* __restrict__ xh,
                                                           const float* __restrict__ unscale, float* __restrict__ y,
                                                           float* __restrict__ partial, int M, int N, int K,
                                                           int split_steps) {
    constexpr int BB = BlockTraits<T>::bytes;
    constexpr int TOK = 32 * CB;                      // tokens per workgroup
    constexpr int THREADS = WAVES * 64;
    constexpr int XCH = TOK * (kStepK / 8) / THREADS;  // 16-byte x chunks per thread per step
    static_assert(XCH * THREADS == TOK * kStepK / 8, "x tile must split evenly");
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][TOK * kXRow];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int hl = lane >> 5;
    const int n0 = blockIdx.x * 32 * WAVES + 32 * wave;
    const int m0 = blockIdx.y * TOK;
    const int nb = K >> 8;
    const int s_begin = blockIdx.z * split_steps;
    const int steps = min(2 * nb, s_begin + split_steps);  // end of this workgroup's steps
    const int row = n0 + (lane & 31);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w, wbytes);
    const uint32_t row_off = row < N ? (uint32_t)row * (uint32_t)(nb * BB) : kGemmOutOfRange;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(xh, (uint32_t)M * (uint32_t)K * 2u);

    // x tile chunk i of a step: token i / 16, 16-byte piece i % 16.
    auto load_x = [&](uint4 (&buf)[XCH], int step) {
#pragma unroll
        for (int j = 0; j < XCH; ++j) {
            const int i = threadIdx.x + THREADS * j;
            const int tok = m0 + (i >> 4);
            const uint32_t off = (tok < M && step < steps)
                                     ? ((uint32_t)tok * (uint32_t)K + (uint32_t)step * kStepK + (i & 15) * 8) * 2u
                                     : kGemmOutOfRange;
            buf[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0));
        }
    };
    auto store_x = [&](const uint4 (&buf)[XCH], int slot) {
#pragma unroll
        for (int j = 0; j < XCH; ++j) {
            const int i = threadIdx.x + THREADS * j;
            *reinterpret_cast<uint4*>(&xs[slot][(i >> 4) * kXRow + (i & 15) * 8]) = buf[j];
        }
    };
    auto w_off = [&](int step) {
        return (row_off == kGemmOutOfRange || step >= steps) ? kGemmOutOfRange
                                                              : row_off + (uint32_t)(step >> 1) * BB;
    };

    float16_v acc[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c) acc[c] = float16_v{};

    // Prologue: x for step 0 first (waited for below), then the weights of
    // steps 0..2 (a four-slot ring, three steps ahead).
    uint4 xbuf[XCH];
    load_x(xbuf, s_begin);
    asm volatile("" ::: "memory");
    StepW<T> wring[kRing];
#pragma unroll
    for (int r = 0; r < kRing - 1; ++r) load_step<T>(wring[r], wr, w_off(s_begin + r), r & 1, hl);
    store_x(xbuf, 0);
    load_x(xbuf, s_begin + 1);
    __syncthreads();

    // Steps run in fours so each one's ring slot and block half are static;
    // padding steps past K load out of range (zeros) and skip the MFMAs.
    auto run_step = [&](auto r_const, int s0) {
        constexpr int r = decltype(r_const)::value;
        constexpr int HALF = r & 1;
        const int step = s0 + r;
        // x of step+1 (loaded a step ago) into the other LDS slot, which every
        // wave finished reading before the last barrier; then x two steps ahead.
        store_x(xbuf, (r + 1) & 1);
        load_x(xbuf, step + 2);
        load_step<T>(wring[(r + kRing - 1) % kRing], wr, w_off(step + kRing - 1), (r + kRing - 1) & 1, hl);
        if (step < steps) {
            StepDec<T> dec;
            decode_step<T, HALF>(wring[r], hl, dec);
            const _Float16* xt = &xs[r & 1][(lane & 31) * kXRow];
            auto chunk = [&](auto c_const) {
                constexpr int C = decltype(c_const)::value;
                int koff;
                const half8_t a = chunk_weights<T, HALF, C>(wring[r], dec, hl, koff);
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    const half8_t b = *reinterpret_cast<const half8_t*>(xt + cb * 32 * kXRow + koff);
                    acc[cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[cb], 0, 0, 0);
                }
            };
            chunk(std::integral_constant<int, 0>{});
            chunk(std::integral_constant<int, 1>{});
            chunk(std::integral_constant<int, 2>{});
            chunk(std::integral_constant<int, 3>{});
            chunk(std::integral_constant<int, 4>{});
            chunk(std::integral_constant<int, 5>{});
            chunk(std::integral_constant<int, 6>{});
            chunk(std::integral_constant<int, 7>{});
        }
        __syncthreads();
    };
    const int padded = s_begin + (steps - s_begin + kRing - 1) / kRing * kRing;
    for (int s0 = s_begin; s0 < padded; s0 += kRing) {
        run_step(std::integral_constant<int, 0>{}, s0);
        run_step(std::integral_constant<int, 1>{}, s0);
        run_step(std::integral_constant<int, 2>{}, s0);
        run_step(std::integral_constant<int, 3>{}, s0);
    }

    // epilogue: C[n][m] -> y[m][n] * unscale[m], or the raw split tile
    float* out = partial ? partial + (size_t)blockIdx.z * M * N : y;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        const int m = m0 + 32 * cb + (lane & 31);
        if (m >= M) continue;
        const float us = partial ? 1.0f : unscale[m];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + 8 * j + 4 * hl;
            float4 o;
            o.x = acc[cb][4 * j + 0] * us;
            o.y = acc[cb][4 * j + 1] * us;
            o.z = acc[cb][4 * j + 2] * us;
            o.w = acc[cb][4 * j + 3] * us;
            float* dst = out + (size_t)m * N + n;
            if (n + 3 < N) {
                *reinterpret_cast<float4*>(dst) = o;
            } else {
                if (n < N) dst[0] = o.x;
                if (n + 1 < N) dst[1] = o.y;
                if (n + 2 < N) dst[2] = o.z;
            }
        }
    }
}

// y[m][n] = unscale[m] * sum over splits z (in order) of partial[z][m][n]
__global__ __launch_bounds__(256) void qgemm_reduce_kernel(const float* __restrict__ partial,
                                                           const float* __restrict__ unscale, float* __restrict__ y,
                                                           int M, int N, int splits) {
    const size_t total = (size_t)M * N;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        float acc = partial[i];
        for (int z = 1; z < splits; ++z) acc += partial[(size_t)z * total + i];
        y[i] = acc * unscale[i / N];
    }
}

// ---------------------------------------------------------------- launchers

constexpr int kMaxSplits = 8;

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t gemm_workspace_bytes(size_t tokens, size_t K, size_t N) {
    // f16 activations, one f32 unscale per token, and room for kMaxSplits
    // partial [tokens][N] tiles (split K)
    return align256(tokens * K * 2) + align256(tokens * 4) + align256((size_t)kMaxSplits * tokens * N * 4);
}

hipError_t launch_act_f16(bool bf16_in, const void* x, const float* gamma, float eps, int M, int K, void* workspace,
                          hipStream_t stream) {
    _Float16* xh = static_cast<_Float16*>(workspace);
    float* us = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + align256((size_t)M * K * 2));
    if (bf16_in) {
        if (gamma) hipLaunchKernelGGL((act_f16_kernel<true, true>), dim3(M), dim3(kActThreads), 0, stream, x, gamma, eps, K, xh, us);
        else hipLaunchKernelGGL((act_f16_kernel<true, false>), dim3(M), dim3(kActThreads), 0, stream, x, gamma, eps, K, xh, us);
    } else {
        if (gamma) hipLaunchKernelGGL((act_f16_kernel<false, true>), dim3(M), dim3(kActThreads), 0, stream, x, gamma, eps, K, xh, us);
        else hipLaunchKernelGGL((act_f16_kernel<false, false>), dim3(M), dim3(kActThreads), 0, stream, x, gamma, eps, K, xh, us);
    }
    return hipGetLastError();
}

template <int T, int CB, int WAVES>
static hipError_t launch_qgemm_t(const uint8_t* w, uint32_t wbytes, void* workspace, size_t workspace_bytes,
                                 float* y, int M, int N, int K, int cu_count, hipStream_t stream) {
    uint8_t* base = static_cast<uint8_t*>(workspace);
    const _Float16* xh = reinterpret_cast<const _Float16*>(base);
    const size_t us_off = align256((size_t)M * K * 2);
    const float* us = reinterpret_cast<const float*>(base + us_off);
    const size_t part_off = us_off + align256((size_t)M * 4);
    float* part = reinterpret_cast<float*>(base + part_off);
    const int gx = (N + 32 * WAVES - 1) / (32 * WAVES), gy = (M + 32 * CB - 1) / (32 * CB);
    // A grid with fewer waves than SIMDs splits K toward two waves per SIMD
    // (whole four-step rounds, as far as the reserved partial space allows);
    // fuller grids do not, since the partial tiles then cost more traffic
    // than they save.
    const int steps = 2 * (K >> 8);
    const int rounds = (steps + kRing - 1) / kRing;
    const long long waves = (long long)gx * gy * WAVES;
    int splits = 1;
    if (waves < 4LL * cu_count) splits = (int)((8LL * cu_count + waves - 1) / waves);
    splits = std::min({splits, kMaxSplits, rounds});
    const size_t tile_bytes = (size_t)M * N * 4;
    const size_t room = workspace_bytes > part_off ? workspace_bytes - part_off : 0;
    if ((size_t)splits * tile_bytes > room) splits = (int)std::max<size_t>(1, room / tile_bytes);
    if (splits < 1) splits = 1;
    const int split_steps = (rounds + splits - 1) / splits * kRing;
    splits = (steps + split_steps - 1) / split_steps;
    const dim3 grid(gx, gy, splits);
    hipLaunchKernelGGL((qgemm_kernel<T, CB, WAVES>), grid, dim3(WAVES * 64), 0, stream, w, wbytes, xh, us, y,
                       splits > 1 ? part : nullptr, M, N, K, split_steps);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    const size_t total = (size_t)M * N;
    const int rgrid = (int)std::min<size_t>((total + 255) / 256, (size_t)cu_count * 8);
    hipLaunchKernelGGL(qgemm_reduce_kernel, dim3(rgrid), dim3(256), 0, stream, part, us, y, M, N, splits);
    return hipGetLastError();
}

// Tile by token count: few tokens take small tiles (more workgroups for the
// weight stream); many tokens take 256-row x 128-token tiles (each
// dequantised weight fragment feeds four MFMAs, 8 waves share each activation
// tile)
// (a sweep over 1-8 token blocks x 2-8 waves at M = 512: 4 x 8 was fastest,
// 4% ahead of 4 x 4 on Q4_K 4096->12288 and level on Q6_K 12288->4096).
template <int T>
static hipError_t launch_qgemm_m(const uint8_t* w, uint32_t wbytes, void* workspace, size_t workspace_bytes, float* y,
                                 int M, int N, int K, int cu_count, hipStream_t stream) {
    if (M <= 32) return launch_qgemm_t<T, 1, 1>(w, wbytes, workspace, workspace_bytes, y, M, N, K, cu_count, stream);
    if (M <= 64) return launch_qgemm_t<T, 2, 2>(w, wbytes, workspace, workspace_bytes, y, M, N, K, cu_count, stream);
    return launch_qgemm_t<T, 4, 8>(w, wbytes, workspace, workspace_bytes, y, M, N, K, cu_count, stream);
}

hipError_t launch_qgemm(int value_type, const uint8_t* w, uint32_t wbytes, void* workspace, size_t workspace_bytes,
                        float* y, int M, int N, int K, int cu_count, hipStream_t stream) {
    switch (value_type) {
    case kQ4K: return launch_qgemm_m<kQ4K>(w, wbytes, workspace, workspace_bytes, y, M, N, K, cu_count, stream);
    case kQ5K: return launch_qgemm_m<kQ5K>(w, wbytes, workspace, workspace_bytes, y, M, N, K, cu_count, stream);
    case kQ6K: return launch_qgemm_m<kQ6K>(w, wbytes, workspace, workspace_bytes, y, M, N, K, cu_count, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace ribn_amd

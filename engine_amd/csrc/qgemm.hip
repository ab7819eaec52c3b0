// Prefill / large-batch matmul for Q4_K / Q5_K / Q6_K on gfx950: y[M][N] =
// x[M][K] . W^T with the weights dequantised in registers straight into MFMA
// operand layout and multiplied on the matrix cores, accumulating in f32.
//
// Kernels:
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
//    packed f16 (below) in the A-operand layout. Each A fragment feeds CB
//    MFMAs (v_mfma_f32_32x32x16_f16).
//  - qgemm_tile_kernel: 192-row x 128-token workgroups of four waves on
//    v_mfma_f32_16x16x32_f16 with packed-f16 dequantisation, for grids that
//    fill the CUs (described where it is defined); 256-row tiles with split K
//    for Q5_K / Q6_K shapes whose 192-row grid does not fill them.
//  - qgemm_reduce_kernel: adds the K splits' partial tiles in split order.
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
constexpr int kActPlain = 0;   // activation prologues of act_f16_kernel
constexpr int kActAdd = 1;
constexpr int kActSwiglu = 2;
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

// PRO selects a prologue on f32 inputs (the decoder's prompt prefill):
// kActAdd adds r into x first and stores the sum back to x (the residual
// stream), kActSwiglu stages silu(x) * r (model_ops.rs:316-328).
template <bool BF16_IN, bool NORM, int PRO = kActPlain>
__global__ __launch_bounds__(kActThreads) void act_f16_kernel(const void* __restrict__ xin,
                                                               const float* __restrict__ gamma, float eps, int K,
                                                               _Float16* __restrict__ xh, float* __restrict__ unscale,
                                                               const float* __restrict__ r = nullptr) {
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
                if constexpr (PRO != kActPlain) {
                    const float4* rs = reinterpret_cast<const float4*>(r + (size_t)m * K + e);
                    const float4 ra = rs[0], rb = rs[1];
                    const float rv[8] = {ra.x, ra.y, ra.z, ra.w, rb.x, rb.y, rb.z, rb.w};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        if constexpr (PRO == kActAdd) {
                            v[c][j] = v[c][j] + rv[j];
                        } else {
                            v[c][j] = (v[c][j] / (1.0f + expf(-v[c][j]))) * rv[j];
                        }
                    }
                    if constexpr (PRO == kActAdd) {
                        float4* out = reinterpret_cast<float4*>(const_cast<float*>(static_cast<const float*>(xin)) +
                                                                (size_t)m * K + e);
                        out[0] = make_float4(v[c][0], v[c][1], v[c][2], v[c][3]);
                        out[1] = make_float4(v[c][4], v[c][5], v[c][6], v[c][7]);
                    }
                }
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

// Weights are dequantised in packed f16 (two per instruction, no conversion
// instructions): a quant byte q becomes the f16 1024 + q (bits 0x6400 | q,
// or 1024 + 16q for a high nibble left in place), and
//   Q4_K/Q5_K: qs = fma(1024 + q, sc, -1024 sc) = q*sc exactly (every value
//              involved is an f16 integer, q*sc <= 1953), then
//              w = fma(qs, d, -f16(dmin*m)): one rounding of d*sc*q - dmin*m
//              besides that of the minimum term;
//   Q6_K:      qm = (1024 + q) - 1056 = q - 32 exactly, then
//              w = fma(qm, a_hi, qm * a_lo) with a = d*sc split into two f16
//              parts: one rounding of a*(q - 32).
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ __forceinline__ uint32_t as_u(half2_t v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ half2_t splat_h2(float v) {
    const _Float16 h = (_Float16)v;
    return half2_t{h, h};
}
// bytes (b0, b1, b2, b3) -> (b0, b2, b1, b3): the halves of x & 0x00ff00ff
// are then elements (0, 1) and those of (x >> 8) elements (2, 3)
__device__ __forceinline__ uint32_t pair_order(uint32_t x) { return __builtin_amdgcn_perm(x, x, 0x03010200u); }

// 0x64006400 in a vector register, so (x & mask) | it is one v_and_or_b32
// (a three-operand instruction takes no literal and reads at most one scalar
// register on gfx9: the mask goes in the scalar register)
__device__ __forceinline__ uint32_t f16_magic() {
    uint32_t k;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(k));
    return k;
}

template <int T>
__device__ __forceinline__ void tile_word(uint32_t x, uint32_t mask, uint32_t extra_a, uint32_t extra_b, half2_t s,
                                          half2_t c, half2_t d, half2_t nb, uint32_t& oa, uint32_t& ob) {
    const uint32_t xp = pair_order(x);
    const uint32_t k = f16_magic();
    const half2_t pa = as_h2((xp & mask) | (extra_a | k));
    const half2_t pb = as_h2(((xp >> 8) & mask) | (extra_b | k));
    oa = as_u(__builtin_elementwise_fma(__builtin_elementwise_fma(pa, s, c), d, nb));
    ob = as_u(__builtin_elementwise_fma(__builtin_elementwise_fma(pb, s, c), d, nb));
}

__device__ __forceinline__ void tile_word6(uint32_t x, half2_t ahi, half2_t alo, uint32_t& oa, uint32_t& ob) {
    const uint32_t xp = pair_order(x);
    const uint32_t k = f16_magic();
    const half2_t off = half2_t{(_Float16)-1056.0f, (_Float16)-1056.0f};
    const half2_t qa = as_h2((xp & 0x003f003fu) | k) + off;
    const half2_t qb = as_h2(((xp >> 8) & 0x003f003fu) | k) + off;
    oa = as_u(__builtin_elementwise_fma(qa, ahi, qa * alo));
    ob = as_u(__builtin_elementwise_fma(qb, ahi, qb * alo));
}

// Eight f16 weights from byte quants q_j (byte j of lo, then of hi):
// Q4_K/Q5_K w = f16(d*sc*q - f16(dmin*m)), Q6_K w = f16(a*(q - 32)), as above.
__device__ __forceinline__ half8_t dequant8_qs(uint32_t lo, uint32_t hi, half2_t s, half2_t c, half2_t d,
                                               half2_t nb) {
    uint32_t o[4];
    tile_word<kQ4K>(lo, 0x00ff00ffu, 0, 0, s, c, d, nb, o[0], o[1]);
    tile_word<kQ4K>(hi, 0x00ff00ffu, 0, 0, s, c, d, nb, o[2], o[3]);
    return __builtin_bit_cast(half8_t, uint4{o[0], o[1], o[2], o[3]});
}

__device__ __forceinline__ half8_t dequant8_q6(uint32_t lo, uint32_t hi, half2_t ahi, half2_t alo) {
    uint32_t o[4];
    tile_word6(lo, ahi, alo, o[0], o[1]);
    tile_word6(hi, ahi, alo, o[2], o[3]);
    return __builtin_bit_cast(half8_t, uint4{o[0], o[1], o[2], o[3]});
}

// A step's weights decoded once: scale and offset of each scale group the
// lane touches, and (Q6_K) the payload windows realigned.
template <int T> struct StepDec;
template <> struct StepDec<kQ4K> { half2_t s[4], c[4], nb[4], d; };
template <> struct StepDec<kQ5K> { half2_t s[4], c[4], nb[4], d; };
template <> struct StepDec<kQ6K> { half2_t ahi[4], alo[4]; uint4 l0, l1, qh; };

template <int T, int HALF>
__device__ __forceinline__ void decode_step(const StepW<T>& s, int hl, StepDec<T>& o) {
    if constexpr (T == kQ4K || T == kQ5K) {
        // groups 4*HALF + i, i = 2t' + p; six-bit scales/minima (lib.rs:573-587)
        const float dmin = half_bits_to_float(s.h.x >> 16);
        o.d = as_h2((s.h.x & 0xffffu) * 0x10001u);
        const uint32_t scw = HALF ? ((s.h.w & 0x0f0f0f0fu) | ((s.h.y >> 2) & 0x30303030u)) : (s.h.y & 0x3f3f3f3fu);
        const uint32_t mnw = HALF ? (((s.h.w >> 4) & 0x0f0f0f0fu) | ((s.h.z >> 2) & 0x30303030u))
                                  : (s.h.z & 0x3f3f3f3fu);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float scf = (float)((scw >> (8 * i)) & 0xffu);
            o.s[i] = splat_h2(scf);
            o.c[i] = splat_h2(-1024.0f * scf);
            o.nb[i] = splat_h2(-(dmin * (float)((mnw >> (8 * i)) & 0xffu)));
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
        const float a[4] = {d * (float)(int8_t)(w0 & 0xffu), d * (float)(int8_t)((w0 >> 16) & 0xffu),
                            d * (float)(int8_t)(w1 & 0xffu), d * (float)(int8_t)((w1 >> 16) & 0xffu)};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const _Float16 h = (_Float16)a[v];
            o.ahi[v] = half2_t{h, h};
            o.alo[v] = splat_h2(a[v] - (float)h);
        }
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
        return dequant8_qs(lo, hi, dec.s[2 * tp + p], dec.c[2 * tp + p], dec.d, dec.nb[2 * tp + p]);
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
        return dequant8_q6(lo, hi, dec.ahi[v], dec.alo[v]);
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

// y[m][n] = unscale[m] * sum over splits z (in order) of partial[z][m][n].
// V = 4: four outputs per thread (16-byte loads and stores; N a multiple of
// 4 and y 16-byte aligned), V = 1 otherwise. Every split's load is issued
// before the first add; each element sees the same operations in the same
// order in either form, so the results are identical.
constexpr int kMaxReduceSplits = 16;

template <int V>
__global__ __launch_bounds__(256) void qgemm_reduce_kernel(const float* __restrict__ partial,
                                                           const float* __restrict__ unscale, float* __restrict__ y,
                                                           int M, int N, int splits) {
    typedef float vec_t __attribute__((ext_vector_type(V)));
    const size_t total = (size_t)M * N;
    const size_t units = total / V;
    const size_t per_row = (size_t)N / V;
    const vec_t* __restrict__ pv = reinterpret_cast<const vec_t*>(partial);
    vec_t* __restrict__ yv = reinterpret_cast<vec_t*>(y);
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < units; i += (size_t)gridDim.x * 256) {
        vec_t v[kMaxReduceSplits];
#pragma unroll
        for (int z = 0; z < kMaxReduceSplits; ++z)
            if (z < splits) v[z] = pv[(size_t)z * units + i];
        vec_t acc = v[0];
#pragma unroll
        for (int z = 1; z < kMaxReduceSplits; ++z)
            if (z < splits) acc += v[z];
        yv[i] = acc * unscale[i / per_row];
    }
}

static hipError_t launch_reduce(const float* part, const float* us, float* y, int M, int N, int splits, int cu_count,
                                hipStream_t stream) {
    if (splits < 2 || splits > kMaxReduceSplits) return hipErrorInvalidValue;
    const bool wide = N % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0;
    const size_t units = (size_t)M * N / (wide ? 4 : 1);
    const int rgrid = (int)std::min<size_t>((units + 255) / 256, (size_t)std::max(1, cu_count) * 8);
    if (wide)
        hipLaunchKernelGGL(qgemm_reduce_kernel<4>, dim3(rgrid), dim3(256), 0, stream, part, us, y, M, N, splits);
    else
        hipLaunchKernelGGL(qgemm_reduce_kernel<1>, dim3(rgrid), dim3(256), 0, stream, part, us, y, M, N, splits);
    return hipGetLastError();
}

// ------------------------------------------------------------- wide tiles
//
// qgemm_tile_kernel<T, RB> (M > 64): four waves, one per SIMD, one workgroup
// per CU. The workgroup owns 64*RB weight rows and 128 tokens; wave w owns
// rows [16*RB*w, 16*RB*(w+1)) as RB blocks of 16 and all 8 token blocks, so
// each dequantised A fragment feeds 8 MFMAs and each B fragment read from LDS
// feeds RB. v_mfma_f32_16x16x32_f16: lane l holds A[l%16][8(l/16)+j],
// B[8(l/16)+j][l%16] and C[4(l/16)+i][l%16]. K advances a super-block (256
// elements, 8 chunks of 32) per step; the x tile [128][256] f16 is staged in
// LDS (padded rows, double-buffered, loaded into registers a step ahead), and
// each lane loads its weight bytes a step ahead.
//
// Chunk c of a super-block and k-piece q = l/16 select 8 consecutive k:
//   Q4_K/Q5_K: c = 4L + 2h + p -> k0 = 128L + 64(q>>1) + 32h + 16(q&1) + 8p,
//              payload bytes 16q + 8p.. of qs half L (64 B), nibble h, scale
//              group 4L + 2(q>>1) + h;
//   Q6_K:      c = 2Q + p -> k0 = 128(q>>1) + 32Q + 16(q&1) + 8p, ql window
//              (Q & 1), nibble Q >> 1, qh bits 2Q, scale 8(q>>1) + 2Q + (q&1).
// (lib.rs:596-661 element order.) Each 16-byte weight load serves 4 chunks.

constexpr int kTileTokMax = 128;                   // most tokens per workgroup (8 blocks of 16)
constexpr int kTileThreads = 256;

typedef float float4_v __attribute__((ext_vector_type(4)));

template <int T> struct SbW;
template <> struct SbW<kQ4K> { uint4 h, p0, p1; };
template <> struct SbW<kQ5K> { uint4 h, qh, p0, p1; };
template <> struct SbW<kQ6K> {
    uint4 a, b, qh, sc;                // dword-aligned-down windows: ql (two), qh, scales
    uint32_t at, bt, qht, sct;         // the dword after each window
    uint32_t d16, shift;
};

template <int T>
__device__ __forceinline__ void load_sb(SbW<T>& s, __amdgpu_buffer_rsrc_t r, uint32_t blk, int q) {
    if constexpr (T == kQ4K) {
        s.h = load_b128(r, blk);
        s.p0 = load_b128(r, blk + 16 + 16 * q);
        s.p1 = load_b128(r, blk + 80 + 16 * q);
    } else if constexpr (T == kQ5K) {
        s.h = load_b128(r, blk);
        s.qh = load_b128(r, blk + 16 + 16 * (q & 1));
        s.p0 = load_b128(r, blk + 48 + 16 * q);
        s.p1 = load_b128(r, blk + 112 + 16 * q);
    } else {
        const uint32_t base = blk & ~3u;
        s.shift = (blk & 3u) * 8u;
        const uint32_t oa = base + 16 * q + 32 * (q >> 1);
        const uint32_t oh = base + 128 + 16 * q;
        s.a = load_b128(r, oa);
        s.at = load_b32(r, oa + 16);
        s.b = load_b128(r, oa + 32);
        s.bt = load_b32(r, oa + 48);
        s.qh = load_b128(r, oh);
        s.qht = load_b32(r, oh + 16);
        s.sc = load_b128(r, base + 192);
        s.sct = load_b32(r, base + 208);
        s.d16 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)(blk + 208), 0, kStreamPolicy);
    }
}

// A super-block's per-lane constants: Q4_K/Q5_K for groups 4L + 2(q>>1) + h
// (s, c as above, d, and -f16(dmin*m)); Q6_K a_hi, a_lo per quarter Q (and the
// realigned windows).
template <int T> struct SbDec;
template <> struct SbDec<kQ4K> { half2_t s[2][2], c[2][2], nb[2][2], d; };
template <> struct SbDec<kQ5K> { half2_t s[2][2], c[2][2], nb[2][2], d; };
template <> struct SbDec<kQ6K> { half2_t ahi[4], alo[4]; uint4 la, lb, qh; };

template <int T>
__device__ __forceinline__ void decode_sb(const SbW<T>& s, int q, SbDec<T>& o) {
    if constexpr (T == kQ4K || T == kQ5K) {
        const float dmin = half_bits_to_float(s.h.x >> 16);
        o.d = as_h2((s.h.x & 0xffffu) * 0x10001u);
        const int sh = 16 * (q >> 1);
        const uint32_t sc[2] = {(s.h.y & 0x3f3f3f3fu) >> sh,
                                ((s.h.w & 0x0f0f0f0fu) | ((s.h.y >> 2) & 0x30303030u)) >> sh};
        const uint32_t mn[2] = {(s.h.z & 0x3f3f3f3fu) >> sh,
                                (((s.h.w >> 4) & 0x0f0f0f0fu) | ((s.h.z >> 2) & 0x30303030u)) >> sh};
#pragma unroll
        for (int L = 0; L < 2; ++L) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float scf = (float)((sc[L] >> (8 * h)) & 0xffu);
                o.s[L][h] = splat_h2(h ? scf * 0.0625f : scf);
                o.c[L][h] = splat_h2(h ? -64.0f * scf : -1024.0f * scf);
                o.nb[L][h] = splat_h2(-(dmin * (float)((mn[L] >> (8 * h)) & 0xffu)));
            }
        }
    } else {
        o.la = funnel4(s.a, s.at, s.shift);
        o.lb = funnel4(s.b, s.bt, s.shift);
        o.qh = funnel4(s.qh, s.qht, s.shift);
        const uint4 scw = funnel4(s.sc, s.sct, s.shift);
        const float d = half_bits_to_float(s.d16);
        // scale 8n + 2Q + (q&1), n = q>>1: byte 2(Q&1) + (q&1) of dword 2n + (Q>>1)
        const uint32_t w0 = ((q >> 1) ? scw.z : scw.x) >> (8 * (q & 1));
        const uint32_t w1 = ((q >> 1) ? scw.w : scw.y) >> (8 * (q & 1));
        const float a[4] = {d * (float)(int8_t)(w0 & 0xffu), d * (float)(int8_t)((w0 >> 16) & 0xffu),
                            d * (float)(int8_t)(w1 & 0xffu), d * (float)(int8_t)((w1 >> 16) & 0xffu)};
#pragma unroll
        for (int Q = 0; Q < 4; ++Q) {
            const _Float16 hi = (_Float16)a[Q];
            o.ahi[Q] = half2_t{hi, hi};
            o.alo[Q] = splat_h2(a[Q] - (float)hi);
        }
    }
}

// Four packed f16 weights from one word of quant bytes (elements j..j+3)
// whose values, after `mask`, sit in the low bits of each byte (plus `extra`
// bits already placed: the Q5_K high bit).
// Chunk C's A fragment (8 f16 weights of the lane's row).
template <int T, int C>
__device__ __forceinline__ half8_t tile_chunk(const SbW<T>& s, const SbDec<T>& dec, int q) {
    uint32_t o[4];
    if constexpr (T == kQ4K || T == kQ5K) {
        constexpr int L = C >> 2, h = (C >> 1) & 1, p = C & 1;
        const uint4 P = L ? s.p1 : s.p0;
        const uint32_t mask = h ? 0x00f000f0u : 0x000f000fu;
        uint32_t ea0 = 0, eb0 = 0, ea1 = 0, eb1 = 0;
        if constexpr (T == kQ5K) {
            // bit g of each qh byte -> bit 4 (low nibble) or 8 (high nibble, 16x) of its f16 half
            const int g = 4 * L + 2 * (q >> 1) + h;
            const uint32_t hm = h ? 0x01000100u : 0x00100010u;
            const int ra = (g + (h ? 24 : 28)) & 31, rb = (g + (h ? 0 : 4)) & 31;
            const uint32_t q0 = pair_order(p ? s.qh.z : s.qh.x), q1 = pair_order(p ? s.qh.w : s.qh.y);
            ea0 = __builtin_amdgcn_alignbit(q0, q0, ra) & hm;
            eb0 = __builtin_amdgcn_alignbit(q0, q0, rb) & hm;
            ea1 = __builtin_amdgcn_alignbit(q1, q1, ra) & hm;
            eb1 = __builtin_amdgcn_alignbit(q1, q1, rb) & hm;
        }
        tile_word<T>(p ? P.z : P.x, mask, ea0, eb0, dec.s[L][h], dec.c[L][h], dec.d, dec.nb[L][h], o[0], o[1]);
        tile_word<T>(p ? P.w : P.y, mask, ea1, eb1, dec.s[L][h], dec.c[L][h], dec.d, dec.nb[L][h], o[2], o[3]);
    } else {
        constexpr int Q = C >> 1, p = C & 1;
        const uint4 W = (Q & 1) ? dec.lb : dec.la;
        // 6-bit bytes: low nibble | (2 high bits << 4); the high bits sit at
        // bits 2Q of each qh byte and move to bits 4-5 in one shift
        auto up = [](uint32_t v) { return Q < 2 ? v << (4 - 2 * Q) : v >> (2 * Q - 4); };
        const uint32_t lo = (((p ? W.z : W.x) >> (4 * (Q >> 1))) & 0x0f0f0f0fu) |
                            (up(p ? dec.qh.z : dec.qh.x) & 0x30303030u);
        const uint32_t hi = (((p ? W.w : W.y) >> (4 * (Q >> 1))) & 0x0f0f0f0fu) |
                            (up(p ? dec.qh.w : dec.qh.y) & 0x30303030u);
        tile_word6(lo, dec.ahi[Q], dec.alo[Q], o[0], o[1]);
        tile_word6(hi, dec.ahi[Q], dec.alo[Q], o[2], o[3]);
    }
    return __builtin_bit_cast(half8_t, uint4{o[0], o[1], o[2], o[3]});
}

template <int T, int C>
__device__ __forceinline__ int tile_k0(int q) {
    if constexpr (T == kQ4K || T == kQ5K) {
        constexpr int L = C >> 2, h = (C >> 1) & 1, p = C & 1;
        return 128 * L + 64 * (q >> 1) + 32 * h + 16 * (q & 1) + 8 * p;
    } else {
        constexpr int Q = C >> 1, p = C & 1;
        return 128 * (q >> 1) + 32 * Q + 16 * (q & 1) + 8 * p;
    }
}

// RB row blocks of 16 per wave, TB token blocks of 16 per workgroup. Split
// K: workgroup z covers super-blocks [z*split_sb, (z+1)*split_sb); with
// partial != null it writes its raw tile to partial[z][M][N] and
// qgemm_reduce_kernel adds the splits in order.
template <int T, int RB, int TB>
__global__ __launch_bounds__(kTileThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void qgemm_tile_kernel(
    const uint8_t* __restrict__ w, uint32_t wbytes, const _Float16* __restrict__ xh, const float* __restrict__ unscale,
    float* __restrict__ y, float* __restrict__ partial, int M, int N, int K, int split_sb) {
    constexpr int kTok = 16 * TB;                        // tokens per workgroup
    constexpr int kWaveTok = kTok / (kTileThreads / 64);  // x tile tokens each wave loads
    constexpr int kLoads = kWaveTok / 2;                  // its 1 KB loads per super-block
    constexpr int BB = BlockTraits<T>::bytes;
    // two x slots as separate objects: the compiler can then tell that the
    // reads of one slot do not alias the loads into the other in flight
    __shared__ __attribute__((aligned(16))) _Float16 xs0[kTok * 256];
    __shared__ __attribute__((aligned(16))) _Float16 xs1[kTok * 256];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int q = lane >> 4;
    const int r16 = lane & 15;
    const int n0 = blockIdx.x * 64 * RB + 16 * RB * wave;
    const int m0 = blockIdx.y * kTok;
    const int nb = K >> 8;
    const int sb_begin = blockIdx.z * split_sb;
    const int sb_end = min(nb, sb_begin + split_sb);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w, wbytes);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(xh, (uint32_t)M * (uint32_t)K * 2u);
    uint32_t row_off[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int row = min(n0 + 16 * rb + r16, N - 1);  // rows past N repeat the last (not stored)
        row_off[rb] = (uint32_t)row * (uint32_t)(nb * BB);
    }

    // x tile of a super-block, loaded straight into LDS (1 KB per wave load,
    // 16 bytes per lane): load i of wave w fills tokens t = 32w + 2i, +1
    // (lanes 0-31 and 32-63), 512 bytes each. LDS slot u of token t holds the
    // 16-byte piece u ^ (t & 15), so the B reads of 16 tokens at one piece
    // fall in distinct banks (measured conflict-free on gfx950). A lane's
    // offset for load i (token and swizzled piece) is fixed; the super-block
    // goes in the uniform offset. Tokens past M read past the activations
    // (zeros) through the lane offset alone.
    uint32_t xoff[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int t = kWaveTok * wave + 2 * i + (lane >> 5);
        xoff[i] = ((uint32_t)(m0 + t) * (uint32_t)K + (uint32_t)((lane & 31) ^ (t & 15)) * 8u) * 2u;
    }
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    // loads [part*kLoads/4, (part+1)*kLoads/4) of the tile
    auto load_x = [&](_Float16* xs, int sb, auto part_const) {
        constexpr int part = decltype(part_const)::value;
#pragma unroll
        for (int i = part * kLoads / 4; i < (part + 1) * kLoads / 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (__attribute__((address_space(3))) void*)&xs[(kWaveTok * wave_u + 2 * i) * 256], 16, (int)xoff[i],
                sb * 512, 0, 0);
        // the tile is written behind the compiler's back: LDS reads must not
        // be folded or moved across this point
        asm volatile("" ::: "memory");
    };
    auto load_w = [&](SbW<T> (&ring)[RB], int sb) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) load_sb<T>(ring[rb], wr, row_off[rb] + (uint32_t)sb * BB, q);
    };

    float4_v acc[RB][TB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) acc[rb][tb] = float4_v{};

    // Prologue: x and weights of the first super-block.
    SbW<T> wring[2][RB];
    load_x(xs0, sb_begin, std::integral_constant<int, 0>{});
    load_x(xs0, sb_begin, std::integral_constant<int, 1>{});
    load_x(xs0, sb_begin, std::integral_constant<int, 2>{});
    load_x(xs0, sb_begin, std::integral_constant<int, 3>{});
    load_w(wring[0], sb_begin);
    __syncthreads();

    // One super-block; slot r (static) holds its x tile and weights.
    // PREFETCH: x of sb+1 into the other LDS slot (every wave finished
    // reading it before the last barrier; a quarter in each of the first four
    // chunks) and the weights of sb+1 (a row block in each of the first RB
    // chunks), most of a step ahead of their use (the barrier below waits
    // for the x tile). The loads are unconditional within the loop, so the
    // compiler's wait counts stay exact; a prefetch of sb+1 = sb_end <= nb
    // reads in-bounds data that is not used (or zeros past the tensors).
    auto step = [&](auto r_const, auto prefetch_const, int sb) {
        constexpr int r = decltype(r_const)::value;
        _Float16* const xcur = r ? xs1 : xs0;
        _Float16* const xnext = r ? xs0 : xs1;
        constexpr bool kNext = decltype(prefetch_const)::value;
        __builtin_amdgcn_sched_barrier(0);
        {
            const SbW<T>(&wcur)[RB] = wring[r];
            SbDec<T> dec[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) decode_sb<T>(wcur[rb], q, dec[rb]);
            const _Float16* xt0 = &xcur[r16 * 256];
            // Software pipeline over the 8 chunks: while chunk C's 8*RB MFMAs
            // run, chunk C+1's A fragments are dequantised (a few VALU
            // instructions after each MFMA, which its 16 cycles hide) and its
            // 8 B fragments are read from LDS (one per token block, a whole
            // chunk ahead of use).
            // token 16tb + r16, piece k0/8: LDS slot (k0/8) ^ r16
            auto bsrc = [&](int k0) { return xt0 + 8 * ((k0 >> 3) ^ r16); };
            half8_t acur[RB], anext[RB], bcur[TB], bnext[TB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) acur[rb] = tile_chunk<T, 0>(wcur[rb], dec[rb], q);
#pragma unroll
            for (int tb = 0; tb < TB; ++tb)
                bcur[tb] = *reinterpret_cast<const half8_t*>(bsrc(tile_k0<T, 0>(q)) + tb * 16 * 256);
            constexpr int kValu = T == kQ5K ? 4 : 3;  // dequant instructions per MFMA
            auto chunk = [&](auto c_const) {
                constexpr int C = decltype(c_const)::value;
                // the next step's loads, spread over the first chunks so the
                // wave never queues them all at once
                if constexpr (kNext && C < 4) load_x(xnext, sb + 1, c_const);
                if constexpr (kNext && C < RB)
                    load_sb<T>(wring[r ^ 1][C], wr, row_off[C] + (uint32_t)(sb + 1) * BB, q);
                if constexpr (C < 7) {
                    const _Float16* nsrc = bsrc(tile_k0<T, C + 1>(q));
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb)
                        bnext[tb] = *reinterpret_cast<const half8_t*>(nsrc + tb * 16 * 256);
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) anext[rb] = tile_chunk<T, C + 1>(wcur[rb], dec[rb], q);
                }
#pragma unroll
                for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
                        acc[rb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(acur[rb], bcur[tb], acc[rb][tb], 0, 0, 0);
                // issue order: each MFMA followed by a share of the next
                // chunk's dequantisation, one B read per token block
#pragma unroll
                for (int tb = 0; tb < TB; ++tb) {
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, kValu, 0);
                    }
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (C < 7) {
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) acur[rb] = anext[rb];
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb) bcur[tb] = bnext[tb];
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
    // pairs of steps, then an odd last one (no conditional work inside a step)
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using Yes = std::true_type;
    int sb = sb_begin;
    for (; sb + 1 < sb_end; sb += 2) {
        step(I0{}, Yes{}, sb);
        step(I1{}, Yes{}, sb + 1);
    }
    if (sb < sb_end) step(I0{}, std::false_type{}, sb);

    // epilogue: C[n][m] -> y[m][n] * unscale[m], or the raw split tile
    float* out = partial ? partial + (size_t)blockIdx.z * M * N : y;
    const bool vec = (N & 3) == 0;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
        const int m = m0 + 16 * tb + r16;
        if (m >= M) continue;
        const float us = partial ? 1.0f : unscale[m];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int n = n0 + 16 * rb + 4 * q;
            const float4_v o = acc[rb][tb] * us;
            float* dst = out + (size_t)m * N + n;
            if (vec && n + 3 < N) {
                *reinterpret_cast<float4_v*>(dst) = o;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (n + i < N) dst[i] = o[i];
            }
        }
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

hipError_t launch_act_f16_residual(float* x, const float* r, const float* gamma, float eps, int M, int K,
                                   void* workspace, hipStream_t stream) {
    if (M < 1 || K < 8 || K > kGemmMaxK || K % 8 != 0 || r == nullptr || gamma == nullptr) return hipErrorInvalidValue;
    _Float16* xh = static_cast<_Float16*>(workspace);
    float* us = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + align256((size_t)M * K * 2));
    hipLaunchKernelGGL((act_f16_kernel<false, true, kActAdd>), dim3(M), dim3(kActThreads), 0, stream, x, gamma, eps,
                       K, xh, us, r);
    return hipGetLastError();
}

hipError_t launch_act_f16_swiglu(const float* gate, const float* up, int M, int K, void* workspace,
                                 hipStream_t stream) {
    if (M < 1 || K < 8 || K > kGemmMaxK || K % 8 != 0 || up == nullptr) return hipErrorInvalidValue;
    _Float16* xh = static_cast<_Float16*>(workspace);
    float* us = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + align256((size_t)M * K * 2));
    hipLaunchKernelGGL((act_f16_kernel<false, false, kActSwiglu>), dim3(M), dim3(kActThreads), 0, stream, gate,
                       nullptr, 0.f, K, xh, us, up);
    return hipGetLastError();
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
    return launch_reduce(part, us, y, M, N, splits, cu_count, stream);
}

// Wide tiles. M > 128 runs 192-row x 128-token workgroups when their grid
// fills at least 70% of its last round of CUs (e.g. Q4_K 4096 -> 12288 at
// M = 512: 64 x 4 = 256 workgroups; at M = 768, 384 of 512: 127.6 against
// 164.6 us on qgemm_kernel). Each wave's 48 rows keep its
// B reads (the whole x tile per wave) within the LDS bandwidth (about 90
// B/clk per CU measured); 32-row waves over 128 tokens are LDS-bound.
// 32 < M <= 128 picks (rows per wave, tokens per workgroup, K split) among
// the grids that fill 90-100% of one round, by an estimate fitted to
// measured calls: about 3 us per super-block step plus 0.05 us per MFMA
// tile block, plus the split's partial tiles (written, read, reduced).
// Q5_K and Q6_K shapes with M > 128 that the 192-row grid does not fill take
// 256-row tiles with split K in one round at least 60% full (wide256_splits);
// other M > 128 shapes take 192-row tiles with split K in one round at least
// 60% full (wide_tile_splits); the rest keep qgemm_kernel.
constexpr int kTileRb = 3;
constexpr int kTileTb = 8;

// The wide-tile grid of RB row blocks per wave fills at least `tenths`
// tenths of its last round of CUs.
static bool use_tile(int M, int N, int cu_count, int rb = kTileRb, int tenths = 7) {
    const long long wgs = (long long)((N + 64 * rb - 1) / (64 * rb)) * ((M + 16 * kTileTb - 1) / (16 * kTileTb));
    const long long cus = std::max(1, cu_count);
    const long long rounds = (wgs + cus - 1) / cus;
    return wgs * 10 >= rounds * cus * tenths;
}

// From this many tokens, 256-row tiles (RB = 4) take every type whose grid
// fills its last round 90%: each B fragment read from LDS then feeds four
// MFMAs instead of three. Measured at M = 2047: Q4_K 4096 -> 12288 244 us
// against 262 (192-row tiles), 4096 -> 4096 87 against 100 (32x32 kernel);
// at M = 1024 (4096 -> 12288, last round half full) 159 against 140.
constexpr int kTileWideM = 1024;

struct TileChoice {
    int rb = 0, tb = 0, splits = 0;  // rb == 0: none fits
};

static TileChoice choose_tile_small(int M, int N, int K, size_t room_bytes, int cu_count) {
    TileChoice best;
    const long long cus = std::max(1, cu_count);
    const int nb = K >> 8;
    const size_t tile_bytes = (size_t)M * N * 4;
    const int room_splits = (int)std::min<size_t>(16, tile_bytes ? room_bytes / tile_bytes : 0);
    double best_t = 1e30;
    const int shapes[3][2] = {{3, 8}, {3, 4}, {2, 4}};
    for (const auto& sh : shapes) {
        const int rb = sh[0], tb = sh[1];
        if (tb == 8 && M <= 64) continue;  // a mostly empty token tile
        const long long tn = (N + 64 * rb - 1) / (64 * rb), tm = (M + 16 * tb - 1) / (16 * tb);
        for (int s = 1; s <= 16 && s <= nb; ++s) {
            if (s > 1 && s > room_splits) break;
            const int split_sb = (nb + s - 1) / s;
            const int splits = (nb + split_sb - 1) / split_sb;
            const long long wgs = tn * tm * splits;
            if (wgs > cus || wgs * 10 < cus * 9) continue;
            double t = split_sb * (3.0 + 0.05 * rb * tb);
            if (splits > 1) t += 1.0 + (double)(2 * splits + 1) * (double)tile_bytes / 4.0e6;
            if (t < best_t - 1e-9) {
                best_t = t;
                best.rb = rb;
                best.tb = tb;
                best.splits = splits;
            }
        }
    }
    return best;
}

template <int T, int RB, int TB>
static hipError_t launch_tile_t(void* workspace, const uint8_t* w, uint32_t wbytes, float* y, int M, int N, int K,
                                int splits, int cu_count, hipStream_t stream) {
    uint8_t* base = static_cast<uint8_t*>(workspace);
    const _Float16* xh = reinterpret_cast<const _Float16*>(base);
    const size_t us_off = align256((size_t)M * K * 2);
    const float* us = reinterpret_cast<const float*>(base + us_off);
    float* part = reinterpret_cast<float*>(base + us_off + align256((size_t)M * 4));
    const int nb = K >> 8;
    const int split_sb = (nb + splits - 1) / splits;
    splits = (nb + split_sb - 1) / split_sb;
    const dim3 grid((N + 64 * RB - 1) / (64 * RB), (M + 16 * TB - 1) / (16 * TB), splits);
    hipLaunchKernelGGL((qgemm_tile_kernel<T, RB, TB>), grid, dim3(kTileThreads), 0, stream, w, wbytes, xh, us, y,
                       splits > 1 ? part : nullptr, M, N, K, split_sb);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    return launch_reduce(part, us, y, M, N, splits, cu_count, stream);
}

// M > 128 where neither rule above applies: 192-row x 128-token tiles with
// K split so the grid fits one round, at least 60% full, by the estimate of
// choose_tile_small. The 32x32 kernel is far slower at these sizes even
// against a partly idle round (Q4_K 4096 -> 12288: M = 192 65.1 -> 43.6 us
// with split 2, M = 256 75.2 -> 48.9 us with split 2, M = 384 85.0 -> 64.8 us
// at 75% fill; Q4_K 4096 -> 4096 at M = 512 44.2 against 46.9 us).
// Returns the split count, or 0 when no grid fits.
static int wide_tile_splits(int M, int N, int K, size_t room_bytes, int cu_count) {
    const long long cus = std::max(1, cu_count);
    const int nb = K >> 8;
    const size_t tile_bytes = (size_t)M * N * 4;
    const long long tiles =
        (long long)((N + 64 * kTileRb - 1) / (64 * kTileRb)) * ((M + 16 * kTileTb - 1) / (16 * kTileTb));
    int best = 0;
    double best_t = 1e30;
    for (int s = 1; s <= kMaxSplits && s <= nb; ++s) {
        const int split_sb = (nb + s - 1) / s;
        const int splits = (nb + split_sb - 1) / split_sb;
        if (splits > 1 && (size_t)splits * tile_bytes > room_bytes) break;
        const long long wgs = tiles * splits;
        if (wgs > cus) break;
        if (wgs * 5 < cus * 3) continue;
        double t = split_sb * (3.0 + 0.05 * kTileRb * kTileTb);
        if (splits > 1) t += 1.0 + (double)(2 * splits + 1) * (double)tile_bytes / 4.0e6;
        if (t < best_t - 1e-9) {
            best_t = t;
            best = splits;
        }
    }
    return best;
}

// Q5_K and Q6_K with M > 128 where the 192-row tiles do not fill the CUs
// (e.g. 12288 -> 4096): 256-row x 128-token tiles of four 64-row waves with
// K split so that the grid fills 60-100% of one round, the split count by
// the estimate of choose_tile_small. 64-row waves read a quarter less LDS
// per MFMA than 48-row ones, which matters for the costlier 5- and 6-bit
// dequantisation. Measured at 12288 -> 4096 against the 32x32 kernel with
// split K: Q6_K 104.5 against 110.3 us at M = 512, 158.2 against 209.2 at
// M = 768; Q5_K 54.9 against 59.0 us at M = 256, 82.9 against 88.6 at
// M = 512, 141.4 against 213.1 at M = 1024. Returns 0 when none fits.
static int wide256_splits(int M, int N, int K, size_t room_bytes, int cu_count) {
    const long long cus = std::max(1, cu_count);
    const int nb = K >> 8;
    const size_t tile_bytes = (size_t)M * N * 4;
    const long long tiles = (long long)((N + 255) / 256) * ((M + 127) / 128);
    int best = 0;
    double best_t = 1e30;
    for (int s = 1; s <= kMaxSplits && s <= nb; ++s) {
        const int split_sb = (nb + s - 1) / s;
        const int splits = (nb + split_sb - 1) / split_sb;
        if (splits > 1 && (size_t)splits * tile_bytes > room_bytes) break;
        const long long wgs = tiles * splits;
        if (wgs > cus) break;
        if (wgs * 5 < cus * 3) continue;
        double t = split_sb * (3.0 + 0.05 * 4 * 8);
        if (splits > 1) t += 1.0 + (double)(2 * splits + 1) * (double)tile_bytes / 4.0e6;
        if (t < best_t - 1e-9) {
            best_t = t;
            best = splits;
        }
    }
    return best;
}

template <int T>
static hipError_t launch_qgemm_tile(void* workspace, const uint8_t* w, uint32_t wbytes, float* y, int M, int N, int K,
                                    int rb, int tb, int splits, int cu_count, hipStream_t stream) {
    if (rb == 3 && tb == 8) return launch_tile_t<T, 3, 8>(workspace, w, wbytes, y, M, N, K, splits, cu_count, stream);
    if (rb == 3 && tb == 4) return launch_tile_t<T, 3, 4>(workspace, w, wbytes, y, M, N, K, splits, cu_count, stream);
    if (rb == 2 && tb == 8) return launch_tile_t<T, 2, 8>(workspace, w, wbytes, y, M, N, K, splits, cu_count, stream);
    if (rb == 2 && tb == 4) return launch_tile_t<T, 2, 4>(workspace, w, wbytes, y, M, N, K, splits, cu_count, stream);
    if (rb == 4 && tb == 8) return launch_tile_t<T, 4, 8>(workspace, w, wbytes, y, M, N, K, splits, cu_count, stream);
    return hipErrorInvalidValue;
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
    // (the tile kernel's activation offsets of its last token tile must stay below 2^32)
    const bool tile_ok = (uint64_t)(M + kTileTokMax) * (uint64_t)K * 2u < (1ull << 32);
    if (tile_ok && M <= 128) {
        const size_t part_off = align256((size_t)M * K * 2) + align256((size_t)M * 4);
        const TileChoice c =
            choose_tile_small(M, N, K, workspace_bytes > part_off ? workspace_bytes - part_off : 0, cu_count);
        if (c.rb) return launch_qgemm_tile<T>(workspace, w, wbytes, y, M, N, K, c.rb, c.tb, c.splits, cu_count, stream);
    }
    if (M <= 64) return launch_qgemm_t<T, 2, 2>(w, wbytes, workspace, workspace_bytes, y, M, N, K, cu_count, stream);
    if (tile_ok && M >= kTileWideM && use_tile(M, N, cu_count, 4, 9))
        return launch_qgemm_tile<T>(workspace, w, wbytes, y, M, N, K, 4, kTileTb, 1, cu_count, stream);
    if (tile_ok && M > 128 && use_tile(M, N, cu_count))
        return launch_qgemm_tile<T>(workspace, w, wbytes, y, M, N, K, kTileRb, kTileTb, 1, cu_count, stream);
    if (tile_ok && M > 128) {
        const size_t part_off = align256((size_t)M * K * 2) + align256((size_t)M * 4);
        const size_t room = workspace_bytes > part_off ? workspace_bytes - part_off : 0;
        if constexpr (T == kQ5K || T == kQ6K) {
            const int s = wide256_splits(M, N, K, room, cu_count);
            if (s) return launch_qgemm_tile<T>(workspace, w, wbytes, y, M, N, K, 4, 8, s, cu_count, stream);
        }
        const int s = wide_tile_splits(M, N, K, room, cu_count);
        if (s) return launch_qgemm_tile<T>(workspace, w, wbytes, y, M, N, K, kTileRb, kTileTb, s, cu_count, stream);
    }
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

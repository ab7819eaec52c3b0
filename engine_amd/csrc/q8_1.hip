// Q8_1 activation packing and the integer-dot k-quant GEMV that consumes it
// (gfx950 / CDNA4, wave64): the reference's experimental lossy projection
// path (crates/nvidia/src/activation.rs, q{4,5,6}_q8_1.rs; selected by
// GemvMode::IntegerDot, decode.rs:1341-1478).
//
// Q8_1 (activation.cu:1-28): each 32-value block of x becomes nine 32-bit
// words, half(d) | half(sum(x)) << 16 followed by 32 signed bytes
// q = round(x / d) (half away from zero) with d = max|x| / 127. The packer
// forms the block maximum and sum with the same xor butterfly over 32 lanes
// (offsets 16, 8, 4, 2, 1), so the words are bit-identical to the
// reference's.
//
// GEMV: row n gains, per 32-value group g of each super-block,
//     ((d * sc_g) * d8_g) * dot_g - (dmin * m_g) * s8_g       (Q4_K, Q5_K)
//     ((d * sc_h) * d8_g) * dot_h   for each 16-value half h   (Q6_K)
// with dot = sum(q_w * q_a) over the group (v_dot4_i32_i8; Q6_K quants enter
// as q - 32, the same integer as the reference's dot - 32 * sum(q_a)). A wave
// takes one row at a time: lane l covers super-block l / 4 of each 16-block
// slice of K and groups 2 (l % 4), 2 (l % 4) + 1, so a wave's weight loads
// are contiguous in the row. Up to kQ8MaxMembers members share each decoded
// weight word; member outputs are [member][row].
#include "kquant_device.hpp"
#include "kquant_launch.hpp"

namespace ribn_amd {

namespace {

constexpr uint32_t kOOR = 0xffffff00u;  // buffer offset past any tensor: loads return 0
constexpr int kThreads = 256;           // four rows (waves) per workgroup

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int acc) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, acc, false);
}

// ------------------------------------------------------------------ packer

__global__ __launch_bounds__(kThreads) void quantize_q8_1_kernel(const float* __restrict__ x, uint32_t* out,
                                                                 uint32_t blocks) {
    const uint32_t block = blockIdx.x * (kThreads / 32) + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    // whole half-waves take part in the butterfly; blocks past the end only
    // skip their loads and stores
    const bool live = block < blocks;
    const float v = live ? x[(size_t)block * 32 + lane] : 0.f;
    float maximum = fabsf(v);
    float sum = v;
#pragma unroll
    for (int offset = 16; offset > 0; offset >>= 1) {
        maximum = fmaxf(maximum, __shfl_xor(maximum, offset, 64));
        sum += __shfl_xor(sum, offset, 64);
    }
    const float d = maximum / 127.0f;
    const int q = maximum == 0.0f ? 0 : (int)roundf(v / d);
    // lane 4i + j contributes byte j of word i
    uint32_t packed = (uint32_t)q & 0xffu;
    packed |= (uint32_t)__shfl_down((int)packed, 1, 64) << 8;
    packed |= (uint32_t)__shfl_down((int)packed, 2, 64) << 16;
    if (!live) return;
    uint32_t* dst = out + (size_t)block * 9;
    if ((lane & 3) == 0) dst[1 + lane / 4] = packed;
    if (lane == 0) {
        const uint16_t dh = __builtin_bit_cast(uint16_t, (_Float16)d);
        const uint16_t sh = __builtin_bit_cast(uint16_t, (_Float16)sum);
        dst[0] = (uint32_t)dh | ((uint32_t)sh << 16);
    }
}

// -------------------------------------------------------------------- GEMV

// The nine words of one member's Q8_1 block: header, then 8 quant words.
struct Q8Block {
    uint32_t head;
    uint4 qa, qb;
};

__device__ __forceinline__ Q8Block load_q8(__amdgpu_buffer_rsrc_t r, uint32_t off, bool live) {
    Q8Block b;
    b.head = load_b32(r, live ? off : kOOR);
    b.qa = load_b128(r, live ? off + 4u : kOOR);
    b.qb = load_b128(r, live ? off + 20u : kOOR);
    return b;
}

__device__ __forceinline__ int dot_words(const uint32_t (&w)[8], const Q8Block& a) {
    int s = 0;
    s = dot4(w[0], a.qa.x, s);
    s = dot4(w[1], a.qa.y, s);
    s = dot4(w[2], a.qa.z, s);
    s = dot4(w[3], a.qa.w, s);
    s = dot4(w[4], a.qb.x, s);
    s = dot4(w[5], a.qb.y, s);
    s = dot4(w[6], a.qb.z, s);
    s = dot4(w[7], a.qb.w, s);
    return s;
}

// Half-window dot: words 0..3 (values 0..15) or 4..7 (values 16..31).
__device__ __forceinline__ int dot_half(const uint32_t (&w)[8], const Q8Block& a, int h) {
    int s = 0;
    if (h == 0) {
        s = dot4(w[0], a.qa.x, s);
        s = dot4(w[1], a.qa.y, s);
        s = dot4(w[2], a.qa.z, s);
        s = dot4(w[3], a.qa.w, s);
    } else {
        s = dot4(w[4], a.qb.x, s);
        s = dot4(w[5], a.qb.y, s);
        s = dot4(w[6], a.qb.z, s);
        s = dot4(w[7], a.qb.w, s);
    }
    return s;
}

struct Q8GemvArgs {
    const uint8_t* w;
    uint32_t wbytes;
    const uint32_t* x;  // [members][K / 32][9]
    float* y;           // [members][N]
    int K, N, members;
};

template <int T>
__global__ __launch_bounds__(kThreads) void q8_1_gemv_kernel(Q8GemvArgs a) {
    constexpr int BB = BlockTraits<T>::bytes;
    const int lane = threadIdx.x & 63;
    const int row = (int)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= a.N) return;  // whole waves
    const int nb = a.K >> 8;
    const int p = lane & 3;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, a.wbytes);
    const uint32_t member_words = (uint32_t)(a.K / 32) * 9u;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)a.members * member_words * 4u);
    float acc[kQ8MaxMembers];
#pragma unroll
    for (int m = 0; m < kQ8MaxMembers; ++m) acc[m] = 0.f;
    for (int s0 = 0; s0 < nb; s0 += 16) {
        const int b = s0 + (lane >> 2);
        const bool live = b < nb;
        const uint32_t off = (uint32_t)row * (uint32_t)nb * BB + (uint32_t)b * BB;
        if constexpr (T == kQ4K || T == kQ5K) {
            const uint4 h = load_b128(wr, live ? off : kOOR);
            const uint32_t qbase = T == kQ4K ? 16u : 48u;
            const uint4 q0 = load_b128(wr, live ? off + qbase + 32u * p : kOOR);
            const uint4 q1 = load_b128(wr, live ? off + qbase + 32u * p + 16u : kOOR);
            uint4 h0 = {0u, 0u, 0u, 0u}, h1 = {0u, 0u, 0u, 0u};
            if constexpr (T == kQ5K) {
                h0 = load_b128(wr, live ? off + 16u : kOOR);
                h1 = load_b128(wr, live ? off + 32u : kOOR);
            }
            const float d = half_bits_to_float(h.x & 0xffffu);
            const float dmin = half_bits_to_float(h.x >> 16);
            const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            const uint32_t hw[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int g = 2 * p + hh;
                uint32_t wq[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    wq[i] = (qw[i] >> (4 * hh)) & 0x0f0f0f0fu;
                    if constexpr (T == kQ5K) wq[i] |= ((hw[i] >> g) & 0x01010101u) << 4;
                }
                uint32_t sc, mn;
                q4k_scale_min(h.y, h.z, h.w, g, sc, mn);
                const float dsc = d * (float)sc;
                const float dmn = dmin * (float)mn;
                // members unrolled with guards: acc[] stays in registers
#pragma unroll
                for (int m = 0; m < kQ8MaxMembers; ++m) {
                    if (m < a.members) {
                        const Q8Block x =
                            load_q8(xr, ((uint32_t)m * member_words + (uint32_t)(b * 8 + g) * 9u) * 4u, live);
                        const int dot = dot_words(wq, x);
                        const float d8 = half_bits_to_float(x.head & 0xffffu);
                        const float s8 = half_bits_to_float(x.head >> 16);
                        // the reference's two accumulator updates, in its order
                        acc[m] += dsc * d8 * (float)dot;
                        acc[m] -= dmn * s8;
                    }
                }
            }
        } else {
            // Q6_K: ql [128] at 0, qh [64] at 128, int8 scales [16] at 192, d at 208
            // (crates/gguf/src/lib.rs:628-661). Group g (values 32g .. 32g + 31):
            // half hf = g / 4, quadrant c = g % 4; value l takes ql byte
            // 64 hf + 32 (c & 1) + l (nibble c / 2), qh byte 128 + 32 hf + l
            // (bits 2c, 2c + 1) and scale 8 hf + 2c + l / 16.
            const int hf = p >> 1;
            const uint4 lq0 = load_16_at_half_aligned(wr, live ? off + 64u * hf : kOOR);
            const uint4 lq1 = load_16_at_half_aligned(wr, live ? off + 64u * hf + 16u : kOOR);
            const uint4 lq2 = load_16_at_half_aligned(wr, live ? off + 64u * hf + 32u : kOOR);
            const uint4 lq3 = load_16_at_half_aligned(wr, live ? off + 64u * hf + 48u : kOOR);
            const uint4 qh0 = load_16_at_half_aligned(wr, live ? off + 128u + 32u * hf : kOOR);
            const uint4 qh1 = load_16_at_half_aligned(wr, live ? off + 128u + 32u * hf + 16u : kOOR);
            const uint4 scw = load_16_at_half_aligned(wr, live ? off + 192u : kOOR);
            const uint32_t dbits = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(wr, live ? (int)(off + 208u) : (int)kOOR, 0, kStreamPolicy);
            const float d = half_bits_to_float(dbits);
            const uint32_t lw[16] = {lq0.x, lq0.y, lq0.z, lq0.w, lq1.x, lq1.y, lq1.z, lq1.w,
                                     lq2.x, lq2.y, lq2.z, lq2.w, lq3.x, lq3.y, lq3.z, lq3.w};
            const uint32_t hw[8] = {qh0.x, qh0.y, qh0.z, qh0.w, qh1.x, qh1.y, qh1.z, qh1.w};
            const uint32_t scs[4] = {scw.x, scw.y, scw.z, scw.w};
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int c = 2 * (p & 1) + hh;  // quadrant of group 2p + hh
                const int g = 2 * p + hh;
                uint32_t wq[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t lo = (lw[8 * (c & 1) + i] >> (4 * (c >> 1))) & 0x0f0f0f0fu;
                    const uint32_t hi = (hw[i] >> (2 * c)) & 0x03030303u;
                    // q - 32 as an int8 per byte (q in 0..63) without carries
                    // between bytes: r = q ^ 32 is q - 32 for q >= 32 and
                    // q + 32 otherwise, where bit 5 is set and sign-extends
                    const uint32_t r = (lo | (hi << 4)) ^ 0x20202020u;
                    wq[i] = r | ((r & 0x20202020u) * 6u);
                }
                float dsc[2];
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2) {
                    const int si = 8 * hf + 2 * c + h2;
                    const int8_t sc = (int8_t)((scs[si >> 2] >> (8 * (si & 3))) & 0xffu);
                    dsc[h2] = d * (float)sc;
                }
#pragma unroll
                for (int m = 0; m < kQ8MaxMembers; ++m) {
                    if (m < a.members) {
                        const Q8Block x =
                            load_q8(xr, ((uint32_t)m * member_words + (uint32_t)(b * 8 + g) * 9u) * 4u, live);
                        const float d8 = half_bits_to_float(x.head & 0xffffu);
#pragma unroll
                        for (int h2 = 0; h2 < 2; ++h2) {
                            const int dot = dot_half(wq, x, h2);
                            acc[m] += dsc[h2] * d8 * (float)dot;
                        }
                    }
                }
            }
        }
    }
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(a.y, (uint32_t)a.members * (uint32_t)a.N * 4u);
#pragma unroll
    for (int m = 0; m < kQ8MaxMembers; ++m) {
        if (m < a.members) {
            const float total = wave_sum(acc[m]);
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, total), yr,
                                                  lane == 0 ? (int)(((uint32_t)m * a.N + row) * 4u) : (int)kOOR, 0,
                                                  0);
        }
    }
}

}  // namespace

hipError_t launch_quantize_q8_1(const float* x, uint32_t* out, uint32_t blocks, hipStream_t stream) {
    if (blocks == 0) return hipErrorInvalidValue;
    const uint32_t per = kThreads / 32;
    hipLaunchKernelGGL(quantize_q8_1_kernel, dim3((blocks + per - 1) / per), dim3(kThreads), 0, stream, x, out,
                       blocks);
    return hipGetLastError();
}

hipError_t launch_gemv_q8_1(int value_type, const uint8_t* w, uint32_t wbytes, const uint32_t* x, float* y, int K,
                            int N, int members, hipStream_t stream) {
    if (K < 256 || K % 256 != 0 || N < 1 || members < 1 || members > kQ8MaxMembers) return hipErrorInvalidValue;
    Q8GemvArgs a{w, wbytes, x, y, K, N, members};
    const dim3 grid((unsigned)((N + kThreads / 64 - 1) / (kThreads / 64)));
    switch (value_type) {
    case kQ4K: hipLaunchKernelGGL(q8_1_gemv_kernel<kQ4K>, grid, dim3(kThreads), 0, stream, a); break;
    case kQ5K: hipLaunchKernelGGL(q8_1_gemv_kernel<kQ5K>, grid, dim3(kThreads), 0, stream, a); break;
    case kQ6K: hipLaunchKernelGGL(q8_1_gemv_kernel<kQ6K>, grid, dim3(kThreads), 0, stream, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace ribn_amd

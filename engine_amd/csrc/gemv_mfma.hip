// Batched k-quant GEMV on the int8 matrix cores (gfx950 / CDNA4, wave64),
// for up to 16 members: the weights-read-once batch product of the decode path
// (quantized.rs batch GEMV, decode.rs:1480-1558) where the wave GEMV's
// per-member integer dot products become VALU-bound.
//
// Activations (pack_act16_kernel, one launch per product)
//  - Each member's x (times the RMSNorm weight gamma when given) is cut into
//    256-element super-blocks. A block with max|x| < 2^e is stored as 15-bit
//    fixed point v = rint(x * 2^(14-e)), |v| <= 2^14, split into two signed
//    digits v = 256 h + l with l in [-128, 127] and h in [-64, 64], so both
//    planes are int8 MFMA operands and every product stays exact.
//  - Per (member tile of 16, block): 8 groups x 64 lanes x 16 bytes of
//    fragments in the MFMA A-operand order (lane = member + 16 * chunk, eight
//    h bytes then eight l bytes of elements 32g + 8 chunk .. + 7), the block
//    unscale 2^(e-14) of each member, and u * X_g (X_g = sum of v over group g)
//    for the minimum term.
//  - Up to 8 members ("HL" layout): the A operand's 16 rows hold the h digits
//    of members 0-7 (rows 0-7) and their l digits (rows 8-15), so one MFMA per
//    group yields both digit sums; 4 x 64 lanes x 16 bytes per block (a lane
//    record = 8 bytes of group 2p, then 8 of group 2p + 1). The minimum term
//    rides on the l rows. A workgroup also writes its partial sum of x^2, so
//    the product applies RMSNorm's 1/rms per member at its output (the wave
//    GEMV's factorisation: y = (W (x * gamma)) / rms).
//
// Product (mfma_gemv_kernel)
//  - A wave owns R tiles of 16 weight rows over a contiguous range of
//    super-blocks, loaded through a two-slot ring refilled unconditionally
//    (blocks past the range load zeros) with the refills pinned between the
//    slots' MFMAs, so each wait covers one slot; the KS waves of a
//    workgroup split K and add their results in LDS in wave order
//    (deterministic).
//  - Per 32-element k-quant group g, two v_mfma_i32_16x16x32_i8 (h and l
//    planes; A = activations [member][k], B = quants [k][row]) give the exact
//    S_g = sum(q v) for 16 members x 16 rows. With the group's scale a_g =
//    d * sc_g (crates/gguf/src/lib.rs:573-612) the block contributes
//    u_b * sum_g a_g S_g; the minimum term sum_g (dmin * m_g) (u_b X_g) is a
//    [member][group] x [group][row] product on v_mfma_f32_16x16x4_f32.
//  - Lane l holds output rows l % 16 for members 4 (l / 16) .. + 3, so each
//    lane decodes the scales of one weight row per block.
//  - HL: rows 0-7 and 8-15 of the result are one member's h and l sums; lane
//    halves combine once at the end (256 h + l).
// Each member's result depends only on its own activations and on the layout
// (up to 8 members, or more): a member's output bits do not change with the
// other members' values.
#include "kquant_device.hpp"
#include "kquant_launch.hpp"

#include <algorithm>
#include <type_traits>

namespace ribn_amd {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr uint32_t kOOR = 0xffffff00u;   // buffer offset past any tensor: loads return 0, stores drop
constexpr int kPackBlocks = 8;           // super-blocks one pack workgroup covers
constexpr int kFragBlockBytes = 8 * 64 * 16;
constexpr int kMinBlockBytes = 64 * 8;
constexpr int kUBlockBytes = 16 * 4;
constexpr int kMaxWaves = 4;             // K-split waves per workgroup

__device__ __forceinline__ uint2 load_b64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}

__device__ __forceinline__ long as_long(uint32_t lo, uint32_t hi) {
    return (long)(((unsigned long)hi << 32) | lo);
}

// ------------------------------------------------------------ activation pack

struct PackArgs {
    const float* x;      // [members][K]
    const float* gamma;  // [K] or null
    uint8_t* act;
    Act16Layout L;
    int K;
};

__global__ __launch_bounds__(256) void pack_act16_kernel(PackArgs a) {
    __shared__ float wsum[4];
    const int m = blockIdx.y;
    const int tid = threadIdx.x;
    const int b = blockIdx.x * kPackBlocks + (tid >> 5);
    const int c = tid & 31;
    const int g = c >> 2, kq = c & 3;
    const int nb = a.L.nb;
    const bool live = b < nb;
    float v[8];
    float ssq = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = 0.f;
    if (live) {
        const size_t e0 = (size_t)m * a.K + (size_t)b * 256 + 32 * g + 8 * kq;
        const float4 x0 = *reinterpret_cast<const float4*>(a.x + e0);
        const float4 x1 = *reinterpret_cast<const float4*>(a.x + e0 + 4);
        v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
        v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
#pragma unroll
        for (int j = 0; j < 8; ++j) ssq += v[j] * v[j];
        if (a.gamma != nullptr) {
            const size_t k0 = (size_t)b * 256 + 32 * g + 8 * kq;
            const float4 g0 = *reinterpret_cast<const float4*>(a.gamma + k0);
            const float4 g1 = *reinterpret_cast<const float4*>(a.gamma + k0 + 4);
            v[0] *= g0.x; v[1] *= g0.y; v[2] *= g0.z; v[3] *= g0.w;
            v[4] *= g1.x; v[5] *= g1.y; v[6] *= g1.z; v[7] *= g1.w;
        }
    }
    // block maximum over the 32 lanes of this block (a half wave)
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    // mx < 2^ex; blocks below 2^-100 quantize to zero
    int ex = mx > 0.f ? __builtin_amdgcn_frexp_expf(mx) : 0;
    ex = ex < -100 ? -100 : ex;
    const int sh = 14 - ex;
    uint32_t hw[2] = {0u, 0u}, lw[2] = {0u, 0u};
    int xs = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q = (int)__builtin_rintf(__builtin_amdgcn_ldexpf(v[j], sh));  // |q| <= 2^14
        xs += q;
        const int lo = ((q + 128) & 255) - 128;
        const int hi = (q - lo) >> 8;
        hw[j >> 2] |= ((uint32_t)hi & 0xffu) << (8 * (j & 3));
        lw[j >> 2] |= ((uint32_t)lo & 0xffu) << (8 * (j & 3));
    }
    xs += __shfl_xor(xs, 1, 64);
    xs += __shfl_xor(xs, 2, 64);  // X_g over the four chunks of group g
    if (live && a.L.hl) {
        const size_t blk = (size_t)b;
        uint8_t* fr = a.act + a.L.frag + (blk * 4 + (g >> 1)) * 1024 + (g & 1) * 8;
        *reinterpret_cast<uint2*>(fr + (m + 16 * kq) * 16) = make_uint2(hw[0], hw[1]);
        *reinterpret_cast<uint2*>(fr + (m + 8 + 16 * kq) * 16) = make_uint2(lw[0], lw[1]);
        if (kq == 0) {
            float* mina = reinterpret_cast<float*>(a.act + a.L.mina);
            mina[(blk * 64 + m + 8 + 16 * (g & 3)) * 2 + (g >> 2)] = __builtin_amdgcn_ldexpf((float)xs, ex - 14);
            mina[(blk * 64 + m + 16 * (g & 3)) * 2 + (g >> 2)] = 0.f;
        }
        if (c == 0) {
            float* ub = reinterpret_cast<float*>(a.act + a.L.ublk);
            ub[blk * 16 + m] = __builtin_amdgcn_ldexpf(1.0f, ex - 14);
            ub[blk * 16 + m + 8] = __builtin_amdgcn_ldexpf(1.0f, ex - 14);
        }
    } else if (live) {
        const int mt = m >> 4, mi = m & 15;
        const size_t blk = (size_t)mt * nb + b;
        uint4 f;
        f.x = hw[0]; f.y = hw[1]; f.z = lw[0]; f.w = lw[1];
        *reinterpret_cast<uint4*>(a.act + a.L.frag + ((blk * 8 + g) * 64 + mi + 16 * kq) * 16) = f;
        if (kq == 0) {
            float* mina = reinterpret_cast<float*>(a.act + a.L.mina);
            mina[(blk * 64 + mi + 16 * (g & 3)) * 2 + (g >> 2)] = __builtin_amdgcn_ldexpf((float)xs, ex - 14);
        }
        if (c == 0) {
            reinterpret_cast<float*>(a.act + a.L.ublk)[blk * 16 + mi] = __builtin_amdgcn_ldexpf(1.0f, ex - 14);
        }
    }
    // this workgroup's share of sum(x^2), for RMSNorm (summed in part order by the product)
    const float ws = wave_sum(ssq);
    if ((tid & 63) == 0) wsum[tid >> 6] = ws;
    __syncthreads();
    if (tid == 0) {
        reinterpret_cast<float*>(a.act + a.L.ssq)[m * a.L.parts + blockIdx.x] =
            (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    }
}

// ------------------------------------------------------------------ product

template <int T> struct WRaw;
template <> struct WRaw<kQ4K> { uint4 h; uint2 q[4]; };
template <> struct WRaw<kQ5K> { uint4 h; uint2 qh; uint2 q[4]; };
// Q6_K: the 16 int8 scales, d, and for each half n the 8 low-nibble bytes of
// both 32-byte quadrant pairs (ql[2n], ql[2n + 1]) and the 8 qh bytes.
template <> struct WRaw<kQ6K> { uint4 sc; uint32_t d16; uint2 ql[4]; uint2 qh[2]; };

// One lane's bytes of a 16-row tile's super-block: the 16-byte header (d,
// dmin, packed scales) and, for each group pair p, the 8 quant bytes of
// elements 8 kq .. 8 kq + 7 (low nibbles: group 2p, high: 2p + 1).
template <int T>
__device__ __forceinline__ void load_w(WRaw<T>& d, __amdgpu_buffer_rsrc_t r, bool live, uint32_t base, int kq) {
    if constexpr (T == kQ6K) {
        // block: ql[128] at 0, qh[64] at 128, scales[16] at 192, d at 208
        d.sc = load_b128(r, live ? base + 192u : kOOR);
        d.d16 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, live ? (int)(base + 208u) : (int)kOOR, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) d.ql[i] = load_b64(r, live ? base + 32u * i + 8u * kq : kOOR);
#pragma unroll
        for (int n = 0; n < 2; ++n) d.qh[n] = load_b64(r, live ? base + 128u + 32u * n + 8u * kq : kOOR);
        return;
    } else {
    d.h = load_b128(r, live ? base : kOOR);
    if constexpr (T == kQ5K) {
        d.qh = load_b64(r, live ? base + 16u + 8u * kq : kOOR);
#pragma unroll
        for (int p = 0; p < 4; ++p) d.q[p] = load_b64(r, live ? base + 48u + 32u * p + 8u * kq : kOOR);
    } else {
#pragma unroll
        for (int p = 0; p < 4; ++p) d.q[p] = load_b64(r, live ? base + 16u + 32u * p + 8u * kq : kOOR);
    }
    }
}

// Q6_K quants of 32-element group g (half n = g / 4, quadrant t = g % 4,
// elements l = 8 kq .. 8 kq + 7 of the quadrant, crates/gguf/src/lib.rs
// 627-661): low nibble of ql[64 n + 32 (t & 1) + l] (high nibble for t >= 2)
// and bits 2t, 2t + 1 of qh[32 n + l], minus 32, as signed bytes. The
// subtraction is carry-free per byte: x = q ^ 32 is q - 32 for q >= 32, and
// q - 32 + 64 otherwise, which setting bits 6-7 turns into q - 32.
__device__ __forceinline__ long q6_group(const WRaw<kQ6K>& d, int g) {
    const int n = g >> 2, t = g & 3;
    const uint2 lo = d.ql[2 * n + (t & 1)];
    const uint2 hi = d.qh[n];
    const int sl = (t >> 1) * 4, sh = 2 * t;
    uint32_t w[2] = {lo.x, lo.y}, h2[2] = {hi.x, hi.y}, out[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t q = ((w[i] >> sl) & 0x0f0f0f0fu) | (((h2[i] >> sh) & 0x03030303u) << 4);
        const uint32_t x = q ^ 0x20202020u;
        out[i] = x | ((x & 0x20202020u) * 6u);
    }
    return as_long(out[0], out[1]);
}

// Q6_K over one super-block: per 32-element group, two MFMAs whose A operand
// keeps only lanes of one 16-element scale group (k 0..15: lanes kq 0-1;
// 16..31: kq 2-3), scaled by d * scale in f32. No minimum term. With `hl`,
// one A plane per MFMA (packed digits); otherwise the h and l planes.
template <bool HL, class Act>
__device__ __forceinline__ void block_mma_q6(const WRaw<kQ6K>& d, const Act& x, int kq, v4f& acc) {
    const float dd = half_bits_to_float(d.d16 & 0xffffu);
    const uint32_t scw[4] = {d.sc.x, d.sc.y, d.sc.z, d.sc.w};
    const v4i zero = {0, 0, 0, 0};
    const bool low_half = kq < 2;
    float accb[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const long bq = q6_group(d, g);
        // scale index 8 n + 2 t + (l / 16): bytes 2g and 2g + 1 of the scales
        const uint32_t sw = scw[g >> 1] >> (16 * (g & 1));
        const float s0 = dd * (float)(int8_t)(sw & 0xffu);
        const float s1 = dd * (float)(int8_t)((sw >> 8) & 0xffu);
        long a_h, a_l;
        if constexpr (HL) {
            const int p = g >> 1;
            a_h = (g & 1) ? as_long(x.f[p].z, x.f[p].w) : as_long(x.f[p].x, x.f[p].y);
            a_l = 0;
        } else {
            a_h = as_long(x.f[g].x, x.f[g].y);
            a_l = as_long(x.f[g].z, x.f[g].w);
        }
        const long h0 = low_half ? a_h : 0, h1 = low_half ? 0 : a_h;
        const v4i c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(h0, bq, zero, 0, 0, 0);
        const v4i c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(h1, bq, zero, 0, 0, 0);
        if constexpr (HL) {
#pragma unroll
            for (int t = 0; t < 4; ++t) accb[t] = __builtin_fmaf(s1, (float)c1[t], __builtin_fmaf(s0, (float)c0[t], accb[t]));
        } else {
            const long l0 = low_half ? a_l : 0, l1 = low_half ? 0 : a_l;
            const v4i e0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(l0, bq, zero, 0, 0, 0);
            const v4i e1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(l1, bq, zero, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                accb[t] = __builtin_fmaf(s0, (float)(c0[t] * 256 + e0[t]), accb[t]);
                accb[t] = __builtin_fmaf(s1, (float)(c1[t] * 256 + e1[t]), accb[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = __builtin_fmaf(x.u[t], accb[t], acc[t]);
}

struct ActBlk {
    uint4 f[8];   // fragments of the 8 groups
    float2 mina;  // u X for groups kq and 4 + kq of member lane % 16
    float4 u;     // block unscale of members 4 kq .. 4 kq + 3
};

// Lanes of absent members (lane % 16 >= members) load nothing: their A rows
// only reach output rows that are never stored.
__device__ __forceinline__ void load_act(ActBlk& x, __amdgpu_buffer_rsrc_t r, const MfmaGemvArgs& A, bool live,
                                         int b, int lane) {
    const bool own = live && (lane & 15) < A.members;
    const uint32_t fb = A.L.frag + ((uint32_t)b * 8u * 64u + (uint32_t)lane) * 16u;
#pragma unroll
    for (int g = 0; g < 8; ++g) x.f[g] = load_b128(r, own ? fb + 1024u * g : kOOR);
    const uint2 mn = load_b64(r, own ? A.L.mina + ((uint32_t)b * 64u + (uint32_t)lane) * 8u : kOOR);
    x.mina = __builtin_bit_cast(float2, mn);
    const bool any = live && 4 * (lane >> 4) < A.members;
    const uint4 uu = load_b128(r, any ? A.L.ublk + ((uint32_t)b * 16u + 4u * (uint32_t)(lane >> 4)) * 4u : kOOR);
    x.u = __builtin_bit_cast(float4, uu);
}

struct ActBlkHL {
    uint4 f[4];   // group pairs: 8 bytes of group 2p, then 8 of group 2p + 1
    float2 mina;  // u X of groups kq and 4 + kq (l rows; zero on h rows)
    float4 u;     // block unscale of rows 4 kq .. 4 kq + 3
};

// Lanes whose row belongs to an absent member load nothing.
__device__ __forceinline__ void load_act_hl(ActBlkHL& x, __amdgpu_buffer_rsrc_t r, const MfmaGemvArgs& A, bool live,
                                            int b, int lane) {
    const bool own = live && (lane & 7) < A.members;
    const uint32_t fb = A.L.frag + ((uint32_t)b * 4u * 64u + (uint32_t)lane) * 16u;
#pragma unroll
    for (int p = 0; p < 4; ++p) x.f[p] = load_b128(r, own ? fb + 1024u * p : kOOR);
    const uint2 mn = load_b64(r, own ? A.L.mina + ((uint32_t)b * 64u + (uint32_t)lane) * 8u : kOOR);
    x.mina = __builtin_bit_cast(float2, mn);
    const uint4 uu = load_b128(r, live ? A.L.ublk + ((uint32_t)b * 16u + 4u * (uint32_t)(lane >> 4)) * 4u : kOOR);
    x.u = __builtin_bit_cast(float4, uu);
}

// block_mma for the HL layout: one MFMA per group gives the h sums (rows
// 0-7) and the l sums (rows 8-15) of up to 8 members.
template <int T>
__device__ __forceinline__ void block_mma_hl(const WRaw<T>& d, const ActBlkHL& x, int kq, v4f& acc, v4f& macc) {
    const uint4 h = d.h;
    const float dd = half_bits_to_float(h.x & 0xffffu);
    const float dmin = half_bits_to_float(h.x >> 16);
    const uint32_t lo_sc = h.y & 0x3f3f3f3fu;
    const uint32_t lo_mn = h.z & 0x3f3f3f3fu;
    const uint32_t hi_sc = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t hi_mn = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
    const v4i zero = {0, 0, 0, 0};
    float accb[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const int p = g >> 1, sh = 4 * (g & 1);
        uint32_t q0 = (d.q[p].x >> sh) & 0x0f0f0f0fu;
        uint32_t q1 = (d.q[p].y >> sh) & 0x0f0f0f0fu;
        if constexpr (T == kQ5K) {
            q0 |= ((d.qh.x >> g) & 0x01010101u) << 4;
            q1 |= ((d.qh.y >> g) & 0x01010101u) << 4;
        }
        const long av = (g & 1) ? as_long(x.f[p].z, x.f[p].w) : as_long(x.f[p].x, x.f[p].y);
        const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, as_long(q0, q1), zero, 0, 0, 0);
        const uint32_t scw = g < 4 ? lo_sc : hi_sc;
        const float a_g = dd * (float)((scw >> (8 * (g & 3))) & 0xffu);
#pragma unroll
        for (int t = 0; t < 4; ++t) accb[t] = __builtin_fmaf(a_g, (float)c[t], accb[t]);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = __builtin_fmaf(x.u[t], accb[t], acc[t]);
    const float b0 = dmin * (float)((lo_mn >> (8 * kq)) & 0xffu);
    const float b1 = dmin * (float)((hi_mn >> (8 * kq)) & 0xffu);
    macc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.mina.x, b0, macc, 0, 0, 0);
    macc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.mina.y, b1, macc, 0, 0, 0);
}

template <int T>
__device__ __forceinline__ void block_mma(const WRaw<T>& d, const ActBlk& x, int kq, v4f& acc, v4f& macc) {
    const uint4 h = d.h;
    const float dd = half_bits_to_float(h.x & 0xffffu);
    const float dmin = half_bits_to_float(h.x >> 16);
    // six-bit scales / minima of the 8 groups, four per word (lib.rs:573-587)
    const uint32_t lo_sc = h.y & 0x3f3f3f3fu;
    const uint32_t lo_mn = h.z & 0x3f3f3f3fu;
    const uint32_t hi_sc = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t hi_mn = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
    const v4i zero = {0, 0, 0, 0};
    float accb[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const int p = g >> 1, sh = 4 * (g & 1);
        uint32_t q0 = (d.q[p].x >> sh) & 0x0f0f0f0fu;
        uint32_t q1 = (d.q[p].y >> sh) & 0x0f0f0f0fu;
        if constexpr (T == kQ5K) {
            // fifth bit of element i of group g: bit g of qh[i]
            q0 |= ((d.qh.x >> g) & 0x01010101u) << 4;
            q1 |= ((d.qh.y >> g) & 0x01010101u) << 4;
        }
        const long bq = as_long(q0, q1);
        const v4i ch = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(x.f[g].x, x.f[g].y), bq, zero, 0, 0, 0);
        const v4i cl = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(x.f[g].z, x.f[g].w), bq, zero, 0, 0, 0);
        const uint32_t scw = g < 4 ? lo_sc : hi_sc;
        const float a_g = dd * (float)((scw >> (8 * (g & 3))) & 0xffu);
#pragma unroll
        for (int t = 0; t < 4; ++t) accb[t] = __builtin_fmaf(a_g, (float)(ch[t] * 256 + cl[t]), accb[t]);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = __builtin_fmaf(x.u[t], accb[t], acc[t]);
    // minimum term of groups kq and 4 + kq (the lane's row): A = u X [member][group], B = dmin m [group][row]
    const float b0 = dmin * (float)((lo_mn >> (8 * kq)) & 0xffu);
    const float b1 = dmin * (float)((hi_mn >> (8 * kq)) & 0xffu);
    macc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.mina.x, b0, macc, 0, 0, 0);
    macc = __builtin_amdgcn_mfma_f32_16x16x4f32(x.mina.y, b1, macc, 0, 0, 0);
}

// One workgroup of KS waves takes R tiles of 16 weight rows; wave w covers
// the super-blocks [nb w / KS, nb (w + 1) / KS) of K with a two-slot ring of
// (R tiles x one super-block) units, and the waves' partial sums meet in LDS
// in wave order.
template <int T, int R, bool PAIR, bool HL>
__global__ __launch_bounds__(512) void mfma_gemv_kernel(MfmaGemvArgs A) {
    constexpr int BB = BlockTraits<T>::bytes;
    constexpr int NBUF = 2;
    static_assert(!PAIR || R % 2 == 0, "pairs split the tiles into gate and up halves");
    extern __shared__ float red[];  // [KS - 1][R][4][64]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ks = (int)(blockDim.x >> 6);
    const int kq = lane >> 4, rl = lane & 15;
    const int nb = A.K >> 8;
    const uint32_t row_bytes = (uint32_t)nb * BB;
    const int kb0 = nb * wave / ks, kb1 = nb * (wave + 1) / ks;

    // tiles: (matrix, first local row); tiles never straddle matrices
    __amdgpu_buffer_rsrc_t wr[R];
    int mat[R], local0[R], rows_mat[R];
    bool live_row[R];
    uint32_t rowoff[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        if constexpr (PAIR) {
            mat[i] = i / (R / 2);
            local0[i] = ((int)blockIdx.x * (R / 2) + i % (R / 2)) * 16;
            rows_mat[i] = A.rows_end[0];
        } else {
            const int row0 = ((int)blockIdx.x * R + i) * 16;
            int mm = 0, start = 0;
#pragma unroll
            for (int j = 0; j < kMaxGroup - 1; ++j) {
                if (j + 1 < A.count && row0 >= A.rows_end[j]) {
                    mm = j + 1;
                    start = A.rows_end[j];
                }
            }
            mat[i] = mm;
            local0[i] = row0 < A.total_rows ? row0 - start : 1 << 30;
            rows_mat[i] = A.rows_end[mm] - start;
        }
        const int mm = mat[i];
        const uint8_t* w = A.w[0];
        uint32_t wb = A.wbytes[0];
#pragma unroll
        for (int j = 1; j < kMaxGroup; ++j) {
            if (mm == j) {
                w = A.w[j];
                wb = A.wbytes[j];
            }
        }
        wr[i] = make_rsrc(w, wb);
        const int lrow = local0[i] + rl;
        live_row[i] = lrow < rows_mat[i];
        rowoff[i] = live_row[i] ? (uint32_t)lrow * row_bytes : 0u;
    }
    const __amdgpu_buffer_rsrc_t ar = make_rsrc(A.act, A.act_bytes);

    v4f acc[R], macc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        acc[i] = (v4f){0.f, 0.f, 0.f, 0.f};
        macc[i] = (v4f){0.f, 0.f, 0.f, 0.f};
    }
    WRaw<T> ring[NBUF][R];
    using ActT = typename std::conditional<HL, ActBlkHL, ActBlk>::type;
    ActT act[NBUF];
    auto fill = [&](int s, int b) {
        const bool lb = b < kb1;
#pragma unroll
        for (int i = 0; i < R; ++i) load_w<T>(ring[s][i], wr[i], lb && live_row[i], rowoff[i] + (uint32_t)b * BB, kq);
        if constexpr (HL) {
            load_act_hl(act[s], ar, A, lb, b, lane);
        } else {
            load_act(act[s], ar, A, lb, b, lane);
        }
    };
    auto mma = [&](int s) {
#pragma unroll
        for (int i = 0; i < R; ++i) {
            if constexpr (T == kQ6K) {
                block_mma_q6<HL>(ring[s][i], act[s], kq, acc[i]);
            } else if constexpr (HL) {
                block_mma_hl<T>(ring[s][i], act[s], kq, acc[i], macc[i]);
            } else {
                block_mma<T>(ring[s][i], act[s], kq, acc[i], macc[i]);
            }
        }
    };
#pragma unroll
    for (int s = 0; s < NBUF; ++s) fill(s, kb0 + s);
    // Passes of NBUF blocks. Refills are unconditional (past the range they
    // load zeros) and pinned between the slots' MFMAs, so the loads behind a
    // slot are always the same and its wait covers that slot only; a
    // conditional refill made the compiler wait for every load at the top of
    // each pass. The last pass refills nothing.
    const int passes = (kb1 - kb0 + NBUF - 1) / NBUF;
    int bp = kb0;
    for (int pass = 0; pass + 1 < passes; ++pass, bp += NBUF) {
#pragma unroll
        for (int s = 0; s < NBUF; ++s) {
            mma(s);
            __builtin_amdgcn_sched_barrier(0);
            fill(s, bp + s + NBUF);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (passes > 0) {
        const int left = kb1 - bp;
#pragma unroll
        for (int s = 0; s < NBUF; ++s) {
            if (s < left) mma(s);
        }
    }

    // ---- K-split reduction in wave order, then the epilogue on wave 0
    float v[R][4];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
        for (int t = 0; t < 4; ++t) v[i][t] = acc[i][t] - macc[i][t];
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int t = 0; t < 4; ++t) red[((wave - 1) * R + i) * 256 + t * 64 + lane] = v[i][t];
    }
    __syncthreads();
    if (wave != 0) return;
    for (int w = 1; w < ks; ++w) {
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int t = 0; t < 4; ++t) v[i][t] += red[((w - 1) * R + i) * 256 + t * 64 + lane];
    }
    // HL: lanes 0-31 hold the h sums of members 4 kq + t, lanes 32-63 the l
    // sums of the same members
    const bool out_lane = !HL || kq < 2;
    if constexpr (HL) {
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float lo = __shfl_xor(v[i][t], 32, 64);
                v[i][t] = __builtin_fmaf(256.0f, v[i][t], lo);
            }
    }
    float inv[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        inv[t] = 1.f;
        const int mem = 4 * kq + t;
        if (A.has_norm && out_lane && mem < A.members) {
            const float* ssq = reinterpret_cast<const float*>(reinterpret_cast<const uint8_t*>(A.act) + A.L.ssq);
            float total = 0.f;
            for (int p = 0; p < A.L.parts; ++p) total += ssq[mem * A.L.parts + p];
            // RMSNorm (qwen_reference.rs:550-556): 1/sqrt(sum(x^2)/K + eps)
            inv[t] = 1.0f / sqrtf(total / (float)A.K + A.eps);
        }
    }
    const bool accumulate = A.accumulate != 0;
    auto put = [&](float value, __amdgpu_buffer_rsrc_t yr, uint32_t off) {
        if (accumulate) {
            __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(value, yr, (int)off, 0, 0);
        } else {
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, value), yr, (int)off, 0, 0);
        }
    };
    if constexpr (PAIR) {
        const int ffn = A.rows_end[0];
        const __amdgpu_buffer_rsrc_t yr = make_rsrc(A.y[0], (uint32_t)A.members * (uint32_t)ffn * 4u);
#pragma unroll
        for (int i = 0; i < R / 2; ++i) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int mem = 4 * kq + t;
                const float gt = v[i][t] * inv[t];
                const float up = v[i + R / 2][t] * inv[t];
                // silu(gate) * up, in the reference's operation order (model_ops.rs:316-328)
                const float out = (gt / (1.0f + expf(-gt))) * up;
                const bool ok = out_lane && live_row[i] && mem < A.members;
                put(out, yr, ok ? (uint32_t)(mem * ffn + local0[i] + rl) * 4u : kOOR);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int mm = mat[i];
            float* y = A.y[0];
#pragma unroll
            for (int j = 1; j < kMaxGroup; ++j) {
                if (mm == j) y = A.y[j];
            }
            const __amdgpu_buffer_rsrc_t yr = make_rsrc(y, (uint32_t)A.members * (uint32_t)rows_mat[i] * 4u);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int mem = 4 * kq + t;
                const bool ok = out_lane && live_row[i] && mem < A.members;
                put(v[i][t] * inv[t], yr, ok ? (uint32_t)(mem * rows_mat[i] + local0[i] + rl) * 4u : kOOR);
            }
        }
    }
}

template <int T, int R, bool PAIR>
hipError_t launch_shape(const MfmaGemvArgs& a, int groups, int ks, hipStream_t stream) {
    const size_t lds = (size_t)(ks - 1) * R * 256 * sizeof(float);
    if (a.L.hl) {
        hipLaunchKernelGGL((mfma_gemv_kernel<T, R, PAIR, true>), dim3((unsigned)groups), dim3((unsigned)(64 * ks)),
                           lds, stream, a);
    } else {
        hipLaunchKernelGGL((mfma_gemv_kernel<T, R, PAIR, false>), dim3((unsigned)groups), dim3((unsigned)(64 * ks)),
                           lds, stream, a);
    }
    return hipGetLastError();
}

template <int T>
hipError_t launch_t(const MfmaGemvArgs& a, hipStream_t stream) {
    const int nb = a.K >> 8;
    const bool pair = a.pair_swiglu != 0;
    const int tiles = pair ? (a.rows_end[0] + 15) / 16 : (a.total_rows + 15) / 16;
    // One tile per wave (a gate tile and its up tile for pairs): from sweeps on
    // MI355X over tiles per wave {1, 2, 4}, K splits {1, 2, 4, 8} and ring
    // depths {2, 3, 4} at 4, 8 and 16 members, the widest grid won.
    const int groups = tiles;
    // The K split depends on K alone, so a row's summation order (and bits)
    // is the same in every launch shape of a layout: grouped or not, any
    // member count up to 8, or any from 9 to 16.
    const int ks = std::min(kMaxWaves, std::max(1, nb / 2));
    if (pair) return launch_shape<T, 2, true>(a, groups, ks, stream);
    return launch_shape<T, 1, false>(a, groups, ks, stream);
}

bool rows_tile_aligned(const WaveGemvArgs& a) {
    if (a.pair_swiglu) return a.count == 2 && a.rows_end[1] == 2 * a.rows_end[0];
    for (int i = 0; i + 1 < a.count; ++i) {
        if (a.rows_end[i] % 16 != 0) return false;
    }
    return true;
}

}  // namespace

Act16Layout act16_layout(int members, int K) {
    Act16Layout L{};
    const int nb = K / 256;
    const int tiles = (members + 15) / 16;
    L.nb = nb;
    L.parts = (nb + kPackBlocks - 1) / kPackBlocks;
    L.hl = members <= 8 ? 1 : 0;
    const uint32_t blocks = (uint32_t)tiles * (uint32_t)nb;
    L.frag = 0;
    L.mina = L.frag + blocks * (L.hl ? kFragBlockBytes / 2 : kFragBlockBytes);
    L.ublk = L.mina + blocks * kMinBlockBytes;
    L.ssq = L.ublk + blocks * kUBlockBytes;
    L.total = L.ssq + (uint32_t)members * (uint32_t)L.parts * 4u;
    return L;
}

bool gemv_mfma_supported(int value_type) { return value_type == kQ4K || value_type == kQ5K || value_type == kQ6K; }

hipError_t launch_pack_act16(const float* x, const float* gamma, int members, int K, void* act,
                             hipStream_t stream) {
    if (members < 1 || members > kMfmaMaxMembers || K < 256 || K % 256 != 0 || K > kWaveMaxK) {
        return hipErrorInvalidValue;
    }
    PackArgs a{};
    a.x = x;
    a.gamma = gamma;
    a.act = static_cast<uint8_t*>(act);
    a.L = act16_layout(members, K);
    a.K = K;
    hipLaunchKernelGGL(pack_act16_kernel, dim3((unsigned)a.L.parts, (unsigned)members), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_gemv_mfma(int value_type, const MfmaGemvArgs& a, int /*cu_count*/, hipStream_t stream) {
    if (a.members < 1 || a.members > kMfmaMaxMembers || a.K < 256 || a.K % 256 != 0 || a.K > kWaveMaxK ||
        a.count < 1 || a.count > kMaxGroup) {
        return hipErrorInvalidValue;
    }
    if (a.pair_swiglu) {
        if (a.count != 2 || a.rows_end[1] != 2 * a.rows_end[0]) return hipErrorInvalidValue;
    } else {
        for (int i = 0; i + 1 < a.count; ++i) {
            if (a.rows_end[i] % 16 != 0) return hipErrorInvalidValue;  // tiles never straddle matrices
        }
    }
    switch (value_type) {
    case kQ4K: return launch_t<kQ4K>(a, stream);
    case kQ5K: return launch_t<kQ5K>(a, stream);
    case kQ6K: return launch_t<kQ6K>(a, stream);
    default: return hipErrorInvalidValue;
    }
}

// ------------------------------------------------------------ dispatcher

// The context scratch serves either the packed activations of the matrix-core
// GEMV or the slice totals of a split f32 launch (never both in one call).
size_t gemv_act_scratch_bytes() {
    const size_t f32mma = ((size_t)f32mma_layout(kF32MmaMaxMembers, kWaveMaxK).total + 255) / 256 * 256 +
                          kF32MmaPartialBytes;
    return std::max<size_t>(std::max<size_t>(act16_layout(kMfmaMaxMembers, kWaveMaxK).total, kF32SplitScratchBytes),
                            f32mma);
}

int gemv_launch_members(int value_type, int K, bool swiglu_prologue, int arith) {
    // a K beyond one launch's staging: launch_gemv runs the whole batch as
    // slice-split groups (f32 arithmetic in either mode)
    if (K > kWaveMaxK) return (!swiglu_prologue && K <= kF32SplitMaxK && K % 256 == 0) ? kF32MmaMaxMembers : 0;
    if (arith == kArithF32) {
        if (K < 256) return 0;
        // the whole batch: launch_gemv takes 9..64 members to the matrix
        // cores and splits smaller calls into the launch groups each wave
        // form stages
        if (gemv_mfma_supported(value_type) && K % 256 == 0) return kF32MmaMaxMembers;
        return swiglu_prologue ? kSwigluMaxMembers : kWaveMaxMembers;
    }
    if (!swiglu_prologue && gemv_mfma_supported(value_type) && K % 256 == 0 && K <= kWaveMaxK) {
        return kMfmaMaxMembers;
    }
    int per = std::min(wave_max_members(K), kWaveMaxMembers);
    if (swiglu_prologue) per = std::min(per, kSwigluMaxMembers);
    return per;
}

hipError_t launch_gemv(int value_type, const WaveGemvArgs& a0, void* act_scratch, int cu_count, hipStream_t stream) {
    WaveGemvArgs a = a0;
    if (a.arith == kArithF32 && act_scratch != nullptr && f32mma_supported(value_type, a) &&
        f32mma_layout(a.members, a.K).total <= gemv_act_scratch_bytes()) {
        return launch_gemv_f32mma(value_type, a, act_scratch, gemv_act_scratch_bytes(), cu_count, stream);
    }
    // any other path: a pending residual update is added on its own first,
    // and this call leaves nothing pending
    if (a.fold != nullptr && a.fold->splits > 0) {
        F32MmaFold f = *a.fold;
        hipError_t e = launch_f32mma_fold_flush(&f, stream);
        if (e != hipSuccess) return e;
        a.fold = nullptr;
    }
    if (a.defer != nullptr) *a.defer = F32MmaFold{};
    a.defer = nullptr;
    if (a.K > kWaveMaxK) {
        // K beyond what one workgroup stages: groups of up to 8 members in the
        // slice-split form (one slice staged per workgroup, the slice totals
        // added in order by the reduce launch), plain or accumulating
        // products, f32 arithmetic in either mode
        const int per = f32_long_k_members(a.K, a.total_rows);
        if (per <= 0 || act_scratch == nullptr || a.x2 != nullptr || a.gamma != nullptr || a.pair_swiglu) {
            return hipErrorInvalidValue;
        }
        for (int m0 = 0; m0 < a.members; m0 += per) {
            WaveGemvArgs c = a;
            c.members = std::min(per, a.members - m0);
            c.x = a.x + (size_t)m0 * a.K;
            for (int i = 0; i < a.count; ++i) {
                const int n = a.rows_end[i] - (i > 0 ? a.rows_end[i - 1] : 0);
                c.y[i] = a.y[i] + (size_t)m0 * n;
            }
            c.partial = static_cast<float*>(act_scratch);
            hipError_t e = launch_gemv_f32_split(value_type, c, cu_count, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    if (a.arith == kArithF32) {
        // the f32 wave GEMV, in launch groups of as many members as it stages;
        // 3..8 members over a K of several slices split by slice when the
        // context scratch holds their slice totals
        int per = f32_max_members(a.K);
        if (a.x2 != nullptr) per = std::min(per, kSwigluMaxMembers);
        if (per <= 0) return hipErrorInvalidValue;
        const bool splittable = a.K > kSliceK && a.x2 == nullptr && a.gamma == nullptr && !a.pair_swiglu &&
                                act_scratch != nullptr &&
                                f32_split_partial_bytes(kWaveMaxMembers, a.K, a.total_rows) <= kF32SplitScratchBytes;
        if (splittable) per = kWaveMaxMembers;
        for (int m0 = 0; m0 < a.members; m0 += per) {
            WaveGemvArgs c = a;
            c.members = std::min(per, a.members - m0);
            c.x = a.x + (size_t)m0 * a.K;
            c.x2 = a.x2 != nullptr ? a.x2 + (size_t)m0 * a.K : nullptr;
            for (int i = 0; i < a.count; ++i) {
                const int n = a.rows_end[i] - (i > 0 ? a.rows_end[i - 1] : 0);
                c.y[i] = a.y[i] + (size_t)m0 * (a.pair_swiglu ? a.rows_end[0] : n);
            }
            hipError_t e;
            if (splittable && c.members > 2) {
                c.partial = static_cast<float*>(act_scratch);
                e = launch_gemv_f32_split(value_type, c, cu_count, stream);
            } else if (c.members > f32_max_members(a.K)) {
                // two-member groups of the one-launch form
                e = hipSuccess;
                for (int j = 0; j < c.members && e == hipSuccess; j += 2) {
                    WaveGemvArgs d = c;
                    d.members = std::min(2, c.members - j);
                    d.x = c.x + (size_t)j * a.K;
                    for (int i = 0; i < a.count; ++i) {
                        const int n = a.rows_end[i] - (i > 0 ? a.rows_end[i - 1] : 0);
                        d.y[i] = c.y[i] + (size_t)j * n;
                    }
                    e = launch_gemv_f32(value_type, d, cu_count, stream);
                }
            } else {
                e = launch_gemv_f32(value_type, c, cu_count, stream);
            }
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    if (a.arith != kArithFixed16) return hipErrorInvalidValue;
    // Measured on MI355X over the Qwen3-8B projections: the matrix cores win
    // from kMfmaMinMembers members (the wave GEMV's member-serial passes are
    // VALU-bound there), and from kMfmaMinMembersLongK where K spans several
    // slices (the wave GEMV then takes two members per launch).
    const bool wanted = a.members >= kMfmaMinMembers || (a.K > kSliceK && a.members >= kMfmaMinMembersLongK);
    const bool mfma = wanted && a.members <= kMfmaMaxMembers && a.x2 == nullptr && act_scratch != nullptr &&
                      gemv_mfma_supported(value_type) && a.K % 256 == 0 && a.K <= kWaveMaxK &&
                      (rows_tile_aligned(a) || !a.pair_swiglu);
    if (!mfma) {
        // the wave GEMV, in launch groups of as many members as it stages
        int per = std::min(wave_max_members(a.K), kWaveMaxMembers);
        if (a.x2 != nullptr) per = std::min(per, kSwigluMaxMembers);
        if (per <= 0) return hipErrorInvalidValue;
        for (int m0 = 0; m0 < a.members; m0 += per) {
            WaveGemvArgs c = a;
            c.members = std::min(per, a.members - m0);
            c.x = a.x + (size_t)m0 * a.K;
            c.x2 = a.x2 != nullptr ? a.x2 + (size_t)m0 * a.K : nullptr;
            for (int i = 0; i < a.count; ++i) {
                const int n = a.rows_end[i] - (i > 0 ? a.rows_end[i - 1] : 0);
                c.y[i] = a.y[i] + (size_t)m0 * (a.pair_swiglu ? a.rows_end[0] : n);
            }
            hipError_t e = launch_gemv_wave(value_type, c, cu_count, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    hipError_t e = launch_pack_act16(a.x, a.gamma, a.members, a.K, act_scratch, stream);
    if (e != hipSuccess) return e;
    MfmaGemvArgs m{};
    for (int i = 0; i < kMaxGroup; ++i) {
        m.w[i] = a.w[i];
        m.wbytes[i] = a.wbytes[i];
        m.y[i] = a.y[i];
        m.rows_end[i] = a.rows_end[i];
    }
    m.count = a.count;
    m.total_rows = a.total_rows;
    m.act = act_scratch;
    m.L = act16_layout(a.members, a.K);
    m.act_bytes = m.L.total;
    m.K = a.K;
    m.members = a.members;
    m.has_norm = a.gamma != nullptr ? 1 : 0;
    m.eps = a.eps;
    m.accumulate = a.accumulate;
    m.pair_swiglu = a.pair_swiglu;
    if (rows_tile_aligned(a)) return launch_gemv_mfma(value_type, m, cu_count, stream);
    // a group whose matrices do not end on whole tiles: one launch per matrix
    // over the shared packed activations, each as its single-matrix call
    for (int i = 0; i < a.count; ++i) {
        MfmaGemvArgs one = m;
        const int start = i > 0 ? a.rows_end[i - 1] : 0;
        one.w[0] = a.w[i];
        one.wbytes[0] = a.wbytes[i];
        one.y[0] = a.y[i];
        one.rows_end[0] = a.rows_end[i] - start;
        one.total_rows = one.rows_end[0];
        one.count = 1;
        e = launch_gemv_mfma(value_type, one, cu_count, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace ribn_amd

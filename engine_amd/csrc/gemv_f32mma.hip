// f32-faithful batched k-quant GEMV on the matrix cores (gfx950 /
// CDNA4, wave64): the default GEMV_WARP arithmetic for 9..64 members, with
// the weights read once for the whole batch (the reference's batch GEMV reads
// them once per launch of at most 8 members: q4_k.cu:161-258,
// quantized.rs:445-487). Up to 8 members the f32 wave GEMV stays in charge:
// its rows are bit-identical to the single-member call, as the reference
// qualifies its batch lane (cuda_reference.rs:5322-5334).
//
// Why this is f32 arithmetic (two forms, by weight type)
//  - Q4_K / Q5_K, f16 form. The quants times their six-bit group scale are
//    exact f16 values: q sc <= 31 * 63 = 1953 < 2^11, built per pair as
//    (1024 + q) sc - 1024 sc by one packed FMA with a single (exact)
//    rounding. Activations are scaled per (member, super-block) by a power
//    of two 2^e that puts the block's largest |x| in [2^14, 2^15), then split
//    into two f16 pieces, hi = f16(x 2^e) and lo = f16(x 2^e - hi): 22
//    significant bits for |x| down to 2^-29 of the block maximum.
//    v_mfma_f32_16x16x32_f16 multiplies exactly (11 x 11 bits) and
//    accumulates in f32, so one chain per piece runs through all 8 groups of
//    a super-block: S = sum (sc_g q_i) (x_i 2^e). The block epilogue adds
//    (d 2^-e) S per value, and the minimum term sum_g (dmin m_g) X_g (X_g the
//    f32 group sums of x) runs on v_mfma_f32_16x16x4_f32 ([member][group] x
//    [group][row]). Because each element carries its own scale, an MFMA step
//    may mix groups: lane quarter kq reads the row's 16-byte quant pieces at
//    16 kq and 64 + 16 kq (the four lanes of a row read 64 contiguous bytes
//    per load), and step c = 4L + 2h + r takes nibble h of bytes 8r .. + 7 of
//    its piece L; the pack writes the activations in that order.
//  - Q6_K, bf16 form. (q - 32) sc needs up to 12 bits, more than f16 holds
//    exactly, so the scale stays in an f32 epilogue per scale group. Each
//    f32 value x is split exactly into three bf16 pieces, x = hi + mid + lo:
//    hi keeps the top 8 significand bits (truncation), mid the top 8 of the
//    exact remainder, lo the remaining <= 8 bits. Quants enter as q - 32
//    (signed, exact). Three v_mfma_f32_16x16x32_bf16 per 32-element group
//    give S_g of each 16-element scale group (the B operand masked to each
//    half) for 16 members x 16 rows; the epilogue adds (d sc_g) S_g.
//  So the products are the dequantised weights times x, with f32 rounding in
//  the sums (and, in the f16 form, x rounded to 22 bits); the order differs
//  from the sequential f32 GEMV, so results agree with it to f32 rounding
//  (within 5e-5 normwise on wide-dynamic-range activations), not bit for bit.
//
// Layout (pack_f32mma_kernel, one launch per product)
//  - Member tile mt of 16, super-block b, MFMA step c, piece s: 64 lanes x
//    16 bytes in the MFMA A-operand order: lane l = member (l % 16) of the
//    tile and its 8 values of lane quarter l / 16 (bf16 form: elements
//    8 (l / 16) .. + 7 of group c; f16 form: the step order above).
//  - X sums (Q4_K / Q5_K minimum term): per (tile, block) 64 lanes x 2 f32,
//    lane mi + 16 q holding X of groups q and 4 + q of member mi (the A
//    operand of the two f32 MFMAs per block); f16 form: the 16 members'
//    2^-e per (tile, block).
//  - Per-member partial sums of x^2 per pack workgroup, for RMSNorm: the
//    product divides its outputs by rms(x) (the wave GEMV's factorisation
//    y = (W (x * gamma)) / rms).
//
// Product (f32mma_gemv_kernel)
//  - One launch serves up to four member tiles (64 members) in the f16 form
//    and two in the bf16 form; more members take further launches over the
//    same packed activations.
//  - A workgroup is W compute waves and one loader wave. The loader streams
//    each super-block's fragments, X sums and inverse block scales for all
//    member tiles straight into LDS (2-4 slots, 1-3 blocks ahead) and waits
//    only for its own loads before each barrier; the compute waves never wait
//    on a load at a barrier. Each compute wave owns one tile of 16 weight rows
//    (gate/up pairs: a gate tile and the up tile of the same rows) over the
//    workgroup's super-blocks and streams its weights through a register ring
//    2-4 blocks deep.
//  - Launch shape: the grid fills the CUs in one round (every workgroup
//    resident at once); among such shapes the one with the fewest (row tile x
//    super-block) units per workgroup wins. Row groups short of the CUs split
//    K across workgroups: raw row sums go to a partial buffer and
//    f32mma_reduce_kernel adds the splits in order (deterministic) and applies
//    the epilogue. The split depends on the weight shape alone.
//  - Lane l holds output row (l % 16) of each tile for members
//    4 (l / 16) .. + 3 of each member tile (the MFMA C layout).
// A member's output depends only on its own activations and the weight
// shape: its bits do not change with the other members' values, their count
// (from 9 members on) or its position in the batch.
#include "kquant_device.hpp"
#include "kquant_launch.hpp"

#include <float.h>

#include <algorithm>
#include <type_traits>

namespace ribn_amd {

namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr uint32_t kOOR = 0xffffff00u;  // buffer offset past any tensor: loads return 0, stores drop
constexpr int kPackBlocks = 2;          // super-blocks per pack workgroup (one wave)
constexpr uint32_t kPieceBytes = 64 * 16;                               // one piece of one group
constexpr uint32_t kXsumBlockBytes = 64 * 2 * 4;                        // per (member tile, block)
constexpr uint32_t kIscaleBlockBytes = 16 * 4;                          // per (member tile, block)
// Activation pieces per element: three bf16 for Q6_K, two f16 for Q4_K / Q5_K.
template <int T> constexpr int pieces_of() { return T == kQ6K ? 3 : 2; }

__device__ __forceinline__ uint32_t top16(float f) { return __builtin_bit_cast(uint32_t, f) & 0xffff0000u; }

// Two bf16 (the top halves of two f32 bit patterns) in one word, the first
// in the low half.
__device__ __forceinline__ uint32_t pack2(uint32_t lo_f32_bits, uint32_t hi_f32_bits) {
    return __builtin_amdgcn_perm(hi_f32_bits, lo_f32_bits, 0x07060302u);
}

struct PackArgs {
    const float* x;      // [members][K]
    const float* x2;     // SwiGLU: silu(x) * x2, or null
    const float* gamma;  // RMSNorm weight [K], or null
    uint8_t* act;
    F32MmaLayout L;
    int K;
    // a pending residual update of x (F32MmaFold): x += the splits' sums in
    // split order, stored back to x, before packing
    const float* fold_partial;
    int fold_splits;
};

template <int PIECES>
__global__ __launch_bounds__(64) void pack_f32mma_kernel(PackArgs a) {
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
        if (a.fold_splits > 0) {
            // y += g with g = ((0 + p_0) + p_1) + ... (f32mma_reduce_kernel's
            // sum and its unit RMSNorm factor), stored back as the residual
            float gs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            const size_t split_elems = (size_t)gridDim.y * a.K;
            for (int sp = 0; sp < a.fold_splits; ++sp) {
                const float* p = a.fold_partial + (size_t)sp * split_elems + e0;
                const float4 p0 = *reinterpret_cast<const float4*>(p);
                const float4 p1 = *reinterpret_cast<const float4*>(p + 4);
                const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
                for (int j = 0; j < 8; ++j) gs[j] += pv[j];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = v[j] + gs[j] * 1.0f;
            float* xw = const_cast<float*>(a.x) + e0;
            *reinterpret_cast<float4*>(xw) = make_float4(v[0], v[1], v[2], v[3]);
            *reinterpret_cast<float4*>(xw + 4) = make_float4(v[4], v[5], v[6], v[7]);
        }
        if (a.x2 != nullptr) {
            const float4 u0 = *reinterpret_cast<const float4*>(a.x2 + e0);
            const float4 u1 = *reinterpret_cast<const float4*>(a.x2 + e0 + 4);
            const float u[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
            // silu(gate) * up, in the reference's operation order (model_ops.rs:316-328)
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = (v[j] / (1.0f + expf(-v[j]))) * u[j];
        } else {
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
    }
    float xs = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) xs += v[j];
    xs += __shfl_xor(xs, 1, 64);
    xs += __shfl_xor(xs, 2, 64);  // X_g over the four 8-element chunks of group g
    const int mt = m >> 4, mi = m & 15;
    const uint32_t blk = (uint32_t)(mt * nb + b);
    // the bf16 form keeps group order (step g, lane quarter kq); the f16 form
    // puts elements 8 kq .. + 7 of group g at step 4 (g >> 2) + 2 (g & 1) +
    // (kq & 1), lane quarter 2 ((g >> 1) & 1) + (kq >> 1) (the product's
    // weight piece order)
    const uint32_t step = PIECES == 3 ? (uint32_t)g : (uint32_t)(4 * (g >> 2) + 2 * (g & 1) + (kq & 1));
    const uint32_t quarter = PIECES == 3 ? (uint32_t)kq : (uint32_t)(2 * ((g >> 1) & 1) + (kq >> 1));
    uint8_t* fr = a.act + a.L.frag + (blk * 8u + step) * PIECES * kPieceBytes + ((uint32_t)mi + 16u * quarter) * 16u;
    if constexpr (PIECES == 3) {
        // x = hi + mid + lo, each piece the top 16 bits of an f32 (a bf16)
        uint32_t hw[8], mw[8], lw[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            hw[j] = top16(v[j]);
            const float r1 = v[j] - __builtin_bit_cast(float, hw[j]);
            mw[j] = top16(r1);
            const float r2 = r1 - __builtin_bit_cast(float, mw[j]);
            lw[j] = top16(r2);  // r2 has at most 8 significant bits: exact
        }
        if (live) {
            const uint32_t* pieces[3] = {hw, mw, lw};
#pragma unroll
            for (int s = 0; s < 3; ++s) {
                const uint32_t* p = pieces[s];
                *reinterpret_cast<uint4*>(fr + s * kPieceBytes) =
                    make_uint4(pack2(p[0], p[1]), pack2(p[2], p[3]), pack2(p[4], p[5]), pack2(p[6], p[7]));
            }
        }
    } else {
        // The block's power-of-two scale 2^e puts its largest |x| in
        // [2^14, 2^15): then x 2^e = hi + lo with hi = f16(x 2^e) and
        // lo = f16(x 2^e - hi) (both RNE) keeps 22 significant bits of x
        // for |x| down to 2^-29 of the block maximum. The product applies
        // 2^-e per (member, block).
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(v[j]));
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        int ex = 0;
        if (mx > 0.f && mx <= FLT_MAX) (void)frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
        const int e = min(126, max(-126, 15 - ex));
        const float sc = __builtin_ldexpf(1.0f, e);
        uint32_t hp[4], lp[4];
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            const float x0 = v[j] * sc, x1 = v[j + 1] * sc;
            const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
            const _Float16 l0 = (_Float16)(x0 - (float)h0), l1 = (_Float16)(x1 - (float)h1);
            hp[j / 2] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            lp[j / 2] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
        }
        if (live) {
            *reinterpret_cast<uint4*>(fr) = make_uint4(hp[0], hp[1], hp[2], hp[3]);
            *reinterpret_cast<uint4*>(fr + kPieceBytes) = make_uint4(lp[0], lp[1], lp[2], lp[3]);
            if (c == 0) reinterpret_cast<float*>(a.act + a.L.iscale)[blk * 16u + (uint32_t)mi] = __builtin_ldexpf(1.0f, -e);
        }
    }
    if (live && kq == 0) {
        float* xsum = reinterpret_cast<float*>(a.act + a.L.xsum);
        xsum[(blk * 64u + (uint32_t)(mi + 16 * (g & 3))) * 2u + (uint32_t)(g >> 2)] = xs;
    }
    // this workgroup's share of sum(x^2), for RMSNorm (summed in part order by the product)
    const float ws = wave_sum(ssq);
    if (tid == 0) reinterpret_cast<float*>(a.act + a.L.ssq)[m * a.L.parts + blockIdx.x] = ws;
}

// Sum of p[0..n) in index order, its loads issued eight at a time (a plain
// loop waits for each load before the next add).
__device__ __forceinline__ float sum_in_order(const float* p, int n) {
    float total = 0.f;
    for (int base = 0; base < n; base += 8) {
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = base + j < n ? p[base + j] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (base + j < n) total += t[j];
        }
    }
    return total;
}

// ------------------------------------------------------------------ product

struct F32MmaArgs {
    const uint8_t* w[kMaxGroup];
    uint32_t wbytes[kMaxGroup];
    float* y[kMaxGroup];
    int rows_end[kMaxGroup];
    int count;
    int total_rows;
    const uint8_t* act;
    uint32_t act_bytes;
    F32MmaLayout L;
    int K;
    int members;   // of the whole call (output and activation extents)
    int member0;   // first member of this launch (a multiple of 16)
    int count_here;  // members of this launch (at most 16 * MT)
    int has_norm;
    float eps;
    int accumulate;
    int pair_swiglu;
    // K split across workgroups (blockIdx.y): each covers split_blocks
    // super-blocks and stores raw row sums to partial[split][member][vrow]
    // (vrow: the row in the launch's virtual row space; pairs: gate rows,
    // then up rows), which f32mma_reduce_kernel adds in split order
    float* partial;
    int splits;
    int split_blocks;
    int skip_reduce;  // the caller takes the split sums (F32MmaFold) instead of a reduce launch
};

template <int T> struct WRaw;
// Q4_K / Q5_K: the header and the lane's two 16-byte quant pieces, bytes
// 16 kq .. + 15 and 64 + 16 kq .. + 15 of the 128 (elements 16 (kq & 1) .. + 15
// of groups 2 (kq >> 1), + 1 and 4 + 2 (kq >> 1), + 1); Q5_K also the 16
// high-bit bytes of those elements.
template <> struct WRaw<kQ4K> { uint4 h, q0, q1; };
template <> struct WRaw<kQ5K> { uint4 h, qh, q0, q1; };
// Q6_K: the 16 int8 scales, d, and for each half n the 8 low-nibble bytes of
// both 32-byte quadrant pairs and the 8 qh bytes.
template <> struct WRaw<kQ6K> { uint4 sc; uint32_t d16; uint2 ql[4]; uint2 qh[2]; };

__device__ __forceinline__ uint2 load_b64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}

// One lane's bytes of a 16-row tile's super-block (row l % 16, elements
// 8 kq .. 8 kq + 7 of every group; crates/gguf/src/lib.rs:596-661 layouts).
template <int T>
__device__ __forceinline__ void load_w(WRaw<T>& d, __amdgpu_buffer_rsrc_t r, bool live, uint32_t base, int kq) {
    if constexpr (T == kQ6K) {
        // ql[128] at 0, qh[64] at 128, scales[16] at 192, d at 208
        d.sc = load_b128(r, live ? base + 192u : kOOR);
        d.d16 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, live ? (int)(base + 208u) : (int)kOOR, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) d.ql[i] = load_b64(r, live ? base + 32u * i + 8u * kq : kOOR);
#pragma unroll
        for (int n = 0; n < 2; ++n) d.qh[n] = load_b64(r, live ? base + 128u + 32u * n + 8u * kq : kOOR);
    } else {
        d.h = load_b128(r, live ? base : kOOR);
        // quants at 16 (Q4_K) or 48 (Q5_K, after the 32 high-bit bytes at 16)
        const uint32_t qs = T == kQ5K ? 48u : 16u;
        if constexpr (T == kQ5K) d.qh = load_b128(r, live ? base + 16u + 16u * (kq & 1) : kOOR);
        // the four lanes of a row read 64 contiguous bytes per load
        d.q0 = load_b128(r, live ? base + qs + 16u * kq : kOOR);
        d.q1 = load_b128(r, live ? base + qs + 64u + 16u * kq : kOOR);
    }
}

// Eight unsigned byte quants q < 128 (two words) as the eight bf16 values
// 128 + q, exactly: bf16 0x4300 is 128.0 with a 7-bit mantissa, so 0x43qq is
// 128 + q. One byte permute per two quants.
__device__ __forceinline__ v8bf bf16_128_plus(uint32_t w0, uint32_t w1) {
    // bytes of the result: q, 0x43 for each half (selector 0-3: w, 4: the constant)
    const uint32_t c = 0x43434343u;
    const uint4 b = make_uint4(__builtin_amdgcn_perm(c, w0, 0x04010400u), __builtin_amdgcn_perm(c, w0, 0x04030402u),
                               __builtin_amdgcn_perm(c, w1, 0x04010400u), __builtin_amdgcn_perm(c, w1, 0x04030402u));
    return __builtin_bit_cast(v8bf, b);
}

// Eight signed byte quants as eight bf16 (exact).
__device__ __forceinline__ v8bf bf16_of_sbytes(uint32_t w0, uint32_t w1) {
    uint32_t f[8];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        // signed byte t of each word (v_cvt_f32_i32 of the sign-extended byte)
        f[t] = __builtin_bit_cast(uint32_t, (float)(int)(int8_t)(w0 >> (8 * t)));
        f[4 + t] = __builtin_bit_cast(uint32_t, (float)(int)(int8_t)(w1 >> (8 * t)));
    }
    const uint4 b = make_uint4(pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7]));
    return __builtin_bit_cast(v8bf, b);
}

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));

// Eight unsigned byte quants q < 32 times the group scale sc (< 64) as f16,
// exactly: the byte permute makes 1024 + q (f16 0x6400 | q), and the packed
// FMA (1024 + q) * sc - 1024 sc rounds once, to the exact q * sc <= 1953.
__device__ __forceinline__ v8h f16_scaled_quants(uint32_t w0, uint32_t w1, h2v sc, h2v nsc) {
    const uint32_t c = 0x64646464u;
    const uint32_t p[4] = {__builtin_amdgcn_perm(c, w0, 0x04010400u), __builtin_amdgcn_perm(c, w0, 0x04030402u),
                           __builtin_amdgcn_perm(c, w1, 0x04010400u), __builtin_amdgcn_perm(c, w1, 0x04030402u)};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        o[k] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2v, p[k]), sc, nsc));
    return __builtin_bit_cast(v8h, make_uint4(o[0], o[1], o[2], o[3]));
}

// Q6_K quants of 32-element group g minus 32, as signed bytes (half n = g / 4,
// quadrant t = g % 4, elements 8 kq .. 8 kq + 7 of the quadrant; lib.rs:635-661):
// low (t < 2) or high nibble of ql[64 n + 32 (t & 1) + l] and bits 2t, 2t + 1 of
// qh[32 n + l]. x = q ^ 32 is q - 32 for q >= 32 and q + 32 otherwise, which
// setting bits 6-7 turns into q - 32.
__device__ __forceinline__ void q6_group(const WRaw<kQ6K>& d, int g, uint32_t& o0, uint32_t& o1) {
    const int n = g >> 2, t = g & 3;
    const uint2 lo = d.ql[2 * n + (t & 1)];
    const uint2 hi = d.qh[n];
    const int sl = (t >> 1) * 4, sh = 2 * t;
    const uint32_t w[2] = {lo.x, lo.y}, h2[2] = {hi.x, hi.y};
    uint32_t out[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t q = ((w[i] >> sl) & 0x0f0f0f0fu) | (((h2[i] >> sh) & 0x03030303u) << 4);
        const uint32_t x = q ^ 0x20202020u;
        out[i] = x | ((x & 0x20202020u) * 6u);
    }
    o0 = out[0];
    o1 = out[1];
}

// Compile-time loop: f(std::integral_constant<int, J>) for J in [I, N).
template <int I, int N> struct StaticFor {
    template <typename F> __device__ __forceinline__ static void run(F& f) {
        if constexpr (I < N) {
            f(std::integral_constant<int, I>{});
            StaticFor<I + 1, N>::run(f);
        }
    }
};

// s_waitcnt vmcnt(n) alone (gfx9 encoding: vmcnt in bits 3:0 and 15:14,
// expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt holds six bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// A workgroup barrier that neither waits for this wave's outstanding loads
// (the compiler's __syncthreads fence would) nor lets the compiler move
// memory accesses across it.
__device__ __forceinline__ void bare_barrier() { asm volatile("s_barrier" ::: "memory"); }
// The same after this wave's LDS reads have returned (the slot they read is
// refilled after the barrier).
__device__ __forceinline__ void lds_done_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One workgroup: W compute waves and one loader wave (the last). Compute wave
// w owns R tiles of 16 weight rows (gate/up pairs: a gate tile and the up
// tile of the same rows) over the workgroup's super-blocks [sb0, sb1) (a K
// split across workgroups when gridDim.y > 1) and streams their weights
// through an NS-block register ring. The loader wave streams every block's
// activation fragments, X sums and inverse block scales for the MT member
// tiles straight into NL LDS slots (NL - 1 blocks ahead), so no compute wave
// ever waits on a load at a barrier: block b's fragments are complete when
// the loader reaches barrier b, and the compute waves' weight loads run NS - 1
// blocks ahead, independent of the barriers.
template <int T, int R, int MT, bool PAIR, int NL, int NS>
__global__ __launch_bounds__(512) void f32mma_gemv_kernel(F32MmaArgs A) {
    constexpr int BB = BlockTraits<T>::bytes;
    constexpr int PC = pieces_of<T>();
    constexpr int FRAGS = MT * 8 * PC;  // 1 KB fragment loads per block
    constexpr int XS = T == kQ6K ? 0 : 2 * MT;  // 256 B X-sum loads per block
    constexpr int IS = T == kQ6K ? 0 : MT;      // inverse block scales (16 lanes x 4 B) per block
    constexpr int NDMA = FRAGS + XS + IS;       // the loader's loads per block
    static_assert(!PAIR || R % 2 == 0, "pairs split the tiles into gate and up halves");
    static_assert(NL >= 2 && NL <= 4 && NS % NL == 0, "the ring cycles through whole LDS slot rounds");
    static_assert((NL - 2) * NDMA < 64, "the loader's wait count fits vmcnt");
    // one object per slot: the compiler can then tell the slots apart
    __shared__ __attribute__((aligned(16))) uint4 fa0[FRAGS * 64];
    __shared__ __attribute__((aligned(16))) uint4 fa1[FRAGS * 64];
    __shared__ __attribute__((aligned(16))) uint4 fa2[NL > 2 ? FRAGS * 64 : 1];
    __shared__ __attribute__((aligned(16))) uint4 fa3[NL > 3 ? FRAGS * 64 : 1];
    __shared__ __attribute__((aligned(16))) float2 xa0[XS ? MT * 64 : 1];
    __shared__ __attribute__((aligned(16))) float2 xa1[XS ? MT * 64 : 1];
    __shared__ __attribute__((aligned(16))) float2 xa2[XS && NL > 2 ? MT * 64 : 1];
    __shared__ __attribute__((aligned(16))) float2 xa3[XS && NL > 3 ? MT * 64 : 1];
    __shared__ __attribute__((aligned(16))) float isa0[IS ? MT * 64 : 1];
    __shared__ __attribute__((aligned(16))) float isa1[IS ? MT * 64 : 1];
    __shared__ __attribute__((aligned(16))) float isa2[IS && NL > 2 ? MT * 64 : 1];
    __shared__ __attribute__((aligned(16))) float isa3[IS && NL > 3 ? MT * 64 : 1];
    auto fa_of = [&](auto slot_c) -> uint4* {
        constexpr int S = decltype(slot_c)::value;
        if constexpr (S == 0) return fa0;
        else if constexpr (S == 1) return fa1;
        else if constexpr (S == 2) return fa2;
        else return fa3;
    };
    auto xa_of = [&](auto slot_c) -> float2* {
        constexpr int S = decltype(slot_c)::value;
        if constexpr (S == 0) return xa0;
        else if constexpr (S == 1) return xa1;
        else if constexpr (S == 2) return xa2;
        else return xa3;
    };
    auto isa_of = [&](auto slot_c) -> float* {
        constexpr int S = decltype(slot_c)::value;
        if constexpr (S == 0) return isa0;
        else if constexpr (S == 1) return isa1;
        else if constexpr (S == 2) return isa2;
        else return isa3;
    };

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int W = __builtin_amdgcn_readfirstlane((int)(blockDim.x >> 6)) - 1;  // compute waves
    const int kq = lane >> 4, rl = lane & 15;
    const int nb = A.K >> 8;
    const uint32_t row_bytes = (uint32_t)nb * BB;
    const int sb0 = (int)blockIdx.y * A.split_blocks;
    const int sb1 = min(nb, sb0 + A.split_blocks);
    const int tile0 = A.member0 >> 4;

    if (wave == W) {
        // ---- loader: block b's fragments into LDS slot (b - sb0) % NL; past
        // the range the loads read zeros into a slot nobody reads
        const __amdgpu_buffer_rsrc_t ar = make_rsrc(A.act, A.act_bytes);
        auto stage = [&](auto slot_c, int b) {
            uint4* const fa = fa_of(slot_c);
            float2* const xa = xa_of(slot_c);
            float* const isa = isa_of(slot_c);
            const bool lb = b < sb1;
#pragma unroll
            for (int j = 0; j < FRAGS; ++j) {
                const int mt = j / (8 * PC);
                const uint32_t off = A.L.frag + ((uint32_t)((tile0 + mt) * nb + b) * (8u * PC) +
                                                 (uint32_t)(j % (8 * PC))) * kPieceBytes + (uint32_t)lane * 16u;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (__attribute__((address_space(3))) void*)&fa[j * 64], 16,
                                                         (int)(lb ? off : kOOR), 0, 0, 0);
            }
#pragma unroll
            for (int h = 0; h < XS; ++h) {
                const int mt = h >> 1;
                const uint32_t off = A.L.xsum + (uint32_t)((tile0 + mt) * nb + b) * kXsumBlockBytes +
                                     (uint32_t)(h & 1) * 256u + (uint32_t)lane * 4u;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ar, (__attribute__((address_space(3))) void*)(reinterpret_cast<float*>(xa) + h * 64), 4,
                    (int)(lb ? off : kOOR), 0, 0, 0);
            }
#pragma unroll
            for (int mt = 0; mt < IS; ++mt) {
                const uint32_t off =
                    A.L.iscale + (uint32_t)((tile0 + mt) * nb + b) * kIscaleBlockBytes + (uint32_t)lane * 4u;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ar, (__attribute__((address_space(3))) void*)(isa + mt * 64),
                                                         4, (int)(lb && lane < 16 ? off : kOOR), 0, 0, 0);
            }
        };
        auto prologue = [&](auto u) { stage(u, sb0 + decltype(u)::value); };
        StaticFor<0, NL - 1>::run(prologue);
        wait_vmcnt<(NL - 2) * NDMA>();  // block sb0's loads are in
        bare_barrier();
        int b = sb0;
        auto step = [&](auto uc) {
            constexpr int u = decltype(uc)::value;
            // the slot of block b + u - 1, which every compute wave finished
            // before the last barrier
            stage(std::integral_constant<int, (u + NL - 1) % NL>{}, b + u + NL - 1);
            wait_vmcnt<(NL - 2) * NDMA>();  // block b + u + 1's loads are in
            bare_barrier();
        };
        // whole ring rounds, then the last blocks (no loop back-edge after a
        // partial round, so no path skips a step and loops again)
        for (; b + NS <= sb1; b += NS) StaticFor<0, NS>::run(step);
        auto tail = [&](auto uc) {
            if (b + decltype(uc)::value < sb1) step(uc);
        };
        StaticFor<0, NS - 1>::run(tail);
        return;
    }

    // this wave's tiles: (matrix, first local row); tiles never straddle matrices
    __amdgpu_buffer_rsrc_t wr[R];
    int mat[R], local0[R], rows_mat[R], vrow0[R];
    bool live_row[R];
    uint32_t rowoff[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        if constexpr (PAIR) {
            mat[i] = i / (R / 2);
            local0[i] = (((int)blockIdx.x * W + wave) * (R / 2) + i % (R / 2)) * 16;
            rows_mat[i] = A.rows_end[0];
            vrow0[i] = (mat[i] ? A.rows_end[0] : 0) + local0[i];
        } else {
            const int row0 = (((int)blockIdx.x * W + wave) * R + i) * 16;
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
            vrow0[i] = row0;
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

    v4f acc[R][MT], macc[R][MT];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            acc[i][mt] = (v4f){0.f, 0.f, 0.f, 0.f};
            macc[i][mt] = (v4f){0.f, 0.f, 0.f, 0.f};
        }
    WRaw<T> ring[NS][R];
    auto fill_w = [&](auto ring_c, int b) {
        constexpr int s = decltype(ring_c)::value;
        const bool lb = b < sb1;
#pragma unroll
        for (int i = 0; i < R; ++i) load_w<T>(ring[s][i], wr[i], lb && live_row[i], rowoff[i] + (uint32_t)b * BB, kq);
    };

    // ---- one super-block from weight ring slot s and LDS slot (fa, xa, isa)
    auto block = [&](auto ring_c, auto slot_c) {
        constexpr int s = decltype(ring_c)::value;
        const uint4* const fa = fa_of(slot_c);
        const float2* const xa = xa_of(slot_c);
        float dd[R], bmin0[R], bmin1[R];
        uint32_t scw_lo[R], scw_hi[R];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            if constexpr (T == kQ6K) {
                dd[i] = half_bits_to_float(ring[s][i].d16 & 0xffffu);
            } else {
                const uint4 h = ring[s][i].h;
                dd[i] = half_bits_to_float(h.x & 0xffffu);
                const float dmn = half_bits_to_float(h.x >> 16);
                // six-bit scales / minima of the 8 groups, four per word (lib.rs:573-587)
                scw_lo[i] = h.y & 0x3f3f3f3fu;
                scw_hi[i] = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
                const uint32_t mnw_lo = h.z & 0x3f3f3f3fu;
                const uint32_t mnw_hi = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
                bmin0[i] = dmn * (float)((mnw_lo >> (8 * kq)) & 0xffu);
                bmin1[i] = dmn * (float)((mnw_hi >> (8 * kq)) & 0xffu);
            }
        }
        if constexpr (T != kQ6K) {
            // minimum term of groups kq and 4 + kq (the lane's k slot):
            // A = X [member][group], B = dmin m [group][row]
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const float2 xs = xa[mt * 64 + lane];
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    macc[i][mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(xs.x, bmin0[i], macc[i][mt], 0, 0, 0);
                    macc[i][mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(xs.y, bmin1[i], macc[i][mt], 0, 0, 0);
                }
            }
            // S = sum over the block of (sc_g q) (2^e x): one chain per
            // activation piece through the block's 8 MFMA steps, then
            // acc += (d 2^-e) S. Step c = 4L + 2h + r takes, in lane quarter
            // kq, nibble h of bytes 8r .. + 7 of the lane's piece L: elements
            // 16 (kq & 1) + 8r .. + 7 of group 4L + 2 (kq >> 1) + h. Each step
            // mixes four scale groups, every element carrying its own scale
            // (the packed activations follow the same order).
            const v4f zero = {0.f, 0.f, 0.f, 0.f};
            v4f ch[R][MT], cl[R][MT];
            h2v sc2[R][4], nsc2[R][4];
#pragma unroll
            for (int i = 0; i < R; ++i) {
#pragma unroll
                for (int lh = 0; lh < 4; ++lh) {
                    const uint32_t scw = (lh >> 1) ? scw_hi[i] : scw_lo[i];
                    const float scf = (float)((scw >> (8 * (2 * (kq >> 1) + (lh & 1)))) & 0xffu);
                    const _Float16 a = (_Float16)scf, na = (_Float16)(-1024.0f * scf);
                    sc2[i][lh] = h2v{a, a};
                    nsc2[i][lh] = h2v{na, na};
                }
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const int L = c >> 2, hn = (c >> 1) & 1, r = c & 1;
                v8h bq[R];
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    const uint4 qw = L ? ring[s][i].q1 : ring[s][i].q0;
                    const uint32_t w0 = r ? qw.z : qw.x, w1 = r ? qw.w : qw.y;
                    uint32_t q0 = (w0 >> (4 * hn)) & 0x0f0f0f0fu;
                    uint32_t q1 = (w1 >> (4 * hn)) & 0x0f0f0f0fu;
                    if constexpr (T == kQ5K) {
                        // fifth bit of element e of group g: bit g of qh[e]
                        const uint4 hw = ring[s][i].qh;
                        const uint32_t h0 = r ? hw.z : hw.x, h1 = r ? hw.w : hw.y;
                        const int gb = 4 * L + 2 * (kq >> 1) + hn;
                        q0 |= ((h0 >> gb) & 0x01010101u) << 4;
                        q1 |= ((h1 >> gb) & 0x01010101u) << 4;
                    }
                    bq[i] = f16_scaled_quants(q0, q1, sc2[i][2 * L + hn], nsc2[i][2 * L + hn]);
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int f = (mt * 8 + c) * PC;
                    const v8h a0 = __builtin_bit_cast(v8h, fa[(f + 0) * 64 + lane]);
                    const v8h a1 = __builtin_bit_cast(v8h, fa[(f + 1) * 64 + lane]);
#pragma unroll
                    for (int i = 0; i < R; ++i) {
                        ch[i][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bq[i], c ? ch[i][mt] : zero, 0, 0, 0);
                        cl[i][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bq[i], c ? cl[i][mt] : zero, 0, 0, 0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            const float* const isa = isa_of(slot_c);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const float4 inv4 = *reinterpret_cast<const float4*>(isa + mt * 64 + 4 * kq);
                const float inv[4] = {inv4.x, inv4.y, inv4.z, inv4.w};
#pragma unroll
                for (int i = 0; i < R; ++i)
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        acc[i][mt][t] = __builtin_fmaf(dd[i] * inv[t], ch[i][mt][t] + cl[i][mt][t], acc[i][mt][t]);
            }
        } else {
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                v8bf bq[R], bq1[R];
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    uint32_t q0, q1;
                    q6_group(ring[s][i], g, q0, q1);
                    // scale groups 2g (elements 0-15: lanes kq 0-1) and 2g + 1 (kq 2-3)
                    const bool low = kq < 2;
                    bq[i] = bf16_of_sbytes(low ? q0 : 0u, low ? q1 : 0u);
                    bq1[i] = bf16_of_sbytes(low ? 0u : q0, low ? 0u : q1);
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int f = (mt * 8 + g) * PC;
                    const v8bf a0 = __builtin_bit_cast(v8bf, fa[(f + 0) * 64 + lane]);
                    const v8bf a1 = __builtin_bit_cast(v8bf, fa[(f + 1) * 64 + lane]);
                    const v8bf a2 = __builtin_bit_cast(v8bf, fa[(f + 2) * 64 + lane]);
                    const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int i = 0; i < R; ++i) {
                        v4f c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bq[i], zero, 0, 0, 0);
                        v4f c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bq1[i], zero, 0, 0, 0);
                        c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bq[i], c0, 0, 0, 0);
                        c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bq1[i], c1, 0, 0, 0);
                        c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, bq[i], c0, 0, 0, 0);
                        c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, bq1[i], c1, 0, 0, 0);
                        // scale index 2g and 2g + 1: bytes 2g, 2g + 1 of the 16 int8 scales
                        const uint32_t scv[4] = {ring[s][i].sc.x, ring[s][i].sc.y, ring[s][i].sc.z, ring[s][i].sc.w};
                        const uint32_t sw = scv[g >> 1] >> (16 * (g & 1));
                        const float s0 = dd[i] * (float)(int8_t)(sw & 0xffu);
                        const float s1 = dd[i] * (float)(int8_t)((sw >> 8) & 0xffu);
#pragma unroll
                        for (int t = 0; t < 4; ++t)
                            acc[i][mt][t] = __builtin_fmaf(s1, c1[t], __builtin_fmaf(s0, c0[t], acc[i][mt][t]));
                    }
                }
                // one group's conversions and MFMA chains at a time (bounds the
                // registers live across groups)
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    // ---- prologue: weights of the first NS - 1 blocks
    auto prologue = [&](auto u) { fill_w(u, sb0 + decltype(u)::value); };
    StaticFor<0, NS - 1>::run(prologue);
    bare_barrier();  // the loader has block sb0's fragments in slot 0
    int b = sb0;
    auto step = [&](auto uc) {
        constexpr int u = decltype(uc)::value;
        // refill the ring slot of block b + u - 1 with block b + u + NS - 1
        fill_w(std::integral_constant<int, (u + NS - 1) % NS>{}, b + u + NS - 1);
        block(uc, std::integral_constant<int, u % NL>{});
        lds_done_barrier();  // slot u % NL may be refilled from here on
    };
    for (; b + NS <= sb1; b += NS) StaticFor<0, NS>::run(step);
    auto tail = [&](auto uc) {
        if (b + decltype(uc)::value < sb1) step(uc);
    };
    StaticFor<0, NS - 1>::run(tail);

    // ---- epilogue: each wave owns its rows over the whole range
    float v[R][MT][4];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int t = 0; t < 4; ++t) v[i][mt][t] = acc[i][mt][t] - macc[i][mt][t];
    if (A.splits > 1) {
        // raw row sums of this split ([split][member of the launch][vrow]);
        // the reduce launch finishes them
        const int vrows = PAIR ? 2 * A.rows_end[0] : A.total_rows;
        const __amdgpu_buffer_rsrc_t pr =
            make_rsrc(A.partial, (uint32_t)A.splits * (uint32_t)A.count_here * (uint32_t)vrows * 4u);
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int ml = 16 * mt + 4 * kq + t;  // member within the launch
                    const bool ok = live_row[i] && ml < A.count_here;
                    const uint32_t off =
                        ok ? (uint32_t)(((int)blockIdx.y * A.count_here + ml) * vrows + vrow0[i] + rl) * 4u : kOOR;
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v[i][mt][t]), pr, (int)off, 0, 0);
                }
        return;
    }
    float inv[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            inv[mt][t] = 1.f;
            const int mem = A.member0 + 16 * mt + 4 * kq + t;
            if (A.has_norm && mem < A.members) {
                const float* ssq = reinterpret_cast<const float*>(A.act + A.L.ssq);
                const float total = sum_in_order(ssq + mem * A.L.parts, A.L.parts);
                // RMSNorm (qwen_reference.rs:550-556): 1/sqrt(sum(x^2)/K + eps)
                inv[mt][t] = 1.0f / sqrtf(total / (float)A.K + A.eps);
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
        for (int i = 0; i < R / 2; ++i)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int mem = A.member0 + 16 * mt + 4 * kq + t;
                    const float gt = v[i][mt][t] * inv[mt][t];
                    const float up = v[i + R / 2][mt][t] * inv[mt][t];
                    // silu(gate) * up, in the reference's operation order (model_ops.rs:316-328)
                    const float out = (gt / (1.0f + expf(-gt))) * up;
                    const bool ok = live_row[i] && mem < A.members && 16 * mt + 4 * kq + t < A.count_here;
                    put(out, yr, ok ? (uint32_t)(mem * ffn + local0[i] + rl) * 4u : kOOR);
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
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int mem = A.member0 + 16 * mt + 4 * kq + t;
                    const bool ok = live_row[i] && mem < A.members && 16 * mt + 4 * kq + t < A.count_here;
                    put(v[i][mt][t] * inv[mt][t], yr, ok ? (uint32_t)(mem * rows_mat[i] + local0[i] + rl) * 4u : kOOR);
                }
        }
    }
}

// Adds the splits' raw row sums in split order and applies the epilogue of
// the one-split form (RMSNorm factor, SwiGLU pair, residual accumulate). One
// thread per (member, output row).
__global__ __launch_bounds__(256) void f32mma_reduce_kernel(F32MmaArgs A) {
    const int pair = A.pair_swiglu;
    const int rows = pair ? A.rows_end[0] : A.total_rows;
    const int vrows = pair ? 2 * rows : A.total_rows;
    const int idx = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (idx >= A.count_here * rows) return;
    const int ml = idx / rows, row = idx - ml * rows;  // member within the launch
    const int mem = A.member0 + ml;
    // the splits' sums in split order (at most 16 splits: every load issued
    // before the first add)
    float gv[16], uv[16];
#pragma unroll
    for (int sp = 0; sp < 16; ++sp) {
        const float* p = A.partial + ((size_t)sp * A.count_here + ml) * vrows;
        gv[sp] = sp < A.splits ? p[row] : 0.f;
        uv[sp] = sp < A.splits && pair ? p[rows + row] : 0.f;
    }
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int sp = 0; sp < 16; ++sp) {
        if (sp < A.splits) {
            g += gv[sp];
            u += uv[sp];
        }
    }
    float inv = 1.f;
    if (A.has_norm) {
        const float* ssq = reinterpret_cast<const float*>(A.act + A.L.ssq);
        const float total = sum_in_order(ssq + mem * A.L.parts, A.L.parts);
        // RMSNorm (qwen_reference.rs:550-556): 1/sqrt(sum(x^2)/K + eps)
        inv = 1.0f / sqrtf(total / (float)A.K + A.eps);
    }
    float* y;
    int local, rows_mat;
    float out;
    if (pair) {
        const float gt = g * inv, up = u * inv;
        // silu(gate) * up, in the reference's operation order (model_ops.rs:316-328)
        out = (gt / (1.0f + expf(-gt))) * up;
        y = A.y[0];
        local = row;
        rows_mat = rows;
    } else {
        int mm = 0, start = 0;
        for (int j = 0; j + 1 < A.count; ++j) {
            if (row >= A.rows_end[j]) {
                mm = j + 1;
                start = A.rows_end[j];
            }
        }
        y = A.y[mm];
        local = row - start;
        rows_mat = A.rows_end[mm] - start;
        out = g * inv;
    }
    float* dst = y + (size_t)mem * rows_mat + local;
    if (A.accumulate) {
        *dst += out;  // one thread per output: a plain read-modify-write
    } else {
        *dst = out;
    }
}

// Member tiles per launch: the f16 form's fragments of a block (16 KB per
// tile) let four tiles (64 members) share one weight stream; the bf16 form's
// (24 KB per tile) two.
template <int T> constexpr int max_tiles() { return T == kQ6K ? 2 : 4; }
// LDS slots (fragment look-ahead + 1): as many as 160 KB of LDS holds, at
// most four, and few enough that the loader's in-flight loads fit its
// six-bit vmcnt wait.
template <int T, int MT> constexpr int lds_slots() {
    return T == kQ6K ? (MT == 1 ? 4 : 3) : (MT == 1 ? 4 : MT <= 3 ? 3 : 2);
}
// Weight ring depth: the LDS slot count, or four blocks beside two slots
// when the ring's registers leave room (one row tile per wave). Measured on
// MI355X at the Qwen3-8B FFN shapes, an eight-block ring at one member tile
// ran M = 16 slower (49.8 against 46-47 us per FFN).
template <int T, int R, int MT> constexpr int ring_depth() {
    constexpr int nl = lds_slots<T, MT>();
    return nl == 2 ? (R == 1 ? 4 : 2) : nl;
}
// Launch shape of one product: compute waves per workgroup, the K split and
// the row groups. The split comes from the weight shape alone (row tiles,
// super-blocks and the partial room a 64-member launch needs), never from the
// member count, so a member's sums are added in the same order whatever the
// batch: among the one-tile-per-wave shapes whose grid fits the CUs in one
// round (all workgroups resident at once), the one with the fewest (row tile
// x super-block) units per workgroup sets it (ties: more compute waves, which
// share the LDS fragments, then fewer splits). Measured on MI355X at the
// Qwen3-8B FFN shapes, two row tiles per wave (halving the LDS fragment
// reads) ran M = 64 slower: 96.0 against 80.3 us per FFN.
struct F32MmaShape {
    int waves, splits, split_blocks, groups;
};
constexpr int kF32MmaMaxComputeWaves = 7;  // plus the loader: eight waves, two per SIMD
F32MmaShape f32mma_split(int tiles, int nb, int max_splits, int cu_count) {
    constexpr int kMaxWaves = kF32MmaMaxComputeWaves;
    F32MmaShape best{kMaxWaves, 1, nb, (tiles + kMaxWaves - 1) / kMaxWaves};
    long best_cost = -1;
    for (int s = 1; s <= std::min(nb, std::max(1, max_splits)); ++s) {
        const int sbk = (nb + s - 1) / s;
        if ((nb + sbk - 1) / sbk != s) continue;  // the same split as a smaller s
        for (int w = 1; w <= kMaxWaves; ++w) {
            const int groups = (tiles + w - 1) / w;
            if ((long)groups * s > cu_count) continue;
            const long cost = (long)w * sbk;
            const bool better = best_cost < 0 || cost < best_cost ||
                                (cost == best_cost && (w > best.waves || (w == best.waves && s < best.splits)));
            if (better) {
                best = {w, s, sbk, groups};
                best_cost = cost;
            }
        }
    }
    return best;
}
// The same split with R row tiles per wave (gate/up pairs: 2): the fewest
// compute waves that still fit the grid in one round.
F32MmaShape f32mma_shape_r(const F32MmaShape& one, int tiles, int R, int cu_count) {
    const int units = (tiles + R - 1) / R;
    const int max_groups = std::max(1, cu_count / one.splits);
    const int w = std::min(kF32MmaMaxComputeWaves, std::max(1, (units + max_groups - 1) / max_groups));
    return {w, one.splits, one.split_blocks, (units + w - 1) / w};
}

template <int T, int R, int MT, bool PAIR>
hipError_t launch_shape(F32MmaArgs a, const F32MmaShape& sh, hipStream_t stream) {
    a.splits = sh.splits;
    a.split_blocks = sh.split_blocks;
    hipLaunchKernelGGL((f32mma_gemv_kernel<T, R, MT, PAIR, lds_slots<T, MT>(), ring_depth<T, R, MT>()>),
                       dim3((unsigned)sh.groups, (unsigned)sh.splits), dim3(64 * (sh.waves + 1)), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.splits == 1 || a.skip_reduce) return e;
    const int rows = a.pair_swiglu ? a.rows_end[0] : a.total_rows;
    const int threads = a.count_here * rows;
    hipLaunchKernelGGL(f32mma_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

template <int T, int MT>
hipError_t launch_mt(const F32MmaArgs& a, const F32MmaShape& one, int tiles, int cu_count, hipStream_t stream) {
    if (a.pair_swiglu) return launch_shape<T, 2, MT, true>(a, f32mma_shape_r(one, tiles, 2, cu_count), stream);
    return launch_shape<T, 1, MT, false>(a, one, stream);
}

template <int T>
hipError_t launch_t(const F32MmaArgs& a, size_t partial_bytes, int cu_count, F32MmaFold* defer, hipStream_t stream) {
    constexpr int kStep = 16 * max_tiles<T>();
    const int nb = a.K >> 8;
    const bool pair = a.pair_swiglu != 0;
    const int tiles = pair ? 2 * ((a.rows_end[0] + 15) / 16) : (a.total_rows + 15) / 16;
    const int vrows = pair ? 2 * a.rows_end[0] : a.total_rows;
    const size_t split_bytes = (size_t)kStep * (size_t)vrows * 4;
    const int max_splits = a.partial == nullptr ? 1 : (int)std::min<size_t>(16, partial_bytes / split_bytes);
    const F32MmaShape one = f32mma_split(tiles, nb, max_splits, cu_count);
    // an accumulating single-weight product of one launch may leave its split
    // sums to the next call (F32MmaFold)
    const bool deferred = defer != nullptr && one.splits > 1 && a.accumulate && !pair && a.count == 1 &&
                          !a.has_norm && a.members <= kStep;
    if (defer != nullptr) {
        *defer = F32MmaFold{};
        if (deferred) *defer = F32MmaFold{a.y[0], a.partial, one.splits, a.members, a.total_rows};
    }
    for (int m0 = 0; m0 < a.members; m0 += kStep) {
        F32MmaArgs c = a;
        c.skip_reduce = deferred ? 1 : 0;
        c.member0 = m0;
        c.count_here = std::min(kStep, a.members - m0);
        const int mts = (c.count_here + 15) / 16;
        hipError_t e;
        if constexpr (max_tiles<T>() == 4) {
            e = mts == 1   ? launch_mt<T, 1>(c, one, tiles, cu_count, stream)
                : mts == 2 ? launch_mt<T, 2>(c, one, tiles, cu_count, stream)
                : mts == 3 ? launch_mt<T, 3>(c, one, tiles, cu_count, stream)
                           : launch_mt<T, 4>(c, one, tiles, cu_count, stream);
        } else {
            e = mts == 1 ? launch_mt<T, 1>(c, one, tiles, cu_count, stream)
                         : launch_mt<T, 2>(c, one, tiles, cu_count, stream);
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

bool rows_tile_aligned(const WaveGemvArgs& a) {
    if (a.pair_swiglu) return a.count == 2 && a.rows_end[1] == 2 * a.rows_end[0] && a.rows_end[0] % 16 == 0;
    for (int i = 0; i + 1 < a.count; ++i) {
        if (a.rows_end[i] % 16 != 0) return false;
    }
    return true;
}

}  // namespace

namespace {

// y[m][r] += ((0 + p_0) + p_1) + ... (a pending F32MmaFold finished on its own:
// f32mma_reduce_kernel's sum and unit factor). One thread per element.
__global__ __launch_bounds__(256) void f32mma_fold_flush_kernel(F32MmaFold f) {
    const int idx = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (idx >= f.members * f.rows) return;
    float g = 0.f;
    for (int sp = 0; sp < f.splits; ++sp) g += f.partial[(size_t)sp * f.members * f.rows + idx];
    f.y[idx] += g * 1.0f;
}

}  // namespace

hipError_t launch_f32mma_fold_flush(F32MmaFold* f, hipStream_t stream) {
    if (f == nullptr || f->splits <= 0) return hipSuccess;
    const int n = f->members * f->rows;
    hipLaunchKernelGGL(f32mma_fold_flush_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, *f);
    *f = F32MmaFold{};
    return hipGetLastError();
}

F32MmaLayout f32mma_layout(int members, int K, int pieces) {
    F32MmaLayout L{};
    const int nb = K / 256;
    L.nb = nb;
    L.tiles = (members + 15) / 16;
    L.parts = (nb + kPackBlocks - 1) / kPackBlocks;
    const uint32_t blocks = (uint32_t)L.tiles * (uint32_t)nb;
    L.frag = 0;
    L.xsum = L.frag + blocks * 8u * (uint32_t)pieces * kPieceBytes;
    L.iscale = L.xsum + blocks * kXsumBlockBytes;
    L.ssq = L.iscale + blocks * kIscaleBlockBytes;
    L.total = L.ssq + (uint32_t)members * (uint32_t)L.parts * 4u;
    return L;
}

bool f32mma_supported(int value_type, const WaveGemvArgs& a) {
    return (value_type == kQ4K || value_type == kQ5K || value_type == kQ6K) && a.members >= kF32MmaMinMembers &&
           a.members <= kF32MmaMaxMembers && a.K >= 256 && a.K % 256 == 0 && a.K <= kWaveMaxK &&
           (a.pair_swiglu == 0 || rows_tile_aligned(a)) && !(a.gamma != nullptr && a.x2 != nullptr);
}

hipError_t launch_gemv_f32mma(int value_type, const WaveGemvArgs& a, void* scratch, size_t scratch_bytes,
                              int cu_count, hipStream_t stream) {
    if (!f32mma_supported(value_type, a) || scratch == nullptr || a.count < 1 || a.count > kMaxGroup) {
        return hipErrorInvalidValue;
    }
    const int pieces = value_type == kQ6K ? 3 : 2;
    const F32MmaLayout L = f32mma_layout(a.members, a.K, pieces);
    if (L.total > scratch_bytes) return hipErrorInvalidValue;
    PackArgs p{};
    p.x = a.x;
    p.x2 = a.x2;
    p.gamma = a.gamma;
    p.act = static_cast<uint8_t*>(scratch);
    p.L = L;
    p.K = a.K;
    if (a.fold != nullptr && a.fold->splits > 0) {
        // the pending update must be of exactly this input
        if (a.fold->y != a.x || a.fold->members != a.members || a.fold->rows != a.K || a.x2 != nullptr) {
            return hipErrorInvalidValue;
        }
        p.fold_partial = a.fold->partial;
        p.fold_splits = a.fold->splits;
    }
    if (pieces == 3) {
        hipLaunchKernelGGL(pack_f32mma_kernel<3>, dim3((unsigned)L.parts, (unsigned)a.members), dim3(64), 0, stream, p);
    } else {
        hipLaunchKernelGGL(pack_f32mma_kernel<2>, dim3((unsigned)L.parts, (unsigned)a.members), dim3(64), 0, stream, p);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    F32MmaArgs m{};
    for (int i = 0; i < kMaxGroup; ++i) {
        m.w[i] = a.w[i];
        m.wbytes[i] = a.wbytes[i];
        m.y[i] = a.y[i];
        m.rows_end[i] = a.rows_end[i];
    }
    m.count = a.count;
    m.total_rows = a.total_rows;
    m.act = static_cast<const uint8_t*>(scratch);
    m.act_bytes = L.total;
    m.L = L;
    m.K = a.K;
    m.members = a.members;
    m.has_norm = a.gamma != nullptr ? 1 : 0;
    m.eps = a.eps;
    m.accumulate = a.accumulate;
    m.pair_swiglu = a.pair_swiglu;
    // split-K partials follow the packed activations in the scratch
    const size_t part_off = ((size_t)L.total + 255) / 256 * 256;
    m.partial = part_off < scratch_bytes ? reinterpret_cast<float*>(static_cast<uint8_t*>(scratch) + part_off) : nullptr;
    const size_t part_bytes = part_off < scratch_bytes ? scratch_bytes - part_off : 0;
    m.splits = 1;
    m.split_blocks = a.K >> 8;
    auto run = [&](const F32MmaArgs& args, F32MmaFold* defer) -> hipError_t {
        switch (value_type) {
        case kQ4K: return launch_t<kQ4K>(args, part_bytes, cu_count, defer, stream);
        case kQ5K: return launch_t<kQ5K>(args, part_bytes, cu_count, defer, stream);
        case kQ6K: return launch_t<kQ6K>(args, part_bytes, cu_count, defer, stream);
        default: return hipErrorInvalidValue;
        }
    };
    if (rows_tile_aligned(a)) return run(m, a.count == 1 ? a.defer : nullptr);
    if (a.defer != nullptr) *a.defer = F32MmaFold{};
    // a group whose matrices do not end on whole tiles: one launch per matrix
    // over the shared packed activations, each as its single-matrix call
    for (int i = 0; i < a.count; ++i) {
        F32MmaArgs one = m;
        const int start = i > 0 ? a.rows_end[i - 1] : 0;
        one.w[0] = a.w[i];
        one.wbytes[0] = a.wbytes[i];
        one.y[0] = a.y[i];
        one.rows_end[0] = a.rows_end[i] - start;
        one.total_rows = one.rows_end[0];
        one.count = 1;
        e = run(one, nullptr);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace ribn_amd

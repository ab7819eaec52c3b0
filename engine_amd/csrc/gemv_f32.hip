// Wave GEMV for Q4_K / Q5_K / Q6_K with f32 activations on gfx950 (CDNA4,
// wave64): the default decode projection, the arithmetic of the reference's
// warp kernels (crates/nvidia/src/kernels/quantized/q4_k.cu:103-159,
// q5_k.cu:37-98, q6_k.cu:45-109): f32 activations against weights dequantised
// in registers, f32 accumulation. Optional fused RMSNorm or SwiGLU prologue,
// grouped weights sharing one input (q/k/v, gate/up) and gate/up pairs with a
// SwiGLU epilogue, as in gemv_wave.hip.
//
// Mapping: the wave / lane layout of wave_rows.hpp (a lane owns 64 weights of
// one super-block per unit of row x slice).
//
// Activations
//  - Each workgroup stages x (times gamma, or silu(x) * x2) once, in f32, into
//    LDS "lane records": the 64 activations a lane multiplies, in the order it
//    uses them, then the f32 sum X_g of each of its scale groups. A record is
//    68 dwords (17 x 16 bytes, odd), so 16 lanes' 128-bit reads hit distinct
//    banks. One member's slice is 17 KB.
//  - One member: a lane keeps its record in VGPRs (64 floats) for every row it
//    reduces. Several members: the records stay in LDS and a pass of the
//    weight ring reads each 4-element piece once per member for all its rows.
//
// Arithmetic of one lane and one unit, per scale group g (32 elements for
// Q4_K / Q5_K, 16 for Q6_K; crates/gguf/src/lib.rs:596-661):
//      S_g  = sum_i q_i * x_i          (f32 FMAs, element order)
//      Q4_K / Q5_K:  part += (d*sc_g) * S_g - (dmin*m_g) * X_g
//      Q6_K:         part += (d*sc_g) * (S_g - 32 X_g)
//  which is sum_i ((d*sc_g)*q_i - dmin*m_g) * x_i (respectively (q_i - 32)) with
//  the same products: the dequantised weight times x, regrouped per scale
//  group. Every quantity is f32; nothing is rounded to a narrower format.
//
// Canonical order of a row (every launch shape and member count follows it,
// so a member's output bits never depend on the batch it runs in):
//   P_s = DPP/readlane wave sum of the lanes' parts of slice s (fixed tree),
//   T   = ((P_0 + P_1) + P_2) ... in slice order,
//   y   = T * inv with inv = 1/sqrt(sum(x^2)/K + eps) for RMSNorm (else y = T),
//   sum(x^2) = per 256-element block, a fixed lane tree; blocks added in order.
#include "wave_rows.hpp"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace ribn_amd {

namespace {

template <int T> struct F32Rec {
    static constexpr int group = (T == kQ6K) ? 16 : 32;  // elements per scale group
    static constexpr int groups = 64 / group;            // scale groups per lane
    static constexpr int stride = 68;                    // dwords per lane record
};

constexpr int kF32Blocks = kWaveMaxK / 256;  // super-blocks of the largest K staged

// Lane record and position of element e (a multiple of 4, within one slice).
template <int T>
__device__ __forceinline__ void f32_slot(int e, int& rec, int& pos) {
    if constexpr (T == kQ6K) {
        const int bs = e >> 8, c = (e >> 7) & 1, v = (e >> 5) & 3, s = (e >> 4) & 1;
        rec = 4 * bs + 2 * c + s;
        pos = 16 * v + (e & 15);
    } else {
        rec = e >> 6;
        pos = e & 63;
    }
}

// Sum over the consecutive lanes holding one scale group (8 or 4 lanes of 4
// elements); every lane of the group receives the same value.
template <int T>
__device__ __forceinline__ float group_sum_f(float v) {
    v = dpp_step<0xb1>(v);  // quad_perm [1,0,3,2]
    v = dpp_step<0x4e>(v);  // quad_perm [2,3,0,1]
    if constexpr (F32Rec<T>::group == 32) v = dpp_step<0x141>(v);  // row_half_mirror
    return v;
}

__device__ __forceinline__ float byte_f(uint32_t w, int t) { return (float)((w >> (8 * t)) & 0xffu); }

// The value passes through an empty asm statement, so the compiler no longer
// knows its bits: byte_f of a masked word then stays one v_cvt_f32_ubyte{t}
// instead of a bit-field extract plus a convert.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm("" : "+v"(v));
    return v;
}
// As opaque(), but volatile: ordered after the previous volatile statements,
// so nothing computed from the value is hoisted above them (bounds the
// registers of the many-member passes).
__device__ __forceinline__ uint32_t pinned(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// --------------------------------------------------------- lane dot product
//
// part[r][m] = this lane's share of row r . x_m for one unit. xf(m, i) returns
// the i-th float4 of member m's lane record, sf(m, g) its group sum X_g. Each
// (r, m) pair sees the same operation sequence whatever NR and MT are.
template <int T, int NR, int MT, class XF, class SF>
__device__ __forceinline__ void rows_dot(const RowData<T> (&d)[NR], int p, XF xf, SF sf, float (&part)[NR][MT]) {
    if constexpr (T == kQ4K || T == kQ5K) {
        float a0[NR], a1[NR], b0[NR], b1[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const uint4 h = d[r].h;
            const float dd = half_bits_to_float(h.x & 0xffffu);
            const float dmin = half_bits_to_float(h.x >> 16);
            // six-bit scales / minima of all 8 groups, four per word (lib.rs:573-587)
            const uint32_t lo_sc = h.y & 0x3f3f3f3fu;
            const uint32_t lo_mn = h.z & 0x3f3f3f3fu;
            const uint32_t hi_sc = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
            const uint32_t hi_mn = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
            const uint32_t scw = (p < 2) ? lo_sc : hi_sc;
            const uint32_t mnw = (p < 2) ? lo_mn : hi_mn;
            const int sh = (p & 1) * 16;
            // Q4_K quants enter as q * 2^-9 (see below): scales carry the 2^9, exactly
            constexpr float kQScale = (T == kQ4K) ? 512.0f : 1.0f;
            a0[r] = (dd * (float)((scw >> sh) & 0xffu)) * kQScale;
            a1[r] = (dd * (float)((scw >> (sh + 8)) & 0xffu)) * kQScale;
            b0[r] = dmin * (float)((mnw >> sh) & 0xffu);
            b1[r] = dmin * (float)((mnw >> (sh + 8)) & 0xffu);
        }
        float sA[NR][MT], sB[NR][MT];
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m) sA[r][m] = sB[r][m] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // group A = 2p (low nibbles), group B = 2p+1 (high nibbles), 5th bit for Q5_K
            float fa[NR][4], fb[NR][4];
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const uint32_t qw[8] = {d[r].qa.x, d[r].qa.y, d[r].qa.z, d[r].qa.w,
                                        d[r].qb.x, d[r].qb.y, d[r].qb.z, d[r].qb.w};
                const uint32_t w = (NR * MT > 2) ? pinned(qw[j]) : qw[j];
                uint32_t qa = w & 0x0f0f0f0fu;
                uint32_t qb = (w >> 4) & 0x0f0f0f0fu;
                if constexpr (T == kQ5K) {
                    const uint32_t hw[8] = {d[r].ha.x, d[r].ha.y, d[r].ha.z, d[r].ha.w,
                                            d[r].hb.x, d[r].hb.y, d[r].hb.z, d[r].hb.w};
                    qa |= ((hw[j] >> (2 * p)) & 0x01010101u) << 4;
                    qb |= ((hw[j] >> (2 * p + 1)) & 0x01010101u) << 4;
                }
                if constexpr (T == kQ4K) {
                    // Bytes 0..15 read as OCP E4M3 are exactly q * 2^-9: two
                    // quants per convert (the 2^9 is folded into the scales).
                    const auto a01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)qa, false);
                    const auto a23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)qa, true);
                    const auto b01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)qb, false);
                    const auto b23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)qb, true);
                    fa[r][0] = a01[0];
                    fa[r][1] = a01[1];
                    fa[r][2] = a23[0];
                    fa[r][3] = a23[1];
                    fb[r][0] = b01[0];
                    fb[r][1] = b01[1];
                    fb[r][2] = b23[0];
                    fb[r][3] = b23[1];
                } else {
                    qa = opaque(qa);
                    qb = opaque(qb);
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        fa[r][t] = byte_f(qa, t);
                        fb[r][t] = byte_f(qb, t);
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float4 xa = xf(m, j);
                const float4 xb = xf(m, 8 + j);
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    sA[r][m] = __builtin_fmaf(fa[r][0], xa.x, sA[r][m]);
                    sA[r][m] = __builtin_fmaf(fa[r][1], xa.y, sA[r][m]);
                    sA[r][m] = __builtin_fmaf(fa[r][2], xa.z, sA[r][m]);
                    sA[r][m] = __builtin_fmaf(fa[r][3], xa.w, sA[r][m]);
                    sB[r][m] = __builtin_fmaf(fb[r][0], xb.x, sB[r][m]);
                    sB[r][m] = __builtin_fmaf(fb[r][1], xb.y, sB[r][m]);
                    sB[r][m] = __builtin_fmaf(fb[r][2], xb.z, sB[r][m]);
                    sB[r][m] = __builtin_fmaf(fb[r][3], xb.w, sB[r][m]);
                }
                // Many accumulators: an empty volatile statement on them after
                // each member keeps the FMAs next to the reads they consume.
                if constexpr (NR * MT > 2) {
#pragma unroll
                    for (int r = 0; r < NR; ++r) asm volatile("" : "+v"(sA[r][m]), "+v"(sB[r][m]));
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float xA = sf(m, 0), xB = sf(m, 1);
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const float tA = __builtin_fmaf(a0[r], sA[r][m], -(b0[r] * xA));
                const float tB = __builtin_fmaf(a1[r], sB[r][m], -(b1[r] * xB));
                part[r][m] = tA + tB;
            }
        }
    } else {
        const int c = p >> 1, s = p & 1;
        float a[NR][4];
        uint32_t law[NR][4], lbw[NR][4], qhw[NR][4];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const uint32_t sh = d[r].shift;
            const uint4 la = funnel(d[r].la, d[r].la_t, sh);
            const uint4 lb = funnel(d[r].lb, d[r].lb_t, sh);
            const uint4 qh = funnel(d[r].qh, d[r].qh_t, sh);
            const uint4 sc = funnel(d[r].sc, d[r].sc_t, sh);  // int8 scales
            const float dd = half_bits_to_float(d[r].d16);
            const uint32_t w0 = c ? sc.z : sc.x;  // scales 8c+0..8c+3
            const uint32_t w1 = c ? sc.w : sc.y;  // scales 8c+4..8c+7
            a[r][0] = dd * (float)(int8_t)((w0 >> (8 * s)) & 0xffu);
            a[r][1] = dd * (float)(int8_t)((w0 >> (8 * (2 + s))) & 0xffu);
            a[r][2] = dd * (float)(int8_t)((w1 >> (8 * s)) & 0xffu);
            a[r][3] = dd * (float)(int8_t)((w1 >> (8 * (2 + s))) & 0xffu);
            law[r][0] = la.x; law[r][1] = la.y; law[r][2] = la.z; law[r][3] = la.w;
            lbw[r][0] = lb.x; lbw[r][1] = lb.y; lbw[r][2] = lb.z; lbw[r][3] = lb.w;
            qhw[r][0] = qh.x; qhw[r][1] = qh.y; qhw[r][2] = qh.z; qhw[r][3] = qh.w;
        }
        // One 16-element group v at a time: quants 0..63 of group v are
        // element 16v + 4j + t of the lane's record (the -32 offset enters
        // through X_v).
        float acc[NR][MT];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            float sv[NR][MT];
#pragma unroll
            for (int r = 0; r < NR; ++r)
#pragma unroll
                for (int m = 0; m < MT; ++m) sv[r][m] = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float f[NR][4];
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    uint32_t q;
                    const uint32_t lw = (NR * MT > 2) ? pinned((v & 1) ? lbw[r][j] : law[r][j])
                                                      : ((v & 1) ? lbw[r][j] : law[r][j]);
                    if (v == 0) q = (lw & 0x0f0f0f0fu) | ((qhw[r][j] << 4) & 0x30303030u);
                    else if (v == 1) q = (lw & 0x0f0f0f0fu) | ((qhw[r][j] << 2) & 0x30303030u);
                    else if (v == 2) q = ((lw >> 4) & 0x0f0f0f0fu) | (qhw[r][j] & 0x30303030u);
                    else q = ((lw >> 4) & 0x0f0f0f0fu) | ((qhw[r][j] >> 2) & 0x30303030u);
                    q = opaque(q);
#pragma unroll
                    for (int t = 0; t < 4; ++t) f[r][t] = byte_f(q, t);
                }
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const float4 xv = xf(m, 4 * v + j);
#pragma unroll
                    for (int r = 0; r < NR; ++r) {
                        sv[r][m] = __builtin_fmaf(f[r][0], xv.x, sv[r][m]);
                        sv[r][m] = __builtin_fmaf(f[r][1], xv.y, sv[r][m]);
                        sv[r][m] = __builtin_fmaf(f[r][2], xv.z, sv[r][m]);
                        sv[r][m] = __builtin_fmaf(f[r][3], xv.w, sv[r][m]);
                    }
                    if constexpr (NR * MT > 2) {
#pragma unroll
                        for (int r = 0; r < NR; ++r) asm volatile("" : "+v"(sv[r][m]));
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float x32 = 32.0f * sf(m, v);  // exact
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    const float t = a[r][v] * (sv[r][m] - x32);
                    acc[r][m] = (v == 0) ? t : acc[r][m] + t;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m) part[r][m] = acc[r][m];
    }
}

}  // namespace

// ------------------------------------------------------------------ kernel

// SPLIT: K spans several slices and each workgroup takes one of them
// (blockIdx.y); it stores each row's slice total P_s (before any RMSNorm
// factor) to args.partial[s][members][rows], and f32_split_reduce_kernel adds
// the slices in order. The result equals the one-launch form bit for bit.
template <int T, int MT, int PRO, bool ONE_SLICE, int NBUF, int WAVES, int GROUP, bool PAIR, bool SPLIT = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_f32_kernel(WaveGemvArgs args) {
    static_assert(NBUF % GROUP == 0, "the ring holds whole row groups");
    static_assert(!SPLIT || (ONE_SLICE && !PAIR && PRO == kProPlain), "slice splits are plain one-slice passes");
    static_assert(!PAIR || (ONE_SLICE && NBUF % 2 == 0), "pairs are whole ring slots of one-slice rows");
    static_assert(MT <= 2 || ONE_SLICE, "several members stage one slice");
    constexpr bool NORM = PRO == kProNorm;
    constexpr bool SWIGLU = PRO == kProSwiglu;
    constexpr bool XREG = MT <= 2;  // lane records held in VGPRs
    constexpr int G = F32Rec<T>::groups;
    constexpr int STRIDE = F32Rec<T>::stride;
    constexpr int BB = BlockTraits<T>::bytes;
    constexpr int NBMAX = ONE_SLICE ? 16 : kF32Blocks;
    constexpr int NBW = (NBMAX + WAVES - 1) / WAVES;  // staging blocks per wave
    extern __shared__ float xs[];                     // [MT][slices][64 records][STRIDE]
    __shared__ float ssq_s[NORM ? MT : 1][NORM ? NBMAX : 1];
    __shared__ __attribute__((aligned(16))) float epi[XREG ? 4 : WAVES * 128];  // many-member pass epilogue, 512 B per wave

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = args.K;
    const int nb = K >> 8;
    const int slices = ONE_SLICE ? 1 : (nb + 15) >> 4;
    const int slice0 = SPLIT ? (int)blockIdx.y : 0;  // the slice this workgroup covers (SPLIT)
    const int members = args.members;
    const int p = lane & 3;
    const int bs = lane >> 2;
    const int nwaves = gridDim.x * WAVES;
    const int wg = blockIdx.x * WAVES + wave;
    const int split = PAIR ? args.total_rows >> 1 : args.total_rows;
    const int r_begin = (PAIR ? 2 : 1) * (int)((long long)split * wg / nwaves);
    const int r_end = (PAIR ? 2 : 1) * (int)((long long)split * (wg + 1) / nwaves);
    const uint32_t row_bytes = (uint32_t)nb * BB;

    auto locate = [&](int row, int& mat, int& local) {
        if constexpr (PAIR) {
            mat = row & 1;
            local = row >> 1;
            return;
        }
        mat = 0;
        int start = 0;
#pragma unroll
        for (int i = 0; i < kMaxGroup - 1; ++i) {
            if (i + 1 < args.count && row >= args.rows_end[i]) {
                mat = i + 1;
                start = args.rows_end[i];
            }
        }
        local = row - start;
    };
    auto pick_w = [&](int mat) {
        const uint8_t* w = args.w[0];
        uint32_t bytes = args.wbytes[0];
#pragma unroll
        for (int i = 1; i < kMaxGroup; ++i) {
            if (mat == i) {
                w = args.w[i];
                bytes = args.wbytes[i];
            }
        }
        return make_rsrc(w, bytes);
    };
    auto pick_y = [&](int mat, int& rows_mat) {
        float* y = args.y[0];
        int begin = 0, end = args.rows_end[0];
#pragma unroll
        for (int i = 1; i < kMaxGroup; ++i) {
            if (mat == i) {
                y = args.y[i];
                begin = args.rows_end[i - 1];
                end = args.rows_end[i];
            }
        }
        rows_mat = end - begin;
        return make_rsrc(y, (uint32_t)members * (uint32_t)rows_mat * 4u);
    };

    // Rows only move forward in one-slice launches, so the matrix of the
    // current row (and its weight / output resources) is tracked by cursors
    // that change only at matrix boundaries instead of being selected per unit.
    struct Cursor {
        int mat, start, end;
        __amdgpu_buffer_rsrc_t rs;
        int rows_mat;
    };
    auto cursor_at = [&](int row, bool out) {
        Cursor c;
        int local;
        locate(row, c.mat, local);
        c.start = row - local;
        const __amdgpu_buffer_rsrc_t yr = pick_y(c.mat, c.rows_mat);
        c.end = c.start + c.rows_mat;
        c.rs = out ? yr : pick_w(c.mat);
        return c;
    };
    auto seek = [&](Cursor& c, int row, bool out) {
        if (row >= c.end && c.mat + 1 < args.count) c = cursor_at(row, out);
    };

    // ---- activation loads first (vector memory returns in order, so the
    // staging waits for these, not for the weight loads issued after them).
    // Wave w stages super-blocks w, w + WAVES, ... of every member.
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(args.x, (uint32_t)members * (uint32_t)K * 4u);
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(args.gamma, NORM ? (uint32_t)K * 4u : 0u);
    const __amdgpu_buffer_rsrc_t ur = make_rsrc(args.x2, SWIGLU ? (uint32_t)members * (uint32_t)K * 4u : 0u);
    float4 xv[NBW][MT];
    float4 gv[NORM ? NBW : 1];
    float4 uv[SWIGLU ? NBW : 1][SWIGLU ? MT : 1];
#pragma unroll
    for (int k = 0; k < NBW; ++k) {
        const int b = 16 * slice0 + wave + WAVES * k;
        const int e = 256 * b + 4 * lane;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const uint32_t off = (b < nb && m < members) ? (uint32_t)(m * K + e) * 4u : kOutOfRange;
            xv[k][m] = load_f4(xr, off);
            if constexpr (SWIGLU) uv[k][m] = load_f4(ur, off);
        }
        if constexpr (NORM) gv[k] = load_f4(gr, b < nb ? (uint32_t)e * 4u : kOutOfRange);
    }
    asm volatile("" ::: "memory");

    // ---- weight ring, primed now; loads are unconditional (dead units read
    // from an out-of-range offset and return zeros), so each wait covers
    // exactly the unit reduced next.
    RowData<T> ring[NBUF];
    int lrow = r_begin, lslice = 0;
    constexpr bool kCursor = ONE_SLICE && !PAIR;
    Cursor lcur = cursor_at(r_begin, false);
    Cursor ccur = cursor_at(r_begin, true);
    // gate/up pairs: the two weights alternate row by row into one output
    const __amdgpu_buffer_rsrc_t pair_w0 = make_rsrc(args.w[0], PAIR ? args.wbytes[0] : 0u);
    const __amdgpu_buffer_rsrc_t pair_w1 = make_rsrc(args.w[1], PAIR ? args.wbytes[1] : 0u);
    const int pair_rows = args.rows_end[0];
    const __amdgpu_buffer_rsrc_t pair_y =
        make_rsrc(args.y[0], PAIR ? (uint32_t)members * (uint32_t)pair_rows * 4u : 0u);
    auto load_next = [&](RowData<T>& dst, int r) {
        const int row = ONE_SLICE ? lrow : lrow + r % GROUP;
        const bool live_row = row < r_end;
        int mat, local;
        __amdgpu_buffer_rsrc_t rs;
        if constexpr (kCursor) {
            if (live_row) seek(lcur, row, false);
            rs = lcur.rs;
            local = row - lcur.start;
        } else if constexpr (PAIR) {
            rs = (row & 1) ? pair_w1 : pair_w0;
            local = row >> 1;
        } else {
            locate(live_row ? row : r_begin, mat, local);
            rs = pick_w(mat);
        }
        const int b = (SPLIT ? slice0 : lslice) * 16 + bs;
        const bool live = live_row && b < nb;
        load_row<T>(dst, rs, live ? (uint32_t)local * row_bytes + (uint32_t)b * BB : kOutOfRange, p);
        if constexpr (ONE_SLICE) {
            ++lrow;
        } else if (r % GROUP == GROUP - 1 && ++lslice == slices) {
            lslice = 0;
            lrow += GROUP;
        }
    };
#pragma unroll
    for (int r = 0; r < NBUF; ++r) load_next(ring[r], r);

    // ---- staging: f32 activations into the lane records, group sums, and
    // per-block sums of squares for RMSNorm.
#pragma unroll
    for (int k = 0; k < NBW; ++k) {
        const int b = 16 * slice0 + wave + WAVES * k;
        const int e = 256 * b + 4 * lane;
        const int slice = (b >> 4) - slice0;  // staged slice (LDS index)
        int rec, pos;
        f32_slot<T>(e - (b >> 4) * kSliceElems, rec, pos);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float4 v = xv[k][m];
            if constexpr (SWIGLU) {
                // silu(gate) * up, in the reference's operation order (model_ops.rs:316-328)
                v.x = (v.x / (1.0f + expf(-v.x))) * uv[k][m].x;
                v.y = (v.y / (1.0f + expf(-v.y))) * uv[k][m].y;
                v.z = (v.z / (1.0f + expf(-v.z))) * uv[k][m].z;
                v.w = (v.w / (1.0f + expf(-v.w))) * uv[k][m].w;
            }
            if constexpr (NORM) {
                const float sq = v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                const float blk = wave_sum_uniform(sq);
                if (lane == 0 && b < nb && m < members) ssq_s[m][b] = blk;
                v.x *= gv[k].x;
                v.y *= gv[k].y;
                v.z *= gv[k].z;
                v.w *= gv[k].w;
            }
            const float gsum = group_sum_f<T>(((v.x + v.y) + v.z) + v.w);
            // Blocks past K inside the last slice are staged as zeros: their
            // lanes multiply zero weights, and 0 * (stale LDS) could be NaN.
            if (b < 16 * (slice0 + slices) && m < members) {
                float* dst = xs + ((m * slices + slice) * 64 + rec) * STRIDE;
                *reinterpret_cast<float4*>(dst + pos) = v;
                if ((lane & (F32Rec<T>::group / 4 - 1)) == 0) dst[64 + pos / F32Rec<T>::group] = gsum;
            }
        }
    }
    __syncthreads();

    float inv[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        inv[m] = 1.f;
        if constexpr (NORM) {
            float total = 0.f;
            for (int b = 0; b < nb; ++b) total += ssq_s[m][b];
            // RMSNorm (qwen_reference.rs:550-556): x * (1/sqrt(sum(x^2)/K + eps)) * gamma
            inv[m] = 1.0f / sqrtf(total / (float)K + args.eps);
        }
    }

    const bool accumulate = args.accumulate != 0;
    auto put = [&](float value, __amdgpu_buffer_rsrc_t yr, uint32_t off) {
        if (accumulate) {
            __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(value, yr, (int)off, 0, 0);
        } else {
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, value), yr, (int)off, 0, 0);
        }
    };
    // silu(gate) * up of one output row (model_ops.rs:316-328)
    auto swiglu = [](float g, float u) { return (g / (1.0f + expf(-g))) * u; };
    const __amdgpu_buffer_rsrc_t partial_r =
        make_rsrc(args.partial, SPLIT ? (uint32_t)gridDim.y * (uint32_t)members * (uint32_t)args.total_rows * 4u : 0u);

    if constexpr (!XREG) {
        // ---- several members, one slice: passes over the whole ring. Each
        // pass reads every 4-element piece of a member's record once and
        // applies it to the ring's rows; then the ring is refilled. The last
        // pass reduces only the wave's remaining NR rows (a wave's share of a
        // short launch is often fewer rows than the ring holds).
        const float* rec_base = xs + lane * STRIDE;
        auto xf = [&](int m, int i) { return *reinterpret_cast<const float4*>(rec_base + m * 64 * STRIDE + 4 * i); };
        auto sf = [&](int m, int g) { return rec_base[m * 64 * STRIDE + 64 + g]; };
        int crow = r_begin;
        float* const ep = epi + wave * 128;  // [4 lane rows][32 values]
        const int vl = lane & 31;
        float inv_l = inv[0];  // the RMSNorm factor of this lane's member
#pragma unroll
        for (int m = 1; m < MT; ++m)
            if (vl % MT == m) inv_l = inv[m];
        auto pass = [&](auto refill_const, auto nr_const) {
            constexpr bool REFILL = decltype(refill_const)::value;
            constexpr int NR = decltype(nr_const)::value;
            static_assert(NR >= 1 && NR <= NBUF && (REFILL ? NR == NBUF : true), "full passes reduce the whole ring");
            static_assert(NR * MT <= 32 && MT % 4 == 0, "a pass's values fit lanes 0-31 in whole float4s");
            // The records never change, but keeping all of them in registers
            // across passes would spill: re-read them every pass.
            asm volatile("" ::: "memory");
            float part[NR][MT];
            rows_dot<T, NR, MT>(reinterpret_cast<const RowData<T>(&)[NR]>(ring), p, xf, sf, part);
            if constexpr (REFILL) {
#pragma unroll
                for (int r = 0; r < NBUF; ++r) load_next(ring[r], r);
            }
            // Epilogue. Each (row r, member m) value's 16-lane row sums (the
            // DPP steps of wave_sum_uniform) go through this wave's LDS
            // scratch, and lane v = r * MT + m finishes value v: the row sums
            // added (r0 + r1) + (r2 + r3), the RMSNorm factor, SwiGLU, the
            // store. Every value sees wave_sum_uniform's operations in its
            // order, so the bits equal the single-member launch's, and the
            // per-value work runs once across lanes instead of once per value.
#pragma unroll
            for (int r = 0; r < NR; ++r)
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    float v = part[r][m];
                    v = dpp_step<0xb1>(v);   // quad_perm [1,0,3,2]
                    v = dpp_step<0x4e>(v);   // quad_perm [2,3,0,1]
                    v = dpp_step<0x141>(v);  // row_half_mirror
                    v = dpp_step<0x140>(v);  // row_mirror
                    part[r][m] = v;
                }
            if ((lane & 15) == 0) {
                float* dst = ep + 32 * (lane >> 4);
#pragma unroll
                for (int i = 0; i < NR * MT; i += 4)
                    *reinterpret_cast<float4*>(dst + i) =
                        float4{part[(i + 0) / MT][(i + 0) % MT], part[(i + 1) / MT][(i + 1) % MT],
                               part[(i + 2) / MT][(i + 2) % MT], part[(i + 3) / MT][(i + 3) % MT]};
            }
            // (one wave's LDS operations complete in order: no barrier)
            auto total_of = [&](int i) { return (ep[i] + ep[32 + i]) + (ep[64 + i] + ep[96 + i]); };
            const int vr = vl / MT, vm = vl % MT;  // this lane's value: row crow + vr, member vm
            const int row = crow + vr;
            // lanes 32-63 repeat lanes 0-31's values and store nothing
            const bool mine = lane < 32 && vl < NR * MT && row < r_end && vm < members;
            if constexpr (SPLIT) {
                const float ps = total_of(vl);
                const uint32_t off = mine ? (uint32_t)((slice0 * members + vm) * args.total_rows + row) * 4u : kOutOfRange;
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, ps), partial_r, (int)off, 0, 0);
            } else if constexpr (PAIR) {
                // gate rows are even, each followed by its up row: lane v
                // (gate) also adds value v + MT (up)
                const bool gate = (vr & 1) == 0 && vl + MT < 32;
                const float g = total_of(vl) * inv_l;
                const float u = total_of(gate ? vl + MT : vl) * inv_l;
                const uint32_t off = (mine && gate) ? (uint32_t)(vm * pair_rows + (row >> 1)) * 4u : kOutOfRange;
                put(swiglu(g, u), pair_y, off);
            } else {
                const float total = total_of(vl) * inv_l;
                // rows move forward; the output resource can change at a
                // matrix boundary inside the pass, so one store per row
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    const int rr = crow + r;
                    if (rr < r_end) seek(ccur, rr, true);
                    const uint32_t off =
                        (mine && vr == r) ? (uint32_t)(vm * ccur.rows_mat + (rr - ccur.start)) * 4u : kOutOfRange;
                    put(total, ccur.rs, off);
                }
            }
            crow += NBUF;
        };
        const int rows_w = r_end - r_begin;
        const int passes = (rows_w + NBUF - 1) / NBUF;
        using Full = std::integral_constant<int, NBUF>;
        for (int ps = 0; ps + 1 < passes; ++ps) pass(std::true_type{}, Full{});
        if (passes == 0) return;
        // 1..NBUF rows left (wave-uniform); gate/up pairs leave an even count
        const int left = rows_w - (passes - 1) * NBUF;
        if constexpr (!PAIR) {
            if (left == 1) return pass(std::false_type{}, std::integral_constant<int, 1>{});
        }
        if constexpr (NBUF > 2) {
            if (left == 2) return pass(std::false_type{}, std::integral_constant<int, 2>{});
        }
        if constexpr (NBUF > 3 && !PAIR) {
            if (left == 3) return pass(std::false_type{}, std::integral_constant<int, 3>{});
        }
        pass(std::false_type{}, Full{});
        return;
    } else {
        // ---- one or two members: records in VGPRs; the ring is reduced one
        // unit at a time and each slot refilled with the unit NBUF ahead.
        float4 xq[MT][16];
        float xg[MT][G];
        auto read_rec = [&](int slice) {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float* src = xs + ((m * slices + slice) * 64 + lane) * STRIDE;
#pragma unroll
                for (int i = 0; i < 16; ++i) xq[m][i] = *reinterpret_cast<const float4*>(src + 4 * i);
                const float4 sums = *reinterpret_cast<const float4*>(src + 64);
                const float sv[4] = {sums.x, sums.y, sums.z, sums.w};
#pragma unroll
                for (int g = 0; g < G; ++g) xg[m][g] = sv[g];
            }
        };
        auto xf = [&](int m, int i) { return xq[m][i]; };
        auto sf = [&](int m, int g) { return xg[m][g]; };
        if constexpr (ONE_SLICE) read_rec(0);

        int crow = r_begin, cslice = 0;
        constexpr int kAcc = ONE_SLICE ? 1 : GROUP;
        float acc[kAcc][MT];
        float gk[MT];
#pragma unroll
        for (int r = 0; r < kAcc; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;
        auto consume = [&](const RowData<T>& d, int r) {
            if constexpr (!ONE_SLICE) {
                if (r % GROUP == 0) read_rec(cslice);
            }
            const RowData<T> one[1] = {d};
            float part[1][MT];
            rows_dot<T, 1, MT>(one, p, xf, sf, part);
            const int ai = ONE_SLICE ? 0 : r % GROUP;
            const int row = ONE_SLICE ? crow : crow + r % GROUP;
            const bool last = ONE_SLICE || cslice == slices - 1;
            int mat, local, rows_mat;
            __amdgpu_buffer_rsrc_t yr;
            if constexpr (kCursor) {
                if (row < r_end) seek(ccur, row, true);
                yr = ccur.rs;
                local = row - ccur.start;
                rows_mat = ccur.rows_mat;
            } else if constexpr (PAIR) {
                yr = pair_y;
                local = row >> 1;
                rows_mat = pair_rows;
            } else {
                locate(row < r_end ? row : r_begin, mat, local);
                yr = pick_y(mat, rows_mat);
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float ps = wave_sum_uniform(part[0][m]);
                acc[ai][m] = (ONE_SLICE || cslice == 0) ? ps : acc[ai][m] + ps;
                const float total = acc[ai][m] * inv[m];
                const uint32_t off = (last && row < r_end && lane == 0 && m < members)
                                         ? (uint32_t)(m * rows_mat + local) * 4u
                                         : kOutOfRange;
                if constexpr (SPLIT) {
                    // this workgroup's slice total P_s, as the several-member pass stores it
                    const uint32_t poff = (row < r_end && lane == 0 && m < members)
                                              ? (uint32_t)((slice0 * members + m) * args.total_rows + row) * 4u
                                              : kOutOfRange;
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, ps), partial_r, (int)poff, 0, 0);
                } else if constexpr (PAIR) {
                    if (r % 2 == 0) {
                        gk[m] = total;
                    } else {
                        put(swiglu(gk[m], total), yr, off);
                    }
                } else {
                    put(total, yr, off);
                }
            }
            if constexpr (ONE_SLICE) {
                ++crow;
            } else if (r % GROUP == GROUP - 1 && ++cslice == slices) {
                cslice = 0;
                crow += GROUP;
            }
        };

        const int rows_w = r_end - r_begin;
        const int units = ONE_SLICE ? rows_w : (rows_w + GROUP - 1) / GROUP * GROUP * slices;
        const int passes = (units + NBUF - 1) / NBUF;
        for (int ps = 0; ps + 1 < passes; ++ps) {
#pragma unroll
            for (int r = 0; r < NBUF; ++r) {
                consume(ring[r], r);
                load_next(ring[r], r);
            }
        }
        if (passes > 0) {
            const int left = units - (passes - 1) * NBUF;
#pragma unroll
            for (int r = 0; r < NBUF; ++r) {
                if (r < left) consume(ring[r], r);
            }
        }
    }
}

// ---------------------------------------------------------------- launcher

namespace {

template <int T>
size_t f32_lds_bytes(int members, int K) {
    const int slices = ((K >> 8) + 15) >> 4;
    return (size_t)members * slices * 64 * F32Rec<T>::stride * sizeof(float);
}

template <int T, int MT, int PRO, bool ONE_SLICE, int NBUF, int WAVES, int GROUP = 1, bool PAIR = false,
          bool SPLIT = false>
struct F32Instance {
    static std::atomic<int> occupancy;  // resident workgroups per CU at the largest LDS size (0: not queried)
    static hipError_t launch(const WaveGemvArgs& a, int cu_count, int per_cu, hipStream_t stream) {
        auto kern = gemv_f32_kernel<T, MT, PRO, ONE_SLICE, NBUF, WAVES, GROUP, PAIR, SPLIT>;
        const size_t lds = f32_lds_bytes<T>(MT, ONE_SLICE ? std::min(a.K, (int)kSliceElems) : a.K);
        int occ = occupancy.load(std::memory_order_relaxed);
        if (occ == 0) {
            const int max_lds = (int)f32_lds_bytes<T>(MT, ONE_SLICE ? kSliceElems : kWaveMaxK);
            (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, max_lds);
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)kern, WAVES * 64, max_lds) !=
                    hipSuccess ||
                occ < 1) {
                occ = 1;
            }
            occupancy.store(occ, std::memory_order_relaxed);
        }
        const int slices = ONE_SLICE ? 1 : ((a.K >> 8) + 15) >> 4;
        const long long units = (long long)a.total_rows * slices;
        const long long want = (units + 2 * WAVES - 1) / (2 * WAVES);
        long long grid = want;
        if (want >= cu_count) {
            grid = (long long)cu_count * std::min<long long>({(want + cu_count - 1) / cu_count, (long long)occ,
                                                               (long long)per_cu});
        }
        if (grid < 1) grid = 1;
        unsigned gy = 1;
        if constexpr (SPLIT) {
            // one slice per grid row; about one workgroup per CU in all
            gy = (unsigned)(((a.K >> 8) + 15) >> 4);
            grid = std::max<long long>(1, std::min<long long>(want, cu_count / (long long)gy));
        }
        hipLaunchKernelGGL(kern, dim3((unsigned)grid, gy), dim3(WAVES * 64), lds, stream, a);
        return hipGetLastError();
    }
};
template <int T, int MT, int PRO, bool ONE_SLICE, int NBUF, int WAVES, int GROUP, bool PAIR, bool SPLIT>
std::atomic<int> F32Instance<T, MT, PRO, ONE_SLICE, NBUF, WAVES, GROUP, PAIR, SPLIT>::occupancy{0};

// y[m][row] (+)= ((P_0 + P_1) + P_2) ... over the slices of a SPLIT launch,
// in slice order: the slice totals of the one-launch form, added the same way.
__global__ __launch_bounds__(256) void f32_split_reduce_kernel(WaveGemvArgs a, int slices) {
    const int total = a.members * a.total_rows;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
        const int m = i / a.total_rows;
        const int row = i - m * a.total_rows;
        float t = a.partial[(size_t)m * a.total_rows + row];
        for (int s = 1; s < slices; ++s) t = t + a.partial[((size_t)s * a.members + m) * a.total_rows + row];
        int mat = 0, start = 0;
        for (int g = 0; g + 1 < a.count; ++g) {
            if (row >= a.rows_end[g]) {
                mat = g + 1;
                start = a.rows_end[g];
            }
        }
        float* y = a.y[0];
        for (int g = 1; g < kMaxGroup; ++g) {
            if (mat == g) y = a.y[g];
        }
        const int rows_mat = a.rows_end[mat] - start;
        float* dst = y + (size_t)m * rows_mat + (row - start);
        *dst = a.accumulate ? *dst + t : t;
    }
}

// One or two members.
template <int T, int MT, int PRO, bool ONE_SLICE, bool PAIR = false>
hipError_t launch_few(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    const int slices = ONE_SLICE ? 1 : ((a.K >> 8) + 15) >> 4;
    const long long units = (long long)a.total_rows * slices;
    const long long per_cu = (units + cu_count - 1) / cu_count;
    if constexpr (!ONE_SLICE) {
        return F32Instance<T, MT, PRO, false, 2, 8, 2>::launch(a, cu_count, 1, stream);
    } else {
        if constexpr (MT == 1) {
            // Streams of more than 48 units per CU (gate/up, the lm_head): a
            // three-unit ring (four for gate/up pairs) over 8-wave workgroups,
            // one per CU. MI355X sweep over ring {2,3,4,6,8} x waves {4,8,16} x
            // workgroups per CU {1,2,4}: 13.3 us for the gate+up group
            // (Q4_K 4096 -> 2 x 12288) against 14.3 us for ring 2 x 2 per CU,
            // and 97 us for the Q6_K 4096 -> 151936 head against 124 us for
            // ring 8 x 4 waves.
            if (per_cu > 48) {
                return F32Instance<T, 1, PRO, true, (PAIR ? 4 : 3), 8, 1, PAIR>::launch(a, cu_count, 1, stream);
            }
        }
        return F32Instance<T, MT, PRO, true, 2, 8, 1, PAIR>::launch(a, cu_count, per_cu > 48 ? 2 : 1, stream);
    }
}

// Three to eight members, one slice.
template <int T, int PRO, bool PAIR>
hipError_t launch_many(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    if (a.members <= 4) return F32Instance<T, 4, PRO, true, 4, 8, 1, PAIR>::launch(a, cu_count, 1, stream);
    // ring depth: 4 rows where the registers allow (Q6_K rows need 22 VGPRs)
    return F32Instance<T, 8, PRO, true, (T != kQ6K ? 4 : PAIR ? 2 : 3), 8, 1, PAIR>::launch(a, cu_count, 1, stream);
}

template <int T, int PRO>
hipError_t launch_plain(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    const bool one = a.K <= kSliceElems;
    if (a.members <= 1) {
        return one ? launch_few<T, 1, PRO, true>(a, cu_count, stream) : launch_few<T, 1, PRO, false>(a, cu_count, stream);
    }
    if (a.members <= 2 || !one) {
        if (a.members > 2) return hipErrorInvalidValue;
        return one ? launch_few<T, 2, PRO, true>(a, cu_count, stream) : launch_few<T, 2, PRO, false>(a, cu_count, stream);
    }
    if constexpr (PRO == kProSwiglu) {
        return hipErrorInvalidValue;  // the host splits SwiGLU-prologue launches into pairs of members
    } else {
        return launch_many<T, PRO, false>(a, cu_count, stream);
    }
}

template <int T, int PRO>
hipError_t launch_pair(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    if (a.members <= 1) return launch_few<T, 1, PRO, true, true>(a, cu_count, stream);
    if (a.members <= 2) return launch_few<T, 2, PRO, true, true>(a, cu_count, stream);
    return launch_many<T, PRO, true>(a, cu_count, stream);
}

template <int T>
hipError_t launch_type(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    if (a.members < 1 || a.members > f32_max_members(a.K)) return hipErrorInvalidValue;
    if (a.pair_swiglu) {
        if (a.x2 != nullptr || a.count != 2 || a.rows_end[1] != 2 * a.rows_end[0] || a.K > kSliceElems) {
            return hipErrorInvalidValue;
        }
        return a.gamma != nullptr ? launch_pair<T, kProNorm>(a, cu_count, stream)
                                  : launch_pair<T, kProPlain>(a, cu_count, stream);
    }
    if (a.x2 != nullptr) {
        if (a.gamma != nullptr || a.members > kSwigluMaxMembers) return hipErrorInvalidValue;
        return launch_plain<T, kProSwiglu>(a, cu_count, stream);
    }
    if (a.gamma != nullptr) return launch_plain<T, kProNorm>(a, cu_count, stream);
    return launch_plain<T, kProPlain>(a, cu_count, stream);
}

// Members over a K of several slices: one workgroup per (row range, slice),
// then the ordered slice reduction. One member (a K beyond kWaveMaxK) keeps
// its records in VGPRs, as the one-launch form does.
template <int T>
hipError_t launch_split(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    hipError_t e = (a.members == 1)
                       ? F32Instance<T, 1, kProPlain, true, 3, 8, 1, false, true>::launch(a, cu_count, 1, stream)
                   : (a.members <= 4)
                       ? F32Instance<T, 4, kProPlain, true, 4, 8, 1, false, true>::launch(a, cu_count, 1, stream)
                       : F32Instance<T, 8, kProPlain, true, (T != kQ6K ? 4 : 3), 8, 1, false, true>::launch(
                             a, cu_count, 1, stream);
    if (e != hipSuccess) return e;
    const int slices = ((a.K >> 8) + 15) >> 4;
    const long long total = (long long)a.members * a.total_rows;
    const unsigned grid = (unsigned)std::min<long long>((total + 255) / 256, (long long)cu_count * 4);
    hipLaunchKernelGGL(f32_split_reduce_kernel, dim3(grid), dim3(256), 0, stream, a, slices);
    return hipGetLastError();
}

}  // namespace

size_t f32_split_partial_bytes(int members, int K, int total_rows) {
    const int slices = ((K >> 8) + 15) >> 4;
    return (size_t)slices * members * total_rows * sizeof(float);
}

hipError_t launch_gemv_f32_split(int value_type, const WaveGemvArgs& args, int cu_count, hipStream_t stream) {
    const int min_members = args.K > kWaveMaxK ? 1 : 3;
    if (args.members < min_members || args.members > kWaveMaxMembers || args.K <= kSliceElems ||
        args.K > kF32SplitMaxK || args.K % 256 != 0 || args.gamma != nullptr || args.x2 != nullptr ||
        args.pair_swiglu || args.partial == nullptr ||
        f32_split_partial_bytes(args.members, args.K, args.total_rows) > kF32SplitScratchBytes) {
        return hipErrorInvalidValue;
    }
    switch (value_type) {
    case kQ4K: return launch_split<kQ4K>(args, cu_count, stream);
    case kQ5K: return launch_split<kQ5K>(args, cu_count, stream);
    case kQ6K: return launch_split<kQ6K>(args, cu_count, stream);
    default: return hipErrorInvalidValue;
    }
}

int f32_long_k_members(int K, int total_rows) {
    if (K <= kWaveMaxK || K > kF32SplitMaxK || K % 256 != 0 || total_rows < 1) return 0;
    int m = kWaveMaxMembers;
    while (m > 0 && f32_split_partial_bytes(m, K, total_rows) > kF32SplitScratchBytes) --m;
    return m;
}

int f32_max_members(int K) {
    if (K < 256 || K > kWaveMaxK) return 0;
    return K <= kSliceElems ? kWaveMaxMembers : 2;
}

hipError_t launch_gemv_f32(int value_type, const WaveGemvArgs& args, int cu_count, hipStream_t stream) {
    switch (value_type) {
    case kQ4K: return launch_type<kQ4K>(args, cu_count, stream);
    case kQ5K: return launch_type<kQ5K>(args, cu_count, stream);
    case kQ6K: return launch_type<kQ6K>(args, cu_count, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace ribn_amd

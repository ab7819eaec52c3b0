// Wave GEMV for Q4_K / Q5_K / Q6_K on gfx950 (CDNA4, wave64): the decode
// path's bandwidth kernel, with an optional fused RMSNorm prologue and a
// grouped form that streams several weights sharing one activation vector
// (q/k/v, gate/up) in a single launch.
//
// Layout and mapping
//  - Weights are the encoded GGML array-of-blocks; row n of a [K, N] tensor is
//    K/256 consecutive super-blocks (crates/nvidia/src/quantized.rs:136-142).
//  - A wave covers 16 consecutive super-blocks of a row per "slice" (K = 4096
//    is one slice); lane l owns block (l >> 2) of the slice and quarter
//    p = (l & 3), i.e. 64 elements:
//      Q4_K / Q5_K: groups 2p and 2p+1 (payload bytes 32p..32p+31, low/high nibbles);
//      Q6_K:        groups 4c..4c+3 at positions 16s..16s+15 (c = p >> 1, s = p & 1).
//  - Activations are quantized once per workgroup into 16-bit fixed point per
//    k-quant scale group (v = round(x * 2^(15-e)), 2^e > max|x| of the group),
//    stored as a signed high byte and an unsigned low byte, so the products
//    with the 4..6-bit quants are v_dot4 integer dot products (exact, int32
//    accumulation). Per group the row gains
//        unscale_g * ((d*sc_g) * S_g - (dmin*m_g) * X_g)     (Q4_K / Q5_K)
//        unscale_g * (d*sc_g) * (S_g - 32 X_g)               (Q6_K)
//    with S_g = sum(q*v) and X_g = sum(v). The activation rounding is at most
//    2^-16 of the group's maximum per element.
//  - The quantized activations sit in LDS in lane order (one padded record
//    per lane and slice), so each wave reads its lane's data with conflict-free
//    128-bit LDS loads. A fused RMSNorm multiplies x by gamma before the
//    quantization and applies 1/rms to each output, which keeps the only
//    cross-wave dependency (the sum of squares) to one workgroup barrier.
//  - Weight loads for a wave's first units are issued right after the
//    activation loads, before the staging, so HBM latency overlaps the
//    prologue. Each wave then keeps a ring of units (row x slice) in
//    registers: a unit is reduced, then its slot is refilled with the unit a
//    full ring ahead.
// Arithmetic per member is independent of the member count, so every row of a
// batched launch is bit-identical to the single-member launch.
#include "kquant_device.hpp"
#include "kquant_launch.hpp"
#include "wave_rows.hpp"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace ribn_amd {

template <int T> struct ActTraits {
    static constexpr int group = (T == kQ6K) ? 16 : 32;  // elements per scale group
    static constexpr int groups = 64 / group;            // scale groups per lane
    // Dwords per lane record: 16 high-byte words, 16 low-byte words, then
    // `groups` unscale factors and `groups` sums. The stride is odd in
    // 16-byte units, so 16 lanes' 128-bit reads fall in distinct banks.
    static constexpr int stride = (T == kQ6K) ? 44 : 36;
};

// One lane's quantized activations for one slice.
template <int T> struct LaneAct {
    uint32_t h[16];  // signed high bytes, four elements per word
    uint32_t l[16];  // unsigned low bytes
    float unscale[ActTraits<T>::groups];
    float xsum[ActTraits<T>::groups];  // X_g as f32 (exact: |X_g| < 2^21)
    int xsum32[ActTraits<T>::groups];  // -32 X_g (Q6_K)
};

// Position of element e (a multiple of 4, within one slice) in the lane
// records: lane, word, scale group.
template <int T>
__device__ __forceinline__ void act_slot(int e, int& lane, int& word, int& group) {
    if constexpr (T == kQ6K) {
        const int bs = e >> 8, c = (e >> 7) & 1, v = (e >> 5) & 3, s = (e >> 4) & 1, j = (e >> 2) & 3;
        lane = 4 * bs + 2 * c + s;
        word = 4 * v + j;
        group = v;
    } else {
        lane = e >> 6;
        word = (e >> 2) & 15;
        group = word >> 3;
    }
}

template <int CTRL>
__device__ __forceinline__ int dpp_sum_step_i(int v) {
    return v + __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

// Max / sum over the lanes holding one scale group (4 or 8 consecutive lanes).
template <int T>
__device__ __forceinline__ float group_max(float v) {
    v = dpp_max_step<0xb1>(v);  // quad_perm [1,0,3,2]
    v = dpp_max_step<0x4e>(v);  // quad_perm [2,3,0,1]
    if constexpr (ActTraits<T>::group == 32) v = dpp_max_step<0x141>(v);  // row_half_mirror
    return v;
}
template <int T>
__device__ __forceinline__ int group_sum(int v) {
    v = dpp_sum_step_i<0xb1>(v);
    v = dpp_sum_step_i<0x4e>(v);
    if constexpr (ActTraits<T>::group == 32) v = dpp_sum_step_i<0x141>(v);
    return v;
}

// Four-way byte dot products: quants (0..63) against the signed high bytes
// and the unsigned low bytes of the fixed-point activations.
__device__ __forceinline__ int sdot4(uint32_t q, uint32_t x, int acc) {
    return __builtin_amdgcn_sdot4((int)q, (int)x, acc, false);
}
__device__ __forceinline__ int udot4(uint32_t q, uint32_t x, int acc) {
    return (int)__builtin_amdgcn_udot4(q, x, (uint32_t)acc, false);
}

// --------------------------------------------------- per-row dot products
//
// part[m] = this lane's share of row . x_m for one unit (already unscaled).
template <int T, int MT>
__device__ __forceinline__ void row_dot(const RowData<T>& d, int p, const LaneAct<T> (&xa)[MT], float (&part)[MT]) {
    if constexpr (T == kQ4K || T == kQ5K) {
        const uint4 h = d.h;
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
        const float a0 = dd * (float)((scw >> sh) & 0xffu);
        const float a1 = dd * (float)((scw >> (sh + 8)) & 0xffu);
        const float b0 = dmin * (float)((mnw >> sh) & 0xffu);
        const float b1 = dmin * (float)((mnw >> (sh + 8)) & 0xffu);
        const uint32_t qw[8] = {d.qa.x, d.qa.y, d.qa.z, d.qa.w, d.qb.x, d.qb.y, d.qb.z, d.qb.w};
        int hA[MT], lA[MT], hB[MT], lB[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) hA[m] = lA[m] = hB[m] = lB[m] = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // group A = 2p (low nibbles), group B = 2p+1 (high nibbles), 5th bit for Q5_K
            uint32_t qa = qw[j] & 0x0f0f0f0fu;
            uint32_t qb = (qw[j] >> 4) & 0x0f0f0f0fu;
            if constexpr (T == kQ5K) {
                const uint32_t hw[8] = {d.ha.x, d.ha.y, d.ha.z, d.ha.w, d.hb.x, d.hb.y, d.hb.z, d.hb.w};
                qa |= ((hw[j] >> (2 * p)) & 0x01010101u) << 4;
                qb |= ((hw[j] >> (2 * p + 1)) & 0x01010101u) << 4;
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                hA[m] = sdot4(qa, xa[m].h[j], hA[m]);
                lA[m] = udot4(qa, xa[m].l[j], lA[m]);
                hB[m] = sdot4(qb, xa[m].h[8 + j], hB[m]);
                lB[m] = udot4(qb, xa[m].l[8 + j], lB[m]);
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float sA = (float)(hA[m] * 256 + lA[m]);
            const float sB = (float)(hB[m] * 256 + lB[m]);
            const float tA = __builtin_fmaf(a0, sA, -(b0 * xa[m].xsum[0]));
            const float tB = __builtin_fmaf(a1, sB, -(b1 * xa[m].xsum[1]));
            part[m] = __builtin_fmaf(tA, xa[m].unscale[0], tB * xa[m].unscale[1]);
        }
    } else {
        const int c = p >> 1, s = p & 1;
        const uint32_t sh = d.shift;
        const uint4 la = funnel(d.la, d.la_t, sh);
        const uint4 lb = funnel(d.lb, d.lb_t, sh);
        const uint4 qh = funnel(d.qh, d.qh_t, sh);
        const uint4 sc = funnel(d.sc, d.sc_t, sh);  // int8 scales
        const float dd = half_bits_to_float(d.d16);
        const uint32_t w0 = c ? sc.z : sc.x;  // scales 8c+0..8c+3
        const uint32_t w1 = c ? sc.w : sc.y;  // scales 8c+4..8c+7
        float a[4];
        a[0] = dd * (float)(int8_t)((w0 >> (8 * s)) & 0xffu);
        a[1] = dd * (float)(int8_t)((w0 >> (8 * (2 + s))) & 0xffu);
        a[2] = dd * (float)(int8_t)((w1 >> (8 * s)) & 0xffu);
        a[3] = dd * (float)(int8_t)((w1 >> (8 * (2 + s))) & 0xffu);
        const uint32_t law[4] = {la.x, la.y, la.z, la.w};
        const uint32_t lbw[4] = {lb.x, lb.y, lb.z, lb.w};
        const uint32_t qhw[4] = {qh.x, qh.y, qh.z, qh.w};
        int hs[MT][4], ls[MT][4];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int v = 0; v < 4; ++v) hs[m][v] = ls[m][v] = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // quants 0..63 (the -32 offset is applied through X_g)
            uint32_t q[4];
            q[0] = (law[j] & 0x0f0f0f0fu) | ((qhw[j] << 4) & 0x30303030u);
            q[1] = (lbw[j] & 0x0f0f0f0fu) | ((qhw[j] << 2) & 0x30303030u);
            q[2] = ((law[j] >> 4) & 0x0f0f0f0fu) | (qhw[j] & 0x30303030u);
            q[3] = ((lbw[j] >> 4) & 0x0f0f0f0fu) | ((qhw[j] >> 2) & 0x30303030u);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    hs[m][v] = sdot4(q[v], xa[m].h[4 * v + j], hs[m][v]);
                    ls[m][v] = udot4(q[v], xa[m].l[4 * v + j], ls[m][v]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float t = 0.f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                // sum((q - 32) v) = S - 32 X, exact in int32
                const float sv = (float)(hs[m][v] * 256 + ls[m][v] + xa[m].xsum32[v]);
                t = __builtin_fmaf(a[v], sv * xa[m].unscale[v], t);
            }
            part[m] = t;
        }
    }
}

// ------------------------------------------------------------------ kernel

template <int T, int MT, int PRO, bool ONE_SLICE, int NBUF, int WAVES, int GROUP, bool PAIR>
__global__ __launch_bounds__(WAVES * 64) void gemv_wave_kernel(WaveGemvArgs args) {
    static_assert(NBUF % GROUP == 0, "the ring holds whole row groups");
    static_assert(!PAIR || (ONE_SLICE && NBUF % 2 == 0), "pairs are whole ring slots of one-slice rows");
    constexpr bool NORM = PRO == kProNorm;
    constexpr bool SWIGLU = PRO == kProSwiglu;
    constexpr int kWaves = WAVES;
    constexpr int kThreads = WAVES * 64;
    constexpr int BB = BlockTraits<T>::bytes;
    constexpr int G = ActTraits<T>::groups;
    constexpr int STRIDE = ActTraits<T>::stride;
    constexpr int CH = ONE_SLICE ? kSliceElems / (4 * kThreads) : kWaveMaxK / (4 * kThreads);
    extern __shared__ uint32_t xs[];  // [MT][slices][64 lanes][STRIDE]
    __shared__ float partial[MT][kWaves];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = args.K;
    const int nb = K >> 8;
    const int slices = ONE_SLICE ? 1 : (nb + 15) >> 4;
    const int members = args.members;
    const int p = lane & 3;
    const int bs = lane >> 2;
    const int nwaves = gridDim.x * kWaves;
    const int wg = blockIdx.x * kWaves + wave;
    // PAIR: units alternate (gate row n, up row n); a wave takes whole pairs
    const int split = PAIR ? args.total_rows >> 1 : args.total_rows;
    const int r_begin = (PAIR ? 2 : 1) * (int)((long long)split * wg / nwaves);
    const int r_end = (PAIR ? 2 : 1) * (int)((long long)split * (wg + 1) / nwaves);
    const uint32_t row_bytes = (uint32_t)nb * BB;

    // Row -> (matrix, local row); the row index is wave-uniform. Fields of
    // the argument arrays are picked by selects, not by a dynamic index
    // (which would reload them from the argument segment every unit).
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

    // ---- activation loads first: vector memory returns in order, so the
    // staging below waits for these and not for the weight loads after them.
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(args.x, (uint32_t)members * (uint32_t)K * 4u);
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(args.gamma, NORM ? (uint32_t)K * 4u : 0u);
    const __amdgpu_buffer_rsrc_t ur = make_rsrc(args.x2, SWIGLU ? (uint32_t)members * (uint32_t)K * 4u : 0u);
    float4 xv[MT][CH];
    float4 gv[CH];
    float4 uv[SWIGLU ? MT : 1][CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int e = 4 * ((int)threadIdx.x + kThreads * c);
        const bool in = e < K;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const uint32_t off = (in && m < members) ? (uint32_t)(m * K + e) * 4u : kOutOfRange;
            xv[m][c] = load_f4(xr, off);
            if constexpr (SWIGLU) uv[m][c] = load_f4(ur, off);
        }
        if constexpr (NORM) gv[c] = load_f4(gr, in ? (uint32_t)e * 4u : kOutOfRange);
    }
    asm volatile("" ::: "memory");

    // ---- weight ring, primed now. Loads are issued unconditionally (units
    // past the wave's range and blocks past K read from an out-of-range
    // offset, which returns zeros), so each stays where it is issued and the
    // wave waits for exactly the unit it reduces next.
    RowData<T> ring[NBUF];
    // Unit order: one slice of K = 4096 carries whole rows (row-major units);
    // longer K goes in groups of GROUP rows, slice by slice (row-minor), so
    // ring slot r always holds row r % GROUP of a group and the activations of
    // a slice are read once per group. The ring spans NBUF / GROUP slices.
    int lrow = r_begin, lslice = 0;  // next unit to load (group base row when K spans slices)
    auto load_next = [&](RowData<T>& dst, int r) {
        const int row = ONE_SLICE ? lrow : lrow + r % GROUP;
        const bool live_row = row < r_end;
        int mat, local;
        locate(live_row ? row : r_begin, mat, local);
        const __amdgpu_buffer_rsrc_t rs = pick_w(mat);
        const int b = lslice * 16 + bs;
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

    // ---- staging: x (times gamma) into per-group fixed point, in lane order.
    float ssq[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) ssq[m] = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int e = 4 * ((int)threadIdx.x + kThreads * c);
        const int slice = e / kSliceElems;
        int al, aw, ag;
        act_slot<T>(e - slice * kSliceElems, al, aw, ag);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float4 v = xv[m][c];
            if constexpr (SWIGLU) {
                // silu(gate) * up, in the reference's operation order (model_ops.rs:316-328)
                v.x = (v.x / (1.0f + expf(-v.x))) * uv[m][c].x;
                v.y = (v.y / (1.0f + expf(-v.y))) * uv[m][c].y;
                v.z = (v.z / (1.0f + expf(-v.z))) * uv[m][c].z;
                v.w = (v.w / (1.0f + expf(-v.w))) * uv[m][c].w;
            }
            if constexpr (NORM) {
                ssq[m] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                v.x *= gv[c].x;
                v.y *= gv[c].y;
                v.z *= gv[c].z;
                v.w *= gv[c].w;
            }
            const float gmax = group_max<T>(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            // gmax < 2^ex; groups below 2^-100 quantize to zero.
            int ex = gmax > 0.f ? __builtin_amdgcn_frexp_expf(gmax) : 0;
            ex = ex < -100 ? -100 : ex;
            const int sh = 15 - ex;
            int q[4];
            q[0] = (int)__builtin_rintf(__builtin_amdgcn_ldexpf(v.x, sh));
            q[1] = (int)__builtin_rintf(__builtin_amdgcn_ldexpf(v.y, sh));
            q[2] = (int)__builtin_rintf(__builtin_amdgcn_ldexpf(v.z, sh));
            q[3] = (int)__builtin_rintf(__builtin_amdgcn_ldexpf(v.w, sh));
            uint32_t hw = 0, lw = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                q[t] = q[t] > 32767 ? 32767 : q[t];  // rounding can reach 2^15
                hw |= ((uint32_t)(q[t] >> 8) & 0xffu) << (8 * t);
                lw |= ((uint32_t)q[t] & 0xffu) << (8 * t);
            }
            const int xsum = group_sum<T>(q[0] + q[1] + q[2] + q[3]);
            if (slice < slices) {
                uint32_t* dst = xs + ((m * slices + slice) * 64 + al) * STRIDE;
                dst[aw] = hw;
                dst[16 + aw] = lw;
                if ((lane & (ActTraits<T>::group / 4 - 1)) == 0) {
                    dst[32 + ag] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_ldexpf(1.0f, ex - 15));
                    dst[32 + G + ag] = (uint32_t)xsum;
                }
            }
        }
    }
    if constexpr (NORM) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float wsum = wave_sum_uniform(ssq[m]);
            if (lane == 0) partial[m][wave] = wsum;
        }
    }
    __syncthreads();

    float inv[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        inv[m] = 1.f;
        if constexpr (NORM) {
            float total = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) total += partial[m][w];
            // RMSNorm (qwen_reference.rs:550-556): x * (1/sqrt(sum(x^2)/K + eps)) * gamma
            inv[m] = 1.0f / sqrtf(total / (float)K + args.eps);
        }
    }

    // Output of one row: a store, or (args.accumulate) an add into y, which
    // fuses the residual connection (each row is added exactly once, so the
    // result is the same as a store followed by an elementwise add).
    const bool accumulate = args.accumulate != 0;
    auto put = [&](float value, __amdgpu_buffer_rsrc_t yr, uint32_t off) {
        if (accumulate) {
            __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(value, yr, (int)off, 0, 0);
        } else {
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, value), yr, (int)off, 0, 0);
        }
    };

    // silu(gate) * up of one output row, in the reference's operation order
    // (model_ops.rs:316-328)
    auto swiglu = [](float g, float u) { return (g / (1.0f + expf(-g))) * u; };

    // One member's lane record of one slice, from LDS.
    auto read_member = [&](LaneAct<T>& dst, int m, int slice) {
        const uint32_t* src = xs + ((m * slices + slice) * 64 + lane) * STRIDE;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 a = *reinterpret_cast<const uint4*>(src + 4 * i);
            const uint4 b = *reinterpret_cast<const uint4*>(src + 16 + 4 * i);
            dst.h[4 * i + 0] = a.x;
            dst.h[4 * i + 1] = a.y;
            dst.h[4 * i + 2] = a.z;
            dst.h[4 * i + 3] = a.w;
            dst.l[4 * i + 0] = b.x;
            dst.l[4 * i + 1] = b.y;
            dst.l[4 * i + 2] = b.z;
            dst.l[4 * i + 3] = b.w;
        }
        uint32_t prm[2 * G];
#pragma unroll
        for (int i = 0; i < 2 * G; i += 4) {
            const uint4 a = *reinterpret_cast<const uint4*>(src + 32 + i);
            prm[i] = a.x;
            prm[i + 1] = a.y;
            prm[i + 2] = a.z;
            prm[i + 3] = a.w;
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            dst.unscale[g] = __builtin_bit_cast(float, prm[g]);
            dst.xsum[g] = (float)(int)prm[G + g];
            dst.xsum32[g] = -32 * (int)prm[G + g];
        }
    };

    if constexpr (MT > 2) {
        // ---- many members (K within one slice): member records stay in LDS.
        // A pass runs over members (a real loop, one record live at a time):
        // each member's record is read once and dotted with every unit of the
        // ring, and its rows are reduced and stored at once; then the ring is
        // refilled. The per-member arithmetic is the single-member kernel's,
        // so each row is bit-identical to a one-member launch.
        static_assert(ONE_SLICE, "the member-serial form covers one slice");
        __shared__ float inv_s[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (threadIdx.x == m) inv_s[m] = inv[m];
        }
        __syncthreads();
        int crow = r_begin;
        auto pass = [&](auto refill_const, int left) {
            constexpr bool REFILL = decltype(refill_const)::value;
            int mat[NBUF], local[NBUF], rows_mat[NBUF];
            __amdgpu_buffer_rsrc_t yr[NBUF];
#pragma unroll
            for (int r = 0; r < NBUF; ++r) {
                const int row = crow + r;
                locate(row < r_end ? row : r_begin, mat[r], local[r]);
                yr[r] = pick_y(PAIR ? 0 : mat[r], rows_mat[r]);
            }
#pragma unroll 1
            for (int m = 0; m < members; ++m) {
                LaneAct<T> x1[1];
                read_member(x1[0], m, 0);
                const float im = inv_s[m];
                float gk = 0.f;
#pragma unroll
                for (int r = 0; r < NBUF; ++r) {
                    float pr[1];
                    row_dot<T, 1>(ring[r], p, x1, pr);
                    const float total = wave_sum_uniform(pr[0]) * im;
                    const bool live = r < left && crow + r < r_end;
                    const uint32_t off =
                        (live && lane == 0) ? (uint32_t)(m * rows_mat[r] + local[r]) * 4u : kOutOfRange;
                    if constexpr (PAIR) {
                        if (r % 2 == 0) {
                            gk = total;
                        } else {
                            put(swiglu(gk, total), yr[r], off);
                        }
                    } else {
                        put(total, yr[r], off);
                    }
                }
            }
            if constexpr (REFILL) {
#pragma unroll
                for (int r = 0; r < NBUF; ++r) load_next(ring[r], r);
            }
            crow += NBUF;
        };
        const int rows_w = r_end - r_begin;
        const int passes = (rows_w + NBUF - 1) / NBUF;
        for (int ps = 0; ps + 1 < passes; ++ps) pass(std::true_type{}, NBUF);
        if (passes > 0) pass(std::false_type{}, rows_w - (passes - 1) * NBUF);
        return;
    }

    LaneAct<T> xa[MT];
    auto read_act = [&](int slice) {
#pragma unroll
        for (int m = 0; m < MT; ++m) read_member(xa[m], m, slice);
    };
    if constexpr (ONE_SLICE) read_act(0);

    // ---- ring: reduce a unit, store its row when the unit completes it
    // (other stores go to an out-of-range offset and are dropped), refill the
    // slot with the unit NBUF ahead.
    int crow = r_begin, cslice = 0;  // unit being reduced (group base row when K spans slices)
    constexpr int kAcc = ONE_SLICE ? 1 : GROUP;
    float acc[kAcc][MT];
    float gk[MT];  // PAIR: the gate row's output, waiting for its up row
#pragma unroll
    for (int r = 0; r < kAcc; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;
    auto consume = [&](const RowData<T>& d, int r) {
        if constexpr (!ONE_SLICE) {
            if (r % GROUP == 0) read_act(cslice);
        }
        float part[MT];
        row_dot<T, MT>(d, p, xa, part);
        const int ai = ONE_SLICE ? 0 : r % GROUP;
        const int row = ONE_SLICE ? crow : crow + r % GROUP;
        const bool last = ONE_SLICE || cslice == slices - 1;
        int mat, local;
        locate(row < r_end ? row : r_begin, mat, local);
        int rows_mat;
        const __amdgpu_buffer_rsrc_t yr = pick_y(PAIR ? 0 : mat, rows_mat);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            acc[ai][m] = (ONE_SLICE || cslice == 0) ? part[m] : acc[ai][m] + part[m];
            const float total = wave_sum_uniform(acc[ai][m]) * inv[m];
            const uint32_t off = (last && row < r_end && lane == 0 && m < members)
                                     ? (uint32_t)(m * rows_mat + local) * 4u
                                     : kOutOfRange;
            if constexpr (PAIR) {
                // ring slots alternate gate / up rows (r_begin and NBUF are even)
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
    // Passes of NBUF units; a partial last group (K spanning slices) runs on
    // zero-filled loads and stores nothing.
    const int units = ONE_SLICE ? rows_w : (rows_w + GROUP - 1) / GROUP * GROUP * slices;
    const int passes = (units + NBUF - 1) / NBUF;
    for (int pass = 0; pass + 1 < passes; ++pass) {
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

// ---------------------------------------------------------------- launcher

// LDS of the activation records: [members][slices][64][stride] dwords.
template <int T>
static size_t act_lds_bytes(int members, int K) {
    const int slices = ((K >> 8) + 15) >> 4;
    return (size_t)members * slices * 64 * ActTraits<T>::stride * sizeof(uint32_t);
}

template <int T, int MT, int PRO, bool ONE_SLICE, int NBUF, int WAVES, int GROUP = 1, bool PAIR = false>
struct WaveInstance {
    static std::atomic<int> occupancy;  // resident workgroups per CU at the largest LDS size (0: not queried)
    // Launches `per_cu` workgroups on every CU (capped by occupancy; fewer
    // when the problem has fewer than two units per wave).
    static hipError_t launch(const WaveGemvArgs& a, int cu_count, int per_cu, hipStream_t stream) {
        auto kern = gemv_wave_kernel<T, MT, PRO, ONE_SLICE, NBUF, WAVES, GROUP, PAIR>;
        const size_t lds = act_lds_bytes<T>(MT, a.K);
        int occ = occupancy.load(std::memory_order_relaxed);
        if (occ == 0) {
            const int max_lds = (int)act_lds_bytes<T>(MT, ONE_SLICE ? kSliceElems : kWaveMaxK);
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
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(WAVES * 64), lds, stream, a);
        return hipGetLastError();
    }
};
template <int T, int MT, int PRO, bool ONE_SLICE, int NBUF, int WAVES, int GROUP, bool PAIR>
std::atomic<int> WaveInstance<T, MT, PRO, ONE_SLICE, NBUF, WAVES, GROUP, PAIR>::occupancy{0};

// Launch shape by units (row x slice) per CU, from sweeps on MI355X over
// workgroup size {2,4,8,16} waves x ring depth {2,4,8} x workgroups per CU
// {1,2,4}: short launches want every wave started at once with a shallow
// ring; long streams want fewer, deeper streams per CU.
template <int T, int MT, int PRO, bool ONE_SLICE, bool PAIR = false>
static hipError_t launch_ring(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    const int slices = ONE_SLICE ? 1 : ((a.K >> 8) + 15) >> 4;
    const long long units = (long long)a.total_rows * slices;
    const long long per_cu = (units + cu_count - 1) / cu_count;
    if constexpr (MT == 1 && ONE_SLICE) {
        if (per_cu >= 128) {
            if constexpr (T == kQ6K) {
                return WaveInstance<T, MT, PRO, ONE_SLICE, 8, 4, 1, PAIR>::launch(a, cu_count, 1, stream);
            }
            return WaveInstance<T, MT, PRO, ONE_SLICE, 4, 8, 1, PAIR>::launch(a, cu_count, 4, stream);
        }
    }
    if constexpr (!ONE_SLICE) {
        // K spanning slices: pairs of rows, slice by slice (deeper rings
        // measured slower for the 12288-wide down projection).
        return WaveInstance<T, MT, PRO, ONE_SLICE, 2, 8, 2>::launch(a, cu_count, 1, stream);
    } else {
        return WaveInstance<T, MT, PRO, ONE_SLICE, 2, 8, 1, PAIR>::launch(a, cu_count, per_cu > 48 ? 2 : 1, stream);
    }
}

template <int T, int MT, int PRO>
static hipError_t launch_tm(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    if (a.K <= kSliceElems) return launch_ring<T, MT, PRO, true>(a, cu_count, stream);
    return launch_ring<T, MT, PRO, false>(a, cu_count, stream);
}

template <int T, int PRO>
static hipError_t launch_t(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    if (a.members <= 1) return launch_tm<T, 1, PRO>(a, cu_count, stream);
    if (a.members <= 2 || a.K > kSliceElems) return launch_tm<T, 2, PRO>(a, cu_count, stream);
    if constexpr (PRO == kProSwiglu) {
        return hipErrorInvalidValue;  // the host splits SwiGLU launches into pairs of members
    } else {
        // 3..8 members: member-serial passes over a four-unit ring
        if (a.members <= 4) return WaveInstance<T, 4, PRO, true, 4, 8>::launch(a, cu_count, 1, stream);
        return WaveInstance<T, 8, PRO, true, 4, 8>::launch(a, cu_count, 1, stream);
    }
}

int wave_max_members(int K) {
    if (K > kWaveMaxK) return 0;
    const long long per_member = (long long)act_lds_bytes<kQ6K>(1, K);
    const long long fit = kWaveMaxLdsBytes / per_member;
    const long long cap = K <= kSliceElems ? kWaveMaxMembers : 2;  // many members: one slice only
    return (int)std::min<long long>(fit, cap);
}

// Gate/up pairs with the SwiGLU epilogue (one-slice K; members as launch_t).
template <int T, int PRO>
static hipError_t launch_pair(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    if (a.members <= 1) return launch_ring<T, 1, PRO, true, true>(a, cu_count, stream);
    if (a.members <= 2) return launch_ring<T, 2, PRO, true, true>(a, cu_count, stream);
    if (a.members <= 4) return WaveInstance<T, 4, PRO, true, 4, 8, 1, true>::launch(a, cu_count, 1, stream);
    return WaveInstance<T, 8, PRO, true, 4, 8, 1, true>::launch(a, cu_count, 1, stream);
}

template <int T>
static hipError_t launch_type(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    if (a.pair_swiglu) {
        if (a.x2 != nullptr || a.count != 2 || a.rows_end[1] != 2 * a.rows_end[0] || a.K > kSliceElems) {
            return hipErrorInvalidValue;
        }
        return a.gamma != nullptr ? launch_pair<T, kProNorm>(a, cu_count, stream)
                                  : launch_pair<T, kProPlain>(a, cu_count, stream);
    }
    if (a.x2 != nullptr) {
        if (a.gamma != nullptr || a.members > kSwigluMaxMembers) return hipErrorInvalidValue;
        return launch_t<T, kProSwiglu>(a, cu_count, stream);
    }
    if (a.gamma != nullptr) return launch_t<T, kProNorm>(a, cu_count, stream);
    return launch_t<T, kProPlain>(a, cu_count, stream);
}

hipError_t launch_gemv_wave(int value_type, const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    switch (value_type) {
    case kQ4K: return launch_type<kQ4K>(a, cu_count, stream);
    case kQ5K: return launch_type<kQ5K>(a, cu_count, stream);
    case kQ6K: return launch_type<kQ6K>(a, cu_count, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace ribn_amd

// Wave GEMV for Q4_K / Q5_K / Q6_K on gfx950 (CDNA4, wave64): the decode
// path's bandwidth kernel, with an optional fused RMSNorm prologue and a
// grouped form that streams several weights sharing one activation vector
// (q/k/v, gate/up) in a single launch.
//
// Layout and mapping
//  - Weights are the encoded GGML array-of-blocks; row n of a [K, N] tensor is
//    K/256 consecutive super-blocks (crates/nvidia/src/quantized.rs:136-142).
//  - A workgroup is 8 waves. It stages the activations [members][K] once into
//    LDS (scaled by inv_rms * gamma when RMSNorm is fused), then each wave
//    streams a contiguous range of output rows.
//  - A wave covers 16 consecutive super-blocks of a row per "slice"; lane l owns
//    block (l >> 2) of the slice and quarter p = (l & 3), i.e. 64 elements:
//      Q4_K / Q5_K: groups 2p and 2p+1 (payload bytes 32p..32p+31, low/high nibbles);
//      Q6_K:        groups 4c..4c+3 at positions 16s..16s+15 (c = p >> 1, s = p & 1).
//  - Per row a lane issues 128-bit buffer loads for its payload and header,
//    forms sum(q*x) per scale group in f32 and applies (d*sc) and (dmin*m) once
//    per group: y = sum_g (d*sc_g)*sum(q*x) - (dmin*m_g)*sum(x).
//  - Weight loads for the next rows are issued before the current rows are
//    reduced (one-deep software pipeline), and the first rows' loads are issued
//    before the activation staging, so HBM latency overlaps the prologue.
// Arithmetic per member is independent of the member count, so every row of a
// batched launch is bit-identical to the single-member launch.
#include "kquant_device.hpp"
#include "kquant_launch.hpp"

namespace ribn_amd {

constexpr int kWaves = 8;          // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kRows = 2;           // rows per pipeline stage

struct LaneX {
    float v[64];
};

__device__ __forceinline__ float4 ld_f4(const float* p) { return *reinterpret_cast<const float4*>(p); }

__device__ __forceinline__ float ubyte_f(uint32_t w, int t) { return (float)((w >> (8 * t)) & 0xffu); }

// Offset within a super-block of lane-local activation j (0..63).
template <int T>
__device__ __forceinline__ int lane_x_offset(int p, int j) {
    if constexpr (T == kQ6K) {
        return 128 * (p >> 1) + 32 * (j >> 4) + 16 * (p & 1) + (j & 15);
    } else {
        return 64 * p + j;
    }
}

// ----------------------------------------------------------- raw row loads

template <int T> struct RowData;
template <> struct RowData<kQ4K> { uint4 h, qa, qb; };
template <> struct RowData<kQ5K> { uint4 h, ha, hb, qa, qb; };
template <> struct RowData<kQ6K> {
    uint4 la, lb, qh, sc;       // dword-aligned-down 16-byte windows
    uint32_t la_t, lb_t, qh_t, sc_t;  // the dword after each window
    uint32_t d16, shift;
};

template <int T>
__device__ __forceinline__ void zero_row(RowData<T>& d) {
    d = RowData<T>{};
}

template <int T>
__device__ __forceinline__ void load_row(RowData<T>& d, __amdgpu_buffer_rsrc_t r, uint32_t off, int p) {
    if constexpr (T == kQ4K) {
        d.h = load_b128(r, off);
        d.qa = load_b128(r, off + 16 + 32 * p);
        d.qb = load_b128(r, off + 32 + 32 * p);
    } else if constexpr (T == kQ5K) {
        d.h = load_b128(r, off);
        d.ha = load_b128(r, off + 16);
        d.hb = load_b128(r, off + 32);
        d.qa = load_b128(r, off + 48 + 32 * p);
        d.qb = load_b128(r, off + 64 + 32 * p);
    } else {
        // 210-byte blocks: offsets are 2-byte aligned; every field of a lane
        // shares the same misalignment, resolved with funnel shifts later.
        const int c = p >> 1, s = p & 1;
        const uint32_t base = off & ~3u;
        d.shift = (off & 3u) * 8u;
        const uint32_t la = base + 64 * c + 16 * s;
        const uint32_t lb = la + 32;
        const uint32_t qh = base + 128 + 32 * c + 16 * s;
        const uint32_t sc = base + 192;
        d.la = load_b128(r, la);
        d.la_t = load_b32(r, la + 16);
        d.lb = load_b128(r, lb);
        d.lb_t = load_b32(r, lb + 16);
        d.qh = load_b128(r, qh);
        d.qh_t = load_b32(r, qh + 16);
        d.sc = load_b128(r, sc);
        d.sc_t = load_b32(r, sc + 16);
        // d by a 16-bit load: a dword could straddle the end of the tensor,
        // and an out-of-range dword reads back as zero.
        d.d16 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)(off + 208), 0, kStreamPolicy);
    }
}

__device__ __forceinline__ uint4 funnel(uint4 a, uint32_t t, uint32_t sh) {
    uint4 o;
    o.x = __builtin_amdgcn_alignbit(a.y, a.x, sh);
    o.y = __builtin_amdgcn_alignbit(a.z, a.y, sh);
    o.z = __builtin_amdgcn_alignbit(a.w, a.z, sh);
    o.w = __builtin_amdgcn_alignbit(t, a.w, sh);
    return o;
}

// --------------------------------------------------- per-row dot products

template <int T, int MT>
__device__ __forceinline__ void row_dot(const RowData<T>& d, int p, const LaneX (&xa)[MT],
                                        const float (&gsum)[MT][4], float (&acc)[MT]) {
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
        float q0[32], q1[32];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t lo = qw[j] & 0x0f0f0f0fu;
            uint32_t hi = (qw[j] >> 4) & 0x0f0f0f0fu;
            if constexpr (T == kQ5K) {
                const uint32_t hw[8] = {d.ha.x, d.ha.y, d.ha.z, d.ha.w, d.hb.x, d.hb.y, d.hb.z, d.hb.w};
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
                s0 = __builtin_fmaf(q0[i], xa[m].v[i], s0);
                s1 = __builtin_fmaf(q1[i], xa[m].v[32 + i], s1);
            }
            float a = acc[m];
            a = __builtin_fmaf(a0, s0, a);
            a = __builtin_fmaf(-b0, gsum[m][0], a);
            a = __builtin_fmaf(a1, s1, a);
            a = __builtin_fmaf(-b1, gsum[m][1], a);
            acc[m] = a;
        }
    } else {
        const int c = p >> 1, s = p & 1;
        const uint32_t sh = d.shift;
        const uint4 la = funnel(d.la, d.la_t, sh);
        const uint4 lb = funnel(d.lb, d.lb_t, sh);
        const uint4 qh = funnel(d.qh, d.qh_t, sh);
        const uint4 sc = funnel(d.sc, d.sc_t, sh);  // int8 scales 0..15
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
                for (int i = 0; i < 16; ++i) sv = __builtin_fmaf(q[v][i], xa[m].v[16 * v + i], sv);
                // sum((q - 32) * x) = sum(q*x) - 32 * sum(x)
                accm = __builtin_fmaf(a[v], sv, accm);
                accm = __builtin_fmaf(-32.f * a[v], gsum[m][v], accm);
            }
            acc[m] = accm;
        }
    }
}

// ------------------------------------------------------------------ kernel

template <int T, int MT, bool NORM, bool ONE_SLICE>
__global__ __launch_bounds__(kThreads) void gemv_wave_kernel(WaveGemvArgs args) {
    constexpr int BB = BlockTraits<T>::bytes;
    extern __shared__ float xs[];  // [MT][K] staged activations
    __shared__ float partial[MT][kWaves];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = args.K;
    const int nb = K >> 8;
    const int slices = (nb + 15) >> 4;
    const int p = lane & 3;
    const int bs = lane >> 2;
    const int nwaves = gridDim.x * kWaves;
    const int wg = blockIdx.x * kWaves + wave;
    const int r_begin = (int)((long long)args.total_rows * wg / nwaves);
    const int r_end = (int)((long long)args.total_rows * (wg + 1) / nwaves);
    const int row_blocks = (r_end - r_begin + kRows - 1) / kRows;
    const int items = row_blocks * slices;
    const uint32_t row_bytes = (uint32_t)nb * BB;

    // Row -> (matrix, local row); the row index is wave-uniform.
    auto locate = [&](int row, int& mat, int& local) {
        mat = 0;
#pragma unroll
        for (int i = 0; i < kMaxGroup - 1; ++i) {
            if (i + 1 < args.count && row >= args.rows_end[i]) mat = i + 1;
        }
        local = row - (mat ? args.rows_end[mat - 1] : 0);
    };

    auto load_item = [&](RowData<T> (&dst)[kRows], int it) {
        const int rb = it / slices;
        const int s = it - rb * slices;
        const int b = s * 16 + bs;
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const int row = r_begin + rb * kRows + r;
            zero_row<T>(dst[r]);
            if (row < r_end) {
                int mat, local;
                locate(row, mat, local);
                const __amdgpu_buffer_rsrc_t rs = make_rsrc(args.w[mat], args.wbytes[mat]);
                if (b < nb) load_row<T>(dst[r], rs, (uint32_t)local * row_bytes + (uint32_t)b * BB, p);
            }
        }
    };

    RowData<T> cur[kRows];
    if (items > 0) load_item(cur, 0);

    // ---- stage activations [members][K] into LDS (normalised when fused)
    const int members = args.members;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        float ssq = 0.f;
        for (int k = threadIdx.x * 4; k < K; k += kThreads * 4) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < members) v = ld_f4(args.x + (size_t)m * K + k);
            *reinterpret_cast<float4*>(&xs[m * K + k]) = v;
            if constexpr (NORM) ssq += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        if constexpr (NORM) {
            ssq = wave_sum(ssq);
            if (lane == 0) partial[m][wave] = ssq;
        }
    }
    if constexpr (NORM) {
        __syncthreads();
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float total = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) total += partial[m][w];
            // RMSNorm (qwen_reference.rs:550-556): x * (1/sqrt(sum(x^2)/K + eps)) * gamma
            const float inv = 1.0f / sqrtf(total / (float)K + args.eps);
            for (int k = threadIdx.x * 4; k < K; k += kThreads * 4) {
                float4 v = *reinterpret_cast<float4*>(&xs[m * K + k]);
                const float4 g = ld_f4(args.gamma + k);
                v.x = v.x * inv * g.x;
                v.y = v.y * inv * g.y;
                v.z = v.z * inv * g.z;
                v.w = v.w * inv * g.w;
                *reinterpret_cast<float4*>(&xs[m * K + k]) = v;
            }
        }
    }
    __syncthreads();

    LaneX xa[MT];
    float gsum[MT][4];
    auto load_x = [&](int s) {
        const int b = s * 16 + bs;
        const bool valid = b < nb;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float* src = xs + m * K + b * 256;
#pragma unroll
            for (int j = 0; j < 64; j += 4) {
                const float4 v = valid ? *reinterpret_cast<const float4*>(src + lane_x_offset<T>(p, j))
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
                xa[m].v[j] = v.x;
                xa[m].v[j + 1] = v.y;
                xa[m].v[j + 2] = v.z;
                xa[m].v[j + 3] = v.w;
            }
            constexpr int NG = (T == kQ6K) ? 4 : 2;
            constexpr int GS = 64 / NG;
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                float sum = 0.f;
#pragma unroll
                for (int j = 0; j < GS; ++j) sum += xa[m].v[g * GS + j];
                gsum[m][g] = sum;
            }
        }
    };
    if constexpr (ONE_SLICE) load_x(0);

    float acc[kRows][MT];
    for (int it = 0; it < items; ++it) {
        RowData<T> nxt[kRows];
        if (it + 1 < items) load_item(nxt, it + 1);
        const int rb = it / slices;
        const int s = it - rb * slices;
        if constexpr (!ONE_SLICE) load_x(s);
        if (s == 0) {
#pragma unroll
            for (int r = 0; r < kRows; ++r)
#pragma unroll
                for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r) row_dot<T, MT>(cur[r], p, xa, gsum, acc[r]);
        if (s == slices - 1) {
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                const int row = r_begin + rb * kRows + r;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const float total = wave_sum(acc[r][m]);
                    if (row < r_end && m < members && lane == 0) {
                        int mat, local;
                        locate(row, mat, local);
                        const int rows_mat = args.rows_end[mat] - (mat ? args.rows_end[mat - 1] : 0);
                        args.y[mat][(size_t)m * rows_mat + local] = total;
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r) cur[r] = nxt[r];
    }
}

// ---------------------------------------------------------------- launcher

template <int T, int MT, bool NORM>
static hipError_t launch_tm(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    const size_t lds = (size_t)MT * a.K * sizeof(float);
    const int min_rows_per_wave = 2;
    int grid = (a.total_rows + kWaves * min_rows_per_wave - 1) / (kWaves * min_rows_per_wave);
    const int max_grid = cu_count * 2;
    if (grid > max_grid) grid = max_grid;
    if (grid < 1) grid = 1;
    if ((a.K >> 8) <= 16) {
        auto kern = gemv_wave_kernel<T, MT, NORM, true>;
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), lds, stream, a);
    } else {
        auto kern = gemv_wave_kernel<T, MT, NORM, false>;
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), lds, stream, a);
    }
    return hipGetLastError();
}

template <int T, bool NORM>
static hipError_t launch_t(const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    if (a.members <= 1) return launch_tm<T, 1, NORM>(a, cu_count, stream);
    if (a.members <= 2) return launch_tm<T, 2, NORM>(a, cu_count, stream);
    return launch_tm<T, 4, NORM>(a, cu_count, stream);
}

int wave_max_members(int K) {
    const long long fit = kWaveMaxLdsBytes / ((long long)K * (long long)sizeof(float));
    if (fit >= 4) return 4;
    if (fit >= 2) return 2;
    return fit >= 1 ? 1 : 0;
}

hipError_t launch_gemv_wave(int value_type, const WaveGemvArgs& a, int cu_count, hipStream_t stream) {
    const bool norm = a.gamma != nullptr;
    switch (value_type) {
    case kQ4K: return norm ? launch_t<kQ4K, true>(a, cu_count, stream) : launch_t<kQ4K, false>(a, cu_count, stream);
    case kQ5K: return norm ? launch_t<kQ5K, true>(a, cu_count, stream) : launch_t<kQ5K, false>(a, cu_count, stream);
    case kQ6K: return norm ? launch_t<kQ6K, true>(a, cu_count, stream) : launch_t<kQ6K, false>(a, cu_count, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace ribn_amd

// Row loads shared by the wave GEMVs (gemv_wave.hip: block fixed-point
// activations; gemv_f32.hip: f32 activations). A wave covers 16 consecutive
// super-blocks of a row per "slice"; lane l owns block (l >> 2) of the slice
// and quarter p = (l & 3) of it, i.e. 64 weights:
//   Q4_K / Q5_K: groups 2p and 2p+1 (payload bytes 32p..32p+31, low / high nibbles);
//   Q6_K:        the 16-element groups 8c+2v+s, v = 0..3 (c = p >> 1, s = p & 1).
// Weights are read through buffer resources sized to the tensor, so offsets
// past the end (including kOutOfRange) read zeros instead of faulting.
#pragma once

#include "kquant_device.hpp"
#include "kquant_launch.hpp"

namespace ribn_amd {

constexpr uint32_t kOutOfRange = 0xffffff00u;  // buffer offset past any tensor: loads return 0, stores drop
constexpr int kSliceElems = kSliceK;           // elements a wave covers per unit (16 super-blocks)

// Activations are read by every workgroup: default cache policy, so they stay in L2.
__device__ __forceinline__ float4 load_f4(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)offset, 0, 0));
}

// ----------------------------------------------------------- raw row loads

template <int T> struct RowData;
template <> struct RowData<kQ4K> { uint4 h, qa, qb; };
template <> struct RowData<kQ5K> { uint4 h, ha, hb, qa, qb; };
template <> struct RowData<kQ6K> {
    uint4 la, lb, qh, sc;             // dword-aligned-down 16-byte windows
    uint32_t la_t, lb_t, qh_t, sc_t;  // the dword after each window
    uint32_t d16, shift;
};

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

}  // namespace ribn_amd

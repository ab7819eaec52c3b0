// Device-side helpers shared by the k-quant kernels (gfx950 / CDNA4, wave64).
//
// Block layouts are GGML's (the reference decodes them in
// crates/gguf/src/lib.rs:596-661); weights stay in the encoded
// array-of-blocks form they were uploaded in, so the device bytes round-trip
// to the host unchanged.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ribn_amd {

constexpr int kQ4K = 12;
constexpr int kQ5K = 13;
constexpr int kQ6K = 14;
constexpr int kQK = 256;  // elements per super-block

template <int T> struct BlockTraits;
template <> struct BlockTraits<kQ4K> { static constexpr int bytes = 144; };
template <> struct BlockTraits<kQ5K> { static constexpr int bytes = 176; };
template <> struct BlockTraits<kQ6K> { static constexpr int bytes = 210; };

// binary16 -> binary32 with the hardware convert (exact for every non-NaN
// pattern; the host decoder canonicalises NaN payloads, lib.rs:558).
__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// Buffer resource over a byte range: loads past num_records return zero
// instead of faulting, which bounds every weight read by the tensor size.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    // dword 3 = 0x00020000: raw (untyped) 32-bit data format on gfx9-family parts.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Cache-policy bits for streamed weights. The non-temporal hint (nt = 2)
// speeds up a purely contiguous stream, but the GEMV's block-strided loads
// touch each 128-byte line from several instructions and lose those re-hits
// under it, so weights use the default policy.
constexpr int kStreamPolicy = 0;

__device__ __forceinline__ uint4 load_b128(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)offset, 0, kStreamPolicy));
}

__device__ __forceinline__ uint32_t load_b32(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)offset, 0, kStreamPolicy);
}

// 16 bytes at a 2-byte-aligned offset: two dword-aligned loads and a funnel
// shift (Q6_K's 210-byte blocks leave odd blocks 2 bytes off dword alignment).
__device__ __forceinline__ uint4 load_16_at_half_aligned(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    const uint32_t base = offset & ~3u;
    const uint32_t shift = (offset & 3u) * 8u;
    const uint4 a = load_b128(r, base);
    const uint32_t e = load_b32(r, base + 16u);
    uint4 out;
    out.x = __builtin_amdgcn_alignbit(a.y, a.x, shift);
    out.y = __builtin_amdgcn_alignbit(a.z, a.y, shift);
    out.z = __builtin_amdgcn_alignbit(a.w, a.z, shift);
    out.w = __builtin_amdgcn_alignbit(e, a.w, shift);
    return out;
}

__device__ __forceinline__ uint32_t byte_of(uint32_t word, int index) {
    return (word >> (8 * index)) & 0xffu;
}

// Six-bit scale / minimum of group g from the 12 packed bytes (a2 in the
// reference: lib.rs:573-587). s0..s2 are scale bytes 0-3, 4-7, 8-11.
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int g,
                                              uint32_t& sc, uint32_t& mn) {
    if (g < 4) {
        sc = byte_of(s0, g) & 63u;
        mn = byte_of(s1, g) & 63u;
    } else {
        const int j = g - 4;
        sc = (byte_of(s2, j) & 15u) | ((byte_of(s0, j) >> 2) & 0x30u);
        mn = (byte_of(s2, j) >> 4) | ((byte_of(s1, j) >> 2) & 0x30u);
    }
}

// DPP row-local reduction (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
// row_mirror) leaves each 16-lane row's sum in all its lanes; four readlanes
// add the rows. The result is wave-uniform and needs no LDS round trip.
template <int CTRL>
__device__ __forceinline__ float dpp_step(float v) {
    const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false);
    return v + __builtin_bit_cast(float, moved);
}

__device__ __forceinline__ float wave_sum_uniform(float v) {
    v = dpp_step<0xb1>(v);   // quad_perm [1,0,3,2]
    v = dpp_step<0x4e>(v);   // quad_perm [2,3,0,1]
    v = dpp_step<0x141>(v);  // row_half_mirror
    v = dpp_step<0x140>(v);  // row_mirror
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

template <int CTRL>
__device__ __forceinline__ float dpp_max_step(float v) {
    const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false);
    return fmaxf(v, __builtin_bit_cast(float, moved));
}

// Sum across the 64 lanes of a wave; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        v += __shfl_xor(v, offset, 64);
    }
    return v;
}

}  // namespace ribn_amd

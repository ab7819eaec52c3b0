// Decode-step kernels for gfx950 (CDNA4, wave64) around the k-quant GEMVs.
//
// attn_decode_kernel: one layer's attention for a batch of decode members.
// It fuses what the reference runs as five launches per layer
// (crates/nvidia/src/decode.rs:929-1034):
//   per-head q/k RMSNorm       strided_rms_norm / q_gate_norm (model_ops.rs:660-685,1009-1041)
//   NEOX rope of q and k       rope_neox (model_ops.rs:393-425)
//   f16 append of the new K/V  kv_append_f16 (model_ops.rs:1256-1275)
//   GQA attention              attn_score_gqa (model_ops.rs:430-566)
// Qwen3 has no q gate, so the attention output is not gated.
//
// Work split (split-T "flash decoding"): the grid is (chunk, KV head,
// member). A workgroup takes one contiguous chunk (at least min_chunk tokens,
// at most the launch's grid chunks per context) of the member's tokens for one KV
// head and all q_per_kv query heads that share it, so each K/V byte is read
// once; workgroups past the context exit. Within the workgroup a 16-lane row
// of a wave owns one token per step (lane j of the row holds dims 8j..8j+7:
// one 16-byte load of K and one of V, kRing steps in flight), and keeps an
// online-softmax state (running max, denominator and output sums) per query
// head, rescaled once per kRing-step block, with scores in log2 units so each
// weight is one exp2. The 16 row states of a workgroup meet in LDS and are
// merged, in row order, into one partial per
// (chunk, head); attn_combine_kernel then merges the chunks' partials of each
// (member, head) into the output (for a context within one chunk it divides
// the one partial by its denominator). The new token's K/V are computed by the
// workgroup whose chunk holds the position: written to the cache, and used
// from LDS by that workgroup. For consecutive tokens of one sequence (a
// prefill chunk) kv_append_kernel stores every member's K/V first and the
// attention launch reads them all from the cache ("appended"), with the same
// values.
//
// Cache descriptors, positions and token ids are device memory, so one
// captured step serves every set of caches and positions; step_inputs_kernel
// writes them in stream order from its kernel arguments.
//
// argmax_slice_kernel + argmax_final_kernel: greedy selection (argmax,
// model_ops.rs:201-258) with the same ordering key, tie rule and NaN rule.
#include "decode_launch.hpp"
#include "kquant_device.hpp"

#include <float.h>

#include <algorithm>

namespace ribn_amd {

namespace {

constexpr uint32_t kOOR = 0xffffff00u;  // buffer offset past any cache: loads return 0
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRing = 4;                  // steps of K/V loads in flight per wave
constexpr int kStepTokens = kWaves * 4;   // tokens a workgroup covers per step
constexpr int kRows = kWaves * 4;         // 16-lane rows of a workgroup, one softmax state each
// A chunk spans at least this many tokens in launches of up to 8 members
// (sweep on MI355X over workgroups of 256/512 threads and 16-256-token minimum
// chunks: batch 1 at 2048 tokens is fastest here, and short contexts need
// fewer chunks and merges), and kMinChunkTokensWide from 9 members, whose
// grids of 64-token chunks run in several rounds (2,048 workgroups at 16
// members and 2,048 tokens): batch-16 decode 3,550 -> 3,730 tok/s, where the
// same chunks at batch 1 cost 1.2%. From 9 members the projections run on
// the matrix cores and agree with single rows to f32 rounding, so the
// bit-for-bit lane (up to 8 members) keeps the 64-token chunks.
constexpr int kMinChunkTokens = 64;
constexpr int kMinChunkTokensWide = 128;
static_assert(kMinChunkTokens % kStepTokens == 0 && kMinChunkTokensWide % kStepTokens == 0,
              "chunks are whole steps");

constexpr int kBitLaneMembers = 8;  // the batch GEMVs' bit-identity lane (f32 wave GEMV)
int attn_min_chunk(int members) { return members > kBitLaneMembers ? kMinChunkTokensWide : kMinChunkTokens; }

// Tokens per chunk for a context of `tokens` in a launch of `chunks` grid
// chunks: min_chunk, or more when the context needs more than `chunks` chunks
// of that size.
__device__ __forceinline__ int chunk_tokens(int tokens, int chunks, int min_chunk) {
    int len = (tokens + chunks - 1) / chunks;
    len = len < min_chunk ? min_chunk : len;
    return (len + kStepTokens - 1) / kStepTokens * kStepTokens;
}

// Sum over the 16 lanes of a DPP row; every lane of the row receives it.
__device__ __forceinline__ float row16_sum(float v) {
    v = dpp_step<0xb1>(v);   // quad_perm [1,0,3,2]
    v = dpp_step<0x4e>(v);   // quad_perm [2,3,0,1]
    v = dpp_step<0x141>(v);  // row_half_mirror
    v = dpp_step<0x140>(v);  // row_mirror
    return v;
}

__device__ __forceinline__ void unpack_f16x8(uint4 w, float (&f)[8]) {
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = half_bits_to_float(a[i] & 0xffffu);
        f[2 * i + 1] = half_bits_to_float(a[i] >> 16);
    }
}

// NEOX rope angle of lane l's pair (l, l + 64): pos * base^(-2l/128)
// (model_ops.rs:393-425). The frequency does not depend on the position, so a
// kernel computes it while the position is still in flight; every head of a
// lane shares the angle, so its sine and cosine are computed once.
__device__ __forceinline__ float rope_freq(float base, int lane) {
    return powf(base, -(2.0f * (float)lane) / (float)kHeadDim);
}

struct Rot {
    float s, c;
};

__device__ __forceinline__ Rot rope_rot(float pos, float freq) {
    Rot r;
    sincosf(pos * freq, &r.s, &r.c);
    return r;
}

// One 128-wide head held by a wave as lane l: x0 = dim l, x1 = dim l + 64.
// RMSNorm with the shared per-head weight (x * inv * w, model_ops.rs:660-685),
// then the rotation of the pair (l, l + 64) by the lane's angle.
__device__ __forceinline__ void norm_rope(float& x0, float& x1, float w0, float w1, float eps, Rot r) {
    const float ssq = wave_sum(x0 * x0 + x1 * x1);
    const float inv = 1.0f / sqrtf(ssq / (float)kHeadDim + eps);
    const float y0 = x0 * inv * w0;
    const float y1 = x1 * inv * w1;
    x0 = y0 * r.c - y1 * r.s;
    x1 = y0 * r.s + y1 * r.c;
}

template <int QPK>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(AttnArgs a) {
    constexpr int kHeadsPerWave = (QPK + kWaves - 1) / kWaves;
    __shared__ float qs[QPK][kHeadDim];
    __shared__ float kv_new[2][kHeadDim];
    __shared__ float2 st_ml[kRows][QPK];  // each row's running maximum and denominator
    __shared__ float st_o[kRows][QPK][kHeadDim];

    const int chunk = blockIdx.x;
    const int kvh = blockIdx.y;
    const int m = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = lane >> 4;  // token slot of this lane's row
    const int j = lane & 15;    // dims 8j..8j+7
    // the member's descriptor and position: two scalar loads, waited for
    // together below
    const AttnMember mb = a.mem[m];
    const int pos = a.positions[m];

    // ---- work that does not need them goes first: this workgroup's query
    // heads and norm weight, the new token's raw K (wave 0) and V (wave 1)
    // with the K norm weight, and the lane's rope frequency
    const float* qm = a.q + ((size_t)m * a.q_heads + (size_t)kvh * QPK) * kHeadDim;
    float qx[kHeadsPerWave][2];
#pragma unroll
    for (int i = 0; i < kHeadsPerWave; ++i) {
        const int h = wave + kWaves * i;
        qx[i][0] = qx[i][1] = 0.f;
        if (h < QPK) {
            qx[i][0] = qm[h * kHeadDim + lane];
            qx[i][1] = qm[h * kHeadDim + 64 + lane];
        }
    }
    const float qw0 = a.q_norm[lane];
    const float qw1 = a.q_norm[lane + 64];
    const float freq = rope_freq(a.rope_base, lane);
    float nx0 = 0.f, nx1 = 0.f, kw0 = 0.f, kw1 = 0.f;
    if (wave < 2) {
        const float* src = (wave == 0 ? a.k : a.v) + ((size_t)m * a.kv_heads + kvh) * kHeadDim;
        nx0 = src[lane];
        nx1 = src[lane + 64];
        if (wave == 0) {
            kw0 = a.k_norm[lane];
            kw1 = a.k_norm[lane + 64];
        }
    }

    // Both scalar loads are needed from here on; without this use the compiler
    // sinks the descriptor's load past the early exit below and waits twice.
    asm volatile("" ::"s"(mb.keys), "s"(mb.values), "s"(mb.partials), "s"(mb.layer_elems), "s"(mb.capacity),
                 "s"(pos), "v"(freq));
    uint16_t* const keys = mb.keys + (size_t)a.layer * mb.layer_elems;
    uint16_t* const values = mb.values + (size_t)a.layer * mb.layer_elems;
    const int tokens = pos + 1;
    const int len = chunk_tokens(tokens, a.chunks, a.min_chunk);
    const int t0 = chunk * len;
    if (t0 >= tokens) return;  // no tokens in this chunk (uniform over the workgroup)
    const int t1 = min(t0 + len, tokens);
    const int steps = (t1 - t0 + kStepTokens - 1) / kStepTokens;
    const bool has_new = !a.appended && pos < t1;

    // ---- cached K/V of this chunk: the first kRing steps are issued before
    // anything else. Unless appended, the new token's slot is not read (it is
    // written below).
    const size_t head_elems = (size_t)mb.capacity * kHeadDim;
    const uint32_t head_bytes = (uint32_t)(head_elems * 2u);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(keys + (size_t)kvh * head_elems, head_bytes);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(values + (size_t)kvh * head_elems, head_bytes);
    uint4 kring[kRing], vring[kRing];
    auto issue = [&](int r, int s) {
        const int t = t0 + s * kStepTokens + 4 * wave + grp;
        const bool live = s < steps && t < t1 && (a.appended || t != pos);
        const uint32_t off = live ? ((uint32_t)t * kHeadDim + 8u * (uint32_t)j) * 2u : kOOR;
        kring[r] = load_b128(kr, off);
        vring[r] = load_b128(vr, off);
    };
#pragma unroll
    for (int r = 0; r < kRing; ++r) issue(r, r);

    // ---- query heads (and the new K/V): norm + rope into LDS
    const bool new_wave = has_new && wave < 2;  // wave 0: K, wave 1: V
    const Rot rot = rope_rot((float)pos, freq);
#pragma unroll
    for (int i = 0; i < kHeadsPerWave; ++i) {
        const int h = wave + kWaves * i;
        if (h < QPK) {
            norm_rope(qx[i][0], qx[i][1], qw0, qw1, a.eps, rot);
            qs[h][lane] = qx[i][0];
            qs[h][lane + 64] = qx[i][1];
        }
    }
    if (new_wave) {
        if (wave == 0) norm_rope(nx0, nx1, kw0, kw1, a.eps, rot);
        // f16 round to nearest even, as kv_append_f16 stores it
        const _Float16 h0 = (_Float16)nx0;
        const _Float16 h1 = (_Float16)nx1;
        if (pos < mb.capacity) {
            uint16_t* dst = (wave == 0 ? keys : values) + (size_t)kvh * head_elems + (size_t)pos * kHeadDim;
            dst[lane] = __builtin_bit_cast(uint16_t, h0);
            dst[lane + 64] = __builtin_bit_cast(uint16_t, h1);
        }
        kv_new[wave][lane] = (float)h0;
        kv_new[wave][lane + 64] = (float)h1;
    }
    __syncthreads();

    float qr[QPK][8];
#pragma unroll
    for (int h = 0; h < QPK; ++h)
#pragma unroll
        for (int i = 0; i < 8; ++i) qr[h][i] = qs[h][8 * j + i];

    // ---- online softmax over the chunk (the reference's running max and
    // rescaled total, model_ops.rs:508-523, extended to the output sums), one
    // block of kRing steps at a time: the block's scores first, then one
    // maximum and one rescale per block. Scores are kept in log2 units
    // (a.scale carries log2 e), so each weight is one v_exp_f32.
    float mrun[QPK], lrun[QPK], o[QPK][8];
#pragma unroll
    for (int h = 0; h < QPK; ++h) {
        mrun[h] = -FLT_MAX;
        lrun[h] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[h][i] = 0.f;
    }
    for (int s0 = 0; s0 < steps; s0 += kRing) {
        // Steps past the chunk are skipped (uniform guards). One of them can
        // cover the new token's position, whose K/V live in kv_new only in the
        // workgroup whose chunk holds it; anywhere else that LDS is
        // uninitialised, and even a zero weight times a NaN left there is NaN.
        const int nr = steps - s0 < kRing ? steps - s0 : kRing;
        float sc[kRing][QPK];
#pragma unroll
        for (int r = 0; r < kRing; ++r) {
#pragma unroll
            for (int h = 0; h < QPK; ++h) sc[r][h] = -INFINITY;
            if (r >= nr) continue;
            const int t = t0 + (s0 + r) * kStepTokens + 4 * wave + grp;
            const bool live = t < t1;
            float kf[8];
            unpack_f16x8(kring[r], kf);
            if (has_new && t == pos) {
#pragma unroll
                for (int i = 0; i < 8; ++i) kf[i] = kv_new[0][8 * j + i];
            }
#pragma unroll
            for (int h = 0; h < QPK; ++h) {
                float d = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) d = __builtin_fmaf(qr[h][i], kf[i], d);
                d = row16_sum(d);
                sc[r][h] = live ? d * a.scale : -INFINITY;
            }
        }
#pragma unroll
        for (int h = 0; h < QPK; ++h) {
            float mb = sc[0][h];
#pragma unroll
            for (int r = 1; r < kRing; ++r) mb = fmaxf(mb, sc[r][h]);
            const float mn = fmaxf(mrun[h], mb);
            const float c = __builtin_amdgcn_exp2f(mrun[h] - mn);
            lrun[h] *= c;
#pragma unroll
            for (int i = 0; i < 8; ++i) o[h][i] *= c;
            mrun[h] = mn;
        }
#pragma unroll
        for (int r = 0; r < kRing; ++r) {
            if (r >= nr) continue;
            const int t = t0 + (s0 + r) * kStepTokens + 4 * wave + grp;
            float vf[8];
            unpack_f16x8(vring[r], vf);
            if (has_new && t == pos) {
#pragma unroll
                for (int i = 0; i < 8; ++i) vf[i] = kv_new[1][8 * j + i];
            }
#pragma unroll
            for (int h = 0; h < QPK; ++h) {
                const float p = __builtin_amdgcn_exp2f(sc[r][h] - mrun[h]);
                lrun[h] += p;
#pragma unroll
                for (int i = 0; i < 8; ++i) o[h][i] = __builtin_fmaf(p, vf[i], o[h][i]);
            }
        }
        // the next block's loads; none past the chunk, whose registers the
        // merge below would otherwise wait for
        if (s0 + kRing < steps) {
#pragma unroll
            for (int r = 0; r < kRing; ++r) issue(r, s0 + r + kRing);
        }
    }

    // ---- merge the workgroup's 16 row states (one per 16-lane row) through
    // LDS into this chunk's partial: each row's maximum, denominator and
    // output sums are scaled to the workgroup maximum and summed in row order
    const int row = wave * 4 + grp;
#pragma unroll
    for (int h = 0; h < QPK; ++h) {
        float4* dst = reinterpret_cast<float4*>(&st_o[row][h][8 * j]);
        dst[0] = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
        dst[1] = make_float4(o[h][4], o[h][5], o[h][6], o[h][7]);
        if (j == 0) st_ml[row][h] = make_float2(mrun[h], lrun[h]);
    }
    __syncthreads();
    // A thread finishes kOut outputs of one head (d0 + kSpan * u): the rows'
    // maxima and denominators are read once for all of them, and every LDS
    // read is issued before the first is used.
    constexpr int kOut = (QPK * kHeadDim + kThreads - 1) / kThreads;
    constexpr int kSpan = kHeadDim / kOut;
    const int h = tid / kSpan;
    const int d0 = tid - h * kSpan;
    if (h >= QPK) return;
    float2 ml[kRows];
    float ov[kOut][kRows];
#pragma unroll
    for (int q = 0; q < kRows; ++q) {
        ml[q] = st_ml[q][h];
#pragma unroll
        for (int u = 0; u < kOut; ++u) ov[u][q] = st_o[q][h][d0 + kSpan * u];
    }
    float mx = -FLT_MAX;
#pragma unroll
    for (int q = 0; q < kRows; ++q) mx = fmaxf(mx, ml[q].x);
    float l = 0.f, acc[kOut];
#pragma unroll
    for (int u = 0; u < kOut; ++u) acc[u] = 0.f;
#pragma unroll
    for (int q = 0; q < kRows; ++q) {
        const float f = __builtin_amdgcn_exp2f(ml[q].x - mx);
        l = __builtin_fmaf(ml[q].y, f, l);
#pragma unroll
        for (int u = 0; u < kOut; ++u) acc[u] = __builtin_fmaf(ov[u][q], f, acc[u]);
    }
    float* const own = a.partials != nullptr ? a.partials + (size_t)m * a.partial_floats : mb.partials;
    float* part = own + ((size_t)(kvh * QPK + h) * kAttnChunks + chunk) * kPartStride;
#pragma unroll
    for (int u = 0; u < kOut; ++u) part[d0 + kSpan * u] = acc[u];
    if (d0 == 0) {
        part[kHeadDim] = mx;
        part[kHeadDim + 1] = l;
    }
}

// The fused kernel's new-token path on its own: wave 0 normalises and ropes
// the member's raw K of one KV head, wave 1 takes V, both stored as f16 at
// the member's position. Grid (KV head, member).
__global__ __launch_bounds__(128) void kv_append_kernel(AttnArgs a) {
    const int kvh = blockIdx.x;
    const int m = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const AttnMember mb = a.mem[m];
    const float* src = (wave == 0 ? a.k : a.v) + ((size_t)m * a.kv_heads + kvh) * kHeadDim;
    float x0 = src[lane];
    float x1 = src[lane + 64];
    const int pos = a.positions[m];
    if (wave == 0) {
        norm_rope(x0, x1, a.k_norm[lane], a.k_norm[lane + 64], a.eps, rope_rot((float)pos, rope_freq(a.rope_base, lane)));
    }
    if (pos < 0 || pos >= mb.capacity) return;
    const size_t head_elems = (size_t)mb.capacity * kHeadDim;
    uint16_t* dst = (wave == 0 ? mb.keys : mb.values) + (size_t)a.layer * mb.layer_elems +
                    (size_t)kvh * head_elems + (size_t)pos * kHeadDim;
    dst[lane] = __builtin_bit_cast(uint16_t, (_Float16)x0);
    dst[lane + 64] = __builtin_bit_cast(uint16_t, (_Float16)x1);
}

struct TokenArgs {
    uint32_t tokens[kTokenArgs];
    uint32_t* dst;
    int count;
};

__global__ __launch_bounds__(256) void token_upload_kernel(TokenArgs in) {
    for (int i = threadIdx.x; i < in.count; i += 256) in.dst[i] = in.tokens[i];
}

__global__ __launch_bounds__(64) void step_inputs_kernel(StepInputs in) {
    const int i = threadIdx.x;
    if (i >= in.count) return;
    if (in.mem_dst != nullptr) in.mem_dst[i] = in.mem[i];
    if (in.tokens_dst != nullptr) in.tokens_dst[i] = in.tokens[i];
    if (in.positions_dst != nullptr) in.positions_dst[i] = in.positions[i];
}

// Merges the chunk partials of one (member, query head) into the attention
// output: o = sum_c O_c e^(m_c - M) / sum_c L_c e^(m_c - M), in chunk order.
// A separate launch: the kernel boundary orders the partials' writes before
// these reads, where an in-kernel hand-off would need a device-scope release
// (an L2 write-back) in every attention workgroup, which costs far more.
// Every thread loads each chunk's maximum and denominator itself (the
// threads of a workgroup read the same words), and every slot the launch can
// hold is loaded before the position says which are live, so the launch
// waits on memory once. One chunk is the same arithmetic: o = O_0 / L_0.
// The store is unconditional: a branch on the position would let the
// compiler sink the loads past its arrival.
// (A few workgroups per CU at most: the occupancy hint lets the compiler keep
// all of a thread's loads in flight instead of trading them for registers.)
__global__ __launch_bounds__(kHeadDim) __attribute__((amdgpu_waves_per_eu(1, 2))) void attn_combine_kernel(AttnArgs a) {
    const int qh = blockIdx.x;
    const int m = blockIdx.y;
    const int d = threadIdx.x;
    const float* own = a.partials != nullptr ? a.partials + (size_t)m * a.partial_floats : a.mem[m].partials;
    // Slots past the launch's chunks are never read (out of the buffer
    // range: zero); slots past this context's chunks hold stale memory
    // (possibly NaN bit patterns) and are replaced by a neutral state (sum 0,
    // maximum -FLT_MAX, denominator 0) before any arithmetic.
    const __amdgpu_buffer_rsrc_t pr =
        make_rsrc(own + (size_t)qh * kAttnChunks * kPartStride, (uint32_t)(a.chunks * kPartStride * 4));
    float o[kAttnChunks];
    float2 ml[kAttnChunks];
#pragma unroll
    for (int c = 0; c < kAttnChunks; ++c) {
        const uint32_t row = (uint32_t)(c * kPartStride) * 4u;
        o[c] = __builtin_bit_cast(float, load_b32(pr, row + (uint32_t)d * 4u));
        ml[c] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(pr, (int)(row + kHeadDim * 4), 0, 0));
    }
    const int tokens = a.positions[m] + 1;
    const int len = chunk_tokens(tokens, a.chunks, a.min_chunk);
    const int chunks = (tokens + len - 1) / len;
    float mx = -FLT_MAX;
#pragma unroll
    for (int c = 0; c < kAttnChunks; ++c) {
        const bool live = c < chunks;
        ml[c].x = live ? ml[c].x : -FLT_MAX;
        ml[c].y = live ? ml[c].y : 0.f;
        o[c] = live ? o[c] : 0.f;
        mx = fmaxf(mx, ml[c].x);
    }
    float l = 0.f, acc = 0.f;
#pragma unroll
    for (int c = 0; c < kAttnChunks; ++c) {
        const float f = __builtin_amdgcn_exp2f(ml[c].x - mx);
        l = __builtin_fmaf(ml[c].y, f, l);
        acc = __builtin_fmaf(o[c], f, acc);
    }
    a.out[((size_t)m * a.q_heads + qh) * kHeadDim + d] = acc / l;
}

// Order-preserving key of a float (model_ops.rs:151-155).
__device__ __forceinline__ uint32_t logit_key(float v) {
    const uint32_t bits = __builtin_bit_cast(uint32_t, v);
    return (bits >> 31) ? ~bits : (bits ^ 0x80000000u);
}

__device__ __forceinline__ void take_better(uint32_t& key, uint32_t& idx, uint32_t ok, uint32_t oi) {
    if (ok > key || (ok == key && oi < idx)) {
        key = ok;
        idx = oi;
    }
}

// Greedy selection in two stages: argmax_slice_kernel
// reduces one contiguous slice of a member's logits per workgroup (grid:
// slices x members) to its best (key, index); argmax_final_kernel reduces a
// member's slice results and applies the step's updates. The result is the
// largest key, the lowest index among equal keys, and 0 when every value is
// NaN (the reference's strict comparisons): each stage keeps the lowest index
// on ties. One workgroup per member would read a 151,936-value row at a
// single CU's bandwidth.
constexpr int kSliceThreads = 256;

__global__ __launch_bounds__(kSliceThreads) void argmax_slice_kernel(const float* logits, int vocab, int slice,
                                                                     uint2* part) {
    __shared__ uint32_t wkey[kSliceThreads / 64];
    __shared__ uint32_t widx[kSliceThreads / 64];
    const int b = blockIdx.x;
    const int m = blockIdx.y;
    const int tid = threadIdx.x;
    const float* row = logits + (size_t)m * vocab;
    const int lo = b * slice;
    const int hi = min(lo + slice, vocab);
    uint32_t key = 0u, idx = 0u;
    auto consider = [&](float v, int p) {
        const uint32_t k = logit_key(v);
        if (v == v && k > key) {
            key = k;
            idx = (uint32_t)p;
        }
    };
    // slices are whole float4s when the row allows it (16-byte aligned rows
    // of a multiple of 4 values); all of a thread's loads are in flight at once
    const bool wide = (vocab & 3) == 0 && (slice & 3) == 0 && ((reinterpret_cast<uintptr_t>(row) & 15) == 0);
    if (wide) {
        constexpr int U = 4;
        const float4* row4 = reinterpret_cast<const float4*>(row);
        for (int base = lo / 4; base < hi / 4; base += kSliceThreads * U) {
            float4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i = base + u * kSliceThreads + tid;
                v[u] = i < hi / 4 ? row4[i] : make_float4(NAN, NAN, NAN, NAN);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int p = 4 * (base + u * kSliceThreads + tid);
                consider(v[u].x, p);
                consider(v[u].y, p + 1);
                consider(v[u].z, p + 2);
                consider(v[u].w, p + 3);
            }
        }
    } else {
        for (int p = lo + tid; p < hi; p += kSliceThreads) consider(row[p], p);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t ok = (uint32_t)__shfl_xor((int)key, off, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)idx, off, 64);
        take_better(key, idx, ok, oi);
    }
    if ((tid & 63) == 0) {
        wkey[tid >> 6] = key;
        widx[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        key = wkey[0];
        idx = widx[0];
        for (int w = 1; w < kSliceThreads / 64; ++w) take_better(key, idx, wkey[w], widx[w]);
        part[(size_t)m * gridDim.x + b] = make_uint2(key, idx);
    }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const uint2* part, int slices, uint32_t* selected,
                                                         uint32_t* tokens, int32_t* positions, int32_t* steps,
                                                         uint32_t* history, int history_stride) {
    const int m = blockIdx.x;
    const int lane = threadIdx.x;
    uint32_t key = 0u, idx = 0u;
    for (int b = lane; b < slices; b += 64) {
        const uint2 r = part[(size_t)m * slices + b];
        take_better(key, idx, r.x, r.y);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t ok = (uint32_t)__shfl_xor((int)key, off, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)idx, off, 64);
        take_better(key, idx, ok, oi);
    }
    if (lane == 0) {
        selected[m] = idx;
        if (tokens != nullptr) tokens[m] = idx;
        if (positions != nullptr) {
            const int s = steps[m];
            history[(size_t)m * history_stride + s] = idx;
            steps[m] = s + 1;
            positions[m] = positions[m] + 1;
        }
    }
}

// ------------------------------------------------------------ prompt prefill
//
// kv_append_seq_kernel: the K/V of a prompt chunk's tokens, as kv_append_kernel
// computes them for one token (K RMSNorm + rope, f16 round to nearest even),
// at positions p0 + t. Grid (KV head, token).
__global__ __launch_bounds__(128) void kv_append_seq_kernel(PrefillAttnArgs a) {
    const int kvh = blockIdx.x;
    const int t = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const float* src = (wave == 0 ? a.k : a.v) + ((size_t)t * a.kv_heads + kvh) * kHeadDim;
    float x0 = src[lane];
    float x1 = src[lane + 64];
    const int pos = a.p0 + t;
    if (wave == 0) {
        norm_rope(x0, x1, a.k_norm[lane], a.k_norm[lane + 64], a.eps, rope_rot((float)pos, rope_freq(a.rope_base, lane)));
    }
    const size_t head_elems = (size_t)a.mem.capacity * kHeadDim;
    uint16_t* dst = (wave == 0 ? a.mem.keys : a.mem.values) + (size_t)a.layer * a.mem.layer_elems +
                    (size_t)kvh * head_elems + (size_t)pos * kHeadDim;
    dst[lane] = __builtin_bit_cast(uint16_t, (_Float16)x0);
    dst[lane + 64] = __builtin_bit_cast(uint16_t, (_Float16)x1);
}

// attn_prefill_kernel: causal attention of a prompt chunk on the matrix cores
// (v_mfma_f32_16x16x32_f16, f32 accumulation), after kv_append_seq_kernel
// stored the chunk's K/V. Token t (position p0 + t) attends positions
// 0 .. p0 + t: the reference's attention (model_ops.rs:430-566) for every
// token of the chunk, as the serial prefill computes it one token at a time.
//
// A wave owns one query head and kPrefillTileTokens tokens; a workgroup holds
// the QPK query heads of one KV head (and, for QPK < 4, 4 / QPK token tiles),
// so every K/V byte it stages serves all of them. Keys advance in blocks of
// 64 through double-buffered LDS (K as [key][dim], V transposed to
// [dim][key]): a block's global loads are issued before the previous block is
// reduced and written to the other buffer after it, one barrier per block.
// V is transposed in registers: a thread loads four consecutive keys of 8
// dims and stores 8-byte rows of V^T. LDS has 32 four-byte banks: K rows are
// unpadded with 16-byte piece p of key k at slot p ^ (k & 15), and V^T rows
// are 68 halfs (34 dwords), so the K and V^T stores and the fragment reads
// of 16 lanes (8 for 16-byte accesses) fall in distinct banks (counted: no
// conflict cycles). The rope angles of the workgroup's tokens are computed
// once per workgroup, not once per query head.
//
// Per block and wave, with S^T = K Q^T (M = 16 keys, N = 16 tokens, K = 128
// dims in 4 steps) the MFMA output puts token l%16 in lane l's column and keys
// 4(l/16)+i in its rows, so the online softmax state of a token lives in its
// four lanes (l%16 + 16g): maxima and denominators combine across them with
// two lane exchanges. The probabilities, rounded to f16, are already the B
// operand of O^T += V^T P^T (M = 16 dims, K = 32 keys): a dot product does not
// depend on the order of its terms, so key slot 8g+j of a 32-key step is key
// 16(j/4) + 4g + (j%4), and the A operand (V^T) reads the same keys.
// Scores are scaled by log2(e)/sqrt(128) in f32 after the product. q is
// normalised and roped in f32 (the decode kernel's operations) and enters the
// products as two f16 pieces, hi = f16(q) and lo = f16(q - hi), and so do the
// f32 probabilities: each product is two MFMAs and carries 22 significant
// bits of the f32 operand (K and V are the cache's f16 values, exact), so the
// attention follows the f32 reference to accumulation-order rounding.
typedef _Float16 pf_half8 __attribute__((ext_vector_type(8)));
typedef _Float16 pf_half4 __attribute__((ext_vector_type(4)));
typedef float pf_float4 __attribute__((ext_vector_type(4)));

constexpr int kPfKeys = 64;              // keys per block
constexpr int kPfVRow = kPfKeys + 4;     // LDS V^T row (halfs): 136 B
constexpr float kPfLazy = 15.0f;         // log2 headroom of the lazy softmax rescale

template <int QPK>
__global__ __launch_bounds__(64 * (QPK < 4 ? 4 : QPK)) void attn_prefill_kernel(PrefillAttnArgs a) {
    constexpr int W = QPK < 4 ? 4 : QPK;  // waves
    constexpr int NT = 64 * W;
    constexpr int TT = W / QPK;           // token tiles per workgroup
    constexpr int KP = kPfKeys * (kHeadDim / 8) / NT;  // 16-byte K pieces per thread and block
    // V: 256 units of 4 keys x 8 dims, one per thread of the first 256
    __shared__ __attribute__((aligned(16))) _Float16 ks[2][kPfKeys][kHeadDim];
    __shared__ __attribute__((aligned(16))) _Float16 vt[2][kHeadDim][kPfVRow];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kvh = blockIdx.y;
    const int hq = kvh * QPK + wave % QPK;
    const int t0 = ((int)blockIdx.x * TT + wave / QPK) * kPrefillTileTokens;
    const int tl = lane & 15;
    const int g = lane >> 4;
    const int t = t0 + tl;
    const bool live = t < a.tokens;
    const int pos = a.p0 + t;
    const int qdim = a.q_heads * kHeadDim;
    // the last position any token of the workgroup attends
    const int wg_end = min(((int)blockIdx.x + 1) * TT * kPrefillTileTokens, a.tokens);
    const int last = a.p0 + wg_end - 1;

    // ---- K/V block loads (positions past `last` read as zero)
    const size_t head_elems = (size_t)a.mem.capacity * kHeadDim;
    const size_t base = (size_t)a.layer * a.mem.layer_elems + (size_t)kvh * head_elems;
    const uint32_t span = (uint32_t)(last + 1) * (uint32_t)(kHeadDim * 2);
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(a.mem.keys + base, span);
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(a.mem.values + base, span);
    const bool v_unit = tid < 256;
    const int va = tid & 15;        // V unit: keys 4va .. 4va + 3
    const int vc = (tid >> 4) & 15; // dims 8vc .. 8vc + 7
    uint4 kp[KP], vp[4];
    auto issue = [&](int kb) {
#pragma unroll
        for (int r = 0; r < KP; ++r) {
            const int idx = tid + NT * r;
            kp[r] = load_b128(kr, ((uint32_t)(kb * kPfKeys + (idx >> 4)) * kHeadDim + 8u * (uint32_t)(idx & 15)) * 2u);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t off = ((uint32_t)(kb * kPfKeys + 4 * va + r) * kHeadDim + 8u * (uint32_t)vc) * 2u;
            vp[r] = load_b128(vr, v_unit ? off : kOOR);
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int r = 0; r < KP; ++r) {
            const int idx = tid + NT * r;
            *reinterpret_cast<uint4*>(&ks[buf][idx >> 4][8 * ((idx & 15) ^ ((idx >> 4) & 15))]) = kp[r];
        }
        if (v_unit) {
            // row j of the unit: dim 8vc + j of keys 4va .. 4va + 3
            const uint32_t w[4][4] = {{vp[0].x, vp[0].y, vp[0].z, vp[0].w}, {vp[1].x, vp[1].y, vp[1].z, vp[1].w},
                                      {vp[2].x, vp[2].y, vp[2].z, vp[2].w}, {vp[3].x, vp[3].y, vp[3].z, vp[3].w}};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int sh = 16 * (j & 1);
                const uint32_t e0 = (w[0][j >> 1] >> sh) & 0xffffu, e1 = (w[1][j >> 1] >> sh) & 0xffffu;
                const uint32_t e2 = (w[2][j >> 1] >> sh) & 0xffffu, e3 = (w[3][j >> 1] >> sh) & 0xffffu;
                *reinterpret_cast<uint2*>(&vt[buf][8 * vc + j][4 * va]) = make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
            }
        }
    };
    issue(0);

    // ---- rope angles of the workgroup's tokens, shared by its QPK query
    // heads: entry (row, d) = the rotation of pair (d, d + 64) at position
    // p0 + first token + row, the same rope_rot / rope_freq values each lane
    // would compute. The table lives in V^T buffer 1, which the first block
    // writes only after every wave has passed the barrier before the loop.
    // (One query head per workgroup token tile, QPK = 1, shares nothing: its
    // lanes compute their own.)
    constexpr int kRotRow = 65;  // float2 per token row (padded)
    float2* const rot_tab = reinterpret_cast<float2*>(&vt[1][0][0]);
    static_assert(QPK == 1 || TT * kPrefillTileTokens * kRotRow * sizeof(float2) <= sizeof(vt[1]),
                  "rope table must fit one V^T buffer");
    if constexpr (QPK > 1) {
#pragma unroll
        for (int r = 0; r < TT * kPrefillTileTokens * 64 / NT; ++r) {
            const int e = tid + NT * r;
            const int row = e >> 6, d = e & 63;
            const Rot rr = rope_rot((float)(a.p0 + (int)blockIdx.x * TT * kPrefillTileTokens + row),
                                    rope_freq(a.rope_base, d));
            rot_tab[row * kRotRow + d] = make_float2(rr.c, rr.s);
        }
        __syncthreads();
    }
    const int rot_row = (wave / QPK) * kPrefillTileTokens + tl;

    // ---- this lane's query dims 32s + 8g + j (s = 0..3, j = 0..7): RMSNorm
    // over the head's 128 dims (the four lanes of the token add their parts),
    // NEOX rope of the pairs (d, d + 64) = (s, s + 2), f16
    float x[4][8];
    const float* qrow = a.q + (size_t)t * qdim + (size_t)hq * kHeadDim;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int d = 32 * s + 8 * g;
        float4 lo = make_float4(0.f, 0.f, 0.f, 0.f), hi = lo;
        if (live) {
            lo = *reinterpret_cast<const float4*>(qrow + d);
            hi = *reinterpret_cast<const float4*>(qrow + d + 4);
        }
        x[s][0] = lo.x; x[s][1] = lo.y; x[s][2] = lo.z; x[s][3] = lo.w;
        x[s][4] = hi.x; x[s][5] = hi.y; x[s][6] = hi.z; x[s][7] = hi.w;
    }
    float ssq = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) ssq = __builtin_fmaf(x[s][j], x[s][j], ssq);
    ssq += __shfl_xor(ssq, 16, 64);
    ssq += __shfl_xor(ssq, 32, 64);
    const float inv = 1.0f / sqrtf(ssq / (float)kHeadDim + a.eps);
    pf_half8 qb[4], ql[4];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int d = 32 * s + 8 * g + j;
            const float y0 = x[s][j] * inv * a.q_norm[d];
            const float y1 = x[s + 2][j] * inv * a.q_norm[d + 64];
            Rot r;
            if constexpr (QPK > 1) {
                const float2 cs = rot_tab[rot_row * kRotRow + d];
                r.c = cs.x;
                r.s = cs.y;
            } else {
                r = rope_rot((float)pos, rope_freq(a.rope_base, d));
            }
            const float q0 = y0 * r.c - y1 * r.s;
            const float q1 = y0 * r.s + y1 * r.c;
            qb[s][j] = (_Float16)q0;
            ql[s][j] = (_Float16)(q0 - (float)qb[s][j]);
            qb[s + 2][j] = (_Float16)q1;
            ql[s + 2][j] = (_Float16)(q1 - (float)qb[s + 2][j]);
        }
    }

    // ---- online softmax over the key blocks
    float m_run = -FLT_MAX, l_run = 0.f;
    pf_float4 o[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) o[d] = pf_float4{0.f, 0.f, 0.f, 0.f};
    const int blocks = last / kPfKeys + 1;
    stage(0);
    __syncthreads();
    for (int kb = 0; kb < blocks; ++kb) {
        const int buf = kb & 1;
        if (kb + 1 < blocks) issue(kb + 1);

        // S^T for the block's four 16-key tiles, issued tile-interleaved:
        // consecutive MFMAs feed different accumulators
        pf_float4 sc[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) sc[kt] = pf_float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            pf_half8 ka[4];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
                ka[kt] = *reinterpret_cast<const pf_half8*>(&ks[buf][16 * kt + tl][8 * ((4 * s + g) ^ tl)]);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kt], qb[s], sc[kt], 0, 0, 0);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kt], ql[s], sc[kt], 0, 0, 0);
        }
        // keys past a token's position are masked; a block wholly at or below
        // the wave's first position needs no mask (a wave-uniform test)
        float bmax = -INFINITY;
        if (kb * kPfKeys + kPfKeys - 1 <= a.p0 + t0) {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    sc[kt][i] *= a.scale;
                    bmax = fmaxf(bmax, sc[kt][i]);
                }
            }
        } else {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = kb * kPfKeys + 16 * kt + 4 * g + i;
                    const float v = key <= pos ? sc[kt][i] * a.scale : -INFINITY;
                    sc[kt][i] = v;
                    bmax = fmaxf(bmax, v);
                }
            }
        }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 16, 64));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
        // Lazy rescaling: the reference point m_run moves (to the block's
        // maximum) only when that maximum passes it by more than kPfLazy.
        // Until then the probabilities exp2(s - m_run) stay below
        // 2^kPfLazy, inside f16 range for the hi/lo split, and O and l keep
        // their scale; O / l is the same softmax. The first block always
        // moves it (from -FLT_MAX, with a zero correction).
        const bool move = bmax > m_run + kPfLazy;
        if (__any(move)) {
            const float m_new = move ? bmax : m_run;
            const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_run *= corr;
#pragma unroll
            for (int d = 0; d < 8; ++d) o[d] *= corr;
        }
        // probabilities in pairs: hi = f16(p) and lo = f16(p - hi), each pair
        // converted by one packed instruction (round toward zero: hi + lo
        // still carries 22 bits of p, since p - hi is exact in f32)
        pf_half8 pb[2], pl[2];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                const float p0 = __builtin_amdgcn_exp2f(sc[kt][i] - m_run);
                const float p1 = __builtin_amdgcn_exp2f(sc[kt][i + 1] - m_run);
                l_run += p0;
                l_run += p1;
                const auto h = __builtin_amdgcn_cvt_pkrtz(p0, p1);
                const auto r = __builtin_amdgcn_cvt_pkrtz(p0 - (float)h[0], p1 - (float)h[1]);
                pb[kt >> 1][4 * (kt & 1) + i] = h[0];
                pb[kt >> 1][4 * (kt & 1) + i + 1] = h[1];
                pl[kt >> 1][4 * (kt & 1) + i] = r[0];
                pl[kt >> 1][4 * (kt & 1) + i + 1] = r[1];
            }
        }
        // O^T += V^T P^T over the block's two 32-key steps, issued
        // dim-tile-interleaved (eight accumulators between dependent MFMAs)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            pf_half8 vf[8];
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                const _Float16* row = &vt[buf][16 * d + tl][32 * u + 4 * g];
                const pf_half4 v0 = *reinterpret_cast<const pf_half4*>(row);
                const pf_half4 v1 = *reinterpret_cast<const pf_half4*>(row + 16);
                vf[d] = pf_half8{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            }
#pragma unroll
            for (int d = 0; d < 8; ++d) o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[d], pb[u], o[d], 0, 0, 0);
#pragma unroll
            for (int d = 0; d < 8; ++d) o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[d], pl[u], o[d], 0, 0, 0);
        }
        // the next block into the other buffer: every wave finished reading
        // it before the previous barrier
        if (kb + 1 < blocks) stage(buf ^ 1);
        __syncthreads();
    }

    // ---- the token's denominator over its four lanes, then O / l
    float l_tot = l_run + __shfl_xor(l_run, 16, 64);
    l_tot += __shfl_xor(l_tot, 32, 64);
    if (!live) return;
    float* dst = a.out + (size_t)t * qdim + (size_t)hq * kHeadDim + 4 * g;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        *reinterpret_cast<float4*>(dst + 16 * d) =
            make_float4(o[d][0] / l_tot, o[d][1] / l_tot, o[d][2] / l_tot, o[d][3] / l_tot);
    }
}

}  // namespace

size_t attn_partials_floats(int q_heads) { return (size_t)q_heads * kAttnChunks * kPartStride; }

int attn_grid_chunks(int max_capacity, int members) {
    // chunks a context can need: capacity / the minimum chunk, up to kAttnChunks
    const int min_chunk = attn_min_chunk(members);
    return std::max(1, std::min(kAttnChunks, (max_capacity + min_chunk - 1) / min_chunk));
}

hipError_t launch_attention(const AttnArgs& args, int members, hipStream_t stream) {
    if (members < 1 || members > kAttnMaxMembers || args.kv_heads < 1 || args.q_heads % args.kv_heads != 0 ||
        args.chunks < 1 || args.chunks > kAttnChunks || args.mem == nullptr) {
        return hipErrorInvalidValue;
    }
    // The chunking depends on the caches' capacity and on the member count's
    // range only, so up to 8 members every member's bits equal its
    // single-sequence step (the reference qualifies batched rows bit for bit
    // against batch-1 rows, cuda_reference.rs:5322-5334), and from 9 to 64
    // they equal its step in any other batch of that range.
    AttnArgs b = args;
    b.min_chunk = attn_min_chunk(members);
    const dim3 grid((unsigned)b.chunks, (unsigned)b.kv_heads, (unsigned)members);
    switch (b.q_heads / b.kv_heads) {
    case 1: hipLaunchKernelGGL(attn_decode_kernel<1>, grid, dim3(kThreads), 0, stream, b); break;
    case 2: hipLaunchKernelGGL(attn_decode_kernel<2>, grid, dim3(kThreads), 0, stream, b); break;
    case 4: hipLaunchKernelGGL(attn_decode_kernel<4>, grid, dim3(kThreads), 0, stream, b); break;
    case 8: hipLaunchKernelGGL(attn_decode_kernel<8>, grid, dim3(kThreads), 0, stream, b); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)b.q_heads, (unsigned)members), dim3(kHeadDim), 0, stream,
                       b);
    return hipGetLastError();
}

namespace {
__global__ __launch_bounds__(256) void swiglu_kernel(const float* gate, const float* up, float* out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const float g = gate[i];
        out[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}
}  // namespace

hipError_t launch_swiglu(const float* gate, const float* up, float* out, size_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const unsigned grid = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(swiglu_kernel, dim3(grid), dim3(256), 0, stream, gate, up, out, n);
    return hipGetLastError();
}

hipError_t launch_kv_append(const AttnArgs& args, int members, hipStream_t stream) {
    if (members < 1 || members > kAttnMaxMembers || args.kv_heads < 1 || args.mem == nullptr) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)args.kv_heads, (unsigned)members), dim3(128), 0, stream,
                       args);
    return hipGetLastError();
}

hipError_t launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t stream) {
    if (a.tokens < 1 || a.kv_heads < 1 || a.q_heads % a.kv_heads != 0 || a.p0 < 0 ||
        (long long)a.p0 + a.tokens > a.mem.capacity || a.mem.keys == nullptr || a.mem.values == nullptr) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(kv_append_seq_kernel, dim3((unsigned)a.kv_heads, (unsigned)a.tokens), dim3(128), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.out == nullptr) return e;
    const int qpk = a.q_heads / a.kv_heads;
    const int tile = kPrefillTileTokens * (qpk < 4 ? 4 / qpk : 1);
    const dim3 grid((unsigned)((a.tokens + tile - 1) / tile), (unsigned)a.kv_heads);
    switch (qpk) {
    case 1: hipLaunchKernelGGL(attn_prefill_kernel<1>, grid, dim3(256), 0, stream, a); break;
    case 2: hipLaunchKernelGGL(attn_prefill_kernel<2>, grid, dim3(256), 0, stream, a); break;
    case 4: hipLaunchKernelGGL(attn_prefill_kernel<4>, grid, dim3(256), 0, stream, a); break;
    case 8: hipLaunchKernelGGL(attn_prefill_kernel<8>, grid, dim3(512), 0, stream, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_token_upload(const uint32_t* tokens, size_t count, uint32_t* dst, hipStream_t stream) {
    if (tokens == nullptr || dst == nullptr) return hipErrorInvalidValue;
    for (size_t i0 = 0; i0 < count; i0 += kTokenArgs) {
        TokenArgs a;
        a.count = (int)std::min<size_t>(kTokenArgs, count - i0);
        for (int i = 0; i < a.count; ++i) a.tokens[i] = tokens[i0 + i];
        a.dst = dst + i0;
        hipLaunchKernelGGL(token_upload_kernel, dim3(1), dim3(256), 0, stream, a);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_step_inputs(const StepInputs& in, hipStream_t stream) {
    if (in.count < 1 || in.count > kStepInputs) return hipErrorInvalidValue;
    hipLaunchKernelGGL(step_inputs_kernel, dim3(1), dim3(64), 0, stream, in);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, int vocab, int members, uint32_t* selected, uint32_t* tokens,
                         int32_t* positions, int32_t* steps, uint32_t* history, int history_stride, uint64_t* part,
                         hipStream_t stream) {
    if (members < 1 || vocab < 1 || part == nullptr) return hipErrorInvalidValue;
    // slices of at least 1024 values, a multiple of 4, at most kArgmaxSlices of them
    int slice = (vocab + kArgmaxSlices - 1) / kArgmaxSlices;
    slice = std::max(1024, (slice + 3) / 4 * 4);
    const int slices = (vocab + slice - 1) / slice;
    uint2* p = reinterpret_cast<uint2*>(part);
    hipLaunchKernelGGL(argmax_slice_kernel, dim3((unsigned)slices, (unsigned)members), dim3(kSliceThreads), 0, stream,
                       logits, vocab, slice, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)members), dim3(64), 0, stream, p, slices, selected, tokens,
                       positions, steps, history, history_stride);
    return hipGetLastError();
}

}  // namespace ribn_amd

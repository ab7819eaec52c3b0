// Internal launcher API of the decode-step kernels (decode_kernels.hip):
// attention over the f16 KV cache and the greedy token selection.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ribn_amd {

// Head geometry the attention kernel is built for (Qwen3: 128-wide heads).
constexpr int kHeadDim = 128;
// Token chunks per (member, KV head): the work of one workgroup, at most
// this many. The count depends on the caches' capacity and on whether the
// launch holds more than 8 members (chunks of at least 64 tokens up to 8, 128
// beyond): a member's arithmetic is the same at any batch size within each
// range, and a captured step serves every position.
constexpr int kAttnChunks = 32;
// Members one attention launch serves (the host splits larger batches): the
// decoder's whole batch. At batch 16 one launch of 16 members ran the step
// 6% faster than two launches of 8 (3,448 against 3,243 tok/s).
constexpr int kAttnMaxMembers = 64;
// Floats per (chunk, query head) partial: 128 output sums, the running
// maximum, the running denominator, two pad words (16-byte rows).
constexpr int kPartStride = kHeadDim + 4;

// One member's cache, as a device-resident descriptor: the attention kernel
// reads it from memory, so a captured step serves any set of caches.
struct AttnMember {
    uint16_t* keys;       // f16 [layers][kv_heads][capacity][128]
    uint16_t* values;     // f16 [layers][kv_heads][capacity][128]
    float* partials;      // [q_heads][kAttnChunks][kPartStride], this member's own
    uint64_t layer_elems; // kv_heads * capacity * 128: one layer's elements
    int capacity;         // cache tokens per (layer, KV head)
    int pad;
};

struct AttnArgs {
    const AttnMember* mem;     // device [members] descriptors
    int layer;
    int chunks;                // grid chunks: attn_grid_chunks(max capacity, members)
    int min_chunk;             // tokens a chunk spans at least (launch_attention sets it)
    int appended;              // 1: every member's K/V is already in its cache (launch_kv_append)
    const float* q;            // [members][q_heads * 128], raw projection
    const float* k;            // [members][kv_heads * 128], raw projection
    const float* v;            // [members][kv_heads * 128]
    const float* q_norm;       // [128] per-head RMSNorm weight
    const float* k_norm;       // [128]
    const int32_t* positions;  // [members] device positions of the new token
    float* out;                // [members][q_heads * 128]
    float* partials;           // when set, member m's partials start at partials + m * partial_floats
                               // (the merge launch then needs no descriptor); else the descriptors'
    uint64_t partial_floats;
    int q_heads;
    int kv_heads;
    float eps;
    float rope_base;
    float scale;               // log2(e) / sqrt(head_dim): scores are kept in log2 units
};

// Floats of one sequence's attention partials ([q_heads][kAttnChunks][kPartStride]).
size_t attn_partials_floats(int q_heads);

// Grid chunks of an attention launch of `members` over caches of at most
// `max_capacity` tokens.
int attn_grid_chunks(int max_capacity, int members);

// Two launches: the chunked attention writing partials, then their merge into
// `out`. members <= kAttnMaxMembers; q_heads / kv_heads in {1, 2, 4, 8}.
// Without `appended`, the workgroup whose chunk holds a member's position
// normalises, ropes and appends that member's new K/V (members must then
// hold distinct caches); with it the caches already hold them.
hipError_t launch_attention(const AttnArgs& args, int members, hipStream_t stream);

// The K/V append of `members` new tokens, ahead of an `appended` attention
// launch: per (member, KV head) the K RMSNorm + rope and the f16 store of K
// and V at positions[m], computed as the fused attention kernel does. Members
// may share a cache (consecutive positions of one sequence).
hipError_t launch_kv_append(const AttnArgs& args, int members, hipStream_t stream);

// out[i] = silu(gate[i]) * up[i] over n values (model_ops.rs:316-328, the
// same operations as the GEMVs' SwiGLU prologue and pair epilogue); out may
// alias gate.
hipError_t launch_swiglu(const float* gate, const float* up, float* out, size_t n, hipStream_t stream);

// Stream-ordered upload of up to kStepInputs members' step inputs through
// kernel arguments (no host buffer outlives the call): descriptors, token
// ids and positions; a null destination is skipped.
constexpr int kStepInputs = 16;
struct StepInputs {
    AttnMember mem[kStepInputs];
    uint32_t tokens[kStepInputs];
    int32_t positions[kStepInputs];
    AttnMember* mem_dst;
    uint32_t* tokens_dst;
    int32_t* positions_dst;
    int count;
};
hipError_t launch_step_inputs(const StepInputs& in, hipStream_t stream);

// Stream-ordered upload of `count` token ids from host memory to dst through
// kernel arguments (launches of up to kTokenArgs ids): the host array is not
// read after the call returns and nothing waits for the stream.
constexpr int kTokenArgs = 960;
hipError_t launch_token_upload(const uint32_t* tokens, size_t count, uint32_t* dst, hipStream_t stream);

// Prompt prefill: `tokens` consecutive tokens of one sequence at positions
// p0 .. p0 + tokens - 1, their q/k/v projections computed for the whole chunk.
struct PrefillAttnArgs {
    AttnMember mem;        // the sequence's cache (partials unused)
    int layer;
    int p0;                // position of the chunk's first token
    int tokens;            // tokens in the chunk
    const float* q;        // [tokens][q_heads * 128], raw projection
    const float* k;        // [tokens][kv_heads * 128]
    const float* v;
    const float* q_norm;   // [128]
    const float* k_norm;
    float* out;            // [tokens][q_heads * 128]; null: K/V append only
    int q_heads;
    int kv_heads;
    float eps;
    float rope_base;
    float scale;           // log2(e) / sqrt(head_dim)
};

// Tokens one prompt-attention workgroup tile covers per query head.
constexpr int kPrefillTileTokens = 16;

// The chunk's K (RMSNorm + rope) and V stored as f16 at their positions, then
// (when `out` is set) causal attention of every token over positions
// 0 .. its own on the matrix cores. q_heads / kv_heads in {1, 2, 4, 8}.
hipError_t launch_prefill_attention(const PrefillAttnArgs& args, hipStream_t stream);

// Slice results a two-stage greedy selection keeps per member.
constexpr int kArgmaxSlices = 64;

// Greedy selection per member over logits [members][vocab] (ties to the lowest
// index, NaN never selected). Writes selected[m]; when `tokens` is not null
// also tokens[m] (the next step's input). When `positions` is not null the
// member's generation advances on the device: history[m * history_stride +
// steps[m]] = selected, then steps[m] and positions[m] grow by one. `part`
// holds [members][kArgmaxSlices] scratch words for the slice results.
hipError_t launch_argmax(const float* logits, int vocab, int members, uint32_t* selected, uint32_t* tokens,
                         int32_t* positions, int32_t* steps, uint32_t* history, int history_stride, uint64_t* part,
                         hipStream_t stream);

}  // namespace ribn_amd

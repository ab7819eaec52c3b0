// Host runtime of the Qwen3 decode step behind the C ABI (include/ribn_amd.h):
// per-sequence KV caches, the step's device buffers, the launch sequence and
// its capture as HIP graphs.
//
// One step for `members` sequences, in the reference's order
// (crates/nvidia/src/decode.rs:544-631 run_step, 929-1034 full_attention_layer),
// with the elementwise launches fused into their neighbours:
//   embedding of tokens[m]                          (q4_k_embedding; device token ids)
//   per layer:
//     q/k/v GEMV, RMSNorm(attn_norm) in the prologue   (rms_norm + 3 gemv)
//     attention: q/k norm, rope, KV append, GQA, then  (5 launches in the reference)
//       the merge of its chunks
//     o GEMV added into the residual stream            (gemv + residual_add)
//     gate/up GEMV pairs, RMSNorm(ffn_norm) in the prologue, silu(gate)*up in
//       the epilogue                                    (rms_norm + 2 gemv + silu_mul)
//     down GEMV added into the stream                  (gemv + residual_add)
//   output head: RMSNorm(output_norm) + lm_head GEMV, argmax (run_output_head, 655-677)
// Six launches per layer (attention is two) instead of the reference's 14. Positions, token
// ids and the members' cache descriptors live in device memory, written by one
// small kernel from its arguments ahead of the step: one captured graph per
// (members, head, mode, grid) serves every position and every set of caches,
// nothing waits on the host before a launch, and a generation loop needs no
// host round trip between steps.
//
// A prefill chunk runs consecutive prompt tokens of one sequence as the
// members of one step (no output head): their K/V are appended by a separate
// launch before the attention launch, which then reads them from the cache.
#include "ribn_amd.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <new>
#include <vector>

#include "abi_internal.hpp"
#include "decode_launch.hpp"
#include "kquant_launch.hpp"
#include "qwen3_internal.hpp"

using namespace ribn_amd_abi;

struct ribn_amd_kv_cache {
    ribn_amd_context* ctx;
    int device;
    uint64_t id;  // distinguishes caches in captured-graph keys
    ribn_amd_qwen3_config cfg;
    uint32_t capacity;
    size_t layer_elems;  // kv_heads * capacity * head_dim
    void* block;         // one allocation: keys, values, partials
    uint16_t* keys;      // [layers][kv_heads][capacity][head_dim]
    uint16_t* values;
    float* partials;     // attention partials of the standalone attention call
};

namespace {

std::atomic<uint64_t> g_cache_ids{1};

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// A captured step: the launches depend on the member count, the output head,
// device-side advance, the append mode and the attention grid, not on which
// caches, tokens or positions the members hold.
struct GraphKey {
    int members;
    bool head;
    bool advance;
    bool appended;
    int chunks;
    bool operator==(const GraphKey& o) const {
        return members == o.members && head == o.head && advance == o.advance && appended == o.appended &&
               chunks == o.chunks;
    }
};

struct GraphEntry {
    GraphKey key;
    hipGraph_t graph;
    hipGraphExec_t exec;
};

constexpr size_t kMaxGraphs = 64;

ribn_amd_status check_config(const ribn_amd_qwen3_config* c) {
    if (c == nullptr) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null config");
    if (c->layers == 0) return fail(RIBN_AMD_INVALID_PLAN, 1, 0, "the plan has no layers");
    if (c->head_dim != (uint32_t)ribn_amd::kHeadDim) {
        return fail(RIBN_AMD_INVALID_PLAN, ribn_amd::kHeadDim, c->head_dim, "head_dim %u is not %d", c->head_dim,
                    ribn_amd::kHeadDim);
    }
    if (c->kv_heads == 0 || c->q_heads == 0 || c->q_heads % c->kv_heads != 0) {
        return fail(RIBN_AMD_INVALID_PLAN, c->kv_heads, c->q_heads, "%u query heads do not group over %u KV heads",
                    c->q_heads, c->kv_heads);
    }
    const uint32_t group = c->q_heads / c->kv_heads;
    if (group != 1 && group != 2 && group != 4 && group != 8) {
        return fail(RIBN_AMD_INVALID_PLAN, 8, group, "query heads per KV head must be 1, 2, 4 or 8 (got %u)", group);
    }
    const uint64_t qdim = (uint64_t)c->q_heads * c->head_dim;
    const uint64_t dims[2] = {c->hidden, qdim};
    for (uint64_t d : dims) {
        if (d == 0 || d % 256 != 0 || d > (uint64_t)ribn_amd::kWaveMaxK) {
            return fail(RIBN_AMD_INVALID_PLAN, (uint64_t)ribn_amd::kWaveMaxK, d,
                        "hidden and q_heads*head_dim must be multiples of 256 up to %d (got %llu)",
                        ribn_amd::kWaveMaxK, (unsigned long long)d);
        }
    }
    // the down projection's K: beyond kWaveMaxK it runs the slice-split GEMV
    if (c->ffn == 0 || c->ffn % 256 != 0 || c->ffn > (uint64_t)ribn_amd::kF32SplitMaxK) {
        return fail(RIBN_AMD_INVALID_PLAN, (uint64_t)ribn_amd::kF32SplitMaxK, c->ffn,
                    "ffn must be a multiple of 256 up to %d (got %u)", ribn_amd::kF32SplitMaxK, c->ffn);
    }
    if (c->vocab == 0 || c->vocab > (uint32_t)std::numeric_limits<int>::max()) {
        return fail(RIBN_AMD_INVALID_PLAN, 1, c->vocab, "vocabulary size %u is out of range", c->vocab);
    }
    if (!(c->rope_base > 0.f) || !std::isfinite(c->rope_base)) {
        return fail(RIBN_AMD_INVALID_PLAN, 0, 0, "rope base must be finite and positive");
    }
    return check_epsilon(c->epsilon);
}

bool same_geometry(const ribn_amd_qwen3_config& a, const ribn_amd_qwen3_config& b) {
    return a.layers == b.layers && a.q_heads == b.q_heads && a.kv_heads == b.kv_heads && a.head_dim == b.head_dim;
}

}  // namespace

struct ribn_amd_qwen3_decode {
    ribn_amd_context* ctx;
    ribn_amd_qwen3_config cfg;
    uint32_t max_members;
    const ribn_amd_quantized_weight* token_embd;
    const ribn_amd_quantized_weight* output;
    const float* output_norm;
    std::vector<ribn_amd_qwen3_layer> layers;
    void* block;  // step buffers, one allocation
    float* hidden;    // [members][hidden] residual stream
    float* q;         // [members][q_heads*128]
    float* k;         // [members][kv_heads*128]
    float* v;
    float* attn;      // [members][q_heads*128]
    float* gate;      // [members][ffn]
    float* up;
    float* logits;    // [members][vocab]
    uint32_t* tokens;     // [members] input token of the next step
    uint32_t* selected;   // [members] greedy selection of the last step
    int32_t* positions;   // [members]
    int32_t* steps;       // [members] generated-token counters
    uint32_t* history;    // [members][history_steps]
    uint32_t history_steps;
    ribn_amd::AttnMember* members_dev;  // [members] cache descriptors of the next step
    float* partials;      // [members][attention partials]
    uint64_t* argmax_part;  // [members][kArgmaxSlices] slice results of the greedy selection
    int chunks;           // attention grid of the next step (from its caches' capacities)
    hipStream_t capture;  // private stream for graph capture
    bool graphs;
    uint32_t gemv_mode;   // RIBN_AMD_GEMV_WARP (f32 activations) or RIBN_AMD_GEMV_FIXED16
    std::vector<GraphEntry> graph_cache;
    // Prompt prefill on the prefill matmul (ribn_amd_qwen3_prefill_prompt):
    // one allocation for chunks of up to prompt_tokens tokens, grown on demand.
    void* prompt_block;
    size_t prompt_bytes;
    uint32_t prompt_tokens;
    uint32_t* p_tokens;   // [chunk] token ids
    float* p_hidden;      // [chunk][hidden] residual stream
    float* p_q;           // [chunk][q_heads*128]
    float* p_k;           // [chunk][kv_heads*128]
    float* p_v;
    float* p_attn;        // [chunk][q_heads*128]
    float* p_gate;        // [chunk][ffn]
    float* p_up;
    float* p_y;           // [chunk][hidden] o / down projection, added by the next activation stage
    void* p_gemm;         // f16 activations, unscales and split-K partials of the prefill matmul
    size_t p_gemm_bytes;
};

namespace {

// GEMV over `count` weights of one value type sharing the activation x, in
// launch groups of as many members as one launch serves (the wave GEMV, or the
// matrix-core GEMV for 3..16 members of Q4_K / Q5_K).
// `fold`: the residual update of x pending from the previous accumulating
// product (the f32-faithful matrix-core GEMV adds it while packing x, or it
// is added on its own first); `defer`: this accumulating product may leave
// its own split sums pending there instead of a reduce launch.
hipError_t wave(const ribn_amd_qwen3_decode* d, const ribn_amd_quantized_weight* const* ws, int count,
                const float* x, const float* x2, const float* gamma, float* const* ys, int members, bool accumulate,
                hipStream_t stream, bool pair = false, ribn_amd::F32MmaFold* fold = nullptr,
                ribn_amd::F32MmaFold* defer = nullptr) {
    const int K = (int)ws[0]->input_size;
    const int arith = arith_of_mode(d->gemv_mode);
    const int per = ribn_amd::gemv_launch_members((int)ws[0]->value_type, K, x2 != nullptr, arith);
    if (per <= 0) return hipErrorInvalidValue;
    if (fold != nullptr && fold->splits > 0 && members > per) {
        // several launch groups: the update goes in on its own first
        hipError_t e = ribn_amd::launch_f32mma_fold_flush(fold, stream);
        if (e != hipSuccess) return e;
    }
    if (members > per) defer = nullptr;
    for (int m0 = 0; m0 < members; m0 += per) {
        const int mc = std::min(per, members - m0);
        ribn_amd::WaveGemvArgs a{};
        int rows = 0;
        for (int i = 0; i < count; ++i) {
            const int n = (int)ws[i]->output_size;
            a.w[i] = ws[i]->data;
            a.wbytes[i] = (uint32_t)ws[i]->encoded_bytes;
            a.y[i] = ys[i] + (size_t)m0 * n;
            rows += n;
            a.rows_end[i] = rows;
        }
        a.count = count;
        a.total_rows = rows;
        a.x = x + (size_t)m0 * K;
        a.x2 = x2 != nullptr ? x2 + (size_t)m0 * K : nullptr;
        a.gamma = gamma;
        a.eps = d->cfg.epsilon;
        a.K = K;
        a.members = mc;
        a.accumulate = accumulate ? 1 : 0;
        a.pair_swiglu = pair ? 1 : 0;
        a.arith = arith;
        a.fold = fold != nullptr && fold->splits > 0 ? fold : nullptr;
        a.defer = defer;
        hipError_t e = ribn_amd::launch_gemv((int)ws[0]->value_type, a, d->ctx->act_scratch, d->ctx->cu_count,
                                             stream);
        if (e != hipSuccess) return e;
        if (fold != nullptr) *fold = ribn_amd::F32MmaFold{};  // consumed (or flushed) by this call
    }
    return hipSuccess;
}

// RMSNorm-fused GEMVs of weights sharing one input: one launch per run of
// equal value types (q/k/v or gate/up of Q4_K_M files may mix types).
hipError_t wave_shared(const ribn_amd_qwen3_decode* d, const ribn_amd_quantized_weight* const* ws, float* const* ys,
                       int count, const float* x, const float* gamma, int members, hipStream_t stream,
                       ribn_amd::F32MmaFold* fold = nullptr) {
    int i = 0;
    while (i < count) {
        int j = i + 1;
        while (j < count && ws[j]->value_type == ws[i]->value_type) ++j;
        // the first launch takes the pending update of x (and clears it)
        hipError_t e = wave(d, ws + i, j - i, x, nullptr, gamma, ys + i, members, false, stream, false, fold);
        if (e != hipSuccess) return e;
        i = j;
    }
    return hipSuccess;
}

// One layer's attention over device descriptors mem[0..members), in launches of
// kAttnMaxMembers; `appended` first stores the launch's members' K/V.
// With `partials` set, member m's attention partials live at partials +
// m * attn_partials_floats (the decoder's own buffer, whose address the merge
// launch then takes from its arguments); else in the descriptors.
hipError_t attention(const ribn_amd_qwen3_config& cfg, const ribn_amd::AttnMember* mem, int chunks, bool appended,
                     int members, uint32_t layer, const float* q, const float* k, const float* v, const float* q_norm,
                     const float* k_norm, const int32_t* positions, float* out, float* partials, hipStream_t stream) {
    const size_t part = ribn_amd::attn_partials_floats((int)cfg.q_heads);
    const size_t qdim = (size_t)cfg.q_heads * cfg.head_dim;
    const size_t kvdim = (size_t)cfg.kv_heads * cfg.head_dim;
    for (int m0 = 0; m0 < members; m0 += ribn_amd::kAttnMaxMembers) {
        const int mc = std::min(ribn_amd::kAttnMaxMembers, members - m0);
        ribn_amd::AttnArgs a{};
        a.mem = mem + m0;
        a.layer = (int)layer;
        a.chunks = chunks;
        a.appended = appended ? 1 : 0;
        a.q = q + m0 * qdim;
        a.k = k + m0 * kvdim;
        a.v = v + m0 * kvdim;
        a.q_norm = q_norm;
        a.k_norm = k_norm;
        a.positions = positions + m0;
        a.out = out + m0 * qdim;
        a.partials = partials != nullptr ? partials + m0 * part : nullptr;
        a.partial_floats = part;
        a.q_heads = (int)cfg.q_heads;
        a.kv_heads = (int)cfg.kv_heads;
        a.eps = cfg.epsilon;
        a.rope_base = cfg.rope_base;
        // softmax weights are exp2 of scores in log2 units: e^x = 2^(x log2 e)
        a.scale = 1.4426950408889634f / sqrtf((float)cfg.head_dim);
        hipError_t e = hipSuccess;
        if (appended) e = ribn_amd::launch_kv_append(a, mc, stream);
        if (e == hipSuccess) e = ribn_amd::launch_attention(a, mc, stream);
        if (e != hipSuccess) return e;
    }
    // appended members in position order: a member reads only earlier
    // positions, stored by its own launch group's append or an earlier one
    return hipSuccess;
}

// The launches of one step (see the file comment).
hipError_t enqueue_step(ribn_amd_qwen3_decode* d, const GraphKey& key, hipStream_t stream) {
    const int members = key.members;
    const ribn_amd_qwen3_config& c = d->cfg;
    hipError_t e = ribn_amd::launch_embedding((int)d->token_embd->value_type, d->token_embd->data,
                                              (uint32_t)d->token_embd->encoded_bytes, d->tokens, 0, d->hidden,
                                              c.hidden / 256, c.vocab, (uint32_t)members, stream);
    if (e != hipSuccess) return e;
    // The o and down products add into the residual d->hidden. With split K
    // on the f32-faithful matrix-core GEMV (9..64 members) they leave their
    // split sums pending and the next RMSNorm-fused GEMV over d->hidden adds
    // them while packing it (the same sums, so the same bits as a reduce
    // launch).
    ribn_amd::F32MmaFold pending{};
    for (uint32_t l = 0; l < c.layers; ++l) {
        const ribn_amd_qwen3_layer& L = d->layers[l];
        const ribn_amd_quantized_weight* qkv[3] = {L.attn_q, L.attn_k, L.attn_v};
        float* qkv_out[3] = {d->q, d->k, d->v};
        e = wave_shared(d, qkv, qkv_out, 3, d->hidden, L.attn_norm, members, stream, &pending);
        if (e != hipSuccess) return e;
        e = attention(c, d->members_dev, key.chunks, key.appended, members, l, d->q, d->k, d->v, L.attn_q_norm,
                      L.attn_k_norm, d->positions, d->attn, d->partials, stream);
        if (e != hipSuccess) return e;
        e = wave(d, &L.attn_output, 1, d->attn, nullptr, nullptr, &d->hidden, members, true, stream, false, nullptr,
                 &pending);
        if (e != hipSuccess) return e;
        const ribn_amd_quantized_weight* gu[2] = {L.ffn_gate, L.ffn_up};
        if (L.ffn_gate->value_type == L.ffn_up->value_type && c.hidden <= (uint32_t)ribn_amd::kSliceK) {
            // gate/up pairs store silu(gate) * up; down reads it as a plain input
            float* act[2] = {d->gate, d->gate};
            e = wave(d, gu, 2, d->hidden, nullptr, L.ffn_norm, act, members, false, stream, true, &pending);
            if (e != hipSuccess) return e;
            e = wave(d, &L.ffn_down, 1, d->gate, nullptr, nullptr, &d->hidden, members, true, stream, false, nullptr,
                     &pending);
        } else if (c.ffn > (uint32_t)ribn_amd::kWaveMaxK) {
            // a down projection wider than the SwiGLU prologue stages:
            // silu(gate) * up on its own, then the plain slice-split product
            float* gu_out[2] = {d->gate, d->up};
            e = wave_shared(d, gu, gu_out, 2, d->hidden, L.ffn_norm, members, stream, &pending);
            if (e != hipSuccess) return e;
            e = ribn_amd::launch_swiglu(d->gate, d->up, d->gate, (size_t)members * c.ffn, stream);
            if (e != hipSuccess) return e;
            e = wave(d, &L.ffn_down, 1, d->gate, nullptr, nullptr, &d->hidden, members, true, stream, false, nullptr,
                     &pending);
        } else {
            float* gu_out[2] = {d->gate, d->up};
            e = wave_shared(d, gu, gu_out, 2, d->hidden, L.ffn_norm, members, stream, &pending);
            if (e != hipSuccess) return e;
            e = wave(d, &L.ffn_down, 1, d->gate, d->up, nullptr, &d->hidden, members, true, stream, false, nullptr,
                     &pending);
        }
        if (e != hipSuccess) return e;
    }
    if (!key.head) return ribn_amd::launch_f32mma_fold_flush(&pending, stream);
    e = wave(d, &d->output, 1, d->hidden, nullptr, d->output_norm, &d->logits, members, false, stream, false,
             &pending);
    if (e != hipSuccess) return e;
    return ribn_amd::launch_argmax(d->logits, (int)c.vocab, members, d->selected, d->tokens,
                                   key.advance ? d->positions : nullptr, d->steps, d->history,
                                   (int)d->history_steps, d->argmax_part, stream);
}

void destroy_graphs(ribn_amd_qwen3_decode* d) {
    for (GraphEntry& g : d->graph_cache) {
        hipGraphExecDestroy(g.exec);
        hipGraphDestroy(g.graph);
    }
    d->graph_cache.clear();
}

// Runs one step of the uploaded members on the context stream: replays
// (capturing on first use) the step's graph, or launches directly when graphs
// are off.
ribn_amd_status run_step(ribn_amd_qwen3_decode* d, int members, bool head, bool advance, bool appended = false) {
    hipStream_t stream = d->ctx->stream;
    const GraphKey key{members, head, advance, appended, d->chunks};
    if (!d->graphs) {
        hipError_t e = enqueue_step(d, key, stream);
        return e == hipSuccess ? ok() : driver(e, "launch decode step");
    }
    GraphEntry* hit = nullptr;
    for (GraphEntry& g : d->graph_cache) {
        if (g.key == key) {
            hit = &g;
            break;
        }
    }
    if (hit == nullptr) {
        if (d->graph_cache.size() >= kMaxGraphs) {
            hipError_t e = hipStreamSynchronize(stream);
            if (e != hipSuccess) return driver(e, "hipStreamSynchronize");
            hipGraphExecDestroy(d->graph_cache.front().exec);
            hipGraphDestroy(d->graph_cache.front().graph);
            d->graph_cache.erase(d->graph_cache.begin());
        }
        hipError_t e = hipStreamBeginCapture(d->capture, hipStreamCaptureModeRelaxed);
        if (e != hipSuccess) return driver(e, "hipStreamBeginCapture");
        const hipError_t le = enqueue_step(d, key, d->capture);
        hipGraph_t graph = nullptr;
        e = hipStreamEndCapture(d->capture, &graph);
        if (le != hipSuccess || e != hipSuccess) {
            if (graph) hipGraphDestroy(graph);
            return driver(le != hipSuccess ? le : e, "capture decode step");
        }
        hipGraphExec_t exec = nullptr;
        e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            hipGraphDestroy(graph);
            return driver(e, "hipGraphInstantiate");
        }
        d->graph_cache.push_back(GraphEntry{key, graph, exec});
        hit = &d->graph_cache.back();
    }
    hipError_t e = hipGraphLaunch(hit->exec, stream);
    return e == hipSuccess ? ok() : driver(e, "hipGraphLaunch");
}

ribn_amd_status check_weight(const ribn_amd_context* ctx, const ribn_amd_quantized_weight* w, uint64_t K, uint64_t N,
                             uint32_t layer, const char* name) {
    if (w == nullptr) return fail(RIBN_AMD_MISSING_TENSOR, 0, 0, "layer %u lacks %s", layer, name);
    if (w->device != ctx->device) {
        return fail(RIBN_AMD_CONTEXT_MISMATCH, (uint64_t)ctx->device, (uint64_t)w->device,
                    "%s of layer %u lives on device %d", name, layer, w->device);
    }
    const uint64_t dims[2] = {w->input_size, w->output_size};
    uint64_t k = 0, n = 0;
    ribn_amd_status st =
        ribn_amd_validate_quantized_geometry(w->value_type, w->value_type, dims, 2, w->encoded_bytes, &k, &n);
    if (st != RIBN_AMD_OK) return st;
    if (k != K || n != N) {
        return fail(RIBN_AMD_INVALID_PLAN, K, k, "%s of layer %u is [%llu, %llu], expected [%llu, %llu]", name, layer,
                    (unsigned long long)k, (unsigned long long)n, (unsigned long long)K, (unsigned long long)N);
    }
    if (w->encoded_bytes > 0xffffffffull) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, 0xffffffffull, w->encoded_bytes, "%s of layer %u exceeds 4 GiB", name,
                    layer);
    }
    return RIBN_AMD_OK;
}

// Validates one step's members: caches of this decoder's geometry on its
// device, distinct unless `shared` (one sequence's consecutive tokens); tokens
// in the vocabulary; positions (plus `extra` further steps) within each cache.
ribn_amd_status check_members(const ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* const* caches,
                              const uint32_t* tokens, const uint32_t* positions, size_t members, uint32_t extra,
                              bool shared = false) {
    if (members == 0) return fail(RIBN_AMD_INPUT_LENGTH, 1, 0, "a step needs at least one member");
    if (members > d->max_members) {
        return fail(RIBN_AMD_INVALID_PLAN, d->max_members, members, "the decoder was built for %u members",
                    d->max_members);
    }
    for (size_t m = 0; m < members; ++m) {
        const ribn_amd_kv_cache* c = caches[m];
        if (c == nullptr) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "member %zu has no KV cache", m);
        if (c->device != d->ctx->device) {
            return fail(RIBN_AMD_CONTEXT_MISMATCH, (uint64_t)d->ctx->device, (uint64_t)c->device,
                        "member %zu's cache lives on device %d", m, c->device);
        }
        if (!same_geometry(c->cfg, d->cfg)) {
            return fail(RIBN_AMD_INVALID_PLAN, 0, 0, "member %zu's cache has another layer or head geometry", m);
        }
        for (size_t o = 0; o < m && !shared; ++o) {
            if (caches[o] == c) return fail(RIBN_AMD_INVALID_PLAN, o, m, "members %zu and %zu share a cache", o, m);
        }
        if (tokens[m] >= d->cfg.vocab) {
            return fail(RIBN_AMD_INVALID_PLAN, d->cfg.vocab, tokens[m], "token %u is outside vocabulary %u",
                        tokens[m], d->cfg.vocab);
        }
        if ((uint64_t)positions[m] + extra >= c->capacity) {
            return fail(RIBN_AMD_POSITION_OVERFLOW, c->capacity, (uint64_t)positions[m] + extra,
                        "token position %llu exceeds KV capacity %u", (unsigned long long)positions[m] + extra,
                        c->capacity);
        }
    }
    return RIBN_AMD_OK;
}

ribn_amd::AttnMember descriptor(const ribn_amd_kv_cache* c, float* partials) {
    ribn_amd::AttnMember m{};
    m.keys = c->keys;
    m.values = c->values;
    m.partials = partials;
    m.layer_elems = c->layer_elems;
    m.capacity = (int)c->capacity;
    return m;
}

// Stream-ordered upload of the members' cache descriptors (with the
// decoder's per-member partials), tokens and positions through kernel
// arguments; records the step's attention grid. Nothing waits on the host.
ribn_amd_status upload_step(ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* const* caches, const uint32_t* tokens,
                            const uint32_t* positions, size_t members) {
    const size_t part = ribn_amd::attn_partials_floats((int)d->cfg.q_heads);
    int max_capacity = 1;
    for (size_t m0 = 0; m0 < members; m0 += ribn_amd::kStepInputs) {
        ribn_amd::StepInputs in{};
        in.count = (int)std::min<size_t>(ribn_amd::kStepInputs, members - m0);
        for (int i = 0; i < in.count; ++i) {
            const size_t m = m0 + i;
            in.mem[i] = descriptor(caches[m], d->partials + m * part);
            in.tokens[i] = tokens[m];
            in.positions[i] = (int32_t)positions[m];
            max_capacity = std::max(max_capacity, (int)caches[m]->capacity);
        }
        in.mem_dst = d->members_dev + m0;
        in.tokens_dst = d->tokens + m0;
        in.positions_dst = d->positions + m0;
        hipError_t e = ribn_amd::launch_step_inputs(in, d->ctx->stream);
        if (e != hipSuccess) return driver(e, "upload step inputs");
    }
    d->chunks = ribn_amd::attn_grid_chunks(max_capacity, (int)members);
    return ok();
}

// Prompt workspace for chunks of `tokens` tokens (grows, never shrinks;
// synchronises the context stream when it replaces the block).
ribn_amd_status reserve_prompt(ribn_amd_qwen3_decode* d, uint32_t tokens) {
    if (d->prompt_block != nullptr && d->prompt_tokens >= tokens) return ok();
    const ribn_amd_qwen3_config& c = d->cfg;
    const size_t T = tokens;
    const size_t qdim = (size_t)c.q_heads * c.head_dim, kvdim = (size_t)c.kv_heads * c.head_dim;
    const size_t max_k = std::max<size_t>({c.hidden, qdim, c.ffn});
    const size_t max_n = std::max<size_t>({c.hidden, qdim, c.ffn});
    const size_t f32_counts[8] = {T * c.hidden, T * qdim, T * kvdim, T * kvdim, T * qdim, T * c.ffn, T * c.ffn,
                                  T * c.hidden};
    size_t bytes = align_up(T * sizeof(uint32_t));
    size_t offsets[8];
    for (int i = 0; i < 8; ++i) {
        offsets[i] = bytes;
        bytes += align_up(f32_counts[i] * sizeof(float));
    }
    const size_t gemm_offset = bytes;
    // activations at the widest K, and split-K room for two partial tiles of
    // up to 512 tokens (grids of more tokens fill the CUs without a split)
    const size_t gemm_bytes = ribn_amd::gemm_workspace_bytes(T, max_k, 0) +
                              align_up(2 * std::min<size_t>(T, 512) * max_n * sizeof(float));
    bytes += gemm_bytes;
    hipError_t e = hipStreamSynchronize(d->ctx->stream);
    if (e != hipSuccess) return driver(e, "synchronize before replacing the prompt workspace");
    if (d->prompt_block != nullptr) {
        hipFree(d->prompt_block);
        d->prompt_block = nullptr;
        d->prompt_tokens = 0;
    }
    void* block = nullptr;
    e = hipMalloc(&block, bytes);
    if (e != hipSuccess) return driver(e, "hipMalloc prompt workspace");
    char* p = static_cast<char*>(block);
    d->prompt_block = block;
    d->prompt_bytes = bytes;
    d->prompt_tokens = tokens;
    d->p_tokens = reinterpret_cast<uint32_t*>(p);
    float** f32s[8] = {&d->p_hidden, &d->p_q, &d->p_k, &d->p_v, &d->p_attn, &d->p_gate, &d->p_up, &d->p_y};
    for (int i = 0; i < 8; ++i) *f32s[i] = reinterpret_cast<float*>(p + offsets[i]);
    d->p_gemm = p + gemm_offset;
    d->p_gemm_bytes = gemm_bytes;
    return ok();
}

// One prefill-matmul projection of the prompt chunk: y[T][N] = x W^T from the
// f16 activations the last activation stage left in the workspace.
hipError_t prompt_gemm(ribn_amd_qwen3_decode* d, const ribn_amd_quantized_weight* w, float* y, int tokens,
                       hipStream_t stream) {
    return ribn_amd::launch_qgemm((int)w->value_type, w->data, (uint32_t)w->encoded_bytes, d->p_gemm, d->p_gemm_bytes,
                                  y, tokens, (int)w->output_size, (int)w->input_size, d->ctx->cu_count, stream);
}

// The launches of one prompt chunk: `tokens` tokens at positions p0.. of
// `cache`, their ids already in p_tokens.
hipError_t enqueue_prompt_chunk(ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* cache, int tokens, int p0,
                                hipStream_t stream) {
    const ribn_amd_qwen3_config& c = d->cfg;
    const int qdim = (int)(c.q_heads * c.head_dim);
    hipError_t e = ribn_amd::launch_embedding((int)d->token_embd->value_type, d->token_embd->data,
                                              (uint32_t)d->token_embd->encoded_bytes, d->p_tokens, 0, d->p_hidden,
                                              c.hidden / 256, c.vocab, (uint32_t)tokens, stream);
    for (uint32_t l = 0; l < c.layers && e == hipSuccess; ++l) {
        const ribn_amd_qwen3_layer& L = d->layers[l];
        // The last layer's attention output, o projection and FFN reach no
        // cache (there is no output head here): only its K/V are computed.
        const bool last = l + 1 == c.layers;
        e = l == 0 ? ribn_amd::launch_act_f16(false, d->p_hidden, L.attn_norm, c.epsilon, tokens, (int)c.hidden,
                                              d->p_gemm, stream)
                   : ribn_amd::launch_act_f16_residual(d->p_hidden, d->p_y, L.attn_norm, c.epsilon, tokens,
                                                       (int)c.hidden, d->p_gemm, stream);
        if (e == hipSuccess && !last) e = prompt_gemm(d, L.attn_q, d->p_q, tokens, stream);
        if (e == hipSuccess) e = prompt_gemm(d, L.attn_k, d->p_k, tokens, stream);
        if (e == hipSuccess) e = prompt_gemm(d, L.attn_v, d->p_v, tokens, stream);
        if (e != hipSuccess) break;
        ribn_amd::PrefillAttnArgs a{};
        a.mem = descriptor(cache, nullptr);
        a.layer = (int)l;
        a.p0 = p0;
        a.tokens = tokens;
        a.q = d->p_q;
        a.k = d->p_k;
        a.v = d->p_v;
        a.q_norm = L.attn_q_norm;
        a.k_norm = L.attn_k_norm;
        a.out = last ? nullptr : d->p_attn;
        a.q_heads = (int)c.q_heads;
        a.kv_heads = (int)c.kv_heads;
        a.eps = c.epsilon;
        a.rope_base = c.rope_base;
        a.scale = 1.4426950408889634f / sqrtf((float)c.head_dim);
        e = ribn_amd::launch_prefill_attention(a, stream);
        if (e != hipSuccess || last) break;
        e = ribn_amd::launch_act_f16(false, d->p_attn, nullptr, 0.f, tokens, qdim, d->p_gemm, stream);
        if (e == hipSuccess) e = prompt_gemm(d, L.attn_output, d->p_y, tokens, stream);
        if (e == hipSuccess) {
            e = ribn_amd::launch_act_f16_residual(d->p_hidden, d->p_y, L.ffn_norm, c.epsilon, tokens, (int)c.hidden,
                                                  d->p_gemm, stream);
        }
        if (e == hipSuccess) e = prompt_gemm(d, L.ffn_gate, d->p_gate, tokens, stream);
        if (e == hipSuccess) e = prompt_gemm(d, L.ffn_up, d->p_up, tokens, stream);
        if (e == hipSuccess) e = ribn_amd::launch_act_f16_swiglu(d->p_gate, d->p_up, tokens, (int)c.ffn, d->p_gemm, stream);
        if (e == hipSuccess) e = prompt_gemm(d, L.ffn_down, d->p_y, tokens, stream);
    }
    return e;
}

constexpr uint32_t kPromptChunkDefault = 2048;
constexpr uint32_t kPromptChunkMin = 16;
constexpr uint32_t kPromptChunkMax = 2048;

ribn_amd_status check_prompt_chunk(uint32_t chunk) {
    if (chunk < kPromptChunkMin || chunk > kPromptChunkMax) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, kPromptChunkMax, chunk, "prompt chunks take %u..%u tokens, not %u",
                    kPromptChunkMin, kPromptChunkMax, chunk);
    }
    return RIBN_AMD_OK;
}

// Dimensions the prefill matmul serves (K up to kGemmMaxK, multiples of 256).
ribn_amd_status check_prompt_geometry(const ribn_amd_qwen3_config& c) {
    const uint64_t qdim = (uint64_t)c.q_heads * c.head_dim;
    const uint64_t ks[3] = {c.hidden, qdim, c.ffn};
    for (uint64_t k : ks) {
        if (k > (uint64_t)ribn_amd::kGemmMaxK || k % 256 != 0) {
            return fail(RIBN_AMD_INVALID_PLAN, ribn_amd::kGemmMaxK, k,
                        "the prompt prefill matmul takes K <= %d in whole super-blocks, not %llu", ribn_amd::kGemmMaxK,
                        (unsigned long long)k);
        }
    }
    return RIBN_AMD_OK;
}

}  // namespace

namespace ribn_amd_decode {

ribn_amd_status enqueue_decode(ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* const* caches, const uint32_t* tokens,
                               const uint32_t* positions, size_t members) {
    if (!d || !caches || !tokens || !positions) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    ribn_amd_status st = check_members(d, caches, tokens, positions, members, 0);
    if (st != RIBN_AMD_OK) return st;
    DeviceGuard guard(d->ctx->device);
    st = upload_step(d, caches, tokens, positions, members);
    return st == RIBN_AMD_OK ? run_step(d, (int)members, true, false) : st;
}

ribn_amd_status enqueue_prefill_chunk(ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* cache, const uint32_t* tokens,
                                      size_t count, uint32_t position) {
    if (!d || !cache || !tokens) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (count < 2) return fail(RIBN_AMD_INPUT_LENGTH, 2, count, "a prefill chunk takes at least two tokens");
    if (count > d->max_members) {
        return fail(RIBN_AMD_INVALID_PLAN, d->max_members, count, "the decoder was built for %u members",
                    d->max_members);
    }
    if ((uint64_t)position + count > 0x7fffffffull) {
        return fail(RIBN_AMD_POSITION_OVERFLOW, 0x7fffffffull, (uint64_t)position + count,
                    "prefill chunk positions overflow");
    }
    std::vector<ribn_amd_kv_cache*> caches(count, cache);
    std::vector<uint32_t> positions(count);
    for (size_t m = 0; m < count; ++m) positions[m] = position + (uint32_t)m;
    ribn_amd_status st = check_members(d, caches.data(), tokens, positions.data(), count, 0, true);
    if (st != RIBN_AMD_OK) return st;
    DeviceGuard guard(d->ctx->device);
    st = upload_step(d, caches.data(), tokens, positions.data(), count);
    return st == RIBN_AMD_OK ? run_step(d, (int)count, false, false, true) : st;
}

ribn_amd_status copy_selected_async(ribn_amd_qwen3_decode* d, size_t member, uint32_t* pinned) {
    if (!d || !pinned) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (member >= d->max_members) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, d->max_members, member, "member %zu of %u", member, d->max_members);
    }
    DeviceGuard guard(d->ctx->device);
    hipError_t e = hipMemcpyAsync(pinned, d->selected + member, sizeof(uint32_t), hipMemcpyDeviceToHost,
                                  d->ctx->stream);
    return e == hipSuccess ? ok() : driver(e, "copy selected token into pinned memory");
}

ribn_amd_context* context(const ribn_amd_qwen3_decode* d) { return d->ctx; }
uint32_t max_members(const ribn_amd_qwen3_decode* d) { return d->max_members; }
const ribn_amd_qwen3_config& config(const ribn_amd_qwen3_decode* d) { return d->cfg; }

}  // namespace ribn_amd_decode

extern "C" {

ribn_amd_status ribn_amd_kv_cache_create(ribn_amd_context* ctx, const ribn_amd_qwen3_config* config,
                                         uint32_t capacity, ribn_amd_kv_cache** out) {
    if (!ctx || !out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    ribn_amd_status st = check_config(config);
    if (st != RIBN_AMD_OK) return st;
    if (capacity == 0 || capacity > (1u << 20)) {
        return fail(RIBN_AMD_INVALID_PLAN, 1u << 20, capacity, "KV capacity must be 1..%u tokens", 1u << 20);
    }
    const size_t layer_elems = (size_t)config->kv_heads * capacity * config->head_dim;
    const size_t cache_bytes = align_up(layer_elems * config->layers * sizeof(uint16_t));
    const size_t part_bytes = align_up(ribn_amd::attn_partials_floats((int)config->q_heads) * sizeof(float));
    DeviceGuard guard(ctx->device);
    void* block = nullptr;
    hipError_t e = hipMalloc(&block, 2 * cache_bytes + part_bytes);
    if (e != hipSuccess) return driver(e, "hipMalloc KV cache");
    char* p = static_cast<char*>(block);
    auto* c = new (std::nothrow) ribn_amd_kv_cache{};
    if (!c) {
        hipFree(block);
        return fail(RIBN_AMD_DRIVER, 0, 0, "host allocation failed");
    }
    c->ctx = ctx;
    c->device = ctx->device;
    c->id = g_cache_ids.fetch_add(1);
    c->cfg = *config;
    c->capacity = capacity;
    c->layer_elems = layer_elems;
    c->block = block;
    c->keys = reinterpret_cast<uint16_t*>(p);
    c->values = reinterpret_cast<uint16_t*>(p + cache_bytes);
    c->partials = reinterpret_cast<float*>(p + 2 * cache_bytes);
    // nothing is cleared: a position is written before it is read, and every
    // partial is written before the merge reads it
    context_retain(ctx);  // released by ribn_amd_kv_cache_destroy, like every other handle's
    *out = c;
    return ok();
}

void ribn_amd_kv_cache_destroy(ribn_amd_kv_cache* cache) {
    if (!cache) return;
    ribn_amd_context* ctx = cache->ctx;
    {
        DeviceGuard guard(cache->device);
        hipFree(cache->block);  // waits for outstanding work on the device
    }
    delete cache;
    context_release(ctx);
}

uint32_t ribn_amd_kv_cache_capacity(const ribn_amd_kv_cache* cache) { return cache ? cache->capacity : 0; }

ribn_amd_status ribn_amd_kv_cache_layer(ribn_amd_kv_cache* cache, uint32_t layer, uint16_t** keys, uint16_t** values) {
    if (!cache || !keys || !values) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (layer >= cache->cfg.layers) {
        return fail(RIBN_AMD_INVALID_PLAN, cache->cfg.layers, layer, "layer %u of a %u-layer cache", layer,
                    cache->cfg.layers);
    }
    *keys = cache->keys + (size_t)layer * cache->layer_elems;
    *values = cache->values + (size_t)layer * cache->layer_elems;
    return ok();
}

ribn_amd_status ribn_amd_attention_prefill(ribn_amd_context* ctx, const ribn_amd_qwen3_config* config,
                                           ribn_amd_kv_cache* cache, uint32_t layer, const float* q, const float* k,
                                           const float* v, const float* q_norm, const float* k_norm, size_t tokens,
                                           uint32_t position, float* output, size_t output_len) {
    if (!ctx || !cache) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    ribn_amd_status st = check_config(config);
    if (st != RIBN_AMD_OK) return st;
    const void* ptrs[6] = {q, k, v, q_norm, k_norm, output};
    const char* names[6] = {"q", "k", "v", "q_norm", "k_norm", "output"};
    for (int i = 0; i < 6; ++i) {
        st = check_device_ptr(ctx, ptrs[i], names[i], 16);
        if (st != RIBN_AMD_OK) return st;
    }
    if (cache->device != ctx->device) {
        return fail(RIBN_AMD_CONTEXT_MISMATCH, (uint64_t)ctx->device, (uint64_t)cache->device,
                    "the cache lives on device %d", cache->device);
    }
    if (!same_geometry(cache->cfg, *config) || layer >= cache->cfg.layers) {
        return fail(RIBN_AMD_INVALID_PLAN, cache->cfg.layers, layer, "the cache does not hold layer %u", layer);
    }
    if (tokens == 0) return fail(RIBN_AMD_INPUT_LENGTH, 1, 0, "a prompt chunk needs at least one token");
    if ((uint64_t)position + tokens > cache->capacity) {
        return fail(RIBN_AMD_POSITION_OVERFLOW, cache->capacity, (uint64_t)position + tokens - 1,
                    "token position %llu exceeds KV capacity %u", (unsigned long long)position + tokens - 1,
                    cache->capacity);
    }
    const size_t want = tokens * config->q_heads * config->head_dim;
    if (output_len != want) {
        return fail(RIBN_AMD_OUTPUT_LENGTH, want, output_len, "attention output has %zu values, expected %zu",
                    output_len, want);
    }
    DeviceGuard guard(ctx->device);
    ribn_amd::PrefillAttnArgs a{};
    a.mem = descriptor(cache, nullptr);
    a.layer = (int)layer;
    a.p0 = (int)position;
    a.tokens = (int)tokens;
    a.q = q;
    a.k = k;
    a.v = v;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.out = output;
    a.q_heads = (int)config->q_heads;
    a.kv_heads = (int)config->kv_heads;
    a.eps = config->epsilon;
    a.rope_base = config->rope_base;
    a.scale = 1.4426950408889634f / sqrtf((float)config->head_dim);
    hipError_t e = ribn_amd::launch_prefill_attention(a, ctx->stream);
    return e == hipSuccess ? ok() : driver(e, "prompt attention launch");
}

ribn_amd_status ribn_amd_attention_decode(ribn_amd_context* ctx, const ribn_amd_qwen3_config* config,
                                          ribn_amd_kv_cache* const* caches, size_t members, uint32_t layer,
                                          const float* q, const float* k, const float* v, const float* q_norm,
                                          const float* k_norm, const int32_t* positions, float* output,
                                          size_t output_len) {
    if (!ctx || !caches) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    ribn_amd_status st = check_config(config);
    if (st != RIBN_AMD_OK) return st;
    if (members == 0 || members > RIBN_AMD_MAX_BATCH_MEMBERS) {
        return fail(RIBN_AMD_INPUT_LENGTH, RIBN_AMD_MAX_BATCH_MEMBERS, members, "attention takes 1..%u members",
                    RIBN_AMD_MAX_BATCH_MEMBERS);
    }
    const void* ptrs[7] = {q, k, v, q_norm, k_norm, positions, output};
    const char* names[7] = {"q", "k", "v", "q_norm", "k_norm", "positions", "output"};
    for (int i = 0; i < 7; ++i) {
        st = check_device_ptr(ctx, ptrs[i], names[i], i == 5 ? 4 : 16);
        if (st != RIBN_AMD_OK) return st;
    }
    for (size_t m = 0; m < members; ++m) {
        const ribn_amd_kv_cache* c = caches[m];
        if (c == nullptr) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "member %zu has no KV cache", m);
        if (c->device != ctx->device) {
            return fail(RIBN_AMD_CONTEXT_MISMATCH, (uint64_t)ctx->device, (uint64_t)c->device,
                        "member %zu's cache lives on device %d", m, c->device);
        }
        if (!same_geometry(c->cfg, *config) || layer >= c->cfg.layers) {
            return fail(RIBN_AMD_INVALID_PLAN, c->cfg.layers, layer, "member %zu's cache does not hold layer %u", m,
                        layer);
        }
        for (size_t o = 0; o < m; ++o) {
            if (caches[o] == c) return fail(RIBN_AMD_INVALID_PLAN, o, m, "members %zu and %zu share a cache", o, m);
        }
    }
    const size_t want = members * config->q_heads * config->head_dim;
    if (output_len != want) {
        return fail(RIBN_AMD_OUTPUT_LENGTH, want, output_len, "attention output has %zu values, expected %zu",
                    output_len, want);
    }
    DeviceGuard guard(ctx->device);
    // the members' descriptors go to the context's descriptor array, in
    // stream order ahead of the launches that read them
    auto* mem = static_cast<ribn_amd::AttnMember*>(ctx->attn_members);
    int max_capacity = 1;
    for (size_t m0 = 0; m0 < members; m0 += ribn_amd::kStepInputs) {
        ribn_amd::StepInputs in{};
        in.count = (int)std::min<size_t>(ribn_amd::kStepInputs, members - m0);
        for (int i = 0; i < in.count; ++i) {
            in.mem[i] = descriptor(caches[m0 + i], caches[m0 + i]->partials);
            max_capacity = std::max(max_capacity, (int)caches[m0 + i]->capacity);
        }
        in.mem_dst = mem + m0;
        hipError_t e = ribn_amd::launch_step_inputs(in, ctx->stream);
        if (e != hipSuccess) return driver(e, "upload attention descriptors");
    }
    // Positions are device values: the kernel checks them against each cache
    // and drops an append past its capacity.
    const int chunks = ribn_amd::attn_grid_chunks(max_capacity, (int)members);
    hipError_t e = attention(*config, mem, chunks, false, (int)members, layer, q, k, v, q_norm, k_norm, positions,
                             output, nullptr, ctx->stream);
    return e == hipSuccess ? ok() : driver(e, "launch attention");
}

ribn_amd_status ribn_amd_argmax(ribn_amd_context* ctx, const float* logits, size_t logits_len, size_t length,
                                uint32_t* selected) {
    if (!ctx) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null context");
    ribn_amd_status st = check_device_ptr(ctx, logits, "logits", 4);
    if (st == RIBN_AMD_OK) st = check_device_ptr(ctx, selected, "selected", 4);
    if (st != RIBN_AMD_OK) return st;
    // model_ops.rs:1583-1674: empty logits, then rows of `length`
    if (logits_len == 0 || length == 0) return fail(RIBN_AMD_EMPTY_INPUT, 1, 0, "argmax input is empty");
    if (logits_len % length != 0) {
        return fail(RIBN_AMD_INPUT_LENGTH, logits_len, length, "logits of %zu values are not rows of %zu", logits_len,
                    length);
    }
    const size_t members = logits_len / length;
    if (length > (size_t)std::numeric_limits<int>::max() || members > 65535) {
        return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "argmax shape exceeds launch limits");
    }
    DeviceGuard guard(ctx->device);
    // The slice results live in the context's activation scratch (stream
    // ordered with every other user of it), in groups of members that fit.
    const size_t group = ribn_amd::gemv_act_scratch_bytes() / (ribn_amd::kArgmaxSlices * sizeof(uint64_t));
    auto* part = static_cast<uint64_t*>(ctx->act_scratch);
    for (size_t m0 = 0; m0 < members; m0 += group) {
        const int mc = (int)std::min(group, members - m0);
        hipError_t e = ribn_amd::launch_argmax(logits + m0 * length, (int)length, mc, selected + m0, nullptr, nullptr,
                                               nullptr, nullptr, 0, part, ctx->stream);
        if (e != hipSuccess) return driver(e, "launch argmax");
    }
    return ok();
}

ribn_amd_status ribn_amd_qwen3_decode_create(ribn_amd_context* ctx, const ribn_amd_qwen3_config* config,
                                             const ribn_amd_quantized_weight* token_embd,
                                             const ribn_amd_quantized_weight* output, const float* output_norm,
                                             const ribn_amd_qwen3_layer* layers, uint32_t max_members,
                                             ribn_amd_qwen3_decode** out) {
    if (!ctx || !out || !layers) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    ribn_amd_status st = check_config(config);
    if (st != RIBN_AMD_OK) return st;
    const ribn_amd_qwen3_config& c = *config;
    if (max_members == 0 || max_members > RIBN_AMD_MAX_BATCH_MEMBERS) {
        return fail(RIBN_AMD_INVALID_PLAN, RIBN_AMD_MAX_BATCH_MEMBERS, max_members, "max_members must be 1..%u",
                    RIBN_AMD_MAX_BATCH_MEMBERS);
    }
    const uint64_t qdim = (uint64_t)c.q_heads * c.head_dim;
    const uint64_t kvdim = (uint64_t)c.kv_heads * c.head_dim;
    // token_embd.weight / output.weight / output_norm.weight (decode.rs:572-576, 662-675)
    st = check_weight(ctx, token_embd, c.hidden, c.vocab, 0, "token_embd");
    if (st == RIBN_AMD_OK) st = check_weight(ctx, output, c.hidden, c.vocab, 0, "output");
    if (st != RIBN_AMD_OK) return st;
    if (output_norm == nullptr) return fail(RIBN_AMD_MISSING_TENSOR, 0, 0, "the plan lacks output_norm");
    st = check_device_ptr(ctx, output_norm, "output_norm");
    if (st != RIBN_AMD_OK) return st;
    for (uint32_t l = 0; l < c.layers; ++l) {
        const ribn_amd_qwen3_layer& L = layers[l];
        struct {
            const ribn_amd_quantized_weight* w;
            uint64_t K, N;
            const char* name;
        } ws[7] = {{L.attn_q, c.hidden, qdim, "attn_q"},        {L.attn_k, c.hidden, kvdim, "attn_k"},
                   {L.attn_v, c.hidden, kvdim, "attn_v"},       {L.attn_output, qdim, c.hidden, "attn_output"},
                   {L.ffn_gate, c.hidden, c.ffn, "ffn_gate"},   {L.ffn_up, c.hidden, c.ffn, "ffn_up"},
                   {L.ffn_down, c.ffn, c.hidden, "ffn_down"}};
        for (auto& w : ws) {
            st = check_weight(ctx, w.w, w.K, w.N, l, w.name);
            if (st != RIBN_AMD_OK) return st;
        }
        const float* norms[4] = {L.attn_norm, L.attn_q_norm, L.attn_k_norm, L.ffn_norm};
        const char* norm_names[4] = {"attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm"};
        for (int i = 0; i < 4; ++i) {
            if (norms[i] == nullptr) return fail(RIBN_AMD_MISSING_TENSOR, 0, 0, "layer %u lacks %s", l, norm_names[i]);
            st = check_device_ptr(ctx, norms[i], norm_names[i]);
            if (st != RIBN_AMD_OK) return st;
        }
    }

    const size_t M = max_members;
    const size_t f32_counts[8] = {M * c.hidden, M * qdim, M * kvdim, M * kvdim, M * qdim, M * c.ffn, M * c.ffn,
                                  M * c.vocab};
    size_t bytes = 0;
    size_t offsets[12];
    for (int i = 0; i < 8; ++i) {
        offsets[i] = bytes;
        bytes += align_up(f32_counts[i] * sizeof(float));
    }
    for (int i = 8; i < 12; ++i) {  // tokens, selected, positions, steps
        offsets[i] = bytes;
        bytes += align_up(M * sizeof(uint32_t));
    }
    const size_t members_offset = bytes;
    bytes += align_up(M * sizeof(ribn_amd::AttnMember));
    const size_t partials_offset = bytes;
    bytes += align_up(M * ribn_amd::attn_partials_floats((int)c.q_heads) * sizeof(float));
    const size_t argmax_offset = bytes;
    bytes += align_up(M * ribn_amd::kArgmaxSlices * sizeof(uint64_t));
    DeviceGuard guard(ctx->device);
    auto* d = new (std::nothrow) ribn_amd_qwen3_decode{};
    if (!d) return fail(RIBN_AMD_DRIVER, 0, 0, "host allocation failed");
    d->ctx = ctx;
    d->cfg = c;
    d->max_members = max_members;
    d->token_embd = token_embd;
    d->output = output;
    d->output_norm = output_norm;
    d->layers.assign(layers, layers + c.layers);
    d->graphs = true;
    d->gemv_mode = RIBN_AMD_GEMV_WARP;
    hipError_t e = hipMalloc(&d->block, bytes);
    if (e != hipSuccess) {
        delete d;
        return driver(e, "hipMalloc decode buffers");
    }
    char* p = static_cast<char*>(d->block);
    float** f32s[8] = {&d->hidden, &d->q, &d->k, &d->v, &d->attn, &d->gate, &d->up, &d->logits};
    for (int i = 0; i < 8; ++i) *f32s[i] = reinterpret_cast<float*>(p + offsets[i]);
    d->tokens = reinterpret_cast<uint32_t*>(p + offsets[8]);
    d->selected = reinterpret_cast<uint32_t*>(p + offsets[9]);
    d->positions = reinterpret_cast<int32_t*>(p + offsets[10]);
    d->steps = reinterpret_cast<int32_t*>(p + offsets[11]);
    d->members_dev = reinterpret_cast<ribn_amd::AttnMember*>(p + members_offset);
    d->partials = reinterpret_cast<float*>(p + partials_offset);
    d->argmax_part = reinterpret_cast<uint64_t*>(p + argmax_offset);
    d->chunks = 1;
    d->history_steps = 256;
    e = hipMalloc(&d->history, M * d->history_steps * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemsetAsync(d->block, 0, bytes, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&d->capture, hipStreamNonBlocking);
    if (e != hipSuccess) {
        if (d->history) hipFree(d->history);
        hipFree(d->block);
        delete d;
        return driver(e, "set up decode buffers");
    }
    context_retain(ctx);
    *out = d;
    return ok();
}

void ribn_amd_qwen3_decode_destroy(ribn_amd_qwen3_decode* d) {
    if (!d) return;
    DeviceGuard guard(d->ctx->device);
    hipStreamSynchronize(d->ctx->stream);
    destroy_graphs(d);
    hipStreamDestroy(d->capture);
    hipFree(d->history);
    hipFree(d->block);
    if (d->prompt_block) hipFree(d->prompt_block);
    ribn_amd_context* ctx = d->ctx;
    delete d;
    context_release(ctx);
}

ribn_amd_status ribn_amd_qwen3_decode_set_graphs(ribn_amd_qwen3_decode* d, int32_t enabled) {
    if (!d) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null decoder");
    d->graphs = enabled != 0;
    return ok();
}

ribn_amd_status ribn_amd_qwen3_decode_set_gemv_mode(ribn_amd_qwen3_decode* d, uint32_t mode) {
    if (!d) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null decoder");
    if (mode != RIBN_AMD_GEMV_WARP && mode != RIBN_AMD_GEMV_FIXED16) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, RIBN_AMD_GEMV_FIXED16, mode, "unknown GEMV mode %u", mode);
    }
    if (mode != d->gemv_mode) {
        DeviceGuard guard(d->ctx->device);
        hipError_t e = hipStreamSynchronize(d->ctx->stream);
        if (e != hipSuccess) return driver(e, "synchronize before a GEMV mode change");
        destroy_graphs(d);  // captured with the other mode's kernels
        d->gemv_mode = mode;
    }
    return ok();
}

uint32_t ribn_amd_qwen3_decode_gemv_mode(const ribn_amd_qwen3_decode* d) {
    return d ? d->gemv_mode : RIBN_AMD_GEMV_WARP;
}

ribn_amd_status ribn_amd_qwen3_decode_step_batch(ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* const* caches,
                                                 const uint32_t* tokens, const uint32_t* positions, size_t members,
                                                 uint32_t* selected) {
    if (!d || !caches || !tokens || !positions || !selected) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    }
    ribn_amd_status st = check_members(d, caches, tokens, positions, members, 0);
    if (st != RIBN_AMD_OK) return st;
    DeviceGuard guard(d->ctx->device);
    st = upload_step(d, caches, tokens, positions, members);
    if (st != RIBN_AMD_OK) return st;
    st = run_step(d, (int)members, true, false);
    if (st != RIBN_AMD_OK) return st;
    // the reference's blocking token readback (decode.rs:634-645)
    hipError_t e = hipMemcpyAsync(selected, d->selected, members * sizeof(uint32_t), hipMemcpyDeviceToHost,
                                  d->ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->ctx->stream);
    return e == hipSuccess ? ok() : driver(e, "read selected tokens");
}

ribn_amd_status ribn_amd_qwen3_decode_step(ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* cache, uint32_t token,
                                           uint32_t position, uint32_t* selected) {
    ribn_amd_kv_cache* caches[1] = {cache};
    return ribn_amd_qwen3_decode_step_batch(d, caches, &token, &position, 1, selected);
}

ribn_amd_status ribn_amd_qwen3_prefill_step(ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* cache, uint32_t token,
                                            uint32_t position) {
    if (!d || !cache) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    ribn_amd_kv_cache* caches[1] = {cache};
    ribn_amd_status st = check_members(d, caches, &token, &position, 1, 0);
    if (st != RIBN_AMD_OK) return st;
    DeviceGuard guard(d->ctx->device);
    st = upload_step(d, caches, &token, &position, 1);
    return st == RIBN_AMD_OK ? run_step(d, 1, false, false) : st;
}

ribn_amd_status ribn_amd_qwen3_prefill_chunk(ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* cache,
                                             const uint32_t* tokens, size_t count, uint32_t position) {
    return ribn_amd_decode::enqueue_prefill_chunk(d, cache, tokens, count, position);
}

ribn_amd_status ribn_amd_qwen3_reserve_prompt(ribn_amd_qwen3_decode* d, uint32_t chunk_tokens) {
    if (!d) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null decoder");
    if (chunk_tokens == 0) chunk_tokens = kPromptChunkDefault;
    ribn_amd_status st = check_prompt_chunk(chunk_tokens);
    if (st == RIBN_AMD_OK) st = check_prompt_geometry(d->cfg);
    if (st != RIBN_AMD_OK) return st;
    DeviceGuard guard(d->ctx->device);
    return reserve_prompt(d, chunk_tokens);
}

ribn_amd_status ribn_amd_qwen3_prefill_prompt(ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* cache,
                                              const uint32_t* tokens, size_t count, uint32_t position,
                                              uint32_t chunk_tokens) {
    if (!d || !cache || !tokens) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (count == 0) return fail(RIBN_AMD_INPUT_LENGTH, 1, 0, "a prompt prefill needs at least one token");
    if (chunk_tokens == 0) chunk_tokens = kPromptChunkDefault;
    ribn_amd_status st = check_prompt_chunk(chunk_tokens);
    if (st == RIBN_AMD_OK) st = check_prompt_geometry(d->cfg);
    if (st != RIBN_AMD_OK) return st;
    if (cache->device != d->ctx->device) {
        return fail(RIBN_AMD_CONTEXT_MISMATCH, (uint64_t)d->ctx->device, (uint64_t)cache->device,
                    "the cache lives on device %d", cache->device);
    }
    if (!same_geometry(cache->cfg, d->cfg)) {
        return fail(RIBN_AMD_INVALID_PLAN, 0, 0, "the cache has another layer or head geometry");
    }
    if ((uint64_t)position + count > cache->capacity) {
        return fail(RIBN_AMD_POSITION_OVERFLOW, cache->capacity, (uint64_t)position + count - 1,
                    "token position %llu exceeds KV capacity %u", (unsigned long long)position + count - 1,
                    cache->capacity);
    }
    for (size_t i = 0; i < count; ++i) {
        if (tokens[i] >= d->cfg.vocab) {
            return fail(RIBN_AMD_INVALID_PLAN, d->cfg.vocab, tokens[i], "token %u is outside vocabulary %u",
                        tokens[i], d->cfg.vocab);
        }
    }
    DeviceGuard guard(d->ctx->device);
    const uint32_t chunk = (uint32_t)std::min<size_t>(chunk_tokens, count);
    st = reserve_prompt(d, chunk);
    if (st != RIBN_AMD_OK) return st;
    hipStream_t stream = d->ctx->stream;
    for (size_t c0 = 0; c0 < count; c0 += chunk) {
        const int n = (int)std::min<size_t>(chunk, count - c0);
        hipError_t e = ribn_amd::launch_token_upload(tokens + c0, (size_t)n, d->p_tokens, stream);
        if (e == hipSuccess) e = enqueue_prompt_chunk(d, cache, n, (int)(position + c0), stream);
        if (e != hipSuccess) return driver(e, "prompt prefill chunk");
    }
    return ok();
}

ribn_amd_status ribn_amd_qwen3_generate(ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* const* caches,
                                        const uint32_t* tokens, const uint32_t* positions, size_t members,
                                        uint32_t steps, uint32_t* out_tokens) {
    if (!d || !caches || !tokens || !positions || !out_tokens) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    }
    if (steps == 0) return fail(RIBN_AMD_INPUT_LENGTH, 1, 0, "generation needs at least one step");
    ribn_amd_status st = check_members(d, caches, tokens, positions, members, steps - 1);
    if (st != RIBN_AMD_OK) return st;
    DeviceGuard guard(d->ctx->device);
    hipStream_t stream = d->ctx->stream;
    if (steps > d->history_steps) {
        // the history buffer is part of the captured graphs: replace both
        hipError_t e = hipStreamSynchronize(stream);
        if (e != hipSuccess) return driver(e, "hipStreamSynchronize");
        destroy_graphs(d);
        hipFree(d->history);
        d->history = nullptr;
        d->history_steps = 0;
        e = hipMalloc(&d->history, (size_t)d->max_members * steps * sizeof(uint32_t));
        if (e != hipSuccess) return driver(e, "hipMalloc generation history");
        d->history_steps = steps;
    }
    st = upload_step(d, caches, tokens, positions, members);
    if (st != RIBN_AMD_OK) return st;
    std::vector<int32_t> zeros(members, 0);
    hipError_t e = hipMemcpyAsync(d->steps, zeros.data(), members * sizeof(int32_t), hipMemcpyHostToDevice, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return driver(e, "reset generation counters");
    for (uint32_t s = 0; s < steps; ++s) {
        st = run_step(d, (int)members, true, true);
        if (st != RIBN_AMD_OK) return st;
    }
    for (size_t m = 0; m < members; ++m) {
        e = hipMemcpyAsync(out_tokens + m * steps, d->history + m * d->history_steps, steps * sizeof(uint32_t),
                           hipMemcpyDeviceToHost, stream);
        if (e != hipSuccess) return driver(e, "read generated tokens");
    }
    e = hipStreamSynchronize(stream);
    return e == hipSuccess ? ok() : driver(e, "hipStreamSynchronize");
}

static ribn_amd_status copy_member(ribn_amd_qwen3_decode* d, const float* base, size_t width, size_t member,
                                   float* host, size_t len) {
    if (!d || !host) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (member >= d->max_members) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, d->max_members, member, "member %zu of %u", member, d->max_members);
    }
    if (len != width) return fail(RIBN_AMD_OUTPUT_LENGTH, width, len, "host buffer holds %zu values, need %zu", len, width);
    DeviceGuard guard(d->ctx->device);
    hipError_t e = hipMemcpyAsync(host, base + member * width, width * sizeof(float), hipMemcpyDeviceToHost,
                                  d->ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->ctx->stream);
    return e == hipSuccess ? ok() : driver(e, "copy to host");
}

ribn_amd_status ribn_amd_qwen3_copy_hidden(ribn_amd_qwen3_decode* d, size_t member, float* host, size_t len) {
    return copy_member(d, d ? d->hidden : nullptr, d ? d->cfg.hidden : 0, member, host, len);
}

ribn_amd_status ribn_amd_qwen3_copy_logits(ribn_amd_qwen3_decode* d, size_t member, float* host, size_t len) {
    return copy_member(d, d ? d->logits : nullptr, d ? d->cfg.vocab : 0, member, host, len);
}

}  // extern "C"

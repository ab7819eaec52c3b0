// Serving dispatcher behind the C ABI (include/ribn_amd.h, "serving
// dispatcher"): the reference's CudaQwen35ServingDispatcher
// (crates/nvidia/src/serving.rs:81-1038) over one Qwen3 decoder, with the
// physical state registry (CudaStateRegistry, state.rs:411-525) and the
// submission ownership rules (submissions.rs, serving_submissions.hpp).
//
// One stream (the decoder context's) carries every row. A submission queues
// its rows without waiting on the device:
//   - an all-decode batch (or, with grouped decode, each compatible group of a
//     mixed batch) runs as one batched decode step; other rows run one by one
//     (prefill: with prompt prefill set, a prefix of at least
//     kPromptMinTokens on the prefill matmul; else leading whole chunks as
//     prefill-chunk steps; the rest as single steps, the sampling token
//     through the output head);
//   - each sampling row's greedy token is copied, stream-ordered, into its own
//     pinned host slot (hipHostMalloc) leased for the submission's lifetime;
//   - one event recorded after the rows covers every kernel and copy.
// poll_batch queries that event without blocking, reads the slots, recycles
// them and publishes the outcomes. Because every launch is stream-ordered,
// later rows may reuse the decoder's device buffers freely.
//
// State: a logical state id maps to one KV cache, created on the id's first
// row (only at prefix 0) and advanced by each completed step. Release while a
// pending submission still uses the state is deferred to its completion. A
// released cache is kept for reuse by a later state of the same capacity
// instead of freed (hipFree would wait for the whole device), and freed only
// when the KV byte budget needs the room.
//
// Failure: an enqueue error drains the stream and recycles the batch's slots
// before returning, so nothing of a failed submission stays queued. A failed
// drain or event query poisons the dispatcher: every later call reports
// RIBN_AMD_DEVICE_FAULTED, records of submissions are retired only after a
// successful drain and are otherwise quarantined (with release refused) until
// teardown.
#include "ribn_amd.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <limits>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "abi_internal.hpp"
#include "qwen3_internal.hpp"
#include "serving_submissions.hpp"

using namespace ribn_amd_abi;

namespace {

constexpr int32_t kNoSlot = -1;
// Shortest prefill prefix the prompt-prefill lane takes (shorter ones keep
// the chunk / serial path, where a matmul launch per projection buys little).
constexpr uint32_t kPromptMinTokens = 16;

// CudaHybridState with its KV family (Qwen3 has no recurrent layers).
struct PhysicalState {
    ribn_amd_kv_cache* cache = nullptr;
    uint32_t capacity = 0;
    uint32_t position = 0;  // token_position: the next position to write
    uint64_t bytes = 0;
};

// PendingSubmission (serving.rs:21-36).
struct Pending {
    hipEvent_t completion = nullptr;
    std::vector<int32_t> outputs;    // pinned slot per row, kNoSlot for rows without sampling
    std::vector<uint64_t> elapsed;   // per-row queueing wall time
    std::vector<uint64_t> state_keys;
};

using ribn_amd_dispatch::QueuedRows;

uint64_t now_ns() {
    return (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

std::string last_message() {
    ribn_amd_error e{};
    ribn_amd_last_error(&e);
    return std::string(e.message);
}

// decode_group's eligibility (serving.rs:526-537).
bool lane_eligible(const ribn_amd_serving_row& r) {
    return r.phase == RIBN_AMD_PHASE_DECODE && r.token_count == 1 && r.requests_sampling != 0 &&
           r.tokens != nullptr && r.logical_position != RIBN_AMD_NO_POSITION && r.kv_tokens != 0;
}

// batch_is_batchable (serving.rs:492-515): every row a single-token sampling
// decode with a token and a logical position, KV specs equal to the first's.
bool batch_is_batchable(const ribn_amd_serving_row* rows, size_t count, uint32_t lane_max) {
    if (count <= 1 || count > lane_max) return false;
    const uint32_t spec = rows[0].kv_tokens;
    for (size_t i = 0; i < count; ++i) {
        const ribn_amd_serving_row& r = rows[i];
        if (r.phase != RIBN_AMD_PHASE_DECODE || r.token_count != 1 || r.requests_sampling == 0 ||
            r.tokens == nullptr || r.logical_position == RIBN_AMD_NO_POSITION || r.kv_tokens != spec) {
            return false;
        }
    }
    return true;
}

std::vector<size_t> decode_group(const ribn_amd_serving_row* rows, size_t count, const std::vector<uint8_t>& scheduled,
                                 size_t first, size_t max_members) {
    std::vector<size_t> group;
    if (!lane_eligible(rows[first])) {
        group.push_back(first);
        return group;
    }
    const uint32_t spec = rows[first].kv_tokens;
    for (size_t i = first; i < count && group.size() < max_members; ++i) {
        if (!scheduled[i] && lane_eligible(rows[i]) && rows[i].kv_tokens == spec) group.push_back(i);
    }
    return group;
}

uint32_t chunked_prefix_len(uint32_t token_count, uint32_t members, bool sampling) {
    if (members == 0) return 0;
    const uint32_t chunkable = sampling ? (token_count == 0 ? 0 : token_count - 1) : token_count;
    return chunkable / members * members;
}

}  // namespace

struct ribn_amd_serving {
    ribn_amd_qwen3_decode* decode;
    ribn_amd_context* ctx;
    ribn_amd_qwen3_config cfg;
    uint32_t lane_max;       // widest batched decode lane
    uint32_t prefill_chunk;  // 0: serial prefill
    uint32_t prompt_chunk;   // 0: off; else prompt prefixes on the prefill matmul in chunks of this many tokens
    bool grouped;
    uint64_t kv_budget;      // 0: unbounded
    uint64_t kv_in_use;
    uint64_t kv_reusable;
    uint32_t* pinned;        // [slots] one-token output slots
    uint32_t slots;
    std::vector<int32_t> free_slots;
    ribn_amd_dispatch::Submissions<Pending> submissions;
    std::vector<uint64_t> deferred;  // released while a pending submission used them
    std::unordered_map<uint64_t, PhysicalState> states;
    std::unordered_map<uint32_t, std::vector<ribn_amd_kv_cache*>> spare;  // capacity -> caches for reuse
    std::vector<hipEvent_t> events;  // completion events for reuse
};

namespace {

hipStream_t stream_of(const ribn_amd_serving* s) { return s->ctx->stream; }

ribn_amd_status check_health(const ribn_amd_serving* s) {
    if (const char* fault = s->submissions.fault()) {
        return fail(RIBN_AMD_DEVICE_FAULTED, 0, 0, "the serving dispatcher is unusable after a device failure: %s",
                    fault);
    }
    return RIBN_AMD_OK;
}

void recycle_slot(ribn_amd_serving* s, int32_t slot) {
    if (slot != kNoSlot) s->free_slots.push_back(slot);
}

void retire(ribn_amd_serving* s, Pending& p) {
    for (int32_t slot : p.outputs) recycle_slot(s, slot);
    p.outputs.clear();
    if (p.completion) s->events.push_back(p.completion);
    p.completion = nullptr;
}

bool referenced(const ribn_amd_serving* s, uint64_t key) {
    for (const auto& kv : s->submissions.pending) {
        const std::vector<uint64_t>& keys = kv.second.state_keys;
        if (std::find(keys.begin(), keys.end(), key) != keys.end()) return true;
    }
    return false;
}

// release_key: the cache goes to the reuse pool.
void release_key(ribn_amd_serving* s, uint64_t key) {
    auto it = s->states.find(key);
    if (it == s->states.end()) return;
    s->spare[it->second.capacity].push_back(it->second.cache);
    s->kv_in_use -= it->second.bytes;
    s->kv_reusable += it->second.bytes;
    s->states.erase(it);
}

void drain_deferred(ribn_amd_serving* s) {
    std::vector<uint64_t> keep;
    for (uint64_t key : s->deferred) {
        if (referenced(s, key)) {
            keep.push_back(key);
        } else {
            release_key(s, key);
        }
    }
    s->deferred.swap(keep);
}

// fail_device (serving.rs:394-410): drain before retiring anything; with a
// failed drain, ownership stays quarantined until teardown.
ribn_amd_status fail_device(ribn_amd_serving* s, const std::string& error) {
    const hipError_t flush = hipStreamSynchronize(stream_of(s));
    std::vector<Pending> retired = s->submissions.fail(error, flush == hipSuccess);
    if (flush != hipSuccess) {
        return fail(RIBN_AMD_DEVICE_FAULTED, 0, 0, "%s; drain failed: %s; resources quarantined until teardown",
                    error.c_str(), hipGetErrorString(flush));
    }
    for (Pending& p : retired) retire(s, p);
    drain_deferred(s);
    return fail(RIBN_AMD_DEVICE_FAULTED, 0, 0, "%s", error.c_str());
}

// After an enqueue error: drain so no queued work outlives the call, recycle
// the slots, and keep the error (a failed drain turns it into a device fault).
ribn_amd_status abandon(ribn_amd_serving* s, ribn_amd_status st, const std::vector<int32_t>& slots) {
    ribn_amd_error saved{};
    ribn_amd_last_error(&saved);
    const std::string error(saved.message);
    const hipError_t flush = hipStreamSynchronize(stream_of(s));
    if (flush != hipSuccess) {
        return fail_device(s, error + "; flush after enqueue failure also failed: " + hipGetErrorString(flush));
    }
    for (int32_t slot : slots) recycle_slot(s, slot);
    return fail(st, saved.expected, saved.actual, "%s", error.c_str());
}

ribn_amd_status lease_slot(ribn_amd_serving* s, int32_t* slot) {
    if (s->free_slots.empty()) {
        return fail(RIBN_AMD_EXECUTION_FAILED, s->slots, s->slots + 1,
                    "pinned output slots exhausted; too many concurrent pending rows (%u slots)", s->slots);
    }
    *slot = s->free_slots.back();
    s->free_slots.pop_back();
    return RIBN_AMD_OK;
}

ribn_amd_status check_row(const ribn_amd_serving_row* r, size_t index) {
    if (r->state == 0) return fail(RIBN_AMD_INVALID_ARGUMENT, 1, 0, "row %zu has no state identity", index);
    return RIBN_AMD_OK;
}

// get_or_create (state.rs:462-486): fresh materialization only at prefix 0;
// the physical position must equal the logical one.
ribn_amd_status materialize(ribn_amd_serving* s, const ribn_amd_serving_row& row, PhysicalState** out) {
    const uint32_t expected = row.logical_position == RIBN_AMD_NO_POSITION ? 0 : row.logical_position;
    auto it = s->states.find(row.state);
    if (it == s->states.end()) {
        if (expected != 0) {
            return fail(RIBN_AMD_STATE_POSITION, 0, expected,
                        "state %llu has no physical materialization for logical prefix %u",
                        (unsigned long long)row.state, expected);
        }
        if (row.kv_tokens == 0) {
            return fail(RIBN_AMD_EXECUTION_FAILED, 1, 0, "the Qwen3 decoder needs full-attention KV state (request %llu)",
                        (unsigned long long)row.request);
        }
        const uint64_t bytes = ribn_amd_qwen3_kv_bytes(&s->cfg, row.kv_tokens);
        ribn_amd_kv_cache* cache = nullptr;
        auto pool = s->spare.find(row.kv_tokens);
        if (pool != s->spare.end() && !pool->second.empty()) {
            cache = pool->second.back();
            pool->second.pop_back();
            s->kv_reusable -= bytes;
        } else {
            if (s->kv_budget != 0 && s->kv_in_use + s->kv_reusable + bytes > s->kv_budget) {
                // free kept caches until the new one fits
                for (auto& kv : s->spare) {
                    while (!kv.second.empty() && s->kv_in_use + s->kv_reusable + bytes > s->kv_budget) {
                        ribn_amd_kv_cache_destroy(kv.second.back());
                        kv.second.pop_back();
                        s->kv_reusable -= ribn_amd_qwen3_kv_bytes(&s->cfg, kv.first);
                    }
                }
            }
            if (s->kv_budget != 0 && s->kv_in_use + bytes > s->kv_budget) {
                return fail(RIBN_AMD_BUDGET_EXCEEDED, s->kv_budget - s->kv_in_use, bytes,
                            "KV state of %u tokens needs %llu bytes; %llu of the %llu-byte budget are free",
                            row.kv_tokens, (unsigned long long)bytes,
                            (unsigned long long)(s->kv_budget - s->kv_in_use), (unsigned long long)s->kv_budget);
            }
            ribn_amd_status st = ribn_amd_kv_cache_create(s->ctx, &s->cfg, row.kv_tokens, &cache);
            if (st != RIBN_AMD_OK) return st;
        }
        PhysicalState phys;
        phys.cache = cache;
        phys.capacity = row.kv_tokens;
        phys.bytes = bytes;
        s->kv_in_use += bytes;
        it = s->states.emplace(row.state, phys).first;
    }
    if (it->second.position != expected) {
        return fail(RIBN_AMD_STATE_POSITION, expected, it->second.position,
                    "state %llu: logical position %u, physical position %u", (unsigned long long)row.state, expected,
                    it->second.position);
    }
    *out = &it->second;
    return RIBN_AMD_OK;
}

// advance_to (state.rs:715-724).
ribn_amd_status advance(PhysicalState* p, uint64_t next) {
    if (next > 0xffffffffull) return fail(RIBN_AMD_POSITION_OVERFLOW, 0xffffffffull, next, "position overflowed");
    if (next < p->position) {
        return fail(RIBN_AMD_STATE_POSITION, p->position, next, "position regression from %u to %llu", p->position,
                    (unsigned long long)next);
    }
    p->position = (uint32_t)next;
    return RIBN_AMD_OK;
}

// The step that produces a row's output token: eager (blocking, token read
// back), into a pinned slot (stream-ordered), or without the head when the
// row requests no output.
ribn_amd_status output_step(ribn_amd_serving* s, PhysicalState* p, uint32_t token, uint32_t position, bool eager,
                            int32_t slot, uint32_t* token_out, bool* has_token) {
    if (eager) {
        ribn_amd_status st = ribn_amd_qwen3_decode_step(s->decode, p->cache, token, position, token_out);
        if (st == RIBN_AMD_OK) *has_token = true;
        return st;
    }
    if (slot == kNoSlot) return ribn_amd_qwen3_prefill_step(s->decode, p->cache, token, position);
    ribn_amd_kv_cache* caches[1] = {p->cache};
    ribn_amd_status st = ribn_amd_decode::enqueue_decode(s->decode, caches, &token, &position, 1);
    if (st == RIBN_AMD_OK) st = ribn_amd_decode::copy_selected_async(s->decode, 0, s->pinned + slot);
    return st;
}

// run_row (serving.rs:176-279).
ribn_amd_status run_row(ribn_amd_serving* s, const ribn_amd_serving_row& row, bool eager, int32_t slot,
                        uint32_t* token_out, bool* has_token, uint64_t* elapsed) {
    *has_token = false;
    if (row.requests_sampling && row.temperature != 0.f) {
        return fail(RIBN_AMD_UNSUPPORTED, 0, 0, "non-greedy Qwen3 sampling is not supported (request %llu)",
                    (unsigned long long)row.request);
    }
    if (row.phase != RIBN_AMD_PHASE_PREFILL && row.phase != RIBN_AMD_PHASE_DECODE) {
        return fail(RIBN_AMD_UNSUPPORTED, 0, row.phase, "execution phase %u is not supported by Qwen3 serving",
                    row.phase);
    }
    PhysicalState* p = nullptr;
    ribn_amd_status st = materialize(s, row, &p);
    if (st != RIBN_AMD_OK) return st;
    if (row.state_position != p->position) {
        return fail(RIBN_AMD_STATE_POSITION, p->position, row.state_position,
                    "segment of request %llu starts at %u, its state holds %u tokens",
                    (unsigned long long)row.request, row.state_position, p->position);
    }
    const uint64_t started = now_ns();
    if (row.phase == RIBN_AMD_PHASE_PREFILL) {
        if (row.tokens == nullptr || row.token_count == 0) {
            return fail(RIBN_AMD_EXECUTION_FAILED, 1, 0, "Qwen3 prefill segment requires prompt token input");
        }
        const bool sampling = row.requests_sampling != 0;
        const uint32_t chunk = s->prefill_chunk;
        uint32_t chunked = chunked_prefix_len(row.token_count, chunk, sampling);
        const uint32_t prefix = sampling ? row.token_count - 1 : row.token_count;
        if (s->prompt_chunk != 0 && prefix >= kPromptMinTokens) {
            // the prompt-prefill lane: every token but the sampling one
            if ((uint64_t)row.state_position + prefix > 0x7fffffffull) {
                return fail(RIBN_AMD_POSITION_OVERFLOW, 0x7fffffffull, (uint64_t)row.state_position + prefix,
                            "prefill position overflowed");
            }
            st = ribn_amd_qwen3_prefill_prompt(s->decode, p->cache, row.tokens, prefix, row.state_position,
                                               s->prompt_chunk);
            if (st == RIBN_AMD_OK) st = advance(p, (uint64_t)row.state_position + prefix);
            if (st != RIBN_AMD_OK) return st;
            chunked = 0;
        }
        const uint32_t serial_from = s->prompt_chunk != 0 && prefix >= kPromptMinTokens ? prefix : chunked;
        for (uint32_t off = 0; off < chunked; off += chunk) {
            const uint64_t position = (uint64_t)row.state_position + off;
            if (position + chunk > 0x7fffffffull) {
                return fail(RIBN_AMD_POSITION_OVERFLOW, 0x7fffffffull, position + chunk, "prefill position overflowed");
            }
            st = ribn_amd_decode::enqueue_prefill_chunk(s->decode, p->cache, row.tokens + off, chunk,
                                                        (uint32_t)position);
            if (st == RIBN_AMD_OK) st = advance(p, position + chunk);
            if (st != RIBN_AMD_OK) return st;
        }
        for (uint32_t off = serial_from; off < row.token_count; ++off) {
            const uint64_t position = (uint64_t)row.state_position + off;
            if (position >= 0x7fffffffull) {
                return fail(RIBN_AMD_POSITION_OVERFLOW, 0x7fffffffull, position, "prefill position overflowed");
            }
            if (sampling && off + 1 == row.token_count) {
                st = output_step(s, p, row.tokens[off], (uint32_t)position, eager, slot, token_out, has_token);
            } else {
                st = ribn_amd_qwen3_prefill_step(s->decode, p->cache, row.tokens[off], (uint32_t)position);
            }
            if (st == RIBN_AMD_OK) st = advance(p, position + 1);
            if (st != RIBN_AMD_OK) return st;
        }
    } else {
        if (row.tokens == nullptr || row.token_count != 1) {
            return fail(RIBN_AMD_EXECUTION_FAILED, 1, row.token_count,
                        "Qwen3 decode segment requires one decode token");
        }
        st = output_step(s, p, row.tokens[0], row.state_position, eager, row.requests_sampling ? slot : kNoSlot,
                         token_out, has_token);
        if (st == RIBN_AMD_OK) st = advance(p, (uint64_t)row.state_position + 1);
        if (st != RIBN_AMD_OK) return st;
    }
    *elapsed = now_ns() - started;
    return RIBN_AMD_OK;
}

// enqueue_batched_decode (serving.rs:552-700): one batched decode step for the
// rows `idx`; per-member pinned copies; every state advanced by one.
ribn_amd_status enqueue_batched_decode(ribn_amd_serving* s, const ribn_amd_serving_row* rows,
                                       const std::vector<size_t>& idx, QueuedRows* out) {
    const size_t n = idx.size();
    const uint64_t started = now_ns();
    out->outputs.assign(n, kNoSlot);
    out->elapsed.assign(n, 0);
    out->state_keys.clear();
    auto run = [&]() -> ribn_amd_status {
        for (size_t i : idx) {
            const ribn_amd_serving_row& r = rows[i];
            if (r.requests_sampling && r.temperature != 0.f) {
                return fail(RIBN_AMD_UNSUPPORTED, 0, 0, "non-greedy Qwen3 sampling is not supported (request %llu)",
                            (unsigned long long)r.request);
            }
        }
        for (size_t m = 0; m < n; ++m) {
            if (rows[idx[m]].requests_sampling) {
                ribn_amd_status st = lease_slot(s, &out->outputs[m]);
                if (st != RIBN_AMD_OK) return st;
            }
        }
        if (n > s->lane_max) {
            return fail(RIBN_AMD_EXECUTION_FAILED, s->lane_max, n, "a batched decode of %zu rows was not prepared", n);
        }
        std::vector<PhysicalState*> members(n);
        std::vector<ribn_amd_kv_cache*> caches(n);
        std::vector<uint32_t> tokens(n), positions(n);
        for (size_t m = 0; m < n; ++m) {
            const ribn_amd_serving_row& r = rows[idx[m]];
            auto it = s->states.find(r.state);
            bool shared = false;
            for (size_t o = 0; o < m; ++o) shared = shared || rows[idx[o]].state == r.state;
            if (it == s->states.end() || shared) {
                return fail(RIBN_AMD_EXECUTION_FAILED, 0, 0,
                            "batched decode found no physical state for a decode row (request %llu)",
                            (unsigned long long)r.request);
            }
            if (r.tokens == nullptr) {
                return fail(RIBN_AMD_EXECUTION_FAILED, 1, 0, "Qwen3 decode segment requires one decode token");
            }
            if (it->second.position != r.state_position) {
                return fail(RIBN_AMD_STATE_POSITION, it->second.position, r.state_position,
                            "segment of request %llu starts at %u, its state holds %u tokens",
                            (unsigned long long)r.request, r.state_position, it->second.position);
            }
            members[m] = &it->second;
            caches[m] = it->second.cache;
            tokens[m] = r.tokens[0];
            positions[m] = r.state_position;
            out->state_keys.push_back(r.state);
        }
        ribn_amd_status st = ribn_amd_decode::enqueue_decode(s->decode, caches.data(), tokens.data(), positions.data(), n);
        if (st != RIBN_AMD_OK) return st;
        for (size_t m = 0; m < n; ++m) {
            if (out->outputs[m] == kNoSlot) continue;
            st = ribn_amd_decode::copy_selected_async(s->decode, m, s->pinned + out->outputs[m]);
            if (st != RIBN_AMD_OK) return st;
        }
        for (size_t m = 0; m < n; ++m) {
            st = advance(members[m], (uint64_t)positions[m] + 1);
            if (st != RIBN_AMD_OK) return st;
        }
        return RIBN_AMD_OK;
    };
    const ribn_amd_status st = run();
    if (st != RIBN_AMD_OK) {
        std::vector<int32_t> leased = out->outputs;
        out->outputs.assign(n, kNoSlot);
        return abandon(s, st, leased);
    }
    const uint64_t elapsed = now_ns() - started;
    std::fill(out->elapsed.begin(), out->elapsed.end(), elapsed);
    return RIBN_AMD_OK;
}

// enqueue_batch (serving.rs:702-808): rows in order, grouped decode lanes
// when enabled.
ribn_amd_status enqueue_batch(ribn_amd_serving* s, const ribn_amd_serving_row* rows, size_t count, QueuedRows* q) {
    q->outputs.assign(count, kNoSlot);
    q->elapsed.assign(count, 0);
    q->state_keys.clear();
    std::vector<uint8_t> scheduled(count, 0);
    auto run = [&]() -> ribn_amd_status {
        for (size_t first = 0; first < count; ++first) {
            if (scheduled[first]) continue;
            if (s->grouped) {
                std::vector<size_t> group = decode_group(rows, count, scheduled, first, s->lane_max);
                if (group.size() > 1) {
                    QueuedRows g;
                    ribn_amd_status st = enqueue_batched_decode(s, rows, group, &g);
                    if (st != RIBN_AMD_OK) return st;  // its own slots are already recycled
                    q->scatter(group, std::move(g));
                    for (size_t i : group) scheduled[i] = 1;
                    continue;
                }
            }
            const ribn_amd_serving_row& r = rows[first];
            int32_t slot = kNoSlot;
            if (r.requests_sampling) {
                ribn_amd_status st = lease_slot(s, &slot);
                if (st != RIBN_AMD_OK) return st;
            }
            q->outputs[first] = slot;  // retained before any fallible launch
            uint32_t token = 0;
            bool has_token = false;
            uint64_t elapsed = 0;
            ribn_amd_status st = run_row(s, r, false, slot, &token, &has_token, &elapsed);
            if (st != RIBN_AMD_OK) return st;
            q->elapsed[first] = elapsed;
            q->state_keys.push_back(r.state);
            scheduled[first] = 1;
        }
        return RIBN_AMD_OK;
    };
    const ribn_amd_status st = run();
    if (st != RIBN_AMD_OK) {
        if (s->submissions.fault() != nullptr) return st;  // a nested drain already failed
        std::vector<int32_t> leased = q->outputs;
        q->outputs.assign(count, kNoSlot);
        return abandon(s, st, leased);
    }
    return RIBN_AMD_OK;
}

ribn_amd_status check_rows(const ribn_amd_serving_row* rows, size_t count) {
    if (!rows) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null rows");
    if (count == 0) return fail(RIBN_AMD_INPUT_LENGTH, 1, 0, "a batch needs at least one row");
    for (size_t i = 0; i < count; ++i) {
        ribn_amd_status st = check_row(&rows[i], i);
        if (st != RIBN_AMD_OK) return st;
    }
    return RIBN_AMD_OK;
}

}  // namespace

extern "C" {

ribn_amd_status ribn_amd_serving_create(ribn_amd_qwen3_decode* decode, uint32_t max_pending_rows,
                                        uint64_t kv_budget_bytes, ribn_amd_serving** out) {
    if (!decode || !out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (max_pending_rows == 0) {
        return fail(RIBN_AMD_EXECUTION_FAILED, 1, 0, "the serving dispatcher requires at least one pinned output slot");
    }
    ribn_amd_context* ctx = ribn_amd_decode::context(decode);
    DeviceGuard guard(ctx->device);
    void* pinned = nullptr;
    hipError_t e = hipHostMalloc(&pinned, (size_t)max_pending_rows * sizeof(uint32_t), hipHostMallocDefault);
    if (e != hipSuccess) return driver(e, "hipHostMalloc output slots");
    auto* s = new (std::nothrow) ribn_amd_serving{};
    if (!s) {
        hipHostFree(pinned);
        return fail(RIBN_AMD_DRIVER, 0, 0, "host allocation failed");
    }
    s->decode = decode;
    s->ctx = ctx;
    s->cfg = ribn_amd_decode::config(decode);
    s->lane_max = std::min(max_pending_rows, ribn_amd_decode::max_members(decode));
    s->kv_budget = kv_budget_bytes;
    s->pinned = static_cast<uint32_t*>(pinned);
    s->slots = max_pending_rows;
    for (uint32_t i = max_pending_rows; i > 0; --i) s->free_slots.push_back((int32_t)(i - 1));
    context_retain(ctx);
    *out = s;
    return ok();
}

void ribn_amd_serving_destroy(ribn_amd_serving* s) {
    if (!s) return;
    DeviceGuard guard(s->ctx->device);
    hipStreamSynchronize(s->ctx->stream);
    for (Pending& p : s->submissions.take_all()) {
        if (p.completion) hipEventDestroy(p.completion);
    }
    for (hipEvent_t ev : s->events) hipEventDestroy(ev);
    for (auto& kv : s->states) ribn_amd_kv_cache_destroy(kv.second.cache);
    for (auto& kv : s->spare) {
        for (ribn_amd_kv_cache* c : kv.second) ribn_amd_kv_cache_destroy(c);
    }
    hipHostFree(s->pinned);
    ribn_amd_context* ctx = s->ctx;
    delete s;
    context_release(ctx);
}

ribn_amd_status ribn_amd_serving_set_prompt_prefill(ribn_amd_serving* s, uint32_t chunk_tokens) {
    if (!s) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null dispatcher");
    if (chunk_tokens == 0) {
        s->prompt_chunk = 0;
        return ok();
    }
    // the workspace now, so no submission allocates or waits for the device
    const ribn_amd_status st = ribn_amd_qwen3_reserve_prompt(s->decode, chunk_tokens);
    if (st != RIBN_AMD_OK) return st;
    s->prompt_chunk = chunk_tokens;
    return ok();
}

ribn_amd_status ribn_amd_serving_set_prefill_chunk(ribn_amd_serving* s, uint32_t members) {
    if (!s) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null dispatcher");
    if (members == 0) {
        s->prefill_chunk = 0;
        return ok();
    }
    if (members < 2) {
        return fail(RIBN_AMD_EXECUTION_FAILED, 2, members,
                    "prefill chunking requires at least two tokens per chunk; use 0 for serial prefill");
    }
    const uint32_t max = ribn_amd_decode::max_members(s->decode);
    if (members > max) {
        return fail(RIBN_AMD_EXECUTION_FAILED, max, members, "the decoder was built for %u members", max);
    }
    s->prefill_chunk = members;
    return ok();
}

ribn_amd_status ribn_amd_serving_set_grouped_decode(ribn_amd_serving* s, int32_t enabled) {
    if (!s) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null dispatcher");
    s->grouped = enabled != 0;
    return ok();
}

ribn_amd_status ribn_amd_serving_dispatch_batch(ribn_amd_serving* s, const ribn_amd_serving_row* rows, size_t count,
                                                ribn_amd_serving_outcome* outcomes) {
    if (!s || !outcomes) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    ribn_amd_status st = check_health(s);
    if (st == RIBN_AMD_OK) st = check_rows(rows, count);
    if (st != RIBN_AMD_OK) return st;
    DeviceGuard guard(s->ctx->device);
    for (size_t i = 0; i < count; ++i) {
        uint32_t token = 0;
        bool has_token = false;
        uint64_t elapsed = 0;
        st = run_row(s, rows[i], true, kNoSlot, &token, &has_token, &elapsed);
        // dispatch_segment_eager: no device work outlives the row
        const hipError_t sync = hipStreamSynchronize(stream_of(s));
        if (sync != hipSuccess) {
            const std::string error = st != RIBN_AMD_OK ? last_message() + "; " : std::string();
            return fail_device(s, error + "completion synchronization failed: " + hipGetErrorString(sync));
        }
        if (st != RIBN_AMD_OK) return st;
        outcomes[i].elapsed_nanos = elapsed;
        outcomes[i].has_token = has_token ? 1u : 0u;
        outcomes[i].token = token;
    }
    return ok();
}

ribn_amd_status ribn_amd_serving_submit_batch(ribn_amd_serving* s, uint64_t submission,
                                              const ribn_amd_serving_row* rows, size_t count) {
    if (!s) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null dispatcher");
    ribn_amd_status st = check_health(s);
    if (st == RIBN_AMD_OK) st = check_rows(rows, count);
    if (st != RIBN_AMD_OK) return st;
    if (submission == 0) return fail(RIBN_AMD_INVALID_ARGUMENT, 1, 0, "submission ids are nonzero");
    if (s->submissions.pending.count(submission)) {
        return fail(RIBN_AMD_EXECUTION_FAILED, 0, submission, "duplicate asynchronous submission %llu",
                    (unsigned long long)submission);
    }
    DeviceGuard guard(s->ctx->device);
    QueuedRows q;
    if (!s->grouped && batch_is_batchable(rows, count, s->lane_max)) {
        std::vector<size_t> all(count);
        for (size_t i = 0; i < count; ++i) all[i] = i;
        st = enqueue_batched_decode(s, rows, all, &q);
    } else {
        st = enqueue_batch(s, rows, count, &q);
    }
    if (st != RIBN_AMD_OK) return st;
    // one completion event after every kernel and pinned copy of the batch
    hipEvent_t ev = nullptr;
    hipError_t e = hipSuccess;
    if (!s->events.empty()) {
        ev = s->events.back();
        s->events.pop_back();
    } else {
        e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    }
    if (e == hipSuccess) e = hipEventRecord(ev, stream_of(s));
    if (e != hipSuccess) {
        if (ev) s->events.push_back(ev);
        const std::string error = std::string("event recording failed: ") + hipGetErrorString(e);
        const hipError_t flush = hipStreamSynchronize(stream_of(s));
        if (flush != hipSuccess) return fail_device(s, error + "; flush also failed: " + hipGetErrorString(flush));
        for (int32_t slot : q.outputs) recycle_slot(s, slot);
        return fail(RIBN_AMD_EXECUTION_FAILED, 0, 0, "%s", error.c_str());
    }
    Pending p;
    p.completion = ev;
    p.outputs = std::move(q.outputs);
    p.elapsed = std::move(q.elapsed);
    p.state_keys = std::move(q.state_keys);
    s->submissions.pending.emplace(submission, std::move(p));
    return ok();
}

ribn_amd_status ribn_amd_serving_poll_batch(ribn_amd_serving* s, uint64_t submission,
                                            ribn_amd_serving_outcome* outcomes, size_t count, int32_t* ready) {
    if (!s || !ready) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    *ready = 0;
    ribn_amd_status st = check_health(s);
    if (st != RIBN_AMD_OK) return st;
    auto it = s->submissions.pending.find(submission);
    if (it == s->submissions.pending.end()) {
        return fail(RIBN_AMD_UNKNOWN_SUBMISSION, 0, submission, "serving submission %llu is unknown",
                    (unsigned long long)submission);
    }
    if (count != it->second.outputs.size() || (!outcomes && count != 0)) {
        return fail(RIBN_AMD_OUTPUT_LENGTH, it->second.outputs.size(), count,
                    "submission %llu has %zu rows, the outcome buffer %zu", (unsigned long long)submission,
                    it->second.outputs.size(), count);
    }
    DeviceGuard guard(s->ctx->device);
    // hipEventQuery tells "not ready" apart from a device fault
    const hipError_t q = hipEventQuery(it->second.completion);
    if (q == hipErrorNotReady) return ok();
    if (q != hipSuccess) return fail_device(s, std::string("completion query failed: ") + hipGetErrorString(q));
    Pending p = std::move(it->second);
    s->submissions.pending.erase(it);
    const volatile uint32_t* slots = s->pinned;
    for (size_t i = 0; i < count; ++i) {
        outcomes[i].elapsed_nanos = p.elapsed[i];
        outcomes[i].has_token = p.outputs[i] != kNoSlot ? 1u : 0u;
        outcomes[i].token = p.outputs[i] != kNoSlot ? slots[p.outputs[i]] : 0u;
    }
    retire(s, p);
    drain_deferred(s);
    *ready = 1;
    return ok();
}

ribn_amd_status ribn_amd_serving_release_state(ribn_amd_serving* s, uint64_t state) {
    if (!s) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null dispatcher");
    if (!s->submissions.release_is_safe()) {
        return fail(RIBN_AMD_DEVICE_FAULTED, 0, 0, "resource release awaits teardown of the faulted dispatcher");
    }
    if (referenced(s, state)) {
        if (std::find(s->deferred.begin(), s->deferred.end(), state) == s->deferred.end()) {
            s->deferred.push_back(state);
        }
    } else {
        release_key(s, state);
    }
    return ok();
}

size_t ribn_amd_serving_pending(const ribn_amd_serving* s) { return s ? s->submissions.pending.size() : 0; }

size_t ribn_amd_serving_state_count(const ribn_amd_serving* s) { return s ? s->states.size() : 0; }

uint64_t ribn_amd_serving_state_bytes(const ribn_amd_serving* s, uint64_t* reusable_bytes) {
    if (reusable_bytes) *reusable_bytes = s ? s->kv_reusable : 0;
    return s ? s->kv_in_use : 0;
}

ribn_amd_status ribn_amd_serving_state_position(const ribn_amd_serving* s, uint64_t state, uint32_t* position) {
    if (!s || !position) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    auto it = s->states.find(state);
    if (it == s->states.end()) {
        return fail(RIBN_AMD_STATE_POSITION, 0, state, "state %llu is not materialized", (unsigned long long)state);
    }
    *position = it->second.position;
    return ok();
}

uint32_t ribn_amd_serving_chunked_prefix_len(uint32_t token_count, uint32_t members, int32_t requests_sampling) {
    return chunked_prefix_len(token_count, members, requests_sampling != 0);
}

size_t ribn_amd_serving_decode_group(const ribn_amd_serving_row* rows, size_t count, const uint8_t* scheduled,
                                     size_t first, size_t max_members, size_t* out) {
    if (!rows || !scheduled || !out || first >= count) return 0;
    std::vector<uint8_t> sched(scheduled, scheduled + count);
    std::vector<size_t> g = decode_group(rows, count, sched, first, max_members);
    std::copy(g.begin(), g.end(), out);
    return g.size();
}

ribn_amd_status ribn_amd_plan_memory(ribn_amd_context* ctx, uint64_t per_sequence_state_bytes,
                                     uint64_t max_sequences, uint64_t continuation_override,
                                     uint64_t headroom_bytes, uint64_t requested_weight_budget,
                                     ribn_amd_memory_plan* out) {
    if (!ctx || !out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    uint64_t reserved = continuation_override;
    if (reserved == 0) {
        if (max_sequences != 0 && per_sequence_state_bytes > std::numeric_limits<uint64_t>::max() / max_sequences) {
            return fail(RIBN_AMD_SHAPE_OVERFLOW, 0, 0, "state reservation overflow");
        }
        reserved = per_sequence_state_bytes * max_sequences;
    }
    if (reserved == 0) return fail(RIBN_AMD_EXECUTION_FAILED, 1, 0, "continuation capacity must be nonzero");
    DeviceGuard guard(ctx->device);
    size_t free_bytes = 0, total_bytes = 0;
    hipError_t e = hipMemGetInfo(&free_bytes, &total_bytes);
    if (e != hipSuccess) return driver(e, "hipMemGetInfo");
    const uint64_t free64 = free_bytes;
    if (reserved > free64 || headroom_bytes > free64 - reserved) {
        return fail(RIBN_AMD_BUDGET_EXCEEDED, free64, reserved + headroom_bytes,
                    "state requires %llu bytes plus %llu bytes headroom, but only %llu bytes are free",
                    (unsigned long long)reserved, (unsigned long long)headroom_bytes, (unsigned long long)free64);
    }
    const uint64_t available = free64 - reserved - headroom_bytes;
    const uint64_t weight = requested_weight_budget ? requested_weight_budget : available;
    if (weight == 0 || weight > available) {
        return fail(RIBN_AMD_BUDGET_EXCEEDED, available, weight,
                    "weight budget %llu exceeds the available %llu bytes after state/headroom reservations",
                    (unsigned long long)weight, (unsigned long long)available);
    }
    out->free_before_preparation_bytes = free64;
    out->weight_budget_bytes = weight;
    out->reserved_sequence_bytes = reserved;
    return ok();
}

uint64_t ribn_amd_qwen3_kv_bytes(const ribn_amd_qwen3_config* c, uint32_t tokens) {
    if (!c) return 0;
    return (uint64_t)c->layers * c->kv_heads * c->head_dim * tokens * 2u * 2u;
}

}  // extern "C"

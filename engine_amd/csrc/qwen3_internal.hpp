// Stream-ordered decoder calls for the serving dispatcher (serving.cpp):
// each validates like its C-ABI counterpart, enqueues on the context stream
// and returns without waiting, so a dispatcher can queue several rows and
// observe them through one recorded event.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "ribn_amd.h"

namespace ribn_amd_decode {

// CudaQwen35BatchDecode::decode_step_batch_enqueue (decode.rs:1884-1891):
// one step with the output head; the selections stay on the device until
// copy_selected_async.
ribn_amd_status enqueue_decode(ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* const* caches, const uint32_t* tokens,
                               const uint32_t* positions, size_t members);
// CudaQwen35BatchDecode::prefill_chunk (decode.rs:1953-1977): tokens at
// position, position + 1, ... of one sequence, without the output head.
ribn_amd_status enqueue_prefill_chunk(ribn_amd_qwen3_decode* d, ribn_amd_kv_cache* cache, const uint32_t* tokens,
                                      size_t count, uint32_t position);
// copy_selected_into_pinned (decode.rs:1900-1915): the last step's selection
// of `member` into pinned host memory, stream-ordered.
ribn_amd_status copy_selected_async(ribn_amd_qwen3_decode* d, size_t member, uint32_t* pinned);

ribn_amd_context* context(const ribn_amd_qwen3_decode* d);
uint32_t max_members(const ribn_amd_qwen3_decode* d);
const ribn_amd_qwen3_config& config(const ribn_amd_qwen3_decode* d);

}  // namespace ribn_amd_decode

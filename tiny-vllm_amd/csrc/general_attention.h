// Paged attention for any head dim up to 256 (decode rows and prefill
// chunks), the path behind tvllm_paged_decode and tvllm_paged_prefill for
// the shapes their MFMA kernels do not take (head_dim != 128, GQA groups
// above 16, unaligned rows).
#pragma once

#include "common.h"

namespace tvllm {

struct GeneralAttention {
    const void* q;  // T elements
    int64_t qts, qhs;
    const void* k;  // cache rows: T elements, or FP8 E4M3 bytes
    const void* v;
    int64_t css, chs;
    void* out;
    int64_t ots, ohs;
    // Decode: item r is the single query token rows[r] and attends its
    // lengths[r] cached tokens. Prefill (rows == nullptr): item r's query
    // tokens are [q_offsets[r], q_offsets[r + 1]), query i attending tokens
    // t <= lengths[r] - query_len + i (lower-right causal).
    const int64_t* rows;
    const int64_t* q_offsets;
    const int64_t* blocks;
    const int64_t* offsets;  // item r's table starts at blocks[offsets[r]]
    const int64_t* lengths;
    int64_t num_items, max_query_len;
    int heads, kv_heads, head_dim, block_size;
    int dtype, cache_dtype;
    float scale;             // softmax scale
    float k_scale, v_scale;  // FP8 cache dequantisation scales (1 otherwise)
};

// Validated by the caller (geometry, dtypes, cache layout); enqueues one
// launch on `stream`.
int launch_general_attention(const GeneralAttention& g, hipStream_t stream);

}  // namespace tvllm

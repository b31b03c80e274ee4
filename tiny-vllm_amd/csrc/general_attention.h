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
    // Decode only: the bound on lengths[] that sizes the launch, and the
    // workspace that holds the partials of contexts split over several
    // workgroups (general_decode_workspace bytes; may be null when that is 0).
    int64_t max_context;
    void* workspace;
    int64_t workspace_bytes;
    // Filled in by the launcher: the split plan and the partials' arrays.
    int64_t splits, split_keys;
    float* part_o;   // [num_items][heads][splits][head_dim]
    float* part_ml;  // [num_items][heads][splits][2]: (max, sum) in base 2
};

// Grid-level key splits of a decode launch of the general kernel (1: none):
// enough workgroups to fill the chip when there are few (row, KV head) units,
// each split keeping at least two rounds of chunks for each of its waves.
struct GeneralSplits {
    int64_t splits;  // workgroups per (row, KV head, head chunk)
    int64_t keys;    // keys per split (a multiple of the kernel's chunk)
};
GeneralSplits general_decode_splits(int64_t rows, int64_t heads, int64_t kv_heads,
                                    int64_t head_dim, int64_t max_context);
// Workspace bytes a decode launch of this geometry needs (0 when unsplit).
int64_t general_decode_workspace(int64_t rows, int64_t heads, int64_t kv_heads,
                                 int64_t head_dim, int64_t max_context);

// Validated by the caller (geometry, dtypes, cache layout); enqueues one
// launch on `stream` (two for a split decode: the split workgroups, then
// the merge of their partials).
int launch_general_attention(const GeneralAttention& g, hipStream_t stream);

}  // namespace tvllm

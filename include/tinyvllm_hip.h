/*
 * tinyvllm_hip.h -- C ABI of the gfx950 (MI355X) kernels behind tiny-vLLM's
 * decode token loop.
 *
 * Every entry point takes plain device pointers, element counts, element
 * strides and the hipStream_t to launch on (pass torch's current stream so
 * the launch is ordered with, and capturable into, the caller's graph).
 * None of them allocates, synchronises or reads device memory on the host.
 *
 * Return value: 0 on success; a negative TVLLM_E* code otherwise, with a
 * human-readable message available from tvllm_last_error() (thread-local).
 * Argument checks mirror the TORCH_CHECK contracts of the reference's host
 * functions; value validity (slot ranges, block ids) is the caller's job, as
 * in the reference, where it is validated on the CPU before launch.
 *
 * Element types: TVLLM_BF16 / TVLLM_F16 for every op; TVLLM_F32 is also
 * accepted by the row-wise pointwise ops (rms_norm, silu_and_mul), like the
 * reference's pointwise.cu dispatch.
 *
 * Paged KV cache (every entry point with key/value caches): num_slots =
 * num_blocks * block_size slots; the row of (slot, KV head) holds head_dim
 * contiguous elements at slot * cache_slot_stride + head * cache_head_stride
 * elements from the cache pointer. Two nestings are accepted, so rows never
 * overlap: token-major (the reference's contiguous [num_slots, kv_heads,
 * head_dim]: slot stride kv_heads * head_dim, head stride head_dim) and
 * head-major ([kv_heads, num_slots, head_dim]: slot stride head_dim, head
 * stride num_slots * head_dim, a page of one head contiguous), or either
 * with padding. The fast kernels need both strides in whole 16-byte units.
 */
#ifndef TINYVLLM_HIP_H
#define TINYVLLM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* tvllm_stream_t; /* == hipStream_t */

enum tvllm_dtype {
    TVLLM_BF16 = 0,
    TVLLM_F16 = 1,
    TVLLM_F32 = 2,
    /* KV-cache storage only: OCP FP8 E4M3 (max 448) with a per-cache scale,
     * stored = fp8(clamp(x * (1 / scale), -448, 448)), read as stored * scale. */
    TVLLM_FP8_E4M3 = 3,
};

enum tvllm_status {
    TVLLM_OK = 0,
    TVLLM_EINVAL = -1,   /* shape / stride / dtype contract violated  */
    TVLLM_ELAUNCH = -2,  /* hipLaunchKernel (or hipGetLastError) failed */
};

/* Message for the last failing call on this thread ("" if none). */
const char* tvllm_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int tvllm_abi_version(void);

/* Hex SHA-256 prefix of the sources (csrc/*.hip, csrc/*.h, include/*.h) the
 * library was built from; the Python loader refuses a library whose digest
 * differs from the sources beside it. No counterpart in the reference (its
 * JIT build recompiles on source change, _extension.py:11-42). */
const char* tvllm_source_hash(void);

/* Scatter K/V rows into the paged cache: cache[slot[t]] = key[t] (bit copy;
 * cache_dtype == dtype, k_scale = v_scale = 1), or for cache_dtype
 * TVLLM_FP8_E4M3 the E4M3 byte of clamp(x * (1 / scale), -448, 448) per
 * element (nearest-even). slot == -1 skips the row (graph padding).
 * key/value: [tokens, kv_heads, head_dim] with the given element strides
 * (last stride must be 1); caches: the paged layout above.
 * Replaces: torch.ops.tinyvllm_cuda.store_kv
 *           (reference tinyvllm/kernels/kv_store.cu:101-232, wrapper
 *            tinyvllm/kernels/kv_store.py:10-30). */
int tvllm_store_kv(const void* key, const void* value,
                   int64_t key_token_stride, int64_t key_head_stride,
                   int64_t value_token_stride, int64_t value_head_stride,
                   void* key_cache, void* value_cache,
                   const int64_t* slots, int64_t num_tokens,
                   int64_t num_kv_heads, int64_t head_dim, int64_t num_slots,
                   int64_t cache_slot_stride, int64_t cache_head_stride,
                   int dtype, int cache_dtype, float k_scale, float v_scale,
                   tvllm_stream_t stream);

/* Apply a step's block-table updates to a device-resident table:
 * updates = [n, index_0, id_0, index_1, id_1, ...] (int64, on the device);
 * table[index_i] = id_i for i < min(n, capacity); indices outside
 * [0, table_size) are skipped. n is read on the device (graph-capturable).
 * No counterpart in the reference (it re-uploads every block table each
 * step, tinyvllm/runtime/inputs.py:70-117); the decode step keeps one table
 * row per request slot and uploads only the entries that changed. */
int tvllm_apply_table_updates(int64_t* table, int64_t table_size,
                              const int64_t* updates, int64_t capacity,
                              tvllm_stream_t stream);

/* Bytes of device workspace tvllm_paged_decode needs for this geometry
 * (split-K partial results). 0 means no workspace is needed.
 * max_context_len bounds the context of any row (the engine's
 * max_model_len); it only sizes the split count, never the grid's validity. */
int64_t tvllm_paged_decode_workspace_size(int64_t num_rows, int64_t num_heads,
                                          int64_t num_kv_heads,
                                          int64_t head_dim,
                                          int64_t max_context_len,
                                          int64_t block_size);

/* The split-K decomposition tvllm_paged_decode uses for this geometry,
 * packed as (waves per KV head << 16) | (workgroups per row << 8) | (KV heads
 * per workgroup) for the MFMA kernel, (1 << 32) | (workgroups per row, KV
 * head and head chunk) for the general kernel (head_dim != 128 or groups
 * above 16), 0 for invalid geometry. It depends on max_context_len, so a
 * caller that bakes launches (graph capture) can tell when a tighter context
 * bound would change it. No reference counterpart (the reference kernel has
 * no split-K). */
int64_t tvllm_paged_decode_split_plan(int64_t num_rows, int64_t num_heads,
                                      int64_t num_kv_heads, int64_t head_dim,
                                      int64_t max_context_len, int64_t block_size);

/* Single-query paged attention for decode rows.
 * For r < num_rows, h < num_heads:
 *   out[rows[r], h] = softmax_t(scale * q[rows[r], h] . k_t) @ v_t,
 *   t < lengths[r], token t at slot blocks[offsets[r] + t / bs] * bs + t % bs
 *   of KV head h / (num_heads / num_kv_heads). lengths[r] == 0 -> zeros.
 * q, out: [*, num_heads, head_dim] with element strides (last == 1).
 * k_cache, v_cache: the paged layout above.
 * rows, offsets (num_rows + 1; only offsets[r], the start of row r's table, is
 * read - a CSR or pitched per-slot rows), lengths, blocks: int64 device vectors.
 * workspace: >= tvllm_paged_decode_workspace_size(...) bytes (may be NULL
 * when that size is 0). head_dim 128 with group <= 16 and 16-byte aligned
 * rows runs the MFMA kernel; any other head_dim <= 256, group or alignment
 * runs the general kernel (a workgroup of four waves per row, KV head and
 * group of up to 16 query heads, sharing each K/V load; when such units are
 * few, each row's keys split over several workgroups and a second launch
 * merges their partials; fp32 arithmetic, no MFMA).
 * cache_dtype: dtype (caches hold q's element type; k_scale = v_scale = 1)
 * or TVLLM_FP8_E4M3 (caches hold E4M3 bytes in the paged layout;
 * K = stored * k_scale, V = stored * v_scale).
 * Replaces: torch.ops.tinyvllm_cuda.paged_decode
 *           (reference tinyvllm/kernels/paged_decode.cu:469-669, wrapper
 *            tinyvllm/kernels/paged_decode.py:10-32). */
int tvllm_paged_decode(const void* q, int64_t q_token_stride,
                       int64_t q_head_stride, const void* k_cache,
                       const void* v_cache, void* out,
                       int64_t out_token_stride, int64_t out_head_stride,
                       const int64_t* rows, const int64_t* blocks,
                       const int64_t* offsets, const int64_t* lengths,
                       int64_t num_rows, int64_t num_heads,
                       int64_t num_kv_heads, int64_t head_dim,
                       int64_t num_slots, int64_t cache_slot_stride,
                       int64_t cache_head_stride, int64_t block_size,
                       int64_t max_context_len, float scale,
                       void* workspace, int64_t workspace_bytes,
                       int dtype, int cache_dtype, float k_scale, float v_scale,
                       tvllm_stream_t stream);

/* tvllm_paged_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The
 * split-K partials go to a static 8 MiB device array per GPU (held until
 * the process ends); a geometry whose tvllm_paged_decode_workspace_size
 * exceeds 8 MiB is rejected with TVLLM_EINVAL (the MFMA kernel's split plan
 * needs at most ~6 MB; the general kernel's can need more at head_dim 256
 * with groups of 16). Allocates nothing. Calls that
 * overlap on one GPU (different streams) share that array and race; calls
 * ordered on one stream are safe. The first call on a device looks up the
 * array's address (hipGetSymbolAddress): make it outside graph capture. */
int tvllm_paged_decode_noalloc(const void* q, int64_t q_token_stride,
                               int64_t q_head_stride, const void* k_cache,
                               const void* v_cache, void* out,
                               int64_t out_token_stride, int64_t out_head_stride,
                               const int64_t* rows, const int64_t* blocks,
                               const int64_t* offsets, const int64_t* lengths,
                               int64_t num_rows, int64_t num_heads,
                               int64_t num_kv_heads, int64_t head_dim,
                               int64_t num_slots, int64_t cache_slot_stride,
                               int64_t cache_head_stride, int64_t block_size,
                               int64_t max_context_len, float scale,
                               int dtype, int cache_dtype, float k_scale,
                               float v_scale, tvllm_stream_t stream);

/* tvllm_qk_norm_rope's fused KV write followed by tvllm_paged_decode, in
 * one kernel, for a step whose rows are all decode rows: q, k, v are the raw
 * projections (element strides, last 1); each workgroup normalises and
 * rotates its query heads in registers, and the wave whose page range holds
 * a row's newest token (position lengths[r] - 1) writes that token's rotated
 * K row and its V row to slot slots[rows[r]] (-1 skips) before reading it.
 * The K rows written are bit-identical to tvllm_qk_norm_rope's (with the
 * same cache_dtype and scales). cos, sin: contiguous [tokens, 64]; q_weight,
 * k_weight: [128]. head_dim must be 128. cache_dtype / k_scale / v_scale as
 * for tvllm_paged_decode.
 * Replaces: the decode-step sequence qk_norm_rope + store_kv + paged_decode
 *           (reference tinyvllm/models/qwen3.py:284-293,
 *            runtime/attention.py:219-285); no single reference counterpart. */
int tvllm_paged_decode_qk_norm_rope(
    const void* q, int64_t q_token_stride, int64_t q_head_stride, const void* k,
    int64_t k_token_stride, int64_t k_head_stride, const void* v, int64_t v_token_stride,
    int64_t v_head_stride, const void* q_weight, const void* k_weight, const void* cos,
    const void* sin, float q_eps, float k_eps, const int64_t* slots, void* k_cache,
    void* v_cache, void* out, int64_t out_token_stride, int64_t out_head_stride,
    const int64_t* rows, const int64_t* blocks, const int64_t* offsets,
    const int64_t* lengths, int64_t num_rows, int64_t num_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t num_slots, int64_t cache_slot_stride,
    int64_t cache_head_stride, int64_t block_size, int64_t max_context_len,
    float scale, void* workspace, int64_t workspace_bytes, int dtype, int cache_dtype,
    float k_scale, float v_scale, tvllm_stream_t stream);

/* tvllm_paged_decode_qk_norm_rope with the raw q/k/v given as four fp32
 * split-K partials of the qkv projection instead of its rounded output:
 * parts[s * slice_stride + row * row_stride + col], s < 4, a row holding
 * the num_heads query heads, then the num_kv_heads key heads, then the
 * value heads, 128 columns each (the [4, tokens, width] fp32 result of a
 * batched torch.bmm over four slices of the reduction axis). Each raw
 * element is ((p0 + p1) + p2) + p3 in fp32, rounded once to dtype - a
 * single fp32-accumulating GEMM's rounding, up to the order of the sum -
 * and then normalised, rotated, written and attended exactly as
 * tvllm_paged_decode_qk_norm_rope does. parts must be 16-byte aligned, both
 * strides whole multiples of 4 elements.
 * No reference counterpart: it lets a decode step's qkv projection run as
 * a split-K batched GEMM (which fills the GPU at decode batch sizes) with
 * no extra launch to sum the slices. */
int tvllm_paged_decode_qk_norm_rope_partials(
    const float* parts, int64_t slice_stride, int64_t row_stride, const void* q_weight,
    const void* k_weight, const void* cos, const void* sin, float q_eps, float k_eps,
    const int64_t* slots, void* k_cache, void* v_cache, void* out, int64_t out_token_stride,
    int64_t out_head_stride, const int64_t* rows, const int64_t* blocks,
    const int64_t* offsets, const int64_t* lengths, int64_t num_rows, int64_t num_heads,
    int64_t num_kv_heads, int64_t head_dim, int64_t num_slots, int64_t cache_slot_stride,
    int64_t cache_head_stride, int64_t block_size, int64_t max_context_len, float scale,
    void* workspace, int64_t workspace_bytes, int dtype, int cache_dtype, float k_scale,
    float v_scale, tvllm_stream_t stream);

/* RMSNorm over rows of width `width`, optionally after a residual add:
 *   x = residual ? round(x + residual) : x
 *   out = round(round(x * rsqrt(mean(x^2) + eps)) * weight)
 *   residual_out = x            (only when residual != NULL)
 * Input rows: count = tokens * heads; row (t, h) starts at
 * t * token_stride + h * head_stride (heads == 1, head_stride == 0 for 2-D).
 * residual rows: t * residual_stride. out / residual_out: dense [count, width].
 * Replaces: torch.ops.tinyvllm_cuda.rms_norm / add_rms_norm
 *           (reference tinyvllm/kernels/pointwise.cu:549-616). */
int tvllm_rms_norm(const void* input, int64_t tokens, int64_t heads,
                   int64_t width, int64_t token_stride, int64_t head_stride,
                   const void* weight, const void* residual,
                   int64_t residual_stride, void* out, void* residual_out,
                   float eps, int dtype, tvllm_stream_t stream);

/* add+RMSNorm whose input x is the sum of fp32 split-K partial products:
 * x[t, c] = round(sum_p partials[p * partial_stride + t * width + c]), then
 * residual_out = round(x + residual) and out = RMSNorm(residual_out) with
 * the rounding points of tvllm_rms_norm. width % 8 == 0, width <= 8192,
 * 1..64 partials; residual rows with stride residual_stride.
 * Replaces: the rounding of the down projection's output (F.linear, reference
 *           models/qwen3.py MLP) fused with torch.ops.tinyvllm_cuda.add_rms_norm
 *           (reference tinyvllm/kernels/pointwise.cu:549-616); no reference
 *           counterpart for the split-K decomposition itself. */
int tvllm_add_rms_norm_partials(const float* partials, int64_t num_partials,
                                int64_t partial_stride, int64_t tokens,
                                int64_t width, const void* weight,
                                const void* residual, int64_t residual_stride,
                                void* out, void* residual_out, float eps,
                                int dtype, tvllm_stream_t stream);

/* out[r, c] = round(round(silu(x[r, c])) * x[r, c + width / 2]) for rows
 * laid out like tvllm_rms_norm's input; out is dense [count, width / 2].
 * Replaces: torch.ops.tinyvllm_cuda.silu_and_mul
 *           (reference tinyvllm/kernels/pointwise.cu:619-680). */
int tvllm_silu_and_mul(const void* input, int64_t tokens, int64_t heads,
                       int64_t width, int64_t token_stride,
                       int64_t head_stride, void* out, int dtype,
                       tvllm_stream_t stream);

/* Per-head Q/K RMSNorm followed by half-split RoPE, with every rounding
 * point of the reference expression:
 *   n = round(round(x * inv_rms) * w);
 *   o1 = round(round(n1 * cos) - round(n2 * sin));
 *   o2 = round(round(n2 * cos) + round(n1 * sin)).
 * q: [tokens, num_heads, head_dim], k: [tokens, num_kv_heads, head_dim],
 * element strides, last stride 1. cos/sin: contiguous [tokens, head_dim/2].
 * q_out, k_out: dense [tokens, heads, head_dim].
 * Fused KV write (not in the reference, which runs store_kv afterwards):
 * when key_cache != NULL, the rotated K row and the V row
 * (v: [tokens, num_kv_heads, head_dim] with the given strides) are also
 * written to key_cache/value_cache at slot slots[t] (the paged layout
 * above; slot -1 skips); k_out may then be NULL. cache_dtype / k_scale / v_scale as for tvllm_store_kv (the FP8
 * cache stores the E4M3 byte of the rounded rotated K element times 1/k_scale).
 * Replaces: torch.ops.tinyvllm_cuda.qk_norm_rope
 *           (reference tinyvllm/kernels/pointwise.cu:453-546) and, when
 *           fused, the following store_kv (runtime/attention.py:219-233). */
int tvllm_qk_norm_rope(const void* q, int64_t q_token_stride,
                       int64_t q_head_stride, const void* k,
                       int64_t k_token_stride, int64_t k_head_stride,
                       const void* q_weight, const void* k_weight,
                       const void* cos, const void* sin, int64_t tokens,
                       int64_t num_heads, int64_t num_kv_heads,
                       int64_t head_dim, float q_eps, float k_eps,
                       void* q_out, void* k_out,
                       const void* v, int64_t v_token_stride,
                       int64_t v_head_stride, void* key_cache,
                       void* value_cache, const int64_t* slots,
                       int64_t num_slots, int64_t cache_slot_stride,
                       int64_t cache_head_stride, int dtype, int cache_dtype,
                       float k_scale, float v_scale, tvllm_stream_t stream);

/* Greedy sampling: out[r] = first index of the maximum of logits[r, :vocab]
 * (row stride row_stride elements). NaN compares greater than any number,
 * as torch.argmax does.
 * Replaces: logits.argmax(dim=-1) in TorchSampler.sample
 *           (reference tinyvllm/sampling.py:42-43). */
int tvllm_argmax(const void* logits, int64_t rows, int64_t vocab,
                 int64_t row_stride, int64_t* out, int dtype,
                 tvllm_stream_t stream);

/* Temperature / top-k / top-p sampling by the exponential race:
 *   s = (logit - max) / temperature;  keep the top_k largest (0 = all);
 *   keep the smallest prefix of the descending order whose probability
 *   mass exceeds top_p (ties broken by lower index);
 *   out[r] = argmax_{kept i} p_i / E_i,  E_i ~ Exp(1) from a counter-based
 *   Philox4x32-10 stream keyed by (seeds[r], counters[r], i).
 * temperature > 0 samples; temperature 0 rows take the argmax.
 * workspace (optional, 16-byte aligned): tvllm_sample_workspace_size(rows,
 * vocab) bytes of per-span argmax partials, so that each row's scan is
 * spread over several workgroups (an extra launch); with workspace_bytes 0
 * each row's workgroup scans the row alone. Same result either way.
 * Replaces: TorchSampler._sample_batch (reference tinyvllm/sampling.py:75-164);
 *           the noise stream differs from torch.Generator's. */
int64_t tvllm_sample_workspace_size(int64_t rows, int64_t vocab);
int tvllm_sample(const void* logits, int64_t rows, int64_t vocab,
                 int64_t row_stride, const float* temperature,
                 const int64_t* top_k, const float* top_p,
                 const int64_t* seeds, const int64_t* counters,
                 int64_t* out, void* workspace, int64_t workspace_bytes,
                 int dtype, tvllm_stream_t stream);

/* Pipelined decode inputs: tokens[i] = prev[src[i]] for 0 <= src[i] <
 * prev_count, other entries unchanged (src[i] = -1 keeps the host token).
 * prev holds the previous step's sampled token ids on the device, so the
 * host can upload step N+1's inputs before step N's tokens reach it.
 * Replaces: the host-side input-id packing of the next decode step
 * (reference tinyvllm/runtime/inputs.py:88-111), which needs the previous
 * step's tokens on the host first (tinyvllm/executor.py:135). */
int tvllm_resolve_tokens(int64_t* tokens, const int64_t* src, const int64_t* prev,
                         int64_t n, int64_t prev_count, tvllm_stream_t stream);

/* Causal paged attention for multi-token query rows (chunked prefill).
 * Item i owns query tokens q[q_offsets[i] : q_offsets[i+1]], the last
 * `query_len` of its `context_lens[i]` tokens (lower-right causal mask:
 * query j of the item sees tokens t <= context_lens[i] - query_len + j).
 * K/V of all context tokens (including this chunk's, already written)
 * come from the paged cache through blocks/block_offsets as in
 * tvllm_paged_decode. Items with q_offsets[i+1] - q_offsets[i] <= 0 are
 * skipped. max_query_len bounds every item's query length (grid size).
 * cache_dtype / k_scale / v_scale as for tvllm_paged_decode.
 * head_dim 128 runs the MFMA kernel (16-byte aligned Q and cache rows, cache
 * strides in whole 8-element units); any other head_dim <= 256 runs the
 * general kernel of tvllm_paged_decode (fp32; a workgroup per KV head and
 * up to 16 (query token, query head) rows of one item).
 * workspace: >= tvllm_paged_prefill_workspace_size(dtype, cache_dtype)
 * bytes, 4-byte aligned, zero before the first call; every call leaves it
 * zero. (A bf16 cache's V is converted to fp16 for the P.V products; a call
 * in which a V value of 65536 or more in magnitude, an infinity or a NaN
 * enters a product raises a flag there, and a second, exact launch
 * recomputes it. Calls that share one workspace must be ordered on one
 * stream.)
 * Replaces: CudaAttention._attend's per-row gather + SDPA for rows with
 * history (reference tinyvllm/runtime/attention.py:102-151, 235-285). */
int tvllm_paged_prefill(const void* q, int64_t q_token_stride,
                        int64_t q_head_stride, const void* k_cache,
                        const void* v_cache, void* out,
                        int64_t out_token_stride, int64_t out_head_stride,
                        const int64_t* q_offsets, const int64_t* blocks,
                        const int64_t* block_offsets,
                        const int64_t* context_lens, int64_t num_items,
                        int64_t max_query_len, int64_t num_heads,
                        int64_t num_kv_heads, int64_t head_dim,
                        int64_t num_slots, int64_t cache_slot_stride,
                        int64_t cache_head_stride, int64_t block_size, float scale,
                        void* workspace, int64_t workspace_bytes,
                        int dtype, int cache_dtype, float k_scale,
                        float v_scale, tvllm_stream_t stream);

/* Bytes of workspace tvllm_paged_prefill needs: 8 for a bf16 query and
 * cache (the fallback guard), 0 otherwise. No counterpart in the reference
 * (its prefill path allocates nothing of the kind). */
int64_t tvllm_paged_prefill_workspace_size(int dtype, int cache_dtype);

#ifdef __cplusplus
}
#endif

#endif /* TINYVLLM_HIP_H */

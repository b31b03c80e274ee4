// Paged KV-cache scatter: cache[slot[t]] = row t of K and V (bit copy), or,
// for an FP8 E4M3 cache, fp8(clamp(x / scale)) of every element.
//
// Reference behaviour: tinyvllm/kernels/kv_store.cu:27-90 (kernel) and
// :101-232 (host checks). slot == -1 marks graph padding and is skipped.
// (The FP8 cache has no reference counterpart.)
//
// Layout: the cache row of (slot, head) starts at slot * slot_stride +
// head * head_stride elements (token-major or head-major cache); a token's
// source row is kv_heads * head_dim elements, possibly a strided view of the
// QKV projection output. Each thread copies one 16-byte chunk of K and of V
// (8 elements of one head).
#include "common.h"

#include <algorithm>

namespace tvllm {
namespace {

constexpr int kThreads = 256;

// Vector path: both sources have packed heads (head stride == head_dim) and
// every row start is 16-byte aligned, so a token row is width/8 16B chunks.
// Cache index (in 8-element units) of chunk `chunk` of a token row stored at
// `slot`: head chunk / row8, unit chunk % row8 of that head's row.
__device__ __forceinline__ int64_t cache_unit(int64_t slot, int chunk, int row8,
                                              int64_t ss8, int64_t hs8) {
    const int head = chunk / row8;
    return slot * ss8 + head * hs8 + (chunk - head * row8);
}

__global__ void __launch_bounds__(kThreads)
store_kv_vec(const U16x8* __restrict__ key, const U16x8* __restrict__ value,
             int64_t key_stride8, int64_t value_stride8,
             U16x8* __restrict__ key_cache, U16x8* __restrict__ value_cache,
             const int64_t* __restrict__ slots, int64_t tokens, int width8, int row8,
             int64_t ss8, int64_t hs8) {
    const int64_t idx = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t token = idx / width8;
    const int chunk = int(idx - token * width8);
    if (token >= tokens) return;
    const int64_t slot = slots[token];
    if (slot < 0) return;
    const int64_t at = cache_unit(slot, chunk, row8, ss8, hs8);
    key_cache[at] = key[token * key_stride8 + chunk];
    value_cache[at] = value[token * value_stride8 + chunk];
}

// FP8 cache, vector path: each thread narrows one 16-byte source chunk into
// one 8-byte cache chunk.
template <typename T>
__global__ void __launch_bounds__(kThreads)
store_kv_vec_fp8(const U16x8* __restrict__ key, const U16x8* __restrict__ value,
                 int64_t key_stride8, int64_t value_stride8,
                 uint2* __restrict__ key_cache, uint2* __restrict__ value_cache,
                 const int64_t* __restrict__ slots, int64_t tokens, int width8, int row8,
                 int64_t ss8, int64_t hs8, float k_inv, float v_inv) {
    const int64_t idx = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t token = idx / width8;
    const int chunk = int(idx - token * width8);
    if (token >= tokens) return;
    const int64_t slot = slots[token];
    if (slot < 0) return;
    const int64_t at = cache_unit(slot, chunk, row8, ss8, hs8);
    key_cache[at] = fp8x8_narrow<T>(key[token * key_stride8 + chunk], k_inv);
    value_cache[at] = fp8x8_narrow<T>(value[token * value_stride8 + chunk], v_inv);
}

// FP8 cache, any strides: element-wise.
template <typename T>
__global__ void __launch_bounds__(kThreads)
store_kv_any_fp8(const T* __restrict__ key, const T* __restrict__ value, int64_t kts,
                 int64_t khs, int64_t vts, int64_t vhs, uint8_t* __restrict__ key_cache,
                 uint8_t* __restrict__ value_cache, const int64_t* __restrict__ slots,
                 int64_t tokens, int64_t heads, int64_t head_dim, int64_t ss, int64_t hs,
                 float k_inv, float v_inv) {
    const int64_t width = heads * head_dim;
    const int64_t token = blockIdx.x;
    if (token >= tokens) return;
    const int64_t slot = slots[token];
    if (slot < 0) return;
    for (int64_t e = threadIdx.x; e < width; e += kThreads) {
        const int64_t h = e / head_dim, d = e - h * head_dim;
        const float kx = to_f<T>(key[token * kts + h * khs + d]) * k_inv;
        const float vx = to_f<T>(value[token * vts + h * vhs + d]) * v_inv;
        key_cache[slot * ss + h * hs + d] = uint8_t(fp8x4_pack(kx, 0.f, 0.f, 0.f));
        value_cache[slot * ss + h * hs + d] = uint8_t(fp8x4_pack(vx, 0.f, 0.f, 0.f));
    }
}

// Generic path: arbitrary head strides (last stride 1), element-wise.
__global__ void __launch_bounds__(kThreads)
store_kv_any(const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
             int64_t kts, int64_t khs, int64_t vts, int64_t vhs,
             uint16_t* __restrict__ key_cache, uint16_t* __restrict__ value_cache,
             const int64_t* __restrict__ slots, int64_t tokens, int64_t heads,
             int64_t head_dim, int64_t ss, int64_t hs) {
    const int64_t width = heads * head_dim;
    const int64_t token = blockIdx.x;
    if (token >= tokens) return;
    const int64_t slot = slots[token];
    if (slot < 0) return;
    for (int64_t e = threadIdx.x; e < width; e += kThreads) {
        const int64_t h = e / head_dim, d = e - h * head_dim;
        key_cache[slot * ss + h * hs + d] = key[token * kts + h * khs + d];
        value_cache[slot * ss + h * hs + d] = value[token * vts + h * vhs + d];
    }
}

}  // namespace
}  // namespace tvllm

using namespace tvllm;

extern "C" int tvllm_store_kv(const void* key, const void* value,
                              int64_t key_token_stride, int64_t key_head_stride,
                              int64_t value_token_stride,
                              int64_t value_head_stride, void* key_cache,
                              void* value_cache, const int64_t* slots,
                              int64_t num_tokens, int64_t num_kv_heads,
                              int64_t head_dim, int64_t num_slots,
                              int64_t cache_slot_stride, int64_t cache_head_stride,
                              int dtype, int cache_dtype, float k_scale, float v_scale,
                              tvllm_stream_t stream) {
    TVLLM_CHECK(dtype == TVLLM_BF16 || dtype == TVLLM_F16,
                "store_kv: KV store requires float16 or bfloat16");
    const bool f8 = cache_dtype == TVLLM_FP8_E4M3;
    TVLLM_CHECK(f8 || cache_dtype == dtype,
                "store_kv: KV cache dtype must match the rows or be FP8 E4M3");
    TVLLM_CHECK(k_scale > 0.f && v_scale > 0.f && k_scale < INFINITY && v_scale < INFINITY,
                "store_kv: KV scales must be positive and finite");
    TVLLM_CHECK(f8 || (k_scale == 1.f && v_scale == 1.f),
                "store_kv: KV scales apply to an FP8 cache only");
    TVLLM_CHECK(num_tokens >= 0 && num_kv_heads > 0 && head_dim > 0,
                "store_kv: KV head geometry mismatch");
    TVLLM_CHECK(num_tokens <= num_slots && num_tokens <= INT32_MAX,
                "store_kv: too many KV rows");
    TVLLM_CHECK(cache_layout_ok(num_slots, num_kv_heads, head_dim, cache_slot_stride,
                                cache_head_stride),
                "store_kv: cache strides must give non-overlapping head rows");
    if (num_tokens == 0) return TVLLM_OK;
    TVLLM_CHECK(key && value && key_cache && value_cache && slots,
                "store_kv: null pointer");
    TVLLM_CHECK(key_cache != value_cache,
                "store_kv: K/V caches must use separate storage");

    const int64_t width = num_kv_heads * head_dim;
    const int64_t ss = cache_slot_stride, hs = cache_head_stride;
    const bool vec = head_dim % 8 == 0 && ss % 8 == 0 && hs % 8 == 0 &&
                     key_head_stride == head_dim &&
                     value_head_stride == head_dim && key_token_stride % 8 == 0 &&
                     value_token_stride % 8 == 0 && aligned16(key) &&
                     aligned16(value) && aligned16(key_cache) &&
                     aligned16(value_cache);
    hipStream_t s = as_hip(stream);
    if (f8) {
        const float k_inv = 1.f / k_scale, v_inv = 1.f / v_scale;
        return dispatch_half(dtype, [&]<int DT>() {
            using T = typename Elem<DT>::T;
            if (vec) {
                const int width8 = int(width / 8);
                const int64_t total = num_tokens * width8;
                const int blocks = int((total + kThreads - 1) / kThreads);
                store_kv_vec_fp8<T><<<blocks, kThreads, 0, s>>>(
                    static_cast<const U16x8*>(key), static_cast<const U16x8*>(value),
                    key_token_stride / 8, value_token_stride / 8,
                    static_cast<uint2*>(key_cache), static_cast<uint2*>(value_cache), slots,
                    num_tokens, width8, int(head_dim / 8), ss / 8, hs / 8, k_inv, v_inv);
            } else {
                store_kv_any_fp8<T><<<int(num_tokens), kThreads, 0, s>>>(
                    static_cast<const T*>(key), static_cast<const T*>(value),
                    key_token_stride, key_head_stride, value_token_stride, value_head_stride,
                    static_cast<uint8_t*>(key_cache), static_cast<uint8_t*>(value_cache), slots,
                    num_tokens, num_kv_heads, head_dim, ss, hs, k_inv, v_inv);
            }
            return launch_status("store_kv");
        });
    }
    if (vec) {
        const int width8 = int(width / 8);
        const int64_t total = num_tokens * width8;
        const int blocks = int((total + kThreads - 1) / kThreads);
        store_kv_vec<<<blocks, kThreads, 0, s>>>(
            static_cast<const U16x8*>(key), static_cast<const U16x8*>(value),
            key_token_stride / 8, value_token_stride / 8,
            static_cast<U16x8*>(key_cache), static_cast<U16x8*>(value_cache),
            slots, num_tokens, width8, int(head_dim / 8), ss / 8, hs / 8);
    } else {
        store_kv_any<<<int(num_tokens), kThreads, 0, s>>>(
            static_cast<const uint16_t*>(key), static_cast<const uint16_t*>(value),
            key_token_stride, key_head_stride, value_token_stride,
            value_head_stride, static_cast<uint16_t*>(key_cache),
            static_cast<uint16_t*>(value_cache), slots, num_tokens, num_kv_heads,
            head_dim, ss, hs);
    }
    return launch_status("store_kv");
}

// ------------------------------------------------- device block tables --
// updates = [n, index_0, id_0, index_1, id_1, ...]: table[index_i] = id_i for
// i < min(n, capacity), skipping indices outside the table. n is read on
// the device, so a captured graph applies each step's own uploaded count.
namespace tvllm {
namespace {

__global__ void __launch_bounds__(256)
apply_table_updates_kernel(int64_t* __restrict__ table, int64_t table_size,
                           const int64_t* __restrict__ updates, int64_t capacity) {
    const int64_t n = min(updates[0], capacity);
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += int64_t(gridDim.x) * blockDim.x) {
        const int64_t index = updates[1 + 2 * i];
        if (index >= 0 && index < table_size) table[index] = updates[2 + 2 * i];
    }
}

}  // namespace
}  // namespace tvllm

extern "C" int tvllm_apply_table_updates(int64_t* table, int64_t table_size,
                                         const int64_t* updates, int64_t capacity,
                                         tvllm_stream_t stream) {
    using namespace tvllm;
    TVLLM_CHECK(table_size >= 0 && capacity >= 0,
                "apply_table_updates: negative sizes");
    if (capacity == 0) return TVLLM_OK;
    TVLLM_CHECK(table && updates, "apply_table_updates: null pointer");
    // Enough threads for a typical step (a page per row); larger uploads
    // (rows entering decode with whole tables) loop.
    const int blocks = int(std::min<int64_t>((capacity + 255) / 256, 64));
    apply_table_updates_kernel<<<blocks, 256, 0, as_hip(stream)>>>(table, table_size,
                                                                     updates, capacity);
    return launch_status("apply_table_updates");
}

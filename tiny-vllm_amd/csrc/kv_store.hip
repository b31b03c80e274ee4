// Paged KV-cache scatter: cache[slot[t]] = row t of K and V (bit copy).
//
// Reference behaviour: tinyvllm/kernels/kv_store.cu:27-90 (kernel) and
// :101-232 (host checks). slot == -1 marks graph padding and is skipped.
//
// Layout: one token row is kv_heads * head_dim 16-bit words (2 KiB for
// Qwen3's 8 x 128). Each thread copies one 16-byte chunk of K and of V; the
// cache row is contiguous, the source rows may be strided views of the QKV
// projection output.
#include "common.h"

namespace tvllm {
namespace {

constexpr int kThreads = 256;

// Vector path: both sources have packed heads (head stride == head_dim) and
// every row start is 16-byte aligned, so a token row is width/8 16B chunks.
__global__ void __launch_bounds__(kThreads)
store_kv_vec(const U16x8* __restrict__ key, const U16x8* __restrict__ value,
             int64_t key_stride8, int64_t value_stride8,
             U16x8* __restrict__ key_cache, U16x8* __restrict__ value_cache,
             const int64_t* __restrict__ slots, int64_t tokens, int width8) {
    const int64_t idx = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t token = idx / width8;
    const int chunk = int(idx - token * width8);
    if (token >= tokens) return;
    const int64_t slot = slots[token];
    if (slot < 0) return;
    key_cache[slot * width8 + chunk] = key[token * key_stride8 + chunk];
    value_cache[slot * width8 + chunk] = value[token * value_stride8 + chunk];
}

// Generic path: arbitrary head strides (last stride 1), element-wise.
__global__ void __launch_bounds__(kThreads)
store_kv_any(const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
             int64_t kts, int64_t khs, int64_t vts, int64_t vhs,
             uint16_t* __restrict__ key_cache, uint16_t* __restrict__ value_cache,
             const int64_t* __restrict__ slots, int64_t tokens, int64_t heads,
             int64_t head_dim) {
    const int64_t width = heads * head_dim;
    const int64_t token = blockIdx.x;
    if (token >= tokens) return;
    const int64_t slot = slots[token];
    if (slot < 0) return;
    for (int64_t e = threadIdx.x; e < width; e += kThreads) {
        const int64_t h = e / head_dim, d = e - h * head_dim;
        key_cache[slot * width + e] = key[token * kts + h * khs + d];
        value_cache[slot * width + e] = value[token * vts + h * vhs + d];
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
                              int64_t head_dim, int64_t num_slots, int dtype,
                              tvllm_stream_t stream) {
    TVLLM_CHECK(dtype == TVLLM_BF16 || dtype == TVLLM_F16,
                "store_kv: KV store requires float16 or bfloat16");
    TVLLM_CHECK(num_tokens >= 0 && num_kv_heads > 0 && head_dim > 0,
                "store_kv: KV head geometry mismatch");
    TVLLM_CHECK(num_tokens <= num_slots && num_tokens <= INT32_MAX,
                "store_kv: too many KV rows");
    if (num_tokens == 0) return TVLLM_OK;
    TVLLM_CHECK(key && value && key_cache && value_cache && slots,
                "store_kv: null pointer");
    TVLLM_CHECK(key_cache != value_cache,
                "store_kv: K/V caches must use separate storage");

    const int64_t width = num_kv_heads * head_dim;
    const bool vec = width % 8 == 0 && key_head_stride == head_dim &&
                     value_head_stride == head_dim && key_token_stride % 8 == 0 &&
                     value_token_stride % 8 == 0 && aligned16(key) &&
                     aligned16(value) && aligned16(key_cache) &&
                     aligned16(value_cache);
    hipStream_t s = as_hip(stream);
    if (vec) {
        const int width8 = int(width / 8);
        const int64_t total = num_tokens * width8;
        const int blocks = int((total + kThreads - 1) / kThreads);
        store_kv_vec<<<blocks, kThreads, 0, s>>>(
            static_cast<const U16x8*>(key), static_cast<const U16x8*>(value),
            key_token_stride / 8, value_token_stride / 8,
            static_cast<U16x8*>(key_cache), static_cast<U16x8*>(value_cache),
            slots, num_tokens, width8);
    } else {
        store_kv_any<<<int(num_tokens), kThreads, 0, s>>>(
            static_cast<const uint16_t*>(key), static_cast<const uint16_t*>(value),
            key_token_stride, key_head_stride, value_token_stride,
            value_head_stride, static_cast<uint16_t*>(key_cache),
            static_cast<uint16_t*>(value_cache), slots, num_tokens, num_kv_heads,
            head_dim);
    }
    return launch_status("store_kv");
}

// Chunked-prefill paged attention on the gfx950 matrix cores.
//
// Reference behaviour: tinyvllm/runtime/attention.py:102-151 (SDPAAttention:
// gather the row's K/V in logical order from the paged cache, then
// F.scaled_dot_product_attention with a lower-right causal mask,
// attention.py:176-214) and :235-285 (CudaAttention._attend). A chunk of
// `query_len` new tokens attends to all `context_len` cached tokens, query j
// seeing tokens t <= context_len - query_len + j.
//
// MI355X design (head_dim 128): one 256-thread workgroup per (item, query
// head, 64-query tile); each wave owns 16 queries. K/V tiles of 64 tokens
// are gathered through the block table into LDS once per workgroup:
//  * S^T = K Q^T with MFMA 16x16x32 (A = K rows straight from LDS, B = the
//    wave's Q rows kept in registers), so the score accumulator of a lane is
//    (4 tokens x 1 query) - exactly the A-operand layout that P.V needs;
//  * P.V with MFMA 16x16x32: A = the lane's probabilities (rounded to the
//    storage type, no data movement), B = V read from an LDS copy stored
//    transposed (dims x tokens) while staging;
//  * online softmax in base 2 with one running (max, sum) per query.
#include "common.h"

#include <type_traits>

namespace tvllm {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ f32x4 mfma(const U16x8& a, const U16x8& b, f32x4 c) {
    if constexpr (std::is_same_v<T, __bf16>) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
            0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(
            __builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
            0, 0);
    }
}

constexpr int D = 128;
constexpr int BQ = 64;          // queries per workgroup (4 waves x 16)
constexpr int BK = 64;          // tokens per KV tile
constexpr int K_LD = D + 8;     // K tile row stride (elements), breaks bank aliasing
constexpr int V_LD = BK + 4;    // V^T tile row stride (elements)
constexpr float kLog2e = 1.4426950408889634f;

template <typename T>
struct PrefillArgs {
    const T* q;
    int64_t qts, qhs;
    const T* k;
    const T* v;
    T* out;
    int64_t ots, ohs;
    const int64_t* q_offsets;
    const int64_t* blocks;
    const int64_t* block_offsets;
    const int64_t* context_lens;
    int heads, kv_heads, block_size, q_tiles;
    float scale_log2;
};

template <typename T>
__global__ void __launch_bounds__(256)
paged_prefill_d128(PrefillArgs<T> a) {
    __shared__ __align__(16) uint16_t ks[BK * K_LD];
    __shared__ __align__(16) uint16_t vt[D * V_LD];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int quad = lane >> 4;
    const int col = lane & 15;

    // blockIdx.x = (item * heads + h) * q_tiles + tile
    const int tile = blockIdx.x % a.q_tiles;
    const int ih = blockIdx.x / a.q_tiles;
    const int h = ih % a.heads;
    const int item = ih / a.heads;
    const int kvh = h / (a.heads / a.kv_heads);

    const int64_t q_begin = a.q_offsets[item];
    const int64_t q_len = a.q_offsets[item + 1] - q_begin;
    const int64_t q0 = int64_t(tile) * BQ;
    if (q_len <= 0 || q0 >= q_len) return;  // uniform per workgroup
    const int64_t ctx = a.context_lens[item];
    const int64_t first_pos = ctx - q_len;  // absolute position of query 0
    const int64_t table = a.block_offsets[item];

    // This wave's queries: q0 + wave*16 + col (B operand), and the last query
    // of the workgroup bounds the KV range.
    const int64_t wq0 = q0 + wave * 16;
    const int64_t q_last = min(q_len - 1, q0 + BQ - 1);
    const int64_t kv_end = min(ctx, first_pos + q_last + 1);
    const bool wave_active = wq0 < q_len;

    U16x8 qb[4];
    {
        const int64_t qi = min(wq0 + col, q_len - 1);
        const T* qrow = a.q + (q_begin + qi) * a.qts + h * a.qhs + quad * 8;
#pragma unroll
        for (int c = 0; c < 4; ++c) qb[c] = *reinterpret_cast<const U16x8*>(qrow + c * 32);
    }
    // Query of this lane's score column, and the queries of its output rows.
    const int64_t my_pos = first_pos + wq0 + col;  // may exceed for padding

    f32x4 o[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) o[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;

    const int bs = a.block_size;
    for (int64_t t0 = 0; t0 < kv_end; t0 += BK) {
        // ---- stage K (row-major) and V (transposed) of tokens [t0, t0+64)
        __syncthreads();
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int c = it * 256 + tid;
            const int tok = c >> 4;
            const int piece = c & 15;
            const int64_t t = min(t0 + tok, kv_end - 1);
            const int64_t page = t / bs;
            const int64_t slot = a.blocks[table + page] * bs + (t - page * bs);
            const int64_t base = (slot * a.kv_heads + kvh) * D + piece * 8;
            const U16x8 kv = *reinterpret_cast<const U16x8*>(a.k + base);
            const U16x8 vv = *reinterpret_cast<const U16x8*>(a.v + base);
            *reinterpret_cast<U16x8*>(&ks[tok * K_LD + piece * 8]) = kv;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vt[(piece * 8 + 2 * e) * V_LD + tok] = uint16_t(vv.w[e] & 0xffffu);
                vt[(piece * 8 + 2 * e + 1) * V_LD + tok] = uint16_t(vv.w[e] >> 16);
            }
        }
        __syncthreads();
        if (!wave_active) continue;

        // ---- S^T tiles: s[j][i] = token t0 + 16j + 4quad + i, query col
        float s[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const U16x8 kk =
                    *reinterpret_cast<const U16x8*>(&ks[(16 * j + col) * K_LD + c * 32 + quad * 8]);
                d = mfma<T>(kk, qb[c], d);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t t = t0 + 16 * j + 4 * quad + i;
                s[j][i] = (t < kv_end && t <= my_pos) ? d[i] * a.scale_log2 : -INFINITY;
            }
        }
        float cmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) cmax = fmaxf(cmax, s[j][i]);
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
        const float m_new = fmaxf(m_run, cmax);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = exp2f(m_run - m_use);
        m_run = m_new;

        float pf[4][4];
        float psum = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = exp2f(s[j][i] - m_use);
                psum += p;
                pf[j][i] = p;
            }
        l_run = l_run * alpha + psum;

        // Rescale output rows (query 4quad + i) by their queries' alpha.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float ai = __shfl(alpha, 4 * quad + i, 64);
#pragma unroll
            for (int n = 0; n < 8; ++n) o[n][i] *= ai;
        }

        // ---- O += P V over two 32-token steps.
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const int ja = 2 * st, jb = 2 * st + 1;
            U16x8 pa;
            pa.w[0] = pack2<T>(pf[ja][0], pf[ja][1]);
            pa.w[1] = pack2<T>(pf[ja][2], pf[ja][3]);
            pa.w[2] = pack2<T>(pf[jb][0], pf[jb][1]);
            pa.w[3] = pack2<T>(pf[jb][2], pf[jb][3]);
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                const uint16_t* vrow = &vt[(16 * n + col) * V_LD];
                U16x8 vb;
                const uint2 lo = *reinterpret_cast<const uint2*>(vrow + 16 * ja + 4 * quad);
                const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16 * jb + 4 * quad);
                vb.w[0] = lo.x; vb.w[1] = lo.y; vb.w[2] = hi.x; vb.w[3] = hi.y;
                o[n] = mfma<T>(pa, vb, o[n]);
            }
        }
    }
    if (!wave_active) return;

    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t qi = wq0 + 4 * quad + i;
        const float li = __shfl(l_run, 4 * quad + i, 64);
        if (qi >= q_len) continue;
        T* orow = a.out + (q_begin + qi) * a.ots + h * a.ohs;
#pragma unroll
        for (int n = 0; n < 8; ++n) orow[16 * n + col] = static_cast<T>(o[n][i] / li);
    }
}

}  // namespace
}  // namespace tvllm

using namespace tvllm;

extern "C" int tvllm_paged_prefill(
    const void* q, int64_t q_token_stride, int64_t q_head_stride,
    const void* k_cache, const void* v_cache, void* out, int64_t out_token_stride,
    int64_t out_head_stride, const int64_t* q_offsets, const int64_t* blocks,
    const int64_t* block_offsets, const int64_t* context_lens, int64_t num_items,
    int64_t max_query_len, int64_t num_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t num_slots, int64_t block_size, float scale,
    int dtype, tvllm_stream_t stream) {
    TVLLM_CHECK(head_dim == 128, "paged_prefill: head_dim must be 128");
    TVLLM_CHECK(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
                "paged_prefill: invalid GQA geometry");
    TVLLM_CHECK(block_size > 0 && num_slots % block_size == 0,
                "paged_prefill: invalid block geometry");
    TVLLM_CHECK(num_items >= 0 && max_query_len >= 0,
                "paged_prefill: negative sizes");
    if (num_items == 0 || max_query_len == 0) return TVLLM_OK;
    TVLLM_CHECK(q && k_cache && v_cache && out && q_offsets && blocks &&
                    block_offsets && context_lens,
                "paged_prefill: null pointer");
    TVLLM_CHECK(aligned16(q) && q_token_stride % 8 == 0 && q_head_stride % 8 == 0 &&
                    aligned16(k_cache) && aligned16(v_cache),
                "paged_prefill: Q and caches must be 16-byte aligned rows");
    const int64_t q_tiles = (max_query_len + BQ - 1) / BQ;
    const int64_t grid = num_items * num_heads * q_tiles;
    TVLLM_CHECK(grid <= INT32_MAX, "paged_prefill: grid too large");
    hipStream_t s = as_hip(stream);
    return dispatch_half(dtype, [&]<int DT>() {
        using T = typename Elem<DT>::T;
        PrefillArgs<T> args;
        args.q = static_cast<const T*>(q);
        args.qts = q_token_stride;
        args.qhs = q_head_stride;
        args.k = static_cast<const T*>(k_cache);
        args.v = static_cast<const T*>(v_cache);
        args.out = static_cast<T*>(out);
        args.ots = out_token_stride;
        args.ohs = out_head_stride;
        args.q_offsets = q_offsets;
        args.blocks = blocks;
        args.block_offsets = block_offsets;
        args.context_lens = context_lens;
        args.heads = int(num_heads);
        args.kv_heads = int(num_kv_heads);
        args.block_size = int(block_size);
        args.q_tiles = int(q_tiles);
        args.scale_log2 = scale * kLog2e;
        paged_prefill_d128<T><<<int(grid), 256, 0, s>>>(args);
        return launch_status("paged_prefill");
    });
}

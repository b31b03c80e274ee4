// Chunked-prefill paged attention on the gfx950 matrix cores.
//
// Reference behaviour: tinyvllm/runtime/attention.py:102-151 (SDPAAttention:
// gather the row's K/V in logical order from the paged cache, then
// F.scaled_dot_product_attention with a lower-right causal mask,
// attention.py:176-214) and :235-285 (CudaAttention._attend). A chunk of
// `query_len` new tokens attends to all `context_len` cached tokens, query j
// seeing tokens t <= context_len - query_len + j.
//
// MI355X design (head_dim 128): one workgroup of W waves per (item, query
// head, tile of 16*QB*W queries); each wave owns QB blocks of 16 queries.
// K/V tiles of 64 tokens are gathered through the block table into LDS once
// per workgroup, double-buffered: the next tile's global loads are issued
// into registers before the current tile's MFMA work and written to the
// other LDS buffer after it, so there is one barrier per tile.
//  * S^T = K Q^T with MFMA 16x16x32 (A = K rows from LDS, shared by the
//    wave's QB query blocks; B = Q rows held in registers). A lane's score
//    accumulator is (4 tokens x its own query) - exactly the B-operand
//    layout of the transposed product below, so P never moves.
//  * O^T += V^T P^T with MFMA 16x16x32: A = V^T read from an LDS copy that
//    staging stores transposed (dims x tokens, 8-byte writes of 4 tokens),
//    B = the lane's probabilities rounded to the storage type. The O^T
//    accumulator of a lane belongs to its own query, so the online-softmax
//    rescale and the final 1/l need no cross-lane traffic.
//  * online softmax in base 2 (v_exp_f32), one running (max, sum) per query,
//    raised lazily (kSlack) so most tiles skip the accumulator rescale;
//    key tiles past a wave's last query are skipped (causal), and tiles
//    entirely below its first query skip the mask.
// Work order: block ids are spread over the 8 XCDs so the workgroups of one
// (item, KV head) share an XCD's L2, and the causal tiles with the most keys
// start first.
#include "common.h"

#include <cstdio>
#include <cstdlib>
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
constexpr int BK = 64;          // tokens per KV tile
constexpr int K_LD = D + 8;     // K tile row stride (elements), breaks bank aliasing
constexpr int V_LD = BK + 4;    // V^T tile row stride (elements)
constexpr int K_TILE = BK * K_LD;
constexpr int V_TILE = D * V_LD;
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
    int heads, kv_heads, block_size, block_shift, q_tiles, grid;
    float scale_log2;
};

// Running maxima are only raised when a tile's maximum exceeds them by more
// than this (log2 units): probabilities then stay below 2^kSlack, and most
// tiles skip the rescale of the output accumulators.
constexpr float kSlack = 8.f;

__device__ __forceinline__ float as_f(uint32_t x) { return __uint_as_float(x); }
__device__ __forceinline__ uint32_t as_u(float x) { return __float_as_uint(x); }

// Reductions over the four lanes col, col+16, col+32, col+48 (the quads that
// share one query), with the gfx950 row-swap permutes instead of LDS shuffles.
__device__ __forceinline__ float quad_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(as_u(x), as_u(x), false, false);
    x = fmaxf(as_f(a[0]), as_f(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(as_u(x), as_u(x), false, false);
    return fmaxf(as_f(b[0]), as_f(b[1]));
}
__device__ __forceinline__ float quad_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(as_u(x), as_u(x), false, false);
    x = as_f(a[0]) + as_f(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(as_u(x), as_u(x), false, false);
    return as_f(b[0]) + as_f(b[1]);
}

__device__ __forceinline__ uint32_t half16(const U16x8& v, int e) {
    return (v.w[e >> 1] >> (16 * (e & 1))) & 0xffffu;
}

template <typename T, int QB, int W>
__global__ void __launch_bounds__(64 * W)
paged_prefill_d128(PrefillArgs<T> a) {
    constexpr int NTH = 64 * W;
    constexpr int BQ = 16 * QB * W;      // queries per workgroup
    constexpr int JOBS = 2 * 16 * 16;    // (K|V) x 16 token quads x 16 pieces
    static_assert(JOBS % NTH == 0, "staging jobs must divide the threads");
    constexpr int JPT = JOBS / NTH;
    __shared__ __align__(16) uint16_t ks[2][K_TILE];
    __shared__ __align__(16) uint16_t vt[2][V_TILE];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int quad = lane >> 4;
    const int col = lane & 15;

    // XCD-aware order: hardware deals block ids round-robin over 8 XCDs;
    // give each XCD a contiguous range of logical work.
    int bid = blockIdx.x;
    if (a.grid % 8 == 0) bid = (bid % 8) * (a.grid / 8) + bid / 8;
    const int tile = a.q_tiles - 1 - bid % a.q_tiles;  // most keys first
    const int ih = bid / a.q_tiles;
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
    const int64_t kv_end = min(ctx, first_pos + min(q_len - 1, q0 + BQ - 1) + 1);

    // This wave's queries: wq0 + 16b + col for block b.
    const int64_t wq0 = q0 + int64_t(wave) * 16 * QB;
    const bool wave_active = wq0 < q_len;
    const int64_t wave_kv_end = min(kv_end, first_pos + min(q_len - 1, wq0 + 16 * QB - 1) + 1);
    const int64_t wave_first_pos = first_pos + wq0;

    U16x8 qb[QB][4];
    int64_t my_pos[QB];
#pragma unroll
    for (int b = 0; b < QB; ++b) {
        const int64_t qi = min(wq0 + 16 * b + col, q_len - 1);
        my_pos[b] = first_pos + qi;
        const T* qrow = a.q + (q_begin + qi) * a.qts + h * a.qhs + quad * 8;
#pragma unroll
        for (int c = 0; c < 4; ++c) qb[b][c] = *reinterpret_cast<const U16x8*>(qrow + c * 32);
    }

    f32x4 o[QB][8];  // O^T: lane = (dims 16n + 4quad + i, query col)
#pragma unroll
    for (int b = 0; b < QB; ++b)
#pragma unroll
        for (int n = 0; n < 8; ++n) o[b][n] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run[QB], l_run[QB];
#pragma unroll
    for (int b = 0; b < QB; ++b) {
        m_run[b] = -INFINITY;
        l_run[b] = 0.f;
    }

    // Staging: job = (kind, piece, token quad); 4 tokens x 16 bytes each.
    const int bs = a.block_size;
    U16x8 stage[JPT][4];
    auto job_coords = [&](int r, bool& is_v, int& tq, int& piece) {
        const int job = tid + r * NTH;
        is_v = job >> 8;
        // K: piece fastest (a token row per 16 lanes, conflict-free 16-byte
        // LDS writes); V: token quad fastest (conflict-free transposed writes).
        tq = is_v ? (job & 15) : ((job >> 4) & 15);
        piece = is_v ? ((job >> 4) & 15) : (job & 15);
    };
    // Block ids are fetched one tile ahead of the K/V loads that use them, so
    // the two dependent global loads never sit back to back on the critical path.
    auto load_ids = [&](int64_t t0, int64_t (&ids)[JPT][4]) {
#pragma unroll
        for (int r = 0; r < JPT; ++r) {
            bool is_v;
            int tq, piece;
            job_coords(r, is_v, tq, piece);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t t = min(t0 + 4 * tq + e, kv_end - 1);
                const int64_t page = a.block_shift >= 0 ? (t >> a.block_shift) : t / bs;
                ids[r][e] = a.blocks[table + page];
            }
        }
    };
    auto load_tile = [&](int64_t t0, const int64_t (&ids)[JPT][4]) {
#pragma unroll
        for (int r = 0; r < JPT; ++r) {
            bool is_v;
            int tq, piece;
            job_coords(r, is_v, tq, piece);
            const T* src = is_v ? a.v : a.k;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t t = min(t0 + 4 * tq + e, kv_end - 1);
                const int64_t in_page = a.block_shift >= 0 ? (t & (bs - 1)) : t % bs;
                const int64_t slot = ids[r][e] * bs + in_page;
                stage[r][e] = *reinterpret_cast<const U16x8*>(
                    src + (slot * a.kv_heads + kvh) * D + piece * 8);
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int r = 0; r < JPT; ++r) {
            bool is_v;
            int tq, piece;
            job_coords(r, is_v, tq, piece);
            if (is_v) {
                // V^T: dim row (piece*8 + dd), tokens 4tq..4tq+3 -> one 8-byte write.
#pragma unroll
                for (int dd = 0; dd < 8; ++dd) {
                    uint2 w;
                    w.x = half16(stage[r][0], dd) | (half16(stage[r][1], dd) << 16);
                    w.y = half16(stage[r][2], dd) | (half16(stage[r][3], dd) << 16);
                    *reinterpret_cast<uint2*>(&vt[buf][(piece * 8 + dd) * V_LD + 4 * tq]) = w;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    *reinterpret_cast<U16x8*>(&ks[buf][(4 * tq + e) * K_LD + piece * 8]) =
                        stage[r][e];
            }
        }
    };

    int64_t ids_next[JPT][4], ids_after[JPT][4];
    load_ids(0, ids_next);
    load_tile(0, ids_next);
    if (BK < kv_end) load_ids(BK, ids_next);
    store_tile(0);
    __syncthreads();
    int buf = 0;
    for (int64_t t0 = 0; t0 < kv_end; t0 += BK, buf ^= 1) {
        const bool has_next = t0 + BK < kv_end;
        if (has_next) {
            load_tile(t0 + BK, ids_next);
            if (t0 + 2 * BK < kv_end) load_ids(t0 + 2 * BK, ids_after);
        }

        if (wave_active && t0 < wave_kv_end) {
            const uint16_t* kt = ks[buf];
            const uint16_t* vtt = vt[buf];
            // ---- S^T tiles: s[b][j][i] = token t0 + 16j + 4quad + i, query (b, col)
            float s[QB][4][4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f32x4 d[QB];
#pragma unroll
                for (int b = 0; b < QB; ++b) d[b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const U16x8 kk = *reinterpret_cast<const U16x8*>(
                        &kt[(16 * j + col) * K_LD + c * 32 + quad * 8]);
#pragma unroll
                    for (int b = 0; b < QB; ++b) d[b] = mfma<T>(kk, qb[b][c], d[b]);
                }
#pragma unroll
                for (int b = 0; b < QB; ++b)
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[b][j][i] = d[b][i];
            }
            if (t0 + BK - 1 > wave_first_pos) {  // tile crosses the diagonal
#pragma unroll
                for (int b = 0; b < QB; ++b)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int64_t t = t0 + 16 * j + 4 * quad + i;
                            if (t > my_pos[b]) s[b][j][i] = -INFINITY;
                        }
            }
            U16x8 pb[QB][2];
#pragma unroll
            for (int b = 0; b < QB; ++b) {
                float cmax = -INFINITY;
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) cmax = fmaxf(cmax, s[b][j][i]);
                const float cm = quad_max(cmax) * a.scale_log2;  // scale > 0
                const bool grow = cm > m_run[b] + kSlack;  // also: first finite max
                float alpha = 1.f;
                if (grow) {
                    alpha = __builtin_amdgcn_exp2f(m_run[b] - cm);
                    m_run[b] = cm;
                }
                if (__builtin_amdgcn_ballot_w64(grow)) {  // wave-uniform
                    l_run[b] *= alpha;
#pragma unroll
                    for (int n = 0; n < 8; ++n) o[b][n] *= alpha;
                }
                const float m_use = m_run[b] == -INFINITY ? 0.f : m_run[b];
                float psum = 0.f;
                float pf[4][4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        pf[j][i] = __builtin_amdgcn_exp2f(
                            __builtin_fmaf(s[b][j][i], a.scale_log2, -m_use));
                        psum += pf[j][i];
                    }
                l_run[b] += psum;
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const int ja = 2 * st, jb = 2 * st + 1;
                    pb[b][st].w[0] = pack2<T>(pf[ja][0], pf[ja][1]);
                    pb[b][st].w[1] = pack2<T>(pf[ja][2], pf[ja][3]);
                    pb[b][st].w[2] = pack2<T>(pf[jb][0], pf[jb][1]);
                    pb[b][st].w[3] = pack2<T>(pf[jb][2], pf[jb][3]);
                }
            }
            // ---- O^T += V^T P^T over two 32-token steps.
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const int ja = 2 * st, jb = 2 * st + 1;
#pragma unroll
                for (int n = 0; n < 8; ++n) {
                    const uint16_t* vrow = &vtt[(16 * n + col) * V_LD];
                    U16x8 va;
                    const uint2 lo = *reinterpret_cast<const uint2*>(vrow + 16 * ja + 4 * quad);
                    const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16 * jb + 4 * quad);
                    va.w[0] = lo.x; va.w[1] = lo.y; va.w[2] = hi.x; va.w[3] = hi.y;
#pragma unroll
                    for (int b = 0; b < QB; ++b) o[b][n] = mfma<T>(va, pb[b][st], o[b][n]);
                }
            }
        }
        if (has_next) store_tile(buf ^ 1);
        __syncthreads();
#pragma unroll
        for (int r = 0; r < JPT; ++r)
#pragma unroll
            for (int e = 0; e < 4; ++e) ids_next[r][e] = ids_after[r][e];
    }
    if (!wave_active) return;

#pragma unroll
    for (int b = 0; b < QB; ++b) {
        const float l = quad_sum(l_run[b]);
        const int64_t qi = wq0 + 16 * b + col;
        if (qi >= q_len) continue;
        const float inv = 1.f / l;
        T* orow = a.out + (q_begin + qi) * a.ots + h * a.ohs + 4 * quad;
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            uint2 w;
            w.x = pack2<T>(o[b][n][0] * inv, o[b][n][1] * inv);
            w.y = pack2<T>(o[b][n][2] * inv, o[b][n][3] * inv);
            *reinterpret_cast<uint2*>(orow + 16 * n) = w;
        }
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
    TVLLM_CHECK(scale > 0.f && scale < INFINITY, "paged_prefill: scale must be positive");
    if (num_items == 0 || max_query_len == 0) return TVLLM_OK;
    TVLLM_CHECK(q && k_cache && v_cache && out && q_offsets && blocks &&
                    block_offsets && context_lens,
                "paged_prefill: null pointer");
    TVLLM_CHECK(aligned16(q) && q_token_stride % 8 == 0 && q_head_stride % 8 == 0 &&
                    aligned16(k_cache) && aligned16(v_cache),
                "paged_prefill: Q and caches must be 16-byte aligned rows");
    TVLLM_CHECK(out_token_stride % 4 == 0 && out_head_stride % 4 == 0 && aligned8(out),
                "paged_prefill: output rows must be 8-byte aligned");
    // Queries per wave: 16*QB; a workgroup of W waves covers 16*QB*W queries.
    // Eight waves per workgroup (two or three per SIMD) keep the MFMA pipes
    // fed while other waves run their softmax; 4-wave shapes measured slower.
    int qb = max_query_len > 128 ? 2 : 1;
    int waves = 8;
    if (const char* env = std::getenv("TVLLM_PREFILL_TUNING")) {
        // Measurement override "qb,waves": one of 1,4 2,4 4,4 1,8 2,8.
        int eq = 0, ew = 0;
        if (std::sscanf(env, "%d,%d", &eq, &ew) == 2 &&
            ((ew == 4 && (eq == 1 || eq == 2 || eq == 4)) ||
             (ew == 8 && (eq == 1 || eq == 2)))) {
            qb = eq;
            waves = ew;
        }
    }
    const int64_t bq = 16 * qb * waves;
    const int64_t q_tiles = (max_query_len + bq - 1) / bq;
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
        args.grid = int(grid);
        args.scale_log2 = scale * kLog2e;
        args.block_shift = (block_size & (block_size - 1)) == 0
                               ? __builtin_ctzll(uint64_t(block_size)) : -1;
        if (waves == 8) {
            if (qb == 2) paged_prefill_d128<T, 2, 8><<<int(grid), 512, 0, s>>>(args);
            else paged_prefill_d128<T, 1, 8><<<int(grid), 512, 0, s>>>(args);
        } else if (qb == 4) {
            paged_prefill_d128<T, 4, 4><<<int(grid), 256, 0, s>>>(args);
        } else if (qb == 2) {
            paged_prefill_d128<T, 2, 4><<<int(grid), 256, 0, s>>>(args);
        } else {
            paged_prefill_d128<T, 1, 4><<<int(grid), 256, 0, s>>>(args);
        }
        return launch_status("paged_prefill");
    });
}

// Paged single-query (decode) attention for gfx950.
//
// Semantics follow the reference kernel tinyvllm/kernels/paged_decode.cu:92-466
// (host contract :469-669): for decode row r and query head h,
//   out[rows[r], h] = sum_t softmax_t(scale * q . k_t) v_t,  t < lengths[r],
// token t lives at slot blocks[offsets[r] + t / bs] * bs + t % bs, KV head
// h / (Hq / Hkv); zero-length rows produce zeros (reference :130-135).
// Unlike the reference kernel, which rounds the PV weights to the storage
// type (:332-333), the weights stay fp32 here: the PV product runs on the
// VALU where that costs nothing, and the result then tracks the reference's
// torch path (SDPAAttention, fp32 softmax) to well under one bf16 ulp.
//
// MI355X design (head_dim 128, the fast path):
//  * one wave64 workgroup per (row, KV head, split): the G = Hq/Hkv query
//    heads of a KV head share every K/V byte it loads, so the cache is read
//    once per KV head instead of once per query head;
//  * split-K inside the workgroup: a row's pages are cut into `splits` (<= 8)
//    equal page ranges, one wave each, so rows x KV heads x splits waves fill
//    the 256 CUs; the waves of one (row, KV head) sit in the same workgroup
//    and merge their (max, sum, unnormalised output) partials through LDS
//    with the usual LSE rescale - no partials in HBM, no merge kernel;
//  * Q.K^T on the matrix cores: per 16-token tile, 4 MFMA 16x16x32 steps with
//    A = K rows (natural cache layout, 64 contiguous bytes per lane quad),
//    B = the G query rows zero-padded to 16 columns;
//  * P.V on the matrix cores too, with no data movement: per 16-token tile,
//    D[head][dim] += P[head][token] V[token][dim] on 16x16x16 MFMAs whose k
//    index is the token. The scores a lane holds (its head, tokens
//    4*quad + i) are exactly its A operand, and the V row pieces it loaded
//    (tokens 4*quad + i, dims 8*col .. +7) hold its B operand of MFMA e
//    (column col = dim 8*col + e): element e of its four rows, gathered
//    with two v_perm. P enters as a pair of storage-type terms (rounded P
//    and the rounded remainder, two MFMAs), so the product keeps about 16
//    bits of P - as accurate as fp32 P on the VALU; the denominator sums
//    the unrounded P;
//  * 64 tokens per iteration: 16 K and 16 V 16-byte loads per lane in flight
//    (32 KiB per wave) before any arithmetic waits on them.
#include "common.h"
#include "general_attention.h"

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <type_traits>

namespace tvllm {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// D[16x16] += A[16x16] B[16x16]: lane l supplies A row l%16 and B column
// l%16 with k = 4*(l/16)..+3 (one 8-byte pair of words each); D as for
// the 16x16x32 form.
template <typename T>
__device__ __forceinline__ f32x4 mfma16x16x16(uint2 a, uint2 b, f32x4 c) {
    typedef short s16x4_t __attribute__((ext_vector_type(4)));
    typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
    if constexpr (std::is_same_v<T, __bf16>) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
            __builtin_bit_cast(s16x4_t, a), __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(
            __builtin_bit_cast(f16x4_t, a), __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
    }
}

template <typename T>
__device__ __forceinline__ f32x4 mfma16x16x32(const U16x8& a, const U16x8& b,
                                              f32x4 c) {
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

// Broadcast lane (row_base + G) of every 16-lane row to the whole row.
template <int G>
__device__ __forceinline__ float row_bcast(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                           0x150 + G, 0xf, 0xf, false));
}

template <int L>
__device__ __forceinline__ float read_lane(float v) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), L));
}

__device__ __forceinline__ uint32_t shfl_u32(uint32_t v, int src) {
    return static_cast<uint32_t>(__shfl(static_cast<int>(v), src, 64));
}

constexpr float kLog2e = 1.4426950408889634f;

// K and V rows are streamed exactly once per step and each load instruction
// covers whole 128-byte lines: non-temporal loads measure ~13% more read
// bandwidth on MI355X for such streams (7.1 vs 6.3 TB/s).
__device__ __forceinline__ U16x8 load_stream(const U16x8* p) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    U16x8 r;
    r.w[0] = t[0];
    r.w[1] = t[1];
    r.w[2] = t[2];
    r.w[3] = t[3];
    return r;
}
__device__ __forceinline__ uint2 load_stream(const uint2* p) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 t = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    return make_uint2(t[0], t[1]);
}

template <typename T>
struct DecodeArgs {
    const T* q;
    int64_t qts, qhs;
    const void* k;  // cache rows: 16 units of 8 elements (16 B, or 8 B for FP8)
    const void* v;
    int64_t css, chs;  // cache slot / head strides (elements, multiples of 8)
    T* out;
    int64_t ots, ohs;
    const int64_t* rows;
    const int64_t* blocks;
    const int64_t* offsets;
    const int64_t* lengths;
    int heads, kv_heads, group, block_size;
    int splits;         // waves per KV head per workgroup
    int grid_splits;    // workgroups per (row, KV head group)
    int num_rows;       // rows of the batch (balanced spans scan their lengths)
    int heads_per_wg;   // KV heads per workgroup
    float scale_log2;   // softmax scale * log2(e) (* k_scale for FP8): base-2 scores
    float v_scale;      // FP8 cache: V dequantisation scale (1 otherwise)
    float k_inv_scale;  // FP8 cache: 1 / scale of the new rows written (fused)
    float v_inv_scale;
    float* part_o;      // [rows, heads, grid_splits, 128] (grid_splits > 1)
    float* part_ml;     // [rows, heads, grid_splits, 2]
    // Fused QK-norm + RoPE + KV write (FUSED kernels only): q above is the
    // raw projection; the row's new K/V come from kraw/vraw (token strides,
    // head strides), are normalised/rotated and written to slot slots[tok].
    const T* kraw;
    int64_t krts, krhs;
    const T* vraw;
    int64_t vrts, vrhs;
    const T* qw;
    const T* kw;
    const T* cos_t;     // [tokens, 64]
    const T* sin_t;
    float q_eps, k_eps;
    void* kcache;       // writable views of k / v
    void* vcache;
    const int64_t* slots;
    // Split-K qkv (PARTS kernels): the raw projections as kQkvParts fp32
    // slices of the reduction, [slice][row][q heads | k heads | v heads]
    // x 128, slice stride pss and row stride pts (elements).
    const float* parts;
    int64_t pss, pts;
};

constexpr int kQkvParts = 4;

constexpr int kMaxWaves = 8;  // 2 resident waves per SIMD at <= 256 VGPRs
// Page ranges per (row, KV head): a single row of 8 KV heads needs 128-256
// to put a wave on every SIMD (1 row x 32k tokens, 8B heads: 58.4 us with
// 64, 36.8 us with 256); the workgroup-level splits stay <= 64 (the merge
// kernel holds one per lane) because a workgroup takes at least four ranges.
constexpr int64_t kMaxSplits = 256;
constexpr int64_t kMaxGridSplits = 64;

__device__ __forceinline__ float fast_exp2(float x) {
    return __builtin_amdgcn_exp2f(x);  // v_exp_f32; inputs here are <= 0
}

// The query's norm weights and RoPE angles (lane: dims c*32 + quad*8 + e),
// loaded in the kernel prologue ahead of the first K/V rows.
struct RopeIn {
    U16x8 w[4], c[2], s[2];
};

template <typename T>
__device__ __forceinline__ RopeIn load_rope_in(const T* __restrict__ w, const T* __restrict__ cs,
                                               const T* __restrict__ sn, int quad) {
    RopeIn in;
#pragma unroll
    for (int c = 0; c < 4; ++c) in.w[c] = *reinterpret_cast<const U16x8*>(w + c * 32 + quad * 8);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        in.c[c] = *reinterpret_cast<const U16x8*>(cs + c * 32 + quad * 8);
        in.s[c] = *reinterpret_cast<const U16x8*>(sn + c * 32 + quad * 8);
    }
    return in;
}

// Fused QK-norm + RoPE for the decode step (head_dim 128), with the
// rounding points of the standalone kernel (reference pointwise.cu:325-450):
//   n = round(round(x * rsqrt(mean(x^2) + eps)) * w);
//   o1 = round(round(n1*cos) - round(n2*sin)), o2 = round(round(n2*cos) + round(n1*sin)).
// Query: in place on the MFMA B operand (lane = head col, quad; dims c*32 +
// quad*8 + e), the sum of squares reduced over the four quads.
template <typename T>
__device__ __forceinline__ void rope_query(U16x8 (&qb)[4], const RopeIn& in, float eps) {
    float x[4][8];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        unpack8<T>(qb[c], x[c]);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += x[c][e] * x[c][e];
    }
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    const float inv = rsqrtf(ss * (1.0f / 128.f) + eps);
    float wv[4][8], cv[2][8], sv[2][8];
#pragma unroll
    for (int c = 0; c < 4; ++c) unpack8<T>(in.w[c], wv[c]);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        unpack8<T>(in.c[c], cv[c]);
        unpack8<T>(in.s[c], sv[c]);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        float o1[8], o2[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float n1 = rnd<T>(rnd<T>(x[c][e] * inv) * wv[c][e]);
            const float n2 = rnd<T>(rnd<T>(x[c + 2][e] * inv) * wv[c + 2][e]);
            o1[e] = rnd<T>(n1 * cv[c][e]) - rnd<T>(n2 * sv[c][e]);
            o2[e] = rnd<T>(n2 * cv[c][e]) + rnd<T>(n1 * sv[c][e]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            qb[c].w[e] = pack2<T>(o1[2 * e], o1[2 * e + 1]);
            qb[c + 2].w[e] = pack2<T>(o2[2 * e], o2[2 * e + 1]);
        }
    }
}

// New K row: normalised and rotated exactly as the standalone kernel does
// (lane l owns the pair (l, l + 64), one wave-wide sum of squares), written
// with the V row into the cache slot.
// FP8 cache (F8): the rounded K element and the V element are quantised
// with the cache's inverse scales, as the standalone kernels do.
// The new K/V row's inputs for lane l: the raw K pair (l, l + 64), its
// norm weights and RoPE angle, and the raw V pair. Loaded by every wave in
// the kernel prologue (a few cached words), so that the wave that writes the
// row does not add a memory round trip of its own.
template <typename T>
struct NewKV {
    float x1, x2, w1, w2, c, s;
    T v1, v2;  // copied bit for bit (16-bit caches)
};

template <typename T>
__device__ __forceinline__ NewKV<T> load_new_kv(const T* __restrict__ k, const T* __restrict__ v,
                                             const T* __restrict__ w, const T* __restrict__ cs,
                                             const T* __restrict__ sn, int lane) {
    return NewKV<T>{to_f<T>(k[lane]), to_f<T>(k[lane + 64]), to_f<T>(w[lane]),
                    to_f<T>(w[lane + 64]), to_f<T>(cs[lane]),  to_f<T>(sn[lane]),
                    v[lane], v[lane + 64]};
}

// The same inputs from split-K partials: each raw element is the fp32 sum of
// its kQkvParts slices in slice order, rounded once to T (what a single GEMM
// with fp32 accumulation stores, up to the order of the sum).
template <typename T>
__device__ __forceinline__ float sum_parts(const float* __restrict__ p, int64_t pss) {
    float x[kQkvParts];
#pragma unroll
    for (int s = 0; s < kQkvParts; ++s) x[s] = p[s * pss];
    float t = x[0];
#pragma unroll
    for (int s = 1; s < kQkvParts; ++s) t += x[s];
    return t;
}

template <typename T>
__device__ __forceinline__ NewKV<T> load_new_kv_parts(const float* __restrict__ k,
                                                   const float* __restrict__ v, int64_t pss,
                                                   const T* __restrict__ w,
                                                   const T* __restrict__ cs,
                                                   const T* __restrict__ sn, int lane) {
    return NewKV<T>{rnd<T>(sum_parts<T>(k + lane, pss)), rnd<T>(sum_parts<T>(k + lane + 64, pss)),
                    to_f<T>(w[lane]), to_f<T>(w[lane + 64]), to_f<T>(cs[lane]),
                    to_f<T>(sn[lane]), static_cast<T>(sum_parts<T>(v + lane, pss)),
                    static_cast<T>(sum_parts<T>(v + lane + 64, pss))};
}

// New K row: normalised and rotated exactly as the standalone kernel does
// (lane l owns the pair (l, l + 64), one wave-wide sum of squares), written
// with the V row into the cache slot.
// FP8 cache (F8): the rounded K element and the V element are quantised
// with the cache's inverse scales, as the standalone kernels do.
template <typename T, bool F8>
__device__ __forceinline__ void write_new_kv(const NewKV<T>& in, float eps,
                                             void* __restrict__ kdst, void* __restrict__ vdst,
                                             float k_inv, float v_inv, int lane) {
    const float ss = wave_sum(in.x1 * in.x1 + in.x2 * in.x2);
    const float inv = rsqrtf(ss * (1.0f / 128.f) + eps);
    const float n1 = rnd<T>(rnd<T>(in.x1 * inv) * in.w1);
    const float n2 = rnd<T>(rnd<T>(in.x2 * inv) * in.w2);
    const float o1 = rnd<T>(rnd<T>(n1 * in.c) - rnd<T>(n2 * in.s));
    const float o2 = rnd<T>(rnd<T>(n2 * in.c) + rnd<T>(n1 * in.s));
    if constexpr (F8) {
        uint8_t* kd = static_cast<uint8_t*>(kdst);
        uint8_t* vd = static_cast<uint8_t*>(vdst);
        const uint32_t kq = fp8x4_pack(o1 * k_inv, o2 * k_inv, 0.f, 0.f);
        const uint32_t vq = fp8x4_pack(to_f<T>(in.v1) * v_inv, to_f<T>(in.v2) * v_inv, 0.f, 0.f);
        kd[lane] = uint8_t(kq);
        kd[lane + 64] = uint8_t(kq >> 8);
        vd[lane] = uint8_t(vq);
        vd[lane + 64] = uint8_t(vq >> 8);
    } else {
        T* kd = static_cast<T*>(kdst);
        T* vd = static_cast<T*>(vdst);
        kd[lane] = static_cast<T>(o1);
        kd[lane + 64] = static_cast<T>(o2);
        vd[lane] = in.v1;
        vd[lane + 64] = in.v2;
    }
}

// GP: group size rounded up to a power of two (<= 16); NT: 16-token MFMA
// tiles per iteration. Wave w of a workgroup owns KV head
// (group of the workgroup) * heads_per_wg + w / splits and page range
// w % splits of its row.
// F8: the cache holds FP8 E4M3 rows (8-byte units; K widened exactly to T
// for the MFMA, V to f32 for P.V, the scales folded into the softmax scale
// and the final normalisation).
template <typename T, int GP, int NT, int MAXW, bool FUSED, bool F8, bool PARTS>
__global__ void __launch_bounds__(64 * MAXW)
paged_decode_d128(DecodeArgs<T> a) {
    static_assert(FUSED || !PARTS, "partial sums feed the fused prologue only");
    constexpr int D = 128;
    constexpr int ROW16 = D / 8;  // 8-element units per cache row of one head
    using Unit = std::conditional_t<F8, uint2, U16x8>;  // 8 cached elements
    constexpr int CH = 16 * NT;   // tokens per iteration
    static_assert(CH <= 64, "one lane resolves one token of an iteration");
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int quad = lane >> 4;   // 16-lane row of the wave
    const int col = lane & 15;

    // blockIdx.x = (r * head_groups + head group) * grid_splits + grid split
    const int head_groups = a.kv_heads / a.heads_per_wg;
    const int gsplit = blockIdx.x % a.grid_splits;
    const int unit = blockIdx.x / a.grid_splits;
    const int r = unit / head_groups;
    const int local_head = wave / a.splits;
    const int split = wave - local_head * a.splits;
    const int kvh = (unit - r * head_groups) * a.heads_per_wg + local_head;
    const int h0 = kvh * a.group;
    // This wave's KV head rows: slot s at unit s * slot_units past kc / vc
    // (32-bit offsets: the host checks that every slot's offset fits).
    const int64_t head_units = int64_t(__builtin_amdgcn_readfirstlane(kvh)) * (a.chs >> 3);
    const Unit* const kc = static_cast<const Unit*>(a.k) + head_units;
    const Unit* const vc = static_cast<const Unit*>(a.v) + head_units;
    const uint64_t slot_units = uint64_t(a.css >> 3);

    const int64_t row = a.rows[r];
    const int64_t length = a.lengths[r];
    const int bs = a.block_size;
    const int64_t pages = (length + bs - 1) / bs;
    const int total_splits = a.splits * a.grid_splits;
    // One workgroup per row (grid_splits == 1): the row's pages are divided
    // evenly among its waves. Several workgroups per row (long contexts):
    // every row uses the same span, sized from the longest row of the batch,
    // so the workgroups of shorter rows past their end exit at once and the
    // dispatcher balances the remaining ones across the CUs.
    int64_t span_pages = pages;
    if (a.grid_splits > 1) {
        int64_t longest = 0;
        for (int i = lane; i < a.num_rows; i += 64) longest = max(longest, a.lengths[i]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            longest = max(longest, static_cast<int64_t>(__shfl_xor(longest, off, 64)));
        span_pages = (longest + bs - 1) / bs;
    }
    // Fused: the range holding the new token starts late (its wave first
    // loads, normalises, rotates and writes the new K/V row), and it is the
    // row's last range, so the others take up to two pages more each, for
    // rows long enough that every range keeps several pages (whole-step
    // Qwen3-8B bs64 ctx2k: 7.885 -> 7.874 ms, 3/3 alternated runs). The
    // ranges still cover [0, pages) exactly.
    const int64_t pad = (FUSED && span_pages >= 8 * total_splits) ? 2 : 0;
    const int64_t per_split = (span_pages + pad + total_splits - 1) / total_splits;
    const int64_t p_begin = int64_t(gsplit * a.splits + split) * per_split;
    const int64_t p_end = min(pages, p_begin + per_split);
    const int64_t t_begin = p_begin * bs;
    const int64_t t_end = min(length, p_end * bs);

    // acc[e][v]: output head 4*quad + v, dim 8*col + e (the P.V MFMA layout).
    f32x4 acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;  // running max (base-2 units), per score lane
    float l_run = 0.f;        // this lane's share of the denominator

    // An empty range (zero-length padding row, or more splits than pages)
    // reads nothing - not even Q or the block table - but still joins the
    // workgroup merge below.
    if (t_begin < t_end) {
        const int64_t table = a.offsets[r];

        // The new token's slot (a scalar load, issued with the row's metadata).
        const int64_t new_slot = FUSED ? a.slots[row] : -1;
        NewKV<T> new_kv{};
        // B operand: query head g = col (zero beyond the group), dims c*32 + quad*8.
        U16x8 qb[4];
        // The query's B operand, loaded after the block ids (below). Lanes
        // beyond the group hold zeros (fused: set after its QK-norm + RoPE,
        // so that nothing ahead of the first K/V loads waits for the query).
        auto mask_q = [&]() {
            const bool has = col < a.group;
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int w = 0; w < 4; ++w) qb[c].w[w] = has ? qb[c].w[w] : 0u;
        };
        auto load_q = [&]() {
            const bool has = col < a.group;
            const int hq = h0 + (has ? col : 0);
            if constexpr (PARTS) {
                // Each 8-element piece: two 16-byte loads per slice, summed
                // in slice order and rounded once. Only the lanes of real
                // query heads load (exec-masked): 512 bytes per lane (4
                // slices x 8 pieces of 16 bytes) would otherwise go out from
                // every column.
                const float* qp = a.parts + row * a.pts + hq * D + quad * 8;
#pragma unroll
                for (int c = 0; c < 4; ++c) qb[c] = U16x8{};
                if (has)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float4 lo[kQkvParts], hi[kQkvParts];
#pragma unroll
                    for (int s = 0; s < kQkvParts; ++s) {
                        lo[s] = *reinterpret_cast<const float4*>(qp + s * a.pss + c * 32);
                        hi[s] = *reinterpret_cast<const float4*>(qp + s * a.pss + c * 32 + 4);
                    }
                    float4 l = lo[0], h = hi[0];
#pragma unroll
                    for (int s = 1; s < kQkvParts; ++s) {
                        l.x += lo[s].x; l.y += lo[s].y; l.z += lo[s].z; l.w += lo[s].w;
                        h.x += hi[s].x; h.y += hi[s].y; h.z += hi[s].z; h.w += hi[s].w;
                    }
                    qb[c].w[0] = pack2<T>(l.x, l.y);
                    qb[c].w[1] = pack2<T>(l.z, l.w);
                    qb[c].w[2] = pack2<T>(h.x, h.y);
                    qb[c].w[3] = pack2<T>(h.z, h.w);
                }
            } else {
                const T* qrow = a.q + row * a.qts + hq * a.qhs + quad * 8;
#pragma unroll
                for (int c = 0; c < 4; ++c) qb[c] = *reinterpret_cast<const U16x8*>(qrow + c * 32);
            }
            if constexpr (!FUSED) mask_q();
        };
        RopeIn rope_in;
        // The wave's range is walked in groups of 64 * IDR pages. Lane p
        // holds the block ids of pages p, p + 64, ... of the group in
        // registers (fetched once per group; only the low word: ids < 2^32,
        // as slots * heads * 16 fits in 32 bits, checked on the host), so
        // the chunk loop has no dependent id load in front of its K/V loads
        // - waiting for one would also wait for every V load issued before
        // it - and its body is one basic block, which keeps the compiler
        // from sinking the next chunk's loads down to their use.
        constexpr int IDR = 4;
        const uint32_t* const ids32 = reinterpret_cast<const uint32_t*>(a.blocks);
        const uint32_t ubs = uint32_t(bs);
        const int64_t group_tokens = int64_t(64 * IDR) * bs;
        int64_t g_begin = t_begin;
        int64_t g_end = min(t_end, g_begin + group_tokens);
        uint32_t g_page = 0;
        uint32_t gid[IDR];
        auto load_group = [&]() {
            g_page = uint32_t(g_begin / bs);
            const uint32_t last = uint32_t((g_end - 1) / bs);
#pragma unroll
            for (int r = 0; r < IDR; ++r)
                gid[r] = ids32[2 * (table + min(g_page + uint32_t(lane + 64 * r), last))];
        };
        // Lane x resolves the cache row (16-byte units) of chunk token t0 + x,
        // clamped to the group's last token so masked lanes read mapped
        // memory (past the group: the same cached row again).
        auto resolve = [&](int64_t t0) -> uint32_t {
            const uint32_t t = uint32_t(min(t0 + (lane % CH), g_end - 1));
            const uint32_t page = t / ubs;
            const uint32_t rel = page - g_page;
            uint32_t id = shfl_u32(gid[0], int(rel & 63u));
#pragma unroll
            for (int r = 1; r < IDR; ++r) {
                const uint32_t other = shfl_u32(gid[r], int(rel & 63u));
                id = (rel >> 6) == uint32_t(r) ? other : id;
            }
            const uint64_t slot = uint64_t(id) * ubs + (t - page * ubs);
            return static_cast<uint32_t>(slot * slot_units);
        };
        Unit kreg[NT][4];  // [tile][k-slice]: token 16*tile + col
        Unit vreg[NT][4];  // [tile][i]:       token 16*tile + 4*quad + i
        auto load_k = [&](uint32_t my_row) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                if constexpr (F8) {
                    // Whole 128-byte rows per instruction (8 tokens each):
                    // lane (col, quad) loads 16-byte chunk 2c + (quad >> 1),
                    // c = 2 (col >> 3) + (quad & 1), of token 16j + (col & 7)
                    // (kreg[j][0..1]) and of token 16j + 8 + (col & 7)
                    // (kreg[j][2..3]). A chunk is k-step c of quads
                    // 2 (quad >> 1) (low half) and 2 (quad >> 1) + 1 (high).
                    const uint32_t lo = shfl_u32(my_row, 16 * j + (col & 7));
                    const uint32_t hi = shfl_u32(my_row, 16 * j + 8 + (col & 7));
                    const uint32_t m = uint32_t(2 * (2 * (col >> 3) + (quad & 1)) + (quad >> 1));
                    const U16x8 x = load_stream(reinterpret_cast<const U16x8*>(kc + lo + 2 * m));
                    const U16x8 y = load_stream(reinterpret_cast<const U16x8*>(kc + hi + 2 * m));
                    kreg[j][0] = make_uint2(x.w[0], x.w[1]);
                    kreg[j][1] = make_uint2(x.w[2], x.w[3]);
                    kreg[j][2] = make_uint2(y.w[0], y.w[1]);
                    kreg[j][3] = make_uint2(y.w[2], y.w[3]);
                } else {
                    // Whole 128-byte lines per instruction: kreg[j][2l]
                    // holds line l of tokens 16j + (col & 7), kreg[j][2l+1]
                    // line l of tokens 16j + 8 + (col & 7); lane (col, quad)
                    // loads 16-byte unit (col >> 3) * 4 + quad of the line.
                    const uint32_t lo = shfl_u32(my_row, 16 * j + (col & 7));
                    const uint32_t hi = shfl_u32(my_row, 16 * j + 8 + (col & 7));
                    const uint32_t u = uint32_t((col >> 3) * 4 + quad);
#pragma unroll
                    for (int l = 0; l < 2; ++l) {
                        kreg[j][2 * l] = load_stream(kc + lo + 8 * l + u);
                        kreg[j][2 * l + 1] = load_stream(kc + hi + 8 * l + u);
                    }
                }
            }
        };
        // MFMA A operand of k-step c: lane (col, quad) = token 16j + col,
        // 16-byte unit 4c + quad. From the line loads: k-step 2l takes
        // kreg[j][2l] in lanes col < 8 and kreg[j][2l+1] rotated by 8 lanes
        // in lanes col >= 8; k-step 2l+1 the other way round (one DPP row
        // rotation and one select per word).
        // FP8: after the loads of tile j arrive, swap the high halves of even
        // quads with the low halves of odd quads (permlane16 swap), so that
        // kreg[j][0] / [1] hold k-steps 2 (col >> 3) and 2 (col >> 3) + 1 of
        // token 16j + (col & 7) for the lane's own quad ([2] / [3]: token
        // 16j + 8 + (col & 7)).
        auto swap_f8 = [&](int j) {
            if constexpr (F8) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    auto a0 = __builtin_amdgcn_permlane16_swap(kreg[j][2 * h].x,
                                                               kreg[j][2 * h + 1].x, false, false);
                    auto a1 = __builtin_amdgcn_permlane16_swap(kreg[j][2 * h].y,
                                                               kreg[j][2 * h + 1].y, false, false);
                    kreg[j][2 * h] = make_uint2(a0[0], a1[0]);
                    kreg[j][2 * h + 1] = make_uint2(a0[1], a1[1]);
                }
            }
        };
        auto k_operand = [&](int j, int c) -> U16x8 {
            if constexpr (F8) {
                // k-steps 0, 1: lanes col < 8 hold them for tokens 0-7, lanes
                // col >= 8 take tokens 8-15 from 8 lanes away; k-steps 2, 3
                // the other way round.
                const bool low = col < 8;
                const uint2 own = kreg[j][c];
                const uint2 other = c < 2 ? kreg[j][c + 2] : kreg[j][c - 2];
                const uint2 rot = make_uint2(
                    uint32_t(__builtin_amdgcn_update_dpp(0, int(other.x), 0x128, 0xf, 0xf, false)),
                    uint32_t(__builtin_amdgcn_update_dpp(0, int(other.y), 0x128, 0xf, 0xf, false)));
                const uint2 v = (c < 2) == low ? own : rot;
                return fp8x8_widen<T>(v);
            } else {
                const int l = c >> 1;
                const bool low = col < 8;
                const U16x8& x = kreg[j][2 * l];
                const U16x8& y = kreg[j][2 * l + 1];
                U16x8 o;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    if ((c & 1) == 0) {
                        const uint32_t yr = uint32_t(__builtin_amdgcn_update_dpp(
                            0, int(y.w[w]), 0x128, 0xf, 0xf, false));  // row_ror:8
                        o.w[w] = low ? x.w[w] : yr;
                    } else {
                        const uint32_t xr = uint32_t(__builtin_amdgcn_update_dpp(
                            0, int(x.w[w]), 0x128, 0xf, 0xf, false));
                        o.w[w] = low ? xr : y.w[w];
                    }
                }
                return o;
            }
        };
        auto load_v = [&](uint32_t my_row) {
#pragma unroll
            for (int j = 0; j < NT; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t vr = shfl_u32(my_row, 16 * j + 4 * quad + i);
                    vreg[j][i] = load_stream(vc + vr + col);
                }
        };

        // Software pipeline: the loads of chunk i+1 are issued as soon as the
        // registers of chunk i are consumed (K after Q.K^T, V after P.V), so
        // every wave keeps HBM requests in flight while it computes. The
        // last chunk of a group loads clamped (cached) rows instead of
        // branching, so the loop's wait counts never cover a skipped path.
        // Prologue order: the block ids first, then the query, its RoPE
        // inputs and (fused) the new token's raw K/V row. Vector loads
        // complete in issue order, so the wait for the ids - all the first
        // K/V loads need - does not include the rest. In a decode step the
        // query and the new row come from the qkv GEMM just written on other
        // XCDs and miss this XCD's cache: issued before the ids they held
        // the first K/V loads back (8B bs64 decode step 7.92 -> 7.85 ms).
        // The new row's loads are used only by the wave that writes it, so
        // the compiler issues them in that wave's branch.
        load_group();
        load_q();
        if constexpr (FUSED)
            rope_in = load_rope_in<T>(a.qw, a.cos_t + row * 64, a.sin_t + row * 64, quad);
        if constexpr (PARTS) {
            const float* prow = a.parts + row * a.pts;
            new_kv = load_new_kv_parts<T>(prow + (a.heads + kvh) * D,
                                          prow + (a.heads + a.kv_heads + kvh) * D, a.pss, a.kw,
                                          a.cos_t + row * 64, a.sin_t + row * 64, lane);
        } else if constexpr (FUSED) {
            new_kv = load_new_kv<T>(a.kraw + row * a.krts + kvh * a.krhs,
                                    a.vraw + row * a.vrts + kvh * a.vrhs, a.kw,
                                    a.cos_t + row * 64, a.sin_t + row * 64, lane);
        }
        if constexpr (FUSED) {
            // The row's new token (position length - 1) is written by the
            // wave whose page range holds it, before that wave reads it.
            if (t_begin <= length - 1 && length - 1 < t_end) {
                const int64_t slot = new_slot;
                if (slot >= 0) {
                    constexpr int EB = F8 ? 1 : int(sizeof(T));  // bytes per element
                    const int64_t off = (slot * a.css + int64_t(kvh) * a.chs) * EB;
                    write_new_kv<T, F8>(new_kv, a.k_eps,
                                        static_cast<char*>(a.kcache) + off,
                                        static_cast<char*>(a.vcache) + off, a.k_inv_scale,
                                        a.v_inv_scale, lane);
                    // Only this wave reads the row, and no CU has it cached
                    // (caches start clean per dispatch): a workgroup-scope
                    // release (store completion, no cache write-back) orders
                    // the stores before this wave's loads.
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                }
            }
        }

        {
            const uint32_t first = resolve(g_begin);
            load_k(first);
            load_v(first);
        }
        // The query's QK-norm + RoPE stays behind the first chunk's loads:
        // without this barrier the scheduler hoists it, and the waits for its
        // inputs, above them (0.5 us per launch at the 8B bs64 shape).
        if constexpr (FUSED) __builtin_amdgcn_sched_barrier(0);
        if constexpr (FUSED) {
            // QK-norm + RoPE of the raw query while the first K/V rows are in
            // flight, in the B-operand layout: lane (head col, quad) holds dims
            // c*32 + quad*8 + e; the RoPE pair of dim d < 64 is d + 64, two
            // k-slices up in the same lane.
            rope_query<T>(qb, rope_in, a.q_eps);
            mask_q();
        }
        // The first chunk's K words pass through an empty asm: otherwise the
        // compiler merges this load and the loop's load of the next chunk
        // into one load at the top of the loop body (a phi of two loads
        // becomes a load of a phi of addresses), which undoes the prefetch.
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                if constexpr (F8) {
                    asm volatile("" : "+v"(kreg[j][c].x));
                    asm volatile("" : "+v"(kreg[j][c].y));
                } else {
#pragma unroll
                    for (int w = 0; w < 4; ++w) asm volatile("" : "+v"(kreg[j][c].w[w]));
                }
            }
        for (;;) {
            for (int64_t t0 = g_begin; t0 < g_end; t0 += CH) {
                const uint32_t next = resolve(t0 + CH);

                // Scores: s[j][i] = token 16j + 4*quad + i, query head col.
                float s[NT][4];
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    swap_f8(j);
                    f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int c = 0; c < 4; ++c) d = mfma16x16x32<T>(k_operand(j, c), qb[c], d);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int64_t t = t0 + 16 * j + 4 * quad + i;
                        s[j][i] = t < g_end ? d[i] * a.scale_log2 : -INFINITY;
                    }
                }
                load_k(next);

                float cmax = -INFINITY;
#pragma unroll
                for (int j = 0; j < NT; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) cmax = fmaxf(cmax, s[j][i]);
                cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
                cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
                const float m_new = fmaxf(m_run, cmax);
                const float alpha = fast_exp2(m_run - m_new);
                m_run = m_new;

                float pw[NT][4];
                float psum = 0.f;
#pragma unroll
                for (int j = 0; j < NT; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float p = fast_exp2(s[j][i] - m_new);
                        psum += p;
                        pw[j][i] = p;
                    }
                l_run = l_run * alpha + psum;

                // Rescale: output row v of this lane is head 4*quad + v, whose
                // alpha lives in score lane (col = that head).
                if constexpr (GP > 1) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        if (4 * v >= 4 * GP) break;
                        const float av = __shfl(alpha, 4 * quad + v, 64);
#pragma unroll
                        for (int e = 0; e < 8; ++e) acc[e][v] *= av;
                    }
                } else {
                    const float av = read_lane<0>(alpha);
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[e] *= av;
                }

#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    uint2 pa, pl;  // A: this lane's head, tokens 4*quad + 0..3
                    pa.x = pack2<T>(pw[j][0], pw[j][1]);
                    pa.y = pack2<T>(pw[j][2], pw[j][3]);
                    pl.x = pack2<T>(pw[j][0] - half_lo<T>(pa.x), pw[j][1] - half_hi<T>(pa.x));
                    pl.y = pack2<T>(pw[j][2] - half_lo<T>(pa.y), pw[j][3] - half_hi<T>(pa.y));
                    U16x8 vr[4];  // the tile's V pieces as T elements
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if constexpr (F8) vr[i] = fp8x8_widen<T>(vreg[j][i]);
                        else vr[i] = vreg[j][i];
                    }
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
                        uint2 vb;  // B: element e of tokens 4*quad + 0..3
                        vb.x = __builtin_amdgcn_perm(vr[1].w[e >> 1], vr[0].w[e >> 1], sel);
                        vb.y = __builtin_amdgcn_perm(vr[3].w[e >> 1], vr[2].w[e >> 1], sel);
                        acc[e] = mfma16x16x16<T>(pa, vb, acc[e]);
                        acc[e] = mfma16x16x16<T>(pl, vb, acc[e]);
                    }
                }
                load_v(next);
            }
            if (g_end >= t_end) break;
            g_begin = g_end;
            g_end = min(t_end, g_begin + group_tokens);
            load_group();
            const uint32_t first = resolve(g_begin);
            load_k(first);
            load_v(first);
        }

    }  // t_begin < t_end

    // The denominator: sum the four 16-lane rows (disjoint token subsets).
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    // (m, l) of this lane's output heads 4*quad + v, from their score lanes.
    float mh[4], lh[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        mh[v] = __shfl(m_run, min(4 * quad + v, 15), 64);
        lh[v] = __shfl(l_run, min(4 * quad + v, 15), 64);
    }

    // Split merge through LDS: waves with split > 0 publish (o, m, l); the
    // split-0 wave of each head rescales and sums them:
    //   out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s,  M = max_s m_s.
    __shared__ float red_o[kMaxWaves - 1][GP][D];
    __shared__ float red_ml[kMaxWaves - 1][GP][2];
    if (a.splits > 1) {
        if (split > 0) {
            const int slot = local_head * (a.splits - 1) + split - 1;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int h = 4 * quad + v;
                if (h >= GP) break;
                float4* po = reinterpret_cast<float4*>(&red_o[slot][h][col * 8]);
                po[0] = make_float4(acc[0][v], acc[1][v], acc[2][v], acc[3][v]);
                po[1] = make_float4(acc[4][v], acc[5][v], acc[6][v], acc[7][v]);
                if (col == 0) {
                    red_ml[slot][h][0] = mh[v];
                    red_ml[slot][h][1] = lh[v];
                }
            }
        }
        __syncthreads();
        if (split > 0) return;
    }

#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int h = 4 * quad + v;
        if (h >= GP || h >= a.group) break;
        float mx = mh[v];
        for (int s = 1; s < a.splits; ++s)
            mx = fmaxf(mx, red_ml[local_head * (a.splits - 1) + s - 1][h][0]);
        float num[8];
        float den = 0.f;
        if (mx == -INFINITY) {
#pragma unroll
            for (int e = 0; e < 8; ++e) num[e] = 0.f;
        } else {
            const float w0 = fast_exp2(mh[v] - mx);
            den = w0 * lh[v];
#pragma unroll
            for (int e = 0; e < 8; ++e) num[e] = w0 * acc[e][v];
            for (int s = 1; s < a.splits; ++s) {
                const int slot = local_head * (a.splits - 1) + s - 1;
                const float ms = red_ml[slot][h][0];
                if (ms == -INFINITY) continue;
                const float ws = fast_exp2(ms - mx);
                den += ws * red_ml[slot][h][1];
                const float4* po = reinterpret_cast<const float4*>(&red_o[slot][h][col * 8]);
                const float4 p0 = po[0], p1 = po[1];
                num[0] += ws * p0.x; num[1] += ws * p0.y; num[2] += ws * p0.z; num[3] += ws * p0.w;
                num[4] += ws * p1.x; num[5] += ws * p1.y; num[6] += ws * p1.z; num[7] += ws * p1.w;
            }
        }
        if (a.grid_splits > 1) {
            // Unnormalised partial of this workgroup's page ranges.
            const int64_t base = (int64_t(r) * a.heads + h0 + h) * a.grid_splits + gsplit;
            float4* po = reinterpret_cast<float4*>(a.part_o + base * D + col * 8);
            po[0] = make_float4(num[0], num[1], num[2], num[3]);
            po[1] = make_float4(num[4], num[5], num[6], num[7]);
            if (col == 0) {
                a.part_ml[base * 2] = mx;
                a.part_ml[base * 2 + 1] = den;
            }
            continue;
        }
        if (mx == -INFINITY) den = 1.f;  // zero-length row: zeros
        U16x8 packed;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            packed.w[e] = pack2<T>(num[2 * e] * a.v_scale / den, num[2 * e + 1] * a.v_scale / den);
        *reinterpret_cast<U16x8*>(a.out + row * a.ots + (h0 + h) * a.ohs + col * 8) = packed;
    }
}

// Merge split partials: out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s.
// One wave per (row, query head) of the 128-dim fast path. Every load is
// issued before any result is needed: lane s holds split s's (max, sum)
// (splits <= 64), lane l the output dims 2l, 2l+1 of eight splits at a time;
// the maxima and sums reduce across the wave and each split's weight is
// broadcast from its lane.
template <typename T>
__global__ void __launch_bounds__(64)
paged_decode_merge(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                   T* __restrict__ out, const int64_t* __restrict__ rows,
                   int64_t ots, int64_t ohs, int heads, int splits, int head_dim,
                   float v_scale) {
    constexpr int D = 128, B = 8;  // head dim; splits loaded per batch
    const int id = blockIdx.x;
    const int r = id / heads;
    const int h = id - r * heads;
    const int lane = threadIdx.x;
    const int64_t base = (int64_t(r) * heads + h) * splits;
    (void)head_dim;
    const float* po = part_o + base * D + 2 * lane;
    float2 ov[B];
#pragma unroll
    for (int i = 0; i < B; ++i)
        ov[i] = i < splits ? *reinterpret_cast<const float2*>(po + int64_t(i) * D)
                           : make_float2(0.f, 0.f);
    float m = -INFINITY, l = 0.f;
    if (lane < splits) {
        const float2 ml = *reinterpret_cast<const float2*>(part_ml + (base + lane) * 2);
        m = ml.x;
        l = ml.y;
    }
    const int64_t row = rows[r];
    float mx = m;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    T* o = out + row * ots + h * ohs + 2 * lane;
    if (mx == -INFINITY) {  // zero-length row
        o[0] = static_cast<T>(0.f);
        o[1] = static_cast<T>(0.f);
        return;
    }
    const float w = m == -INFINITY ? 0.f : exp2f(m - mx);  // this lane's split
    float den = w * l;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) den += __shfl_xor(den, off, 64);
    float2 acc = make_float2(0.f, 0.f);
    for (int s0 = 0; s0 < splits; s0 += B) {
        if (s0 > 0) {
#pragma unroll
            for (int i = 0; i < B; ++i)
                ov[i] = s0 + i < splits
                            ? *reinterpret_cast<const float2*>(po + int64_t(s0 + i) * D)
                            : make_float2(0.f, 0.f);
        }
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const float ws = __shfl(w, s0 + i, 64);  // 0 past the last split
            acc.x += ws * ov[i].x;
            acc.y += ws * ov[i].y;
        }
    }
    const float scale = v_scale / den;
    o[0] = static_cast<T>(acc.x * scale);
    o[1] = static_cast<T>(acc.y * scale);
}



// Launch shape of the MFMA decode kernel. `target` is the number of
// (row, KV head, split) waves the split heuristic aims for (0 = the default
// rule in choose_splits); `tiles` 16-token MFMA tiles per iteration (4: one
// wave per SIMD with a 512-register budget, 32 KiB of K/V loads in flight per
// wave, workgroups of at most 4 waves; 2: two waves per SIMD, 16 KiB each);
// `waves` the preferred waves per workgroup. Measured on MI355X at Qwen3-8B
// bs64 ctx2048 with cold KV: 2 tiles 89 us, 4 tiles 94 us (since P.V moved
// to the matrix cores and freed vector registers).
struct Tuning {
    int64_t target = 0;
    int tiles = 0;  // 16-token tiles per iteration: 0 = 2 (16-bit cache) or 4 (FP8)
    int waves = 4;
    int split_waves = kMaxWaves;  // most page ranges of one head per workgroup
    bool overridden = false;      // set from the environment: no shape heuristics
};

// Defaults can be overridden for measurement with
// TVLLM_DECODE_TUNING="target,tiles,waves[,split_waves]" (read once per
// process).
const Tuning& tuning() {
    static const Tuning t = [] {
        Tuning v;
        if (const char* env = std::getenv("TVLLM_DECODE_TUNING")) {
            long long target = 0;
            int tiles = 0, waves = 0, split_waves = kMaxWaves;
            const int n = std::sscanf(env, "%lld,%d,%d,%d", &target, &tiles, &waves,
                                      &split_waves);
            if (n >= 3 && target >= 0 && (tiles == 2 || tiles == 4) && waves >= 1 &&
                waves <= kMaxWaves && split_waves >= 1 && split_waves <= kMaxWaves) {
                v.target = target;
                v.tiles = tiles;
                v.waves = waves;
                v.split_waves = split_waves;
                v.overridden = true;
            }
        }
        return v;
    }();
    return t;
}

// narrow: the kernel variant runs one 16-token tile per iteration (a 16-bit
// cache at GQA groups above 4, an FP8 cache above 8): half the bytes in
// flight per wave of the other variants, so it wants about twice the waves.
int64_t choose_splits(int64_t rows, int64_t kv_heads, bool narrow, int64_t max_context,
                      int64_t block_size) {
    const int64_t units = rows * kv_heads;
    if (units <= 0) return 1;
    // Page ranges per (row, KV head): enough waves to cover the 256 CUs, at
    // most one workgroup per CU (measured over 1-128 rows of the Qwen3-8B and
    // -32B shapes at 1500-3500 tokens). A tuning override sets the wave
    // target directly.
    int64_t s;
    if (tuning().target) {
        s = (tuning().target + units - 1) / units;
    } else if (units < 256) {
        // At most one workgroup per CU: units * grid <= 256 workgroups of
        // eight page ranges (grid a power of two), or, when not even two
        // fit per unit, one four-wave workgroup per unit (Qwen3-8B shape,
        // 2048 tokens: 12 rows 30 us with 16 ranges against 41 us with 22
        // (24); 20 / 24 / 28 rows 38 / 41 / 45 us with 4 against 54 / 56 /
        // 59 us with 13 / 11 / 10 (16)).
        // Narrow variants: one eight-wave workgroup per unit there (Qwen3-32B
        // shape, bf16, 24 rows x 2048 tokens: 43 us with 8 ranges against 52
        // us with 4).
        int64_t g = 1;
        while (units * g * 2 <= 256) g *= 2;
        s = g >= 2 || units * 2 <= 256 || narrow ? 8 * g : 4;
    } else {
        // One wave per SIMD at most, in whole four-wave workgroups: the
        // largest power of two with units * s <= 1024. Three ranges make
        // three-wave workgroups, and past 1024 waves some CUs take two
        // workgroups while others idle (Qwen3-8B shape, 2048 tokens: 40 / 48
        // / 56 rows 66 / 71 / 79 us with 2 ranges against 78 / 83 / 90 us
        // with 4 / 3 / 3; 72 / 80 / 96 rows 121 / 122 / 128 us with 1 against
        // 135 / 139 / 146 us with 2).
        // Narrow variants: two waves per SIMD, 2048 (Qwen3-32B shape, bf16, 48
        // rows x 2048 tokens: 80 us with 4 ranges against 93 us with 2; its
        // FP8 variant, 64 tokens per iteration, keeps 1024: 47 us with 2
        // against 55 us with 4).
        const int64_t waves = narrow ? 2048 : 1024;
        s = 1;
        while (units * s * 2 <= waves) s *= 2;
    }
    const int64_t max_pages = (max_context + block_size - 1) / block_size;
    // Each split should own at least one full 32-token iteration; at context
    // bounds up to 256 two, up to 512 four (short ranges' prologue and merge -
    // a second launch once the splits outgrow one workgroup - cost more than
    // the parallelism returns; Qwen3-0.6B decode steps at contexts 64 / 200
    // and 1-16 rows 4-6 % faster, e.g. 1 row x 64 tokens 1.407 -> 1.328 ms;
    // the decode launch at 300 / 500 tokens and 1-16 rows 9.2-13.9 us with 4
    // splits against 11.8-15.5 us with 16-32; at bounds past 512 the 32-token
    // ranges measured faster).
    const int64_t min_tokens = max_context <= 256 ? 64 : max_context <= 512 ? 128 : 32;
    const int64_t by_tokens = (max_context + min_tokens - 1) / min_tokens;
    s = std::min(s, std::min(max_pages, by_tokens));
    s = std::min<int64_t>(s, kMaxSplits);
    return std::max<int64_t>(s, 1);
}

// Splits of one (row, KV head): `waves` page ranges inside a workgroup
// (merged in LDS) times `grid` workgroups (merged by a second kernel).
struct SplitPlan {
    int64_t waves, grid;
    int heads;  // KV heads per workgroup
};

int heads_per_group(int64_t kv_heads, int64_t splits, int64_t waves);

SplitPlan plan_splits(int64_t rows, int64_t kv_heads, int64_t group, bool f8,
                      int64_t max_context, int64_t block_size) {
    const bool narrow = group > (f8 ? 8 : 4);
    const int64_t total = choose_splits(rows, kv_heads, narrow, max_context, block_size);
    int split_waves = tuning().split_waves, waves = tuning().waves;
    // Few (row, KV head) units with long page ranges per split (small batch,
    // long context): workgroups of two KV heads x four page ranges. The two
    // heads' waves read the two halves of the same 512-byte stretch of each
    // token's cache row at about the same time, which the DRAM serves better
    // than one head's 256-byte pieces alone (C5 decode shape, cold cache:
    // 276 -> 257 us). Short ranges keep one head per workgroup: the extra
    // grid-level partials would cost more than the locality gains. So do
    // plans past 128 units (one workgroup each): pairing heads there halves
    // the workgroups to far fewer than the CUs (20-28 rows of the Qwen3-8B
    // shape at a 4096 bound: 97-106 us against 59-71 us at 3500 tokens).
    if (!tuning().overridden && rows * kv_heads <= 128 && max_context >= 512 * total) {
        split_waves = 4;
        waves = 8;
    }
    SplitPlan p;
    p.waves = std::min<int64_t>(total, split_waves);
    // The merge launch holds one workgroup split per lane: at most 64, even
    // when a tuning override makes the page ranges per workgroup few.
    p.grid = std::min<int64_t>((total + p.waves - 1) / p.waves, kMaxGridSplits);
    p.heads = heads_per_group(kv_heads, p.waves, waves);
    return p;
}

// KV heads per workgroup: the largest power of two dividing kv_heads with
// heads * splits <= the preferred waves per workgroup.
int heads_per_group(int64_t kv_heads, int64_t splits, int64_t waves) {
    int h = 1;
    while (h * 2 * splits <= std::max<int64_t>(waves, splits) && kv_heads % (h * 2) == 0)
        h *= 2;
    return h;
}

// css / chs: the cache's slot and head strides (elements). 16-byte loads
// need them in whole 16-byte units (8 elements, 16 for FP8 bytes), and the
// kernel's 32-bit row offsets need every slot's offset below 2^32 units.
bool fast_path(int64_t head_dim, int64_t group, const void* q, int64_t qts,
               int64_t qhs, const void* out, int64_t ots, int64_t ohs,
               const void* k, const void* v, int64_t num_slots, int64_t css, int64_t chs,
               bool f8) {
    const int64_t unit = f8 ? 16 : 8;
    return head_dim == 128 && group <= 16 && aligned16(q) && qts % 8 == 0 &&
           qhs % 8 == 0 && aligned16(out) && ots % 8 == 0 && ohs % 8 == 0 &&
           aligned16(k) && aligned16(v) && css % unit == 0 && chs % unit == 0 &&
           num_slots * (css / 8) <= int64_t(UINT32_MAX);
}

}  // namespace
}  // namespace tvllm

using namespace tvllm;

extern "C" int64_t tvllm_paged_decode_split_plan(int64_t num_rows, int64_t num_heads,
                                                 int64_t num_kv_heads, int64_t head_dim,
                                                 int64_t max_context_len,
                                                 int64_t block_size) {
    if (num_rows <= 0 || num_kv_heads <= 0 || block_size <= 0 || max_context_len <= 0 ||
        num_heads % num_kv_heads != 0)
        return 0;
    if (head_dim != 128 || num_heads / num_kv_heads > 16) {
        // The general kernel: its workgroup-level split count, tagged.
        const GeneralSplits g = general_decode_splits(num_rows, num_heads, num_kv_heads,
                                                      head_dim, max_context_len);
        return (int64_t(1) << 32) | g.splits;
    }
    // The plan of a 16-bit cache (an FP8 cache's can differ where the grid
    // is 1: the id only groups context bounds into graphs).
    const SplitPlan p = plan_splits(num_rows, num_kv_heads, num_heads / num_kv_heads, false,
                                    max_context_len, block_size);
    return (p.waves << 16) | (p.grid << 8) | int64_t(p.heads);
}

extern "C" int64_t tvllm_paged_decode_workspace_size(int64_t num_rows,
                                                     int64_t num_heads,
                                                     int64_t num_kv_heads,
                                                     int64_t head_dim,
                                                     int64_t max_context_len,
                                                     int64_t block_size) {
    // Partials of the waves of one workgroup merge in LDS; only contexts
    // split over several workgroups (few rows, long contexts) need HBM
    // partials for a merge kernel. Other head dims and groups above 16 take
    // the general kernel; so do head-dim-128 calls with unaligned rows,
    // which is why those sizes cover both plans.
    if (num_rows <= 0 || num_kv_heads <= 0 || block_size <= 0 || max_context_len <= 0 ||
        num_heads % num_kv_heads != 0)
        return 0;
    const int64_t general = general_decode_workspace(num_rows, num_heads, num_kv_heads,
                                                     head_dim, max_context_len);
    if (head_dim != 128 || num_heads / num_kv_heads > 16) return general;
    int64_t mfma = 0;
    for (const bool f8 : {false, true}) {  // the cache dtype is not an argument: cover both
        const SplitPlan p = plan_splits(num_rows, num_kv_heads, num_heads / num_kv_heads, f8,
                                        max_context_len, block_size);
        if (p.grid > 1)
            mfma = std::max(mfma, num_rows * num_heads * p.grid * (head_dim + 2) *
                                      int64_t(sizeof(float)));
    }
    return std::max(mfma, general);
}

namespace tvllm {
namespace {

struct FusedIn {
    const void* k;
    int64_t kts, khs;
    const void* v;
    int64_t vts, vhs;
    const void* qw;
    const void* kw;
    const void* cos;
    const void* sin;
    float q_eps, k_eps;
    const int64_t* slots;
    const float* parts;  // split-K qkv partials (then k, v are unused)
    int64_t pss, pts;
};

int paged_decode_impl(
    const void* q, int64_t q_token_stride, int64_t q_head_stride,
    const void* k_cache, const void* v_cache, void* out, int64_t out_token_stride,
    int64_t out_head_stride, const int64_t* rows, const int64_t* blocks,
    const int64_t* offsets, const int64_t* lengths, int64_t num_rows,
    int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t num_slots,
    int64_t cache_slot_stride, int64_t cache_head_stride, int64_t block_size,
    int64_t max_context_len, float scale, void* workspace,
    int64_t workspace_bytes, int dtype, int cache_dtype, float k_scale, float v_scale,
    tvllm_stream_t stream, const FusedIn* fused) {
    TVLLM_CHECK(head_dim > 0 && head_dim <= 256 && num_heads > 0 && num_kv_heads > 0,
                "paged_decode: invalid attention head geometry");
    TVLLM_CHECK(num_heads % num_kv_heads == 0 && block_size > 0 &&
                    block_size <= INT32_MAX && num_slots % block_size == 0,
                "paged_decode: invalid GQA or block geometry");
    TVLLM_CHECK(num_rows >= 0 && num_rows <= INT32_MAX / num_heads,
                "paged_decode: decode grid is too large");
    TVLLM_CHECK(max_context_len > 0, "paged_decode: max_context_len must be positive");
    const bool f8 = cache_dtype == TVLLM_FP8_E4M3;
    TVLLM_CHECK(f8 || cache_dtype == dtype,
                "paged_decode: KV cache dtype must match the query dtype or be FP8 E4M3");
    TVLLM_CHECK(k_scale > 0.f && v_scale > 0.f && k_scale < INFINITY && v_scale < INFINITY,
                "paged_decode: KV scales must be positive and finite");
    TVLLM_CHECK(f8 || (k_scale == 1.f && v_scale == 1.f),
                "paged_decode: KV scales apply to an FP8 cache only");
    TVLLM_CHECK(cache_layout_ok(num_slots, num_kv_heads, head_dim, cache_slot_stride,
                                cache_head_stride),
                "paged_decode: cache strides must give non-overlapping head rows");
    if (num_rows == 0) return TVLLM_OK;
    TVLLM_CHECK(q && k_cache && v_cache && out && rows && blocks && offsets && lengths,
                "paged_decode: null pointer");
    const int64_t group = num_heads / num_kv_heads;
    hipStream_t s = as_hip(stream);
    const float scale_log2 = scale * kLog2e;

    return dispatch_half(dtype, [&]<int DT>() {
        using T = typename Elem<DT>::T;
        const bool fast = fast_path(head_dim, group, q, q_token_stride, q_head_stride, out,
                                    out_token_stride, out_head_stride, k_cache, v_cache,
                                    num_slots, cache_slot_stride, cache_head_stride, f8);
        TVLLM_CHECK(fused == nullptr || fast,
                    "paged_decode_qk_norm_rope: needs head_dim 128, group <= 16 and "
                    "16-byte aligned rows");
        if (!fast) {
            // Other head dims, GQA groups above 16 or unaligned rows: the
            // general kernel (a workgroup per row, KV head and group of up to
            // 16 query heads, and split of the keys when there are few of
            // those; fp32 arithmetic).
            GeneralAttention g{};
            g.q = q;
            g.qts = q_token_stride;
            g.qhs = q_head_stride;
            g.k = k_cache;
            g.v = v_cache;
            g.css = cache_slot_stride;
            g.chs = cache_head_stride;
            g.out = out;
            g.ots = out_token_stride;
            g.ohs = out_head_stride;
            g.rows = rows;
            g.q_offsets = nullptr;
            g.blocks = blocks;
            g.offsets = offsets;
            g.lengths = lengths;
            g.num_items = num_rows;
            g.max_query_len = 1;
            g.heads = int(num_heads);
            g.kv_heads = int(num_kv_heads);
            g.head_dim = int(head_dim);
            g.block_size = int(block_size);
            g.dtype = dtype;
            g.cache_dtype = cache_dtype;
            g.scale = scale;
            g.k_scale = k_scale;
            g.v_scale = v_scale;
            g.max_context = max_context_len;
            g.workspace = workspace;
            g.workspace_bytes = workspace_bytes;
            return launch_general_attention(g, s);
        }
        const SplitPlan plan =
            plan_splits(num_rows, num_kv_heads, group, f8, max_context_len, block_size);
        const int hpg = plan.heads;
        const int64_t grid = num_rows * (num_kv_heads / hpg) * plan.grid;
        TVLLM_CHECK(grid <= INT32_MAX, "paged_decode: decode grid is too large");
        TVLLM_CHECK(plan.grid <= kMaxGridSplits,
                    "paged_decode: at most 64 workgroup splits per row");
        const int threads = int(64 * hpg * plan.waves);
        const int64_t need = plan.grid > 1
            ? num_rows * num_heads * plan.grid * (head_dim + 2) * int64_t(sizeof(float))
            : 0;
        TVLLM_CHECK(workspace_bytes >= need && (need == 0 || workspace != nullptr),
                    "paged_decode: workspace of %lld bytes required, %lld given",
                    (long long)need, (long long)workspace_bytes);
        TVLLM_CHECK(need == 0 || aligned16(workspace),
                    "paged_decode: workspace must be 16-byte aligned");

        DecodeArgs<T> args;
        args.q = static_cast<const T*>(q);
        args.qts = q_token_stride;
        args.qhs = q_head_stride;
        args.k = k_cache;
        args.v = v_cache;
        args.css = cache_slot_stride;
        args.chs = cache_head_stride;
        args.out = static_cast<T*>(out);
        args.ots = out_token_stride;
        args.ohs = out_head_stride;
        args.rows = rows;
        args.blocks = blocks;
        args.offsets = offsets;
        args.lengths = lengths;
        args.heads = int(num_heads);
        args.kv_heads = int(num_kv_heads);
        args.group = int(group);
        args.block_size = int(block_size);
        args.splits = int(plan.waves);
        args.grid_splits = int(plan.grid);
        args.num_rows = int(num_rows);
        args.heads_per_wg = hpg;
        args.scale_log2 = scale_log2 * k_scale;
        args.v_scale = v_scale;
        args.k_inv_scale = 1.f / k_scale;
        args.v_inv_scale = 1.f / v_scale;
        args.part_o = static_cast<float*>(workspace);
        args.part_ml = need ? args.part_o + num_rows * num_heads * plan.grid * head_dim
                            : nullptr;
        args.kraw = nullptr;
        args.vraw = nullptr;
        args.slots = nullptr;
        args.parts = nullptr;
        if (fused) {
            args.kraw = static_cast<const T*>(fused->k);
            args.krts = fused->kts;
            args.krhs = fused->khs;
            args.vraw = static_cast<const T*>(fused->v);
            args.vrts = fused->vts;
            args.vrhs = fused->vhs;
            args.qw = static_cast<const T*>(fused->qw);
            args.kw = static_cast<const T*>(fused->kw);
            args.cos_t = static_cast<const T*>(fused->cos);
            args.sin_t = static_cast<const T*>(fused->sin);
            args.q_eps = fused->q_eps;
            args.k_eps = fused->k_eps;
            args.kcache = const_cast<void*>(k_cache);
            args.vcache = const_cast<void*>(v_cache);
            args.slots = fused->slots;
            args.parts = fused->parts;
            args.pss = fused->pss;
            args.pts = fused->pts;
        }

        // Four tiles per iteration (64 tokens, twice the bytes in flight)
        // pay for the FP8 layout, where a 16-byte load carries 16 tokens'
        // elements; bf16 at the 8B bs64 shape measured 87.6 -> 92.5 us with
        // them, FP8 53.3 -> 49.5 us.
        const bool tiles4 = tuning().tiles ? tuning().tiles == 4 : f8;
        auto launch = [&]<bool F, bool F8, bool P>() {
#define TVLLM_DEC(GP)                                                                \
    do {                                                                             \
        if (tiles4 && threads <= 256)                                                \
            paged_decode_d128<T, GP, 4, 4, F, F8, P><<<int(grid), threads, 0, s>>>(args); \
        else                                                                         \
            paged_decode_d128<T, GP, 2, kMaxWaves, F, F8, P>                         \
                <<<int(grid), threads, 0, s>>>(args);                                \
    } while (0)
            // Groups above 4 carry 64+ accumulator registers per lane. A bf16
            // cache keeps one 16-token tile per iteration there (two fit in
            // 227 VGPRs but measured slower: Qwen3-32B C5 shape 237.5 ->
            // 243 us); an FP8 tile is half the bytes, so FP8 takes four
            // tiles at group 8 (218 VGPRs; C5 shape 168.6 -> 138.7 us: one
            // tile left a wave with 2 KiB of K in flight) and two at 16.
            if (group <= 1) TVLLM_DEC(1);
            else if (group <= 2) TVLLM_DEC(2);
            else if (group <= 4) TVLLM_DEC(4);
            else if (group <= 8)
                paged_decode_d128<T, 8, F8 ? 4 : 1, kMaxWaves, F, F8, P>
                    <<<int(grid), threads, 0, s>>>(args);
            else
                paged_decode_d128<T, 16, F8 ? 2 : 1, kMaxWaves, F, F8, P>
                    <<<int(grid), threads, 0, s>>>(args);
        };
        const bool parts = fused && fused->parts;
        if (parts && f8) launch.template operator()<true, true, true>();
        else if (parts) launch.template operator()<true, false, true>();
        else if (fused && f8) launch.template operator()<true, true, false>();
        else if (fused) launch.template operator()<true, false, false>();
        else if (f8) launch.template operator()<false, true, false>();
        else launch.template operator()<false, false, false>();
#undef TVLLM_DEC
        const int st = launch_status("paged_decode");
        if (st != TVLLM_OK || plan.grid <= 1) return st;
        paged_decode_merge<T><<<int(num_rows * num_heads), 64, 0, s>>>(
            args.part_o, args.part_ml, static_cast<T*>(out), rows, out_token_stride,
            out_head_stride, int(num_heads), int(plan.grid), int(head_dim), v_scale);
        return launch_status("paged_decode merge");
    });
}

}  // namespace
}  // namespace tvllm

extern "C" int tvllm_paged_decode(
    const void* q, int64_t q_token_stride, int64_t q_head_stride,
    const void* k_cache, const void* v_cache, void* out, int64_t out_token_stride,
    int64_t out_head_stride, const int64_t* rows, const int64_t* blocks,
    const int64_t* offsets, const int64_t* lengths, int64_t num_rows,
    int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t num_slots,
    int64_t cache_slot_stride, int64_t cache_head_stride, int64_t block_size,
    int64_t max_context_len, float scale, void* workspace,
    int64_t workspace_bytes, int dtype, int cache_dtype, float k_scale, float v_scale,
    tvllm_stream_t stream) {
    return paged_decode_impl(q, q_token_stride, q_head_stride, k_cache, v_cache, out,
                             out_token_stride, out_head_stride, rows, blocks, offsets,
                             lengths, num_rows, num_heads, num_kv_heads, head_dim,
                             num_slots, cache_slot_stride, cache_head_stride, block_size,
                             max_context_len, scale, workspace,
                             workspace_bytes, dtype, cache_dtype, k_scale, v_scale, stream,
                             nullptr);
}

// ---------------------------------------------------------- no-alloc --
// tvllm_paged_decode_noalloc: the split-K partials live in this file-scope
// device array instead of a caller workspace. Each GPU holds its own copy;
// host code reaches it only through the address hipGetSymbolAddress returns
// for the current device, taken once per device on first use.
namespace tvllm {
namespace {

// The split planner asks for at most ~6 MB (520 bytes per (row, query head,
// workgroup split); its largest plan, 63 rows x 64 query heads x 3
// workgroup splits at group 16, is 12,096 of them); 8 MiB leaves room for
// other plans.
constexpr int64_t kScratchBytes = int64_t(8) << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Address of this device's scratch array (nullptr with the error set).
void* scratch_for_current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("paged_decode_noalloc: no current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || ptr == nullptr) {
            set_error("paged_decode_noalloc: hipGetSymbolAddress failed: %s",
                      hipGetErrorString(err));
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace tvllm

extern "C" int tvllm_paged_decode_noalloc(
    const void* q, int64_t q_token_stride, int64_t q_head_stride,
    const void* k_cache, const void* v_cache, void* out, int64_t out_token_stride,
    int64_t out_head_stride, const int64_t* rows, const int64_t* blocks,
    const int64_t* offsets, const int64_t* lengths, int64_t num_rows,
    int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t num_slots,
    int64_t cache_slot_stride, int64_t cache_head_stride, int64_t block_size,
    int64_t max_context_len, float scale, int dtype,
    int cache_dtype, float k_scale, float v_scale, tvllm_stream_t stream) {
    const int64_t need = tvllm_paged_decode_workspace_size(
        num_rows, num_heads, num_kv_heads, head_dim, max_context_len, block_size);
    TVLLM_CHECK(need <= kScratchBytes,
                "paged_decode_noalloc: this geometry needs %lld bytes of split-K "
                "workspace, above the %lld-byte static scratch; use tvllm_paged_decode",
                (long long)need, (long long)kScratchBytes);
    void* ws = nullptr;
    if (need > 0) {
        ws = scratch_for_current_device();
        if (ws == nullptr) return int(TVLLM_ELAUNCH);
    }
    // Every split workgroup writes its partials before the merge reads them,
    // so the scratch needs no clearing between calls.
    return paged_decode_impl(q, q_token_stride, q_head_stride, k_cache, v_cache, out,
                             out_token_stride, out_head_stride, rows, blocks, offsets,
                             lengths, num_rows, num_heads, num_kv_heads, head_dim,
                             num_slots, cache_slot_stride, cache_head_stride, block_size,
                             max_context_len, scale, ws,
                             need > 0 ? kScratchBytes : 0, dtype, cache_dtype, k_scale,
                             v_scale, stream, nullptr);
}

extern "C" int tvllm_paged_decode_qk_norm_rope(
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
    float k_scale, float v_scale, tvllm_stream_t stream) {
    TVLLM_CHECK(head_dim == 128, "paged_decode_qk_norm_rope: head_dim must be 128");
    TVLLM_CHECK(num_rows == 0 || (k && v && q_weight && k_weight && cos && sin && slots),
                "paged_decode_qk_norm_rope: null pointer");
    TVLLM_CHECK(aligned16(q_weight) && aligned16(cos) && aligned16(sin),
                "paged_decode_qk_norm_rope: weights and RoPE tables must be 16-byte aligned");
    const FusedIn f{k, k_token_stride, k_head_stride, v, v_token_stride, v_head_stride,
                    q_weight, k_weight, cos, sin, q_eps, k_eps, slots, nullptr, 0, 0};
    return paged_decode_impl(q, q_token_stride, q_head_stride, k_cache, v_cache, out,
                             out_token_stride, out_head_stride, rows, blocks, offsets,
                             lengths, num_rows, num_heads, num_kv_heads, head_dim,
                             num_slots, cache_slot_stride, cache_head_stride, block_size,
                             max_context_len, scale, workspace,
                             workspace_bytes, dtype, cache_dtype, k_scale, v_scale, stream,
                             &f);
}

extern "C" int tvllm_paged_decode_qk_norm_rope_partials(
    const float* parts, int64_t slice_stride, int64_t row_stride, const void* q_weight,
    const void* k_weight, const void* cos, const void* sin, float q_eps, float k_eps,
    const int64_t* slots, void* k_cache, void* v_cache, void* out, int64_t out_token_stride,
    int64_t out_head_stride, const int64_t* rows, const int64_t* blocks,
    const int64_t* offsets, const int64_t* lengths, int64_t num_rows, int64_t num_heads,
    int64_t num_kv_heads, int64_t head_dim, int64_t num_slots, int64_t cache_slot_stride,
    int64_t cache_head_stride, int64_t block_size, int64_t max_context_len, float scale,
    void* workspace, int64_t workspace_bytes, int dtype, int cache_dtype, float k_scale,
    float v_scale, tvllm_stream_t stream) {
    TVLLM_CHECK(head_dim == 128,
                "paged_decode_qk_norm_rope_partials: head_dim must be 128");
    TVLLM_CHECK(num_heads > 0 && num_kv_heads > 0 &&
                    row_stride >= (num_heads + 2 * num_kv_heads) * head_dim,
                "paged_decode_qk_norm_rope_partials: a row holds q, k and v heads");
    TVLLM_CHECK(slice_stride >= 0 && row_stride % 4 == 0 && slice_stride % 4 == 0,
                "paged_decode_qk_norm_rope_partials: strides must be whole float4 units");
    TVLLM_CHECK(num_rows == 0 || (parts && q_weight && k_weight && cos && sin && slots),
                "paged_decode_qk_norm_rope_partials: null pointer");
    TVLLM_CHECK(aligned16(parts) && aligned16(q_weight) && aligned16(cos) && aligned16(sin),
                "paged_decode_qk_norm_rope_partials: partials, weights and RoPE tables must "
                "be 16-byte aligned");
    const FusedIn f{nullptr, 0, 0, nullptr, 0, 0, q_weight, k_weight, cos, sin,
                    q_eps, k_eps, slots, parts, slice_stride, row_stride};
    // The query pointer only passes the host checks (the kernel reads parts).
    return paged_decode_impl(parts, 0, 0, k_cache, v_cache, out, out_token_stride,
                             out_head_stride, rows, blocks, offsets, lengths, num_rows,
                             num_heads, num_kv_heads, head_dim, num_slots, cache_slot_stride,
                             cache_head_stride, block_size, max_context_len, scale, workspace,
                             workspace_bytes, dtype, cache_dtype, k_scale, v_scale, stream, &f);
}

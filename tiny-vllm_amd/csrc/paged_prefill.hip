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
// head, tile of 32*W queries); each wave owns 32 queries. The products use
// the 32x32x16 MFMA, which issues twice the work per cycle of the 16x16x32
// form on gfx950.
//  * K/V tiles of 64 tokens are gathered through the block table into LDS
//    once per workgroup, double-buffered: tile i+2's global loads are in
//    flight and tile i+1 waits in registers while tile i is computed, so a
//    tile costs one barrier. Block ids are fetched a tile ahead of the K/V
//    loads that use them.
//  * S^T = K Q^T (A = 32 K rows from LDS, B = the wave's 32 queries held in
//    registers). A lane's score accumulator covers its own query and 16
//    tokens - exactly the k values the transposed product below needs, so P
//    never moves between lanes.
//  * O^T += V^T P^T (A = V^T from an LDS copy that staging stores transposed,
//    with the tokens of each 16-token step ordered the way the MFMA k index
//    visits them; B = the lane's probabilities) on fp16 MFMAs: P rounded to
//    fp16 keeps 11 bits (a bf16 P would leave ~1e-3 relative error in the
//    output, the whole bf16 tolerance), and a bf16 cache's V is converted to
//    fp16 as it is staged, which is exact below 65536. A V value beyond that
//    (or an infinity or NaN) becomes an fp16 infinity or NaN and makes the
//    outputs it reaches non-finite; a wave whose accumulators end
//    non-finite raises a guard, and a second launch recomputes the call on
//    bf16 MFMAs with P as a rounded value plus its rounded remainder (about
//    16 bits of P, two MFMAs per product).
//    The O^T accumulator of a lane belongs to its own query: the softmax
//    rescale and the final 1/l are lane-local.
//  * online softmax in base 2 (v_exp_f32) with one running (max, sum) per
//    query, raised lazily (kSlack) so most tiles skip the rescale; key tiles
//    past a wave's last query are skipped (causal) and tiles entirely below
//    its first query skip the mask.
// Work order: block ids are spread over the 8 XCDs so the workgroups of one
// (item, KV head) share an XCD's L2, and the causal tiles with the most keys
// start first.
#include "common.h"
#include "general_attention.h"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace tvllm {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// D[32x32] += A[32x16] B[16x32]. Lane l: A row l%32 and B column l%32 with
// k = 8*(l/32)..+7; D column l%32, rows 8*(v/4) + 4*(l/32) + v%4 for v < 16.
template <typename T>
__device__ __forceinline__ f32x16 mfma32(const U16x8& a, const U16x8& b, f32x16 c) {
    if constexpr (std::is_same_v<T, __bf16>) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(
            __builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    }
}

constexpr int D = 128;
constexpr int BK = 64;          // tokens per KV tile
constexpr int K_LD = D + 8;     // K tile row stride (elements): 68 dwords
constexpr int V_LD = BK + 8;    // V^T tile row stride (elements): 36 dwords
constexpr int K_TILE = BK * K_LD;
constexpr int V_TILE = D * V_LD;
constexpr float kLog2e = 1.4426950408889634f;

// V^T rows order each 16-token P.V step as the MFMA k index visits it:
// tile token 16s + 8jj + 4h + i sits at 16s + 8h + 4jj + i, so the eight k
// values of a lane in half h are one 16-byte read. First slot of quad tq:
__device__ __forceinline__ int vt_pos(int tq) {
    return 16 * (tq >> 2) + 8 * (tq & 1) + 4 * ((tq >> 1) & 1);
}

// Running maxima are only raised when a tile's maximum exceeds them by more
// than this (log2 units): probabilities then stay below 2^kSlack, and most
// tiles skip the rescale of the output accumulators.
constexpr float kSlack = 8.f;

// Workgroups of the exact fallback launch (each loops over tasks).
constexpr int64_t kExactWorkgroups = 32;

template <typename T>
struct PrefillArgs {
    const T* q;
    int64_t qts, qhs;
    const void* k;  // cache rows: T elements, or FP8 E4M3 bytes (F8 kernels)
    const void* v;
    int64_t css, chs;  // cache slot / head strides (elements)
    T* out;
    int64_t ots, ohs;
    const int64_t* q_offsets;
    const int64_t* blocks;
    const int64_t* block_offsets;
    const int64_t* context_lens;
    int heads, kv_heads, block_size, block_shift, q_tiles, grid;
    float scale_log2;  // softmax scale * log2(e) (* k_scale for an FP8 cache)
    float v_scale;     // FP8 cache: V dequantisation scale (1 otherwise)
    int* guard;        // bf16 cache: [recompute needed, exact-launch arrivals]
};

__device__ __forceinline__ float as_f(uint32_t x) { return __uint_as_float(x); }
__device__ __forceinline__ uint32_t as_u(float x) { return __float_as_uint(x); }

// Lanes l and l+32 hold the same query: combine them with one row swap.
__device__ __forceinline__ float pair_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(as_u(x), as_u(x), false, false);
    return fmaxf(as_f(r[0]), as_f(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(as_u(x), as_u(x), false, false);
    return as_f(r[0]) + as_f(r[1]);
}

// F8: K/V rows are FP8 E4M3 bytes; staging loads 8 bytes per 8-element
// piece and widens them exactly to T before the LDS store.
// EXACT: the bf16 fallback launch. It runs after the main launch on the same
// stream; its workgroups do nothing unless the main launch raised guard[0].
// Then every workgroup counts its arrival in guard[1] after reading guard[0];
// the last one clears both words, so the guard is zero between calls.
template <typename T, int W, bool QUAD, bool F8, bool EXACT>
__global__ void __launch_bounds__(64 * W, 8 / W)  // two waves per SIMD
paged_prefill_d128(PrefillArgs<T> a) {
    using SU = std::conditional_t<F8, uint2, U16x8>;  // one staged piece
    constexpr int EB = F8 ? 1 : int(sizeof(T));        // bytes per cached element
    constexpr int NTH = 64 * W;
    constexpr int BQ = 32 * W;           // queries per workgroup
    constexpr int JOBS = 2 * 16 * 16;    // (K|V) x 16 token quads x 16 pieces
    static_assert(JOBS % NTH == 0, "staging jobs must divide the threads");
    constexpr int JPT = JOBS / NTH;
    __shared__ __align__(16) uint16_t ks[2][K_TILE];
    __shared__ __align__(16) uint16_t vt[2][V_TILE];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int col = lane & 31;
    const int half = lane >> 5;

    if constexpr (EXACT) {
        __shared__ int redo;
        if (tid == 0) {
            const int raised = __hip_atomic_load(&a.guard[0], __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
            // A clear guard has nothing to reset: return without counting.
            // A raised one is seen by every workgroup (it is cleared only
            // after the last of them has read it and arrived).
            if (raised) {
                __threadfence();  // the read completes before the arrival is counted
                if (atomicAdd(&a.guard[1], 1) == int(gridDim.x) - 1) {  // the last arrival
                    __hip_atomic_store(&a.guard[1], 0, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&a.guard[0], 0, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            redo = raised;
        }
        __syncthreads();
        if (!redo) return;  // uniform
    }

    // One task = one (item, head, query tile). The main launch has a
    // workgroup per task; the exact launch, needed only for inputs beyond
    // fp16's range, loops a few workgroups over all tasks.
    auto task = [&](int bid) {
        // XCD-aware order: hardware deals block ids round-robin over 8 XCDs;
        // give each XCD a contiguous range of logical work.
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

        // This wave's queries: wq0 + col.
        const int64_t wq0 = q0 + int64_t(wave) * 32;
        const bool wave_active = wq0 < q_len;
        const int64_t wave_kv_end = min(kv_end, first_pos + min(q_len - 1, wq0 + 31) + 1);
        const int64_t wave_first_pos = first_pos + wq0;
        const int64_t qi_lane = min(wq0 + col, q_len - 1);
        const int64_t my_pos = first_pos + qi_lane;

        U16x8 qv[8];  // B operand of k-step c: dims 16c + 8*half .. +7
        {
            const T* qrow = a.q + (q_begin + qi_lane) * a.qts + h * a.qhs + 8 * half;
    #pragma unroll
            for (int c = 0; c < 8; ++c) qv[c] = *reinterpret_cast<const U16x8*>(qrow + 16 * c);
        }

        // A bf16 cache's V is converted to fp16 while it is staged. A finite
        // bf16 value below 65536 in magnitude converts exactly (or, below
        // 2^-14, to within 2^-25); a larger, infinite or NaN one becomes an
        // fp16 infinity or NaN, and then so does every output it reaches
        // (p * inf, 0 * inf = NaN; with p <= 2^kSlack and |v| < 65536 the
        // fp32 sums stay finite otherwise). So a wave whose accumulators end
        // non-finite raises the guard, and the exact launch redoes the call.
        constexpr bool kConvertV = std::is_same_v<T, __bf16> && !F8 && !EXACT;

        const int bs = a.block_size;
        // Staging: job = (K|V, piece, token quad); 4 tokens x 16 bytes each.
        auto job_coords = [&](int r, bool& is_v, int& tq, int& piece) {
            const int job = tid + r * NTH;
            is_v = job >> 8;
            // K: piece fastest (a token row per 16 lanes, conflict-free 16-byte
            // LDS writes); V: token quad fastest (conflict-free transposed writes).
            tq = is_v ? (job & 15) : ((job >> 4) & 15);
            piece = is_v ? ((job >> 4) & 15) : (job & 15);
        };
        // Token positions fit in 32 bits (contexts < 2^31), slots and the
        // slot stride in bytes too (checked on the host); the byte offset of a
        // slot is formed in 64 bits.
        const int end1 = int(kv_end) - 1;
        const uint32_t slot_elems = uint32_t(a.css);
        const int64_t head_elems = int64_t(kvh) * a.chs;
        // QUAD (power-of-two pages of >= 4 tokens): a job's 4 tokens share a
        // page, so one block id serves all four. A template parameter, not a
        // branch: two load paths in the loop would make the wait-count pass
        // treat the prefetch registers as possibly pending and stall on them.
        constexpr bool quad_pages = QUAD;
        // Staging is branch-free: tiles past the end (or before the start, in the
        // prologue) load clamped, valid rows and store them into a buffer nobody
        // reads again, so every load is consumed on every path and the wait-count
        // pass never has to assume a prefetch register is still in flight.
        // Staging runs ahead of the math: at iteration i the K rows of tile i+1
        // (for S(i+1)) and the V rows of tile i (for P.V) are in LDS, and this
        // iteration writes K(i+2) and V(i+1) from registers loaded during the
        // previous one. `lead` is that distance for the job's kind.
        auto lead_of = [](bool is_v) { return is_v ? 1 : 2; };
        auto load_ids = [&](int tile_base, uint32_t (&ids)[JPT][4]) {
    #pragma unroll
            for (int r = 0; r < JPT; ++r) {
                bool is_v;
                int tq, piece;
                job_coords(r, is_v, tq, piece);
                const int t0 = max(tile_base + lead_of(is_v), 0) * BK;
                if constexpr (quad_pages) {
                    ids[r][0] = uint32_t(a.blocks[table + (min(t0 + 4 * tq, end1) >> a.block_shift)]);
                } else {
    #pragma unroll
                    for (int e = 0; e < 4; ++e)
                        ids[r][e] = uint32_t(a.blocks[table + min(t0 + 4 * tq + e, end1) / bs]);
                }
            }
        };
        auto load_tile = [&](int tile_base, const uint32_t (&ids)[JPT][4], SU (&stage)[JPT][4]) {
    #pragma unroll
            for (int r = 0; r < JPT; ++r) {
                bool is_v;
                int tq, piece;
                job_coords(r, is_v, tq, piece);
                const int t0 = max(tile_base + lead_of(is_v), 0) * BK;
                const char* src = static_cast<const char*>(is_v ? a.v : a.k) +
                                  (head_elems + piece * 8) * EB;
                const uint32_t row_bytes = slot_elems * EB;
                if constexpr (quad_pages) {
                    // The quad's tokens are consecutive slots of one page:
                    // token min(tb + e, end1) is row min(e, d) past the first.
                    const int tb = t0 + 4 * tq;
                    const int tc = min(tb, end1);
                    const uint32_t d = uint32_t(end1 - tc);
                    const char* p0 = src + uint64_t(ids[r][0] * uint32_t(bs) +
                                                    uint32_t(tc & (bs - 1))) * row_bytes;
    #pragma unroll
                    for (int e = 0; e < 4; ++e)
                        stage[r][e] = *reinterpret_cast<const SU*>(
                            p0 + uint64_t(min(uint32_t(e), d)) * row_bytes);
                } else {
    #pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int t = min(t0 + 4 * tq + e, end1);
                        const uint32_t slot = ids[r][e] * uint32_t(bs) + uint32_t(t % bs);
                        stage[r][e] = *reinterpret_cast<const SU*>(src + uint64_t(slot) * row_bytes);
                    }
                }
            }
        };
        // EXACT: V^T staged as the cache's own bf16 values; otherwise as fp16.
        auto store_tile = [&](int tile_base, const SU (&raw)[JPT][4]) {
            constexpr bool convert = kConvertV;
    #pragma unroll
            for (int r = 0; r < JPT; ++r) {
                bool is_v;
                int tq, piece;
                job_coords(r, is_v, tq, piece);
                const int buf = (tile_base + lead_of(is_v)) & 1;
                U16x8 pc[4];  // the job's four token pieces, as staged
    #pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if constexpr (F8) {
                        pc[e] = is_v ? fp8x8_widen<_Float16>(raw[r][e]) : fp8x8_widen<T>(raw[r][e]);
                    } else {
                        pc[e] = raw[r][e];
                    }
                }
                if (convert && is_v) {
                    // V^T in fp16: each conversion takes one dim of two tokens,
                    // so its result is already the transposed (token, token)
                    // word (bf16 -> f32 is a shift or a mask of the raw word).
    #pragma unroll
                    for (int dd = 0; dd < 8; ++dd) {
                        auto f = [&](int e) {
                            const uint32_t b = pc[e].w[dd >> 1];
                            return (dd & 1) ? half_hi<T>(b) : half_lo<T>(b);
                        };
                        uint2 w;
                        w.x = pack2<_Float16>(f(0), f(1));
                        w.y = pack2<_Float16>(f(2), f(3));
                        *reinterpret_cast<uint2*>(&vt[buf][(piece * 8 + dd) * V_LD + vt_pos(tq)]) = w;
                    }
                } else if (is_v) {
                    // V^T: dim row (piece*8 + dd), the quad's 4 tokens -> one 8-byte write;
                    // v_perm picks the low (even dd) or high (odd dd) halves of two words.
    #pragma unroll
                    for (int dd = 0; dd < 8; ++dd) {
                        const uint32_t sel = (dd & 1) ? 0x07060302u : 0x05040100u;
                        uint2 w;
                        w.x = __builtin_amdgcn_perm(pc[1].w[dd >> 1], pc[0].w[dd >> 1], sel);
                        w.y = __builtin_amdgcn_perm(pc[3].w[dd >> 1], pc[2].w[dd >> 1], sel);
                        *reinterpret_cast<uint2*>(&vt[buf][(piece * 8 + dd) * V_LD + vt_pos(tq)]) = w;
                    }
                } else {
    #pragma unroll
                    for (int e = 0; e < 4; ++e)
                        *reinterpret_cast<U16x8*>(&ks[buf][(4 * tq + e) * K_LD + piece * 8]) =
                            pc[e];
                }
            }
        };

        const int ntiles = int((kv_end + BK - 1) / BK);
        const int wt = wave_active ? int((wave_kv_end + BK - 1) / BK) : 0;  // this wave's tiles
        // Ping-pong: waves 0..W/2-1 ("matrix first") and W/2..W-1 ("vector
        // first") pair up on each SIMD. Every tile is split in two halves at a
        // barrier; in each half one wave of a pair issues MFMAs (P.V of tile i
        // and S of tile i+1) while the other runs exponentials, so the matrix
        // cores and the vector ALUs work at the same time.
        const bool matrix_first = wave < W / 2;
        // With eight waves, waves 0-3 own the K staging jobs and waves 4-7 the V
        // jobs; each group stages in the half where it issues MFMAs, so staging
        // runs alongside the other group's exponentials instead of in a phase of
        // its own. K(i+2) goes to the buffer of K(i), V(i+1) to that of V(i-1):
        // both were last read before the previous barrier, and neither buffer is
        // read in the half that writes it.
        constexpr bool split_staging = W == 8;

        f32x16 o[4];  // O^T: lane = (dims 32n + 8g + 4*half + i, query col)
        float m_run, l_run;

        // The pass over the key tiles. EXACT: P.V on bf16 MFMAs with P as the
        // rounded value plus the rounded remainder (about 16 bits of P), V as
        // cached. Otherwise P.V on fp16 MFMAs: P rounded to fp16 (11 bits; a
        // single bf16 P would leave ~1e-3 relative error, the whole tolerance)
        // and V converted to fp16 (exact for a bf16 or FP8 cache in range).
        {
            using PV = std::conditional_t<EXACT, T, _Float16>;
    #pragma unroll
            for (int n = 0; n < 4; ++n) o[n] = f32x16{};
            m_run = -INFINITY;
            l_run = 0.f;

            // ---- per-wave math on one tile j ----------------------------------
            f32x16 sc[2];  // raw S^T of the tile: sc[tb][v] = token 32tb + 8(v/4) + 4*half + v%4
            U16x8 pb[4];   // P of the tile, k-step st: token 16st + 8jj + 4*half + i at k = 4jj + i
            U16x8 pr[4];   // EXACT: P - pb (the rounding remainder), same layout
            // LDS operands are read ahead of the MFMAs that use them (K two
            // k-steps ahead, V one 16-token step ahead), so a read's latency
            // hides behind the matrix instructions already issued.
            auto scores = [&](int j) {
                const uint16_t* kt = ks[j & 1];
                sc[0] = f32x16{};
                sc[1] = f32x16{};
                constexpr int KB = EXACT ? 1 : 3;  // k-steps read ahead (fewer in the rare exact pass)
                U16x8 kk[KB][2];
                auto load_k = [&](int c, U16x8 (&dst)[2]) {
    #pragma unroll
                    for (int tb = 0; tb < 2; ++tb)
                        dst[tb] = *reinterpret_cast<const U16x8*>(
                            &kt[(32 * tb + col) * K_LD + 16 * c + 8 * half]);
                };
    #pragma unroll
                for (int c = 0; c < KB - 1; ++c) load_k(c, kk[c]);
    #pragma unroll
                for (int c = 0; c < 8; ++c) {
                    if (c + KB - 1 < 8) load_k(c + KB - 1, kk[(c + KB - 1) % KB]);
    #pragma unroll
                    for (int tb = 0; tb < 2; ++tb) sc[tb] = mfma32<T>(kk[c % KB][tb], qv[c], sc[tb]);
                }
            };
            auto softmax = [&](int j) {
                const int64_t t0 = int64_t(j) * BK;
                if (t0 + BK - 1 > wave_first_pos) {  // tile crosses the diagonal
                    // Keys past this lane's query: offset within the tile > lim.
                    const int lim = int(my_pos - t0) - 4 * half;
    #pragma unroll
                    for (int tb = 0; tb < 2; ++tb)
    #pragma unroll
                        for (int v = 0; v < 16; ++v)
                            if (32 * tb + 8 * (v >> 2) + (v & 3) > lim) sc[tb][v] = -INFINITY;
                }
                // Maxima and sums in four independent chains (a single chain of 32
                // dependent instructions stalls the wave).
                float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    #pragma unroll
                for (int tb = 0; tb < 2; ++tb)
    #pragma unroll
                    for (int v = 0; v < 16; ++v) mx[v & 3] = fmaxf(mx[v & 3], sc[tb][v]);
                const float cmax = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
                const float cm = pair_max(cmax) * a.scale_log2;  // scale > 0
                const bool grow = cm > m_run + kSlack;  // also: first finite max
                float alpha = 1.f;
                if (grow) {
                    alpha = __builtin_amdgcn_exp2f(m_run - cm);
                    m_run = cm;
                }
                if (__builtin_amdgcn_ballot_w64(grow)) {  // wave-uniform
                    l_run *= alpha;
    #pragma unroll
                    for (int n = 0; n < 4; ++n) o[n] *= alpha;
                }
                const float m_use = m_run == -INFINITY ? 0.f : m_run;
                float ps[4] = {0.f, 0.f, 0.f, 0.f};
    #pragma unroll
                for (int tb = 0; tb < 2; ++tb) {
                    float p[16];
    #pragma unroll
                    for (int v = 0; v < 16; ++v)
                        p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[tb][v], a.scale_log2, -m_use));
    #pragma unroll
                    for (int sh = 0; sh < 2; ++sh)
    #pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float p0 = p[8 * sh + 2 * e], p1 = p[8 * sh + 2 * e + 1];
                            const uint32_t hw = pack2<PV>(p0, p1);
                            pb[2 * tb + sh].w[e] = hw;
                            if constexpr (EXACT) {
                                pr[2 * tb + sh].w[e] =
                                    pack2<PV>(p0 - half_lo<PV>(hw), p1 - half_hi<PV>(hw));
                                ps[e] += p0 + p1;
                            } else {
                                // The denominator sums the fp16 weights P.V uses.
                                typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
                                const h2_t ones = {1.f16, 1.f16};
                                ps[e] = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, hw), ones,
                                                               ps[e], false);
                            }
                        }
                }
                l_run += (ps[0] + ps[1]) + (ps[2] + ps[3]);
            };
            auto pv = [&](int j) {  // O^T += V^T P^T over four 16-token steps
                const uint16_t* vtt = vt[j & 1];
                constexpr int VB = EXACT ? 1 : 2;
                U16x8 va[VB][4];
                auto load_v = [&](int st, U16x8 (&dst)[4]) {
    #pragma unroll
                    for (int n = 0; n < 4; ++n)
                        dst[n] = *reinterpret_cast<const U16x8*>(
                            &vtt[(32 * n + col) * V_LD + 16 * st + 8 * half]);
                };
                if constexpr (VB > 1) load_v(0, va[0]);
    #pragma unroll
                for (int st = 0; st < 4; ++st) {
                    if constexpr (VB > 1) {
                        if (st + 1 < 4) load_v(st + 1, va[(st + 1) % VB]);
                    } else {
                        load_v(st, va[0]);
                    }
                    if constexpr (EXACT) {  // remainders first: four accumulators apart
    #pragma unroll
                        for (int n = 0; n < 4; ++n) o[n] = mfma32<PV>(va[st % VB][n], pr[st], o[n]);
                    }
    #pragma unroll
                    for (int n = 0; n < 4; ++n) o[n] = mfma32<PV>(va[st % VB][n], pb[st], o[n]);
                }
            };

            // Prologue: K(0), K(1), V(0) into LDS, and K(2), V(1) into registers,
            // with the three tiles' block ids and rows fetched concurrently. (The
            // first staging call also writes V(0) into the spare V buffer.)
            SU stage[JPT][4];
            uint32_t ids[JPT][4];
            {
                SU st0[JPT][4], st1[JPT][4];
                uint32_t id0[JPT][4], id1[JPT][4];
                load_ids(-2, id0);
                load_ids(-1, id1);
                load_ids(0, ids);
                load_tile(-2, id0, st0);
                load_tile(-1, id1, st1);
                load_tile(0, ids, stage);
                load_ids(1, ids);
                store_tile(-2, st0);
                store_tile(-1, st1);
            }
            __syncthreads();
            if (wt > 0) {
                scores(0);
                if (matrix_first) softmax(0);
            }
            auto stage_next = [&](int i) {
                store_tile(i, stage);
                load_tile(i + 1, ids, stage);
                load_ids(i + 2, ids);
            };
            // K(2) overwrites K(0), which every wave read above in scores(0).
            if constexpr (split_staging) __syncthreads();
            // A wave's MFMA half with its staging in one basic block (the common
            // case i + 1 < wt), so the scheduler can slot the staging instructions
            // between the matrix instructions.
            auto matrix_half = [&](int i) {
                if (i + 1 < wt) {
                    pv(i);
                    scores(i + 1);
                    if constexpr (split_staging) stage_next(i);
                } else if (i < wt) {
                    pv(i);
                    if constexpr (split_staging) stage_next(i);
                } else if constexpr (split_staging) {
                    stage_next(i);
                }
            };
            for (int i = 0; i < ntiles; ++i) {
                // First half: tile i's P.V and tile i+1's S (matrix first), or
                // tile i's softmax (vector first).
                if (matrix_first) matrix_half(i);
                else if (i < wt) softmax(i);
                __syncthreads();
                // Second half: the roles swap.
                if (matrix_first) {
                    if (i + 1 < wt) softmax(i + 1);
                } else {
                    matrix_half(i);
                }
                if constexpr (!split_staging) stage_next(i);
                __syncthreads();
            }
        }

        if constexpr (kConvertV) {
            float total = 0.f;  // inf or NaN if any accumulator is
    #pragma unroll
            for (int n = 0; n < 4; ++n)
    #pragma unroll
                for (int v = 0; v < 16; ++v) total += o[n][v];
            if (__builtin_amdgcn_ballot_w64(!(__builtin_fabsf(total) < INFINITY))) {
                if (lane == 0) a.guard[0] = 1;  // the EXACT launch redoes this call
                return;
            }
        }
        if (!wave_active) return;

        const float l = pair_sum(l_run);
        const int64_t qi = wq0 + col;
        if (qi >= q_len) return;
        const float inv = a.v_scale / l;
        T* orow = a.out + (q_begin + qi) * a.ots + h * a.ohs + 4 * half;
    #pragma unroll
        for (int n = 0; n < 4; ++n)
    #pragma unroll
            for (int g = 0; g < 4; ++g) {
                uint2 w;
                w.x = pack2<T>(o[n][4 * g + 0] * inv, o[n][4 * g + 1] * inv);
                w.y = pack2<T>(o[n][4 * g + 2] * inv, o[n][4 * g + 3] * inv);
                *reinterpret_cast<uint2*>(orow + 32 * n + 8 * g) = w;
            }
    };
    if constexpr (EXACT) {
        for (int t = blockIdx.x; t < a.grid; t += gridDim.x) {
            __syncthreads();  // the previous task's LDS reads are done
            task(t);
        }
    } else {
        task(blockIdx.x);
    }
}

}  // namespace
}  // namespace tvllm

using namespace tvllm;

extern "C" int64_t tvllm_paged_prefill_workspace_size(int dtype, int cache_dtype) {
    // The fallback guard (two ints) of a bf16 cache, whose V is converted to
    // fp16 for the P.V products.
    return dtype == TVLLM_BF16 && cache_dtype == TVLLM_BF16 ? 2 * int64_t(sizeof(int)) : 0;
}

extern "C" int tvllm_paged_prefill(
    const void* q, int64_t q_token_stride, int64_t q_head_stride,
    const void* k_cache, const void* v_cache, void* out, int64_t out_token_stride,
    int64_t out_head_stride, const int64_t* q_offsets, const int64_t* blocks,
    const int64_t* block_offsets, const int64_t* context_lens, int64_t num_items,
    int64_t max_query_len, int64_t num_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t num_slots, int64_t cache_slot_stride,
    int64_t cache_head_stride, int64_t block_size, float scale,
    void* workspace, int64_t workspace_bytes,
    int dtype, int cache_dtype, float k_scale, float v_scale, tvllm_stream_t stream) {
    TVLLM_CHECK(head_dim > 0 && head_dim <= 256, "paged_prefill: head_dim must be in 1..256");
    const bool f8 = cache_dtype == TVLLM_FP8_E4M3;
    TVLLM_CHECK(f8 || cache_dtype == dtype,
                "paged_prefill: KV cache dtype must match Q or be FP8 E4M3");
    TVLLM_CHECK(k_scale > 0.f && v_scale > 0.f && k_scale < INFINITY && v_scale < INFINITY,
                "paged_prefill: KV scales must be positive and finite");
    TVLLM_CHECK(f8 || (k_scale == 1.f && v_scale == 1.f),
                "paged_prefill: KV scales apply to an FP8 cache only");
    TVLLM_CHECK(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
                "paged_prefill: invalid GQA geometry");
    TVLLM_CHECK(block_size > 0 && num_slots % block_size == 0,
                "paged_prefill: invalid block geometry");
    TVLLM_CHECK(num_slots <= INT32_MAX, "paged_prefill: at most 2^31-1 cache slots");
    TVLLM_CHECK(cache_layout_ok(num_slots, num_kv_heads, head_dim, cache_slot_stride,
                                cache_head_stride),
                "paged_prefill: cache strides must give non-overlapping head rows");
    TVLLM_CHECK(num_items >= 0 && max_query_len >= 0,
                "paged_prefill: negative sizes");
    TVLLM_CHECK(scale > 0.f && scale < INFINITY, "paged_prefill: scale must be positive");
    const int64_t need = tvllm_paged_prefill_workspace_size(dtype, cache_dtype);
    TVLLM_CHECK(workspace_bytes >= need && (need == 0 || workspace != nullptr),
                "paged_prefill: workspace of %lld bytes required, %lld given",
                (long long)need, (long long)workspace_bytes);
    TVLLM_CHECK(need == 0 || (reinterpret_cast<uintptr_t>(workspace) & 3) == 0,
                "paged_prefill: workspace must be 4-byte aligned");
    if (num_items == 0 || max_query_len == 0) return TVLLM_OK;
    TVLLM_CHECK(q && k_cache && v_cache && out && q_offsets && blocks &&
                    block_offsets && context_lens,
                "paged_prefill: null pointer");
    if (head_dim != 128) {
        // Other head dims: the general kernel (one wave per query token, KV
        // head and group of up to 16 query heads; fp32 arithmetic, so no
        // fallback guard is raised).
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
        g.rows = nullptr;
        g.q_offsets = q_offsets;
        g.blocks = blocks;
        g.offsets = block_offsets;
        g.lengths = context_lens;
        g.num_items = num_items;
        g.max_query_len = max_query_len;
        g.heads = int(num_heads);
        g.kv_heads = int(num_kv_heads);
        g.head_dim = int(head_dim);
        g.block_size = int(block_size);
        g.dtype = dtype;
        g.cache_dtype = cache_dtype;
        g.scale = scale;
        g.k_scale = k_scale;
        g.v_scale = v_scale;
        return launch_general_attention(g, as_hip(stream));
    }
    TVLLM_CHECK(cache_slot_stride % 8 == 0 && cache_head_stride % 8 == 0 &&
                    cache_slot_stride * (f8 ? 1 : 2) <= int64_t(UINT32_MAX),
                "paged_prefill: cache strides must be whole 8-element units "
                "(slot stride below 2^32 bytes)");
    TVLLM_CHECK(aligned16(q) && q_token_stride % 8 == 0 && q_head_stride % 8 == 0 &&
                    aligned16(k_cache) && aligned16(v_cache),
                "paged_prefill: Q and caches must be 16-byte aligned rows");
    TVLLM_CHECK(out_token_stride % 4 == 0 && out_head_stride % 4 == 0 && aligned8(out),
                "paged_prefill: output rows must be 8-byte aligned");
    // 32 queries per wave. Eight waves per workgroup (two per SIMD) keep the
    // MFMA pipes fed while the other wave runs its softmax. Chunks of at most
    // 128 queries use four-wave workgroups when there are enough of them to
    // put two on every CU (512); with fewer, a CU would hold four waves and
    // the eight-wave kernel is faster even with half its waves idle (3 x 100
    // queries at 20k keys, 64 heads: 696 vs 1052 us; 8 x 64 queries at 24.5k:
    // 1146 vs 1026 us).
    const int64_t grid4 = num_items * num_heads * ((max_query_len + 127) / 128);
    int waves = max_query_len > 128 || grid4 < 512 ? 8 : 4;
    if (const char* env = std::getenv("TVLLM_PREFILL_TUNING")) {
        const int ew = std::atoi(env);  // measurement override: 4 or 8 waves
        if (ew == 4 || ew == 8) waves = ew;
    }
    const int64_t bq = 32 * waves;
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
        args.k = k_cache;
        args.v = v_cache;
        args.css = cache_slot_stride;
        args.chs = cache_head_stride;
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
        args.scale_log2 = scale * kLog2e * k_scale;
        args.v_scale = v_scale;
        args.guard = static_cast<int*>(workspace);
        args.block_shift = (block_size & (block_size - 1)) == 0
                               ? __builtin_ctzll(uint64_t(block_size)) : -1;
        const bool quad = args.block_shift >= 2;
        auto go = [&]<bool F8, bool EXACT>() {
            // The exact launch: few workgroups (few arrivals on the guard).
            const int g = EXACT ? int(std::min<int64_t>(grid, kExactWorkgroups)) : int(grid);
            if (waves == 8) {
                if (quad) paged_prefill_d128<T, 8, true, F8, EXACT><<<g, 512, 0, s>>>(args);
                else paged_prefill_d128<T, 8, false, F8, EXACT><<<g, 512, 0, s>>>(args);
            } else {
                if (quad) paged_prefill_d128<T, 4, true, F8, EXACT><<<g, 256, 0, s>>>(args);
                else paged_prefill_d128<T, 4, false, F8, EXACT><<<g, 256, 0, s>>>(args);
            }
        };
        if (f8) {
            go.template operator()<true, false>();
            return launch_status("paged_prefill");
        }
        go.template operator()<false, false>();
        int st = launch_status("paged_prefill");
        if constexpr (std::is_same_v<T, __bf16>) {
            if (st == TVLLM_OK) {
                go.template operator()<false, true>();  // no-op unless V left fp16 range
                st = launch_status("paged_prefill exact fallback");
            }
        }
        return st;
    });
}

// Paged attention for any head dim up to 256: the decode rows and prefill
// chunks that the MFMA kernels (head_dim 128, GQA groups <= 16, 16-byte
// aligned rows) do not take.
//
// Reference behaviour: tinyvllm/kernels/paged_decode.cu:572-666 dispatches
// head dims 32, 64, 128 and 256 to one templated kernel; chunked prefill is
// SDPA with a lower-right causal mask (tinyvllm/runtime/attention.py:102-151,
// 176-214). Output = softmax(scale * q.K^T) V over each row's cached tokens
// in logical order (a padded decode row of length 0 gives zeros).
//
// Design: one wave per (query token, KV head, group of up to 16 query heads
// of that KV head), so the query heads of a KV head share every K/V load.
// The wave walks its keys in chunks of 64: lane j scores key j of the chunk
// against all of the wave's heads (the query rows sit in LDS, read as
// broadcasts), the online softmax runs per head across the wave, and P.V
// runs with the lanes over the head dims (lane l: dims l, l + 64, ...), the
// chunk's probabilities read back from LDS. Everything is fp32 (the query
// pre-multiplied by scale * log2(e)); no matrix cores - these shapes are
// outside every benchmark configuration, and the fp32 path is exact enough
// to need no fallback of its own.
#include "general_attention.h"

#include <algorithm>
#include <type_traits>

namespace tvllm {
namespace {

constexpr int GH = 16;     // query heads per wave
constexpr int DMAX = 256;  // largest head dim
constexpr float kLog2eG = 1.4426950408889634f;
constexpr int kRowWaves = 4;  // waves per workgroup of the row-tiled kernel

// Orders one wave's LDS writes before its own later reads (no other wave is
// involved): a compiler barrier - the wave's LDS operations run in order.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Eight elements of a cache row starting at element e (FP8: bytes), as
// floats; elements at or past `left` read as 0.
template <typename T, bool F8, bool VEC>
__device__ __forceinline__ void load8(const void* __restrict__ base, int64_t e, int left,
                                      float (&x)[8]) {
    if constexpr (F8) {
        const uint8_t* b = static_cast<const uint8_t*>(base) + e;
        if constexpr (VEC) {
            fp8x8_unpack(*reinterpret_cast<const uint2*>(b), x);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                x[i] = i < left ? __builtin_amdgcn_cvt_f32_fp8(int(b[i]), 0) : 0.f;
        }
    } else {
        const T* p = static_cast<const T*>(base) + e;
        if constexpr (VEC) {
            unpack8<T>(*reinterpret_cast<const U16x8*>(p), x);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = i < left ? to_f<T>(p[i]) : 0.f;
        }
    }
}

template <typename T, bool F8>
__device__ __forceinline__ float load1(const void* __restrict__ base, int64_t e) {
    if constexpr (F8) {
        return __builtin_amdgcn_cvt_f32_fp8(int(static_cast<const uint8_t*>(base)[e]), 0);
    } else {
        return to_f<T>(static_cast<const T*>(base)[e]);
    }
}

template <typename T, bool F8, bool VEC>
__global__ void __launch_bounds__(64) general_attention_kernel(GeneralAttention a) {
    __shared__ __align__(16) float qs[GH][DMAX];
    __shared__ float ps[GH][64];
    const int lane = threadIdx.x;
    const int group = a.heads / a.kv_heads;
    const int chunks = (group + GH - 1) / GH;
    const int64_t bx = blockIdx.x;
    const int hc = int(bx % chunks);
    const int64_t ik = bx / chunks;
    const int kvh = int(ik % a.kv_heads);
    const int64_t item = ik / a.kv_heads;
    const int64_t qi = blockIdx.y;

    int64_t tok, qlen;
    if (a.rows) {
        tok = a.rows[item];
        qlen = 1;
    } else {
        const int64_t qb = a.q_offsets[item];
        qlen = a.q_offsets[item + 1] - qb;
        if (qi >= qlen) return;  // uniform per wave
        tok = qb + qi;
    }
    const int64_t ctx = a.lengths[item];
    const int64_t kv_end = ctx - qlen + qi + 1;  // decode: ctx
    const int g0 = hc * GH;
    const int gw = min(GH, group - g0);
    const int h0 = kvh * group + g0;
    const int D = a.head_dim;
    const int D8 = (D + 7) & ~7;
    T* const out = static_cast<T*>(a.out) + tok * a.ots;

    if (kv_end <= 0) {  // nothing to attend (a padded row): zeros
        for (int g = 0; g < gw; ++g)
            for (int d = lane; d < D; d += 64) out[(h0 + g) * a.ohs + d] = static_cast<T>(0.f);
        return;
    }

    const float qscale = a.scale * kLog2eG * a.k_scale;
    const T* const q = static_cast<const T*>(a.q) + tok * a.qts;
    for (int g = 0; g < gw; ++g)
        for (int d = lane; d < D8; d += 64)
            qs[g][d] = d < D ? to_f<T>(q[(h0 + g) * a.qhs + d]) * qscale : 0.f;
    __syncthreads();

    float m[GH], l[GH], acc[GH][4];
#pragma unroll
    for (int g = 0; g < GH; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[g][i] = 0.f;
    }
    const int64_t table = a.offsets[item];
    const int bs = a.block_size;
    const int64_t head_off = int64_t(kvh) * a.chs;

    for (int64_t t0 = 0; t0 < kv_end; t0 += 64) {
        const bool valid = t0 + lane < kv_end;
        const int64_t t = min(t0 + lane, kv_end - 1);  // masked lanes read a valid row
        const int64_t page = t / bs;
        const int64_t slot = a.blocks[table + page] * bs + (t - page * bs);
        const int64_t kb = slot * a.css + head_off;

        float s[GH];
#pragma unroll
        for (int g = 0; g < GH; ++g) s[g] = 0.f;
        for (int d = 0; d < D8; d += 8) {
            float x[8];
            load8<T, F8, VEC>(a.k, kb + d, D - d, x);
#pragma unroll
            for (int g = 0; g < GH; ++g) {
                if (g >= gw) continue;  // uniform
                const float4 qa = *reinterpret_cast<const float4*>(&qs[g][d]);
                const float4 qb = *reinterpret_cast<const float4*>(&qs[g][d + 4]);
                float v = s[g];
                v = fmaf(qa.x, x[0], v);
                v = fmaf(qa.y, x[1], v);
                v = fmaf(qa.z, x[2], v);
                v = fmaf(qa.w, x[3], v);
                v = fmaf(qb.x, x[4], v);
                v = fmaf(qb.y, x[5], v);
                v = fmaf(qb.z, x[6], v);
                v = fmaf(qb.w, x[7], v);
                s[g] = v;
            }
        }
        // Online softmax per head (base 2); lane 0's key is always valid, so
        // every chunk maximum is finite.
#pragma unroll
        for (int g = 0; g < GH; ++g) {
            if (g >= gw) continue;
            const float sg = valid ? s[g] : -INFINITY;
            const float mn = fmaxf(m[g], wave_max(sg));
            const float alpha = exp2f(m[g] - mn);
            const float p = exp2f(sg - mn);
            l[g] = l[g] * alpha + wave_sum(p);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[g][i] *= alpha;
            m[g] = mn;
            ps[g][lane] = p;
        }
        __syncthreads();
        const int n = int(min<int64_t>(64, kv_end - t0));
        const uint32_t slo = uint32_t(slot), shi = uint32_t(uint64_t(slot) >> 32);
#pragma unroll 4
        for (int j = 0; j < n; ++j) {
            const int64_t sj = int64_t((uint64_t(uint32_t(__shfl(int(shi), j, 64))) << 32) |
                                       uint32_t(__shfl(int(slo), j, 64)));
            const int64_t vb = sj * a.css + head_off;
            float vv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = lane + 64 * i;
                vv[i] = d < D ? load1<T, F8>(a.v, vb + d) : 0.f;
            }
#pragma unroll
            for (int g = 0; g < GH; ++g) {
                if (g >= gw) continue;
                const float p = ps[g][j];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[g][i] = fmaf(p, vv[i], acc[g][i]);
            }
        }
        __syncthreads();  // ps is rewritten by the next chunk
    }

#pragma unroll
    for (int g = 0; g < GH; ++g) {
        if (g >= gw) continue;
        const float inv = a.v_scale / l[g];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = lane + 64 * i;
            if (d < D) out[(h0 + g) * a.ohs + d] = static_cast<T>(acc[g][i] * inv);
        }
    }
}

// The reference's head dims (32, 64, 128, 256) with vector-aligned rows.
// A workgroup serves up to 16 (query token, query head) rows of one KV head:
// one query's group of heads (up to 16), or for groups below 16 several
// consecutive queries of one prefill item, each row with its own causal
// bound. Its four waves take interleaved chunks of KPC keys: LPK lanes share
// a key (each holds EPL <= 64 of its dims), K and V pieces of the whole
// chunk are loaded at once and the wave's next chunk is in flight during
// this chunk's P.V; V is staged in the wave's own LDS buffer (FP8 widened
// exactly to T) for P.V with the lanes over the dims, each key's
// probabilities broadcast from the lanes that scored it. The waves' (max,
// sum, accumulator) merge through LDS at the end.
template <typename T, bool F8, int D>
__global__ void __launch_bounds__(64 * kRowWaves) rows_attention_kernel(GeneralAttention a) {
    constexpr int LPK = D > 64 ? D / 64 : 1;  // lanes per key
    constexpr int EPL = D / LPK;               // elements per lane
    constexpr int KPC = 64 / LPK;              // keys per chunk
    constexpr int NV = EPL / 8;                // 8-element pieces per lane
    constexpr int DI = (D + 63) / 64;          // output dims per lane
    using Piece = std::conditional_t<F8, uint2, uint4>;  // native vectors: kept in registers
    constexpr int NW = kRowWaves;
    // LDS: the rows' queries and each wave's staged V chunk; after the key
    // loop the same bytes hold waves 1..NW-1's partial results for the merge.
    // Staged V rows are padded by 16 bytes, so the lanes' 16-byte row writes
    // (one key per lane, rows D * 2 bytes apart) spread over the LDS banks.
    constexpr int VS = D + 8;  // staged V row stride (elements)
    constexpr int kMain = GH * D * 4 + NW * KPC * VS * 2;
    constexpr int kMerge = (NW - 1) * GH * (D + 2) * 4;
    __shared__ __align__(16) unsigned char smem[kMain > kMerge ? kMain : kMerge];
    float (*const qs)[D] = reinterpret_cast<float (*)[D]>(smem);
    const int wave = threadIdx.x >> 6;
    U16x8 (*const vs)[VS / 8] =
        reinterpret_cast<U16x8 (*)[VS / 8]>(smem + GH * D * 4 + wave * KPC * VS * 2);

    const int lane = threadIdx.x & 63;
    const int group = a.heads / a.kv_heads;
    const int hpq = group >= GH ? GH : group;   // heads per query in a wave
    const int qpw = group >= GH ? 1 : GH / group;  // queries per wave
    const int chunks = (group + GH - 1) / GH;
    const int64_t bx = blockIdx.x;
    const int hc = int(bx % chunks);
    const int64_t ik = bx / chunks;
    const int kvh = int(ik % a.kv_heads);
    const int64_t item = ik / a.kv_heads;
    // Prefill: y is the workgroup's tile of queries. Decode: its split of
    // the row's keys (one query).
    const int64_t q0 = a.rows ? 0 : int64_t(blockIdx.y) * qpw;
    const int64_t split = a.rows ? int64_t(blockIdx.y) : 0;

    int64_t tok0, qlen;
    if (a.rows) {
        tok0 = a.rows[item];
        qlen = 1;
    } else {
        tok0 = a.q_offsets[item];
        qlen = a.q_offsets[item + 1] - tok0;
        if (q0 >= qlen) return;  // uniform per workgroup
        tok0 += q0;
    }
    const int64_t nq = min<int64_t>(qpw, qlen - q0);
    const int g0 = hc * GH;
    const int hw = min(hpq, group - g0);
    const int nrows = int(nq) * hw;
    const int64_t ctx = a.lengths[item];
    const int64_t first_end = ctx - qlen + q0 + 1;  // causal bound of the wave's first query
    const int64_t kv_max = first_end + nq - 1;       // ... and of its last
    const float qscale = a.scale * kLog2eG * a.k_scale;
    const T* const q = static_cast<const T*>(a.q);
    T* const out = static_cast<T*>(a.out);
    auto row_token = [&](int r) { return tok0 + r / hw; };
    auto row_head = [&](int r) { return kvh * group + g0 + r % hw; };
    // Keys [k_begin, k_end) of this split (all of them when unsplit). The
    // last split also takes any keys past splits * split_keys (a row longer
    // than the max_context the plan was sized for): slow, never wrong.
    const int64_t k_begin = split * a.split_keys;
    const int64_t k_end = a.splits > 1 && split + 1 < a.splits
        ? min(kv_max, k_begin + a.split_keys) : kv_max;
    auto part_index = [&](int r) { return (item * a.heads + row_head(r)) * a.splits + split; };

    if (a.splits > 1 && k_begin >= k_end) {  // no key of the row in this split
        for (int r = threadIdx.x; r < nrows; r += 64 * NW) {
            a.part_ml[2 * part_index(r)] = -INFINITY;  // the merge skips it
            a.part_ml[2 * part_index(r) + 1] = 0.f;
        }
        return;  // uniform per workgroup
    }

    if (kv_max <= 0) {  // no key for any row (a padded decode row): zeros, and
                        // no read of its block table, which may hold no entry
        for (int r = 0; r < nrows; ++r)
            for (int d = threadIdx.x; d < D; d += 64 * NW)
                out[row_token(r) * a.ots + row_head(r) * a.ohs + d] = static_cast<T>(0.f);
        return;  // uniform per workgroup
    }
    for (int r = 0; r < nrows; ++r)
        for (int d = threadIdx.x; d < D; d += 64 * NW)
            qs[r][d] = to_f<T>(q[row_token(r) * a.qts + row_head(r) * a.qhs + d]) * qscale;
    __syncthreads();

    float m[GH], l[GH], acc[GH][DI];
#pragma unroll
    for (int r = 0; r < GH; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.f;
#pragma unroll
        for (int i = 0; i < DI; ++i) acc[r][i] = 0.f;
    }
    const int64_t table = a.offsets[item];
    const int bs = a.block_size;
    const int kp = lane / LPK;    // the lane's key within a chunk
    const int part = lane % LPK;  // ... and its share of the dims
    const int64_t lane_off = int64_t(kvh) * a.chs + part * EPL;

    struct Chunk {
        Piece k[NV], v[NV];
    };
    auto load_chunk = [&](int64_t t0) -> Chunk {
        const int64_t t = max<int64_t>(min(t0 + kp, kv_max - 1), 0);  // a valid row
        const int64_t page = t / bs;
        const int64_t base = (a.blocks[table + page] * bs + (t - page * bs)) * a.css + lane_off;
        Chunk c;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            if constexpr (F8) {
                c.k[v] = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(a.k) + base + 8 * v);
                c.v[v] = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(a.v) + base + 8 * v);
            } else {
                c.k[v] = *reinterpret_cast<const uint4*>(static_cast<const T*>(a.k) + base + 8 * v);
                c.v[v] = *reinterpret_cast<const uint4*>(static_cast<const T*>(a.v) + base + 8 * v);
            }
        }
        return c;
    };

    // Wave w takes chunks w, w + NW, ... of the keys.
    Chunk cur = load_chunk(k_begin + int64_t(wave) * KPC);
    for (int64_t t0 = k_begin + int64_t(wave) * KPC; t0 < k_end; t0 += NW * KPC) {
        // The chunk's V pieces into LDS, its K pieces unpacked to floats.
        float x[NV][8];
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            if constexpr (F8) {
                vs[kp][(part * EPL) / 8 + v] = fp8x8_widen<T>(cur.v[v]);  // exact in T
                fp8x8_unpack(cur.k[v], x[v]);
            } else {
                vs[kp][(part * EPL) / 8 + v] = __builtin_bit_cast(U16x8, cur.v[v]);
                unpack8<T>(__builtin_bit_cast(U16x8, cur.k[v]), x[v]);
            }
        }
        float s[GH];
#pragma unroll
        for (int r = 0; r < GH; ++r) {
            s[r] = 0.f;
            if (r < nrows) {  // uniform
                float y = 0.f;
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    const int d = part * EPL + 8 * v;
                    const float4 qa = *reinterpret_cast<const float4*>(&qs[r][d]);
                    const float4 qb = *reinterpret_cast<const float4*>(&qs[r][d + 4]);
                    y = fmaf(qa.x, x[v][0], y);
                    y = fmaf(qa.y, x[v][1], y);
                    y = fmaf(qa.z, x[v][2], y);
                    y = fmaf(qa.w, x[v][3], y);
                    y = fmaf(qb.x, x[v][4], y);
                    y = fmaf(qb.y, x[v][5], y);
                    y = fmaf(qb.z, x[v][6], y);
                    y = fmaf(qb.w, x[v][7], y);
                }
                s[r] = y;
            }
        }
        const int64_t key = t0 + kp;
        float pr[GH];  // this lane's key's probability for each row
#pragma unroll
        for (int r = 0; r < GH; ++r) {
            pr[r] = 0.f;
            if (r >= nrows) continue;
            float sr = s[r];
            if constexpr (LPK > 1) sr += __shfl_xor(sr, 1, 64);
            if constexpr (LPK > 2) sr += __shfl_xor(sr, 2, 64);
            // Row r (query r / hw) sees keys below its own causal bound.
            const float sg = key < first_end + r / hw && key < k_end ? sr : -INFINITY;
            const float mn = fmaxf(m[r], wave_max(sg));
            const float alpha = mn == -INFINITY ? 1.f : exp2f(m[r] - mn);
            const float p = sg == -INFINITY ? 0.f : exp2f(sg - mn);
            l[r] = l[r] * alpha + wave_sum(part == 0 ? p : 0.f);
#pragma unroll
            for (int i = 0; i < DI; ++i) acc[r][i] *= alpha;
            m[r] = mn;
            pr[r] = p;
        }
        wave_sync();  // the chunk's V rows are in LDS
        // The next chunk's rows (past the end: clamped, valid rows, loaded
        // unconditionally so the loaded registers are no loop-carried
        // choice) are in flight during P.V.
        cur = load_chunk(t0 + NW * KPC);
        const int n = int(min<int64_t>(KPC, k_end - t0));
        const uint16_t* const vrow = reinterpret_cast<const uint16_t*>(&vs[0][0]);
        // Eight keys at a time: their V elements are read from LDS together,
        // and each key's probabilities come from the lanes that scored it
        // (a register broadcast, no LDS round trip).
        for (int j0 = 0; j0 < n; j0 += 8) {
            float vv[8][DI];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj)
#pragma unroll
                for (int i = 0; i < DI; ++i) {
                    const int d = lane + 64 * i;
                    vv[jj][i] = (j0 + jj < n && d < D)
                        ? to_f<T>(__builtin_bit_cast(T, vrow[(j0 + jj) * VS + d])) : 0.f;
                }
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                if (j0 + jj >= n) continue;  // uniform
#pragma unroll
                for (int r = 0; r < GH; ++r) {
                    if (r >= nrows) continue;
                    const float p = __builtin_bit_cast(
                        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pr[r]),
                                                         (j0 + jj) * LPK));
#pragma unroll
                    for (int i = 0; i < DI; ++i) acc[r][i] = fmaf(p, vv[jj][i], acc[r][i]);
                }
            }
        }
        wave_sync();  // the wave's V buffer is rewritten by the next chunk
    }

    // Merge the waves' partial results: out = sum_w 2^(m_w - M) acc_w /
    // sum_w 2^(m_w - M) l_w per row (M the largest m_w); a row with no key
    // in any wave gives zeros.
    __syncthreads();  // every wave is past its last LDS read of qs and vs
    float* const part_acc = reinterpret_cast<float*>(smem);          // [NW-1][GH][D]
    float* const part_ml = part_acc + (NW - 1) * GH * D;             // [NW-1][GH][2]
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < GH; ++r) {
            if (r >= nrows) continue;
            float* const pa = part_acc + ((wave - 1) * GH + r) * D;
#pragma unroll
            for (int i = 0; i < DI; ++i) {
                const int d = lane + 64 * i;
                if (d < D) pa[d] = acc[r][i];
            }
            if (lane == 0) {
                part_ml[((wave - 1) * GH + r) * 2] = m[r];
                part_ml[((wave - 1) * GH + r) * 2 + 1] = l[r];
            }
        }
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int r = 0; r < GH; ++r) {
        if (r >= nrows) continue;
        float mx = m[r];
        for (int w = 1; w < NW; ++w) mx = fmaxf(mx, part_ml[((w - 1) * GH + r) * 2]);
        float den = 0.f;
        float num[DI];
        const float w0 = mx == -INFINITY ? 0.f : exp2f(m[r] - mx);
        den = w0 * l[r];
#pragma unroll
        for (int i = 0; i < DI; ++i) num[i] = w0 * acc[r][i];
        for (int w = 1; w < NW; ++w) {
            const float mw = part_ml[((w - 1) * GH + r) * 2];
            const float ww = mx == -INFINITY ? 0.f : exp2f(mw - mx);
            den += ww * part_ml[((w - 1) * GH + r) * 2 + 1];
            const float* const pa = part_acc + ((w - 1) * GH + r) * D;
#pragma unroll
            for (int i = 0; i < DI; ++i) {
                const int d = lane + 64 * i;
                if (d < D) num[i] += ww * pa[d];
            }
        }
        if (a.splits > 1) {  // the split's partials, merged by general_merge
            float* const po = a.part_o + part_index(r) * D;
#pragma unroll
            for (int i = 0; i < DI; ++i) {
                const int d = lane + 64 * i;
                if (d < D) po[d] = num[i];
            }
            if (lane == 0) {
                a.part_ml[2 * part_index(r)] = mx;
                a.part_ml[2 * part_index(r) + 1] = den;
            }
            continue;
        }
        const float inv = den > 0.f ? a.v_scale / den : 0.f;
        T* const o = out + row_token(r) * a.ots + row_head(r) * a.ohs;
#pragma unroll
        for (int i = 0; i < DI; ++i) {
            const int d = lane + 64 * i;
            if (d < D) o[d] = static_cast<T>(num[i] * inv);
        }
    }
}

// Merge a split decode: out = v_scale * sum_s 2^(m_s - M) o_s / sum_s
// 2^(m_s - M) l_s, M the largest m_s; splits with no key (m_s = -inf) are
// skipped, so their o_s is never read, and a row with none gives zeros. One
// wave per (row, query head): lane s holds split s's (max, sum) (splits <=
// 64), lane l the output dims l, l + 64, ...
template <typename T, int D>
__global__ void __launch_bounds__(64)
general_merge(const float* __restrict__ part_o, const float* __restrict__ part_ml,
              T* __restrict__ out, const int64_t* __restrict__ rows, int64_t ots, int64_t ohs,
              int heads, int splits, float v_scale) {
    constexpr int DI = (D + 63) / 64;
    const int id = blockIdx.x;
    const int r = id / heads;
    const int h = id - r * heads;
    const int lane = threadIdx.x;
    const int64_t base = (int64_t(r) * heads + h) * splits;
    float m = -INFINITY, l = 0.f;
    if (lane < splits) {
        m = part_ml[2 * (base + lane)];
        l = part_ml[2 * (base + lane) + 1];
    }
    const float mx = wave_max(m);
    T* const o = out + rows[r] * ots + h * ohs;
    float acc[DI];
#pragma unroll
    for (int i = 0; i < DI; ++i) acc[i] = 0.f;
    float inv = 0.f;
    if (mx != -INFINITY) {  // uniform
        const float w = m == -INFINITY ? 0.f : exp2f(m - mx);
        inv = v_scale / wave_sum(w * l);
        for (int s0 = 0; s0 < splits; ++s0) {
            const float ws = __shfl(w, s0, 64);
            if (ws == 0.f) continue;  // uniform: an empty split (or a negligible one)
            const float* const po = part_o + (base + s0) * D;
#pragma unroll
            for (int i = 0; i < DI; ++i) {
                const int d = lane + 64 * i;
                if (d < D) acc[i] = fmaf(ws, po[d], acc[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < DI; ++i) {
        const int d = lane + 64 * i;
        if (d < D) o[d] = static_cast<T>(acc[i] * inv);
    }
}

// Keys per chunk of the row-tiled kernel at head dim D (LPK lanes per key).
int64_t keys_per_chunk(int64_t D) { return D > 64 ? 64 / (D / 64) : 64; }

bool rows_kernel_dim(int64_t D) { return D == 32 || D == 64 || D == 128 || D == 256; }

}  // namespace

GeneralSplits general_decode_splits(int64_t rows, int64_t heads, int64_t kv_heads,
                                    int64_t head_dim, int64_t max_context) {
    GeneralSplits p{1, max_context};
    if (rows <= 0 || kv_heads <= 0 || heads % kv_heads != 0 || max_context <= 0 ||
        !rows_kernel_dim(head_dim))
        return p;
    // Aim for 512 workgroups (two of four waves per CU); a split keeps at
    // least two rounds of chunks per wave, and one merge lane per split.
    constexpr int64_t kTarget = 512, kMaxSplits = 64;
    const int64_t units = rows * kv_heads * ((heads / kv_heads + GH - 1) / GH);
    const int64_t kpc = keys_per_chunk(head_dim);
    const int64_t min_keys = 2 * kRowWaves * kpc;
    int64_t s = std::min((kTarget + units - 1) / units, kMaxSplits);
    s = std::min(s, (max_context + min_keys - 1) / min_keys);
    if (s <= 1) return p;
    // Exactly s splits (a trailing one may hold no key: it writes an empty
    // partial), so the workspace never shrinks as max_context grows.
    p.splits = s;
    p.keys = ((max_context + s - 1) / s + kpc - 1) / kpc * kpc;
    return p;
}

int64_t general_decode_workspace(int64_t rows, int64_t heads, int64_t kv_heads,
                                 int64_t head_dim, int64_t max_context) {
    const GeneralSplits p = general_decode_splits(rows, heads, kv_heads, head_dim, max_context);
    return p.splits > 1 ? rows * heads * p.splits * (head_dim + 2) * int64_t(sizeof(float)) : 0;
}

int launch_general_attention(const GeneralAttention& g_in, hipStream_t stream) {
    GeneralAttention g = g_in;
    TVLLM_CHECK(g.head_dim > 0 && g.head_dim <= DMAX, "attention: head_dim must be in 1..256");
    TVLLM_CHECK(g.heads > 0 && g.kv_heads > 0 && g.heads % g.kv_heads == 0,
                "attention: query heads must be a multiple of the KV heads");
    if (g.num_items == 0) return TVLLM_OK;
    const int64_t chunks = (g.heads / g.kv_heads + GH - 1) / GH;
    const int64_t gx = g.num_items * g.kv_heads * chunks;
    const int64_t gy = g.rows ? 1 : g.max_query_len;
    TVLLM_CHECK(gx <= INT32_MAX && gy >= 1 && gy <= 65535,
                "attention: launch grid out of range (query chunks of at most 65535 tokens)");
    const bool f8 = g.cache_dtype == TVLLM_FP8_E4M3;
    const bool vec = g.head_dim % 8 == 0 && g.css % 8 == 0 && g.chs % 8 == 0 &&
                     (f8 ? aligned8(g.k) && aligned8(g.v) : aligned16(g.k) && aligned16(g.v));
    const int D = g.head_dim;
    const bool rows_kernel = vec && rows_kernel_dim(D);
    const int group = g.heads / g.kv_heads;
    const int64_t qpw = rows_kernel && group < GH ? GH / group : 1;
    g.splits = 1;
    g.split_keys = 0;
    g.part_o = g.part_ml = nullptr;
    if (g.rows && rows_kernel) {
        TVLLM_CHECK(g.max_context > 0, "attention: decode needs a positive max_context");
        const GeneralSplits p = general_decode_splits(g.num_items, g.heads, g.kv_heads, D,
                                                      g.max_context);
        if (p.splits > 1) {
            const int64_t need = g.num_items * g.heads * p.splits * (D + 2) * int64_t(sizeof(float));
            TVLLM_CHECK(g.workspace_bytes >= need && g.workspace != nullptr,
                        "paged_decode: workspace of %lld bytes required, %lld given",
                        (long long)need, (long long)g.workspace_bytes);
            TVLLM_CHECK(aligned16(g.workspace), "paged_decode: workspace must be 16-byte aligned");
            g.splits = p.splits;
            g.split_keys = p.keys;
            g.part_o = static_cast<float*>(g.workspace);
            g.part_ml = g.part_o + g.num_items * g.heads * p.splits * D;
        }
    }
    const int64_t gy_rows = g.rows ? g.splits : (g.max_query_len + qpw - 1) / qpw;
    const dim3 grid{static_cast<uint32_t>(gx), static_cast<uint32_t>(rows_kernel ? gy_rows : gy),
                    1u};
    return dispatch_half(g.dtype, [&]<int DT>() {
        using T = typename Elem<DT>::T;
        if (rows_kernel) {
            auto go = [&]<int DD>() {
                if (f8) rows_attention_kernel<T, true, DD><<<grid, 64 * kRowWaves, 0, stream>>>(g);
                else rows_attention_kernel<T, false, DD><<<grid, 64 * kRowWaves, 0, stream>>>(g);
            };
            if (D == 32) go.template operator()<32>();
            else if (D == 64) go.template operator()<64>();
            else if (D == 128) go.template operator()<128>();
            else go.template operator()<256>();
            if (g.splits > 1) {
                const int st = launch_status("attention (general head dims)");
                if (st != TVLLM_OK) return st;
                auto merge = [&]<int DD>() {
                    general_merge<T, DD><<<int(g.num_items * g.heads), 64, 0, stream>>>(
                        g.part_o, g.part_ml, static_cast<T*>(g.out), g.rows, g.ots, g.ohs,
                        g.heads, int(g.splits), g.v_scale);
                };
                if (D == 32) merge.template operator()<32>();
                else if (D == 64) merge.template operator()<64>();
                else if (D == 128) merge.template operator()<128>();
                else merge.template operator()<256>();
                return launch_status("attention merge (general head dims)");
            }
        } else if (f8 && vec) general_attention_kernel<T, true, true><<<grid, 64, 0, stream>>>(g);
        else if (f8) general_attention_kernel<T, true, false><<<grid, 64, 0, stream>>>(g);
        else if (vec) general_attention_kernel<T, false, true><<<grid, 64, 0, stream>>>(g);
        else general_attention_kernel<T, false, false><<<grid, 64, 0, stream>>>(g);
        return launch_status("attention (general head dims)");
    });
}

}  // namespace tvllm

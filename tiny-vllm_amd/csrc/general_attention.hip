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

namespace tvllm {
namespace {

constexpr int GH = 16;     // query heads per wave
constexpr int DMAX = 256;  // largest head dim
constexpr float kLog2eG = 1.4426950408889634f;

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
                if (g >= gw) break;  // uniform
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
            if (g >= gw) break;
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
                if (g >= gw) break;
                const float p = ps[g][j];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[g][i] = fmaf(p, vv[i], acc[g][i]);
            }
        }
        __syncthreads();  // ps is rewritten by the next chunk
    }

#pragma unroll
    for (int g = 0; g < GH; ++g) {
        if (g >= gw) break;
        const float inv = a.v_scale / l[g];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = lane + 64 * i;
            if (d < D) out[(h0 + g) * a.ohs + d] = static_cast<T>(acc[g][i] * inv);
        }
    }
}

}  // namespace

int launch_general_attention(const GeneralAttention& g, hipStream_t stream) {
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
    const dim3 grid{static_cast<uint32_t>(gx), static_cast<uint32_t>(gy), 1u};
    return dispatch_half(g.dtype, [&]<int DT>() {
        using T = typename Elem<DT>::T;
        if (f8 && vec) general_attention_kernel<T, true, true><<<grid, 64, 0, stream>>>(g);
        else if (f8) general_attention_kernel<T, true, false><<<grid, 64, 0, stream>>>(g);
        else if (vec) general_attention_kernel<T, false, true><<<grid, 64, 0, stream>>>(g);
        else general_attention_kernel<T, false, false><<<grid, 64, 0, stream>>>(g);
        return launch_status("attention (general head dims)");
    });
}

}  // namespace tvllm

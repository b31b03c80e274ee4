// Token sampling over [rows, vocab] logits: greedy argmax, and temperature /
// top-k / top-p sampling by the exponential race.
//
// Reference behaviour: tinyvllm/sampling.py:21-72 (TorchSampler.sample:
// greedy rows use logits.argmax) and :75-164 (_sample_batch):
//   s = (logit.float() - rowmax) / T; optional top-k; stable descending sort;
//   softmax; drop every token whose preceding cumulative probability exceeds
//   top_p (the first token crossing top_p is kept); choice = argmax p / E,
//   E ~ Exp(1).
//
// MI355X design: one 1024-thread workgroup per row, no sort. The kept set is
// found by radix selection over an order-preserving 32-bit key of s (four
// 8-bit digit passes, histograms in LDS), weighting each token by its
// probability mass in 2^-40 fixed point so the sums are exact and
// deterministic; ties on s are resolved by token index (three more passes),
// which is exactly the stable sort's order. The noise is a counter-based
// Philox4x32-10 stream (Salmon et al., SC'11) keyed by the request seed and
// its sample counter, so a step is reproducible and graph-capturable.
#include "common.h"

namespace tvllm {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

template <typename T>
__device__ __forceinline__ float load_logit(const T* row, int64_t i) {
    return to_f<T>(row[i]);
}

// Better = larger value; NaN beats numbers; ties go to the lower index.
__device__ __forceinline__ bool better(float a, int64_t ia, float b, int64_t ib) {
    const bool na = a != a, nb = b != b;
    if (na || nb) return na && (!nb || ia < ib);
    return a > b || (a == b && ia < ib);
}

__device__ __forceinline__ void wave_argmax(float& v, int64_t& idx) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int64_t oi = __shfl_xor(idx, off, 64);
        if (better(ov, oi, v, idx)) { v = ov; idx = oi; }
    }
}

// Block-wide argmax over W waves; every thread gets the result.
template <int W>
__device__ void block_argmax_w(float& v, int64_t& idx) {
    __shared__ float sv[W];
    __shared__ int64_t si[W];
    wave_argmax(v, idx);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[w] = v; si[w] = idx; }
    __syncthreads();
    v = sv[0];
    idx = si[0];
    for (int i = 1; i < W; ++i)
        if (better(sv[i], si[i], v, idx)) { v = sv[i]; idx = si[i]; }
    __syncthreads();
}

// Block-wide argmax; every thread gets the result.
__device__ void block_argmax(float& v, int64_t& idx) {
    __shared__ float sv[kWaves];
    __shared__ int64_t si[kWaves];
    wave_argmax(v, idx);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[w] = v; si[w] = idx; }
    __syncthreads();
    v = sv[0];
    idx = si[0];
    for (int i = 1; i < kWaves; ++i)
        if (better(sv[i], si[i], v, idx)) { v = sv[i]; idx = si[i]; }
    __syncthreads();
}

template <typename T, bool VEC>
__global__ void __launch_bounds__(kThreads)
argmax_kernel(const T* __restrict__ logits, int64_t vocab, int64_t stride,
              int64_t* __restrict__ out);

// ------------------------------------------------------------ sampling ----

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as
// easy as 1, 2, 3", SC'11): 10 rounds of the 4x32 multiply-xor bijection.
__device__ __forceinline__ uint4 philox4x32_10(uint4 ctr, uint2 key) {
    constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u;
    constexpr uint32_t kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;
#pragma unroll
    for (int round = 0; round < 10; ++round) {
        const uint32_t hi0 = __umulhi(kM0, ctr.x), lo0 = kM0 * ctr.x;
        const uint32_t hi1 = __umulhi(kM1, ctr.z), lo1 = kM1 * ctr.z;
        ctr = make_uint4(hi1 ^ ctr.y ^ key.x, lo1, hi0 ^ ctr.w ^ key.y, lo0);
        key.x += kW0;
        key.y += kW1;
    }
    return ctr;
}

// Order-preserving map float -> uint32 (larger float, larger key).
__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

constexpr double kMassScale = 1099511627776.0;  // 2^40 fixed point

struct RowCtx {
    float mx;     // row max of the logits
    float temp;   // temperature
};

template <typename T>
__device__ __forceinline__ float score_of(const T* row, int64_t i, const RowCtx& c) {
    return (load_logit(row, i) - c.mx) / c.temp;
}

__device__ __forceinline__ uint64_t mass_of(float s) {
    return static_cast<uint64_t>(static_cast<double>(expf(s)) * kMassScale);
}

// Selection result: kept = key > k or (key == k and index <= idx).
struct Cut {
    uint32_t key;
    int64_t idx;
    bool all;  // total weight never exceeds the target: keep everything
};

__device__ __forceinline__ bool kept(const Cut& c, uint32_t key, int64_t i) {
    return c.all || key > c.key || (key == c.key && i <= c.idx);
}

// Finds the first element, in (key descending, index ascending) order among
// elements with in(i), whose inclusive cumulative weight exceeds `target`.
// weight(i) is 1 (MASS = false) or the fixed-point probability mass.
template <typename T, bool MASS, typename In>
__device__ Cut radix_cut(const T* row, int64_t vocab, const RowCtx& ctx,
                         uint64_t target, In&& in) {
    __shared__ uint64_t hist[256];
    __shared__ uint32_t s_prefix;
    __shared__ uint64_t s_above;
    __shared__ int s_found;
    uint32_t prefix = 0;
    uint64_t above = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int b = threadIdx.x; b < 256; b += kThreads) hist[b] = 0;
        __syncthreads();
        for (int64_t i = threadIdx.x; i < vocab; i += kThreads) {
            if (!in(i)) continue;
            const float s = score_of(row, i, ctx);
            const uint32_t k = fkey(s);
            if (shift < 24 && ((k ^ prefix) >> (shift + 8)) != 0) continue;
            atomicAdd(reinterpret_cast<unsigned long long*>(&hist[(k >> shift) & 255]),
                      static_cast<unsigned long long>(MASS ? mass_of(s) : 1));
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t cum = above;
            int found = -1;
            for (int b = 255; b >= 0; --b) {
                if (cum + hist[b] > target) { found = b; break; }
                cum += hist[b];
            }
            s_found = found;
            s_prefix = found >= 0 ? prefix | (uint32_t(found) << shift) : prefix;
            s_above = cum;
        }
        __syncthreads();
        if (s_found < 0) {
            Cut c{0u, 0, true};
            __syncthreads();
            return c;
        }
        prefix = s_prefix;
        above = s_above;
        __syncthreads();
    }
    // prefix is the boundary key; every tie there has the same weight w.
    // The boundary is the j-th tie in index order, j = (target - above) / w.
    uint64_t w = 1;
    if constexpr (MASS) {
        w = 0;
        // All ties share s, hence the same mass; recompute from any of them.
        __shared__ uint64_t s_w;
        if (threadIdx.x == 0) s_w = 0;
        __syncthreads();
        for (int64_t i = threadIdx.x; i < vocab; i += kThreads) {
            if (!in(i)) continue;
            const float s = score_of(row, i, ctx);
            if (fkey(s) == prefix) { s_w = mass_of(s); break; }
        }
        __syncthreads();
        w = s_w;
        __syncthreads();
    }
    const uint64_t j = w ? (target - above) / w : 0;
    // Ascending radix select of the j-th tie index (indices < 2^24).
    __shared__ uint32_t ihist[256];
    __shared__ uint32_t s_iprefix;
    __shared__ uint64_t s_ibelow;
    uint32_t iprefix = 0;
    uint64_t below = 0;
    for (int shift = 16; shift >= 0; shift -= 8) {
        for (int b = threadIdx.x; b < 256; b += kThreads) ihist[b] = 0;
        __syncthreads();
        for (int64_t i = threadIdx.x; i < vocab; i += kThreads) {
            if (!in(i)) continue;
            const uint32_t ui = static_cast<uint32_t>(i);
            if (shift < 16 && ((ui ^ iprefix) >> (shift + 8)) != 0) continue;
            if (fkey(score_of(row, i, ctx)) != prefix) continue;
            atomicAdd(&ihist[(ui >> shift) & 255], 1u);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t cum = below;
            int found = 255;
            for (int b = 0; b < 256; ++b) {
                if (cum + ihist[b] > j) { found = b; break; }
                cum += ihist[b];
            }
            s_iprefix = iprefix | (uint32_t(found) << shift);
            s_ibelow = cum;
        }
        __syncthreads();
        iprefix = s_iprefix;
        below = s_ibelow;
        __syncthreads();
    }
    return Cut{prefix, static_cast<int64_t>(iprefix), false};
}

// Per-thread running argmax over a row (16-byte vector loads when VEC).
template <typename T, bool VEC>
__device__ __forceinline__ void thread_argmax(const T* row, int64_t vocab, float& best,
                                              int64_t& bi) {
    int64_t tail = 0;
    if constexpr (VEC) {
        const int64_t nvec = vocab / 8;
        const U16x8* rv = reinterpret_cast<const U16x8*>(row);
        // Rows of up to kOnePass * kThreads vectors (vocabularies up to
        // 163840): every load of the thread is issued at once - out-of-range
        // ones read vector 0 and are skipped - so the row costs one memory
        // round trip instead of one per loop iteration.
        constexpr int kOnePass = 20;
        if (nvec <= int64_t(kOnePass) * kThreads) {
            U16x8 raw[kOnePass];
            const uint32_t n32 = uint32_t(nvec);
#pragma unroll
            for (int u = 0; u < kOnePass; ++u) {  // 32-bit offsets from the row base
                const uint32_t c = threadIdx.x + uint32_t(u) * kThreads;
                raw[u] = rv[c < n32 ? c : 0u];
            }
            // Two cheap passes over the registers instead of a NaN-aware
            // compare per element (which left the row scan VALU-bound): the
            // maximum, then the first index holding it. A thread that saw a
            // NaN redoes its elements with the exact compare.
            float m = -INFINITY;
            bool nan = false;
#pragma unroll
            for (int u = 0; u < kOnePass; ++u) {
                const uint32_t c = threadIdx.x + uint32_t(u) * kThreads;
                if (c >= n32) break;
                float x[8];
                unpack8<T>(raw[u], x);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    m = fmaxf(m, x[e]);
                    nan |= x[e] != x[e];
                }
            }
            if (!nan) {
                uint32_t first = UINT32_MAX;
#pragma unroll
                for (int u = 0; u < kOnePass; ++u) {
                    const uint32_t c = threadIdx.x + uint32_t(u) * kThreads;
                    if (c >= n32) break;
                    float x[8];
                    unpack8<T>(raw[u], x);
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        first = x[e] == m ? min(first, c * 8u + uint32_t(e)) : first;
                }
                if (first != UINT32_MAX) {
                    best = m;
                    bi = first;
                }
            } else {
#pragma unroll
                for (int u = 0; u < kOnePass; ++u) {
                    const int64_t c = threadIdx.x + int64_t(u) * kThreads;
                    if (c >= nvec) break;
                    float x[8];
                    unpack8<T>(raw[u], x);
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (better(x[e], c * 8 + e, best, bi)) { best = x[e]; bi = c * 8 + e; }
                }
            }
        } else {
        // Four independent 16-byte loads in flight per thread, then compare
        // in index order (ties keep the lower index either way).
        constexpr int U = 4;
        int64_t c = threadIdx.x;
        for (; c + (U - 1) * kThreads < nvec; c += U * kThreads) {
            U16x8 raw[U];
#pragma unroll
            for (int u = 0; u < U; ++u) raw[u] = rv[c + u * kThreads];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float x[8];
                unpack8<T>(raw[u], x);
                const int64_t base = (c + u * kThreads) * 8;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (better(x[e], base + e, best, bi)) { best = x[e]; bi = base + e; }
            }
        }
        for (; c < nvec; c += kThreads) {
            float x[8];
            unpack8<T>(rv[c], x);
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (better(x[e], c * 8 + e, best, bi)) { best = x[e]; bi = c * 8 + e; }
        }
        }
        tail = nvec * 8;
    }
    for (int64_t i = tail + threadIdx.x; i < vocab; i += kThreads) {
        const float x = load_logit(row, i);
        if (better(x, i, best, bi)) { best = x; bi = i; }
    }
}

// Greedy scan split over workgroups: row r's span s (kPartSpan elements)
// is scanned by one 256-thread workgroup, 4 vectors per thread in flight at
// once; the sampling kernel combines the spans. One 1024-thread workgroup
// per row left the scan VALU-bound on one CU (28 us per 151936-wide row);
// spans of 4 / 8 / 16 vectors per thread measured 14.1 / 15.6 / 21.1 us at
// 64 rows.
constexpr int kPartThreads = 256;
constexpr int kPartVecs = 4;
constexpr int64_t kPartSpan = int64_t(kPartThreads) * kPartVecs * 8;

struct ArgPart {
    float v;
    int32_t i;  // -1: empty span
};

template <typename T, bool VEC>
__global__ void __launch_bounds__(kPartThreads)
argmax_part_kernel(const T* __restrict__ logits, int64_t vocab, int64_t stride, int nparts,
                   ArgPart* __restrict__ parts) {
    const int r = blockIdx.x / nparts;
    const int span = blockIdx.x - r * nparts;
    const T* row = logits + int64_t(r) * stride;
    const int64_t begin = int64_t(span) * kPartSpan;
    const int64_t end = min(vocab, begin + kPartSpan);
    float best = -INFINITY;
    int64_t bi = INT64_MAX;
    int64_t tail = begin;
    if constexpr (VEC) {
        const U16x8* rv = reinterpret_cast<const U16x8*>(row);
        const uint32_t v0 = uint32_t(begin / 8), v1 = uint32_t(end / 8);  // whole vectors
        U16x8 raw[kPartVecs];
#pragma unroll
        for (int u = 0; u < kPartVecs; ++u) {
            const uint32_t c = v0 + threadIdx.x + uint32_t(u) * kPartThreads;
            raw[u] = rv[c < v1 ? c : v0];
        }
        float m = -INFINITY;
        bool nan = false;
#pragma unroll
        for (int u = 0; u < kPartVecs; ++u) {
            const uint32_t c = v0 + threadIdx.x + uint32_t(u) * kPartThreads;
            if (c >= v1) break;
            float x[8];
            unpack8<T>(raw[u], x);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                m = fmaxf(m, x[e]);
                nan |= x[e] != x[e];
            }
        }
#pragma unroll
        for (int u = 0; u < kPartVecs; ++u) {
            const uint32_t c = v0 + threadIdx.x + uint32_t(u) * kPartThreads;
            if (c >= v1) break;
            float x[8];
            unpack8<T>(raw[u], x);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int64_t i = int64_t(c) * 8 + e;
                if (nan ? better(x[e], i, best, bi) : (x[e] == m && i < bi)) {
                    best = x[e];
                    bi = i;
                }
            }
        }
        tail = int64_t(v1) * 8;
    }
    for (int64_t i = tail + threadIdx.x; i < end; i += kPartThreads) {
        const float x = load_logit(row, i);
        if (better(x, i, best, bi)) { best = x; bi = i; }
    }
    block_argmax_w<kPartThreads / 64>(best, bi);
    if (threadIdx.x == 0)
        parts[blockIdx.x] = ArgPart{best, bi == INT64_MAX ? -1 : int32_t(bi)};
}

template <typename T, bool VEC>
__global__ void __launch_bounds__(kThreads)
sample_kernel(const T* __restrict__ logits, int64_t vocab, int64_t stride,
              const float* __restrict__ temperature, const int64_t* __restrict__ top_k,
              const float* __restrict__ top_p, const int64_t* __restrict__ seeds,
              const int64_t* __restrict__ counters, int64_t* __restrict__ out,
              const ArgPart* __restrict__ parts, int nparts) {
    const int r = blockIdx.x;
    const T* row = logits + int64_t(r) * stride;

    // Row max (also the greedy answer): from the per-span partials of
    // argmax_part_kernel when given, else scanned here.
    float best = -INFINITY;
    int64_t bi = INT64_MAX;
    if (parts != nullptr) {
        for (int i = threadIdx.x; i < nparts; i += kThreads) {
            const ArgPart p = parts[int64_t(r) * nparts + i];
            const int64_t pi = p.i < 0 ? INT64_MAX : int64_t(p.i);
            if (better(p.v, pi, best, bi)) { best = p.v; bi = pi; }
        }
    } else {
        thread_argmax<T, VEC>(row, vocab, best, bi);
    }
    block_argmax(best, bi);
    const float temp = temperature[r];
    if (!(temp > 0.f)) {
        if (threadIdx.x == 0) out[r] = bi;
        return;
    }
    const RowCtx ctx{best, temp};
    const int64_t k = top_k[r];
    const float p = top_p[r];

    Cut kcut{0u, 0, true};
    if (k > 0 && k < vocab) {
        kcut = radix_cut<T, false>(row, vocab, ctx, uint64_t(k - 1),
                                   [](int64_t) { return true; });
    }
    auto in_k = [&](int64_t i) {
        return kcut.all || kept(kcut, fkey(score_of(row, i, ctx)), i);
    };

    Cut pcut{0u, 0, true};
    if (p < 1.f) {
        // Z = total mass of the top-k candidates (the softmax denominator).
        __shared__ unsigned long long s_z;
        if (threadIdx.x == 0) s_z = 0;
        __syncthreads();
        unsigned long long z = 0;
        for (int64_t i = threadIdx.x; i < vocab; i += kThreads)
            if (in_k(i)) z += mass_of(score_of(row, i, ctx));
        atomicAdd(&s_z, z);
        __syncthreads();
        const uint64_t target = static_cast<uint64_t>(static_cast<double>(p) *
                                                      static_cast<double>(s_z));
        pcut = radix_cut<T, true>(row, vocab, ctx, target, in_k);
    }

    // Exponential race over the kept set: argmax s_i - log(E_i).
    const uint2 key = make_uint2(static_cast<uint32_t>(seeds[r]),
                                 static_cast<uint32_t>(uint64_t(seeds[r]) >> 32));
    const uint64_t step = static_cast<uint64_t>(counters[r]);
    float bv = -INFINITY;
    int64_t bidx = INT64_MAX;
    for (int64_t i = threadIdx.x; i < vocab; i += kThreads) {
        const float s = score_of(row, i, ctx);
        const uint32_t kk = fkey(s);
        if (!kcut.all && !kept(kcut, kk, i)) continue;
        if (!pcut.all && !kept(pcut, kk, i)) continue;
        const uint4 rnd4 = philox4x32_10(
            make_uint4(static_cast<uint32_t>(i >> 2), static_cast<uint32_t>(i >> 34),
                       static_cast<uint32_t>(step), static_cast<uint32_t>(step >> 32)),
            key);
        const int lane4 = int(i & 3);
        const uint32_t bits = lane4 == 0 ? rnd4.x : lane4 == 1 ? rnd4.y
                            : lane4 == 2 ? rnd4.z : rnd4.w;
        const float u = (float(bits >> 8) + 0.5f) * (1.0f / 16777216.0f);
        const float e = -logf(u);
        const float g = s - logf(e);
        if (better(g, i, bv, bidx)) { bv = g; bidx = i; }
    }
    block_argmax(bv, bidx);
    if (threadIdx.x == 0) out[r] = bidx;
}

template <typename T, bool VEC>
__global__ void __launch_bounds__(kThreads)
argmax_kernel(const T* __restrict__ logits, int64_t vocab, int64_t stride,
              int64_t* __restrict__ out) {
    const T* row = logits + int64_t(blockIdx.x) * stride;
    float best = -INFINITY;
    int64_t bi = INT64_MAX;
    thread_argmax<T, VEC>(row, vocab, best, bi);
    block_argmax(best, bi);
    if (threadIdx.x == 0) out[blockIdx.x] = bi;
}

}  // namespace
}  // namespace tvllm

using namespace tvllm;

extern "C" int tvllm_argmax(const void* logits, int64_t rows, int64_t vocab,
                            int64_t row_stride, int64_t* out, int dtype,
                            tvllm_stream_t stream) {
    TVLLM_CHECK(rows >= 0 && vocab > 0 && row_stride >= vocab,
                "argmax: invalid logits geometry");
    TVLLM_CHECK(rows <= INT32_MAX, "argmax: too many rows");
    if (rows == 0) return TVLLM_OK;
    TVLLM_CHECK(logits && out, "argmax: null pointer");
    hipStream_t s = as_hip(stream);
    return dispatch_float(dtype, [&]<int DT>() {
        using T = typename Elem<DT>::T;
        const bool vec = row_stride % 8 == 0 && aligned16(logits);
        if constexpr (sizeof(T) == 2) {
            if (vec) {
                argmax_kernel<T, true><<<int(rows), kThreads, 0, s>>>(
                    static_cast<const T*>(logits), vocab, row_stride, out);
                return launch_status("argmax");
            }
        }
            argmax_kernel<T, false><<<int(rows), kThreads, 0, s>>>(
                static_cast<const T*>(logits), vocab, row_stride, out);
        return launch_status("argmax");
    });
}

extern "C" int64_t tvllm_sample_workspace_size(int64_t rows, int64_t vocab) {
    // One (value, index) partial per kPartSpan-wide span of each row.
    if (rows <= 0 || vocab <= 0) return 0;
    return rows * ((vocab + kPartSpan - 1) / kPartSpan) * int64_t(sizeof(ArgPart));
}

extern "C" int tvllm_sample(const void* logits, int64_t rows, int64_t vocab,
                            int64_t row_stride, const float* temperature,
                            const int64_t* top_k, const float* top_p,
                            const int64_t* seeds, const int64_t* counters,
                            int64_t* out, void* workspace, int64_t workspace_bytes,
                            int dtype, tvllm_stream_t stream) {
    TVLLM_CHECK(rows >= 0 && vocab > 0 && row_stride >= vocab,
                "sample: invalid logits geometry");
    TVLLM_CHECK(vocab < (int64_t(1) << 24), "sample: vocab must be < 2^24");
    TVLLM_CHECK(rows <= INT32_MAX, "sample: too many rows");
    if (rows == 0) return TVLLM_OK;
    TVLLM_CHECK(logits && temperature && top_k && top_p && seeds && counters && out,
                "sample: null pointer");
    TVLLM_CHECK(workspace_bytes >= 0 && (workspace_bytes == 0 || workspace != nullptr),
                "sample: null workspace");
    hipStream_t s = as_hip(stream);
    // With a workspace of tvllm_sample_workspace_size bytes the row scan is
    // split over spans (argmax_part_kernel); without one each row's
    // workgroup scans it alone.
    const int64_t nparts = (vocab + kPartSpan - 1) / kPartSpan;
    const bool split = workspace_bytes >= tvllm_sample_workspace_size(rows, vocab) &&
                       aligned16(workspace) && rows * nparts <= INT32_MAX;
    ArgPart* parts = split ? static_cast<ArgPart*>(workspace) : nullptr;
    return dispatch_float(dtype, [&]<int DT>() {
        using T = typename Elem<DT>::T;
        const bool vec = sizeof(T) == 2 && row_stride % 8 == 0 && aligned16(logits);
        auto go = [&]<bool V>() {
            if (split) {
                argmax_part_kernel<T, V><<<int(rows * nparts), kPartThreads, 0, s>>>(
                    static_cast<const T*>(logits), vocab, row_stride, int(nparts), parts);
                const int status = launch_status("sample");
                if (status != TVLLM_OK) return status;
            }
            sample_kernel<T, V><<<int(rows), kThreads, 0, s>>>(
                static_cast<const T*>(logits), vocab, row_stride, temperature, top_k,
                top_p, seeds, counters, out, parts, int(nparts));
            return launch_status("sample");
        };
        if constexpr (sizeof(T) == 2) {
            if (vec) return go.template operator()<true>();
        }
        return go.template operator()<false>();
    });
}

// ------------------------------------------------ pipelined input tokens ----

namespace tvllm {
namespace {

// tokens[i] = prev[src[i]] where 0 <= src[i] < prev_count, else unchanged.
__global__ void __launch_bounds__(256)
resolve_tokens_kernel(int64_t* __restrict__ tokens, const int64_t* __restrict__ src,
                      const int64_t* __restrict__ prev, int64_t n, int64_t prev_count) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const int64_t s = src[i];
    if (s >= 0 && s < prev_count) tokens[i] = prev[s];
}

}  // namespace
}  // namespace tvllm

extern "C" int tvllm_resolve_tokens(int64_t* tokens, const int64_t* src,
                                    const int64_t* prev, int64_t n, int64_t prev_count,
                                    tvllm_stream_t stream) {
    using namespace tvllm;
    TVLLM_CHECK(n >= 0 && prev_count >= 0, "resolve_tokens: negative size");
    TVLLM_CHECK(n <= (int64_t(INT32_MAX) - 255), "resolve_tokens: too many tokens");
    if (n == 0) return TVLLM_OK;
    TVLLM_CHECK(tokens && src && (prev || prev_count == 0), "resolve_tokens: null pointer");
    resolve_tokens_kernel<<<int((n + 255) / 256), 256, 0, as_hip(stream)>>>(
        tokens, src, prev, n, prev_count);
    return launch_status("resolve_tokens");
}

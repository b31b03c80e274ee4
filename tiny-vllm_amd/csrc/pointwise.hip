// Row-wise pointwise kernels of the Qwen3 layer: RMSNorm (+ residual add),
// SiLU(gate) * up, and per-head Q/K RMSNorm + half-split RoPE with an
// optional fused slot-mapped KV-cache write.
//
// Rounding points follow the reference kernels, which restate the PyTorch
// expressions (tinyvllm/kernels/pointwise.cu:95-116 rotate_pair, :128-214
// rms_norm_kernel, :260-321 silu_and_mul, :325-450 qk_norm_rope_kernel):
//   add:      x = round(x + residual)
//   rmsnorm:  y = round(round(x * rsqrt(mean_fp32(x^2) + eps)) * w)
//   silu:     o = round(round(g / (1 + exp(-g))) * u)
//   rope:     o1 = round(round(n1*c) - round(n2*s)); o2 = round(round(n2*c) + round(n1*s))
// All arithmetic is fp32 with contraction disabled at compile time, so each
// product and sum is rounded exactly where the expression says.
//
// Mapping: every row is owned by one wave64 (narrow rows) or one 256-thread
// workgroup (wide rows); a row is held in registers between the reduction
// and the write, so the input is read once.
#include "common.h"

namespace tvllm {
namespace {

// ------------------------------------------------------------ RMSNorm ----

// Loads 8 consecutive elements (16B vector when possible).
template <typename T, bool VEC>
__device__ __forceinline__ void load8(const T* p, int valid, float (&v)[8]) {
    if constexpr (VEC && sizeof(T) == 2) {
        if (valid >= 8) {
            U16x8 raw = *reinterpret_cast<const U16x8*>(p);
            unpack8<T>(raw, v);
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = i < valid ? to_f<T>(p[i]) : 0.f;
}

// 16-byte vector load of 8 elements at base[c] when ok, zeros otherwise.
// The load is unconditional (from base[0] when !ok, which must be mapped),
// so that a thread's loads are all in flight at once: loads under a branch
// are each waited for before the branch closes.
template <typename T>
__device__ __forceinline__ void load8_masked(const T* base, int c, bool ok,
                                             float (&v)[8]) {
    const U16x8 raw = *reinterpret_cast<const U16x8*>(base + (ok ? c : 0));
    unpack8<T>(raw, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = ok ? v[i] : 0.f;
}

template <typename T, bool VEC>
__device__ __forceinline__ void store8(T* p, int valid, const float (&v)[8]) {
    if constexpr (VEC && sizeof(T) == 2) {
        if (valid >= 8) {
            U16x8 raw;
#pragma unroll
            for (int i = 0; i < 4; ++i) raw.w[i] = pack2<T>(v[2 * i], v[2 * i + 1]);
            *reinterpret_cast<U16x8*>(p) = raw;
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (i < valid) p[i] = static_cast<T>(v[i]);
}

// TPR threads per row (64 = one wave, or 256 = one workgroup); NV chunks of
// 8 elements per thread are kept in registers (width <= TPR * 8 * NV).
template <typename T, int TPR, int NV, bool RESIDUAL, bool VEC>
__global__ void __launch_bounds__(256)
rms_norm_kernel(const T* __restrict__ x, int64_t rows, int64_t heads, int width,
                int64_t token_stride, int64_t head_stride,
                const T* __restrict__ weight, const T* __restrict__ residual,
                int64_t residual_stride, T* __restrict__ out,
                T* __restrict__ residual_out, float eps) {
    constexpr int RPB = 256 / TPR;  // rows per block
    const int sub = threadIdx.x / TPR;
    const int t = threadIdx.x % TPR;
    const int64_t row = int64_t(blockIdx.x) * RPB + sub;
    const bool active = row < rows;

    const int64_t r = active ? row : 0;
    // rows <= INT32_MAX (checked on the host): 32-bit division.
    const int64_t tok = uint32_t(r) / uint32_t(heads);
    const T* src = x + tok * token_stride + (r - tok * heads) * head_stride;
    const T* res = RESIDUAL ? residual + tok * residual_stride : nullptr;

    // Weights are loaded up front so their latency overlaps the reduction.
    float v[NV][8], wv[NV][8];
    float ss = 0.f;
    float rv[NV][8];
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        const int c = (n * TPR + t) * 8;
        if constexpr (VEC && sizeof(T) == 2) {  // width % 8 == 0: whole chunks
            const bool ok = c < width;  // inactive threads read row 0
            load8_masked<T>(src, c, ok, v[n]);
            load8_masked<T>(weight, c, ok, wv[n]);
            if constexpr (RESIDUAL) load8_masked<T>(res, c, ok, rv[n]);
        } else {
            const int valid = active ? min(8, width - c) : 0;
            load8<T, VEC>(src + c, valid, v[n]);
            load8<T, VEC>(weight + c, valid, wv[n]);
            if constexpr (RESIDUAL) load8<T, VEC>(res + c, valid, rv[n]);
        }
    }
    // Keep the weight loads in flight with the row's: without this the
    // compiler sinks them past the reduction, a second memory round trip.
#pragma unroll
    for (int n = 0; n < NV; ++n)
#pragma unroll
        for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(wv[n][i]));
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        if constexpr (RESIDUAL) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[n][i] = rnd<T>(v[n][i] + rv[n][i]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += v[n][i] * v[n][i];
    }
    ss = wave_sum(ss);
    if constexpr (TPR > 64) {
        __shared__ float partial[4];
        if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
        __syncthreads();
        ss = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    }
    if (!active) return;
    const float inv = rsqrtf(ss * (1.0f / float(width)) + eps);

    T* dst = out + row * int64_t(width);
    T* rdst = RESIDUAL ? residual_out + row * int64_t(width) : nullptr;
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        const int c = (n * TPR + t) * 8;
        const int valid = min(8, width - c);
        if (valid <= 0) continue;
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = rnd<T>(rnd<T>(v[n][i] * inv) * wv[n][i]);
        store8<T, VEC>(dst + c, valid, y);
        if constexpr (RESIDUAL) store8<T, VEC>(rdst + c, valid, v[n]);
    }
}

// Wide rows that do not fit in registers: two passes over the (cached) row.
template <typename T, bool RESIDUAL>
__global__ void __launch_bounds__(256)
rms_norm_wide_kernel(const T* __restrict__ x, int64_t rows, int64_t heads,
                     int width, int64_t token_stride, int64_t head_stride,
                     const T* __restrict__ weight, const T* __restrict__ residual,
                     int64_t residual_stride, T* __restrict__ out,
                     T* __restrict__ residual_out, float eps) {
    const int64_t row = blockIdx.x;
    const int64_t tok = row / heads;
    const T* src = x + tok * token_stride + (row - tok * heads) * head_stride;
    const T* res = RESIDUAL ? residual + tok * residual_stride : nullptr;
    float ss = 0.f;
    for (int c = threadIdx.x; c < width; c += 256) {
        float a = to_f<T>(src[c]);
        if constexpr (RESIDUAL) a = rnd<T>(a + to_f<T>(res[c]));
        ss += a * a;
    }
    ss = wave_sum(ss);
    __shared__ float partial[4];
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    const float inv = rsqrtf(ss * (1.0f / float(width)) + eps);
    for (int c = threadIdx.x; c < width; c += 256) {
        float a = to_f<T>(src[c]);
        if constexpr (RESIDUAL) {
            a = rnd<T>(a + to_f<T>(res[c]));
            residual_out[row * width + c] = static_cast<T>(a);
        }
        out[row * width + c] =
            static_cast<T>(rnd<T>(a * inv) * to_f<T>(weight[c]));
    }
}

template <typename T, bool RESIDUAL>
int launch_rms(const void* x, int64_t rows, int64_t heads, int width,
               int64_t ts, int64_t hs, const void* w, const void* res,
               int64_t rs, void* out, void* rout, float eps, hipStream_t s) {
    const T* xp = static_cast<const T*>(x);
    const T* wp = static_cast<const T*>(w);
    const T* rp = static_cast<const T*>(res);
    T* op = static_cast<T*>(out);
    T* rop = static_cast<T*>(rout);
    const bool vec = sizeof(T) == 2 && width % 8 == 0 && ts % 8 == 0 &&
                     hs % 8 == 0 && (!RESIDUAL || rs % 8 == 0) && aligned16(x) &&
                     aligned16(w) && aligned16(out) &&
                     (!RESIDUAL || (aligned16(res) && aligned16(rout)));
    const int chunks = (width + 7) / 8;
#define TVLLM_RMS(TPR, NV, V)                                                   \
    rms_norm_kernel<T, TPR, NV, RESIDUAL, V>                                    \
        <<<int((rows + 256 / TPR - 1) / (256 / TPR)), 256, 0, s>>>(              \
            xp, rows, heads, width, ts, hs, wp, rp, rs, op, rop, eps)
#define TVLLM_RMS_V(TPR, NV) \
    do { if (vec) TVLLM_RMS(TPR, NV, true); else TVLLM_RMS(TPR, NV, false); } while (0)
    if (chunks <= 64) TVLLM_RMS_V(64, 1);
    else if (chunks <= 128) TVLLM_RMS_V(64, 2);
    else if (chunks <= 256) TVLLM_RMS_V(256, 1);
    else if (chunks <= 512) TVLLM_RMS_V(256, 2);
    else if (chunks <= 1024) TVLLM_RMS_V(256, 4);
    else
        rms_norm_wide_kernel<T, RESIDUAL><<<int(rows), 256, 0, s>>>(
            xp, rows, heads, width, ts, hs, wp, rp, rs, op, rop, eps);
#undef TVLLM_RMS_V
#undef TVLLM_RMS
    return launch_status(RESIDUAL ? "add_rms_norm" : "rms_norm");
}

// add+RMSNorm whose x is the sum of fp32 split-K partial products
// (partials[p][row][c], p < nparts): x = round(sum_p partials), then exactly
// the add+RMSNorm above. One 256-thread workgroup per row; NV chunks of 8.
// NP > 0 fixes the partial count at compile time so that every load of a
// thread is in flight at once (the sum order stays p = 0, 1, ...).
template <typename T, int NV, int NP>
__global__ void __launch_bounds__(256)
add_rms_norm_partials_kernel(const float* __restrict__ parts, int nparts,
                             int64_t part_stride, int width,
                             const T* __restrict__ weight,
                             const T* __restrict__ residual,
                             int64_t residual_stride, T* __restrict__ out,
                             T* __restrict__ residual_out, float eps) {
    const int64_t row = blockIdx.x;
    const int t = threadIdx.x;
    float v[NV][8], wv[NV][8], rv[NV][8];
    float acc[NV][8];
    float ss = 0.f;
    // Every load of the thread is issued before any is used (out-of-range
    // chunks read chunk 0 and are masked).
    constexpr int NPP = NP > 0 ? NP : 1;
    float4 pa[NV][NPP][2];
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        const int c = (n * 256 + t) * 8;
        const bool ok = c < width;  // width % 8 == 0 (checked on the host)
        const float* src = parts + row * int64_t(width) + (ok ? c : 0);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[n][i] = 0.f;
        if constexpr (NP > 0) {
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                pa[n][p][0] = *reinterpret_cast<const float4*>(src + p * part_stride);
                pa[n][p][1] = *reinterpret_cast<const float4*>(src + p * part_stride + 4);
            }
        } else {
            for (int p = 0; p < nparts; ++p) {
                const float4 a = *reinterpret_cast<const float4*>(src + p * part_stride);
                const float4 b = *reinterpret_cast<const float4*>(src + p * part_stride + 4);
                acc[n][0] += a.x; acc[n][1] += a.y; acc[n][2] += a.z; acc[n][3] += a.w;
                acc[n][4] += b.x; acc[n][5] += b.y; acc[n][6] += b.z; acc[n][7] += b.w;
            }
        }
        load8_masked<T>(weight, c, ok, wv[n]);
        load8_masked<T>(residual + row * residual_stride, c, ok, rv[n]);
    }
    if constexpr (NP > 0) {
        // Materialise the partials here: the compiler would otherwise move
        // part of their loads under the chunk's range check, after the rest.
#pragma unroll
        for (int n = 0; n < NV; ++n)
#pragma unroll
            for (int p = 0; p < NP; ++p)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    asm volatile("" : "+v"(pa[n][p][h].x), "+v"(pa[n][p][h].y),
                                 "+v"(pa[n][p][h].z), "+v"(pa[n][p][h].w));
#pragma unroll
        for (int n = 0; n < NV; ++n)
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                acc[n][0] += pa[n][p][0].x; acc[n][1] += pa[n][p][0].y;
                acc[n][2] += pa[n][p][0].z; acc[n][3] += pa[n][p][0].w;
                acc[n][4] += pa[n][p][1].x; acc[n][5] += pa[n][p][1].y;
                acc[n][6] += pa[n][p][1].z; acc[n][7] += pa[n][p][1].w;
            }
    }
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        const bool ok = (n * 256 + t) * 8 < width;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[n][i] = ok ? rnd<T>(rnd<T>(acc[n][i]) + rv[n][i]) : 0.f;
            ss += v[n][i] * v[n][i];
        }
    }
    ss = wave_sum(ss);
    __shared__ float partial[4];
    if ((t & 63) == 0) partial[t >> 6] = ss;
    __syncthreads();
    ss = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    const float inv = rsqrtf(ss * (1.0f / float(width)) + eps);
#pragma unroll
    for (int n = 0; n < NV; ++n) {
        const int c = (n * 256 + t) * 8;
        if (c >= width) continue;
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = rnd<T>(rnd<T>(v[n][i] * inv) * wv[n][i]);
        store8<T, true>(out + row * int64_t(width) + c, 8, y);
        store8<T, true>(residual_out + row * int64_t(width) + c, 8, v[n]);
    }
}

// --------------------------------------------------------- SiLU * up ----

// NARROW: rows * chunks_per_row < 2^32, so the index splits in 32 bits.
template <typename T, bool VEC, bool NARROW>
__global__ void __launch_bounds__(256)
silu_mul_kernel(const T* __restrict__ x, int64_t rows, int64_t heads, int half,
                int64_t token_stride, int64_t head_stride, T* __restrict__ out,
                int chunks_per_row) {
    const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int64_t row = NARROW ? int64_t(uint32_t(idx) / uint32_t(chunks_per_row))
                               : idx / chunks_per_row;
    if (row >= rows) return;
    const int c = int(idx - row * chunks_per_row) * 8;
    const int valid = min(8, half - c);
    const int64_t tok = NARROW ? int64_t(uint32_t(row) / uint32_t(heads)) : row / heads;
    const T* src = x + tok * token_stride + (row - tok * heads) * head_stride;
    float g[8], u[8], y[8];
    if constexpr (VEC && sizeof(T) == 2) {  // half % 8 == 0: c + 8 <= half
        load8_masked<T>(src, c, true, g);
        load8_masked<T>(src + half, c, true, u);
    } else {
        load8<T, VEC>(src + c, valid, g);
        load8<T, VEC>(src + half + c, valid, u);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float act = rnd<T>(g[i] / (1.0f + expf(-g[i])));
        y[i] = act * u[i];
    }
    store8<T, VEC>(out + row * int64_t(half) + c, valid, y);
}

// ------------------------------------------------- QK norm + RoPE + KV ----

// One wave per (token, head) row. Rows [0, T*Hq) are query heads, rows
// [T*Hq, T*(Hq+Hkv)) key heads; a key-row wave also copies the matching V
// row into the cache when the KV write is fused. Lane l owns the rotation
// pairs (d, d + D/2) for d = l, l + 64, ...; NP pairs per lane. F8: the
// cache holds FP8 E4M3 bytes, x -> fp8(clamp(round_T(x) * inv_scale)).
template <typename T, int NP, bool F8>
__global__ void __launch_bounds__(256)
qk_norm_rope_kernel(const T* __restrict__ q, int64_t qts, int64_t qhs,
                    const T* __restrict__ k, int64_t kts, int64_t khs,
                    const T* __restrict__ qw, const T* __restrict__ kw,
                    const T* __restrict__ cos_t, const T* __restrict__ sin_t,
                    int64_t tokens, int heads, int kv_heads, int head_dim,
                    float q_eps, float k_eps, T* __restrict__ q_out,
                    T* __restrict__ k_out, const T* __restrict__ v, int64_t vts,
                    int64_t vhs, void* __restrict__ key_cache,
                    void* __restrict__ value_cache, int64_t css, int64_t chs,
                    const int64_t* __restrict__ slots, float k_inv, float v_inv) {
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t q_rows = tokens * heads;
    if (row >= q_rows + tokens * kv_heads) return;

    const bool is_q = row < q_rows;
    const int64_t r = is_q ? row : row - q_rows;
    const int nh = is_q ? heads : kv_heads;
    const int64_t tok = r / nh;
    const int h = int(r - tok * nh);
    const T* src = is_q ? q + tok * qts + h * qhs : k + tok * kts + h * khs;
    const T* w = is_q ? qw : kw;
    const float eps = is_q ? q_eps : k_eps;
    const int half = head_dim / 2;

    // Row, weights and RoPE angles are all loaded before the reduction.
    float x1[NP], x2[NP], w1[NP], w2[NP], cs[NP], sn[NP];
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int d = lane + 64 * p;
        const bool ok = d < half;
        const int dd = ok ? d : 0;  // unconditional loads: all in flight at once
        const float a1 = to_f<T>(src[dd]), a2 = to_f<T>(src[dd + half]);
        const float b1 = to_f<T>(w[dd]), b2 = to_f<T>(w[dd + half]);
        const float c1 = to_f<T>(cos_t[tok * half + dd]);
        const float s1 = to_f<T>(sin_t[tok * half + dd]);
        x1[p] = ok ? a1 : 0.f;
        x2[p] = ok ? a2 : 0.f;
        w1[p] = ok ? b1 : 0.f;
        w2[p] = ok ? b2 : 0.f;
        cs[p] = ok ? c1 : 0.f;
        sn[p] = ok ? s1 : 0.f;
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        asm volatile("" : "+v"(w1[p]), "+v"(w2[p]), "+v"(cs[p]), "+v"(sn[p]));
        ss += x1[p] * x1[p];
        ss += x2[p] * x2[p];
    }
    ss = wave_sum(ss);
    const float inv = rsqrtf(ss * (1.0f / float(head_dim)) + eps);

    int64_t slot = -1;
    T* dst = nullptr;
    uint8_t* dst8 = nullptr;  // FP8 cache row
    if (is_q) {
        dst = q_out + r * head_dim;
    } else if (key_cache != nullptr) {
        slot = slots[tok];
        if (slot >= 0) {
            const int64_t off = slot * css + h * chs;
            if constexpr (F8) dst8 = static_cast<uint8_t*>(key_cache) + off;
            else dst = static_cast<T*>(key_cache) + off;
        }
    } else {
        dst = k_out + r * head_dim;
    }
    // With the fused write, a dense K copy is still produced if requested.
    T* dense_k = (!is_q && key_cache != nullptr && k_out != nullptr)
                     ? k_out + r * head_dim : nullptr;

#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int d = lane + 64 * p;
        if (d >= half) continue;
        const float n1 = rnd<T>(rnd<T>(x1[p] * inv) * w1[p]);
        const float n2 = rnd<T>(rnd<T>(x2[p] * inv) * w2[p]);
        const float c = cs[p];
        const float s = sn[p];
        const float o1 = rnd<T>(n1 * c) - rnd<T>(n2 * s);
        const float o2 = rnd<T>(n2 * c) + rnd<T>(n1 * s);
        if (dst != nullptr) {
            dst[d] = static_cast<T>(o1);
            dst[d + half] = static_cast<T>(o2);
        }
        if constexpr (F8) {
            if (dst8 != nullptr) {
                const uint32_t b = fp8x4_pack(rnd<T>(o1) * k_inv, rnd<T>(o2) * k_inv, 0.f, 0.f);
                dst8[d] = uint8_t(b);
                dst8[d + half] = uint8_t(b >> 8);
            }
        }
        if (dense_k != nullptr) {
            dense_k[d] = static_cast<T>(o1);
            dense_k[d + half] = static_cast<T>(o2);
        }
    }

    if (!is_q && key_cache != nullptr && slot >= 0) {
        const T* vsrc = v + tok * vts + h * vhs;
        const int64_t off = slot * css + h * chs;
        if constexpr (F8) {
            uint8_t* vdst = static_cast<uint8_t*>(value_cache) + off;
            for (int d = lane; d < head_dim; d += 64)
                vdst[d] = uint8_t(fp8x4_pack(to_f<T>(vsrc[d]) * v_inv, 0.f, 0.f, 0.f));
        } else {
            T* vdst = static_cast<T*>(value_cache) + off;
            for (int d = lane; d < head_dim; d += 64) vdst[d] = vsrc[d];
        }
    }
}

// head_dim 128 with 8-byte aligned rows: 16 lanes per (token, head) row,
// four rows per wave. Lane j owns the rotation pairs (d, d + 64) for
// d = 4j .. 4j+3, so every load and store moves 4 elements. The sum of
// squares reproduces the one-pair-per-lane kernel's butterfly exactly: the
// steps across lanes d ^ 32 .. d ^ 4 are shuffles across lanes j ^ 8 .. j ^ 1
// of the same pair index, the steps d ^ 2 and d ^ 1 adds within a lane, so
// every addition pairs the same two partial sums (the results, including
// the fused KV write, are bit-identical to that kernel and to the decode
// kernel's fused write).
template <typename T, bool F8>
__global__ void __launch_bounds__(256)
qk_norm_rope_d128(const T* __restrict__ q, int64_t qts, int64_t qhs,
                  const T* __restrict__ k, int64_t kts, int64_t khs,
                  const T* __restrict__ qw, const T* __restrict__ kw,
                  const T* __restrict__ cos_t, const T* __restrict__ sin_t,
                  int64_t tokens, int heads, int kv_heads, float q_eps, float k_eps,
                  T* __restrict__ q_out, T* __restrict__ k_out, const T* __restrict__ v,
                  int64_t vts, int64_t vhs, void* __restrict__ key_cache,
                  void* __restrict__ value_cache, int64_t css, int64_t chs,
                  const int64_t* __restrict__ slots, float k_inv, float v_inv) {
    constexpr int D = 128, H = 64;
    const int j = threadIdx.x & 15;
    const int64_t row = int64_t(blockIdx.x) * 16 + (threadIdx.x >> 4);
    const int64_t q_rows = tokens * heads;
    if (row >= q_rows + tokens * kv_heads) return;  // whole 16-lane groups

    const bool is_q = row < q_rows;
    const int64_t r = is_q ? row : row - q_rows;
    const int nh = is_q ? heads : kv_heads;
    const int64_t tok = r / nh;
    const int h = int(r - tok * nh);
    const T* src = is_q ? q + tok * qts + h * qhs : k + tok * kts + h * khs;
    const T* w = is_q ? qw : kw;
    const float eps = is_q ? q_eps : k_eps;

    auto load4 = [](const T* p, float (&x)[4]) {
        const uint2 u = *reinterpret_cast<const uint2*>(p);
        x[0] = half_lo<T>(u.x);
        x[1] = half_hi<T>(u.x);
        x[2] = half_lo<T>(u.y);
        x[3] = half_hi<T>(u.y);
    };
    float x1[4], x2[4], w1[4], w2[4], cs[4], sn[4];
    load4(src + 4 * j, x1);
    load4(src + H + 4 * j, x2);
    load4(w + 4 * j, w1);
    load4(w + H + 4 * j, w2);
    load4(cos_t + tok * H + 4 * j, cs);
    load4(sin_t + tok * H + 4 * j, sn);
    int64_t slot = -1;
    if (!is_q && key_cache != nullptr) slot = slots[tok];

    float ss[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) ss[t] = x1[t] * x1[t] + x2[t] * x2[t];
#pragma unroll
    for (int off = 8; off > 0; off >>= 1)  // pair distance 4 * off
#pragma unroll
        for (int t = 0; t < 4; ++t) ss[t] += __shfl_xor(ss[t], off, 64);
    float s2[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) s2[t] = ss[t] + ss[t ^ 2];  // distance 2
    const float total = s2[0] + s2[1];                      // distance 1
    const float inv = rsqrtf(total * (1.0f / float(D)) + eps);

    float o1[4], o2[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const float n1 = rnd<T>(rnd<T>(x1[t] * inv) * w1[t]);
        const float n2 = rnd<T>(rnd<T>(x2[t] * inv) * w2[t]);
        o1[t] = rnd<T>(rnd<T>(n1 * cs[t]) - rnd<T>(n2 * sn[t]));
        o2[t] = rnd<T>(rnd<T>(n2 * cs[t]) + rnd<T>(n1 * sn[t]));
    }
    auto store4 = [](T* p, const float (&x)[4]) {
        uint2 u;
        u.x = pack2<T>(x[0], x[1]);
        u.y = pack2<T>(x[2], x[3]);
        *reinterpret_cast<uint2*>(p) = u;
    };
    if (is_q) {
        T* dst = q_out + r * D;
        store4(dst + 4 * j, o1);
        store4(dst + H + 4 * j, o2);
        return;
    }
    if (key_cache == nullptr || k_out != nullptr) {  // the dense K rows
        T* dst = k_out + r * D;
        store4(dst + 4 * j, o1);
        store4(dst + H + 4 * j, o2);
    }
    if (key_cache == nullptr || slot < 0) return;
    const int64_t off = slot * css + h * chs;
    const T* vsrc = v + tok * vts + h * vhs + 8 * j;
    const uint2 va = *reinterpret_cast<const uint2*>(vsrc);
    const uint2 vb = *reinterpret_cast<const uint2*>(vsrc + 4);
    if constexpr (F8) {
        uint8_t* kd = static_cast<uint8_t*>(key_cache) + off;
        *reinterpret_cast<uint32_t*>(kd + 4 * j) =
            fp8x4_pack(o1[0] * k_inv, o1[1] * k_inv, o1[2] * k_inv, o1[3] * k_inv);
        *reinterpret_cast<uint32_t*>(kd + H + 4 * j) =
            fp8x4_pack(o2[0] * k_inv, o2[1] * k_inv, o2[2] * k_inv, o2[3] * k_inv);
        uint2 vq;
        vq.x = fp8x4_pack(half_lo<T>(va.x) * v_inv, half_hi<T>(va.x) * v_inv,
                          half_lo<T>(va.y) * v_inv, half_hi<T>(va.y) * v_inv);
        vq.y = fp8x4_pack(half_lo<T>(vb.x) * v_inv, half_hi<T>(vb.x) * v_inv,
                          half_lo<T>(vb.y) * v_inv, half_hi<T>(vb.y) * v_inv);
        *reinterpret_cast<uint2*>(static_cast<uint8_t*>(value_cache) + off + 8 * j) = vq;
    } else {
        T* kd = static_cast<T*>(key_cache) + off;
        store4(kd + 4 * j, o1);
        store4(kd + H + 4 * j, o2);
        T* vd = static_cast<T*>(value_cache) + off + 8 * j;
        *reinterpret_cast<uint2*>(vd) = va;
        *reinterpret_cast<uint2*>(vd + 4) = vb;
    }
}

}  // namespace
}  // namespace tvllm

using namespace tvllm;

extern "C" int tvllm_rms_norm(const void* input, int64_t tokens, int64_t heads,
                              int64_t width, int64_t token_stride,
                              int64_t head_stride, const void* weight,
                              const void* residual, int64_t residual_stride,
                              void* out, void* residual_out, float eps, int dtype,
                              tvllm_stream_t stream) {
    TVLLM_CHECK(tokens >= 0 && heads > 0 && width > 0,
                "rms_norm: rows must have positive width");
    TVLLM_CHECK(width <= INT32_MAX - 127 && tokens * heads <= INT32_MAX,
                "rms_norm: RMSNorm dimensions exceed index range");
    TVLLM_CHECK(residual == nullptr || heads == 1,
                "add_rms_norm: residual requires a 2D input");
    TVLLM_CHECK(residual == nullptr || residual_out != nullptr,
                "add_rms_norm: residual_out is required");
    const int64_t rows = tokens * heads;
    if (rows == 0) return TVLLM_OK;
    TVLLM_CHECK(input && weight && out, "rms_norm: null pointer");
    hipStream_t s = as_hip(stream);
    return dispatch_float(dtype, [&]<int DT>() {
        using T = typename Elem<DT>::T;
        if (residual)
            return launch_rms<T, true>(input, rows, heads, int(width), token_stride,
                                       head_stride, weight, residual,
                                       residual_stride, out, residual_out, eps, s);
        return launch_rms<T, false>(input, rows, heads, int(width), token_stride,
                                    head_stride, weight, nullptr, 0, out, nullptr,
                                    eps, s);
    });
}

extern "C" int tvllm_add_rms_norm_partials(
    const float* partials, int64_t num_partials, int64_t partial_stride,
    int64_t tokens, int64_t width, const void* weight, const void* residual,
    int64_t residual_stride, void* out, void* residual_out, float eps, int dtype,
    tvllm_stream_t stream) {
    TVLLM_CHECK(tokens >= 0 && width > 0 && width % 8 == 0 && width <= 8 * 256 * 4,
                "add_rms_norm_partials: width must be a multiple of 8, at most 8192");
    TVLLM_CHECK(num_partials >= 1 && num_partials <= 64,
                "add_rms_norm_partials: 1..64 partial products");
    TVLLM_CHECK(tokens <= INT32_MAX, "add_rms_norm_partials: too many rows");
    if (tokens == 0) return TVLLM_OK;
    TVLLM_CHECK(partials && weight && residual && out && residual_out,
                "add_rms_norm_partials: null pointer");
    TVLLM_CHECK(partial_stride >= tokens * width && partial_stride % 4 == 0 &&
                    aligned16(partials) && residual_stride % 8 == 0 && aligned16(weight) &&
                    aligned16(residual) && aligned16(out) && aligned16(residual_out),
                "add_rms_norm_partials: operands must be 16-byte aligned dense rows");
    hipStream_t s = as_hip(stream);
    return dispatch_half(dtype, [&]<int DT>() {
        using T = typename Elem<DT>::T;
        const T* wp = static_cast<const T*>(weight);
        const T* rp = static_cast<const T*>(residual);
        T* op = static_cast<T*>(out);
        T* rop = static_cast<T*>(residual_out);
        const int np = int(num_partials), w = int(width);
        auto go = [&]<int NV>() {
#define TVLLM_PARTS(NP)                                                            \
    add_rms_norm_partials_kernel<T, NV, NP><<<int(tokens), 256, 0, s>>>(           \
        partials, np, partial_stride, w, wp, rp, residual_stride, op, rop, eps)
            if (np == 4) TVLLM_PARTS(4);
            else if (np == 8) TVLLM_PARTS(8);
            else if (np == 2) TVLLM_PARTS(2);
            else TVLLM_PARTS(0);
#undef TVLLM_PARTS
        };
        if (width <= 2048) go.template operator()<1>();
        else if (width <= 4096) go.template operator()<2>();
        else go.template operator()<4>();
        return launch_status("add_rms_norm_partials");
    });
}

extern "C" int tvllm_silu_and_mul(const void* input, int64_t tokens,
                                  int64_t heads, int64_t width,
                                  int64_t token_stride, int64_t head_stride,
                                  void* out, int dtype, tvllm_stream_t stream) {
    TVLLM_CHECK(tokens >= 0 && heads > 0 && width > 0,
                "silu_and_mul: rows must have positive width");
    TVLLM_CHECK(width % 2 == 0, "silu_and_mul: SiLU input width must be even");
    TVLLM_CHECK(width <= INT32_MAX - 16, "silu_and_mul: width too large");
    const int64_t rows = tokens * heads;
    if (rows == 0) return TVLLM_OK;
    TVLLM_CHECK(input && out, "silu_and_mul: null pointer");
    const int half = int(width / 2);
    const int chunks = (half + 7) / 8;
    const int64_t total = rows * chunks;
    TVLLM_CHECK((total + 255) / 256 <= INT32_MAX, "silu_and_mul: too many rows");
    hipStream_t s = as_hip(stream);
    return dispatch_float(dtype, [&]<int DT>() {
        using T = typename Elem<DT>::T;
        const bool vec = sizeof(T) == 2 && half % 8 == 0 && token_stride % 8 == 0 &&
                         head_stride % 8 == 0 && aligned16(input) && aligned16(out);
        const int blocks = int((total + 255) / 256);
        const bool narrow = int64_t(blocks) * 256 <= int64_t(UINT32_MAX);
        auto go = [&]<bool V, bool N>() {
            silu_mul_kernel<T, V, N><<<blocks, 256, 0, s>>>(
                static_cast<const T*>(input), rows, heads, half, token_stride,
                head_stride, static_cast<T*>(out), chunks);
        };
        if (vec && narrow) go.template operator()<true, true>();
        else if (vec) go.template operator()<true, false>();
        else if (narrow) go.template operator()<false, true>();
        else go.template operator()<false, false>();
        return launch_status("silu_and_mul");
    });
}

extern "C" int tvllm_qk_norm_rope(
    const void* q, int64_t q_token_stride, int64_t q_head_stride, const void* k,
    int64_t k_token_stride, int64_t k_head_stride, const void* q_weight,
    const void* k_weight, const void* cos, const void* sin, int64_t tokens,
    int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, float q_eps,
    float k_eps, void* q_out, void* k_out, const void* v, int64_t v_token_stride,
    int64_t v_head_stride, void* key_cache, void* value_cache,
    const int64_t* slots, int64_t num_slots, int64_t cache_slot_stride,
    int64_t cache_head_stride, int dtype, int cache_dtype, float k_scale, float v_scale,
    tvllm_stream_t stream) {
    TVLLM_CHECK(tokens >= 0 && num_heads > 0 && num_kv_heads > 0,
                "qk_norm_rope: Q/K must have positive head counts");
    const bool f8 = cache_dtype == TVLLM_FP8_E4M3;
    TVLLM_CHECK(f8 || cache_dtype == dtype,
                "qk_norm_rope: KV cache dtype must match Q/K or be FP8 E4M3");
    TVLLM_CHECK(k_scale > 0.f && v_scale > 0.f && k_scale < INFINITY && v_scale < INFINITY,
                "qk_norm_rope: KV scales must be positive and finite");
    TVLLM_CHECK(f8 || (k_scale == 1.f && v_scale == 1.f),
                "qk_norm_rope: KV scales apply to an FP8 cache only");
    TVLLM_CHECK(head_dim > 0 && head_dim % 2 == 0 && head_dim <= 1024,
                "qk_norm_rope: RoPE input must have an even head_dim <= 1024");
    TVLLM_CHECK(tokens * (num_heads + num_kv_heads) <= INT32_MAX * int64_t(4),
                "qk_norm_rope: Q/K RMSNorm dimensions exceed index range");
    const bool fused = key_cache != nullptr;
    TVLLM_CHECK(!fused || (value_cache && v && slots && key_cache != value_cache),
                "qk_norm_rope: fused KV write needs v, value_cache and slots");
    TVLLM_CHECK(fused || k_out != nullptr, "qk_norm_rope: k_out is required");
    TVLLM_CHECK(!fused || tokens <= num_slots, "qk_norm_rope: too many KV rows");
    TVLLM_CHECK(!fused || cache_layout_ok(num_slots, num_kv_heads, head_dim,
                                          cache_slot_stride, cache_head_stride),
                "qk_norm_rope: cache strides must give non-overlapping head rows");
    const int64_t css = cache_slot_stride, chs = cache_head_stride;
    const int64_t rows = tokens * (num_heads + num_kv_heads);
    if (rows == 0) return TVLLM_OK;
    TVLLM_CHECK(q && k && q_weight && k_weight && cos && sin && q_out,
                "qk_norm_rope: null pointer");
    hipStream_t s = as_hip(stream);
    const auto a8 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; };
    const bool d128 = head_dim == 128 && q_token_stride % 4 == 0 && q_head_stride % 4 == 0 &&
                      k_token_stride % 4 == 0 && k_head_stride % 4 == 0 && a8(q) && a8(k) &&
                      a8(q_weight) && a8(k_weight) && a8(cos) && a8(sin) && a8(q_out) &&
                      (k_out == nullptr || a8(k_out)) &&
                      (!fused || (v_token_stride % 4 == 0 && v_head_stride % 4 == 0 && a8(v) &&
                                  a8(key_cache) && a8(value_cache) && css % 8 == 0 &&
                                  chs % 8 == 0));
    return dispatch_half(dtype, [&]<int DT>() {
        using T = typename Elem<DT>::T;
        const int blocks = int((rows + 3) / 4);
        const int half = int(head_dim / 2);
        const float k_inv = 1.f / k_scale, v_inv = 1.f / v_scale;
        if (d128) {
            const int64_t groups = (rows + 15) / 16;
            TVLLM_CHECK(groups <= INT32_MAX, "qk_norm_rope: grid too large");
            auto go128 = [&]<bool F8>() {
                qk_norm_rope_d128<T, F8><<<int(groups), 256, 0, s>>>(
                    static_cast<const T*>(q), q_token_stride, q_head_stride,
                    static_cast<const T*>(k), k_token_stride, k_head_stride,
                    static_cast<const T*>(q_weight), static_cast<const T*>(k_weight),
                    static_cast<const T*>(cos), static_cast<const T*>(sin), tokens,
                    int(num_heads), int(num_kv_heads), q_eps, k_eps, static_cast<T*>(q_out),
                    static_cast<T*>(k_out), static_cast<const T*>(v), v_token_stride,
                    v_head_stride, key_cache, value_cache, css, chs, slots, k_inv, v_inv);
            };
            if (f8) go128.template operator()<true>();
            else go128.template operator()<false>();
            return launch_status("qk_norm_rope");
        }
        auto go = [&]<bool F8>() {
#define TVLLM_QKR(NP)                                                            \
    qk_norm_rope_kernel<T, NP, F8><<<blocks, 256, 0, s>>>(                       \
        static_cast<const T*>(q), q_token_stride, q_head_stride,                 \
        static_cast<const T*>(k), k_token_stride, k_head_stride,                 \
        static_cast<const T*>(q_weight), static_cast<const T*>(k_weight),        \
        static_cast<const T*>(cos), static_cast<const T*>(sin), tokens,          \
        int(num_heads), int(num_kv_heads), int(head_dim), q_eps, k_eps,          \
        static_cast<T*>(q_out), static_cast<T*>(k_out),                          \
        static_cast<const T*>(v), v_token_stride, v_head_stride,                 \
        key_cache, value_cache, css, chs, slots, k_inv, v_inv)
            if (half <= 64) TVLLM_QKR(1);
            else if (half <= 128) TVLLM_QKR(2);
            else if (half <= 256) TVLLM_QKR(4);
            else TVLLM_QKR(8);
#undef TVLLM_QKR
        };
        if (f8) go.template operator()<true>();
        else go.template operator()<false>();
        return launch_status("qk_norm_rope");
    });
}

// Shared helpers for the gfx950 kernels: element types, rounding helpers,
// wave64 reductions, the C-ABI error channel and launch checking.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdarg>

#include "../../include/tinyvllm_hip.h"

namespace tvllm {

// ---------------------------------------------------------------- errors --

void set_error(const char* fmt, ...);
void clear_error();

#define TVLLM_CHECK(cond, ...)                                   \
    do {                                                         \
        if (!(cond)) {                                           \
            ::tvllm::set_error(__VA_ARGS__);                     \
            return int(TVLLM_EINVAL);                            \
        }                                                        \
    } while (0)

// Reports the launch status of the kernel just enqueued. hipGetLastError is
// legal during stream capture, so this is safe inside graph capture.
inline int launch_status(const char* what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        set_error("%s: kernel launch failed: %s", what, hipGetErrorString(err));
        return int(TVLLM_ELAUNCH);
    }
    clear_error();
    return TVLLM_OK;
}

inline hipStream_t as_hip(tvllm_stream_t s) {
    return reinterpret_cast<hipStream_t>(s);
}

inline bool aligned8(const void* p) {
    return (reinterpret_cast<uintptr_t>(p) & 7u) == 0;
}

inline bool aligned16(const void* p) {
    return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

// Paged KV-cache geometry: the row of (slot, KV head) starts at element
// slot * slot_stride + head * head_stride and holds head_dim contiguous
// elements. Rows must not overlap, which holds for the two nestings:
// token-major (a slot's heads side by side: head_stride >= head_dim,
// slot_stride >= kv_heads * head_stride) and head-major (a head's slots side
// by side: slot_stride >= head_dim, head_stride >= num_slots * slot_stride).
inline bool cache_layout_ok(int64_t num_slots, int64_t kv_heads, int64_t head_dim,
                            int64_t slot_stride, int64_t head_stride) {
    if (num_slots <= 0 || kv_heads <= 0 || head_dim <= 0) return false;
    const bool token_major = head_stride >= head_dim &&
                             slot_stride / kv_heads >= head_stride;
    const bool head_major = slot_stride >= head_dim &&
                            head_stride / num_slots >= slot_stride;
    return token_major || head_major;
}

// Elements spanned by the cache (one past its last element).
inline int64_t cache_extent(int64_t num_slots, int64_t kv_heads, int64_t head_dim,
                            int64_t slot_stride, int64_t head_stride) {
    return (num_slots - 1) * slot_stride + (kv_heads - 1) * head_stride + head_dim;
}

// ------------------------------------------------------------- elements --

template <int DT> struct Elem;
template <> struct Elem<TVLLM_BF16> { using T = __bf16; };
template <> struct Elem<TVLLM_F16> { using T = _Float16; };
template <> struct Elem<TVLLM_F32> { using T = float; };

template <typename T>
__device__ __forceinline__ float to_f(T x) { return static_cast<float>(x); }

// Round a float to the storage type and back (round-to-nearest-even).
template <typename T>
__device__ __forceinline__ float rnd(float x) {
    return static_cast<float>(static_cast<T>(x));
}

// 16-byte vector of raw 16-bit elements.
struct alignas(16) U16x8 {
    uint32_t w[4];
};

template <typename T>
__device__ __forceinline__ float half_lo(uint32_t w);
template <typename T>
__device__ __forceinline__ float half_hi(uint32_t w);

template <>
__device__ __forceinline__ float half_lo<__bf16>(uint32_t w) {
    return __uint_as_float(w << 16);
}
template <>
__device__ __forceinline__ float half_hi<__bf16>(uint32_t w) {
    return __uint_as_float(w & 0xffff0000u);
}
template <>
__device__ __forceinline__ float half_lo<_Float16>(uint32_t w) {
    _Float16 h;
    uint16_t b = static_cast<uint16_t>(w & 0xffffu);
    __builtin_memcpy(&h, &b, 2);
    return static_cast<float>(h);
}
template <>
__device__ __forceinline__ float half_hi<_Float16>(uint32_t w) {
    _Float16 h;
    uint16_t b = static_cast<uint16_t>(w >> 16);
    __builtin_memcpy(&h, &b, 2);
    return static_cast<float>(h);
}

template <typename T>
__device__ __forceinline__ uint16_t bits_of(float x) {
    T v = static_cast<T>(x);
    uint16_t b;
    __builtin_memcpy(&b, &v, 2);
    return b;
}

// Two floats rounded (nearest-even) into one word; a single v_cvt_pk_* on gfx950.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef T t2_t __attribute__((ext_vector_type(2)));
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, t2_t));
}

template <typename T>
__device__ __forceinline__ void unpack8(const U16x8& v, float (&out)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = half_lo<T>(v.w[i]);
        out[2 * i + 1] = half_hi<T>(v.w[i]);
    }
}

// ------------------------------------------------------ fp8 KV cache --
// Cache rows may be stored as OCP FP8 E4M3 (max 448, no infinities) with a
// per-cache scale: stored = fp8(clamp(x * inv_scale, -448, 448)), nearest-
// even (the v_cvt_pk_fp8_f32 rounding, identical to torch's float8_e4m3fn
// cast); read back as stored * scale. Decoding an E4M3 value to f32, bf16 or
// f16 is exact.

constexpr float kFp8Max = 448.f;

__device__ __forceinline__ float fp8_clamp(float x) {
    return fminf(fmaxf(x, -kFp8Max), kFp8Max);  // NaN stays NaN
}

// Four floats (already scaled) -> four E4M3 bytes, element 0 in byte 0.
__device__ __forceinline__ uint32_t fp8x4_pack(float a, float b, float c, float d) {
    uint32_t w = __builtin_amdgcn_cvt_pk_fp8_f32(fp8_clamp(a), fp8_clamp(b), 0u, false);
    return __builtin_amdgcn_cvt_pk_fp8_f32(fp8_clamp(c), fp8_clamp(d), w, true);
}

// Eight E4M3 bytes (element 0 in the low byte of w.x) -> eight floats.
__device__ __forceinline__ void fp8x8_unpack(uint2 w, float (&out)[8]) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t a = __builtin_amdgcn_cvt_pk_f32_fp8(w.x, false);
    const f32x2_t b = __builtin_amdgcn_cvt_pk_f32_fp8(w.x, true);
    const f32x2_t c = __builtin_amdgcn_cvt_pk_f32_fp8(w.y, false);
    const f32x2_t d = __builtin_amdgcn_cvt_pk_f32_fp8(w.y, true);
    out[0] = a[0]; out[1] = a[1]; out[2] = b[0]; out[3] = b[1];
    out[4] = c[0]; out[5] = c[1]; out[6] = d[0]; out[7] = d[1];
}

// Eight E4M3 bytes -> eight 16-bit elements of type T (exact).
template <typename T>
__device__ __forceinline__ U16x8 fp8x8_widen(uint2 w) {
    U16x8 r;
    if constexpr (__is_same(T, __bf16)) {
        r.w[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, 1.f, false));
        r.w[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, 1.f, true));
        r.w[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, 1.f, false));
        r.w[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, 1.f, true));
    } else {
        r.w[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.x, 1.f, false));
        r.w[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.x, 1.f, true));
        r.w[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.y, 1.f, false));
        r.w[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w.y, 1.f, true));
    }
    return r;
}

// Eight 16-bit elements -> eight E4M3 bytes of x * inv_scale.
template <typename T>
__device__ __forceinline__ uint2 fp8x8_narrow(const U16x8& v, float inv_scale) {
    float x[8];
    unpack8<T>(v, x);
    uint2 r;
    r.x = fp8x4_pack(x[0] * inv_scale, x[1] * inv_scale, x[2] * inv_scale, x[3] * inv_scale);
    r.y = fp8x4_pack(x[4] * inv_scale, x[5] * inv_scale, x[6] * inv_scale, x[7] * inv_scale);
    return r;
}

// ------------------------------------------------------- wave64 reduces --

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Dispatch helper: calls f.template operator()<DT>() for the runtime dtype.
template <typename F>
int dispatch_half(int dtype, F&& f) {
    switch (dtype) {
        case TVLLM_BF16: return f.template operator()<TVLLM_BF16>();
        case TVLLM_F16: return f.template operator()<TVLLM_F16>();
        default:
            set_error("dtype %d not supported (expected bf16 or fp16)", dtype);
            return int(TVLLM_EINVAL);
    }
}

template <typename F>
int dispatch_float(int dtype, F&& f) {
    switch (dtype) {
        case TVLLM_BF16: return f.template operator()<TVLLM_BF16>();
        case TVLLM_F16: return f.template operator()<TVLLM_F16>();
        case TVLLM_F32: return f.template operator()<TVLLM_F32>();
        default:
            set_error("dtype %d not supported", dtype);
            return int(TVLLM_EINVAL);
    }
}

}  // namespace tvllm

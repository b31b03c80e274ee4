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

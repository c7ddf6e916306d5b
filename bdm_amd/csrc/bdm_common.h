// Shared helpers for the gfx950 BDM kernels: element conversion, error
// reporting and launch checks.  Device code only targets CDNA4 (wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/bdm_hip.h"

namespace bdm {

constexpr int kWave = 64;

// ---------------------------------------------------------------- elements
// BF16 is carried as its 16-bit pattern.  (__bf16)x lowers to the gfx950
// v_cvt_pk_bf16_f32 instruction, which rounds to nearest even like torch.
struct bf16_t {
    uint16_t bits;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float(uint32_t(x.bits) << 16); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
    __bf16 b = (__bf16)x;
    return bf16_t{__builtin_bit_cast(uint16_t, b)};
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// x rounded to BF16 (nearest even) and widened back to FP32 by one
// v_cvt_pk_bf16_f32 with a zero low operand: the high half of its result is
// bf16(x) and the low half bf16(0) = 0, so the 32 bits are the widened value.
__device__ __forceinline__ float round_bf16(float x) {
    const f32x2_t f = {0.f, x};
    return __builtin_bit_cast(float, __builtin_convertvector(f, bf16x2_t));
}

// Round an FP32 value to the storage type T and widen it back.
template <typename T> __device__ __forceinline__ float round_to(float x) { return to_f32(from_f32<T>(x)); }
template <> __device__ __forceinline__ float round_to<bf16_t>(float x) { return round_bf16(x); }

// Round two values to T and widen them back (one conversion each: cheaper
// than one packed conversion and two instructions to unpack it).
template <typename T> __device__ __forceinline__ void round_pair(float &a, float &b);
template <> __device__ __forceinline__ void round_pair<float>(float &, float &) {}
template <> __device__ __forceinline__ void round_pair<bf16_t>(float &a, float &b) {
    a = round_bf16(a);
    b = round_bf16(b);
}

// Load `N` consecutive elements of T starting at p (16-byte aligned when the
// caller's layout guarantees it) and widen them to FP32.
template <int N>
__device__ __forceinline__ void load_row(const bf16_t *p, float (&out)[N]) {
    static_assert(N % 2 == 0 || N == 1, "row width");
    if constexpr (N % 8 == 0) {
#pragma unroll
        for (int i = 0; i < N / 8; ++i) {
            uint4 u = reinterpret_cast<const uint4 *>(p)[i];
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                out[8 * i + 2 * j] = __uint_as_float(w[j] << 16);
                out[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
            }
        }
    } else if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            uint2 u = reinterpret_cast<const uint2 *>(p)[i];
            out[4 * i] = __uint_as_float(u.x << 16);
            out[4 * i + 1] = __uint_as_float(u.x & 0xffff0000u);
            out[4 * i + 2] = __uint_as_float(u.y << 16);
            out[4 * i + 3] = __uint_as_float(u.y & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) out[i] = to_f32(p[i]);
    }
}

template <int N>
__device__ __forceinline__ void load_row(const float *p, float (&out)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            float4 u = reinterpret_cast<const float4 *>(p)[i];
            out[4 * i] = u.x;
            out[4 * i + 1] = u.y;
            out[4 * i + 2] = u.z;
            out[4 * i + 3] = u.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) out[i] = p[i];
    }
}

// Two FP32 values rounded to BF16 (nearest even) and packed, low half first,
// with one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2_t f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

template <int N>
__device__ __forceinline__ void store_row(bf16_t *p, const float (&in)[N]) {
    if constexpr (N % 8 == 0) {
#pragma unroll
        for (int i = 0; i < N / 8; ++i) {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2(in[8 * i + 2 * j], in[8 * i + 2 * j + 1]);
            reinterpret_cast<uint4 *>(p)[i] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    } else if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i)
            reinterpret_cast<uint2 *>(p)[i] =
                make_uint2(pack_bf16x2(in[4 * i], in[4 * i + 1]), pack_bf16x2(in[4 * i + 2], in[4 * i + 3]));
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) p[i] = from_f32<bf16_t>(in[i]);
    }
}

template <int N>
__device__ __forceinline__ void store_row(float *p, const float (&in)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i)
            reinterpret_cast<float4 *>(p)[i] = make_float4(in[4 * i], in[4 * i + 1], in[4 * i + 2], in[4 * i + 3]);
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) p[i] = in[i];
    }
}

// ---------------------------------------------------------------- errors
void set_error(const char *fmt, ...);
int fail(int code, const char *fmt, ...);
int check_launch(const char *what);

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void *p, size_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

}  // namespace bdm

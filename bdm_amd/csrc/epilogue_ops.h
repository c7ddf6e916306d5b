// Device helpers shared by the elementwise epilogues (epilogue.hip) and the
// decode-step GEMV's prologues (gemv.hip), so a fused prologue rounds and
// sums exactly as the standalone kernel it replaces.
#pragma once

#include "bdm_common.h"

namespace bdm {

// silu and sigmoid with the hardware exp and reciprocal (v_exp_f32,
// v_rcp_f32): a few FP32 ulps, below the BF16 rounding every result gets
__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
__device__ __forceinline__ float silu_f(float x) { return x * sigmoid_f(x); }
// F.softplus with beta 1 and threshold 20
__device__ __forceinline__ float softplus_f(float x) { return x > 20.f ? x : log1pf(expf(x)); }

// The shell's SwiGLU element: round(round(silu(a)) * b) in T, silu evaluated
// as x / (1 + exp(-x)) with IEEE division, as torch does.
template <typename T>
__device__ __forceinline__ float swiglu_value(float a, float b) {
    return round_to<T>(round_to<T>(a / (1.f + expf(-a))) * b);
}

__device__ __forceinline__ float param_at(const void *p, int dtype, int64_t i) {
    return dtype == BDM_BF16 ? to_f32(static_cast<const bf16_t *>(p)[i]) : static_cast<const float *>(p)[i];
}

// Eight consecutive elements of T (FP32 or BF16 parameters given by dtype
// for param8) widened to FP32: 16-byte vector loads when VEC (the caller
// checked 16-byte alignment of every such group), element loads otherwise.
template <typename T, bool VEC>
__device__ __forceinline__ void load8(const T *p, float (&x)[8]) {
    if constexpr (VEC && sizeof(T) == 2) {
        const uint4 r = *reinterpret_cast<const uint4 *>(p);
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            x[2 * q] = __uint_as_float(w[q] << 16);
            x[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
        }
    } else if constexpr (VEC) {
        const float4 a = *reinterpret_cast<const float4 *>(p), b = *reinterpret_cast<const float4 *>(p + 4);
        x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = to_f32(p[j]);
    }
}

template <bool VEC>
__device__ __forceinline__ void param8(const void *p, int dtype, int64_t at, float (&x)[8]) {
    if (dtype == BDM_BF16)
        load8<bf16_t, VEC>(static_cast<const bf16_t *>(p) + at, x);
    else
        load8<float, VEC>(static_cast<const float *>(p) + at, x);
}

// One head's controller rows (heads.py:11-22), from the projection outputs;
// every value here is what the controller epilogue stores (the caller rounds
// q, k and b to the controller dtype as the store does; g stays FP32).
// q or k: silu rounded to T, then the l2 normalization over the S values
// (qk_norm 1: x * rsqrt(sum x^2 + 1e-6); 0: x / max(|x|_2, 1e-12)).
template <typename T, int S, bool VEC>
__device__ __forceinline__ void qk_row(const T *src, int qk_norm, float (&y)[S]) {
    float x[S], ss = 0.f;
#pragma unroll
    for (int r0 = 0; r0 < S; r0 += 8) {
        float t[8];
        load8<T, VEC>(src + r0, t);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            x[r0 + j] = round_to<T>(silu_f(t[j]));
            ss = fmaf(x[r0 + j], x[r0 + j], ss);
        }
    }
    const float inv = qk_norm == 1 ? rsqrtf(ss + 1e-6f) : 0.f;
    const float norm = fmaxf(sqrtf(ss), 1e-12f);
#pragma unroll
    for (int r = 0; r < S; ++r) y[r] = qk_norm == 1 ? x[r] * inv : x[r] / norm;
}

// b: sigmoid of the projection
template <typename T, int S, bool VEC>
__device__ __forceinline__ void sigmoid_row(const T *src, float (&y)[S]) {
#pragma unroll
    for (int r0 = 0; r0 < S; r0 += 8) {
        float t[8];
        load8<T, VEC>(src + r0, t);
#pragma unroll
        for (int j = 0; j < 8; ++j) y[r0 + j] = sigmoid_f(t[j]);
    }
}

// g = -exp(A_log[h]) * softplus(f + dt_bias) in FP32 for head h
template <typename T, int S, bool VEC>
__device__ __forceinline__ void decay_row(const T *f, const void *a_log, const void *dt_bias, int param_dtype, int h,
                                          float (&y)[S]) {
    const float a = -expf(param_at(a_log, param_dtype, h));
#pragma unroll
    for (int r0 = 0; r0 < S; r0 += 8) {
        float t[8], bias[8];
        load8<T, VEC>(f + r0, t);
        param8<VEC>(dt_bias, param_dtype, int64_t(h) * S + r0, bias);
#pragma unroll
        for (int j = 0; j < 8; ++j) y[r0 + j] = a * softplus_f(t[j] + bias[j]);
    }
}

// Butterfly sum over N lanes, the result in every lane.
template <int N>
__device__ __forceinline__ float wave_total(float x) {
#pragma unroll
    for (int m = N / 2; m >= 1; m >>= 1) x += __shfl_xor(x, m, N);
    return x;
}

}  // namespace bdm

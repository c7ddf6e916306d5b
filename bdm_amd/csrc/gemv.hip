// Skinny linear maps of the decode step: y[m] = W x[m] + bias for a few rows
// m (one per sequence of a decode batch), W [N, K] row-major as nn.Linear
// stores it.
//
// At one to four rows every weight byte is read once and used M times, so
// the map is a stream over W at HBM bandwidth, not a matrix product: the
// GEMM libraries' tiles for M = 1 leave most of that bandwidth unused.  Each
// wave owns R consecutive output rows; lane l reads the 16-byte groups
// l, l + 64, ... of each of its rows (coalesced 1 KiB per row and load), all
// of them issued before the first FMA, and keeps one FP32 sum per (m, row).
// The sums are reduced across the wave and lane (m, row) adds the bias and
// stores the output, rounded once to the output dtype as torch's
// F.linear does (FP32 accumulation, bias added in FP32).
#include <type_traits>

#include "bdm_common.h"

namespace bdm {
namespace {

template <int N>
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int m = N / 2; m >= 1; m >>= 1) x += __shfl_xor(x, m, N);
    return x;
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Eight consecutive elements from a 16-byte aligned address, widened to FP32.
__device__ __forceinline__ void load8(const bf16_t *p, float (&x)[8]) {
    const u32x4_t r = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        x[2 * q] = __uint_as_float(w[q] << 16);
        x[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
    }
}
__device__ __forceinline__ void load8(const float *p, float (&x)[8]) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
    x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
}

// x rows are read through the cache (every wave reads them), W rows are
// streamed once (nontemporal for BF16).
template <typename T>
__device__ __forceinline__ void load8_cached(const T *p, float (&x)[8]) {
    float t[8];
    load_row<8>(p, t);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = t[j];
}

// M rows of x, R output rows per wave, KC 512-element chunks of K unrolled
// per pass (all loads of a pass in flight together).
template <typename T, int M, int R, int KC>
__global__ __launch_bounds__(256) void gemv_kernel(const T *__restrict__ x, const T *__restrict__ w,
                                                   const T *__restrict__ bias, T *__restrict__ y, int64_t n,
                                                   int k) {
    const int lane = threadIdx.x % kWave;
    const int64_t row0 = (int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave) * R;
    if (row0 >= n) return;
    float acc[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.f;
    const int groups = k / 8;  // 16-byte groups per row
    for (int g0 = 0; g0 < groups; g0 += KC * kWave) {
        float wv[KC][R][8];
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int g = min(g0 + c * kWave + lane, groups - 1);  // past the end: re-read the last group
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int64_t row = min(row0 + r, n - 1);
                load8(w + row * k + int64_t(g) * 8, wv[c][r]);
            }
        }
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int gi = g0 + c * kWave + lane;
            const bool live = gi < groups;
            const int g = min(gi, groups - 1);
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float xv[8];
                load8_cached(x + int64_t(m) * k + int64_t(g) * 8, xv);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float s = 0.f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) s = fmaf(wv[c][r][j], xv[j], s);
                    acc[m][r] += live ? s : 0.f;
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = wave_sum<kWave>(acc[m][r]);
    // lane m*R + r stores output (m, row0 + r)
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t row = row0 + r;
            if (lane == m * R + r && row < n) {
                float v = acc[m][r];
                if (bias) v += to_f32(bias[row]);
                y[int64_t(m) * n + row] = from_f32<T>(v);
            }
        }
}

template <typename T, int M>
int launch_gemv_m(const T *x, const T *w, const T *bias, T *y, int64_t n, int k, hipStream_t s) {
    // enough waves to keep HBM busy: 4 rows per wave once there are >= 8192
    // rows, fewer (more waves) below that
    const int groups = k / 8;
    const int kc = groups >= 4 * kWave ? 4 : (groups >= 2 * kWave ? 2 : 1);
    auto go = [&](auto r_tag) {
        constexpr int R = decltype(r_tag)::value;
        const int64_t waves = (n + R - 1) / R;
        const unsigned blocks = unsigned((waves + 3) / 4);
        if (kc == 4)
            gemv_kernel<T, M, R, 4><<<blocks, 256, 0, s>>>(x, w, bias, y, n, k);
        else if (kc == 2)
            gemv_kernel<T, M, R, 2><<<blocks, 256, 0, s>>>(x, w, bias, y, n, k);
        else
            gemv_kernel<T, M, R, 1><<<blocks, 256, 0, s>>>(x, w, bias, y, n, k);
    };
    if (n >= 8192)
        go(std::integral_constant<int, 4>{});
    else if (n >= 2048)
        go(std::integral_constant<int, 2>{});
    else
        go(std::integral_constant<int, 1>{});
    return check_launch("gemv_kernel");
}

template <typename T>
int launch_gemv(const void *x, const void *w, const void *bias, void *y, int64_t m, int64_t n, int k,
                hipStream_t s) {
    const T *xp = static_cast<const T *>(x), *wp = static_cast<const T *>(w), *bp = static_cast<const T *>(bias);
    T *yp = static_cast<T *>(y);
    switch (m) {
        case 1: return launch_gemv_m<T, 1>(xp, wp, bp, yp, n, k, s);
        case 2: return launch_gemv_m<T, 2>(xp, wp, bp, yp, n, k, s);
        case 3: return launch_gemv_m<T, 3>(xp, wp, bp, yp, n, k, s);
        case 4: return launch_gemv_m<T, 4>(xp, wp, bp, yp, n, k, s);
        default: return fail(BDM_ERR_UNSUPPORTED, "gemv: %lld rows (at most 4)", (long long)m);
    }
}

}  // namespace
}  // namespace bdm

extern "C" int bdm_gemv(const void *x, const void *weight, const void *bias, void *y, int64_t rows, int64_t n,
                        int64_t k, int32_t dtype, void *stream) {
    using namespace bdm;
    if (rows <= 0 || n <= 0 || k <= 0 || k % 8 != 0) return fail(BDM_ERR_INVALID, "gemv: bad geometry");
    if (k > INT32_MAX) return fail(BDM_ERR_UNSUPPORTED, "gemv: K past int32");
    if (dtype != BDM_BF16 && dtype != BDM_F32) return fail(BDM_ERR_INVALID, "gemv: dtype");
    if (!x || !weight || !y) return fail(BDM_ERR_INVALID, "gemv: null pointer");
    if (!aligned(x, 16) || !aligned(weight, 16)) return fail(BDM_ERR_INVALID, "gemv: x and W must be 16-byte aligned");
    if ((n + 3) / 4 > int64_t(UINT32_MAX)) return fail(BDM_ERR_UNSUPPORTED, "gemv: too many rows");
    hipStream_t s = as_stream(stream);
    if (dtype == BDM_BF16) return launch_gemv<bf16_t>(x, weight, bias, y, rows, n, int(k), s);
    return launch_gemv<float>(x, weight, bias, y, rows, n, int(k), s);
}

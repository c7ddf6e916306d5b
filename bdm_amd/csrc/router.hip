// Product-key router: top-s per factor, top-B over the Cartesian candidates,
// FP32 softmax of the selected pair sums.
//
// Reference: product_key_route, implementation/bdm/gdn2_banks.py:74-114.
// One lane owns one score row.  A row is tiny (J1+J2 scores, J1+J2 <= 96 in
// every benchmark geometry), so the selection runs entirely in registers:
// sorted insertion into a fixed-size list ordered by (value desc, index asc).
// That order is the pinned tie rule: equal values keep the lower index first.
//
// Only pairs (i, l) of the two sorted factor lists with (i+1)(l+1) <= B can
// reach the top B: the (i+1)(l+1)-1 pairs (i', l') <= (i, l) are all at least
// as large (rounding is monotone) and come earlier in the flattened
// i*s + l order, so they all precede (i, l).  The candidate loop visits just
// those pairs, in increasing flattened index.
#include <cfloat>

#include "bdm_common.h"

namespace bdm {
namespace {

template <int N>
__device__ __forceinline__ void insert_sorted(float (&val)[N], int (&idx)[N], float x, int i) {
#pragma unroll
    for (int p = 0; p < N; ++p) {
        const bool before = (x > val[p]) || (x == val[p] && i < idx[p]);
        const float tv = before ? val[p] : x;
        const int ti = before ? idx[p] : i;
        val[p] = before ? x : val[p];
        idx[p] = before ? i : idx[p];
        x = tv;
        i = ti;
    }
}

// Elements per 16-byte load of a score row.
template <typename T> constexpr int kVec = 16 / int(sizeof(T));

template <typename T, int SMAX>
__global__ __launch_bounds__(64) void router_kernel(const T *__restrict__ scores, int64_t rows,
                                                     int64_t stride, int j1, int j2, int selected,
                                                     T *__restrict__ weights,
                                                     int64_t *__restrict__ indices) {
    const int64_t row = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const T *z = scores + row * stride;
    const int s = min(selected, min(j1, j2));
    const int count = min(selected, s * s);

    float fv[SMAX], sv[SMAX];
    int fi[SMAX], si[SMAX];
#pragma unroll
    for (int p = 0; p < SMAX; ++p) {
        fv[p] = sv[p] = -INFINITY;
        fi[p] = si[p] = INT32_MAX;
    }
    if ((stride * int64_t(sizeof(T))) % 16 == 0 && (j1 + j2) % kVec<T> == 0) {
        // whole 16-byte chunks of the row
        for (int i0 = 0; i0 < j1 + j2; i0 += kVec<T>) {
            float chunk[kVec<T>];
            load_row<kVec<T>>(z + i0, chunk);
#pragma unroll
            for (int e = 0; e < kVec<T>; ++e) {
                const int i = i0 + e;
                if (i < j1)
                    insert_sorted(fv, fi, chunk[e], i);
                else
                    insert_sorted(sv, si, chunk[e], i - j1);
            }
        }
    } else {
        for (int i = 0; i < j1; ++i) insert_sorted(fv, fi, to_f32(z[i]), i);
        for (int i = 0; i < j2; ++i) insert_sorted(sv, si, to_f32(z[j1 + i]), i);
    }

    float pv[SMAX];
    int pi[SMAX];
#pragma unroll
    for (int p = 0; p < SMAX; ++p) {
        pv[p] = -INFINITY;
        pi[p] = INT32_MAX;
    }
#pragma unroll
    for (int i = 0; i < SMAX; ++i) {
#pragma unroll
        for (int l = 0; l < SMAX / (i + 1); ++l) {
            if (i < s && l < s && (i + 1) * (l + 1) <= count) {
                // The pair sum is formed in the score dtype (gdn2_banks.py:106).
                const float pair = round_to<T>(fv[i] + sv[l]);
                insert_sorted(pv, pi, pair, i * s + l);
            }
        }
    }

    // softmax over the selected sums in FP32, cast to the score dtype (:114)
    const float top = pv[0];
    float e[SMAX];
    float total = 0.f;
#pragma unroll
    for (int p = 0; p < SMAX; ++p) {
        e[p] = p < count ? expf(pv[p] - top) : 0.f;
        total += e[p];
    }
    T *wout = weights + row * count;
    int64_t *iout = indices + row * count;
#pragma unroll
    for (int p = 0; p < SMAX; ++p) {
        if (p < count) {
            const int a = pi[p] / s, c = pi[p] - a * s;
            int first = 0, second = 0;
            // select the a-th / c-th entries without dynamic register indexing
#pragma unroll
            for (int q = 0; q < SMAX; ++q) {
                first = (q == a) ? fi[q] : first;
                second = (q == c) ? si[q] : second;
            }
            wout[p] = from_f32<T>(e[p] / total);
            iout[p] = int64_t(first) * j2 + second;
        }
    }
}

template <typename T>
int launch_router(const void *scores, int64_t rows, int64_t stride, int j1, int j2, int selected,
                  void *weights, int64_t *indices, hipStream_t stream) {
    // 64 rows per workgroup: one row per lane, and enough workgroups to cover
    // every CU at the benchmark sizes (32K rows -> 512 workgroups)
    const dim3 block(64), grid(unsigned((rows + 63) / 64));
    if (selected <= 8) {
        router_kernel<T, 8><<<grid, block, 0, stream>>>(static_cast<const T *>(scores), rows, stride, j1,
                                                        j2, selected, static_cast<T *>(weights), indices);
    } else {
        router_kernel<T, 16><<<grid, block, 0, stream>>>(static_cast<const T *>(scores), rows, stride, j1,
                                                         j2, selected, static_cast<T *>(weights), indices);
    }
    return check_launch("router_kernel");
}

}  // namespace
}  // namespace bdm

extern "C" int bdm_router_select(const void *scores, int32_t score_dtype, int64_t rows, int64_t row_stride,
                                 int32_t factor_first, int32_t factor_second, int32_t selected,
                                 void *weights, int64_t *indices, void *stream) {
    using namespace bdm;
    if (rows < 0 || factor_first <= 0 || factor_second <= 0 || row_stride < factor_first + factor_second)
        return fail(BDM_ERR_INVALID, "router: bad geometry rows=%lld J1=%d J2=%d stride=%lld", (long long)rows,
                    factor_first, factor_second, (long long)row_stride);
    if (selected < 1 || int64_t(selected) > int64_t(factor_first) * factor_second)
        return fail(BDM_ERR_INVALID, "router: selected=%d outside the bank table", selected);
    if (selected > 16) return fail(BDM_ERR_UNSUPPORTED, "router: selected=%d > 16 is not implemented", selected);
    if (rows == 0) return BDM_OK;
    if (!scores || !weights || !indices) return fail(BDM_ERR_INVALID, "router: null pointer");
    if (!aligned(scores, 16)) return fail(BDM_ERR_INVALID, "router: scores must be 16-byte aligned");
    if (rows > int64_t(INT32_MAX) * 64) return fail(BDM_ERR_UNSUPPORTED, "router: too many rows");
    switch (score_dtype) {
        case BDM_BF16:
            return launch_router<bf16_t>(scores, rows, row_stride, factor_first, factor_second, selected, weights,
                                         indices, as_stream(stream));
        case BDM_F32:
            return launch_router<float>(scores, rows, row_stride, factor_first, factor_second, selected, weights,
                                        indices, as_stream(stream));
        default:
            return fail(BDM_ERR_INVALID, "router: unknown score dtype %d", score_dtype);
    }
}

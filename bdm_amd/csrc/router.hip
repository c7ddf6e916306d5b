// Product-key router: top-s per factor, top-B over the Cartesian candidates,
// FP32 softmax of the selected pair sums.
//
// Reference: product_key_route, implementation/bdm/gdn2_banks.py:74-114.
// Selection is by rank, with one lane per score (a 32- or 64-lane group per
// row), so a row costs a few dozen compares per lane instead of a serial
// insertion sort.  The order is (value desc, index asc): that is the pinned
// tie rule, equal values keep the lower index first.
//
// Only pairs (i, l) of the two sorted factor lists with (i+1)(l+1) <= B can
// reach the top B: the (i+1)(l+1)-1 pairs (i', l') <= (i, l) are all at least
// as large (rounding is monotone) and come earlier in the flattened
// i*s + l order, so they all precede (i, l).  Only those candidates are
// formed, numbered in increasing flattened index.
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

// One lane per score (a G-lane group per row, G = 32 or 64), selection by
// rank: an entry of a factor list is kept at position
//   rank = #{entries before it in (value desc, index asc) order}
// when rank < s.  NaN scores order as -inf (ties among them by index), so the
// ranks always form a permutation.  The candidate pairs (i, l) with
// (i+1)(l+1) <= count are enumerated in increasing flattened index i*s + l
// and ranked the same way among themselves; the softmax sums the selected
// exponentials in selection order, one lane per output.
constexpr int kRouterBlock = 256;
constexpr int kRouterMaxScores = 256;  // J1 + J2 per row
constexpr int kRouterMaxSel = 16;
constexpr int kRouterMaxCand = 64;     // pairs with (i+1)(l+1) <= 16: 50

__device__ __forceinline__ float order_key(float x) { return x != x ? -INFINITY : x; }

// a (value va, index ia) precedes b (value vb, index ib)
__device__ __forceinline__ bool precedes(float va, int ia, float vb, int ib) {
    return va > vb || (va == vb && ia < ib);
}

template <typename T, int G>
__global__ __launch_bounds__(kRouterBlock) void router_rank_kernel(const T *__restrict__ scores, int64_t rows,
                                                                   int64_t stride, int j1, int j2, int selected,
                                                                   T *__restrict__ weights,
                                                                   int64_t *__restrict__ indices) {
    constexpr int RB = kRouterBlock / G;  // rows per workgroup
    __shared__ float s_val[RB][kRouterMaxScores];
    __shared__ float s_sv[RB][2][kRouterMaxSel];  // sorted factor lists: values
    __shared__ int s_si[RB][2][kRouterMaxSel];    // ... and indices
    __shared__ float s_cand[RB][kRouterMaxCand];
    __shared__ float s_pv[RB][kRouterMaxSel];     // selected pair sums, in order
    __shared__ int s_pc[RB][kRouterMaxSel];       // ... and their candidate numbers
    __shared__ float s_pe[RB][kRouterMaxSel];     // exp(selected - top)

    const int g = threadIdx.x / G, lane = threadIdx.x % G;
    const int64_t row = int64_t(blockIdx.x) * RB + g;
    const bool live = row < rows;
    const int jt = j1 + j2;
    const int s = min(selected, min(j1, j2));
    const int count = min(selected, s * s);
    const T *z = scores + (live ? row : 0) * stride;

    // (1) the row's scores
    for (int e = lane; e < jt; e += G) s_val[g][e] = live ? order_key(to_f32(z[e])) : 0.f;
    __syncthreads();
    // (2) rank of each score within its factor; the top s form the sorted lists
    for (int e = lane; e < jt; e += G) {
        const int f = e < j1 ? 0 : 1;
        const int lo = f ? j1 : 0, n = f ? j2 : j1, i = e - lo;
        const float x = s_val[g][e];
        int rank = 0;
#pragma unroll 8
        for (int jj = 0; jj < n; ++jj) rank += precedes(s_val[g][lo + jj], jj, x, i) ? 1 : 0;
        if (rank < s) {
            s_sv[g][f][rank] = x;
            s_si[g][f][rank] = i;
        }
    }
    __syncthreads();
    // (3) candidate pairs in increasing flattened index; their pair sums are
    // formed in the score dtype (gdn2_banks.py:106)
    int ci = -1, cl = -1;
    {
        int c = 0;
        for (int i = 0; i < s; ++i) {
            const int nl = min(s, count / (i + 1));
            if (lane >= c && lane < c + nl) {
                ci = i;
                cl = lane - c;
            }
            c += nl;
        }
    }
    const bool cand = ci >= 0;
    float pair = 0.f;
    if (cand) {
        pair = order_key(round_to<T>(s_sv[g][0][ci] + s_sv[g][1][cl]));
        s_cand[g][lane] = pair;
    }
    int ncand = 0;
    for (int i = 0; i < s; ++i) ncand += min(s, count / (i + 1));
    __syncthreads();
    if (cand) {
        int rank = 0;
#pragma unroll 8
        for (int c = 0; c < ncand; ++c) rank += precedes(s_cand[g][c], c, pair, lane) ? 1 : 0;
        if (rank < count) {
            s_pv[g][rank] = pair;
            s_pc[g][rank] = lane;
        }
    }
    __syncthreads();
    // (4) softmax over the selected sums in FP32, cast to the score dtype (:114);
    // the exponentials are summed in selection order
    const bool out = live && lane < count;
    float mine = 0.f;
    if (out) {
        mine = expf(s_pv[g][lane] - s_pv[g][0]);
        s_pe[g][lane] = mine;
    }
    __syncthreads();
    if (out) {
        float total = 0.f;
        for (int p = 0; p < count; ++p) total += s_pe[g][p];
        // candidate number -> (i, l): candidates are numbered row by row of i
        const int c = s_pc[g][lane];
        int i = 0, base = 0;
        while (i + 1 < s && c >= base + min(s, count / (i + 1))) {
            base += min(s, count / (i + 1));
            ++i;
        }
        const int l = c - base;
        weights[row * count + lane] = from_f32<T>(mine / total);
        indices[row * count + lane] = int64_t(s_si[g][0][i]) * j2 + s_si[g][1][l];
    }
}

template <typename T>
int launch_router(const void *scores, int64_t rows, int64_t stride, int j1, int j2, int selected,
                  void *weights, int64_t *indices, hipStream_t stream) {
    // one lane per score and per candidate pair: 32-lane groups (8 rows per
    // workgroup) when both fit in 32, else 64-lane groups (4 rows)
    const int s = min(selected, min(j1, j2)), count = min(selected, s * s);
    int ncand = 0;
    for (int i = 0; i < s; ++i) ncand += min(s, count / (i + 1));
    if (j1 + j2 <= 32 && ncand <= 32) {
        const dim3 grid(unsigned((rows + 7) / 8));
        router_rank_kernel<T, 32><<<grid, kRouterBlock, 0, stream>>>(
            static_cast<const T *>(scores), rows, stride, j1, j2, selected, static_cast<T *>(weights), indices);
    } else {
        const dim3 grid(unsigned((rows + 3) / 4));
        router_rank_kernel<T, 64><<<grid, kRouterBlock, 0, stream>>>(
            static_cast<const T *>(scores), rows, stride, j1, j2, selected, static_cast<T *>(weights), indices);
    }
    return check_launch("router_rank_kernel");
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
    if (selected > kRouterMaxSel) return fail(BDM_ERR_UNSUPPORTED, "router: selected=%d > 16 is not implemented", selected);
    if (factor_first + factor_second > kRouterMaxScores)
        return fail(BDM_ERR_UNSUPPORTED, "router: J1 + J2 = %d > %d scores per row", factor_first + factor_second,
                    kRouterMaxScores);
    if (rows == 0) return BDM_OK;
    if (!scores || !weights || !indices) return fail(BDM_ERR_INVALID, "router: null pointer");
    if (!aligned(scores, 16)) return fail(BDM_ERR_INVALID, "router: scores must be 16-byte aligned");
    if (rows > int64_t(INT32_MAX) * 4) return fail(BDM_ERR_UNSUPPORTED, "router: too many rows");
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

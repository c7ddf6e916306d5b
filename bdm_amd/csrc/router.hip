// Product-key router: top-s per factor, top-B over the Cartesian candidates,
// FP32 softmax of the selected pair sums.
//
// Reference: product_key_route, implementation/bdm/gdn2_banks.py:74-114.
// One lane per row: the row's scores stream through two sorted top-s lists
// held in registers (one per factor), then the candidate pairs through a
// third; no LDS and no barriers.  Order is (value desc, index asc), the pinned
// tie rule: entries arrive in increasing index and an arrival goes behind
// every equal entry, so equal values keep the lower index first.
// Values are compared as order-preserving 32-bit keys (NaN as -inf, -0 as
// +0), with key 0 marking an empty slot below every score.
//
// Only pairs (i, l) of the two sorted factor lists with (i+1)(l+1) <= B can
// reach the top B: the (i+1)(l+1)-1 pairs (i', l') <= (i, l) are all at least
// as large (rounding is monotone) and come earlier in the flattened
// i*s + l order, so they all precede (i, l).  Only those candidates are
// formed, in increasing flattened index.
#include <cfloat>

#include "bdm_common.h"
#include "router_ops.h"

namespace bdm {
namespace {

constexpr int kRouterMaxScores = 4096;  // J1 + J2 per row (entries pack 16-bit factor ids)
constexpr int kRouterMaxSel = 16;

// Insert (k, id) into a list sorted by key desc, behind every entry with an
// equal or larger key; the entries after it move down one slot and the last
// one falls off.  c[p] = key[p] >= k is true on a prefix of the list, so slot
// p keeps its entry (c[p]), takes the new one (first p with !c[p]) or takes
// the entry of slot p-1.
template <int N>
__device__ __forceinline__ void insert_key(uint32_t (&key)[N], int (&id)[N], uint32_t k, int i) {
    bool c[N];
#pragma unroll
    for (int p = 0; p < N; ++p) c[p] = key[p] >= k;
#pragma unroll
    for (int p = N - 1; p >= 0; --p) {
        const bool prev = p == 0 ? true : c[p - 1];
        const uint32_t nk = prev ? k : key[p > 0 ? p - 1 : 0];
        const int ni = prev ? i : id[p > 0 ? p - 1 : 0];
        key[p] = c[p] ? key[p] : nk;
        id[p] = c[p] ? id[p] : ni;
    }
}

// Slot p of the list with x inserted is the (p+1)-th largest of list + {x}:
// max(list[p], min(list[p-1], x)) (entries are distinct).  Every slot is
// independent of the others, so the insertion has no serial chain.
template <int N>
__device__ __forceinline__ void insert_entry(uint32_t (&list)[N], uint32_t x) {
#pragma unroll
    for (int p = N - 1; p > 0; --p) list[p] = max(list[p], min(list[p - 1], x));
    list[0] = max(list[0], x);
}

// Eight scores of a row starting at element e0 (vector loads when VEC: the
// row is 16-byte aligned; elements past the row repeat its last score).
template <typename T, bool VEC>
__device__ __forceinline__ void load_block(const T *z, int e0, int n, float (&x)[8]) {
    if constexpr (VEC && sizeof(T) == 2) {
        const uint4 raw = *reinterpret_cast<const uint4 *>(z + e0);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            x[2 * q] = __uint_as_float(w[q] << 16);
            x[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
        }
    } else if constexpr (VEC) {
        const float4 a = *reinterpret_cast<const float4 *>(z + e0), b = *reinterpret_cast<const float4 *>(z + e0 + 4);
        x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
    } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) x[q] = to_f32(z[min(e0 + q, n - 1)]);
    }
}

// SM: list slots (>= selected); VEC: rows are 16-byte aligned and hold a
// multiple of 8 scores.
// Up to two routing roles (the write and read routers of one layer) in one
// launch: blockIdx.y picks the role.
template <typename T>
struct RouterRoles {
    const T *scores[2];
    int64_t stride[2];
    T *weights[2];
    int64_t *indices[2];
};

template <typename T, int SM, bool VEC>
__global__ __launch_bounds__(64) void router_lane_kernel(RouterRoles<T> roles, int64_t rows, int j1, int j2,
                                                         int selected) {
    const int role = int(blockIdx.y);
    const T *__restrict__ scores = roles.scores[role];
    const int64_t stride = roles.stride[role];
    T *__restrict__ weights = roles.weights[role];
    int64_t *__restrict__ indices = roles.indices[role];
    const int64_t row = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const T *z = scores + row * stride;
    const int s = min(selected, min(j1, j2));
    const int count = min(selected, s * s);
    const int n = j1 + j2;

    // blocks e0 + 8 and e0 + 16 are in flight while block e0 is inserted
    const int last = ((n - 1) / 8) * 8;  // start of the row's last block
    float x0[8], x1[8], x2[8];
    load_block<T, VEC>(z, 0, n, x0);
    load_block<T, VEC>(z, min(8, last), n, x1);
    T *wout = weights + row * count;
    int64_t *iout = indices + row * count;
    float ex[SM];
    int bank[SM];

    if constexpr (sizeof(T) == 2) {
        // (1) top-s of each factor, packed entries; a block of 8 scores is
        // branch-free unless it straddles the factor boundary
        uint32_t f0[SM], f1[SM];
#pragma unroll
        for (int p = 0; p < SM; ++p) f0[p] = f1[p] = 0u;
        for (int e0 = 0; e0 < n; e0 += 8) {
            load_block<T, VEC>(z, min(e0 + 16, last), n, x2);
            if (e0 + 8 <= j1) {
                uint32_t en[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) en[q] = pack_entry(x0[q], e0 + q);
#pragma unroll
                for (int q = 0; q < 8; ++q) insert_entry<SM>(f0, en[q]);
            } else if (e0 >= j1 && e0 + 8 <= n) {
                uint32_t en[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) en[q] = pack_entry(x0[q], e0 + q - j1);
#pragma unroll
                for (int q = 0; q < 8; ++q) insert_entry<SM>(f1, en[q]);
            } else {
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const int e = e0 + q;
                    if (e < j1)
                        insert_entry<SM>(f0, pack_entry(x0[q], e));
                    else if (e < n)
                        insert_entry<SM>(f1, pack_entry(x0[q], e - j1));
                }
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) x0[q] = x1[q], x1[q] = x2[q];
        }
        float v0[SM], v1[SM];
        int i0[SM], i1[SM];
#pragma unroll
        for (int p = 0; p < SM; ++p) {
            v0[p] = entry_value(f0[p]), v1[p] = entry_value(f1[p]);
            i0[p] = entry_id(f0[p]), i1[p] = entry_id(f1[p]);
        }
        // (2) candidate pairs (i+1)(l+1) <= count, packed with id i*SM + l
        // (increasing flattened index); pair sums formed in BF16
        // (gdn2_banks.py:106)
        uint32_t pl[SM];
#pragma unroll
        for (int p = 0; p < SM; ++p) pl[p] = 0u;
        auto candidate = [&](int i, int l) { insert_entry<SM>(pl, pack_entry(round_to<T>(v0[i] + v1[l]), i * SM + l)); };
        if (s == SM && count == SM) {  // every (i+1)(l+1) <= SM pair: straight-line
#pragma unroll
            for (int i = 0; i < SM; ++i)
#pragma unroll
                for (int l = 0; l < SM / (i + 1); ++l) candidate(i, l);
        } else {
#pragma unroll
            for (int i = 0; i < SM; ++i)
#pragma unroll
                for (int l = 0; l < SM / (i + 1); ++l)
                    if (i < s && l < s && (i + 1) * (l + 1) <= count) candidate(i, l);
        }
        // the selected pairs' bank ids through a per-lane table of the two lists' ids
        __shared__ int s_ids[64][2 * SM];
        const int lane = threadIdx.x;
#pragma unroll
        for (int p = 0; p < SM; ++p) s_ids[lane][p] = i0[p], s_ids[lane][SM + p] = i1[p];
        const float top = entry_value(pl[0]);
#pragma unroll
        for (int p = 0; p < SM; ++p) {
            ex[p] = expf(entry_value(pl[p]) - top);
            const int c = entry_id(pl[p]) & (SM * SM - 1);  // empty slots (past count) stay in the table
            bank[p] = s_ids[lane][c / SM] * j2 + s_ids[lane][SM + c % SM];
        }
    } else {
        // (1) top-s of each factor: FP32 keys with the index alongside
        uint32_t k0[SM], k1[SM];
        int i0[SM], i1[SM];
#pragma unroll
        for (int p = 0; p < SM; ++p) k0[p] = k1[p] = 0u, i0[p] = i1[p] = 0;
        for (int e0 = 0; e0 < n; e0 += 8) {
            load_block<T, VEC>(z, min(e0 + 16, last), n, x2);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int e = e0 + q;
                if (e < j1)
                    insert_key<SM>(k0, i0, score_key(x0[q]), e);
                else if (e < n)
                    insert_key<SM>(k1, i1, score_key(x0[q]), e - j1);
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) x0[q] = x1[q], x1[q] = x2[q];
        }
        float v0[SM], v1[SM];
#pragma unroll
        for (int p = 0; p < SM; ++p) v0[p] = key_value(k0[p]), v1[p] = key_value(k1[p]);
        // (2) candidate pairs in increasing flattened index, carrying the bank
        uint32_t kp[SM];
#pragma unroll
        for (int p = 0; p < SM; ++p) kp[p] = 0u, bank[p] = 0;
#pragma unroll
        for (int i = 0; i < SM; ++i) {
#pragma unroll
            for (int l = 0; l < SM / (i + 1); ++l) {  // (i+1)(l+1) <= SM
                if (i < s && l < s && (i + 1) * (l + 1) <= count)
                    insert_key<SM>(kp, bank, score_key(round_to<T>(v0[i] + v1[l])), i0[i] * j2 + i1[l]);
            }
        }
        const float top = key_value(kp[0]);
#pragma unroll
        for (int p = 0; p < SM; ++p) ex[p] = expf(key_value(kp[p]) - top);
    }

    // (3) softmax over the selected sums in FP32, cast to the score dtype
    // (:114); the exponentials are summed in selection order
    float total = 0.f;
#pragma unroll
    for (int p = 0; p < SM; ++p)
        if (p < count) total += ex[p];
#pragma unroll
    for (int p = 0; p < SM; ++p) {
        if (p < count) {
            wout[p] = from_f32<T>(ex[p] / total);
            iout[p] = int64_t(bank[p]);
        }
    }
}

__global__ __launch_bounds__(256) void router_wave_kernel(const bf16_t *__restrict__ scores, int64_t rows,
                                                          int64_t stride, int j1, int j2, int selected,
                                                          bf16_t *__restrict__ weights,
                                                          int64_t *__restrict__ indices) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;
    float weight;
    int64_t bank;
    const int count = route_row_wave(scores + row * stride, j1, j2, selected, lane, weight, bank);
    if (lane < count) {
        weights[row * count + lane] = from_f32<bf16_t>(weight);
        indices[row * count + lane] = bank;
    }
}

template <typename T, int SM>
void launch_router_sm(const RouterRoles<T> &roles, int nroles, int64_t rows, int j1, int j2, int selected,
                      hipStream_t stream) {
    // one lane per row, 64-lane workgroups spread over the CUs
    const dim3 grid(unsigned((rows + 63) / 64), unsigned(nroles));
    const int n = j1 + j2;
    bool vec = n % 8 == 0;
    for (int r = 0; r < nroles; ++r)
        vec = vec && aligned(roles.scores[r], 16) && (roles.stride[r] * int64_t(sizeof(T))) % 16 == 0;
    if (vec)
        router_lane_kernel<T, SM, true><<<grid, 64, 0, stream>>>(roles, rows, j1, j2, selected);
    else
        router_lane_kernel<T, SM, false><<<grid, 64, 0, stream>>>(roles, rows, j1, j2, selected);
}

template <typename T>
int launch_router(const RouterRoles<T> &roles, int nroles, int64_t rows, int j1, int j2, int selected,
                  hipStream_t stream) {
    if constexpr (sizeof(T) == 2) {
        // few rows (decode): one wave per row instead of one lane per row
        if (rows <= 2048 && selected <= 8 && j1 <= kWave && j2 <= kWave) {
            for (int r = 0; r < nroles; ++r) {
                router_wave_kernel<<<unsigned((rows + 3) / 4), 256, 0, stream>>>(
                    roles.scores[r], rows, roles.stride[r], j1, j2, selected, roles.weights[r], roles.indices[r]);
                if (int rc = check_launch("router_wave_kernel")) return rc;
            }
            return BDM_OK;
        }
    }
    if (selected <= 8)
        launch_router_sm<T, 8>(roles, nroles, rows, j1, j2, selected, stream);
    else
        launch_router_sm<T, 16>(roles, nroles, rows, j1, j2, selected, stream);
    return check_launch("router_lane_kernel");
}

int check_router_geometry(int64_t rows, int64_t row_stride, int32_t factor_first, int32_t factor_second,
                          int32_t selected) {
    if (rows < 0 || factor_first <= 0 || factor_second <= 0 || row_stride < factor_first + factor_second)
        return fail(BDM_ERR_INVALID, "router: bad geometry rows=%lld J1=%d J2=%d stride=%lld", (long long)rows,
                    factor_first, factor_second, (long long)row_stride);
    if (selected < 1 || int64_t(selected) > int64_t(factor_first) * factor_second)
        return fail(BDM_ERR_INVALID, "router: selected=%d outside the bank table", selected);
    if (selected > kRouterMaxSel) return fail(BDM_ERR_UNSUPPORTED, "router: selected=%d > 16 is not implemented", selected);
    if (factor_first + factor_second > kRouterMaxScores)
        return fail(BDM_ERR_UNSUPPORTED, "router: J1 + J2 = %d > %d scores per row", factor_first + factor_second,
                    kRouterMaxScores);
    if (rows > int64_t(INT32_MAX) * 32) return fail(BDM_ERR_UNSUPPORTED, "router: too many rows");
    return BDM_OK;
}

template <typename T>
int route_roles(const void *const *scores, const int64_t *strides, void *const *weights, int64_t *const *indices,
                int nroles, int64_t rows, int j1, int j2, int selected, hipStream_t stream) {
    RouterRoles<T> roles{};
    for (int r = 0; r < nroles; ++r) {
        roles.scores[r] = static_cast<const T *>(scores[r]);
        roles.stride[r] = strides[r];
        roles.weights[r] = static_cast<T *>(weights[r]);
        roles.indices[r] = indices[r];
    }
    return launch_router<T>(roles, nroles, rows, j1, j2, selected, stream);
}

int route(const void *const *scores, const int64_t *strides, void *const *weights, int64_t *const *indices,
          int nroles, int32_t score_dtype, int64_t rows, int j1, int j2, int selected, hipStream_t stream) {
    for (int r = 0; r < nroles; ++r) {
        if (int rc = check_router_geometry(rows, strides[r], j1, j2, selected)) return rc;
    }
    if (rows == 0) return BDM_OK;
    for (int r = 0; r < nroles; ++r) {
        if (!scores[r] || !weights[r] || !indices[r]) return fail(BDM_ERR_INVALID, "router: null pointer");
        if (!aligned(scores[r], 16)) return fail(BDM_ERR_INVALID, "router: scores must be 16-byte aligned");
    }
    switch (score_dtype) {
        case BDM_BF16: return route_roles<bf16_t>(scores, strides, weights, indices, nroles, rows, j1, j2, selected, stream);
        case BDM_F32: return route_roles<float>(scores, strides, weights, indices, nroles, rows, j1, j2, selected, stream);
        default: return fail(BDM_ERR_INVALID, "router: unknown score dtype %d", score_dtype);
    }
}

}  // namespace
}  // namespace bdm

extern "C" int bdm_router_select(const void *scores, int32_t score_dtype, int64_t rows, int64_t row_stride,
                                 int32_t factor_first, int32_t factor_second, int32_t selected,
                                 void *weights, int64_t *indices, void *stream) {
    const void *sc[1] = {scores};
    const int64_t st[1] = {row_stride};
    void *w[1] = {weights};
    int64_t *ix[1] = {indices};
    return bdm::route(sc, st, w, ix, 1, score_dtype, rows, factor_first, factor_second, selected,
                      bdm::as_stream(stream));
}

extern "C" int bdm_router_select_pair(const void *scores_a, int64_t row_stride_a, const void *scores_b,
                                      int64_t row_stride_b, int32_t score_dtype, int64_t rows, int32_t factor_first,
                                      int32_t factor_second, int32_t selected, void *weights_a,
                                      int64_t *indices_a, void *weights_b, int64_t *indices_b, void *stream) {
    const void *sc[2] = {scores_a, scores_b};
    const int64_t st[2] = {row_stride_a, row_stride_b};
    void *w[2] = {weights_a, weights_b};
    int64_t *ix[2] = {indices_a, indices_b};
    return bdm::route(sc, st, w, ix, 2, score_dtype, rows, factor_first, factor_second, selected,
                      bdm::as_stream(stream));
}

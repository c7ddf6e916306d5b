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
#include "route_dispatch.h"

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

// Four lanes per row (a DPP quad), BF16 scores, selected = 8 from J1, J2 in
// [8, 64]: the lane kernel's selection and softmax with a quarter of its
// serial chain (one lane per row runs ~1,500 dependent instructions, which
// sets that kernel's time at any row count).  Lanes q = 0, 1 take factor 0
// and q = 2, 3 factor 1; lane q sorts its blocks of 8 entries (blocks
// q%2, q%2 + 2, ... of its factor) with a 19-comparator network and merges
// them into a top 8; the quad then merges across lanes with DPP quad
// permutes.  The 20 candidate pairs (i+1)(l+1) <= 8 are formed 5 per lane,
// sorted and merged the same way, and lane q keeps selection slots 2q, 2q+1.
// Entries are the packed (value desc, index asc) keys of router_ops.h, a
// strict order, so any exact top-8 selection gives the lane kernel's list;
// the softmax sums the 8 exponentials in selection order as it does.
__device__ __forceinline__ void cex(uint32_t &a, uint32_t &b) {
    const uint32_t hi = max(a, b), lo = min(a, b);
    a = hi;
    b = lo;
}

// Sort 8 entries descending (Knuth's 19-comparator network).
__device__ __forceinline__ void sort8(uint32_t (&x)[8]) {
    cex(x[0], x[2]), cex(x[1], x[3]), cex(x[4], x[6]), cex(x[5], x[7]);
    cex(x[0], x[4]), cex(x[1], x[5]), cex(x[2], x[6]), cex(x[3], x[7]);
    cex(x[0], x[1]), cex(x[2], x[3]), cex(x[4], x[5]), cex(x[6], x[7]);
    cex(x[2], x[4]), cex(x[3], x[5]);
    cex(x[1], x[4]), cex(x[3], x[6]);
    cex(x[1], x[2]), cex(x[3], x[4]), cex(x[5], x[6]);
}

// a := the 8 largest of a and b (each sorted descending), sorted descending:
// max(a[p], b[7-p]) holds them as a bitonic sequence, which a bitonic merge sorts.
__device__ __forceinline__ void merge_top8(uint32_t (&a)[8], const uint32_t (&b)[8]) {
#pragma unroll
    for (int p = 0; p < 8; ++p) a[p] = max(a[p], b[7 - p]);
    cex(a[0], a[4]), cex(a[1], a[5]), cex(a[2], a[6]), cex(a[3], a[7]);
    cex(a[0], a[2]), cex(a[1], a[3]), cex(a[4], a[6]), cex(a[5], a[7]);
    cex(a[0], a[1]), cex(a[2], a[3]), cex(a[4], a[5]), cex(a[6], a[7]);
}

// Lane (lane & ~3) + perm[lane & 3] of the quad, perm packed 2 bits per lane.
template <int PERM>
__device__ __forceinline__ uint32_t quad_get(uint32_t x) {
    return uint32_t(__builtin_amdgcn_update_dpp(0, int(x), PERM, 0xF, 0xF, false));
}

template <int PERM>
__device__ __forceinline__ void quad_merge(uint32_t (&a)[8]) {
    uint32_t b[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) b[p] = quad_get<PERM>(a[p]);
    merge_top8(a, b);
}

__device__ __forceinline__ uint32_t pick4(int q, uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3) {
    const uint32_t lo = (q & 1) ? a1 : a0, hi = (q & 1) ? a3 : a2;
    return (q & 2) ? hi : lo;
}

constexpr int kQuadXor1 = 0xB1;  // quad_perm [1, 0, 3, 2]
constexpr int kQuadXor2 = 0x4E;  // quad_perm [2, 3, 0, 1]

template <int NB>
__global__ __launch_bounds__(256) void router_quad_kernel(RouterRoles<bf16_t> roles, int64_t rows, int j1, int j2) {
    const int role = int(blockIdx.y);
    const int q = int(threadIdx.x) & 3;
    const int64_t row_raw = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 2;
    const bool live = row_raw < rows;  // uniform over a quad
    const int64_t row = live ? row_raw : rows - 1;
    const int factor = q >> 1, half = q & 1;
    const int jf = factor ? j2 : j1;
    const bf16_t *zf = roles.scores[role] + row * roles.stride[role] + (factor ? j1 : 0);

    // (1) top 8 of each factor
    uint4 raw[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int e0 = (half + 2 * b) * 8;
        raw[b] = *reinterpret_cast<const uint4 *>(zf + (e0 < jf ? e0 : 0));
    }
    uint32_t top[8];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int e0 = (half + 2 * b) * 8;
        const uint32_t w[4] = {raw[b].x, raw[b].y, raw[b].z, raw[b].w};
        // packed unconditionally, then cleared past the factor (a select, not a branch per entry)
        const uint32_t keep = e0 < jf ? 0xffffffffu : 0u;
        uint32_t en[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float x = __uint_as_float(k & 1 ? (w[k / 2] & 0xffff0000u) : (w[k / 2] << 16));
            en[k] = pack_entry(x, e0 + k) & keep;
        }
        sort8(en);
        if (b == 0) {
#pragma unroll
            for (int p = 0; p < 8; ++p) top[p] = en[p];
        } else {
            merge_top8(top, en);
        }
    }
    quad_merge<kQuadXor1>(top);  // the factor's top 8 in both of its lanes
    uint32_t f0[8], f1[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const uint32_t other = quad_get<kQuadXor2>(top[p]);
        f0[p] = factor ? other : top[p];
        f1[p] = factor ? top[p] : other;
    }
    // factor ids of the two lists, one byte each, for the bank lookup at the end
    __shared__ uint32_t s_ids[256][4];
    uint32_t packed[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t(&f)[8] = w < 2 ? f0 : f1;
        const int p0 = (w & 1) * 4;
        packed[w] = uint32_t(entry_id(f[p0])) | uint32_t(entry_id(f[p0 + 1])) << 8 |
                    uint32_t(entry_id(f[p0 + 2])) << 16 | uint32_t(entry_id(f[p0 + 3])) << 24;
    }
    *reinterpret_cast<uint4 *>(s_ids[threadIdx.x]) = make_uint4(packed[0], packed[1], packed[2], packed[3]);

    // (2) candidates (0, q), (0, 4+q), (1, q), (2 + q/2, q%2), (4+q, 0) with
    // ids i*8 + l, pair sums in BF16 (gdn2_banks.py:106)
    const float a0 = entry_value(f0[0]), a1 = entry_value(f0[1]), b0 = entry_value(f1[0]);
    const float bq = entry_value(pick4(q, f1[0], f1[1], f1[2], f1[3]));
    const float bq4 = entry_value(pick4(q, f1[4], f1[5], f1[6], f1[7]));
    const float aq4 = entry_value(pick4(q, f0[4], f0[5], f0[6], f0[7]));
    const float a3 = entry_value((q & 2) ? f0[3] : f0[2]);
    const float b3 = entry_value((q & 1) ? f1[1] : f1[0]);
    uint32_t c[8];
    c[0] = pack_entry(round_to<bf16_t>(a0 + bq), q);
    c[1] = pack_entry(round_to<bf16_t>(a0 + bq4), 4 + q);
    c[2] = pack_entry(round_to<bf16_t>(a1 + bq), 8 + q);
    c[3] = pack_entry(round_to<bf16_t>(a3 + b3), 16 + 8 * (q >> 1) + (q & 1));
    c[4] = pack_entry(round_to<bf16_t>(aq4 + b0), 32 + 8 * q);
    c[5] = c[6] = c[7] = 0u;
    sort8(c);
    quad_merge<kQuadXor1>(c);
    quad_merge<kQuadXor2>(c);

    // (3) softmax over the selected sums in FP32, the exponentials summed in
    // selection order (gdn2_banks.py:114); lane q keeps slots 2q and 2q+1
    const float top_value = entry_value(c[0]);
    const uint32_t ea = pick4(q, c[0], c[2], c[4], c[6]), eb = pick4(q, c[1], c[3], c[5], c[7]);
    const float xa = expf(entry_value(ea) - top_value), xb = expf(entry_value(eb) - top_value);
    const uint32_t ua = __float_as_uint(xa), ub = __float_as_uint(xb);
    const float ex[8] = {__uint_as_float(quad_get<0x00>(ua)), __uint_as_float(quad_get<0x00>(ub)),
                         __uint_as_float(quad_get<0x55>(ua)), __uint_as_float(quad_get<0x55>(ub)),
                         __uint_as_float(quad_get<0xAA>(ua)), __uint_as_float(quad_get<0xAA>(ub)),
                         __uint_as_float(quad_get<0xFF>(ua)), __uint_as_float(quad_get<0xFF>(ub))};
    float total = 0.f;
#pragma unroll
    for (int p = 0; p < 8; ++p) total += ex[p];
    const uint8_t *ids = reinterpret_cast<const uint8_t *>(s_ids[threadIdx.x]);
    auto bank_of = [&](uint32_t e) {
        const int cid = entry_id(e) & 63;
        return int64_t(ids[cid >> 3]) * j2 + int64_t(ids[8 + (cid & 7)]);
    };
    const int64_t bank_a = bank_of(ea), bank_b = bank_of(eb);
    if (live) {
        const uint32_t wa = __float_as_uint(round_to<bf16_t>(xa / total)) >> 16;
        const uint32_t wb = __float_as_uint(round_to<bf16_t>(xb / total)) & 0xffff0000u;
        *reinterpret_cast<uint32_t *>(roles.weights[role] + row * 8 + 2 * q) = wa | wb;
        int64_t *iout = roles.indices[role] + row * 8 + 2 * q;
        *reinterpret_cast<longlong2 *>(iout) = make_longlong2(bank_a, bank_b);
    }
}

// Two lanes per row, BF16 scores, selected = 8 from J1, J2 in [8, 32]: half
// the quad kernel's instructions per row (no work is repeated in four lanes)
// at half its lanes.  Lane h sorts factor h's blocks of 8 and merges them;
// the pair swaps lists (DPP quad_perm [1, 0, 3, 2]), lane 0 forms the
// candidate pairs of flattened index 0..9 and lane 1 the other 10, each
// sorts its 10 into a top 8, and one swap and merge leaves the selection in
// both lanes; lane h keeps slots 4h..4h+3.
// One row's routes, with two lanes (h = 0, 1: adjacent lanes of a quad) per
// row: lane h returns selection slots 4h .. 4h + 3 (bank ids and BF16 weight
// bits).  ids: this lane's 16 bytes of LDS (the row's factor ids, read back
// by both lanes of the pair).
template <int NB>
__device__ __forceinline__ void route_pair_row(const bf16_t *zrow, int j1, int j2, int h, uint32_t *ids_lds,
                                               int64_t (&bank)[4], uint32_t (&wbits)[4]) {
    const int jf = h ? j2 : j1;
    const bf16_t *zf = zrow + (h ? j1 : 0);

    // (1) top 8 of factor h
    uint4 raw[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) raw[b] = *reinterpret_cast<const uint4 *>(zf + (b * 8 < jf ? b * 8 : 0));
    uint32_t top[8];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const uint32_t w[4] = {raw[b].x, raw[b].y, raw[b].z, raw[b].w};
        const uint32_t keep = b * 8 < jf ? 0xffffffffu : 0u;
        uint32_t en[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float x = __uint_as_float(k & 1 ? (w[k / 2] & 0xffff0000u) : (w[k / 2] << 16));
            en[k] = pack_entry(x, b * 8 + k) & keep;
        }
        sort8(en);
        if (b == 0) {
#pragma unroll
            for (int p = 0; p < 8; ++p) top[p] = en[p];
        } else {
            merge_top8(top, en);
        }
    }
    uint32_t f0[8], f1[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const uint32_t other = quad_get<kQuadXor1>(top[p]);
        f0[p] = h ? other : top[p];
        f1[p] = h ? top[p] : other;
    }
    uint32_t packed[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t(&f)[8] = w < 2 ? f0 : f1;
        const int p0 = (w & 1) * 4;
        packed[w] = uint32_t(entry_id(f[p0])) | uint32_t(entry_id(f[p0 + 1])) << 8 |
                    uint32_t(entry_id(f[p0 + 2])) << 16 | uint32_t(entry_id(f[p0 + 3])) << 24;
    }
    *reinterpret_cast<uint4 *>(ids_lds) = make_uint4(packed[0], packed[1], packed[2], packed[3]);

    // (2) candidates: lane 0 (0,0..7), (1,0), (1,1); lane 1 (1,2), (1,3),
    // (2,0), (2,1), (3,0), (3,1), (4..7,0); ids i*8 + l, sums in BF16
    float a[8], b[8];
#pragma unroll
    for (int p = 0; p < 8; ++p) a[p] = entry_value(f0[p]), b[p] = entry_value(f1[p]);
    // (operands passed as values: an index chosen per lane would become a
    // select over all eight registers)
    auto cand = [&](float x0, float y0, int id0, float x1, float y1, int id1) {
        return pack_entry(round_to<bf16_t>(h ? x1 + y1 : x0 + y0), h ? id1 : id0);
    };
    uint32_t c[8];
    c[0] = cand(a[0], b[0], 0, a[1], b[2], 10);
    c[1] = cand(a[0], b[1], 1, a[1], b[3], 11);
    c[2] = cand(a[0], b[2], 2, a[2], b[0], 16);
    c[3] = cand(a[0], b[3], 3, a[2], b[1], 17);
    c[4] = cand(a[0], b[4], 4, a[3], b[0], 24);
    c[5] = cand(a[0], b[5], 5, a[3], b[1], 25);
    c[6] = cand(a[0], b[6], 6, a[4], b[0], 32);
    c[7] = cand(a[0], b[7], 7, a[5], b[0], 40);
    const uint32_t extra0 = cand(a[1], b[0], 8, a[6], b[0], 48);
    const uint32_t extra1 = cand(a[1], b[1], 9, a[7], b[0], 56);
    sort8(c);
    insert_entry<8>(c, extra0);
    insert_entry<8>(c, extra1);
    quad_merge<kQuadXor1>(c);

    // (3) softmax over the selected sums in FP32, the exponentials summed in
    // selection order (gdn2_banks.py:114)
    const float top_value = entry_value(c[0]);
    // slot 4h + k by a bit mask: a select between c[k] and c[4 + k] is
    // turned into an index chosen per lane, which moves c to LDS
    const uint32_t upper = 0u - uint32_t(h);
    uint32_t e[4];
    float xs[4], ex[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        e[k] = c[k] ^ ((c[k] ^ c[4 + k]) & upper);
        xs[k] = expf(entry_value(e[k]) - top_value);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float other = __uint_as_float(quad_get<kQuadXor1>(__float_as_uint(xs[k])));
        ex[k] = h ? other : xs[k];
        ex[4 + k] = h ? xs[k] : other;
    }
    float total = 0.f;
#pragma unroll
    for (int p = 0; p < 8; ++p) total += ex[p];
    const uint8_t *ids = reinterpret_cast<const uint8_t *>(ids_lds);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int cid = entry_id(e[k]) & 63;
        bank[k] = int64_t(ids[cid >> 3]) * j2 + int64_t(ids[8 + (cid & 7)]);
        wbits[k] = __float_as_uint(round_to<bf16_t>(xs[k] / total)) >> 16;
    }
}

template <int NB>
__global__ __launch_bounds__(256) void router_pair_kernel(RouterRoles<bf16_t> roles, int64_t rows, int j1, int j2) {
    const int role = int(blockIdx.y);
    const int h = int(threadIdx.x) & 1;
    const int64_t row_raw = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 1;
    const bool live = row_raw < rows;  // uniform over a pair
    const int64_t row = live ? row_raw : rows - 1;
    __shared__ uint32_t s_ids[256][4];
    int64_t bank[4];
    uint32_t wbits[4];
    route_pair_row<NB>(roles.scores[role] + row * roles.stride[role], j1, j2, h, s_ids[threadIdx.x], bank, wbits);
    if (live) {
        *reinterpret_cast<uint2 *>(roles.weights[role] + row * 8 + 4 * h) =
            make_uint2(wbits[0] | wbits[1] << 16, wbits[2] | wbits[3] << 16);
        longlong2 *iout = reinterpret_cast<longlong2 *>(roles.indices[role] + row * 8 + 4 * h);
        iout[0] = make_longlong2(bank[0], bank[1]);
        iout[1] = make_longlong2(bank[2], bank[3]);
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
    if constexpr (sizeof(T) == 2) {
        // selected = 8 from J1, J2 in [8, 64] (multiples of 8), aligned rows: four lanes per row
        bool quad = selected == 8 && j1 >= 8 && j2 >= 8 && j1 <= 64 && j2 <= 64 && j1 % 8 == 0 && j2 % 8 == 0;
        for (int r = 0; r < nroles; ++r)
            quad = quad && aligned(roles.scores[r], 16) && roles.stride[r] % 8 == 0 && aligned(roles.weights[r], 4) &&
                   aligned(roles.indices[r], 16);
        const int jmax = j1 > j2 ? j1 : j2;
        if (quad && jmax <= 32 && rows * 2 <= int64_t(UINT32_MAX)) {
            // two lanes per row up to 4 blocks of 8 per factor
            for (int r = 0; r < nroles; ++r) quad = quad && aligned(roles.weights[r], 8);
            if (quad) {
                const dim3 grid(unsigned((rows * 2 + 255) / 256), unsigned(nroles));
                switch ((jmax + 7) / 8) {
                    case 1: router_pair_kernel<1><<<grid, 256, 0, stream>>>(roles, rows, j1, j2); break;
                    case 2: router_pair_kernel<2><<<grid, 256, 0, stream>>>(roles, rows, j1, j2); break;
                    case 3: router_pair_kernel<3><<<grid, 256, 0, stream>>>(roles, rows, j1, j2); break;
                    default: router_pair_kernel<4><<<grid, 256, 0, stream>>>(roles, rows, j1, j2); break;
                }
                return check_launch("router_pair_kernel");
            }
            quad = true;  // weights only 4-byte aligned: the quad kernel takes them
        }
        if (quad && rows * 4 <= int64_t(UINT32_MAX)) {
            const dim3 grid(unsigned((rows * 4 + 255) / 256), unsigned(nroles));
            const int nb = (jmax + 15) / 16;
            switch (nb) {
                case 1: router_quad_kernel<1><<<grid, 256, 0, stream>>>(roles, rows, j1, j2); break;
                case 2: router_quad_kernel<2><<<grid, 256, 0, stream>>>(roles, rows, j1, j2); break;
                case 3: router_quad_kernel<3><<<grid, 256, 0, stream>>>(roles, rows, j1, j2); break;
                default: router_quad_kernel<4><<<grid, 256, 0, stream>>>(roles, rows, j1, j2); break;
            }
            return check_launch("router_quad_kernel");
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

// Routing fused with the dispatch's tile count (bdm_route_dispatch): one
// workgroup per tile of 32 tokens of one sequence routes the tile's rows for
// both roles (two lanes per row, route_pair_row), stores the routes, and sets
// bit 2 t + role of the LDS mask of every selected bank (t the token in the
// tile, role 1 for a read), as dispatch_tile_count does from stored routes;
// the popcount of a bank's mask is the tile's count of events in it.
// The grid is one-dimensional over the (sequence, tile) items, mapped as the
// scatter maps them: when their number is a multiple of 8, XCD x (blocks x,
// x + 8, ... in dispatch order) takes the x-th eighth in sequence-major
// order, so the routes and counts of a sequence stay in the L2 of the XCD
// whose scatter (and, for 8 sequences, tile scan) reads them next.
template <int NB>
__global__ __launch_bounds__(128) void route_tile_count_kernel(RouterRoles<bf16_t> roles, int64_t time, int tiles,
                                                               int batch, int j1, int j2,
                                                               int32_t *__restrict__ tile_counts,
                                                               int32_t *__restrict__ status) {
    extern __shared__ unsigned long long masks[];  // one per bank
    __shared__ uint32_t s_ids[128][4];
    const int banks = j1 * j2;
    const int64_t items = int64_t(tiles) * batch, lin = blockIdx.x;
    const int64_t item = items % 8 == 0 ? (lin % 8) * (items / 8) + lin / 8 : lin;
    const int tile = int(item % tiles), b = int(item / tiles);
    const int t = int(threadIdx.x), role = t >> 6, tl = (t & 63) >> 1, h = t & 1;
    for (int x = t; x < banks; x += 128) masks[x] = 0ull;
    const int64_t tt = int64_t(tile) * 32 + tl;
    const bool live = tt < time;  // uniform over a pair
    const int64_t row = int64_t(b) * time + (live ? tt : time - 1);
    int64_t bank[4];
    uint32_t wbits[4];
    route_pair_row<NB>(roles.scores[role] + row * roles.stride[role], j1, j2, h, s_ids[t], bank, wbits);
    if (live) {
        *reinterpret_cast<uint2 *>(roles.weights[role] + row * 8 + 4 * h) =
            make_uint2(wbits[0] | wbits[1] << 16, wbits[2] | wbits[3] << 16);
        longlong2 *iout = reinterpret_cast<longlong2 *>(roles.indices[role] + row * 8 + 4 * h);
        iout[0] = make_longlong2(bank[0], bank[1]);
        iout[1] = make_longlong2(bank[2], bank[3]);
    }
    __syncthreads();  // the masks are clear
    if (live) {
        const unsigned long long bit = 1ull << (2 * tl + role);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const unsigned long long old = atomicOr(&masks[bank[k]], bit);
            if (old & bit) atomicOr(status, int(BDM_ROUTE_DUPLICATE));
        }
    }
    __syncthreads();
    int32_t *out = tile_counts + (int64_t(b) * tiles + tile) * banks;
    for (int x = t; x < banks; x += 128) out[x] = __popcll(masks[x]);
}

}  // namespace

// Whether route_tile_count_kernel takes this routing: BF16 scores, 8 banks per
// role from factors of 8..32 (multiples of 8), 16-byte aligned score rows,
// 8-byte aligned weights and 16-byte aligned indices.
bool route_tile_count_supported(const void *const *scores, const int64_t *strides, void *const *weights,
                                int64_t *const *indices, int32_t score_dtype, int32_t j1, int32_t j2,
                                int32_t selected) {
    bool ok = score_dtype == BDM_BF16 && selected == 8 && j1 >= 8 && j2 >= 8 && j1 <= 32 && j2 <= 32 &&
              j1 % 8 == 0 && j2 % 8 == 0;
    for (int r = 0; r < 2; ++r)
        ok = ok && aligned(scores[r], 16) && strides[r] % 8 == 0 && strides[r] >= j1 + j2 && aligned(weights[r], 8) &&
             aligned(indices[r], 16);
    return ok;
}

int launch_route_tile_count(const void *const *scores, const int64_t *strides, void *const *weights,
                            int64_t *const *indices, int64_t batch, int64_t time, int32_t j1, int32_t j2,
                            int32_t *tile_counts, int32_t *status, hipStream_t stream) {
    RouterRoles<bf16_t> roles{};
    for (int r = 0; r < 2; ++r) {
        roles.scores[r] = static_cast<const bf16_t *>(scores[r]);
        roles.stride[r] = strides[r];
        roles.weights[r] = static_cast<bf16_t *>(weights[r]);
        roles.indices[r] = indices[r];
    }
    const int tiles = int((time + 31) / 32);
    if (batch > INT32_MAX || int64_t(tiles) * batch > int64_t(UINT32_MAX))
        return fail(BDM_ERR_UNSUPPORTED, "route_dispatch: too many tiles");
    const unsigned grid = unsigned(int64_t(tiles) * batch);
    const int nb = int(batch);
    const size_t lds = size_t(j1) * size_t(j2) * sizeof(unsigned long long);
    switch ((max(j1, j2) + 7) / 8) {
        case 1: route_tile_count_kernel<1><<<grid, 128, lds, stream>>>(roles, time, tiles, nb, j1, j2, tile_counts, status); break;
        case 2: route_tile_count_kernel<2><<<grid, 128, lds, stream>>>(roles, time, tiles, nb, j1, j2, tile_counts, status); break;
        case 3: route_tile_count_kernel<3><<<grid, 128, lds, stream>>>(roles, time, tiles, nb, j1, j2, tile_counts, status); break;
        default: route_tile_count_kernel<4><<<grid, 128, lds, stream>>>(roles, time, tiles, nb, j1, j2, tile_counts, status); break;
    }
    return check_launch("route_tile_count_kernel");
}

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

// Device pieces of the product-key router (gdn2_banks.py:74-114) shared by
// the router kernels (router.hip) and the fused decode step (decode.hip), so
// both select banks and form weights with the same instructions.
#pragma once

#include "bdm_common.h"

namespace bdm {

// Order-preserving key of a score: NaN orders as -inf, -0 as +0; keys of real
// values are >= 0x007FFFFF, so 0 can mark an empty slot.
__device__ __forceinline__ uint32_t score_key(float x) {
    if (x != x) x = -INFINITY;
    uint32_t b = __float_as_uint(x);
    if (b == 0x80000000u) b = 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

// BF16 scores have 16-bit keys: an entry packs key16 << 16 | (0xffff - id),
// so the larger entry is the earlier one in (value desc, index asc) order
// and insertion is a max/min compare-exchange chain.  0 is an empty slot.
__device__ __forceinline__ uint32_t pack_entry(float bf16_value, int id) {
    return (score_key(bf16_value) & 0xffff0000u) | uint32_t(0xffff - id);
}

__device__ __forceinline__ float entry_value(uint32_t e) {
    const uint32_t k = e >> 16;
    return key_value((k << 16) | ((k & 0x8000u) ? 0u : 0xffffu));
}

__device__ __forceinline__ int entry_id(uint32_t e) { return 0xffff - int(e & 0xffffu); }

// One wave per row, for few rows (a decode step): BF16 scores, J1, J2 <= 64,
// B <= 8.  Lane l holds score l of each factor as a packed entry; the top s
// of a factor are s rounds of a wave-wide max (the winner's lane clears its
// entry), the top B pairs B rounds over the candidates, one per lane
// (i, l) = (lane / 8, lane % 8).  The entries, tie rule, pair sums and
// softmax are router_lane_kernel's, so the results are identical; a round
// is a register-only wave maximum (DPP and permlane swaps, no LDS).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_max(uint32_t x) {
    return max(x, uint32_t(__builtin_amdgcn_update_dpp(0, int(x), CTRL, 0xF, 0xF, false)));
}

// Maximum over the wave in every lane, without LDS: DPP within each 16-lane
// row (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then
// v_permlane16_swap and v_permlane32_swap across rows.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
    x = dpp_max<0xB1>(x);
    x = dpp_max<0x4E>(x);
    x = dpp_max<0x141>(x);
    x = dpp_max<0x140>(x);
    const auto r16 = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    x = max(uint32_t(r16[0]), uint32_t(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return max(uint32_t(r32[0]), uint32_t(r32[1]));
}

// One row of BF16 scores routed by one wave (J1, J2 <= 64, selected <= 8):
// the router_wave_kernel algorithm above.  Lane j < count ends with slot j's
// weight (rounded to BF16) and bank id; other lanes' outputs are unspecified.
// Returns count = min(selected, s*s), s = min(selected, J1, J2).
__device__ __forceinline__ int route_row_wave(const bf16_t *__restrict__ z, int j1, int j2, int selected, int lane,
                                              float &weight, int64_t &bank_out) {
    constexpr int SM = 8;
    const int s = min(selected, min(j1, j2));
    const int count = min(selected, s * s);
    uint32_t e0 = lane < j1 ? pack_entry(to_f32(z[lane]), lane) : 0u;
    uint32_t e1 = lane < j2 ? pack_entry(to_f32(z[j1 + lane]), lane) : 0u;
    // (1) top-s of each factor, in order
    uint32_t f0[SM], f1[SM];
#pragma unroll
    for (int p = 0; p < SM; ++p) {
        f0[p] = f1[p] = 0u;
        if (p < s) {  // uniform
            const uint32_t m0 = wave_max_u32(e0), m1 = wave_max_u32(e1);
            e0 = e0 == m0 ? 0u : e0;
            e1 = e1 == m1 ? 0u : e1;
            f0[p] = m0;
            f1[p] = m1;
        }
    }
    // lane q < SM keeps the ids of slot q of both lists for the bank lookup
    int id0 = 0, id1 = 0;
    float v0 = 0.f, v1 = 0.f;
    const int ci = lane / SM, cl = lane % SM;
#pragma unroll
    for (int p = 0; p < SM; ++p) {
        if (p == lane) id0 = entry_id(f0[p]), id1 = entry_id(f1[p]);
        if (p == ci) v0 = entry_value(f0[p]);
        if (p == cl) v1 = entry_value(f1[p]);
    }
    // (2) candidate (ci, cl) with (i+1)(l+1) <= count, packed with id i*SM + l
    uint32_t pe = (ci < s && cl < s && (ci + 1) * (cl + 1) <= count)
                      ? pack_entry(round_to<bf16_t>(v0 + v1), ci * SM + cl)
                      : 0u;
    uint32_t pl[SM];
#pragma unroll
    for (int p = 0; p < SM; ++p) {
        pl[p] = 0u;
        if (p < count) {
            const uint32_t m = wave_max_u32(pe);
            pe = pe == m ? 0u : pe;
            pl[p] = m;
        }
    }
    // (3) softmax over the selected sums in FP32, summed in selection order
    const float top = entry_value(pl[0]);
    float ex[SM], total = 0.f;
#pragma unroll
    for (int p = 0; p < SM; ++p) {
        ex[p] = expf(entry_value(pl[p]) - top);
        if (p < count) total += ex[p];
    }
    float mine = 0.f;
    int64_t bank = 0;
#pragma unroll
    for (int p = 0; p < SM; ++p) {
        const int c = entry_id(pl[p]) & (SM * SM - 1);
        const int b0 = __builtin_amdgcn_readlane(id0, c / SM), b1 = __builtin_amdgcn_readlane(id1, c % SM);
        if (p == lane) {
            mine = ex[p];
            bank = int64_t(b0) * j2 + b1;
        }
    }
    weight = round_to<bf16_t>(mine / total);
    bank_out = bank;
    return count;
}

}  // namespace bdm

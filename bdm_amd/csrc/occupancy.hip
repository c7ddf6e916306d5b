// Bank occupancy over the segments of a write-only dispatch.
//
// Reference: bank_occupancy (reproduction/experiments/
// elastic_bank_regularizer.py:10-25), which scatters log1p(-p) and a 1 per
// write event into [batch, J].  Here the dispatch has already grouped the
// writes by (sequence, bank): one wave per segment sums its events with a
// fixed butterfly, so the totals need no atomics and repeat bit for bit.
//
// The same pass can record each bank's first write position.  That is the
// copy-on-write accounting of the reference (APPENDIX.md:511-584,
// scripts/verify_results.py:190-235): a bank holds private
// state from its first write on, so the banks held after a prefix of t
// positions are those whose first write is < t, and written_bank_curve_kernel
// counts them for any list of prefixes without another pass over the routes.
#include "bdm_common.h"

namespace bdm {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void bank_occupancy_kernel(const T *__restrict__ weights,
                                                             const uint8_t *__restrict__ valid,
                                                             const int64_t *__restrict__ order,
                                                             const int64_t *__restrict__ cu, int64_t segments,
                                                             int64_t routes, int kw, int64_t time,
                                                             float *__restrict__ totals,
                                                             int32_t *__restrict__ counts,
                                                             int32_t *__restrict__ first_write) {
    const int lane = threadIdx.x % kWave;
    const int64_t seg = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (seg >= segments) return;
    const int64_t start = cu[seg], end = cu[seg + 1];
    float sum = 0.f;
    int count = 0;
    int first = INT32_MAX;  // no valid write
    for (int64_t e = start + lane; e < end; e += kWave) {
        int64_t route = order[e];
        route = route < 0 ? 0 : (route >= routes ? routes - 1 : route);
        const int64_t token = route / kw;
        const bool ok = valid == nullptr || valid[token] != 0;
        const float p = weights ? fminf(fmaxf(to_f32(weights[route]), 0.f), 1.f - 1e-6f) : 0.f;
        sum += ok ? log1pf(-p) : 0.f;
        count += ok ? 1 : 0;
        first = ok ? min(first, int(token % time)) : first;
    }
#pragma unroll
    for (int m = kWave / 2; m >= 1; m >>= 1) {
        sum += __shfl_xor(sum, m, kWave);
        count += __shfl_xor(count, m, kWave);
        first = min(first, __shfl_xor(first, m, kWave));
    }
    if (lane == 0) {
        totals[seg] = sum;
        counts[seg] = count;
        if (first_write) first_write[seg] = first;
    }
}

// One wave per (sequence, prefix): the banks of the sequence whose first
// write lies before the prefix end.
__global__ __launch_bounds__(256) void written_bank_curve_kernel(const int32_t *__restrict__ first_write,
                                                                 int64_t batch, int banks,
                                                                 const int64_t *__restrict__ prefixes,
                                                                 int prefix_count, int32_t *__restrict__ written) {
    const int lane = threadIdx.x % kWave;
    const int64_t item = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (item >= batch * prefix_count) return;
    const int64_t b = item / prefix_count;
    const int64_t limit = prefixes[item % prefix_count];
    const int32_t *row = first_write + b * banks;
    int count = 0;
    for (int j = lane; j < banks; j += kWave) count += int64_t(row[j]) < limit ? 1 : 0;
#pragma unroll
    for (int m = kWave / 2; m >= 1; m >>= 1) count += __shfl_xor(count, m, kWave);
    if (lane == 0) written[item] = count;
}

}  // namespace
}  // namespace bdm

extern "C" int bdm_bank_occupancy(const void *write_weights, int32_t weight_dtype, const uint8_t *valid,
                                  const int64_t *order, const int64_t *cu_seqlens, int64_t batch, int64_t time,
                                  int32_t write_banks, int32_t bank_count, float *totals, int32_t *counts,
                                  int32_t *first_write, void *stream) {
    using namespace bdm;
    if (batch <= 0 || time <= 0 || write_banks <= 0 || bank_count <= 0)
        return fail(BDM_ERR_INVALID, "occupancy: bad geometry");
    if (weight_dtype != BDM_BF16 && weight_dtype != BDM_F32) return fail(BDM_ERR_INVALID, "occupancy: dtype");
    if (!order || !cu_seqlens || !totals || !counts)
        return fail(BDM_ERR_INVALID, "occupancy: null pointer");
    if (time > INT32_MAX) return fail(BDM_ERR_UNSUPPORTED, "occupancy: positions past int32");
    if (batch * int64_t(bank_count) > int64_t(INT32_MAX) * 4)
        return fail(BDM_ERR_UNSUPPORTED, "occupancy: too many segments");
    const int64_t segments = batch * bank_count, routes = batch * time * write_banks;
    const unsigned blocks = unsigned((segments + 3) / 4);
    hipStream_t s = as_stream(stream);
    if (weight_dtype == BDM_BF16)
        bank_occupancy_kernel<bf16_t><<<blocks, 256, 0, s>>>(static_cast<const bf16_t *>(write_weights), valid,
                                                             order, cu_seqlens, segments, routes, write_banks,
                                                             time, totals, counts, first_write);
    else
        bank_occupancy_kernel<float><<<blocks, 256, 0, s>>>(static_cast<const float *>(write_weights), valid,
                                                            order, cu_seqlens, segments, routes, write_banks,
                                                            time, totals, counts, first_write);
    return check_launch("bank_occupancy_kernel");
}

extern "C" int bdm_written_bank_curve(const int32_t *first_write, int64_t batch, int32_t bank_count,
                                      const int64_t *prefixes, int32_t prefix_count, int32_t *written,
                                      void *stream) {
    using namespace bdm;
    if (batch <= 0 || bank_count <= 0 || prefix_count <= 0)
        return fail(BDM_ERR_INVALID, "written_bank_curve: bad geometry");
    if (!first_write || !prefixes || !written) return fail(BDM_ERR_INVALID, "written_bank_curve: null pointer");
    const int64_t items = batch * prefix_count;
    if ((items + 3) / 4 > int64_t(INT32_MAX)) return fail(BDM_ERR_UNSUPPORTED, "written_bank_curve: too many rows");
    written_bank_curve_kernel<<<unsigned((items + 3) / 4), 256, 0, as_stream(stream)>>>(
        first_write, batch, bank_count, prefixes, prefix_count, written);
    return check_launch("written_bank_curve_kernel");
}

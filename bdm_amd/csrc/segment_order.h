// Longest-first segment order for the recurrence kernels: one workgroup
// per segment (and head group), blocks reach the 8 XCDs round-robin in
// dispatch order (x fastest), and a block starts when a slot frees.  Ranking
// each XCD range's segments by length lets the k-th block of XCD x run item
// k of its range, long segments in the first rounds and short ones in the
// last, so the rounds end together instead of in a long tail.
#pragma once

#include <cstdlib>
#include <mutex>

#include "bdm_common.h"

namespace bdm {
namespace {

// Ranges of at most this many segments are ranked (a range's lengths sit in LDS).
constexpr int kOrderMaxRange = 1024;

// order[x * range + rank] = the segment of rank `rank` in XCD range x (the
// `range` consecutive segments from x * range), by decreasing length, ties by
// index: a segment's rank counts the longer segments and the equal ones
// before it.  Grid (8, ceil(range / 16)) of 256 threads: a workgroup ranks 16
// segments of its range, each against 16 slices of the range (one thread per
// segment and slice), the 16 counts summed in LDS.
constexpr int kOrderRows = 16;
constexpr int kOrderParts = 256 / kOrderRows;
__global__ __launch_bounds__(256) void segment_order_kernel(const int64_t *__restrict__ cu, int range,
                                                            int *__restrict__ order) {
    // (launched with 256 threads per workgroup)
    // lengths padded to a multiple of 16 with -1 (never longer than or equal
    // to a real length), read four at a time
    __shared__ __align__(16) int s_len[kOrderMaxRange];
    __shared__ int s_rank[kOrderRows];
    const int base = int(blockIdx.x) * range;
    const int padded = (range + 15) & ~15;
    const int t = int(threadIdx.x);
    // (all of a thread's loads in flight together: at most kOrderMaxRange / 256 per thread)
#pragma unroll
    for (int n = 0; n < kOrderMaxRange / 256; ++n) {
        const int i = t + n * 256;
        if (i < padded) s_len[i] = i < range ? int(cu[base + i + 1] - cu[base + i]) : -1;
    }
    if (t < kOrderRows) s_rank[t] = 0;
    __syncthreads();
    const int i = int(blockIdx.y) * kOrderRows + (t % kOrderRows);
    const int part = t / kOrderRows;
    if (i < range) {
        const int li = s_len[i];
        // slice `part`: groups [part * per, (part + 1) * per) of four
        // lengths, the last slices short or empty
        const int per = (padded / 4 + kOrderParts - 1) / kOrderParts;
        const int g0 = part * per, g1 = min(padded / 4, g0 + per);
        const int j0 = 4 * g0;
        const int4 *lens = reinterpret_cast<const int4 *>(s_len + j0);
        int rank = 0;
#pragma unroll 4
        for (int m = 0; m < g1 - g0; ++m) {
            const int4 l = lens[m];
            const int j = j0 + 4 * m;
            rank += (l.x > li || (l.x == li && j < i)) ? 1 : 0;
            rank += (l.y > li || (l.y == li && j + 1 < i)) ? 1 : 0;
            rank += (l.z > li || (l.z == li && j + 2 < i)) ? 1 : 0;
            rank += (l.w > li || (l.w == li && j + 3 < i)) ? 1 : 0;
        }
        atomicAdd(&s_rank[t % kOrderRows], rank);
    }
    __syncthreads();
    if (part == 0 && i < range) order[base + s_rank[t]] = base + i;
}

// Launch of segment_order_kernel over `nseg` segments (8 ranges).
inline void launch_segment_order(const int64_t *cu, int64_t nseg, int *order, hipStream_t stream) {
    const int range = int(nseg / 8);
    segment_order_kernel<<<dim3(8, unsigned((range + kOrderRows - 1) / kOrderRows)), 256, 0, stream>>>(cu, range,
                                                                                                       order);
}

// The item of the k-th block on an XCD: rounds of `gpr` head groups (the
// groups whose blocks for every segment of the range the XCD's slots hold at
// once, so a token's write segments share that XCD's L2), each round
// segment-major over the range in decreasing length.  The slot that the
// shortest segment of a round frees first takes the longest of the next.
__device__ __forceinline__ void order_item(int64_t k, int range, int groups, int gpr, int &rank, int &group) {
    const int64_t per_round = int64_t(range) * gpr;
    const int round = int(k / per_round);
    const int in_round = min(gpr, groups - round * gpr);
    const int w = int(k - round * per_round);
    rank = w / in_round;
    group = round * gpr + w % in_round;
}

// Blocks of `kernel` (block_threads each) that one XCD holds at once: its
// CUs times the resident blocks per CU.  The occupancy query costs ~10 us of
// host time, on the path between two launches, so each (kernel, threads,
// device) is asked once; 0 if the runtime cannot tell.
inline int64_t xcd_slots(const void *kernel, int block_threads) {
    struct Entry {
        const void *kernel;
        int threads, dev, slots;
    };
    static std::mutex mu;
    static Entry cache[64];
    static int used = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < used; ++i)
        if (cache[i].kernel == kernel && cache[i].threads == block_threads && cache[i].dev == dev)
            return cache[i].slots;
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block_threads, 0) != hipSuccess)
        return 0;
    const int slots = (cus / 8) * per_cu;
    if (used < 64) cache[used++] = Entry{kernel, block_threads, dev, slots};
    return slots;
}

// Head groups per round: slots of one XCD over the range's segments, in
// [1, groups].
inline int order_groups_per_round(const void *kernel, int block_threads, int64_t nseg, int groups) {
    const int64_t slots = xcd_slots(kernel, block_threads);
    if (slots <= 0) return 1;
    const int64_t gpr = slots / (nseg / 8);
    return int(gpr < 1 ? 1 : (gpr > groups ? groups : gpr));
}

// Whether a launch over `nseg` segments can take the order.
inline bool order_geometry(int64_t nseg) { return nseg > 0 && nseg % 8 == 0 && nseg / 8 <= kOrderMaxRange; }

// BDM_SEGMENT_ORDER=0 keeps bank order (results are identical either way).
inline bool order_enabled() {
    const char *e = getenv("BDM_SEGMENT_ORDER");
    return !(e && e[0] == '0' && e[1] == 0);
}

}  // namespace
}  // namespace bdm

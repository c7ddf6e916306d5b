// Causal bank dispatch: a stable counting sort of (token, bank) events into
// per-(batch, bank) segments.
//
// Reference: role_bank_dispatch.py:15-38 (_keys, _bounds), :143-153
// (metadata: torch.sort of the int64 keys ((b*J + bank)*T + t)*2 + is_read)
// and the INVERSE/TOKENS maps of _pack (:72-73).  The keys are unique, so the
// sorting permutation is unique; a counting sort by segment that keeps each
// segment's events in (t, write-before-read) order produces the same one.
//
// Three passes over tiles of 32 tokens of one batch:
//   1. tile_count: LDS bit-masks mask[bank] with bit 2*t_local + is_read set
//      for every event of the tile (64-bit LDS atomic OR; order-independent,
//      so deterministic).  popcount(mask[bank]) is the tile's bucket count.
//   2. scan: an exclusive scan over tiles for every (batch, bank) — a tile's
//      base inside its segment — in parallel over banks and tile ranges, and
//      per batch an exclusive scan over banks (segment starts): one
//      workgroup per batch for up to 1024 banks, a multiple of 4
//      (dispatch_batch_scan, which adds the starts to the tile bases and can
//      rank the segments for the recurrence's longest-first order), else per
//      (batch, 64 banks) with the starts left to the scatter.  Batch b's segments start at
//      b*T*(KW+KR): every token adds exactly KW+KR events to its own batch.
//   3. scatter: rebuild the masks; an event's rank inside its tile-bucket is
//      popcount(mask[bank] & below(bit)), i.e. the number of earlier
//      (t, phase) slots of the tile that hit the same bank.  That is the
//      stable order, computed without any serial step.
//
// The masks take one 64-bit LDS word per bank, so that path serves up to
// 8192 banks.  Above that (the reference's T = N = 2^20 whole-model run has
// J = 131,072) the keys themselves are radix-sorted (hipCUB, over only the
// key bits the geometry can set) with the original event index as the value;
// unique keys make the result the same permutation.
#include <hipcub/hipcub.hpp>

#include <mutex>

#include "bdm_common.h"
#include "route_dispatch.h"
#include "segment_order.h"

namespace bdm {
namespace {

constexpr int kTileTokens = 32;  // 2 bits per token in a 64-bit mask
constexpr int kMaxBanks = 8192;  // LDS masks: 64 KiB

struct DispatchGeometry {
    int64_t batch, time, nt;
    int kw, kr, banks;
    int tiles;  // tiles per batch
};

__device__ __forceinline__ int load_bank(const int64_t *__restrict__ wi, const int64_t *__restrict__ ri,
                                         const DispatchGeometry &g, int64_t token, int j, int32_t *status) {
    const int64_t raw = j < g.kw ? wi[token * g.kw + j] : ri[token * g.kr + (j - g.kw)];
    if (raw < 0 || raw >= g.banks) {
        atomicOr(status, int(BDM_ROUTE_OUT_OF_RANGE));
        return raw < 0 ? 0 : g.banks - 1;
    }
    return int(raw);
}

// Fill the tile's LDS masks.  Returns after a barrier.
__device__ void build_masks(unsigned long long *masks, const int64_t *__restrict__ wi,
                            const int64_t *__restrict__ ri, const DispatchGeometry &g, int b, int tile,
                            int32_t *status) {
    for (int x = threadIdx.x; x < g.banks; x += blockDim.x) masks[x] = 0ull;
    __syncthreads();
    const int per_token = g.kw + g.kr;
    const int t0 = tile * kTileTokens;
    const int ntok = min(kTileTokens, int(g.time - t0));
    for (int i = threadIdx.x; i < ntok * per_token; i += blockDim.x) {
        const int tl = i / per_token, j = i - tl * per_token;
        const int64_t token = int64_t(b) * g.time + t0 + tl;
        const int bank = load_bank(wi, ri, g, token, j, status);
        const unsigned long long bit = 1ull << (2 * tl + (j >= g.kw));
        const unsigned long long old = atomicOr(&masks[bank], bit);
        if (old & bit) atomicOr(status, int(BDM_ROUTE_DUPLICATE));
    }
    __syncthreads();
}

__global__ __launch_bounds__(512) void dispatch_tile_count(const int64_t *__restrict__ wi,
                                                           const int64_t *__restrict__ ri, DispatchGeometry g,
                                                           int32_t *__restrict__ tile_counts, int32_t *status) {
    extern __shared__ unsigned long long masks[];
    const int tile = blockIdx.x, b = blockIdx.y;
    build_masks(masks, wi, ri, g, b, tile, status);
    int32_t *out = tile_counts + (int64_t(b) * g.tiles + tile) * g.banks;
    for (int x = threadIdx.x; x < g.banks; x += blockDim.x) out[x] = __popcll(masks[x]);
}

// Per (batch, 64-bank chunk): tile_counts[b][t][bank] becomes each tile's
// offset inside its segment, and totals[b][bank] the segment length.  The
// tiles are split over the kScanWaves waves of the workgroup; a wave loads its
// range kScanBatch counts at a time (all in flight together) and sums it, the
// waves' sums are scanned through LDS, then each wave rewrites its range as
// running offsets, from the counts it still holds when the range is one batch
// (sequences of up to 8,192 tokens), else reloading them a batch at a time.
// It also clears the route flags: the counting pass before it raised them
// and the scatter pass after it raises every one of them again (both build
// the same tile masks), so the caller need not clear the word.
constexpr int kScanWaves = 16, kScanBatch = 16;

__global__ __launch_bounds__(kScanWaves * kWave) void dispatch_tile_scan(DispatchGeometry g,
                                                                         int32_t *__restrict__ tile_counts,
                                                                         int32_t *__restrict__ totals,
                                                                         int32_t *status) {
    __shared__ int32_t part[kScanWaves][kWave];
    const int b = blockIdx.x;
    if (b == 0 && blockIdx.y == 0 && threadIdx.x == 0) *status = 0;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int bank = blockIdx.y * kWave + lane;
    const bool live = bank < g.banks;
    const int per = (g.tiles + kScanWaves - 1) / kScanWaves;
    const int t0 = min(g.tiles, wave * per), t1 = min(g.tiles, t0 + per);
    int32_t *base = tile_counts + int64_t(b) * g.tiles * g.banks + bank;
    auto load_batch = [&](int t, int32_t (&c)[kScanBatch]) {
#pragma unroll
        for (int k = 0; k < kScanBatch; ++k) c[k] = (live && t + k < t1) ? base[int64_t(t + k) * g.banks] : 0;
    };
    int32_t c[kScanBatch];
    int32_t sum = 0;
    for (int t = t0; t < t1; t += kScanBatch) {
        load_batch(t, c);
#pragma unroll
        for (int k = 0; k < kScanBatch; ++k) sum += c[k];
    }
    part[wave][lane] = sum;
    __syncthreads();
    int32_t running = 0;
    for (int w = 0; w < wave; ++w) running += part[w][lane];
    const bool held = t1 - t0 <= kScanBatch;  // c still holds the wave's whole range
    for (int t = t0; t < t1; t += kScanBatch) {
        if (!held) load_batch(t, c);
#pragma unroll
        for (int k = 0; k < kScanBatch; ++k) {
            if (live && t + k < t1) base[int64_t(t + k) * g.banks] = running;
            running += c[k];
        }
    }
    if (live && wave == kScanWaves - 1) totals[int64_t(b) * g.banks + bank] = running;
}

// Per batch, for up to kBatchScanBanks banks (a multiple of 4): one
// workgroup of 16 waves does the tile scan, the segment starts and, when
// asked, the longest-first segment ranking, so that the scatter after it
// reads each event's position base with one load.  A lane owns 4 consecutive
// banks (16-byte loads and stores: a workgroup moves a batch's counts
// through one CU, whose vector memory unit takes a wave's addresses at a
// fixed rate per lane), the banks split into chunks of 256 (a wave's lanes)
// and the batch's tiles into 16 / chunks ranges, a wave per (chunk, range):
//   1. each wave sums its banks' counts over its tile range;
//   2. a bank's segment length is the sum of its ranges' sums; the exclusive
//      scan of the lengths over banks gives the segment starts, stored as
//      cu_seqlens (batch b's events start at b*T*(KW+KR));
//   3. each wave rewrites its counts as start + the counts of the earlier
//      tiles: the number of the segment's events before the tile, counted
//      from the batch's first event;
//   4. with seg_order, each XCD range inside the batch (the `range`
//      consecutive segments from x * range, the caller's check that the
//      batch holds whole ranges) is ranked by decreasing length, ties by
//      index, as segment_order_kernel ranks it.
// It also clears the route flags, as dispatch_tile_scan does.
constexpr int kBatchScanBanks = 16 * kWave;

// Ascending bitonic sort of 256 keys held by one wave, 4 per lane (item
// 4 * lane + r in k[r]): compare-exchanges of partners 1 and 2 apart inside a
// lane, of partners 4..128 apart across lanes (__shfl_xor).
constexpr int kWaveSortItems = 4 * kWave;
__device__ __forceinline__ void wave_bitonic_sort(uint32_t (&k)[4], int lane) {
#pragma unroll
    for (int size = 2; size <= kWaveSortItems; size <<= 1) {
#pragma unroll
        for (int j = size >> 1; j > 0; j >>= 1) {
            if (j >= 4) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int e = 4 * lane + r;
                    const uint32_t other = __shfl_xor(k[r], j >> 2, kWave);
                    // the lower index of a pair keeps the smaller key in an
                    // ascending block, the larger in a descending one
                    const bool keep_min = ((e & j) == 0) == ((e & size) == 0);
                    k[r] = keep_min ? min(k[r], other) : max(k[r], other);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (r & j) continue;
                    const bool up = ((4 * lane + r) & size) == 0;
                    const uint32_t lo = min(k[r], k[r | j]), hi = max(k[r], k[r | j]);
                    k[r] = up ? lo : hi;
                    k[r | j] = up ? hi : lo;
                }
            }
        }
    }
}
constexpr int kBatchScanHold = 8;  // tiles whose counts a lane keeps between passes 1 and 3

__global__ __launch_bounds__(kBatchScanBanks) void dispatch_batch_scan(DispatchGeometry g,
                                                                       int32_t *__restrict__ tile_counts,
                                                                       int64_t *__restrict__ cu_seqlens,
                                                                       int32_t *status, int *__restrict__ seg_order,
                                                                       int range) {
    __shared__ int4 part[16][kWave];
    __shared__ int32_t s_len[kBatchScanBanks];
    __shared__ int32_t s_start[kBatchScanBanks];
    __shared__ int32_t wave_sums[16];
    const int b = int(blockIdx.x), t = int(threadIdx.x);
    if (b == 0 && t == 0) *status = 0;
    // (wave-uniform values in scalar registers, so that a row's address is
    // scalar arithmetic plus the lane's fixed offset)
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave), lane = t % kWave;
    const int chunks = (g.banks + 4 * kWave - 1) / (4 * kWave), slices = 16 / chunks;
    const int chunk = wave % chunks, slice = wave / chunks;
    const int bank4 = 4 * (chunk * kWave + lane);  // the lane's first bank
    const bool active = slice < slices, live = active && bank4 < g.banks;
    const int per = (g.tiles + slices - 1) / slices;
    const int t0 = min(g.tiles, slice * per), t1 = min(g.tiles, t0 + per);
    // a batch's counts take under 4 GiB; lanes past the last bank read banks
    // 0..3 and keep nothing
    char *base = reinterpret_cast<char *>(tile_counts + int64_t(b) * g.tiles * g.banks);
    const uint32_t row_bytes = uint32_t(g.banks) * 4u, lane_off = uint32_t(live ? bank4 : 0) * 4u;
    auto cell = [&](int tt) -> int4 & {
        return *reinterpret_cast<int4 *>(base + size_t(uint32_t(tt) * row_bytes) + lane_off);
    };
    // counts of tiles tt .. tt + kBatchScanHold - 1 of the wave's range (0 past it)
    auto load_cells = [&](int tt, int4 (&c)[kBatchScanHold]) {
        if (tt + kBatchScanHold <= t1) {
#pragma unroll
            for (int k = 0; k < kBatchScanHold; ++k) c[k] = cell(tt + k);
        } else {
#pragma unroll
            for (int k = 0; k < kBatchScanHold; ++k) c[k] = tt + k < t1 ? cell(tt + k) : make_int4(0, 0, 0, 0);
        }
    };
    // 1. range sums
    int4 c[kBatchScanHold];
    int4 sum = make_int4(0, 0, 0, 0);
    if (active) {
        for (int tt = t0; tt < t1; tt += kBatchScanHold) {
            load_cells(tt, c);
#pragma unroll
            for (int k = 0; k < kBatchScanHold; ++k) {
                sum.x += c[k].x;
                sum.y += c[k].y;
                sum.z += c[k].z;
                sum.w += c[k].w;
            }
        }
        part[wave][lane] = sum;
    }
    __syncthreads();
    // 2. lengths and starts (thread t takes bank t)
    int32_t len = 0;
    if (t < g.banks) {
        const int c4 = t / (4 * kWave), l4 = (t / 4) % kWave, e = t % 4;
        for (int s = 0; s < slices; ++s) len += reinterpret_cast<const int32_t *>(&part[s * chunks + c4][l4])[e];
        s_len[t] = len;
    }
    int32_t incl = len;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int32_t up = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += up;
    }
    if (lane == kWave - 1) wave_sums[wave] = incl;
    __syncthreads();
    int32_t start = incl - len;
    for (int w = 0; w < wave; ++w) start += wave_sums[w];
    const int64_t batch_base = int64_t(b) * g.time * (g.kw + g.kr);
    if (t < g.banks) {
        s_start[t] = start;
        cu_seqlens[int64_t(b) * g.banks + t] = batch_base + start;
    }
    if (b == g.batch - 1 && t == 0) cu_seqlens[g.batch * g.banks] = g.nt * (g.kw + g.kr);
    __syncthreads();
    // 3. tile bases
    if (active) {
        int4 running = make_int4(s_start[lane_off / 4u], s_start[lane_off / 4u + 1], s_start[lane_off / 4u + 2],
                                 s_start[lane_off / 4u + 3]);
        for (int s = 0; s < slice; ++s) {
            const int4 q = part[s * chunks + chunk][lane];
            running.x += q.x;
            running.y += q.y;
            running.z += q.z;
            running.w += q.w;
        }
        const bool held = t1 - t0 <= kBatchScanHold;  // c still holds the wave's whole range
        for (int tt = t0; tt < t1; tt += kBatchScanHold) {
            if (!held) load_cells(tt, c);
#pragma unroll
            for (int k = 0; k < kBatchScanHold; ++k) {
                if (tt + k < t1 && live) cell(tt + k) = running;
                running.x += c[k].x;
                running.y += c[k].y;
                running.z += c[k].z;
                running.w += c[k].w;
            }
        }
    }
    // 4. ranking (a range divides the batch's banks).  Ranges of up to 256
    //    segments whose lengths fit in 24 bits (segments hold at most
    //    time * (kw + kr) events): wave w sorts range w of the batch by keys
    //    that order longest first, then lowest index — the complemented
    //    length above the 8-bit index — with padding keys last.
    constexpr uint32_t kSortLenMax = (1u << 24) - 1;
    if (seg_order && range <= kWaveSortItems && g.time * (g.kw + g.kr) <= int64_t(kSortLenMax)) {
        if (wave < g.banks / range) {
            uint32_t k[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 4 * lane + r;
                k[r] = i < range ? ((kSortLenMax - uint32_t(s_len[wave * range + i])) << 8) | uint32_t(i)
                                 : 0xffffffffu;
            }
            wave_bitonic_sort(k, lane);
            const int seg0 = b * g.banks + wave * range;  // the range's first segment
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int pos = 4 * lane + r;
                if (pos < range) seg_order[seg0 + pos] = seg0 + int(k[r] & 255u);
            }
        }
    } else if (seg_order) {
        // kBatchScanBanks / banks threads per segment, each counting the
        // longer (or equal and earlier) segments in a slice of its range
        __shared__ int32_t s_rank[kBatchScanBanks];
        if (t < g.banks) s_rank[t] = 0;
        __syncthreads();
        const int parts = kBatchScanBanks / g.banks;
        const int i = t / parts, q = t - i * parts;
        if (i < g.banks) {
            const int li = s_len[i];
            const int r0 = i / range * range, per = (range + parts - 1) / parts;
            const int j0 = r0 + min(range, q * per), j1 = r0 + min(range, (q + 1) * per);
            // before i: the longer or equal ones; from i on: the longer ones
            const int jm = max(j0, min(j1, i));
            int rank = 0;
#pragma unroll 8
            for (int j = j0; j < jm; ++j) rank += s_len[j] >= li ? 1 : 0;
#pragma unroll 8
            for (int j = jm; j < j1; ++j) rank += s_len[j] > li ? 1 : 0;
            atomicAdd(&s_rank[i], rank);
        }
        __syncthreads();
        if (t < g.banks) {
            const int seg = b * g.banks + t;
            seg_order[seg / range * range + s_rank[t]] = seg;
        }
    }
}

// One workgroup per (tile, batch).  With STARTS, the batch's segment starts
// first (an exclusive scan of the segment lengths over banks, in LDS; every
// tile of the batch computes the same scan, and tile 0 stores it as
// cu_seqlens), and each of the tile's events goes to start + its tile's
// offset in the segment + its rank in the tile's mask.  Without, tile_base
// already holds start + offset (dispatch_batch_scan).  Batch b's segments
// start at b*T*(KW+KR): every token adds exactly KW+KR events to its own
// batch.
//
// The grid is one-dimensional.  When its size is a multiple of 8, XCD x (the
// blocks x, x + 8, ... in dispatch order) takes the x-th eighth of the
// (batch, tile) items in batch-major order, so one batch's segments are
// written through one XCD's L2 and their cache lines fill there before they
// go to HBM; otherwise block i takes item i.
//
// inverse and tokens may be null (not stored).
template <bool STARTS>
__global__ __launch_bounds__(512) void dispatch_scatter(const int64_t *__restrict__ wi,
                                                        const int64_t *__restrict__ ri, DispatchGeometry g,
                                                        const int32_t *__restrict__ tile_base,
                                                        const int32_t *__restrict__ totals,
                                                        int64_t *__restrict__ cu_seqlens,
                                                        int64_t *__restrict__ order, int64_t *__restrict__ inverse,
                                                        int64_t *__restrict__ tokens, int32_t *status) {
    extern __shared__ unsigned long long masks[];
    int32_t *starts = reinterpret_cast<int32_t *>(masks + g.banks);
    __shared__ int32_t wave_sums[512 / kWave];
    const int64_t items = int64_t(g.tiles) * g.batch, lin = blockIdx.x;
    const int64_t item = items % 8 == 0 ? (lin % 8) * (items / 8) + lin / 8 : lin;
    const int b = int(item / g.tiles), tile = int(item % g.tiles);
    if (STARTS) {
        const int32_t *tot = totals + int64_t(b) * g.banks;
        const int per = (g.banks + int(blockDim.x) - 1) / int(blockDim.x);
        const int lo = min(g.banks, int(threadIdx.x) * per), hi = min(g.banks, lo + per);
        int32_t local = 0;
        for (int x = lo; x < hi; ++x) local += tot[x];
        const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
        int32_t incl = local;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const int32_t up = __shfl_up(incl, d, kWave);
            if (lane >= d) incl += up;
        }
        if (lane == kWave - 1) wave_sums[wave] = incl;
        __syncthreads();
        int32_t running = incl - local;
        for (int w = 0; w < wave; ++w) running += wave_sums[w];
        const int64_t batch_base = int64_t(b) * g.time * (g.kw + g.kr);
        for (int x = lo; x < hi; ++x) {
            starts[x] = running;
            if (tile == 0) cu_seqlens[int64_t(b) * g.banks + x] = batch_base + running;
            running += tot[x];
        }
        if (tile == 0 && b == g.batch - 1 && threadIdx.x == 0) cu_seqlens[g.batch * g.banks] = g.nt * (g.kw + g.kr);
    }
    build_masks(masks, wi, ri, g, b, tile, status);  // ends with a barrier, which also publishes starts
    const int per_token = g.kw + g.kr;
    const int t0 = tile * kTileTokens;
    const int ntok = min(kTileTokens, int(g.time - t0));
    const int32_t *tb = tile_base + (int64_t(b) * g.tiles + tile) * g.banks;
    const int64_t events = g.nt * per_token;
    const int64_t batch_base = int64_t(b) * g.time * per_token;
    for (int i = threadIdx.x; i < ntok * per_token; i += blockDim.x) {
        const int tl = i / per_token, j = i - tl * per_token;
        const int64_t token = int64_t(b) * g.time + t0 + tl;
        const int64_t raw = j < g.kw ? wi[token * g.kw + j] : ri[token * g.kr + (j - g.kw)];
        const int bank = raw < 0 ? 0 : (raw >= g.banks ? g.banks - 1 : int(raw));
        const int bit = 2 * tl + (j >= g.kw);
        const int rank = __popcll(masks[bank] & ((1ull << bit) - 1ull));
        int64_t pos = batch_base + (STARTS ? starts[bank] : 0) + tb[bank] + rank;
        pos = pos < 0 ? 0 : (pos >= events ? events - 1 : pos);
        const int64_t original = j < g.kw ? token * g.kw + j : g.nt * g.kw + token * g.kr + (j - g.kw);
        order[pos] = original;
        if (inverse) inverse[original] = pos;
        if (tokens) tokens[pos] = token;
    }
}

// ---- sort path (bank_count > kMaxBanks)

__device__ __forceinline__ int64_t event_token(int64_t e, const DispatchGeometry &g) {
    return e < g.nt * g.kw ? e / g.kw : (e - g.nt * g.kw) / g.kr;
}

// key[e] = ((b*J + bank)*T + t)*2 + is_read and value[e] = e for every event
// in original order (writes, then reads).
__global__ __launch_bounds__(256) void dispatch_sort_keys(const int64_t *__restrict__ wi,
                                                          const int64_t *__restrict__ ri, DispatchGeometry g,
                                                          uint64_t *__restrict__ keys, int32_t *__restrict__ values,
                                                          int32_t *status) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t events = g.nt * (g.kw + g.kr);
    if (e >= events) return;
    const bool rd = e >= g.nt * g.kw;
    const int64_t raw = rd ? ri[e - g.nt * g.kw] : wi[e];
    int64_t bank = raw;
    if (raw < 0 || raw >= g.banks) {
        atomicOr(status, int(BDM_ROUTE_OUT_OF_RANGE));
        bank = raw < 0 ? 0 : g.banks - 1;
    }
    const int64_t token = event_token(e, g);
    const int64_t b = token / g.time, t = token - b * g.time;
    keys[e] = uint64_t(((b * g.banks + bank) * g.time + t) * 2 + (rd ? 1 : 0));
    values[e] = int32_t(e);
}

// Slot i of the sorted keys: order, inverse and tokens, the segment bounds
// that fall at i, and the duplicate flag (equal neighbouring keys).
__global__ __launch_bounds__(256) void dispatch_sort_finish(const uint64_t *__restrict__ keys,
                                                            const int32_t *__restrict__ values, DispatchGeometry g,
                                                            int64_t *__restrict__ order, int64_t *__restrict__ inverse,
                                                            int64_t *__restrict__ tokens,
                                                            int64_t *__restrict__ cu_seqlens, int32_t *status) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t events = g.nt * (g.kw + g.kr);
    const int64_t nseg = g.batch * g.banks;
    if (i >= events) return;
    const int64_t o = values[i];
    order[i] = o;
    inverse[o] = i;
    tokens[i] = event_token(o, g);
    const uint64_t key = keys[i];
    const int64_t seg = int64_t(key / uint64_t(2 * g.time));
    int64_t prev = -1;
    if (i > 0) {
        const uint64_t pk = keys[i - 1];
        if (pk == key) atomicOr(status, int(BDM_ROUTE_DUPLICATE));
        prev = int64_t(pk / uint64_t(2 * g.time));
    }
    for (int64_t sg = prev + 1; sg <= seg; ++sg) cu_seqlens[sg] = i;  // segments that start here
    if (i == events - 1)
        for (int64_t sg = seg + 1; sg <= nseg; ++sg) cu_seqlens[sg] = events;
}

__global__ void dispatch_clear_status(int32_t *status) {
    if (threadIdx.x == 0) *status = 0;
}

// The LDS-mask path (bank_count <= kMaxBanks): per-tile counts, then, for up
// to kBatchScanBanks banks (a multiple of 4) and a batch's counts under 4 GiB,
// dispatch_batch_scan (tile bases with the segment starts, cu_seqlens, the
// ranking when seg_order is given) and the scatter; otherwise
// dispatch_tile_scan (per-bank tile offsets and segment lengths) and the
// scatter with the segment starts.  Both scans clear the route flags.
// Scratch: batch * (tiles + 1) * banks int32, every element written before
// it is read.  *ranked tells whether seg_order was written (the batch scan
// ranks when every batch holds whole ranges of the order's 8).
int launch_mask_dispatch(const int64_t *wi, const int64_t *ri, const DispatchGeometry &g, int64_t *order,
                         int64_t *inverse, int64_t *tokens, int64_t *cu_seqlens, int32_t *status, void *scratch,
                         hipStream_t s, bool counted = false, int *seg_order = nullptr, bool *ranked = nullptr) {
    auto *tile_counts = static_cast<int32_t *>(scratch);
    const size_t mask_bytes = size_t(g.banks) * sizeof(unsigned long long);
    if (ranked) *ranked = false;
    if (!counted) {  // (the fused routing pass already stored the per-tile counts)
        dispatch_tile_count<<<dim3(unsigned(g.tiles), unsigned(g.batch)), 512, mask_bytes, s>>>(wi, ri, g,
                                                                                              tile_counts, status);
        if (int rc = check_launch("dispatch_tile_count")) return rc;
    }
    const unsigned items = unsigned(int64_t(g.tiles) * g.batch);
    int32_t *totals = tile_counts + int64_t(g.batch) * g.tiles * g.banks;
    if (g.banks <= kBatchScanBanks && g.banks % 4 == 0 && int64_t(g.tiles) * g.banks * 4 < (int64_t(1) << 32) &&
        aligned(scratch, 16)) {
        const int64_t nseg = g.batch * int64_t(g.banks);
        const bool rank = seg_order && order_geometry(nseg) && 8 % g.batch == 0;
        dispatch_batch_scan<<<unsigned(g.batch), kBatchScanBanks, 0, s>>>(g, tile_counts, cu_seqlens, status,
                                                                         rank ? seg_order : nullptr,
                                                                         int(nseg / 8));
        if (int rc = check_launch("dispatch_batch_scan")) return rc;
        if (ranked) *ranked = rank;
        dispatch_scatter<false><<<items, 512, mask_bytes, s>>>(wi, ri, g, tile_counts, nullptr, cu_seqlens, order,
                                                               inverse, tokens, status);
        return check_launch("dispatch_scatter");
    }
    dispatch_tile_scan<<<dim3(unsigned(g.batch), unsigned((g.banks + kWave - 1) / kWave)), kScanWaves * kWave, 0,
                         s>>>(g, tile_counts, totals, status);
    if (int rc = check_launch("dispatch_tile_scan")) return rc;
    const size_t scatter_lds = mask_bytes + size_t(g.banks) * sizeof(int32_t);
    if (scatter_lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void *>(dispatch_scatter<true>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, int(scatter_lds)) != hipSuccess)
        return fail(BDM_ERR_LAUNCH, "dispatch: %zu bytes of LDS for %d banks", scatter_lds, g.banks);
    dispatch_scatter<true><<<items, 512, scatter_lds, s>>>(wi, ri, g, tile_counts, totals, cu_seqlens, order,
                                                           inverse, tokens, status);
    return check_launch("dispatch_scatter");
}

struct SortWorkspace {
    size_t keys = 0, values = 0, temp = 0, total = 0;
};

int key_bits(int64_t batch, int64_t time, int32_t banks) {
    const uint64_t max_key = uint64_t(batch) * uint64_t(banks) * uint64_t(time) * 2;  // exclusive bound
    int bits = 1;
    while (bits < 64 && (uint64_t(1) << bits) < max_key) ++bits;
    return bits;
}

SortWorkspace sort_workspace(int64_t batch, int64_t time, int32_t banks, int64_t events) {
    auto up = [](size_t x) { return (x + 255) / 256 * 256; };
    SortWorkspace w;
    w.keys = up(size_t(events) * sizeof(uint64_t));
    w.values = up(size_t(events) * sizeof(int32_t));
    size_t temp = 0;
    // a failed size query leaves temp 0; the sort itself then reports the error
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, temp, static_cast<const uint64_t *>(nullptr),
                                       static_cast<uint64_t *>(nullptr), static_cast<const int32_t *>(nullptr),
                                       static_cast<int32_t *>(nullptr), int(events), 0,
                                       key_bits(batch, time, banks));
    w.temp = up(temp);
    w.total = 2 * w.keys + 2 * w.values + w.temp;
    return w;
}

}  // namespace
}  // namespace bdm

using bdm::kMaxBanks;
using bdm::kTileTokens;

static int64_t tiles_per_batch(int64_t time) { return (time + kTileTokens - 1) / kTileTokens; }

extern "C" size_t bdm_dispatch_workspace_size(int64_t batch, int64_t time, int32_t bank_count) {
    if (batch <= 0 || time <= 0 || bank_count <= 0 || bank_count > kMaxBanks) return 0;
    // per-tile bucket counts, then per-segment totals
    return size_t(batch) * (size_t(tiles_per_batch(time)) + 1) * size_t(bank_count) * sizeof(int32_t);
}

extern "C" size_t bdm_dispatch_workspace_size_ex(int64_t batch, int64_t time, int32_t bank_count,
                                                 int32_t write_banks, int32_t read_banks) {
    if (batch <= 0 || time <= 0 || bank_count <= 0 || write_banks < 0 || read_banks < 0) return 0;
    if (bank_count <= kMaxBanks) return bdm_dispatch_workspace_size(batch, time, bank_count);
    const int64_t events = batch * time * (int64_t(write_banks) + read_banks);
    if (events <= 0 || events >= (int64_t(1) << 31)) return 0;
    return bdm::sort_workspace(batch, time, bank_count, events).total;
}

extern "C" int bdm_dispatch_build(const int64_t *write_indices, const int64_t *read_indices, int64_t batch,
                                  int64_t time, int32_t write_banks, int32_t read_banks, int32_t bank_count,
                                  int64_t *order, int64_t *inverse, int64_t *tokens, int64_t *cu_seqlens,
                                  int32_t *status, void *workspace, size_t workspace_bytes, void *stream) {
    using namespace bdm;
    if (batch <= 0 || time <= 0 || write_banks < 0 || read_banks < 0 || write_banks + read_banks == 0 ||
        bank_count <= 0)
        return fail(BDM_ERR_INVALID, "dispatch: bad geometry batch=%lld time=%lld KW=%d KR=%d J=%d",
                    (long long)batch, (long long)time, write_banks, read_banks, bank_count);
    const int64_t nt = batch * time;
    const int64_t events = nt * (write_banks + read_banks);
    if (events >= (int64_t(1) << 31) || batch > 65535)
        return fail(BDM_ERR_UNSUPPORTED, "dispatch: %lld events exceed the int32 ranks", (long long)events);
    if ((write_banks && !write_indices) || (read_banks && !read_indices) || !order || !inverse || !tokens ||
        !cu_seqlens || !status)
        return fail(BDM_ERR_INVALID, "dispatch: null pointer");
    const size_t need = bdm_dispatch_workspace_size_ex(batch, time, bank_count, write_banks, read_banks);
    if (!workspace || workspace_bytes < need)
        return fail(BDM_ERR_WORKSPACE, "dispatch: workspace %zu < %zu bytes", workspace_bytes, need);
    DispatchGeometry g{batch, time, nt, write_banks, read_banks, bank_count, int(tiles_per_batch(time))};
    hipStream_t s = as_stream(stream);
    if (bank_count > kMaxBanks) {
        const SortWorkspace w = sort_workspace(batch, time, bank_count, events);
        char *base = static_cast<char *>(workspace);
        auto *keys_in = reinterpret_cast<uint64_t *>(base);
        auto *keys_out = reinterpret_cast<uint64_t *>(base + w.keys);
        auto *vals_in = reinterpret_cast<int32_t *>(base + 2 * w.keys);
        auto *vals_out = reinterpret_cast<int32_t *>(base + 2 * w.keys + w.values);
        void *temp = base + 2 * w.keys + 2 * w.values;
        const unsigned blocks = unsigned((events + 255) / 256);
        dispatch_clear_status<<<1, 64, 0, s>>>(status);
        if (int rc = check_launch("dispatch_clear_status")) return rc;
        dispatch_sort_keys<<<blocks, 256, 0, s>>>(write_indices, read_indices, g, keys_in, vals_in, status);
        if (int rc = check_launch("dispatch_sort_keys")) return rc;
        size_t temp_bytes = w.temp;
        if (hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, keys_in, keys_out, vals_in, vals_out, int(events), 0,
                                               key_bits(batch, time, bank_count), s) != hipSuccess)
            return fail(BDM_ERR_LAUNCH, "dispatch: radix sort failed");
        dispatch_sort_finish<<<blocks, 256, 0, s>>>(keys_out, vals_out, g, order, inverse, tokens, cu_seqlens,
                                                     status);
        return check_launch("dispatch_sort_finish");
    }
    return bdm::launch_mask_dispatch(write_indices, read_indices, g, order, inverse, tokens, cu_seqlens, status,
                                     workspace, s);
}

// ---- the allocation-free dispatch (for callers that cannot allocate: code
//      under HIP graph capture, serving loops, harnesses that forbid it)
//
// Its scratch is this file-scope device array, one copy per GPU, held until
// the process ends.  Host code never passes the array's name to a kernel: the
// name is a host-side stand-in.  The device address comes from
// hipGetSymbolAddress, taken once per device with that device current and
// kept per device.  Every call on a GPU shares that GPU's copy, so calls that
// overlap on one GPU race.  No part of it needs clearing: the counting pass
// writes every per-tile count and the tile scan every segment length before
// anything reads them.
namespace {
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[BDM_DISPATCH_STATIC_SCRATCH_BYTES];
std::mutex g_scratch_lock;
void *g_scratch[kMaxDevices] = {};

int static_scratch(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return bdm::fail(BDM_ERR_LAUNCH, "dispatch (no allocation): no usable current device (%d)", dev);
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    if (!g_scratch[dev]) {
        void *ptr = nullptr;
        const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !ptr)
            return bdm::fail(BDM_ERR_LAUNCH, "dispatch (no allocation): hipGetSymbolAddress on device %d: %s", dev,
                             hipGetErrorString(err));
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return BDM_OK;
}
}  // namespace

extern "C" int bdm_dispatch_build_static(const int64_t *write_indices, const int64_t *read_indices, int64_t batch,
                                         int64_t time, int32_t write_banks, int32_t read_banks, int32_t bank_count,
                                         int64_t *order, int64_t *inverse, int64_t *tokens, int64_t *cu_seqlens,
                                         int32_t *status, void *stream) {
    using namespace bdm;
    if (batch <= 0 || time <= 0 || write_banks < 0 || read_banks < 0 || write_banks + read_banks == 0 ||
        bank_count <= 0)
        return fail(BDM_ERR_INVALID, "dispatch (no allocation): bad geometry batch=%lld time=%lld KW=%d KR=%d J=%d",
                    (long long)batch, (long long)time, write_banks, read_banks, bank_count);
    const int64_t nt = batch * time;
    const int64_t events = nt * (write_banks + read_banks);
    if (events >= (int64_t(1) << 31) || batch > 65535)
        return fail(BDM_ERR_UNSUPPORTED, "dispatch (no allocation): %lld events exceed the int32 ranks",
                    (long long)events);
    if (bank_count > kMaxBanks)
        return fail(BDM_ERR_UNSUPPORTED, "dispatch (no allocation): bank_count %d above %d (the radix-sort path "
                    "needs bdm_dispatch_build and a workspace)", bank_count, kMaxBanks);
    const size_t need = bdm_dispatch_workspace_size(batch, time, bank_count);
    if (need > size_t(BDM_DISPATCH_STATIC_SCRATCH_BYTES))
        return fail(BDM_ERR_UNSUPPORTED, "dispatch (no allocation): needs %zu bytes of scratch, above the %zu-byte "
                    "static buffer; use bdm_dispatch_build with a workspace", need,
                    size_t(BDM_DISPATCH_STATIC_SCRATCH_BYTES));
    if ((write_banks && !write_indices) || (read_banks && !read_indices) || !order || !inverse || !tokens ||
        !cu_seqlens || !status)
        return fail(BDM_ERR_INVALID, "dispatch (no allocation): null pointer");
    void *ptr = nullptr;
    if (int rc = static_scratch(&ptr)) return rc;
    const DispatchGeometry g{batch, time, nt, write_banks, read_banks, bank_count, int(tiles_per_batch(time))};
    return launch_mask_dispatch(write_indices, read_indices, g, order, inverse, tokens, cu_seqlens, status, ptr,
                                as_stream(stream));
}

// ---- routing and dispatch in one call

extern "C" size_t bdm_route_dispatch_workspace_size(const bdm_route_dispatch_args *a) {
    if (!a) return 0;
    return bdm_dispatch_workspace_size_ex(a->batch, a->time, a->factor_first * a->factor_second, a->selected,
                                          a->selected);
}

extern "C" int bdm_route_dispatch(const bdm_route_dispatch_args *a, void *workspace, size_t workspace_bytes,
                                  void *stream) {
    using namespace bdm;
    if (!a) return fail(BDM_ERR_INVALID, "route_dispatch: null args");
    if (a->batch <= 0 || a->time <= 0 || a->factor_first <= 0 || a->factor_second <= 0 || a->selected <= 0)
        return fail(BDM_ERR_INVALID, "route_dispatch: bad geometry batch=%lld time=%lld factors %d x %d, %d banks",
                    (long long)a->batch, (long long)a->time, a->factor_first, a->factor_second, a->selected);
    if (!a->write_scores || !a->read_scores || !a->write_weights || !a->read_weights || !a->write_indices ||
        !a->read_indices || !a->order || !a->cu_seqlens || !a->status)
        return fail(BDM_ERR_INVALID, "route_dispatch: null pointer");
    const int64_t banks64 = int64_t(a->factor_first) * a->factor_second;
    if (banks64 > INT32_MAX) return fail(BDM_ERR_UNSUPPORTED, "route_dispatch: too many banks");
    const int32_t banks = int32_t(banks64);
    const int64_t nt = a->batch * a->time;
    const int k = a->selected;
    const size_t need = bdm_route_dispatch_workspace_size(a);
    if (!workspace || workspace_bytes < need)
        return fail(BDM_ERR_WORKSPACE, "route_dispatch: workspace %zu < %zu bytes", workspace_bytes, need);
    hipStream_t s = as_stream(stream);
    const void *scores[2] = {a->write_scores, a->read_scores};
    const int64_t strides[2] = {a->write_stride, a->read_stride};
    void *weights[2] = {a->write_weights, a->read_weights};
    int64_t *indices[2] = {a->write_indices, a->read_indices};
    const bool fused = banks <= kMaxBanks && nt * 2 * k < (int64_t(1) << 31) && a->batch <= 65535 &&
                       route_tile_count_supported(scores, strides, weights, indices, a->score_dtype,
                                                  a->factor_first, a->factor_second, k);
    bool ranked = false;  // the dispatch's scan ranked the segments
    if (!fused) {
        // the router and the dispatch as separate launches
        if (int rc = bdm_router_select_pair(a->write_scores, a->write_stride, a->read_scores, a->read_stride,
                                            a->score_dtype, nt, a->factor_first, a->factor_second, k,
                                            a->write_weights, a->write_indices, a->read_weights, a->read_indices,
                                            stream))
            return rc;
        if (a->inverse && a->tokens) {
            if (int rc = bdm_dispatch_build(a->write_indices, a->read_indices, a->batch, a->time, k, k, banks,
                                            a->order, a->inverse, a->tokens, a->cu_seqlens, a->status, workspace,
                                            workspace_bytes, stream))
                return rc;
        } else {
            if (banks > kMaxBanks)
                return fail(BDM_ERR_UNSUPPORTED, "route_dispatch: %d banks need the inverse and token maps", banks);
            const DispatchGeometry g{a->batch, a->time, nt, k, k, banks, int(tiles_per_batch(a->time))};
            if (int rc = launch_mask_dispatch(a->write_indices, a->read_indices, g, a->order, a->inverse, a->tokens,
                                              a->cu_seqlens, a->status, workspace, s, false, a->segment_order,
                                              &ranked))
                return rc;
        }
    } else {
        const DispatchGeometry g{a->batch, a->time, nt, k, k, banks, int(tiles_per_batch(a->time))};
        if (int rc = launch_route_tile_count(scores, strides, weights, indices, a->batch, a->time, a->factor_first,
                                             a->factor_second, static_cast<int32_t *>(workspace), a->status, s))
            return rc;
        if (int rc = launch_mask_dispatch(a->write_indices, a->read_indices, g, a->order, a->inverse, a->tokens,
                                          a->cu_seqlens, a->status, workspace, s, true, a->segment_order, &ranked))
            return rc;
    }
    if (a->segment_order && !ranked && order_geometry(a->batch * int64_t(banks))) {
        launch_segment_order(a->cu_seqlens, a->batch * int64_t(banks), a->segment_order, s);
        return check_launch("segment_order_kernel");
    }
    return BDM_OK;
}

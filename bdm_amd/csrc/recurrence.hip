// Routed GDN2 bank recurrence (forward) and the r-weighted read combine.
//
// Reference semantics: _pack (role_bank_dispatch.py:41-73), decay_transform
// (routed_update.py:5-13), _role_forward/_write (role_bank_kernel.py:32-73),
// _readout (role_bank_dispatch.py:201-231); stateful variants in
// forward_rows.py:10-194 (final state) and inference.py:70-85.
//
// Layout of the work (MI355X): one workgroup per (batch, bank) segment runs
// that segment's events in packed order for every head at once.  A lane owns
// CPL value columns of one head and keeps all S rows of those columns in
// registers (S*CPL FP32 values), so the erase reduction over rows is in-lane
// and a write costs three FMA-class ops per state element.  The per-event
// metadata (token, route weight, role) is shared by all heads and staged
// through LDS 64 events at a time; the per-token controller rows are
// prefetched one event ahead in registers.
//
// Segments of one batch are mapped to one XCD where the grid allows it
// (segment = (blockIdx % 8) * (segments / 8) + blockIdx / 8): the 16 events of
// a token then run on the same XCD and its controller rows are fetched into
// one L2 instead of eight.
//
// Read results (one S-row contraction per read event and head) go to a BF16
// (ctrl dtype) buffer indexed by the read's original slot token*KR + j; the
// combine kernel adds a token's KR reads in increasing bank id, rounding after
// every add (the production readout order).
#include <type_traits>

#include "bdm_common.h"
#include "recurrence_ops.h"

namespace bdm {
namespace {

constexpr int kStage = 64;  // events staged per LDS batch

template <typename T>
struct ForwardParams {
    const T *q, *k, *b;
    const float *g;
    const T *v, *w;
    const T *ww, *rw;
    const int64_t *order, *cu;
    const void *initial;
    void *final_state;
    void *snap;
    T *zbuf;
    int64_t init_bstride;
    int64_t nt, time;
    int heads, s_real, width, banks, kw, kr;
    int lanes_per_head, heads_per_block;
    int round_interval, routed_decay;
    int snap_interval;  // events between snapshots (0: none); equals round_interval when rounding
    int init_dtype, final_dtype, snap_dtype;
    int xcd_remap;
    float scale;
};

// Load `S` per-row controller values of one (token, head); rows >= s_real are 0.
template <int S, typename E>
__device__ __forceinline__ void load_rows(const E *p, int s_real, float (&out)[S]) {
    if (s_real == S) {
        load_row<S>(p, out);
    } else {
#pragma unroll
        for (int r = 0; r < S; ++r) out[r] = r < s_real ? to_f32(p[r]) : 0.f;
    }
}

template <int S, int CPL>
__device__ __forceinline__ void load_state(const void *base, int dtype, int64_t offset, int width, int s_real,
                                           float (&h)[S][CPL]) {
#pragma unroll
    for (int r = 0; r < S; ++r) {
        if (r < s_real) {
            if (dtype == BDM_BF16)
                load_row<CPL>(static_cast<const bf16_t *>(base) + offset + int64_t(r) * width, h[r]);
            else
                load_row<CPL>(static_cast<const float *>(base) + offset + int64_t(r) * width, h[r]);
        } else {
#pragma unroll
            for (int c = 0; c < CPL; ++c) h[r][c] = 0.f;
        }
    }
}

template <int S, int CPL>
__device__ __forceinline__ void store_state(void *base, int dtype, int64_t offset, int width, int s_real,
                                            const float (&h)[S][CPL]) {
#pragma unroll
    for (int r = 0; r < S; ++r) {
        if (r < s_real) {
            if (dtype == BDM_BF16)
                store_row<CPL>(static_cast<bf16_t *>(base) + offset + int64_t(r) * width, h[r]);
            else
                store_row<CPL>(static_cast<float *>(base) + offset + int64_t(r) * width, h[r]);
        }
    }
}

// Registers of one event's per-lane operands (one head).
template <int S, int CPL>
struct EventOperands {
    float key[S];   // k for a write, q for a read
    float gate[S];  // g
    float erase[S]; // b
    float value[CPL];
    float wgate[CPL];
};

template <typename T, int S, int CPL>
__device__ __forceinline__ void fetch_event(const ForwardParams<T> &p, int64_t token, bool is_read, int head,
                                            int col0, EventOperands<S, CPL> &ev) {
    const int64_t row = token * p.heads + head;
    if (is_read) {
        load_rows<S>(p.q + row * p.s_real, p.s_real, ev.key);
    } else {
        load_rows<S>(p.k + row * p.s_real, p.s_real, ev.key);
        load_rows<S>(p.g + row * p.s_real, p.s_real, ev.gate);
        load_rows<S>(p.b + row * p.s_real, p.s_real, ev.erase);
        load_row<CPL>(p.v + row * p.width + col0, ev.value);
        load_row<CPL>(p.w + row * p.width + col0, ev.wgate);
    }
}

template <typename T, int S, int CPL>
__global__ __launch_bounds__(256) void routed_forward_kernel(ForwardParams<T> p) {
    __shared__ int64_t s_token[kStage];
    __shared__ int64_t s_slot[kStage];  // read: original read slot; write: -1
    __shared__ float s_weight[kStage];

    const int nseg = gridDim.x;
    const int seg = p.xcd_remap ? int((blockIdx.x % 8) * (nseg / 8) + blockIdx.x / 8) : int(blockIdx.x);
    const int bank = seg % p.banks;
    const int64_t bidx = seg / p.banks;
    const int head = blockIdx.y * p.heads_per_block + int(threadIdx.x) / p.lanes_per_head;
    const bool active = int(threadIdx.x) < p.heads_per_block * p.lanes_per_head && head < p.heads;
    const int col0 = (int(threadIdx.x) % p.lanes_per_head) * CPL;
    const int64_t start = p.cu[seg], end = p.cu[seg + 1];
    const int64_t write_events = p.nt * p.kw;
    const int64_t events = p.nt * (p.kw + p.kr);
    const bool rounding = p.round_interval > 0;

    float h[S][CPL];
    const int64_t state_offset = ((int64_t(bank) * p.heads + head) * p.s_real) * p.width + col0;
    if (active) {
        load_state<S, CPL>(p.initial, p.init_dtype, bidx * p.init_bstride + state_offset, p.width, p.s_real, h);
        if (rounding) {
#pragma unroll
            for (int r = 0; r < S; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) h[r][c] = round_bf16(h[r][c]);
        }
    }

    for (int64_t base = start; base < end; base += kStage) {
        const int n = int(min(int64_t(kStage), end - base));
        __syncthreads();
        if (int(threadIdx.x) < n) {
            int64_t o = p.order[base + threadIdx.x];
            o = o < 0 ? 0 : (o >= events ? events - 1 : o);
            const bool rd = o >= write_events;
            const int64_t route = rd ? o - write_events : o;
            s_token[threadIdx.x] = rd ? route / p.kr : route / p.kw;
            s_slot[threadIdx.x] = rd ? route : -1;
            s_weight[threadIdx.x] = rd ? to_f32(p.rw[route]) : to_f32(p.ww[route]);
        }
        __syncthreads();
        if (!active) continue;

        EventOperands<S, CPL> cur, nxt;
        fetch_event<T, S, CPL>(p, s_token[0], s_slot[0] >= 0, head, col0, cur);
        for (int i = 0; i < n; ++i) {
            const int64_t slot = s_slot[i];
            const float pw = s_weight[i];
            if (i + 1 < n) fetch_event<T, S, CPL>(p, s_token[i + 1], s_slot[i + 1] >= 0, head, col0, nxt);
            const int64_t offset = base + i - start;
            if (p.snap_interval > 0 && offset > 0 && offset % p.snap_interval == 0) {
                if (rounding) {
#pragma unroll
                    for (int r = 0; r < S; ++r)
#pragma unroll
                        for (int c = 0; c < CPL; ++c) h[r][c] = round_bf16(h[r][c]);
                }
                // Snapshot of the state before event base+i, the start of a
                // replay chunk (role_bank_kernel.py:59-66).  Boundaries of one
                // segment are snap_interval apart and segments are disjoint,
                // so slot = position / interval - 1 is unique per boundary.
                if (p.snap) {
                    const int64_t slot = (base + i) / p.snap_interval - 1;
                    store_state<S, CPL>(p.snap, p.snap_dtype,
                                        ((slot * p.heads + head) * p.s_real) * p.width + col0, p.width,
                                        p.s_real, h);
                }
            }
            if (slot < 0) {
                // write: hd = exp(eg) M ; u = bf(w p) v - (bf(b p) k)^T hd ; M = hd + k u^T
                WriteRows<S> rows;
                prepare_write_rows<T, S>(cur.key, cur.gate, cur.erase, pw, p.routed_decay, rows);
                float ew[CPL];
#pragma unroll
                for (int c = 0; c < CPL; ++c) ew[c] = round_to<T>(cur.wgate[c] * pw);
                apply_write<S, CPL>(h, rows, ew, cur.value);
            } else {
                // read: z = scale * bf(q r)^T M, stored in the value dtype
                float qr[S];
#pragma unroll
                for (int r = 0; r < S; ++r) qr[r] = round_to<T>(cur.key[r] * pw);
                float z[CPL];
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    float acc = 0.f;
#pragma unroll
                    for (int r = 0; r < S; ++r) acc = fmaf(qr[r], h[r][c], acc);
                    z[c] = acc * p.scale;
                }
                store_row<CPL>(p.zbuf + (slot * p.heads + head) * p.width + col0, z);
            }
            cur = nxt;
        }
    }
    if (active && p.final_state) {
        const int64_t final_offset = bidx * (int64_t(p.banks) * p.heads * p.s_real * p.width) + state_offset;
        store_state<S, CPL>(p.final_state, p.final_dtype, final_offset, p.width, p.s_real, h);
    }
}

// ----------------------------------------------------------------------------
// Lazy-decay segment kernel for S <= 8 (the production geometry).
//
// The state of one (segment, head) is kept as M = diag(s) * Mh with a per-row
// scale s.  A write's decay then only updates s (s' = s * exp(eg)), and with
// a = bf(b*p) * k, x = bf(w*p) * v:
//   erase = sum_r (a_r s'_r) Mh_r,   u = x - erase,   Mh_r += (k_r / s'_r) u
// which is M' = hd + k u^T divided row-wise by s', at two FMAs per state
// element instead of three.  Stages of kLazyStage events start at segment
// offsets that are multiples of 16, the rounding/snapshot interval, and s is
// folded back into Mh (Mh *= s, s = 1) at every stage start and at the
// segment end, so every rounding point and snapshot sees the true state, as
// the reference rounds it.  A stage in which some row's s would fall below
// kScaleFloor runs in eager form instead (Mh = M: hd = exp(eg) * M applied
// explicitly: M' = diag(d) M + k u^T, erase = sum_r (a_r d_r) M_r), so
// k / s' stays finite.  A read uses
// gamma_r = scale * bf(q*r)_r * s_r.
//
// The row quantities of every (event, head, row) are computed once per stage
// for the workgroup: all threads compute exp(eg), k, a (or scale*bf(q*r)) in
// parallel, then one lane per (head, row) scans the stage carrying s and
// turns them into alpha = a s', beta = k / s' (or, eager, a and k with the
// decay kept) or gamma.  The lanes that own value columns read them from LDS
// by broadcast; the event loop never rescales the state conditionally.
// CPL consecutive columns of T kept as raw 32-bit words (BF16 pairs unpacked
// on use), so a prefetched row costs CPL/2 (BF16) or CPL (FP32) registers.
template <typename T, int CPL>
struct RawCols;

template <int CPL>
struct RawCols<bf16_t, CPL> {
    static_assert(CPL % 2 == 0, "BF16 pairs");
    uint32_t u[CPL / 2];
    __device__ __forceinline__ void load(const bf16_t *p) {
        if constexpr (CPL % 8 == 0) {
#pragma unroll
            for (int i = 0; i < CPL / 8; ++i) {
                const uint4 q = reinterpret_cast<const uint4 *>(p)[i];
                u[4 * i] = q.x;
                u[4 * i + 1] = q.y;
                u[4 * i + 2] = q.z;
                u[4 * i + 3] = q.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < CPL / 4; ++i) {
                const uint2 q = reinterpret_cast<const uint2 *>(p)[i];
                u[2 * i] = q.x;
                u[2 * i + 1] = q.y;
            }
        }
    }
    __device__ __forceinline__ float get(int c) const {
        const uint32_t word = u[c / 2];
        return __uint_as_float((c & 1) ? (word & 0xffff0000u) : (word << 16));
    }
};

template <int CPL>
struct RawCols<float, CPL> {
    float f[CPL];
    __device__ __forceinline__ void load(const float *p) { load_row<CPL>(p, f); }
    __device__ __forceinline__ float get(int c) const { return f[c]; }
};

__device__ __forceinline__ int64_t uniform_i64(int64_t x) {
    const int lo = __builtin_amdgcn_readfirstlane(int(uint32_t(uint64_t(x))));
    const int hi = __builtin_amdgcn_readfirstlane(int(uint32_t(uint64_t(x) >> 32)));
    return int64_t((uint64_t(uint32_t(hi)) << 32) | uint64_t(uint32_t(lo)));
}

constexpr int kLazyStage = 16;
constexpr int kLazyHeads = 8;  // heads per workgroup
constexpr float kScaleFloor = 0x1p-32f;

// Writes whose v, w rows are in flight.  Measured on C2: deeper prefetch (2,
// 3) or 8 columns per lane at 2 waves/SIMD were slower than this 1-deep
// prefetch with 4 columns per lane at 4 waves/SIMD (128 VGPRs).
constexpr int kPrefetch = 1;

template <typename T, int CPL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8))) void lazy_forward_kernel(
    ForwardParams<T> p) {
    constexpr int S = 8;
    __shared__ int64_t s_token[kLazyStage];
    __shared__ int64_t s_slot[kLazyStage];  // read: original read slot; write: -1
    __shared__ float s_weight[kLazyStage];
    __shared__ float s_rows[kLazyStage][kLazyHeads][3][S];
    __shared__ float s_fold[kLazyHeads][S];
    __shared__ int s_eager;
    __shared__ int s_wpos[kLazyStage + 1];  // event index of each write of the stage, then n
    __shared__ int s_nw;

    const int nseg = gridDim.x;
    const int seg = p.xcd_remap ? int((blockIdx.x % 8) * (nseg / 8) + blockIdx.x / 8) : int(blockIdx.x);
    const int bank = seg % p.banks;
    const int64_t bidx = seg / p.banks;
    const int head0 = blockIdx.y * p.heads_per_block;
    const int nheads = min(p.heads_per_block, p.heads - head0);
    const int tid = threadIdx.x;
    // Lanes past the block's heads (when nheads * lanes_per_head is not a
    // multiple of the wave) shadow lanes of the last head: they compute the
    // identical values and store them to the same addresses, so every lane
    // runs the same control flow and no store needs a lane condition.
    const int lh = min(tid / p.lanes_per_head, nheads - 1);  // head within the block
    const int head = head0 + lh;
    const int col0 = (tid % p.lanes_per_head) * CPL;
    const bool scanner = tid < nheads * S;  // all in the first wave
    const int scan_head = tid / S, scan_row = tid % S;
    const int64_t start = p.cu[seg], end = p.cu[seg + 1];
    const int64_t write_events = p.nt * p.kw;
    const int64_t events = p.nt * (p.kw + p.kr);
    const bool rounding = p.round_interval > 0;
    float sc = 1.f;  // the scanner's s of (scan_head, scan_row)

    float h[S][CPL];
    const int64_t state_offset = ((int64_t(bank) * p.heads + head) * p.s_real) * p.width + col0;
    load_state<S, CPL>(p.initial, p.init_dtype, bidx * p.init_bstride + state_offset, p.width, p.s_real, h);
    if (rounding) {
#pragma unroll
        for (int r = 0; r < S; ++r)
#pragma unroll
            for (int c = 0; c < CPL; ++c) h[r][c] = round_bf16(h[r][c]);
    }

    for (int64_t base = start; base < end; base += kLazyStage) {
        const int n = int(min(int64_t(kLazyStage), end - base));
        __syncthreads();  // the previous stage's readers are done
        if (tid < n) {
            int64_t o = p.order[base + tid];
            o = o < 0 ? 0 : (o >= events ? events - 1 : o);
            const bool rd = o >= write_events;
            const int64_t route = rd ? o - write_events : o;
            s_token[tid] = rd ? route / p.kr : route / p.kw;
            s_slot[tid] = rd ? route : -1;
            s_weight[tid] = rd ? to_f32(p.rw[route]) : to_f32(p.ww[route]);
        }
        if (tid == 0) s_eager = 0;
        __syncthreads();
        if (tid == 0) {
            int nw = 0;
            for (int i = 0; i < n; ++i)
                if (s_slot[i] < 0) s_wpos[nw++] = i;
            s_wpos[nw] = n;
            s_nw = nw;
        }
        // (1) per (event, head, row): exp(eg), k, a for a write; scale*bf(q*r) for
        // a read.  Thread t owns (head, row) = ((t % 64) / S, t % S) and visits
        // every (blockDim / 64)-th event.
        for (int i = tid / (kLazyHeads * S); i < n; i += blockDim.x / (kLazyHeads * S)) {
            const int hl = (tid % (kLazyHeads * S)) / S, r = tid % S;
            if (hl >= nheads) continue;
            const int64_t at = (s_token[i] * p.heads + head0 + hl) * p.s_real + r;
            const bool live = r < p.s_real;
            const float pw = s_weight[i];
            if (s_slot[i] >= 0) {
                const float q = live ? to_f32(p.q[at]) : 0.f;
                s_rows[i][hl][0][r] = p.scale * round_to<T>(q * pw);
            } else {
                const float k = live ? to_f32(p.k[at]) : 0.f;
                const float g = live ? p.g[at] : 0.f;
                const float b = live ? to_f32(p.b[at]) : 0.f;
                s_rows[i][hl][0][r] = __expf(p.routed_decay ? g * pw : g);
                s_rows[i][hl][1][r] = k;
                s_rows[i][hl][2][r] = round_to<T>(b * pw) * k;
            }
        }
        __syncthreads();
        // (2) one lane per (head, row): fold s at the stage start, then scan
        if (scanner) {
            s_fold[scan_head][scan_row] = sc;
            float run = 1.f;
            bool low = false;
#pragma unroll 1
            for (int i = 0; i < n; ++i) {
                if (s_slot[i] < 0) {
                    run *= s_rows[i][scan_head][0][scan_row];
                    low |= !(run >= kScaleFloor);  // NaN also takes the eager form
                }
            }
            if (low) s_eager = 1;  // benign race: every writer stores 1
        }
        __syncthreads();
        // LDS values every lane reads alike are made wave-uniform explicitly, so
        // the branches on them are scalar and the state is never copied
        const bool eager = __builtin_amdgcn_readfirstlane(s_eager) != 0;
        if (scanner) {
            sc = 1.f;
#pragma unroll 1
            for (int i = 0; i < n; ++i) {
                float *row = &s_rows[i][scan_head][0][scan_row];
                if (s_slot[i] >= 0) {
                    row[0] *= sc;  // gamma
                } else if (!eager) {
                    const float d = row[0], k = row[S], a = row[2 * S];
                    sc *= d;
                    row[0] = a * sc;  // alpha
                    row[S] = k / sc;  // beta
                } else {
                    // eager: alpha = a * decay, beta = k, and the decay itself
                    const float d = row[0], a = row[2 * S];
                    row[0] = a * d;
                    row[2 * S] = d;
                }
            }
        }
        __syncthreads();

        // (3) the value columns.  Fold s into Mh: the true state at the stage
        // start, which is a rounding/snapshot point when the offset is > 0.
#pragma unroll
        for (int r = 0; r < S; ++r) {
            const float f = s_fold[lh][r];
#pragma unroll
            for (int c = 0; c < CPL; ++c) h[r][c] *= f;
        }
        if (base > start) {
            if (rounding) {
#pragma unroll
                for (int r = 0; r < S; ++r)
#pragma unroll
                    for (int c = 0; c < CPL; ++c) h[r][c] = round_bf16(h[r][c]);
            }
            // snapshot of the state before event `base` (see routed_forward_kernel)
            if (p.snap) {
                const int64_t slot = base / p.snap_interval - 1;
                store_state<S, CPL>(p.snap, p.snap_dtype, ((slot * p.heads + head) * p.s_real) * p.width + col0,
                                    p.width, p.s_real, h);
            }
        }
        // Events in packed order, as runs: the reads before each write, then
        // the write, so the state is updated exactly once per iteration and
        // never merged from branches.  The next write's v and w are
        // prefetched as raw rows.
        auto read_event = [&](int i) {
            const int64_t slot = uniform_i64(s_slot[i]);
            const float *row = &s_rows[i][lh][0][0];
            float gamma[S];
#pragma unroll
            for (int r = 0; r < S; ++r) gamma[r] = row[r];
            float z[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                float acc = 0.f;
#pragma unroll
                for (int r = 0; r < S; ++r) acc = fmaf(gamma[r], h[r][c], acc);
                z[c] = acc;
            }
            store_row<CPL>(p.zbuf + (slot * p.heads + head) * p.width + col0, z);
        };
        auto fetch = [&](int i, RawCols<T, CPL> &vv, RawCols<T, CPL> &ww) {
            const int64_t row = uniform_i64(s_token[i]) * p.heads + head;
            vv.load(p.v + row * p.width + col0);
            ww.load(p.w + row * p.width + col0);
        };
        const int nw = __builtin_amdgcn_readfirstlane(s_nw);
        // One loop nest per write form, so the state is carried through a
        // single update form and only merged once per stage.
        auto run = [&](auto eager_form) {
            constexpr bool kEager = decltype(eager_form)::value;
            // v and w of the next kPrefetch writes are in flight while a write
            // and its preceding reads run
            RawCols<T, CPL> vq[kPrefetch], wq[kPrefetch];
#pragma unroll
            for (int d = 0; d < kPrefetch; ++d)
                if (d < nw) fetch(__builtin_amdgcn_readfirstlane(s_wpos[d]), vq[d], wq[d]);
            int i = 0;
#pragma unroll 1
            for (int wk = 0; wk < nw; ++wk) {
                const int wi_ = __builtin_amdgcn_readfirstlane(s_wpos[wk]);
                const RawCols<T, CPL> vc = vq[0], wc = wq[0];
#pragma unroll
                for (int d = 0; d + 1 < kPrefetch; ++d) {
                    vq[d] = vq[d + 1];
                    wq[d] = wq[d + 1];
                }
                if (wk + kPrefetch < nw)
                    fetch(__builtin_amdgcn_readfirstlane(s_wpos[wk + kPrefetch]), vq[kPrefetch - 1], wq[kPrefetch - 1]);
#pragma unroll 1
                for (; i < wi_; ++i) read_event(i);
                i = wi_ + 1;
                const float *row = &s_rows[wi_][lh][0][0];
                const float pw = s_weight[wi_];
                float alpha[S], beta[S], decay[S];
#pragma unroll
                for (int r = 0; r < S; ++r) {
                    alpha[r] = row[r];
                    beta[r] = row[S + r];
                    if constexpr (kEager) decay[r] = row[2 * S + r];
                }
                // x = bf(w p) * v, rounded two columns per conversion
                float x[CPL];
#pragma unroll
                for (int c = 0; c < CPL; c += 2) {
                    float e0 = wc.get(c) * pw, e1 = wc.get(c + 1) * pw;
                    round_pair<T>(e0, e1);
                    x[c] = e0 * vc.get(c);
                    x[c + 1] = e1 * vc.get(c + 1);
                }
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    float erase = 0.f;
#pragma unroll
                    for (int r = 0; r < S; ++r) erase = fmaf(alpha[r], h[r][c], erase);
                    const float u = x[c] - erase;
#pragma unroll
                    for (int r = 0; r < S; ++r) {
                        if constexpr (kEager)
                            h[r][c] = fmaf(decay[r], h[r][c], beta[r] * u);  // M' = d M + k u
                        else
                            h[r][c] = fmaf(beta[r], u, h[r][c]);  // Mh' = Mh + (k / s') u
                    }
                }
            }
#pragma unroll 1
            for (; i < n; ++i) read_event(i);
        };
        if (eager)
            run(std::true_type{});
        else
            run(std::false_type{});
    }
    __syncthreads();
    if (scanner) s_fold[scan_head][scan_row] = sc;
    __syncthreads();
    if (p.final_state) {
#pragma unroll
        for (int r = 0; r < S; ++r) {
            const float f = s_fold[lh][r];
#pragma unroll
            for (int c = 0; c < CPL; ++c) h[r][c] *= f;
        }
        const int64_t final_offset = bidx * (int64_t(p.banks) * p.heads * p.s_real * p.width) + state_offset;
        store_state<S, CPL>(p.final_state, p.final_dtype, final_offset, p.width, p.s_real, h);
    }
}

// y[token, :] = fold over the token's reads in increasing bank id of
// bf(total + z).  One workgroup per token; a thread owns CPL columns.
template <typename T, int CPL>
__global__ __launch_bounds__(256) void ordered_combine_kernel(const T *__restrict__ zbuf,
                                                              const int64_t *__restrict__ read_indices,
                                                              T *__restrict__ y, int kr, int row_width) {
    __shared__ int64_t s_idx[32];
    __shared__ int s_rank_slot[32];
    const int64_t token = blockIdx.x;
    if (int(threadIdx.x) < kr) s_idx[threadIdx.x] = read_indices[token * kr + threadIdx.x];
    __syncthreads();
    if (int(threadIdx.x) < kr) {
        const int64_t mine = s_idx[threadIdx.x];
        int rank = 0;
        for (int j = 0; j < kr; ++j) {
            const int64_t other = s_idx[j];
            rank += (other < mine) || (other == mine && j < int(threadIdx.x));
        }
        s_rank_slot[rank] = threadIdx.x;
    }
    __syncthreads();
    for (int col0 = threadIdx.x * CPL; col0 < row_width; col0 += blockDim.x * CPL) {
        float total[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) total[c] = 0.f;
        for (int j = 0; j < kr; ++j) {
            float z[CPL];
            load_row<CPL>(zbuf + (token * kr + s_rank_slot[j]) * row_width + col0, z);
#pragma unroll
            for (int c = 0; c < CPL; ++c) total[c] = round_to<T>(total[c] + z[c]);
        }
        store_row<CPL>(y + token * row_width + col0, total);
    }
}

// A kernel rather than hipMemsetAsync, so callers may capture it in a graph.
template <typename T>
__global__ __launch_bounds__(256) void zero_fill_kernel(T *__restrict__ out, int64_t count) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < count) out[i] = from_f32<T>(0.f);
}

template <typename T, int S, int CPL, bool kLazy = false>
int launch_forward(const bdm_forward_args &a, T *zbuf, hipStream_t stream) {
    if (a.head_width / CPL > 256)
        return fail(BDM_ERR_UNSUPPORTED, "forward: head_width %d needs more than 256 lanes", a.head_width);
    ForwardParams<T> p{};
    p.q = static_cast<const T *>(a.q);
    p.k = static_cast<const T *>(a.k);
    p.b = static_cast<const T *>(a.b);
    p.g = a.g;
    p.v = static_cast<const T *>(a.v);
    p.w = static_cast<const T *>(a.w);
    p.ww = static_cast<const T *>(a.write_weights);
    p.rw = static_cast<const T *>(a.read_weights);
    p.order = a.order;
    p.cu = a.cu_seqlens;
    p.initial = a.initial;
    p.final_state = a.final_state;
    p.zbuf = zbuf;
    p.init_bstride = a.initial_batch_stride;
    p.nt = a.batch * a.time;
    p.time = a.time;
    p.heads = a.heads;
    p.s_real = a.bank_size;
    p.width = a.head_width;
    p.banks = a.bank_count;
    p.kw = a.write_banks;
    p.kr = a.read_banks;
    p.lanes_per_head = a.head_width / CPL;
    p.heads_per_block = 256 / p.lanes_per_head;
    if (kLazy && p.heads_per_block > kLazyHeads) p.heads_per_block = kLazyHeads;
    if (p.heads_per_block > a.heads) p.heads_per_block = a.heads;
    p.round_interval = a.round_interval;
    p.routed_decay = a.routed_decay;
    p.snap = a.snapshots;
    p.snap_interval = a.round_interval > 0 ? a.round_interval : (a.snapshots ? a.snapshot_interval : 0);
    p.snap_dtype = a.snapshot_dtype;
    p.init_dtype = a.initial_dtype;
    p.final_dtype = a.final_dtype;
    p.scale = a.scale;
    const int64_t nseg = a.batch * a.bank_count;
    p.xcd_remap = (nseg % 8 == 0) ? 1 : 0;
    const int threads = ((p.heads_per_block * p.lanes_per_head + kWave - 1) / kWave) * kWave;
    const dim3 grid(unsigned(nseg), unsigned((a.heads + p.heads_per_block - 1) / p.heads_per_block));
    if constexpr (kLazy) {
        lazy_forward_kernel<T, CPL><<<grid, threads, 0, stream>>>(p);
        if (int rc = check_launch("lazy_forward_kernel")) return rc;
    } else {
        routed_forward_kernel<T, S, CPL><<<grid, threads, 0, stream>>>(p);
        if (int rc = check_launch("routed_forward_kernel")) return rc;
    }

    const int row_width = a.heads * a.head_width;
    const int64_t nt = a.batch * a.time;
    if (a.read_banks > 0) {
        // 16-byte rows where the layout allows (8 BF16 or 4 FP32 columns)
        constexpr int CC = sizeof(T) == 2 ? 8 : 4;
        if (row_width % CC == 0 && a.head_width % CC == 0) {
            const int cthreads = min(256, max(kWave, ((row_width / CC + kWave - 1) / kWave) * kWave));
            ordered_combine_kernel<T, CC><<<unsigned(nt), cthreads, 0, stream>>>(
                zbuf, a.read_indices, static_cast<T *>(a.output), a.read_banks, row_width);
        } else {
            const int cthreads = min(256, max(kWave, ((row_width + kWave - 1) / kWave) * kWave));
            ordered_combine_kernel<T, 1><<<unsigned(nt), cthreads, 0, stream>>>(
                zbuf, a.read_indices, static_cast<T *>(a.output), a.read_banks, row_width);
        }
    } else {
        const int64_t count = nt * row_width;
        zero_fill_kernel<T><<<unsigned((count + 255) / 256), 256, 0, stream>>>(static_cast<T *>(a.output), count);
    }
    return check_launch("ordered_combine_kernel");
}

template <typename T>
int dispatch_forward(const bdm_forward_args &a, T *zbuf, hipStream_t stream) {
    // Vector row loads need 16-byte aligned rows: aligned bases, and a state
    // batch stride that keeps them aligned.
    const bool vec = a.initial_batch_stride % 8 == 0;
    if (a.bank_size <= 8) {
        const int fold = a.round_interval > 0 ? a.round_interval : (a.snapshots ? a.snapshot_interval : kLazyStage);
        constexpr int lc = 4;  // value columns per lane of the lazy kernel
        if (vec && a.head_width % lc == 0 && a.head_width / lc <= 64 && fold == kLazyStage)
            return launch_forward<T, 8, lc, true>(a, zbuf, stream);
        if (vec && a.head_width % 8 == 0) return launch_forward<T, 8, 8>(a, zbuf, stream);
        return launch_forward<T, 8, 1>(a, zbuf, stream);
    }
    if (a.bank_size <= 16) {
        if (vec && a.head_width % 4 == 0) return launch_forward<T, 16, 4>(a, zbuf, stream);
        return launch_forward<T, 16, 1>(a, zbuf, stream);
    }
    if (vec && a.head_width % 2 == 0) return launch_forward<T, 32, 2>(a, zbuf, stream);
    return launch_forward<T, 32, 1>(a, zbuf, stream);
}

size_t elem_size(int dtype) { return dtype == BDM_BF16 ? 2 : 4; }

}  // namespace
}  // namespace bdm

extern "C" size_t bdm_forward_workspace_size(const bdm_forward_args *a) {
    if (!a || a->batch <= 0 || a->time <= 0 || a->heads <= 0 || a->head_width <= 0 || a->read_banks < 0) return 0;
    const size_t bytes = size_t(a->batch) * size_t(a->time) * size_t(a->read_banks) * size_t(a->heads) *
                         size_t(a->head_width) * bdm::elem_size(a->ctrl_dtype);
    return (bytes + 255) / 256 * 256;
}

extern "C" int bdm_forward(const bdm_forward_args *a, void *workspace, size_t workspace_bytes, void *stream) {
    using namespace bdm;
    if (!a) return fail(BDM_ERR_INVALID, "forward: null args");
    if (a->batch <= 0 || a->time <= 0 || a->heads <= 0 || a->bank_size <= 0 || a->head_width <= 0 ||
        a->bank_count <= 0 || a->write_banks < 0 || a->read_banks < 0)
        return fail(BDM_ERR_INVALID, "forward: bad geometry");
    if (a->bank_size > 32) return fail(BDM_ERR_UNSUPPORTED, "forward: bank_size %d > 32", a->bank_size);
    if (a->read_banks > 32) return fail(BDM_ERR_UNSUPPORTED, "forward: read_banks %d > 32", a->read_banks);
    if (a->ctrl_dtype != BDM_BF16 && a->ctrl_dtype != BDM_F32)
        return fail(BDM_ERR_INVALID, "forward: ctrl dtype %d", a->ctrl_dtype);
    if ((a->initial_dtype != BDM_BF16 && a->initial_dtype != BDM_F32) ||
        (a->final_state && a->final_dtype != BDM_BF16 && a->final_dtype != BDM_F32))
        return fail(BDM_ERR_INVALID, "forward: state dtype");
    if (a->batch * a->bank_count > int64_t(INT32_MAX) || a->batch * a->time > (int64_t(1) << 40))
        return fail(BDM_ERR_UNSUPPORTED, "forward: grid too large");
    if (!a->q || !a->k || !a->g || !a->b || !a->v || !a->w || !a->write_weights || !a->read_weights ||
        !a->read_indices || !a->order || !a->cu_seqlens || !a->initial || !a->output)
        return fail(BDM_ERR_INVALID, "forward: null pointer");
    if (a->snapshots) {
        if (a->snapshot_interval <= 0 || (a->round_interval > 0 && a->round_interval != a->snapshot_interval))
            return fail(BDM_ERR_INVALID, "forward: snapshot interval %d must be positive and equal the rounding "
                        "interval %d", a->snapshot_interval, a->round_interval);
        if (a->snapshot_dtype != BDM_BF16 && a->snapshot_dtype != BDM_F32)
            return fail(BDM_ERR_INVALID, "forward: snapshot dtype");
        if (a->round_interval == 0 && a->snapshot_dtype != BDM_F32)
            return fail(BDM_ERR_INVALID, "forward: an unrounded state needs FP32 snapshots");
    }
    const void *ptrs[] = {a->q, a->k, a->g, a->b, a->v, a->w, a->initial, a->output, a->final_state, a->snapshots,
                          workspace};
    for (const void *ptr : ptrs)
        if (ptr && !aligned(ptr, 16)) return fail(BDM_ERR_INVALID, "forward: tensors must be 16-byte aligned");
    const size_t need = bdm_forward_workspace_size(a);
    if (need && (!workspace || workspace_bytes < need))
        return fail(BDM_ERR_WORKSPACE, "forward: workspace %zu < %zu bytes", workspace_bytes, need);
    hipStream_t s = as_stream(stream);
    if (a->ctrl_dtype == BDM_BF16) return dispatch_forward<bf16_t>(*a, static_cast<bf16_t *>(workspace), s);
    return dispatch_forward<float>(*a, static_cast<float *>(workspace), s);
}

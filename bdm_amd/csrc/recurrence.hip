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
// (ctrl dtype) buffer at row token*KR + j, j the read's route slot; the
// combine kernel then streams each token's KR consecutive rows and adds them
// in increasing bank id, rounding after every add (the production readout
// order), ordering the token's KR bank ids itself.
#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <cstring>
#include <type_traits>

#include "bdm_common.h"
#include "recurrence_ops.h"
#include "chunk_forward.h"
#include "segment_order.h"

// The raw buffer load and store intrinsics (MUBUF) of the AMDGPU backend, by
// their intrinsic names (declared at file scope: external linkage).
typedef int32_t i32x2_t __attribute__((ext_vector_type(2)));
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
__device__ i32x2_t raw_buffer_load_x2(i32x4_t rsrc, int32_t voffset, int32_t soffset,
                                      int32_t aux) __asm("llvm.amdgcn.raw.buffer.load.v2i32");
__device__ void raw_buffer_store_x2(i32x2_t data, i32x4_t rsrc, int32_t voffset, int32_t soffset,
                                    int32_t aux) __asm("llvm.amdgcn.raw.buffer.store.v2i32");

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
    int k_shift;  // log2 of KW and KR when both are that power of two, else -1 (route -> token by shift)
    int lanes_per_head, heads_per_block;
    // Column split of wide heads (lazy kernel): `heads` and `width` above are
    // then virtual heads of `width` columns, `split` of them per real head;
    // q, k, g, b rows are per real head (s_heads of them), and the state,
    // snapshot and final-state rows of a real head are row_stride elements.
    int split, s_heads;
    int64_t row_stride;
    int round_interval, routed_decay;
    int snap_interval;  // events between snapshots (0: none); equals round_interval when rounding
    int init_dtype, final_dtype, snap_dtype;
    int xcd_remap;
    float scale;
    // Long segments cut into pieces (prefill policy only, see lazy_forward_kernel):
    const int4 *items;     // pieces of cut segments: (segment, piece q, pieces of the segment, state slot)
    const int *n_items;    // [0]: number of pieces
    int nseg;              // segments (batch * J)
    int piece_blocks;      // MODE 2: blocks of pieces ahead of the segments (a multiple of 8)
    float *pstate;         // [slots, H, S, v] FP32: zero-start end state R_q, then start state M_(q+1)
    float *ptrans;         // [slots, H, S, S] FP32: transition P_q of piece q
    // MODE 0 with xcd_remap: the segments of each XCD's range, longest first
    // (segment_order_kernel), run in rounds of order_gpr head groups; null
    // keeps the range in bank order
    const int *seg_order;
    int order_gpr;
    // MODE 0: the launch runs head groups group_base .. group_base + gridDim.y
    // - 1 (one round of a launch split into rounds; 0 for a whole launch)
    int group_base;
    // Stage path of the rounding policy (MODE 3 and stage_scan_kernel):
    // MODE 0 leaves segments longer than kPieceEvents to it (skip_long), and
    // MODE 3 stores, per stage slot, R and P in pstate / ptrans and, per read
    // route slot, the zero-start read row (z0buf, [NT*KR, H*v] FP32) and its
    // coefficients on the stage's start state (cbuf, [NT*KR, H, S] FP32),
    // and per stage slot the read route slot of each of its 16 events, -1
    // for a write or past the segment (tgt, [slots, 16] int32).
    int skip_long;
    float *z0buf, *cbuf;
    int *tgt;
};

// Events per piece when long segments are cut (a multiple of the stage size).
constexpr int kPieceEvents = 512;

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
    // event and route indices fit in 32 bits (checked by the launcher)
    const int write_events = int(p.nt * p.kw);
    const int events = int(p.nt * (p.kw + p.kr));
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
            s_slot[threadIdx.x] = rd ? route : -1;  // a read's row of zbuf: its route
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
// Lazy-decay segment kernel for S = 8 (the production geometry).
//
// The state of one (segment, head) is kept as M = diag(s) * Mh with a per-row
// scale s.  A write's decay then only updates s (s' = s * exp(eg)), and with
// a = bf(b*p) * k, x = bf(w*p) * v:
//   u = x - sum_r (a_r s'_r) Mh_r,   Mh_r += (k_r / s'_r) u
// which is M' = hd + k u^T divided row-wise by s', at two FMAs per state
// element instead of three.  Stages of kLazyStage events start at segment
// offsets that are multiples of 16, the rounding/snapshot interval, and s is
// folded back into Mh (Mh *= s, s = 1) at every stage start and at the
// segment end, so every rounding point and snapshot sees the true state, as
// the reference rounds it.  A stage in which some row's s would fall below
// kScaleFloor runs in eager form instead (Mh = M: hd = diag(d) M, then
// u = x - sum_r a_r hd_r, M' = hd + k u^T), so k / s' stays finite.  A read uses
// gamma_r = scale * bf(q*r)_r * s_r.
//
// Work of a stage is split in two so its latency is off the critical path:
//  * prep: one lane per (event, head, half of the rows) loads the event's
//    q/k/g/b rows and route weight, computes exp(eg), k, a (or scale*bf(q*r)),
//    and the running scale s of its 4 rows as an inclusive prefix product
//    over the stage's 16 events with DPP row shifts (a 16-lane DPP row holds
//    the 16 events of one (head, half)); it writes -alpha = -a s', beta =
//    k / s' (or the eager operands) and gamma to LDS.
//  * value columns: a lane owns CPL columns of one head with all 8 rows in
//    registers and runs the stage's events in order, reading the row
//    operands from LDS by broadcast.
// The prep of stage s+1 overlaps the value loop of stage s: its row loads are
// issued before the value loop and consumed after it; the packed order is
// loaded and decoded four stages at a time, two such groups ahead of its use
// (an event metadata ring of 8 stages).
// v and w of the next write are prefetched one write ahead within a stage.
//
// x = bf(w*p) * v: w*p is an exact FP32 product of two BF16 values, rounded
// to nearest even by v_cvt_pk_bf16_f32; the product bf(w*p) * v is added to
// the erase sum by v_dot2c_f32_bf16 against an operand whose other half is
// zero, which adds the exact FP32 product of the two BF16 values (the zero
// half multiplies a finite neighbour column).  w*p itself is formed the same
// way, against (p, 0) or (0, p).

// Raw buffer access (MUBUF): a wave-uniform 128-bit resource (base address,
// no stride, no range limit), a per-lane byte offset in a vector register and
// a wave-uniform byte offset in a scalar register, so a row address costs no
// vector instruction.  Offsets are 32-bit: the launcher takes this form only
// for tensors below 4 GiB.
constexpr int32_t kBufferNontemporal = 2;  // cache policy bit: nt

__device__ __forceinline__ i32x4_t buffer_resource(const void *base) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    i32x4_t r;
    r[0] = __builtin_amdgcn_readfirstlane(int32_t(uint32_t(a)));
    r[1] = __builtin_amdgcn_readfirstlane(int32_t(uint32_t(a >> 32) & 0xffffu));  // stride 0
    r[2] = -1;                                                                     // records: no limit
    r[3] = 0x00020000;                                                             // 32-bit data format
    return r;
}

// CPL consecutive columns of T kept as raw 32-bit words (BF16 pairs unpacked
// on use), so a prefetched row costs CPL/2 (BF16) or CPL (FP32) registers.
template <typename T, int CPL>
struct RawCols;

template <int CPL>
struct RawCols<bf16_t, CPL> {
    static_assert(CPL % 4 == 0, "BF16 column groups of 4");
    uint32_t u[CPL / 2];
    // through a buffer resource: row at byte soffset, this lane's columns at voffset
    __device__ __forceinline__ void load_buffer(i32x4_t rsrc, uint32_t voffset, uint32_t soffset);
    __device__ __forceinline__ void load(const bf16_t *p) {
#pragma unroll
        for (int i = 0; i < CPL / 4; ++i) {
            const uint2 q = reinterpret_cast<const uint2 *>(p)[i];
            u[2 * i] = q.x;
            u[2 * i + 1] = q.y;
        }
    }
};

template <int CPL>
__device__ __forceinline__ void RawCols<bf16_t, CPL>::load_buffer(i32x4_t rsrc, uint32_t voffset, uint32_t soffset) {
#pragma unroll
    for (int i = 0; i < CPL / 4; ++i) {
        const i32x2_t q = raw_buffer_load_x2(rsrc, int32_t(voffset + 8 * i), int32_t(soffset), 0);
        u[2 * i] = uint32_t(q[0]);
        u[2 * i + 1] = uint32_t(q[1]);
    }
}

template <int CPL>
struct RawCols<float, CPL> {
    float f[CPL];
    __device__ __forceinline__ void load(const float *p) { load_row<CPL>(p, f); }
};

typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));

// The exact FP32 products of the BF16 halves of a0 and a1 with p (whose
// other half is zero in p_lo = (p, 0) and p_hi = (0, p)): e = {lo(a0) p,
// hi(a0) p, lo(a1) p, hi(a1) p}, as the VOP3P v_dot2_f32_bf16 with the
// inline constant 0 (the builtin with a zero accumulator is selected as
// v_dot2c_f32_bf16, whose accumulator is its destination, and costs a v_mov
// of zero first).  A VALU read of a DOT instruction's result needs 3 wait
// states after it; the compiler inserts them for the DOT instructions it
// generates but cannot see the ones in inline assembly, so the block ends
// with them (s_nop 2), whatever the compiler schedules next.  `after` is a
// value the block is placed after (an unused operand: the block waits for
// a0, a1 from memory, so it goes after work that does not).
__device__ __forceinline__ void dot_products4(uint32_t a0, uint32_t a1, uint32_t p_lo, uint32_t p_hi,
                                              float (&e)[4], float after) {
    asm("v_dot2_f32_bf16 %0, %4, %6, 0\n\t"
        "v_dot2_f32_bf16 %1, %4, %7, 0\n\t"
        "v_dot2_f32_bf16 %2, %5, %6, 0\n\t"
        "v_dot2_f32_bf16 %3, %5, %7, 0\n\t"
        "s_nop 2"
        : "=&v"(e[0]), "=&v"(e[1]), "=&v"(e[2]), "=&v"(e[3])
        : "v"(a0), "v"(a1), "v"(p_lo), "v"(p_hi), "v"(after));
}

// acc + (the exact FP32 product of the BF16 halves of a and b_masked that
// b_masked keeps; its other half is zero): v_dot2c_f32_bf16.
__device__ __forceinline__ float dot_half_acc(float acc, uint32_t a, uint32_t b_masked) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v_t, a), __builtin_bit_cast(bf16x2v_t, b_masked),
                                           acc, false);
}

// A read row of CPL columns stored with nontemporal stores (4-byte words).
template <int CPL>
__device__ __forceinline__ void store_row_nt(bf16_t *p, const float (&z)[CPL]) {
    uint32_t *dst = reinterpret_cast<uint32_t *>(p);
#pragma unroll
    for (int i = 0; i < CPL / 2; ++i) __builtin_nontemporal_store(pack_bf16x2(z[2 * i], z[2 * i + 1]), dst + i);
}
template <int CPL>
__device__ __forceinline__ void store_row_nt(float *p, const float (&z)[CPL]) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) __builtin_nontemporal_store(z[i], p + i);
}

// The gated value of a write, x[c] = bf(w[c] * pw) * v[c], kept in a form
// whose product is added to an accumulator as the last step of the erase sum.
template <typename T, int CPL>
struct GatedValues;

template <int CPL>
struct GatedValues<bf16_t, CPL> {
    // bf(w * pw) of each column, packed with a zero in the other half:
    // lo[i] = (bf(w[2i] pw), 0), hi[i] = (0, bf(w[2i+1] pw))
    uint32_t lo[CPL / 2], hi[CPL / 2];
    uint32_t v[CPL / 2];
    // pw is a BF16 value (the route weight) widened to FP32, so its low 16
    // bits are zero: w * pw is an exact FP32 product, formed by
    // v_dot2_f32_bf16 from the packed w pair and (pw, 0) or (0, pw)
    // (CPL a multiple of 4).
    // p_hi: the weight's FP32 bits, p_lo: the same >> 16 (vector registers:
    // a scalar operand of the inline instruction is outside the compiler's
    // hazard checks, and a scalar write right after it can change the value
    // the instruction reads)
    __device__ __forceinline__ void make_pair(const RawCols<bf16_t, CPL> &w, const RawCols<bf16_t, CPL> &vv,
                                              uint32_t p_hi, uint32_t p_lo, float after) {
#pragma unroll
        for (int i = 0; i < CPL / 2; i += 2) {
            float e[4];
            dot_products4(w.u[i], w.u[i + 1], p_lo, p_hi, e, after);
            lo[i] = pack_bf16x2(e[0], 0.f);
            hi[i] = pack_bf16x2(0.f, e[1]);
            lo[i + 1] = pack_bf16x2(e[2], 0.f);
            hi[i + 1] = pack_bf16x2(0.f, e[3]);
        }
#pragma unroll
        for (int i = 0; i < CPL / 2; ++i) v[i] = vv.u[i];
    }
    // acc + x[c]
    __device__ __forceinline__ float add_to(float acc, int c) const {
        return dot_half_acc(acc, (c & 1) ? hi[c / 2] : lo[c / 2], v[c / 2]);
    }
};

template <int CPL>
struct GatedValues<float, CPL> {
    float x[CPL];
    __device__ __forceinline__ void make(const RawCols<float, CPL> &w, const RawCols<float, CPL> &vv, float pw) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) x[c] = (w.f[c] * pw) * vv.f[c];
    }
    __device__ __forceinline__ void make_pair(const RawCols<float, CPL> &w, const RawCols<float, CPL> &vv,
                                              uint32_t p_hi, uint32_t, float) {
        make(w, vv, __uint_as_float(p_hi));
    }
    __device__ __forceinline__ float add_to(float acc, int c) const { return acc + x[c]; }
};

// Inclusive prefix product over the 16 lanes of a DPP row (lane order).  Each
// step is one v_mul_f32 with a row_shr DPP source and bound_ctrl off: a lane
// whose source lies before the row start does not write, so it keeps x (the
// product with 1), one instruction where a DPP move of 1.0-filled lanes and a
// multiply take two.  The s_nop gives the 2 wait states a DPP read of a VGPR
// needs after a VALU write of it.
__device__ __forceinline__ float row_prefix_product(float x) {
    asm volatile(
        "s_nop 1\n\t"
        "v_mul_f32_dpp %0, %0, %0 row_shr:1 row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_mul_f32_dpp %0, %0, %0 row_shr:2 row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_mul_f32_dpp %0, %0, %0 row_shr:4 row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_mul_f32_dpp %0, %0, %0 row_shr:8 row_mask:0xf bank_mask:0xf"
        : "+v"(x));
    return x;
}

constexpr int kLazyStage = 16;
constexpr float kScaleFloor = 0x1p-32f;

// Raw row data one prep lane loads for its (event, head, 4 rows).
template <typename T>
struct PrepLoads;
template <>
struct PrepLoads<bf16_t> {
    uint2 key, erase;  // k (or q for a read), b: 4 BF16 each
    float4 gate;       // g
    uint32_t weight;   // route weight, BF16 in the low half
    __device__ __forceinline__ float key_at(int r) const {
        const uint32_t w = r < 2 ? key.x : key.y;
        return __uint_as_float((r & 1) ? (w & 0xffff0000u) : (w << 16));
    }
    __device__ __forceinline__ float erase_at(int r) const {
        const uint32_t w = r < 2 ? erase.x : erase.y;
        return __uint_as_float((r & 1) ? (w & 0xffff0000u) : (w << 16));
    }
    __device__ __forceinline__ float weight_f() const { return __uint_as_float(weight << 16); }
};
template <>
struct PrepLoads<float> {
    float4 key, erase, gate;
    float weight_raw;
    __device__ __forceinline__ float key_at(int r) const { return (&key.x)[r]; }
    __device__ __forceinline__ float erase_at(int r) const { return (&erase.x)[r]; }
    __device__ __forceinline__ float weight_f() const { return weight_raw; }
};

template <typename T>
__device__ __forceinline__ void load_vec4(const T *p, uint2 &out) {
    out = *reinterpret_cast<const uint2 *>(p);
}
__device__ __forceinline__ void load_vec4(const float *p, float4 &out) { out = *reinterpret_cast<const float4 *>(p); }

// HB heads per workgroup of 32 * HB threads (HB = 2: one wave, so its
// barriers never wait for other waves; HB = 8 for narrow heads, where the
// value columns of 8 heads fit in 256 lanes).
//
// MODE 0 runs whole segments (one workgroup each).  Under the prefill policy
// (no rounding inside the recurrence, no snapshots) a segment is an affine
// map of its start state, M_end = P M_start + R, so segments longer than
// kPieceEvents are cut into pieces to balance skewed routing:
//   MODE 1 runs, in one launch, the pieces of every cut segment but the
//          last (in the first blocks, so the long ones start first): a
//          middle piece q from a zero state, without reads, storing its end
//          state R_q and transition P_q (the lanes 0..7 of a head also carry
//          the 8 columns of P, started at the identity, through the same
//          write updates with x = 0); a first piece from the segment's
//          initial state with its reads, storing its end state as R_0 and
//          P_0 = 0; then the uncut segments whole, with reads and the final
//          state, in the slots the pieces leave free;
//   piece_scan_kernel composes M_(q+1) = P_q M_q + R_q from the segment's
//          initial state;
//   MODE 2 runs pieces 1.. of each cut segment from their start states M_q,
//          with reads; the last piece stores the final state.
// Under the rounding policy the state is rounded at every stage start, so a
// segment is affine per stage only.  Segments longer than kPieceEvents then
// take the stage path (MODE 0 skips them):
//   MODE 3 runs every piece of those segments with each 16-event stage
//          started from zero: at the stage end it stores the stage's R and P
//          (P carried by lanes 0..7 as in MODE 1) in the stage's slot, and
//          for each read the zero-start row z0 = gamma^T R_t and the
//          coefficients c = gamma^T P_t on the stage's start state;
//   stage_scan_kernel runs M_(k+1) = round(P_k M_k + R_k) along each segment
//          from its rounded initial state, storing each M_k;
//   stage_reads_kernel forms each read of stage k as c^T M_k + z0.
// The sums differ from the sequential form's in FP32 association (and so in
// the BF16 roundings that flips).  MODE 3 takes three waves per SIMD (148
// VGPRs): held to four (128, a few per-lane addresses spilled and reloaded
// once per stage) it ran no faster at C4.
//
// BUF: v, w rows are read and read rows written through buffer resources
// with 32-bit offsets (BF16 controllers; v, w and the read buffer below
// 4 GiB), which spares the vector address arithmetic of every event.
template <typename T, int CPL, int HB, int MODE, bool BUF = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MODE == 3 ? 3 : 4, 8))) void lazy_forward_kernel(
    ForwardParams<T> p) {
    static_assert(!BUF || (std::is_same<T, bf16_t>::value && CPL == 4), "buffer form: BF16, 4 columns per lane");
    constexpr int S = 8;
    constexpr int NE = kLazyStage;
    // Event metadata ring: stage s lives in slot s % kRing.  The packed order
    // is loaded and decoded kGroup stages at a time (64 events, one per lane
    // of wave 0), two groups ahead of their use.
    constexpr int kGroup = 4, kRing = 2 * kGroup;
    __shared__ int s_tok[kRing][NE];
    __shared__ int s_route[kRing][NE];
    __shared__ int s_wpos[kRing][NE + 1];  // stage positions of the writes, then n
    __shared__ int s_wtok[kRing][NE];      // tokens of the writes, in write order
    __shared__ int s_nw[kRing];
    __shared__ int s_n[kRing];
    __shared__ unsigned s_rmask[kRing];    // bit e: event e of the stage is a read
    // Row operands of the current stage (written by the prep of a stage after
    // every wave has left the previous stage's value loop): lazy [0] = -alpha,
    // [1] = beta; eager [0] = -a, [1] = k, [2] = d; a read [0] = gamma; and
    // [3][0..1] the event's route weight bits and bits >> 16 (read with the
    // row's address, into vector registers).  An event's rows are padded by
    // 16 bytes, so that the prep's 16-byte stores from the 16 event lanes of
    // a row fall in distinct banks.
    constexpr int kEventRow = HB * 4 * S + 4;
    __shared__ __align__(16) float s_rows[NE][kEventRow];
    __shared__ float s_fold[HB][S];  // s at the end of the stage (1 for eager)
    __shared__ int s_eager;
    __shared__ int s_flag[2];  // by stage parity: reset two barriers before its next use

    int seg = 0, piece = 0, pieces = 1, pslot = -1;
    int group = int(blockIdx.y);  // head group of the block
    int block = int(blockIdx.x);  // MODE 1, 2: the piece item
    bool is_piece = MODE == 2;
    // Blocks reach the XCDs round-robin in dispatch order (x fastest).  With
    // p.seg_order the k-th segment block of XCD x takes item k of that XCD's
    // range: rounds of head groups (order_item), segments longest first.
    auto ordered_segment = [&](int64_t k, int gpr) {
        const int range = p.nseg / 8;
        int rank;
        order_item(k / 8, range, int(gridDim.y), gpr, rank, group);
        return p.seg_order[int(k % 8) * range + rank];
    };
    if constexpr (MODE == 0) {
        if (p.seg_order) {
            seg = ordered_segment(int64_t(blockIdx.y) * gridDim.x + blockIdx.x, p.order_gpr);
        } else {
            seg = p.xcd_remap ? int((block % 8) * (p.nseg / 8) + block / 8) : block;
        }
        group += p.group_base;
        // the stage path runs the long segments (the whole workgroup leaves together)
        if (p.skip_long && p.cu[seg + 1] - p.cu[seg] > kPieceEvents) return;
    } else if constexpr (MODE == 3) {
        is_piece = true;  // every piece of every long segment, one per block
    } else if constexpr (MODE == 1) {
        // Every head group's pieces first, then the segments: dispatched row
        // by row, the later groups' pieces would wait behind the first
        // group's thousands of short segments; the segments longest first
        // (the cut ones, which leave at once, then the longest uncut), so no
        // long segment starts last.  piece_blocks is a multiple of 8, so the
        // segment part starts on XCD 0.
        const int groups = int(gridDim.y);
        const int64_t linear = int64_t(blockIdx.y) * gridDim.x + blockIdx.x;
        const int64_t piece_part = int64_t(p.piece_blocks) * groups;
        if (linear < piece_part) {
            block = int(linear / groups);
            group = int(linear % groups);
            is_piece = true;
        } else {
            const int64_t k = linear - piece_part;
            if (p.seg_order) {
                seg = ordered_segment(k, groups);
            } else if (p.xcd_remap) {
                const int64_t k8 = k / 8;
                group = int(k8 % groups);
                const int sb = int((k8 / groups) * 8 + k % 8);
                seg = (sb % 8) * (p.nseg / 8) + sb / 8;
            } else {
                group = int(k % groups);
                seg = int(k / groups);
            }
            // a cut segment runs as its pieces (the whole workgroup leaves together)
            if (p.cu[seg + 1] - p.cu[seg] > kPieceEvents) return;
        }
    }
    if (is_piece) {
        // the grid is an upper bound on the pieces
        if (block >= p.n_items[0]) return;
        const int4 it = p.items[block];
        seg = it.x;
        piece = it.y;
        pieces = it.z;
        pslot = it.w;
        if (MODE == 1 && piece == pieces - 1) return;  // the scan never uses a last piece's R and P
        if (MODE == 2 && piece == 0) return;           // MODE 1 ran it from the true start
    }
    // MODE 1 roles: a middle piece runs from zero with its transition and no
    // reads; a first piece from the segment's initial state with its reads,
    // storing its end state as R and a zero P; an uncut segment whole.
    // MODE 3: every stage from zero with its transition, reads kept apart.
    constexpr bool kTrans = MODE == 1 || MODE == 3;  // lanes 0..7 may carry P
    const bool from_zero = (MODE == 1 && pslot >= 0 && piece > 0) || MODE == 3;
    const bool reads_on = MODE != 1 || !from_zero;
    const int bank = seg % p.banks;
    const int64_t bidx = seg / p.banks;
    const int head0 = group * p.heads_per_block;
    const int nheads = min(p.heads_per_block, p.heads - head0);
    const int tid = threadIdx.x;
    // value-column role.  Lanes past the block's heads shadow lanes of the
    // last head: identical values to identical addresses.
    const int lh = min(tid / p.lanes_per_head, nheads - 1);
    const int head = head0 + lh;
    const int col0 = (tid % p.lanes_per_head) * CPL;
    const int64_t hw = int64_t(p.heads) * p.width;  // elements of one token row of v, w, z
    // this lane's byte offset in such a row (rows are addressed from a
    // wave-uniform base plus this 32-bit offset)
    const uint32_t lane_bytes = uint32_t((head * p.width + col0) * int(sizeof(T)));
    // prep role: (event pe, head ph, rows 4*half .. 4*half+3); 32 lanes per head
    const int pe = tid & (NE - 1);
    const int ph = (tid >> 4) >> 1;
    const int half = (tid >> 4) & 1;
    const bool prep_head = ph < nheads;

    int64_t start = p.cu[seg], end = p.cu[seg + 1];
    // MODE 3: the slot of the piece's first stage (stage k of segment s has
    // slot cu[s] / 16 + s + k, distinct over all segments' stages)
    const int64_t stage_slot0 = start / NE + seg + int64_t(piece) * (kPieceEvents / NE);
    if constexpr (MODE != 0) {
        if (pieces > 1) {
            start += int64_t(piece) * kPieceEvents;
            end = min(end, start + kPieceEvents);
        }
    }
    const int64_t write_events = p.nt * p.kw;
    const int64_t events = p.nt * (p.kw + p.kr);
    const bool rounding = MODE == 0 && p.round_interval > 0;
    const int nstages = int((end - start + NE - 1) / NE);

    // Pointers used once per stage or less live in LDS rather than in SGPRs:
    // the event loop keeps most scalar registers busy, and each SGPR the
    // compiler spills to a VGPR lane costs a v_readlane at every use.  Only
    // v, w and zbuf (addressed at every event) stay scalar.
    enum { P_ORDER, P_Q, P_K, P_B, P_G, P_WW, P_RW, P_SNAP, P_FINAL, P_COUNT };
    __shared__ uint64_t s_ptr[P_COUNT];
    if (tid == 0) {
        s_ptr[P_ORDER] = reinterpret_cast<uint64_t>(p.order);
        s_ptr[P_Q] = reinterpret_cast<uint64_t>(p.q);
        s_ptr[P_K] = reinterpret_cast<uint64_t>(p.k);
        s_ptr[P_B] = reinterpret_cast<uint64_t>(p.b);
        s_ptr[P_G] = reinterpret_cast<uint64_t>(p.g);
        s_ptr[P_WW] = reinterpret_cast<uint64_t>(p.ww);
        s_ptr[P_RW] = reinterpret_cast<uint64_t>(p.rw);
        s_ptr[P_SNAP] = reinterpret_cast<uint64_t>(p.snap);
        s_ptr[P_FINAL] = reinterpret_cast<uint64_t>(p.final_state);
    }
    __syncthreads();
    // (a pointer read back from LDS is generic; casting it through the global
    // address space keeps its accesses global, not flat, which would also
    // count against the LDS wait counter)
    auto lds_ptr = [&](int which) -> void * {
        return (void *)(__attribute__((address_space(1))) char *)(s_ptr[which]);
    };

    // ---- metadata of a group of kGroup stages from its packed order entries
    //      (lane e of wave 0: event e % 16 of the group's stage e / 16)
    auto load_group = [&](int group) -> int {
        const int64_t pos = start + int64_t(group) * (kGroup * NE) + tid;
        if (tid < kGroup * NE && pos < end) return int(static_cast<const int64_t *>(lds_ptr(P_ORDER))[pos]);
        return -1;
    };
    auto decode_group = [&](int group, int o) {
        const int sub = (tid >> 4) & (kGroup - 1), e = tid & (NE - 1);
        const int slot = (group * kGroup + sub) % kRing;
        const bool live = o >= 0;
        o = o < 0 ? 0 : (o >= events ? events - 1 : o);
        const bool rd = o >= write_events;
        const int route = rd ? o - write_events : o;
        const uint64_t live_mask = __ballot(live);
        const uint64_t read_mask = __ballot(live && rd);
        const uint64_t write_mask = live_mask & ~read_mask;
        const uint64_t stage_bits = uint64_t(0xffff) << (NE * sub);
        // (a wave-uniform choice: the shift when KW = KR = 2^k, else a division)
        const int tok = p.k_shift >= 0 ? int(uint32_t(route) >> p.k_shift)
                                       : int(uint32_t(route) / uint32_t(rd ? p.kr : p.kw));
        s_tok[slot][e] = tok;
        s_route[slot][e] = route;
        if (live && !rd) {
            const int wk = __popcll(write_mask & stage_bits & ((uint64_t(1) << (tid & 63)) - 1));
            s_wpos[slot][wk] = e;
            s_wtok[slot][wk] = tok;
        }
        if (e == 0) {
            const int n = __popcll(live_mask & stage_bits), nw = __popcll(write_mask & stage_bits);
            s_n[slot] = n;
            s_nw[slot] = nw;
            s_wpos[slot][nw] = n;
            s_rmask[slot] = unsigned((read_mask >> (NE * sub)) & 0xffffu);
        }
    };

    // ---- prep loads of a stage (issued before, consumed after a value loop)
    PrepLoads<T> pl{};
    auto issue_prep = [&](int stage) {
        const int slot = stage % kRing;
        if (stage >= nstages || !prep_head || pe >= s_n[slot]) return;
        const bool rd = (s_rmask[slot] >> pe) & 1u;
        const int64_t row = (int64_t(s_tok[slot][pe]) * p.s_heads + (head0 + ph) / p.split) * S + 4 * half;
        const int route = s_route[slot][pe];
        if (rd) {
            // q in the erase slot: the prep rounds (erase slot) * p for both kinds
            load_vec4(static_cast<const T *>(lds_ptr(P_Q)) + row, pl.erase);
            const T *rw = static_cast<const T *>(lds_ptr(P_RW));
            if constexpr (std::is_same<T, bf16_t>::value)
                pl.weight = rw[route].bits;
            else
                pl.weight_raw = rw[route];
        } else {
            load_vec4(static_cast<const T *>(lds_ptr(P_K)) + row, pl.key);
            load_vec4(static_cast<const T *>(lds_ptr(P_B)) + row, pl.erase);
            pl.gate = *reinterpret_cast<const float4 *>(static_cast<const float *>(lds_ptr(P_G)) + row);
            const T *ww = static_cast<const T *>(lds_ptr(P_WW));
            if constexpr (std::is_same<T, bf16_t>::value)
                pl.weight = ww[route].bits;
            else
                pl.weight_raw = ww[route];
        }
    };
    // compute the row operands of `stage` into buffer stage & 1 (two barriers)
    auto finish_prep = [&](int stage) {
        const int slot = stage % kRing;
        const int n = s_n[slot];
        const bool live = prep_head && pe < n && stage < nstages;
        const bool rd = live && ((s_rmask[slot] >> pe) & 1u);
        const float pw = live ? pl.weight_f() : 0.f;
        // Branch-free over the stage's mix of reads and writes (both kinds
        // share a wave):
        //   write: d = exp(g p) (or exp(g)), prod = -(bf(b p) k) = -a
        //   read:  d = 1, prod = bf(q p) scale = gamma (q sits in the erase slot)
        // Lanes past the stage's events keep d = 1 (the prefix products) and
        // store nothing.
        const bool wr = live && !rd;
        const float gscale = p.routed_decay ? pw : 1.f;  // g * 1 is g exactly
        float d[4], prod[4], sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float e = __expf((&pl.gate.x)[r] * gscale);
            prod[r] = round_to<T>(pl.erase_at(r) * pw) * (rd ? p.scale : -pl.key_at(r));
            d[r] = wr ? e : 1.f;
            sc[r] = row_prefix_product(d[r]);
        }
        bool low = false;
#pragma unroll
        for (int r = 0; r < 4; ++r) low |= !(sc[r] >= kScaleFloor);  // NaN also takes the eager form
        if (__ballot(low) != 0 && (tid & 63) == 0) atomicOr(&s_flag[stage & 1], 1);
        __syncthreads();  // also: every wave has left the previous value loop
        const bool eager = __builtin_amdgcn_readfirstlane(s_flag[stage & 1]) != 0;
        if (live) {
            // lazy: [0] = prod s' (a read: gamma s; a write: -(a s')),
            // [1] = k / s' (v_rcp_f32); eager: [0] = prod, [1] = k, [2] = d.
            // All three rows are stored for every event (a read uses [0] only;
            // [2] is read in eager stages only).
            float4 *row = reinterpret_cast<float4 *>(&s_rows[pe][ph * 4 * S + 4 * half]);
            float r0[4], r1[4];
            if (eager) {  // (wave-uniform)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    r0[r] = prod[r];
                    r1[r] = pl.key_at(r);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    r0[r] = prod[r] * sc[r];
                    r1[r] = pl.key_at(r) * __builtin_amdgcn_rcpf(sc[r]);
                }
            }
            row[0] = make_float4(r0[0], r0[1], r0[2], r0[3]);
            row[S / 4] = make_float4(r1[0], r1[1], r1[2], r1[3]);
            row[2 * S / 4] = make_float4(d[0], d[1], d[2], d[3]);
            if (half == 0) {
                const uint32_t bits = __float_as_uint(pw);
                *reinterpret_cast<uint2 *>(&s_rows[pe][ph * 4 * S + 3 * S]) = make_uint2(bits, bits >> 16);
            }
            if (pe == n - 1) {
#pragma unroll
                for (int r = 0; r < 4; ++r) s_fold[ph][4 * half + r] = eager ? 1.f : sc[r];
            }
        }
        if (tid == 0) s_eager = eager ? 1 : 0;
        __syncthreads();
        if (tid == 0) s_flag[stage & 1] = 0;
    };

    // ---- prologue: metadata of stages 0 and 1, operands of stage 0
    float h[S][CPL];
    // state rows of this (bank, head, columns): a real head's S rows of
    // row_stride elements, this virtual head's span of them
    const int64_t head_cols = int64_t(head / p.split) * S * p.row_stride + int64_t(head % p.split) * p.width + col0;
    const int64_t state_offset = int64_t(bank) * p.s_heads * S * p.row_stride + head_cols;
    // piece-state rows of this (piece, head): [S, v] FP32
    const int64_t pstate_offset = ((int64_t(pslot) * p.heads + head) * S) * p.width + col0;
    if (from_zero) {
#pragma unroll
        for (int r = 0; r < S; ++r)
#pragma unroll
            for (int c = 0; c < CPL; ++c) h[r][c] = 0.f;
    } else if (MODE == 2 && piece > 0) {
        // M_piece, stored by piece_scan_kernel in the previous piece's slot
        load_state<S, CPL>(p.pstate, BDM_F32, pstate_offset - int64_t(p.heads) * S * p.width, p.width, S, h);
    } else {
        load_state<S, CPL>(p.initial, p.init_dtype, bidx * p.init_bstride + state_offset, p.row_stride, S, h);
    }
    // MODE 1: lanes 0..7 of a head carry column (lane) of the piece's transition
    const int pcol = tid % p.lanes_per_head;
    float pc[S];
#pragma unroll
    for (int r = 0; r < S; ++r) pc[r] = (from_zero && r == pcol) ? 1.f : 0.f;
    if (rounding) {
#pragma unroll
        for (int r = 0; r < S; ++r)
#pragma unroll
            for (int c = 0; c < CPL; ++c) h[r][c] = round_bf16(h[r][c]);
    }
    if (tid < 2) s_flag[tid] = 0;
    {
        const int o0 = load_group(0), o1 = load_group(1);
        if (HB == 2 || tid < 64) {
            decode_group(0, o0);
            decode_group(1, o1);
        }
    }
    __syncthreads();
    issue_prep(0);
    finish_prep(0);

    // v, w of the writes in stream order, in register sets used in turn
    // (three in MODE 0, two otherwise): write k's rows are loaded into the
    // set that the write before write k's predecessors used, so no registers
    // are copied.
    RawCols<T, CPL> va, wa, vb, wb, vc, wc;
    // v, w rows of a write by its (wave-uniform) token
    i32x4_t rsrc_v{}, rsrc_w{}, rsrc_z{};
    if constexpr (BUF) {
        rsrc_v = buffer_resource(p.v);
        rsrc_w = buffer_resource(p.w);
        rsrc_z = buffer_resource(p.zbuf);
    }
    const uint32_t row_bytes = uint32_t(hw) * uint32_t(sizeof(T));  // one token row of v, w or z (BUF)
    auto fetch_token = [&](int token, RawCols<T, CPL> &vv, RawCols<T, CPL> &ww) {
        if constexpr (BUF) {
            const uint32_t off = uint32_t(token) * row_bytes;
            vv.load_buffer(rsrc_v, lane_bytes, off);
            ww.load_buffer(rsrc_w, lane_bytes, off);
        } else {
            const int64_t row = int64_t(token) * hw;
            vv.load(reinterpret_cast<const T *>(reinterpret_cast<const char *>(p.v + row) + lane_bytes));
            ww.load(reinterpret_cast<const T *>(reinterpret_cast<const char *>(p.w + row) + lane_bytes));
        }
    };

    // Groups of kGroup stages: the packed order of the group after next is
    // loaded at a group's start and decoded after its last stage, so the load
    // is consumed on every path through the loop.
#pragma unroll 1
    for (int st0 = 0; st0 < nstages; st0 += kGroup) {
    const int o_group = load_group(st0 / kGroup + 2);
    const int st1 = min(nstages, st0 + kGroup);
#pragma unroll 1
    for (int st = st0; st < st1; ++st) {
        const int slot = st % kRing;
        // next stage's prep loads, in flight during this stage's value loop
        issue_prep(st + 1);

        // The state at the stage start (folded at the end of the previous
        // stage) is a rounding/snapshot point when the offset is > 0.
        if (st > 0) {
            if (rounding) {
                // two values per v_cvt_pk_bf16_f32
#pragma unroll
                for (int r = 0; r < S; ++r)
#pragma unroll
                    for (int c = 0; c < CPL; c += 2) round_pair<bf16_t>(h[r][c], h[r][c + 1]);
            }
            // snapshot of the state before event `base` (see routed_forward_kernel)
            if (void *snap = lds_ptr(P_SNAP)) {
                // stage starts are the multiples of snap_interval = kLazyStage
                const int64_t sslot = (start / NE) + st - 1;
                store_state<S, CPL>(snap, p.snap_dtype, sslot * p.s_heads * S * p.row_stride + head_cols,
                                    p.row_stride, S, h);
            }
        }

        const int n = __builtin_amdgcn_readfirstlane(s_n[slot]);
        const int nw = __builtin_amdgcn_readfirstlane(s_nw[slot]);
        const int eager = __builtin_amdgcn_readfirstlane(s_eager);
        // The stage's event metadata in registers, lane e holding event e's
        // (write position, write token, route, route weight), each taken to a
        // scalar register by one v_readlane where an event uses it.
        const int el = tid & (NE - 1);
        const int m_wpos = s_wpos[slot][el];
        const int m_wtok = s_wtok[slot][el];
        const int m_route = s_route[slot][el];

        auto read_event = [&](int i) {
            if (MODE == 1 && !reads_on) return;  // a read does not change the state (wave-uniform)
            const int zrow = __builtin_amdgcn_readlane(m_route, i);
            const float *row = &s_rows[i][lh * 4 * S];
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
            if constexpr (MODE == 3) {
                // the zero-start row in FP32, and in lanes 0..7 of the head
                // the coefficient c_j = gamma^T P e_j of the read on the
                // stage's start state
                float zc = 0.f;
#pragma unroll
                for (int r = 0; r < S; ++r) zc = fmaf(gamma[r], pc[r], zc);
                float *zr = p.z0buf + int64_t(zrow) * hw + (head * p.width + col0);
#pragma unroll
                for (int c = 0; c < CPL; ++c) __builtin_nontemporal_store(z[c], zr + c);
                if (pcol < S && tid < nheads * p.lanes_per_head)
                    p.cbuf[(int64_t(zrow) * p.heads + head) * S + pcol] = zc;
                return;
            }
            // nontemporal: the rows are read once, by the combine after the
            // recurrence, and should not displace the v, w rows that the
            // token's other write banks are about to read from L2
            if constexpr (BUF) {
                const i32x2_t packed{int32_t(pack_bf16x2(z[0], z[1])), int32_t(pack_bf16x2(z[2], z[3]))};
                raw_buffer_store_x2(packed, rsrc_z, int32_t(lane_bytes), int32_t(uint32_t(zrow) * row_bytes),
                                    kBufferNontemporal);
            } else {
                store_row_nt<CPL>(
                    reinterpret_cast<T *>(reinterpret_cast<char *>(p.zbuf + int64_t(zrow) * hw) + lane_bytes), z);
            }
        };
        // write `wi_` of the stage with its v, w rows in (vc, wc)
        auto write_event = [&](int wi_, const RawCols<T, CPL> &vc, const RawCols<T, CPL> &wc) {
            const float *row = &s_rows[wi_][lh * 4 * S];
            // (first: the gated value's wait then covers this read only)
            const uint2 pw2 = *reinterpret_cast<const uint2 *>(row + 3 * S);
            if (__builtin_amdgcn_readfirstlane(eager) != 0) {
                // hd = diag(d) M first; the update below then uses a and k
                // (a wave-uniform branch: the stage's form is uniform)
#pragma unroll
                for (int r = 0; r < S; ++r) {
                    const float d = row[2 * S + r];
#pragma unroll
                    for (int c = 0; c < CPL; ++c) h[r][c] *= d;
                    if constexpr (kTrans) pc[r] *= d;
                }
            }
            float nalpha[S], beta[S];
#pragma unroll
            for (int r = 0; r < S; ++r) {
                nalpha[r] = row[r];
                beta[r] = row[S + r];
            }
            // lazy: u = x - sum (a s') Mh, Mh += (k / s') u;  eager: u = x - sum a hd, M = hd + k u.
            // The sums over rows come first: they need no v, w, whose loads
            // are waited for only when the gated value x is formed.
            float u[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                u[c] = nalpha[0] * h[0][c];
#pragma unroll
                for (int r = 1; r < S; ++r) u[c] = fmaf(nalpha[r], h[r][c], u[c]);
            }
            GatedValues<T, CPL> x;
            x.make_pair(wc, vc, pw2.x, pw2.y, u[CPL - 1]);
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                u[c] = x.add_to(u[c], c);
#pragma unroll
                for (int r = 0; r < S; ++r) h[r][c] = fmaf(beta[r], u[c], h[r][c]);
            }
            if (kTrans && from_zero) {
                // the transition column: the same update with x = 0
                float uc = nalpha[0] * pc[0];
#pragma unroll
                for (int r = 1; r < S; ++r) uc = fmaf(nalpha[r], pc[r], uc);
#pragma unroll
                for (int r = 0; r < S; ++r) pc[r] = fmaf(beta[r], uc, pc[r]);
            }
        };
        // Events in packed order, as runs: the reads before each write, then
        // the write, so the state is updated exactly once per iteration and
        // never merged from branches.  MODE 0: writes rotate over the register
        // sets A, B and C (three writes per loop iteration), each write's rows
        // loaded two writes ahead; MODE 1 and 2 alternate A and B, one write
        // ahead (a third set would spill there).  A stage's first writes are
        // fetched here, not prefetched by the previous stage: a stage that
        // found them in other sets would have to copy them, and a copy waits
        // for every memory access issued before it.
        {
            // the rows of write k (past the last write, the last write's rows
            // again: harmless).  Always two loads, so that the compiler can
            // wait for a set with a count instead of draining the loads issued
            // after it.
            auto fetch_write = [&](int k, RawCols<T, CPL> &vv, RawCols<T, CPL> &ww) {
                fetch_token(__builtin_amdgcn_readlane(m_wtok, k < nw ? k : nw - 1), vv, ww);
            };
            int i = 0;
            if constexpr (MODE == 0) {
                if (nw > 0) {
                    fetch_write(0, va, wa);
                    fetch_write(1, vb, wb);
                }
#pragma unroll 1
                for (int wk = 0; wk < nw; wk += 3) {
                    int wi_ = __builtin_amdgcn_readlane(m_wpos, wk);
                    fetch_write(wk + 2, vc, wc);
#pragma unroll 1
                    for (; i < wi_; ++i) read_event(i);
                    i = wi_ + 1;
                    write_event(wi_, va, wa);
                    if (wk + 1 >= nw) break;
                    wi_ = __builtin_amdgcn_readlane(m_wpos, wk + 1);
                    fetch_write(wk + 3, va, wa);
#pragma unroll 1
                    for (; i < wi_; ++i) read_event(i);
                    i = wi_ + 1;
                    write_event(wi_, vb, wb);
                    if (wk + 2 >= nw) break;
                    wi_ = __builtin_amdgcn_readlane(m_wpos, wk + 2);
                    fetch_write(wk + 4, vb, wb);
#pragma unroll 1
                    for (; i < wi_; ++i) read_event(i);
                    i = wi_ + 1;
                    write_event(wi_, vc, wc);
                }
            } else {
                if (nw > 0) fetch_write(0, va, wa);
#pragma unroll 1
                for (int wk = 0; wk < nw; wk += 2) {
                    int wi_ = __builtin_amdgcn_readlane(m_wpos, wk);
                    fetch_write(wk + 1, vb, wb);
#pragma unroll 1
                    for (; i < wi_; ++i) read_event(i);
                    i = wi_ + 1;
                    write_event(wi_, va, wa);
                    if (wk + 1 >= nw) break;
                    wi_ = __builtin_amdgcn_readlane(m_wpos, wk + 1);
                    fetch_write(wk + 2, va, wa);
#pragma unroll 1
                    for (; i < wi_; ++i) read_event(i);
                    i = wi_ + 1;
                    write_event(wi_, vb, wb);
                }
            }
#pragma unroll 1
            for (; i < n; ++i) read_event(i);
        }

        // fold s into Mh: the true state at the stage end
#pragma unroll
        for (int r = 0; r < S; ++r) {
            const float f = s_fold[lh][r];
#pragma unroll
            for (int c = 0; c < CPL; ++c) h[r][c] *= f;
            if constexpr (kTrans) pc[r] *= f;
        }
        if constexpr (MODE == 3) {
            // the stage's R and P into its slot, then the next stage from zero
            const int64_t sl = stage_slot0 + st;
            if (group == 0 && tid < NE)
                p.tgt[sl * NE + tid] = (tid < n && ((s_rmask[slot] >> tid) & 1u)) ? s_route[slot][tid] : -1;
            // R by column: [slot, head, width, 8] (the scan loads a column's 8 rows at once)
            float *rc = p.pstate + ((sl * p.heads + head) * p.width + col0) * S;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                reinterpret_cast<float4 *>(rc + c * S)[0] = make_float4(h[0][c], h[1][c], h[2][c], h[3][c]);
                reinterpret_cast<float4 *>(rc + c * S)[1] = make_float4(h[4][c], h[5][c], h[6][c], h[7][c]);
            }
            if (pcol < S && tid < nheads * p.lanes_per_head) {
                float *pt = p.ptrans + ((sl * p.heads + head) * S) * S;
#pragma unroll
                for (int r = 0; r < S; ++r) pt[r * S + pcol] = pc[r];
            }
#pragma unroll
            for (int r = 0; r < S; ++r) {
#pragma unroll
                for (int c = 0; c < CPL; ++c) h[r][c] = 0.f;
                pc[r] = r == pcol ? 1.f : 0.f;
            }
        }
        // operands of stage st+1
        if (st + 1 < nstages) finish_prep(st + 1);
    }
    // the metadata of the group after next, into this group's slots (wave 0;
    // the barriers of the stages in between publish it)
    if (HB == 2 || tid < 64) decode_group(st0 / kGroup + 2, o_group);
    }
    if (MODE == 1 && pslot >= 0) {
        // R_q and P_q of this piece (a first piece: its end state and P = 0,
        // so the scan's M_1 = P_0 M_0 + R_0 is that end state)
        store_state<S, CPL>(p.pstate, BDM_F32, pstate_offset, p.width, S, h);
        if (pcol < S && tid < nheads * p.lanes_per_head) {
            float *pt = p.ptrans + ((int64_t(pslot) * p.heads + head) * S) * S;
#pragma unroll
            for (int r = 0; r < S; ++r) pt[r * S + pcol] = from_zero ? pc[r] : 0.f;
        }
    } else if (MODE != 3 && lds_ptr(P_FINAL) && piece == pieces - 1) {
        const int64_t final_offset = bidx * (int64_t(p.banks) * p.s_heads * S * p.row_stride) + state_offset;
        store_state<S, CPL>(lds_ptr(P_FINAL), p.final_dtype, final_offset, p.row_stride, S, h);
    }
}

// Exclusive prefix of x over the 1024 threads of the workgroup, and the
// total in *total: within each wave by shuffles, then over the 16 wave totals
// by the first wave.  lds: 1024 / kWave + 1 ints.
__device__ int block_exclusive_scan(int x, int *lds, int *total) {
    const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
    constexpr int kWaves = 1024 / kWave;
    int incl = x;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int up = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += up;
    }
    if (lane == kWave - 1) lds[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        // (lane l reads lds[l] before it rewrites it; one wave, in order)
        const int wt = lane < kWaves ? lds[lane] : 0;
        int w = wt;
#pragma unroll
        for (int off = 1; off < kWaves; off <<= 1) {
            const int up = __shfl_up(w, off, kWave);
            if (lane >= off) w += up;
        }
        if (lane < kWaves) lds[lane] = w - wt;  // exclusive prefix of the waves
        if (lane == kWaves - 1) lds[kWaves] = w;
    }
    __syncthreads();
    *total = lds[kWaves];
    return lds[wave] + incl - x;
}

// The piece list: a segment longer than kPieceEvents becomes
// ceil(len / kPieceEvents) pieces with consecutive piece-state slots.  One
// workgroup of 1024 threads; thread t handles a contiguous run of segments.
// With segs: also the item of each cut segment's first piece, in segment
// order, and their count in n_segs.
__global__ __launch_bounds__(1024) void piece_table_kernel(const int64_t *__restrict__ cu, int nseg,
                                                           int4 *__restrict__ items, int *__restrict__ n_items,
                                                           int *__restrict__ segs, int *__restrict__ n_segs) {
    __shared__ int s_scan[2][1024 / kWave + 1];
    const int t = threadIdx.x;
    const int per = (nseg + 1023) / 1024;
    const int s0 = min(nseg, t * per), s1 = min(nseg, s0 + per);
    int cut = 0, cut_segs = 0;
    // (unrolled: the loads of a thread's segments are independent and go out together)
#pragma unroll 8
    for (int sg = s0; sg < s1; ++sg) {
        const int64_t len = cu[sg + 1] - cu[sg];
        if (len > kPieceEvents) {
            cut += int((len + kPieceEvents - 1) / kPieceEvents);
            ++cut_segs;
        }
    }
    int pieces_total = 0, segs_total = 0;
    int pos = block_exclusive_scan(cut, s_scan[0], &pieces_total);
    int spos = segs ? block_exclusive_scan(cut_segs, s_scan[1], &segs_total) : 0;
#pragma unroll 8
    for (int sg = s0; sg < s1; ++sg) {
        const int64_t len = cu[sg + 1] - cu[sg];
        if (len > kPieceEvents) {
            const int np = int((len + kPieceEvents - 1) / kPieceEvents);
            if (segs) segs[spos++] = pos;
            for (int q = 0; q < np; ++q, ++pos) items[pos] = make_int4(sg, q, np, pos);
        }
    }
    if (t == 0) {
        n_items[0] = pieces_total;
        if (segs) n_segs[0] = segs_total;
    }
}

// For each cut segment (its first piece's item) and head: M_0 = the
// segment's initial state, M_(q+1) = P_q M_q + R_q in FP32, stored over R_q
// (the slot that piece q+1 reads its start state from).  One thread per value
// column.  R_q and P_q do not depend on the chain, so they are loaded
// kPieceScanDepth steps ahead: a step's 8 R loads, 8 stores and one P load
// (lane l of each wave loads entry l of P_q, taken to scalar registers by
// v_readlane) keep 51 memory operations in flight, under the 63 the wave's
// counter holds.
constexpr int kPieceScanDepth = 3;

__global__ __launch_bounds__(256) void piece_scan_kernel(const int4 *__restrict__ items,
                                                         const int *__restrict__ n_items, const void *initial,
                                                         int init_dtype, int64_t init_bstride, int banks, int heads,
                                                         int width, int split, int64_t row_stride,
                                                         float *__restrict__ pstate,
                                                         const float *__restrict__ ptrans) {
    constexpr int S = 8, D = kPieceScanDepth;
    if (int(blockIdx.x) >= n_items[0]) return;
    const int4 it = items[blockIdx.x];
    if (it.y != 0) return;  // not a first piece
    const int seg = it.x, pieces = it.z, slot0 = it.w, head = blockIdx.y;
    const int bank = seg % banks;
    const int64_t bidx = seg / banks;
    const int steps = pieces - 1;  // a cut segment has at least two pieces
    const int lane = int(threadIdx.x) % kWave;
    for (int c0 = 0; c0 < width; c0 += int(blockDim.x)) {
        // (every lane of a wave takes part in the P loads; lanes past the
        // last column shadow it)
        const int c = c0 + int(threadIdx.x);
        const int cc = c < width ? c : width - 1;
        float m[S];
        // heads, width: virtual heads of the column split (split per real head)
        const int64_t off = bidx * init_bstride + ((int64_t(bank) * (heads / split) + head / split) * S) * row_stride +
                            int64_t(head % split) * width + cc;
        if (init_dtype == BDM_BF16) {
#pragma unroll
            for (int r = 0; r < S; ++r) m[r] = to_f32(static_cast<const bf16_t *>(initial)[off + int64_t(r) * row_stride]);
        } else {
#pragma unroll
            for (int r = 0; r < S; ++r) m[r] = static_cast<const float *>(initial)[off + int64_t(r) * row_stride];
        }
        // step q's R column and this lane's entry of P (past the last step,
        // the last step's again: loaded, never used)
        auto load_step = [&](int q, float (&rq)[S], float &pq) {
            const int qq = q < steps ? q : steps - 1;
            const int64_t slot = int64_t(slot0 + qq) * heads + head;
#pragma unroll
            for (int r = 0; r < S; ++r) rq[r] = pstate[(slot * S + r) * width + cc];
            pq = ptrans[slot * S * S + lane];
        };
        // step q from the registers of depth d, then the loads of step q + D
        // into them (issued before the stores; lanes past the last column
        // store the values of the column they shadow, which its own lane
        // stores too)
        float rq[D][S], pq[D];
        auto step = [&](int q, int d) {
            float nm[S];
#pragma unroll
            for (int r = 0; r < S; ++r) {
                float acc = rq[d][r];
#pragma unroll
                for (int j = 0; j < S; ++j)
                    acc = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(pq[d]), r * S + j)), m[j], acc);
                nm[r] = acc;
            }
            load_step(q + D, rq[d], pq[d]);
            const int64_t slot = int64_t(slot0 + q) * heads + head;
#pragma unroll
            for (int r = 0; r < S; ++r) {
                m[r] = nm[r];
                pstate[(slot * S + r) * width + cc] = nm[r];
            }
        };
#pragma unroll
        for (int d = 0; d < D; ++d) load_step(d, rq[d], pq[d]);
        // whole groups of D steps: every step issues the same memory
        // operations, so each waits with a count for the loads D steps back
        int q0 = 0;
        for (; q0 + D <= steps; q0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) step(q0 + d, d);
        }
#pragma unroll
        for (int d = 0; d < D - 1; ++d)
            if (q0 + d < steps) step(q0 + d, d);
    }
}

// The stage path after MODE 3 (rounding policy, segments longer than
// kPieceEvents), in two kernels on one wave per (..., virtual head, 64 value
// columns), a lane per column.
//
// stage_scan_kernel, per long segment: M_0 = the segment's initial state
// rounded to BF16; M_(k+1) = round(P_k M_k + R_k) along the stages, the last
// map unrounded (the final state); each stage start state M_k (BF16 values,
// the rounding points) is stored over R_k, which it no longer needs.  This is
// the serial chain, so it holds the state update only: a stage is 2 loads of
// R (a column's 8 rows, [slot, head, width, 8]), 1 of P and 1 store of M_k,
// and the loads of stage k + 7 are issued while stage k is computed (eight
// register sets used in turn, every load and store unconditional, so the
// compiler waits for counted loads and the wave's counter of outstanding
// memory operations does not fill).  P
// reaches every lane through LDS.  Block b takes long segments b,
// b + gridDim.x, ...
//
// stage_reads_kernel, per piece (in parallel): each read of stage k gets
// z = c^T M_k + z0 (c and z0 from MODE 3), stored to the read buffer.  A
// stage's M_k and targets are loaded one stage ahead; its c rows and the 16
// events' z0 rows (a missing read loads row 0) go out together, before any of
// its stores, so a stage waits for one round trip.
template <typename T>
struct StageParams {
    const int *segs, *n_segs;  // first-piece item of each long segment (piece_table_kernel)
    const int4 *items;
    const int *n_items;
    const int64_t *cu;
    const int *tgt;            // [slots, 16]: read route slot of each event, -1 otherwise
    const void *initial;
    void *final_state;
    float *pstate;             // R per stage slot ([slots, heads, width, 8]), then M_k (BF16) over it
    const float *ptrans, *z0buf, *cbuf;
    T *zbuf;
    int64_t init_bstride, row_stride;
    int init_dtype, final_dtype;
    int banks, heads, s_heads, split, width;
};

struct ScanOperands {
    float r[8];  // R_k rows of the lane's column
    float pt;    // P_k element `lane` (row lane / 8, column lane % 8)
};
constexpr int kScanDepth = 8;

template <typename T>
__global__ __launch_bounds__(64) void stage_scan_kernel(StageParams<T> p) {
    constexpr int S = 8, NE = 16;
    __shared__ __align__(16) float s_p[S * S];
    const int lane = threadIdx.x;
    const int head = blockIdx.y;
    const int col = int(blockIdx.z) * kWave + lane;
    const bool live = col < p.width;
    // lanes past the width repeat the last column: same values to the same
    // addresses, so their stores need no mask
    const int colc = live ? col : p.width - 1;
    const int nsegs = p.n_segs[0];
    for (int j = blockIdx.x; j < nsegs; j += gridDim.x) {
        const int seg = p.items[p.segs[j]].x;
        const int64_t start = p.cu[seg], end = p.cu[seg + 1];
        const int nst = int((end - start + NE - 1) / NE);
        const int64_t slot0 = start / NE + seg;
        const int bank = seg % p.banks;
        const int64_t bidx = seg / p.banks;
        const int64_t state_offset = int64_t(bank) * p.s_heads * S * p.row_stride +
                                     int64_t(head / p.split) * S * p.row_stride +
                                     int64_t(head % p.split) * p.width + colc;
        float m[S];
        {
            const int64_t off = bidx * p.init_bstride + state_offset;
#pragma unroll
            for (int r = 0; r < S; ++r)
                m[r] = round_bf16(p.init_dtype == BDM_BF16
                                      ? to_f32(static_cast<const bf16_t *>(p.initial)[off + r * p.row_stride])
                                      : static_cast<const float *>(p.initial)[off + r * p.row_stride]);
        }
        auto rows_of = [&](int k) {  // stage k's R (then M_k) column; k past the last: the last
            return p.pstate + (((slot0 + min(k, nst - 1)) * p.heads + head) * p.width + colc) * S;
        };
        auto issue = [&](int k, ScanOperands &o) {
            const float4 *rr = reinterpret_cast<const float4 *>(rows_of(k));
            const float4 a = rr[0], b = rr[1];
            o.r[0] = a.x, o.r[1] = a.y, o.r[2] = a.z, o.r[3] = a.w;
            o.r[4] = b.x, o.r[5] = b.y, o.r[6] = b.z, o.r[7] = b.w;
            o.pt = p.ptrans[((slot0 + min(k, nst - 1)) * p.heads + head) * S * S + lane];
        };
        auto compute = [&](int k, const ScanOperands &o) {
            __syncthreads();  // the previous stage's LDS reads are done
            s_p[lane] = o.pt;
            __syncthreads();
            float nm[S];
#pragma unroll
            for (int r = 0; r < S; ++r) {
                const float4 p0 = *reinterpret_cast<const float4 *>(&s_p[r * S]);
                const float4 p1 = *reinterpret_cast<const float4 *>(&s_p[r * S + 4]);
                const float pv[S] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
                float acc = o.r[r];
#pragma unroll
                for (int q = 0; q < S; ++q) acc = fmaf(pv[q], m[q], acc);
                nm[r] = acc;
            }
            // M_k over R_k (read above into o.r, whose use in nm has waited
            // for it), as 8 BF16 values (exact: the rounded start state)
            *reinterpret_cast<uint4 *>(rows_of(k)) =
                make_uint4(pack_bf16x2(m[0], m[1]), pack_bf16x2(m[2], m[3]), pack_bf16x2(m[4], m[5]),
                           pack_bf16x2(m[6], m[7]));
            const bool last = k + 1 >= nst;
#pragma unroll
            for (int r = 0; r < S; ++r) m[r] = last ? nm[r] : round_bf16(nm[r]);
        };
        // kScanDepth register sets in turn, each stage's operands loaded
        // kScanDepth - 1 stages ahead (more than an HBM round trip of this
        // loop's stages); the loop is unrolled so every set is a fixed
        // register range, never copied (a copy would wait for the loads in
        // flight into it)
        ScanOperands o[kScanDepth];
#pragma unroll
        for (int i = 0; i + 1 < kScanDepth; ++i) issue(i, o[i]);
#pragma unroll 1
        for (int k = 0; k < nst; k += kScanDepth) {
#pragma unroll
            for (int i = 0; i < kScanDepth; ++i) {
                issue(k + i + kScanDepth - 1, o[(i + kScanDepth - 1) % kScanDepth]);
                compute(k + i, o[i]);
                if (k + i + 1 >= nst) break;
            }
        }
        if (p.final_state && live) {
            const int64_t off = bidx * (int64_t(p.banks) * p.s_heads * S * p.row_stride) + state_offset;
#pragma unroll
            for (int r = 0; r < S; ++r) {
                if (p.final_dtype == BDM_BF16)
                    static_cast<bf16_t *>(p.final_state)[off + r * p.row_stride] = from_f32<bf16_t>(m[r]);
                else
                    static_cast<float *>(p.final_state)[off + r * p.row_stride] = m[r];
            }
        }
        __syncthreads();  // LDS reused by the block's next segment
    }
}

template <typename T>
__global__ __launch_bounds__(64) void stage_reads_kernel(StageParams<T> p) {
    constexpr int S = 8, NE = 16;
    __shared__ __align__(16) float s_c[NE][S];
    if (int(blockIdx.x) >= p.n_items[0]) return;
    const int4 it = p.items[blockIdx.x];
    const int seg = it.x, piece = it.y;
    const int lane = threadIdx.x;
    const int head = blockIdx.y;
    const int col = int(blockIdx.z) * kWave + lane;
    const bool live = col < p.width;
    const int colc = live ? col : p.width - 1;
    const int64_t hw = int64_t(p.heads) * p.width;
    const int64_t zcol = int64_t(head) * p.width + colc;
    const int64_t seg_start = p.cu[seg];
    const int64_t start = seg_start + int64_t(piece) * kPieceEvents;
    const int64_t end = min(p.cu[seg + 1], start + kPieceEvents);
    const int nst = int((end - start + NE - 1) / NE);
    const int64_t slot0 = seg_start / NE + seg + int64_t(piece) * (kPieceEvents / NE);
    // stage st's M_k column (8 BF16 values) and its events' targets (lane e
    // % 16: event e's read route slot, -1 for a write); past the last stage,
    // the last stage's again
    auto load_stage = [&](int st, uint4 &mq, int &t) {
        const int64_t sl = slot0 + min(st, nst - 1);
        mq = *reinterpret_cast<const uint4 *>(p.pstate + ((sl * p.heads + head) * p.width + colc) * S);
        t = p.tgt[sl * NE + (lane & (NE - 1))];
    };
    uint4 mq;
    int t;
    load_stage(0, mq, t);
#pragma unroll 1
    for (int st = 0; st < nst; ++st) {
        uint4 mq_next;
        int t_next;
        load_stage(st + 1, mq_next, t_next);
        const uint32_t mw[4] = {mq.x, mq.y, mq.z, mq.w};
        float m[S];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            m[2 * i] = __uint_as_float(mw[i] << 16);
            m[2 * i + 1] = __uint_as_float(mw[i] & 0xffff0000u);
        }
        const int zr = max(__shfl(t, lane >> 2, kWave), 0);
        const float2 cc = *reinterpret_cast<const float2 *>(p.cbuf + (int64_t(zr) * p.heads + head) * S + 2 * (lane & 3));
        float z[NE];
#pragma unroll
        for (int e = 0; e < NE; ++e) z[e] = p.z0buf[int64_t(max(__builtin_amdgcn_readlane(t, e), 0)) * hw + zcol];
        __syncthreads();  // the previous stage's LDS reads are done
        *reinterpret_cast<float2 *>(&s_c[lane >> 2][2 * (lane & 3)]) = cc;
        __syncthreads();
#pragma unroll
        for (int e = 0; e < NE; ++e) {
            const int row = __builtin_amdgcn_readlane(t, e);
            const float4 c0 = *reinterpret_cast<const float4 *>(&s_c[e][0]);
            const float4 c1 = *reinterpret_cast<const float4 *>(&s_c[e][4]);
            const float cv[S] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            float ze = z[e];
#pragma unroll
            for (int r = 0; r < S; ++r) ze = fmaf(cv[r], m[r], ze);
            if (live && row >= 0) p.zbuf[int64_t(row) * hw + int64_t(head) * p.width + col] = from_f32<T>(ze);
        }
        mq = mq_next;
        t = t_next;
    }
}

// y[token, :] = fold over the token's reads in increasing bank id of
// bf(total + z) (role_bank_dispatch.py:209-215).  A token's KR rows of the
// read buffer are in route order (row token*KR + j), so each thread orders the
// token's KR bank ids itself: keys (bank << bits | j) sort by bank, ties by
// route slot, and the low bits give each fold position its row.  The token's
// indices are 64 bytes that every thread of the token reads (from L1); the
// rows themselves are loaded in fold order, so no row moves twice.  Banks are
// clamped to [0, banks) as the dispatch clamps them.  One thread per (token,
// CPL columns).  EACH = false is the narrow-head rule (head width <= 32,
// role_bank_dispatch.py:222-226): the reference then sums with index_add_,
// which accumulates a token's reads in FP32 and rounds once.
__device__ __forceinline__ void sort8_ascending(uint32_t (&x)[8]) {
    auto cex = [](uint32_t &a, uint32_t &b) {
        const uint32_t lo = min(a, b), hi = max(a, b);
        a = lo;
        b = hi;
    };
    cex(x[0], x[2]), cex(x[1], x[3]), cex(x[4], x[6]), cex(x[5], x[7]);
    cex(x[0], x[4]), cex(x[1], x[5]), cex(x[2], x[6]), cex(x[3], x[7]);
    cex(x[0], x[1]), cex(x[2], x[3]), cex(x[4], x[5]), cex(x[6], x[7]);
    cex(x[2], x[4]), cex(x[3], x[5]);
    cex(x[1], x[4]), cex(x[3], x[6]);
    cex(x[1], x[2]), cex(x[3], x[4]), cex(x[5], x[6]);
}

template <typename T, int CPL, int KFIX, bool EACH>
__global__ __launch_bounds__(256) void ordered_combine_kernel(const T *__restrict__ zbuf,
                                                              const int64_t *__restrict__ read_indices,
                                                              T *__restrict__ y, int64_t nt, int kr, int row_width,
                                                              int banks, int col_begin, int col_count) {
    // columns col_begin .. col_begin + col_count - 1 of every token (all of
    // them, or one round's heads when the combine runs beside the recurrence)
    const int chunks = col_count / CPL;
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t token = idx / chunks;
    if (token >= nt) return;
    const int col0 = col_begin + int(idx - token * chunks) * CPL;
    const T *z = zbuf + token * kr * row_width + col0;
    const int64_t *ri = read_indices + token * kr;
    auto bank_of = [&](int j) -> uint32_t {
        const int64_t b = ri[j];
        return uint32_t(b < 0 ? 0 : (b >= banks ? banks - 1 : b));
    };
    float total[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) total[c] = 0.f;
    auto add = [&](const float (&v)[CPL]) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) total[c] = EACH ? round_to<T>(total[c] + v[c]) : total[c] + v[c];
    };
    if constexpr (KFIX == 8) {
        // eight reads: a 19-comparator sort of (bank << 3 | slot), banks < 2^29
        uint32_t key[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) key[j] = (bank_of(j) << 3) | uint32_t(j);
        sort8_ascending(key);
        if constexpr (sizeof(T) == 2 && CPL == 8) {
            // 16-byte nontemporal loads (the rows are used once), all in flight before the fold
            typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
            u32x4 raw[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                raw[i] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4 *>(z + int64_t(key[i] & 7u) * row_width));
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
                float v[CPL];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v[2 * q] = __uint_as_float(w[q] << 16);
                    v[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
                }
                add(v);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float v[CPL];
                load_row<CPL>(z + int64_t(key[i] & 7u) * row_width, v);
                add(v);
            }
        }
    } else {
        // up to 32 reads: the next row is the one with the smallest key above
        // the last row's, keys (bank << 5 | slot) in 64 bits
        constexpr int KMAX = 32;
        uint64_t key[KMAX];
#pragma unroll
        for (int j = 0; j < KMAX; ++j) key[j] = j < kr ? (uint64_t(bank_of(j)) << 5) | uint64_t(j) : ~uint64_t(0);
        uint64_t last = 0;
        for (int i = 0; i < kr; ++i) {
            uint64_t next = ~uint64_t(0);
#pragma unroll
            for (int j = 0; j < KMAX; ++j)
                if ((i == 0 || key[j] > last) && key[j] < next) next = key[j];
            last = next;
            float v[CPL];
            load_row<CPL>(z + int64_t(next & 31u) * row_width, v);
            add(v);
        }
    }
    store_row<CPL>(y + token * row_width + col0, total);
}

// A kernel rather than hipMemsetAsync, so callers may capture it in a graph.
template <typename T>
__global__ __launch_bounds__(256) void zero_fill_kernel(T *__restrict__ out, int64_t count) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < count) out[i] = from_f32<T>(0.f);
}

// Virtual heads per real head on the lazy path: 1 for heads of at most 256
// columns (4 per lane, 64 lanes); a wider head whose width is a multiple of
// 128 runs as width/128 heads of 128 columns (value columns are independent
// in the recurrence, and 128-column heads are the kernel's two-heads-per-wave
// shape); 0 when neither applies.
int lazy_split(const bdm_forward_args &a) {
    if (a.head_width % 4 != 0) return 0;
    if (a.head_width / 4 <= 64) return 1;
    return a.head_width % 128 == 0 ? a.head_width / 128 : 0;
}

// Scratch carved from the bdm_forward workspace: the cut-segment path's and
// the longest-first segment order's.
struct PieceBuffers {
    int4 *items = nullptr;
    int *count = nullptr;
    float *pstate = nullptr, *ptrans = nullptr;
    int64_t max_pieces = 0;  // 0: the path is off
    int *seg_order = nullptr;  // null: segments in bank order
    bool order_given = false;  // seg_order holds the caller's order (bdm_route_dispatch): no ranking launch
    // The rounding policy's stage path (0 pieces: off): its piece list and
    // counts ([0] pieces, [1] long segments), the long segments' first
    // pieces, the stage slots' R and P, the reads' zero-start rows and
    // coefficients.
    int64_t stage_pieces = 0;
    int4 *st_items = nullptr;
    int *st_count = nullptr, *st_segs = nullptr;
    float *st_r = nullptr, *st_p = nullptr, *st_z0 = nullptr, *st_c = nullptr;
    int *st_tgt = nullptr;
};

// Profiling events of bdm_forward (phase_events): 0 before the recurrence,
// 1 before the combine, 2 after it.
int record_phase(const bdm_forward_args &a, int which, hipStream_t stream) {
    if (!a.phase_events[0] || !a.phase_events[which]) return BDM_OK;
    if (hipEventRecord(static_cast<hipEvent_t>(a.phase_events[which]), stream) != hipSuccess)
        return fail(BDM_ERR_LAUNCH, "forward: recording profiling event %d", which);
    return BDM_OK;
}

// The read combine of bdm_forward: y from the read buffer (or zeros when the
// routes have no reads).
template <typename T>
int launch_combine_kernels(const bdm_forward_args &a, const T *zbuf, hipStream_t stream, int col_begin = 0,
                           int col_count = -1) {
    const int row_width = a.heads * a.head_width;
    if (col_count < 0) col_count = row_width;
    const int64_t nt = a.batch * a.time;
    if (a.read_banks > 0) {
        // 16-byte rows where the layout allows (8 BF16 or 4 FP32 columns)
        constexpr int CC = sizeof(T) == 2 ? 8 : 4;
        const bool wide = row_width % CC == 0 && col_begin % CC == 0 && col_count % CC == 0;
        const int cc = wide ? CC : 1;
        const unsigned blocks = unsigned((nt * (col_count / cc) + 255) / 256);
        T *y = static_cast<T *>(a.output);
        const int kr = a.read_banks, banks = a.bank_count;
        if (a.head_width <= 32) {
            // narrow heads: FP32 sum, one rounding (index_add_)
            if (wide)
                ordered_combine_kernel<T, CC, 0, false><<<blocks, 256, 0, stream>>>(zbuf, a.read_indices, y, nt, kr,
                                                                                    row_width, banks, col_begin,
                                                                                    col_count);
            else
                ordered_combine_kernel<T, 1, 0, false><<<blocks, 256, 0, stream>>>(zbuf, a.read_indices, y, nt, kr,
                                                                                   row_width, banks, col_begin,
                                                                                   col_count);
        } else if (wide) {
            if (a.read_banks == 8 && a.bank_count < (1 << 29))
                ordered_combine_kernel<T, CC, 8, true><<<blocks, 256, 0, stream>>>(zbuf, a.read_indices, y, nt, kr,
                                                                                   row_width, banks, col_begin,
                                                                                   col_count);
            else
                ordered_combine_kernel<T, CC, 0, true><<<blocks, 256, 0, stream>>>(zbuf, a.read_indices, y, nt, kr,
                                                                                   row_width, banks, col_begin,
                                                                                   col_count);
        } else {
            ordered_combine_kernel<T, 1, 0, true><<<blocks, 256, 0, stream>>>(zbuf, a.read_indices, y, nt, kr,
                                                                              row_width, banks, col_begin, col_count);
        }
    } else {
        const int64_t count = nt * row_width;
        zero_fill_kernel<T><<<unsigned((count + 255) / 256), 256, 0, stream>>>(static_cast<T *>(a.output), count);
    }
    return check_launch("ordered_combine_kernel");
}

template <typename T>
int launch_combine(const bdm_forward_args &a, const T *zbuf, hipStream_t stream) {
    if (int rc = record_phase(a, 1, stream)) return rc;
    if (int rc = launch_combine_kernels(a, zbuf, stream)) return rc;
    return record_phase(a, 2, stream);
}

// ---- The read combine beside the recurrence.
//
// The combine of a token's columns can start once every segment of those
// columns' heads has run.  Where the longest-first order runs the head
// groups in rounds (each round fills every slot of the GPU), the rounds are
// launched separately, alternating between the caller's stream and an
// auxiliary one, and each round's combine over its own heads' columns
// follows it on the same stream.  The combine of round r then runs beside
// round r + 1: the recurrence holds 4 waves of <= 112 VGPRs per SIMD, which
// leaves the 64 that a combine wave needs (ordered_combine_kernel takes 46),
// and the combine is HBM-bound where the recurrence is VALU-bound.  Only the
// last round's combine is left after the recurrence.  The columns a combine
// reads are written by its own round only, and y's column ranges are
// disjoint, so results are those of the serial order bit for bit.
//
// The auxiliary streams join the caller's through events (a fork after the
// segment order, a join after each auxiliary stream's combine), so the
// sequence may be captured in a graph.  One-lane kernels ahead of each later
// round on its auxiliary stream (one per earlier round) let the earlier
// rounds' blocks reach every slot before its own are dispatched (otherwise
// the rounds would share the slots from the start, and the first would end
// no earlier than the last).  Per device: three streams (default priority)
// and their events, created on the first call that is not under capture;
// BDM_COMBINE_OVERLAP=0 keeps the serial order.
constexpr int kOverlapAux = 3;  // auxiliary streams: at most 4 parts

struct OverlapAux {
    hipStream_t stream[kOverlapAux] = {};
    hipEvent_t fork = nullptr, join[kOverlapAux] = {};
};

bool overlap_enabled() {
    const char *e = getenv("BDM_COMBINE_OVERLAP");
    return !(e && e[0] == '0' && e[1] == 0);
}

// Launches the head groups are split into (2..4; default: one per round).
int overlap_parts(int rounds, int groups) {
    const char *e = getenv("BDM_COMBINE_PARTS");
    int n = e ? atoi(e) : rounds;
    n = n < 2 ? 2 : (n > kOverlapAux + 1 ? kOverlapAux + 1 : n);
    return n > groups ? groups : n;
}

__global__ void overlap_gate_kernel() {}

std::mutex &overlap_launch_mutex() {
    static std::mutex mu;
    return mu;
}

// The device's auxiliary streams and events, or null (then the serial order
// runs): creation failed, or the caller's stream is being captured and they
// do not exist yet (resources are not created under capture).
const OverlapAux *overlap_aux(hipStream_t caller) {
    constexpr int kMaxDev = 64;
    static std::mutex mu;
    static OverlapAux aux[kMaxDev];
    static bool failed[kMaxDev] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (aux[dev].fork) return &aux[dev];
    if (failed[dev]) return nullptr;
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(caller, &status) != hipSuccess || status != hipStreamCaptureStatusNone) return nullptr;
    OverlapAux made;
    bool ok = hipEventCreateWithFlags(&made.fork, hipEventDisableTiming) == hipSuccess;
    for (int i = 0; ok && i < kOverlapAux; ++i)
        ok = hipStreamCreateWithFlags(&made.stream[i], hipStreamNonBlocking) == hipSuccess &&
             hipEventCreateWithFlags(&made.join[i], hipEventDisableTiming) == hipSuccess;
    if (!ok) {
        (void)hipGetLastError();
        failed[dev] = true;
        return nullptr;
    }
    aux[dev] = made;
    return &aux[dev];
}

// The lazy kernel's MODE 0 instance: HB heads per workgroup, buffer form
// where it applies.
template <typename T, int CPL>
const void *mode0_kernel(int hb, bool buf) {
    if constexpr (std::is_same<T, bf16_t>::value && CPL == 4) {
        if (buf)
            return hb == 2 ? reinterpret_cast<const void *>(&lazy_forward_kernel<T, CPL, 2, 0, true>)
                           : reinterpret_cast<const void *>(&lazy_forward_kernel<T, CPL, 8, 0, true>);
    }
    return hb == 2 ? reinterpret_cast<const void *>(&lazy_forward_kernel<T, CPL, 2, 0>)
                   : reinterpret_cast<const void *>(&lazy_forward_kernel<T, CPL, 8, 0>);
}

// Whether the v, w rows and the read buffer fit the buffer form's 32-bit
// byte offsets (BF16 controllers, 4 columns per lane).
template <typename T, int CPL>
bool buffer_form(const bdm_forward_args &a) {
    if (!(std::is_same<T, bf16_t>::value && CPL == 4)) return false;
    const uint64_t row = uint64_t(a.heads) * uint64_t(a.head_width) * sizeof(T);
    const uint64_t nt = uint64_t(a.batch) * uint64_t(a.time);
    const uint64_t reads = nt * uint64_t(a.read_banks > 0 ? a.read_banks : 1);
    return nt * row < (uint64_t(1) << 32) && reads * row < (uint64_t(1) << 32);
}

template <typename T>
int launch_mode0(const void *kernel, dim3 grid, int threads, ForwardParams<T> p, hipStream_t stream) {
    void *args[] = {&p};
    const hipError_t err = hipLaunchKernel(kernel, grid, dim3(unsigned(threads)), args, 0, stream);
    if (err != hipSuccess) return fail(BDM_ERR_LAUNCH, "lazy_forward_kernel: %s", hipGetErrorString(err));
    return check_launch("lazy_forward_kernel");
}

// MODE 0 of the lazy kernel as `parts` launches over consecutive head
// groups (each with its own longest-first rounds), part i on stream i (the
// caller's, then the auxiliary ones) behind i one-lane gate kernels, each
// part's combine over its heads' columns after it on the same stream.
// Phase events: 0 before the first part, 1 after the last part's
// recurrence, 2 after the join.
// The rounding policy's stage path on stream st (see lazy_forward_kernel):
// the piece list of the segments longer than kPieceEvents, MODE 3 over their
// pieces, the scan.  p0: the MODE 0 parameters; groups: all head groups.
template <typename T, int CPL>
int launch_stage_path(const ForwardParams<T> &p0, const PieceBuffers &pb, int threads, int groups, hipStream_t st,
                      hipEvent_t pieces_done = nullptr) {
    piece_table_kernel<<<1, 1024, 0, st>>>(p0.cu, p0.nseg, pb.st_items, pb.st_count, pb.st_segs, pb.st_count + 1);
    if (int rc = check_launch("piece_table_kernel")) return rc;
    ForwardParams<T> p = p0;
    p.items = pb.st_items;
    p.n_items = pb.st_count;
    p.pstate = pb.st_r;
    p.ptrans = pb.st_p;
    p.z0buf = pb.st_z0;
    p.cbuf = pb.st_c;
    p.tgt = pb.st_tgt;
    p.seg_order = nullptr;
    p.skip_long = 0;
    p.group_base = 0;
    const dim3 grid(unsigned(pb.stage_pieces), unsigned(groups));
    if (threads == 64)
        lazy_forward_kernel<T, CPL, 2, 3><<<grid, 64, 0, st>>>(p);
    else
        lazy_forward_kernel<T, CPL, 8, 3><<<grid, 256, 0, st>>>(p);
    if (int rc = check_launch("lazy_forward_kernel")) return rc;
    if (pieces_done && hipEventRecord(pieces_done, st) != hipSuccess)
        return fail(BDM_ERR_LAUNCH, "forward: recording the stage pieces' end");
    StageParams<T> sp{};
    sp.segs = pb.st_segs;
    sp.n_segs = pb.st_count + 1;
    sp.items = pb.st_items;
    sp.n_items = pb.st_count;
    sp.cu = p.cu;
    sp.tgt = pb.st_tgt;
    sp.initial = p.initial;
    sp.final_state = p.final_state;
    sp.pstate = pb.st_r;
    sp.ptrans = pb.st_p;
    sp.z0buf = pb.st_z0;
    sp.cbuf = pb.st_c;
    sp.zbuf = p.zbuf;
    sp.init_bstride = p.init_bstride;
    sp.row_stride = p.row_stride;
    sp.init_dtype = p.init_dtype;
    sp.final_dtype = p.final_dtype;
    sp.banks = p.banks;
    sp.heads = p.heads;
    sp.s_heads = p.s_heads;
    sp.split = p.split;
    sp.width = p.width;
    const unsigned tiles = unsigned((p.width + kWave - 1) / kWave);
    // one block per long segment up to 256 of them (a segment's chain is
    // the longest stage sequence; more segments than blocks take turns)
    const int64_t long_max = std::min<int64_t>(p.nseg, p.nt * (p.kw + p.kr) / (kPieceEvents + 1));
    const unsigned blocks = unsigned(std::max<int64_t>(1, std::min<int64_t>(long_max, 256)));
    stage_scan_kernel<T><<<dim3(blocks, unsigned(p.heads), tiles), kWave, 0, st>>>(sp);
    if (int rc = check_launch("stage_scan_kernel")) return rc;
    stage_reads_kernel<T><<<dim3(unsigned(pb.stage_pieces), unsigned(p.heads), tiles), kWave, 0, st>>>(sp);
    return check_launch("stage_reads_kernel");
}

// With the stage path (long segments under the rounding policy) its chain of
// kernels is the critical path, and all of it runs on the caller's stream:
// the pieces (MODE 3) alone on the device, then the scan, which is bound by
// its chain's latency, beside the sequential kernel over the other segments
// (on an auxiliary stream, after the pieces), then the reads and the
// combine over every column.
template <typename T, int CPL>
int launch_overlapped_stage(const bdm_forward_args &a, ForwardParams<T> p, const void *kernel, unsigned nseg,
                            int groups, int threads, const T *zbuf, const OverlapAux &ax, const PieceBuffers &pb,
                            hipStream_t stream) {
    p.skip_long = 1;  // the sequential kernel leaves the long segments to the stage path
    if (int rc = launch_stage_path<T, CPL>(p, pb, threads, groups, stream, ax.fork)) return rc;
    hipStream_t side = ax.stream[0];
    if (hipStreamWaitEvent(side, ax.fork, 0) != hipSuccess)
        return fail(BDM_ERR_LAUNCH, "forward: forking the stage path");
    if (int rc = launch_mode0<T>(kernel, dim3(nseg, unsigned(groups)), threads, p, side)) return rc;
    if (hipEventRecord(ax.join[0], side) != hipSuccess || hipStreamWaitEvent(stream, ax.join[0], 0) != hipSuccess)
        return fail(BDM_ERR_LAUNCH, "forward: joining the stage path");
    if (int rc = record_phase(a, 1, stream)) return rc;
    if (int rc = launch_combine_kernels<T>(a, zbuf, stream)) return rc;
    return record_phase(a, 2, stream);
}

template <typename T, int CPL>
int launch_overlapped(const bdm_forward_args &a, ForwardParams<T> p, const void *kernel, unsigned nseg, int groups,
                      int threads, const T *zbuf, const OverlapAux &ax, const PieceBuffers &pb, hipStream_t stream) {
    if (pb.stage_pieces > 0)
        return launch_overlapped_stage<T, CPL>(a, p, kernel, nseg, groups, threads, zbuf, ax, pb, stream);
    const int gpr = p.order_gpr;
    const int parts = overlap_parts((groups + gpr - 1) / gpr, groups);
    if (hipEventRecord(ax.fork, stream) != hipSuccess)
        return fail(BDM_ERR_LAUNCH, "forward: forking the combine streams");
    for (int i = 1; i < parts; ++i) {
        if (hipStreamWaitEvent(ax.stream[i - 1], ax.fork, 0) != hipSuccess)
            return fail(BDM_ERR_LAUNCH, "forward: forking the combine streams");
        for (int gate = 0; gate < i; ++gate) overlap_gate_kernel<<<1, 1, 0, ax.stream[i - 1]>>>();
        if (int rc = check_launch("overlap_gate_kernel")) return rc;
    }
    for (int i = 0; i < parts; ++i) {
        hipStream_t st = i ? ax.stream[i - 1] : stream;
        // the larger parts first: the last part's combine is the one left
        // exposed after the recurrence
        const int g0 = groups - int(int64_t(groups) * (parts - i) / parts);
        const int g1 = groups - int(int64_t(groups) * (parts - i - 1) / parts);
        ForwardParams<T> pr = p;
        pr.group_base = g0;
        pr.order_gpr = min(gpr, g1 - g0);
        if (int rc = launch_mode0<T>(kernel, dim3(nseg, unsigned(g1 - g0)), threads, pr, st)) return rc;
        if (i == parts - 1)
            if (int rc = record_phase(a, 1, st)) return rc;
        const int h0 = g0 * p.heads_per_block;
        const int h1 = min(g1 * p.heads_per_block, p.heads);
        if (int rc = launch_combine_kernels<T>(a, zbuf, st, h0 * p.width, (h1 - h0) * p.width)) return rc;
    }
    for (int i = 1; i < parts; ++i)
        if (hipEventRecord(ax.join[i - 1], ax.stream[i - 1]) != hipSuccess ||
            hipStreamWaitEvent(stream, ax.join[i - 1], 0) != hipSuccess)
            return fail(BDM_ERR_LAUNCH, "forward: joining the combine streams");
    return record_phase(a, 2, stream);
}

template <typename T, int S, int CPL, bool kLazy = false>
int launch_forward(const bdm_forward_args &a, T *zbuf, const PieceBuffers &pb, hipStream_t stream) {
    const int split = kLazy ? lazy_split(a) : 1;
    if (a.head_width / split / CPL > 256)
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
    p.heads = a.heads * split;
    p.s_real = a.bank_size;
    p.width = a.head_width / split;
    p.split = split;
    p.s_heads = a.heads;
    p.row_stride = a.head_width;
    p.banks = a.bank_count;
    p.kw = a.write_banks;
    p.kr = a.read_banks;
    p.k_shift = -1;
    for (int sh = 0; sh < 8; ++sh)
        if (a.write_banks == (1 << sh) && a.read_banks == (1 << sh)) p.k_shift = sh;
    p.lanes_per_head = p.width / CPL;
    p.heads_per_block = 256 / p.lanes_per_head;
    // lazy kernel: 2 heads per one-wave workgroup when a head has 32 lanes, else 8 per 256 threads
    const int lazy_hb = p.lanes_per_head == 32 ? 2 : 8;
    if (kLazy && p.heads_per_block > lazy_hb) p.heads_per_block = lazy_hb;
    if (p.heads_per_block > p.heads) p.heads_per_block = p.heads;
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
    const dim3 grid(unsigned(nseg), unsigned((p.heads + p.heads_per_block - 1) / p.heads_per_block));
    p.nseg = int(nseg);
    if (int rc = record_phase(a, 0, stream)) return rc;
    if constexpr (kLazy) {
        // the prep role needs one lane per (event, head, half): 32 per head
        const int lthreads = lazy_hb == 2 ? 64 : 256;
        if (pb.max_pieces > 0) {
            // prefill policy: long segments run as balanced pieces
            p.items = pb.items;
            p.n_items = pb.count;
            p.pstate = pb.pstate;
            p.ptrans = pb.ptrans;
            piece_table_kernel<<<1, 1024, 0, stream>>>(a.cu_seqlens, int(nseg), pb.items, pb.count, nullptr,
                                                       nullptr);
            if (int rc = check_launch("piece_table_kernel")) return rc;
            if (pb.seg_order) {
                if (!pb.order_given) {
                    launch_segment_order(a.cu_seqlens, nseg, pb.seg_order, stream);
                    if (int rc = check_launch("segment_order_kernel")) return rc;
                }
                p.seg_order = pb.seg_order;
            }
            // MODE 1: the pieces (in the first blocks, so the long ones start
            // first), then the uncut segments in the slots they leave free
            p.piece_blocks = int((pb.max_pieces + 7) / 8 * 8);
            const dim3 pgrid(unsigned(p.piece_blocks + nseg), grid.y);
            if (lazy_hb == 2)
                lazy_forward_kernel<T, CPL, 2, 1><<<pgrid, lthreads, 0, stream>>>(p);
            else
                lazy_forward_kernel<T, CPL, 8, 1><<<pgrid, lthreads, 0, stream>>>(p);
            if (int rc = check_launch("lazy_forward_kernel")) return rc;
            piece_scan_kernel<<<dim3(unsigned(pb.max_pieces), unsigned(p.heads)), 128, 0, stream>>>(
                pb.items, pb.count, a.initial, a.initial_dtype, a.initial_batch_stride, a.bank_count, p.heads,
                p.width, p.split, p.row_stride, pb.pstate, pb.ptrans);
            if (int rc = check_launch("piece_scan_kernel")) return rc;
            const dim3 g2(unsigned(p.piece_blocks), grid.y);  // MODE 2: pieces 1.. of each cut segment
            if (lazy_hb == 2)
                lazy_forward_kernel<T, CPL, 2, 2><<<g2, lthreads, 0, stream>>>(p);
            else
                lazy_forward_kernel<T, CPL, 8, 2><<<g2, lthreads, 0, stream>>>(p);
        } else {
            const void *kernel = mode0_kernel<T, CPL>(lazy_hb, buffer_form<T, CPL>(a));
            if (pb.seg_order) {
                if (!pb.order_given) {
                    launch_segment_order(a.cu_seqlens, nseg, pb.seg_order, stream);
                    if (int rc = check_launch("segment_order_kernel")) return rc;
                }
                p.seg_order = pb.seg_order;
                p.order_gpr = order_groups_per_round(kernel, lthreads, nseg, int(grid.y));
                // rounds whose heads' columns split y in whole 16-byte groups
                const bool aligned_rounds = (int64_t(p.heads_per_block) * p.width * sizeof(T)) % 16 == 0 &&
                                            (int64_t(a.heads) * a.head_width * sizeof(T)) % 16 == 0;
                if (a.read_banks > 0 && int(grid.y) > p.order_gpr && aligned_rounds && overlap_enabled()) {
                    if (const OverlapAux *ax = overlap_aux(stream)) {
                        // the shared events are recorded and waited for by one call at a time
                        std::lock_guard<std::mutex> lock(overlap_launch_mutex());
                        return launch_overlapped<T, CPL>(a, p, kernel, grid.x, int(grid.y), lthreads, zbuf, *ax, pb,
                                                         stream);
                    }
                }
            }
            // the stage path after the sequential kernel, on the same stream
            if (pb.stage_pieces > 0) {
                ForwardParams<T> ps = p;
                ps.skip_long = 1;
                if (int rc = launch_mode0<T>(kernel, grid, lthreads, ps, stream)) return rc;
                if (int rc = launch_stage_path<T, CPL>(p, pb, lthreads, int(grid.y), stream)) return rc;
                return launch_combine<T>(a, zbuf, stream);
            }
            if (int rc = launch_mode0<T>(kernel, grid, lthreads, p, stream)) return rc;
        }
        if (int rc = check_launch("lazy_forward_kernel")) return rc;
    } else {
        routed_forward_kernel<T, S, CPL><<<grid, threads, 0, stream>>>(p);
        if (int rc = check_launch("routed_forward_kernel")) return rc;
    }

    return launch_combine<T>(a, zbuf, stream);
}

// The S = 8 lazy kernel takes: 16-byte aligned state rows, 4-column lane
// groups of at most 64 lanes per head, stages of 16 events matching the
// rounding/snapshot interval, and token and route indices in 32 bits.
bool lazy_path(const bdm_forward_args &a) {
    const bool vec = a.initial_batch_stride % 8 == 0;
    const int fold = a.round_interval > 0 ? a.round_interval : (a.snapshots ? a.snapshot_interval : kLazyStage);
    const int64_t nt = a.batch * a.time;
    const bool small_index = nt * (a.write_banks > a.read_banks ? a.write_banks : a.read_banks) < INT32_MAX;
    return vec && a.bank_size == 8 && lazy_split(a) > 0 && fold == kLazyStage && small_index;
}

// Upper bound on the pieces of cut segments (0: the path is off).  It is
// taken under the prefill policy only: no rounding inside the recurrence and
// no snapshots, so a segment is an affine map of its start state.  A cut
// segment has len > L events and ceil(len/L) < len/L + 1 pieces, and fewer
// than E/L segments are cut, so the pieces number fewer than 2E/L + 1.
int64_t max_pieces(const bdm_forward_args &a) {
    if (!lazy_path(a) || a.round_interval > 0 || a.snapshots) return 0;
    const int64_t events = a.batch * a.time * (int64_t(a.write_banks) + a.read_banks);
    return 2 * (events / kPieceEvents) + 1;
}

// BDM_STAGE_PATH=1 runs segments longer than kPieceEvents under the
// rounding policy on the stage path; otherwise they run whole (the default:
// its launches cost a forward without long segments ~3 % at C2, and its
// buffers ~2-3 GiB of workspace at the C2 and C4 sizes).
bool stage_enabled() {
    const char *e = getenv("BDM_STAGE_PATH");
    return e && e[0] == '1' && e[1] == 0;
}

// Upper bound on the stage path's pieces (0: the path is off).  It runs
// beside the longest-first MODE 0 launches (their order and auxiliary
// streams), under the rounding policy without snapshots, where reads exist.
int64_t stage_pieces(const bdm_forward_args &a) {
    if (!lazy_path(a) || a.round_interval <= 0 || a.snapshots || a.read_banks <= 0 ||
        !order_geometry(a.batch * a.bank_count) || !stage_enabled())
        return 0;
    const int64_t events = a.batch * a.time * (int64_t(a.write_banks) + a.read_banks);
    return 2 * (events / kPieceEvents) + 1;
}

// Stage slots: stage k of segment s has slot cu[s] / 16 + s + k < E / 16 + segments.
int64_t stage_slots(const bdm_forward_args &a) {
    const int64_t events = a.batch * a.time * (int64_t(a.write_banks) + a.read_banks);
    return events / kLazyStage + a.batch * a.bank_count + 1;
}

// Whether the lazy kernel takes each XCD range's segments longest first
// (segment_order_kernel; MODE 0, and MODE 1's segment blocks): ranges that
// the XCD remap forms, at most kOrderMaxRange segments each.
bool order_path(const bdm_forward_args &a) { return lazy_path(a) && order_geometry(a.batch * a.bank_count); }

// BDM_FORWARD_KERNEL=mfma selects the matrix-core recurrence where it
// applies; the vector-ALU kernel is the default (both are complete
// implementations of the same forward; the variable is read at every call).
// On MI355X at the C2 geometry the matrix-core form is the slower one: its
// coefficient scan and exact gated-value split cost more vector instructions
// than the state update they move to the matrix cores.
bool chunk_enabled() {
    const char *e = getenv("BDM_FORWARD_KERNEL");
    return e && strcmp(e, "mfma") == 0;
}

// The matrix-core recurrence (chunk_forward.hip), then the combine.
int launch_chunked(const bdm_forward_args &a, bf16_t *zbuf, hipStream_t stream) {
    const int64_t nt = a.batch * a.time;
    if (int rc = record_phase(a, 0, stream)) return rc;
    const int split = a.head_width > 256 ? a.head_width / 128 : 1;
    ChunkForwardParams p{};
    p.q = static_cast<const bf16_t *>(a.q);
    p.k = static_cast<const bf16_t *>(a.k);
    p.b = static_cast<const bf16_t *>(a.b);
    p.g = a.g;
    p.v = static_cast<const bf16_t *>(a.v);
    p.w = static_cast<const bf16_t *>(a.w);
    p.ww = static_cast<const bf16_t *>(a.write_weights);
    p.rw = static_cast<const bf16_t *>(a.read_weights);
    p.order = a.order;
    p.cu = a.cu_seqlens;
    p.initial = a.initial;
    p.final_state = a.final_state;
    p.snap = static_cast<bf16_t *>(a.snapshots);
    p.zbuf = zbuf;
    p.init_bstride = a.initial_batch_stride;
    p.nt = nt;
    p.split = split;
    p.s_heads = a.heads;
    p.heads = a.heads * split;
    p.width = a.head_width / split;
    p.row_stride = a.head_width;
    p.banks = a.bank_count;
    p.kw = a.write_banks;
    p.kr = a.read_banks;
    p.kw_shift = (a.write_banks > 0 && (a.write_banks & (a.write_banks - 1)) == 0) ? __builtin_ctz(a.write_banks) : -1;
    p.kr_shift = (a.read_banks > 0 && (a.read_banks & (a.read_banks - 1)) == 0) ? __builtin_ctz(a.read_banks) : -1;
    p.routed_decay = a.routed_decay;
    p.init_dtype = a.initial_dtype;
    p.final_dtype = a.final_dtype;
    p.nseg = int(a.batch * a.bank_count);
    p.xcd_remap = p.nseg % 8 == 0 ? 1 : 0;
    p.scale = a.scale;
    if (int rc = launch_chunk_forward(p, p.width / 32, stream)) return rc;
    return launch_combine<bf16_t>(a, zbuf, stream);
}

template <typename T>
int dispatch_forward(const bdm_forward_args &a, T *zbuf, const PieceBuffers &pb, hipStream_t stream) {
    // Vector row loads need 16-byte aligned rows: aligned bases, and a state
    // batch stride that keeps them aligned.
    const bool vec = a.initial_batch_stride % 8 == 0;
    if constexpr (std::is_same<T, bf16_t>::value) {
        if (chunk_path(a) && chunk_enabled()) return launch_chunked(a, zbuf, stream);
    }
    if (a.bank_size <= 8) {
        if (lazy_path(a)) return launch_forward<T, 8, 4, true>(a, zbuf, pb, stream);
        if (vec && a.head_width % 8 == 0) return launch_forward<T, 8, 8>(a, zbuf, pb, stream);
        return launch_forward<T, 8, 1>(a, zbuf, pb, stream);
    }
    if (a.bank_size <= 16) {
        if (vec && a.head_width % 4 == 0) return launch_forward<T, 16, 4>(a, zbuf, pb, stream);
        return launch_forward<T, 16, 1>(a, zbuf, pb, stream);
    }
    if (vec && a.head_width % 2 == 0) return launch_forward<T, 32, 2>(a, zbuf, pb, stream);
    return launch_forward<T, 32, 1>(a, zbuf, pb, stream);
}

size_t elem_size(int dtype) { return dtype == BDM_BF16 ? 2 : 4; }

}  // namespace
}  // namespace bdm

// Workspace of bdm_forward: the read buffer (one ctrl_dtype row of H*v per
// read event, row token*KR + j), then, under the prefill policy, the piece
// list, its count and the FP32 piece states and transitions ([pieces, H, 8,
// v] and [pieces, H, 8, 8]), or else, where segments run longest first, the
// segment order (int32 per segment).
static size_t round256(size_t x) { return (x + 255) / 256 * 256; }

static size_t forward_zbuf_bytes(const bdm_forward_args *a) {
    return round256(size_t(a->batch) * size_t(a->time) * size_t(a->read_banks) * size_t(a->heads) *
                    size_t(a->head_width) * bdm::elem_size(a->ctrl_dtype));
}

static size_t forward_piece_bytes(const bdm_forward_args *a) {
    const size_t n = size_t(bdm::max_pieces(*a));
    if (!n) return 0;
    // transitions per virtual head of the column split
    return round256(n * sizeof(int4)) + 256 + round256(n * a->heads * 8 * size_t(a->head_width) * 4) +
           round256(n * a->heads * size_t(bdm::lazy_split(*a)) * 64 * 4);
}

static size_t forward_order_bytes(const bdm_forward_args *a) {
    return bdm::order_path(*a) ? round256(size_t(a->batch) * size_t(a->bank_count) * 4) : 0;
}

// The stage path's buffers, in this order (sizes in bytes).
static void forward_stage_parts(const bdm_forward_args *a, size_t (&part)[8]) {
    const size_t n = size_t(bdm::stage_pieces(*a));
    for (size_t &x : part) x = 0;
    if (!n) return;
    const size_t slots = size_t(bdm::stage_slots(*a));
    const size_t reads = size_t(a->batch) * size_t(a->time) * size_t(a->read_banks);
    const size_t cols = size_t(a->heads) * size_t(a->head_width);
    const size_t vheads = size_t(a->heads) * size_t(bdm::lazy_split(*a));
    part[0] = round256(n * sizeof(int4));  // piece list
    part[1] = 256;                          // counts
    part[2] = round256(n * 4);              // first pieces of the long segments
    part[3] = round256(slots * 8 * cols * 4);     // R per stage slot: [slots, heads, 8, width]
    part[4] = round256(slots * vheads * 64 * 4);  // P per stage slot: [slots, heads, 8, 8]
    part[5] = round256(reads * cols * 4);         // zero-start read rows: [NT*KR, H*v]
    part[6] = round256(reads * vheads * 8 * 4);   // read coefficients: [NT*KR, heads, 8]
    part[7] = round256(slots * 16 * 4);           // read targets per stage slot: [slots, 16]
}

static size_t forward_stage_bytes(const bdm_forward_args *a) {
    size_t part[8], total = 0;
    forward_stage_parts(a, part);
    for (size_t x : part) total += x;
    return total;
}

extern "C" size_t bdm_forward_workspace_size(const bdm_forward_args *a) {
    if (!a || a->batch <= 0 || a->time <= 0 || a->heads <= 0 || a->head_width <= 0 || a->read_banks < 0 ||
        a->write_banks < 0 || a->bank_size <= 0)
        return 0;
    return forward_zbuf_bytes(a) + forward_piece_bytes(a) + forward_order_bytes(a) + forward_stage_bytes(a);
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
    if (a->batch * a->time * a->read_banks > int64_t(INT32_MAX))
        return fail(BDM_ERR_UNSUPPORTED, "forward: more than 2^31 read events");
    hipStream_t s = as_stream(stream);
    char *ws = static_cast<char *>(workspace);
    PieceBuffers pb;
    pb.max_pieces = max_pieces(*a);
    if (pb.max_pieces > INT32_MAX / 2) return fail(BDM_ERR_UNSUPPORTED, "forward: too many pieces");
    if (pb.max_pieces) {
        char *at = ws + forward_zbuf_bytes(a);
        const size_t n = size_t(pb.max_pieces);
        pb.items = reinterpret_cast<int4 *>(at);
        at += round256(n * sizeof(int4));
        pb.count = reinterpret_cast<int *>(at);
        at += 256;
        pb.pstate = reinterpret_cast<float *>(at);
        at += round256(n * a->heads * 8 * size_t(a->head_width) * 4);
        pb.ptrans = reinterpret_cast<float *>(at);
    }
    if (order_path(*a) && order_enabled()) {
        pb.seg_order = reinterpret_cast<int *>(ws + forward_zbuf_bytes(a) + forward_piece_bytes(a));
        pb.order_given = a->segment_order != nullptr;
        if (pb.order_given) pb.seg_order = const_cast<int *>(a->segment_order);
    }
    pb.stage_pieces = stage_pieces(*a);
    if (pb.stage_pieces > INT32_MAX / 2) return fail(BDM_ERR_UNSUPPORTED, "forward: too many pieces");
    if (pb.stage_pieces) {
        size_t part[8];
        forward_stage_parts(a, part);
        char *at = ws + forward_zbuf_bytes(a) + forward_piece_bytes(a) + forward_order_bytes(a);
        char *ptr[8];
        for (int i = 0; i < 8; ++i) {
            ptr[i] = at;
            at += part[i];
        }
        pb.st_items = reinterpret_cast<int4 *>(ptr[0]);
        pb.st_count = reinterpret_cast<int *>(ptr[1]);
        pb.st_segs = reinterpret_cast<int *>(ptr[2]);
        pb.st_r = reinterpret_cast<float *>(ptr[3]);
        pb.st_p = reinterpret_cast<float *>(ptr[4]);
        pb.st_z0 = reinterpret_cast<float *>(ptr[5]);
        pb.st_c = reinterpret_cast<float *>(ptr[6]);
        pb.st_tgt = reinterpret_cast<int *>(ptr[7]);
    }
    if (a->ctrl_dtype == BDM_BF16)
        return dispatch_forward<bf16_t>(*a, static_cast<bf16_t *>(workspace), pb, s);
    return dispatch_forward<float>(*a, static_cast<float *>(workspace), pb, s);
}

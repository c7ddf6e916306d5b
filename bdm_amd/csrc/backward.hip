// Backward of the routed GDN2 bank recurrence and the token-level VJP.
//
// Reference: _role_backward (role_bank_kernel.py:76-150, launched by
// backward() at :205-228), RoutedUpdate.backward (routed_update.py:31-49:
// the decay term of d(ww) and dg scaled by p) and _vjp
// (role_bank_dispatch.py:76-132, with its BF16 rounding points).
//
// Per write event the adjoint dM (S x v) of the state after the event gives
//   du = dM^T k;  U = dM u;  X = hd du;  P = rowsum(dM o hd)
//   dM <- (dM - a du^T) o decay                (role_bank_kernel.py:128-138)
// and per read event dq = scale M dy, dM += scale eq dy^T (:141-143).  U, X
// and P (S values each) are stored per event; the token kernel forms
// dk = U - eb X, db = -k X, dg = P - a X from them and the event's operands.
//
// chunk_backward_kernel (S = 8, replay interval 16): one wave per (segment,
// head, column tile); a lane owns 2 value columns and all 8 rows.  Chunks of
// 16 events are visited in reverse.  The chunk's states are rebuilt exactly
// from its snapshot by the forward's write update, in two halves of 8 events:
// the states before events 8..15 are kept in registers while the second half
// is differentiated, then those before events 0..7.  Per event operands (the
// write's k, decay, a rows and bf(w p), v columns; the read's eq*scale row
// and dy columns) are staged in LDS one chunk ahead: the next chunk's loads
// are issued before the current chunk's last half is differentiated.  The
// S-wide column reductions use permlane swaps and DPP row sums
// (reduce-scatter: each output ends in one lane, no LDS round trip).
//
// routed_backward_kernel: the general path (any S <= 32, intervals 4/8/16).
// Same arithmetic; pieces of SUB events, operands loaded per event.
//
// token_grad_kernel: one workgroup per token, one wave per head.  Lane
// (j, r) = (lane / 8, lane % 8) handles route slot j and state row r of the
// S-side gradients; lanes own 2 value columns for dv, dw.  The token's KW
// write events and KR read events are folded in route order with the
// reference's rounding (role_bank_dispatch.py:99-131); route-weight
// gradients add the heads' contributions in head order in FP32.
// token_vjp_kernel: the same for shapes outside that kernel's limits.
#include "bdm_common.h"
#include "recurrence_ops.h"
#include "segment_order.h"

namespace bdm {
namespace {

constexpr int kLanes = 64;

template <typename T>
struct BackwardParams {
    const T *q, *k, *b;
    const float *g;
    const T *v, *w;
    const T *ww, *rw;
    const int64_t *order, *cu;
    const void *initial;
    const void *snap;
    const T *dy;
    float *du;      // [NT*KW, H, v]
    float *wpart;   // [tiles, NT*KW, H, 3, S]: U, X, P of each write slot
    float *rpart;   // [tiles, NT*KR, H, S]: dq of each read slot
    const int4 *meta;  // [E]: token, route slot, is_read, route weight (FP32 bits)
    float *dinit;   // [batch, J, H, S, v]
    int64_t init_bstride, nt;
    int heads, s_real, width, banks, kw, kr, tiles;
    int init_dtype, snap_dtype, routed_decay, rounding;
    int xcd_remap;
    float scale;
    // chunk kernel: each XCD range's segments longest first
    // (segment_order_kernel), in rounds of order_gpr (head, tile) items;
    // null keeps bank order
    const int *seg_order;
    int order_gpr;
};

// The (segment, head, column tile) of this block.  In order: segments
// remapped so each XCD takes a contiguous range, head = y, tile = z.  With
// p.seg_order: blocks reach the XCDs round-robin in dispatch order (x
// fastest), and the k-th block of XCD x runs item k of its range
// (order_item): rounds of (head, tile) groups, segments longest first.
template <typename T>
__device__ __forceinline__ void block_item(const BackwardParams<T> &p, int &seg, int &head, int &tile) {
    const int nseg = gridDim.x;
    if (p.seg_order) {
        const int64_t linear = (int64_t(blockIdx.z) * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
        const int range = nseg / 8;
        int rank, group;
        order_item(linear / 8, range, int(gridDim.y * gridDim.z), p.order_gpr, rank, group);
        seg = p.seg_order[int(linear % 8) * range + rank];
        head = group / int(gridDim.z);
        tile = group % int(gridDim.z);
    } else {
        seg = p.xcd_remap ? int((blockIdx.x % 8) * (nseg / 8) + blockIdx.x / 8) : int(blockIdx.x);
        head = blockIdx.y;
        tile = blockIdx.z;
    }
}

__device__ __forceinline__ int64_t uniform64(int64_t x) {
    const int lo = __builtin_amdgcn_readfirstlane(int(uint32_t(uint64_t(x))));
    const int hi = __builtin_amdgcn_readfirstlane(int(uint32_t(uint64_t(x) >> 32)));
    return int64_t((uint64_t(uint32_t(hi)) << 32) | uint64_t(uint32_t(lo)));
}

template <int N>
__device__ __forceinline__ void wave_reduce(float (&x)[N]) {
    // Butterfly: every lane ends with the same total (each step adds the
    // same two operands on both partners, and FP32 addition commutes).
#pragma unroll
    for (int m = kLanes / 2; m >= 1; m >>= 1) {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] += __shfl_xor(x[i], m, kLanes);
    }
}

template <int S, typename E>
__device__ __forceinline__ void load_s(const E *p, int s_real, float (&out)[S]) {
#pragma unroll
    for (int r = 0; r < S; ++r) out[r] = r < s_real ? to_f32(p[r]) : 0.f;
}

template <int CPL, typename E>
__device__ __forceinline__ void load_cols(const E *row, int col0, int width, float (&out)[CPL]) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) out[c] = col0 + c < width ? to_f32(row[col0 + c]) : 0.f;
}

template <int S, int CPL>
__device__ __forceinline__ void load_state_cols(const void *base, int dtype, int64_t offset, int width, int s_real,
                                                int col0, float (&h)[S][CPL]) {
#pragma unroll
    for (int r = 0; r < S; ++r)
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const bool live = r < s_real && col0 + c < width;
            const int64_t at = offset + int64_t(r) * width + c;
            h[r][c] = !live ? 0.f
                            : (dtype == BDM_BF16 ? to_f32(static_cast<const bf16_t *>(base)[at])
                                                 : static_cast<const float *>(base)[at]);
        }
}

template <typename T, int S, int CPL>
struct WriteEvent {
    WriteRows<S> rows;
    float ew[CPL], value[CPL];
};

template <typename T, int S, int CPL>
__device__ __forceinline__ void load_write(const BackwardParams<T> &p, int64_t token, float pw, int head, int col0,
                                           WriteEvent<T, S, CPL> &ev) {
    const int64_t row = token * p.heads + head;
    float k[S], g[S], b[S], wv[CPL];
    load_s<S>(p.k + row * p.s_real, p.s_real, k);
    load_s<S>(p.g + row * p.s_real, p.s_real, g);
    load_s<S>(p.b + row * p.s_real, p.s_real, b);
    prepare_write_rows<T, S>(k, g, b, pw, p.routed_decay, ev.rows);
    load_cols<CPL>(p.v + row * p.width, col0, p.width, ev.value);
    load_cols<CPL>(p.w + row * p.width, col0, p.width, wv);
#pragma unroll
    for (int c = 0; c < CPL; ++c) ev.ew[c] = round_to<T>(wv[c] * pw);
}

template <typename T, int S, int CPL, int C>
__global__ __launch_bounds__(64) void routed_backward_kernel(BackwardParams<T> p) {
    constexpr int SUB = C < 4 ? C : 4;
    constexpr int NCK = C / SUB;
    __shared__ int64_t s_token[C];
    __shared__ int64_t s_slot[C];  // write: token*KW + j; read: token*KR + j
    __shared__ float s_weight[C];
    __shared__ int s_read[C];

    int seg, head, tile;
    block_item(p, seg, head, tile);
    const int bank = seg % p.banks;
    const int64_t bidx = seg / p.banks;
    const int lane = threadIdx.x;
    const int col0 = (tile * kLanes + lane) * CPL;
    const int64_t start = p.cu[seg], end = p.cu[seg + 1];
    const int64_t write_events = p.nt * p.kw;
    const int64_t events = p.nt * (p.kw + p.kr);

    float dm[S][CPL];
#pragma unroll
    for (int r = 0; r < S; ++r)
#pragma unroll
        for (int c = 0; c < CPL; ++c) dm[r][c] = 0.f;

    const int64_t count = (end - start + C - 1) / C;
    for (int64_t chunk = count - 1; chunk >= 0; --chunk) {
        const int64_t base = start + chunk * C;
        const int len = int(min(int64_t(C), end - base));
        __syncthreads();
        if (lane < len) {
            int64_t o = p.order[base + lane];
            o = o < 0 ? 0 : (o >= events ? events - 1 : o);
            const bool rd = o >= write_events;
            const int64_t route = rd ? o - write_events : o;
            s_token[lane] = rd ? route / p.kr : route / p.kw;
            s_slot[lane] = route;
            s_weight[lane] = rd ? to_f32(p.rw[route]) : to_f32(p.ww[route]);
            s_read[lane] = rd;
        }
        __syncthreads();

        // state before the chunk's first event
        float m0[S][CPL];
        if (chunk == 0) {
            const int64_t off = bidx * p.init_bstride + (int64_t(bank) * p.heads + head) * p.s_real * p.width + col0;
            load_state_cols<S, CPL>(p.initial, p.init_dtype, off, p.width, p.s_real, col0, m0);
            if (p.rounding) {
#pragma unroll
                for (int r = 0; r < S; ++r)
#pragma unroll
                    for (int c = 0; c < CPL; ++c) m0[r][c] = round_bf16(m0[r][c]);
            }
        } else {
            const int64_t row = base / C - 1;
            load_state_cols<S, CPL>(p.snap, p.snap_dtype, (row * p.heads + head) * p.s_real * p.width + col0,
                                    p.width, p.s_real, col0, m0);
        }

        // The state before each event of piece sc (events sc*SUB .. sc*SUB+SUB-1)
        // is rebuilt from m0 by replaying the chunk's earlier writes; pieces
        // are visited in reverse.  The piece loop is not unrolled, so no
        // register array is indexed by it.
#pragma unroll 1
        for (int sc = NCK - 1; sc >= 0; --sc) {
            float m[S][CPL];
#pragma unroll
            for (int r = 0; r < S; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) m[r][c] = m0[r][c];
#pragma unroll 1
            for (int j = 0; j < sc * SUB; ++j) {
                if (j < len && !s_read[j]) {
                    WriteEvent<T, S, CPL> ev;
                    load_write<T, S, CPL>(p, uniform64(s_token[j]), s_weight[j], head, col0, ev);
                    apply_write<S, CPL>(m, ev.rows, ev.ew, ev.value);
                }
            }
            float st[SUB][S][CPL];
#pragma unroll
            for (int jj = 0; jj < SUB; ++jj) {
#pragma unroll
                for (int r = 0; r < S; ++r)
#pragma unroll
                    for (int c = 0; c < CPL; ++c) st[jj][r][c] = m[r][c];
                const int j = sc * SUB + jj;
                if (jj + 1 < SUB && j < len && !s_read[j]) {
                    WriteEvent<T, S, CPL> ev;
                    load_write<T, S, CPL>(p, uniform64(s_token[j]), s_weight[j], head, col0, ev);
                    apply_write<S, CPL>(m, ev.rows, ev.ew, ev.value);
                }
            }
#pragma unroll
            for (int jj = SUB - 1; jj >= 0; --jj) {
                const int j = sc * SUB + jj;
                if (j >= len) continue;
                const int64_t token = uniform64(s_token[j]);
                const int64_t slot = uniform64(s_slot[j]);
                const float pw = s_weight[j];
                if (!s_read[j]) {
                    WriteEvent<T, S, CPL> ev;
                    load_write<T, S, CPL>(p, token, pw, head, col0, ev);
                    // hd, u exactly as the forward computed them
                    float hd[S][CPL], u[CPL], du[CPL];
                    float red[3 * S];  // U = sum dm*u, X = sum hd*du, P = sum dm*hd, per row
#pragma unroll
                    for (int i = 0; i < 3 * S; ++i) red[i] = 0.f;
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        float erase = 0.f;
#pragma unroll
                        for (int r = 0; r < S; ++r) {
                            hd[r][c] = st[jj][r][c] * ev.rows.decay[r];
                            erase = fmaf(ev.rows.a[r], hd[r][c], erase);
                        }
                        u[c] = fmaf(ev.ew[c], ev.value[c], -erase);
                        float acc = 0.f;
#pragma unroll
                        for (int r = 0; r < S; ++r) acc = fmaf(dm[r][c], ev.rows.key[r], acc);
                        du[c] = acc;
                    }
#pragma unroll
                    for (int r = 0; r < S; ++r)
#pragma unroll
                        for (int c = 0; c < CPL; ++c) {
                            red[r] = fmaf(dm[r][c], u[c], red[r]);
                            red[S + r] = fmaf(hd[r][c], du[c], red[S + r]);
                            red[2 * S + r] = fmaf(dm[r][c], hd[r][c], red[2 * S + r]);
                            // dh <- (dh - a du^T) * decay (role_bank_kernel.py:130-138)
                            dm[r][c] = (dm[r][c] - ev.rows.a[r] * du[c]) * ev.rows.decay[r];
                        }
                    float *du_row = p.du + (slot * p.heads + head) * p.width;
#pragma unroll
                    for (int c = 0; c < CPL; ++c)
                        if (col0 + c < p.width) du_row[col0 + c] = du[c];
                    wave_reduce<3 * S>(red);
                    // U, X, P of row `lane` (the token kernel forms dk, db, dg)
                    float out_u = 0.f, out_x = 0.f, out_p = 0.f;
#pragma unroll
                    for (int r = 0; r < S; ++r) {
                        if (lane == r) {
                            out_u = red[r];
                            out_x = red[S + r];
                            out_p = red[2 * S + r];
                        }
                    }
                    if (lane < p.s_real) {
                        const int64_t nslots = p.nt * p.kw;
                        float *wp = p.wpart + ((int64_t(tile) * nslots + slot) * p.heads + head) * 3 * p.s_real;
                        wp[lane] = out_u;
                        wp[p.s_real + lane] = out_x;
                        wp[2 * p.s_real + lane] = out_p;
                    }
                } else {
                    const int64_t row = token * p.heads + head;
                    float q[S], eq[S], dy[CPL];
                    load_s<S>(p.q + row * p.s_real, p.s_real, q);
#pragma unroll
                    for (int r = 0; r < S; ++r) eq[r] = round_to<T>(q[r] * pw);
                    load_cols<CPL>(p.dy + row * p.width, col0, p.width, dy);
                    float red[S];
#pragma unroll
                    for (int r = 0; r < S; ++r) {
                        red[r] = 0.f;
#pragma unroll
                        for (int c = 0; c < CPL; ++c) red[r] = fmaf(st[jj][r][c], dy[c], red[r]);
                    }
                    // dh += scale * q do^T (role_bank_kernel.py:141-143)
#pragma unroll
                    for (int r = 0; r < S; ++r)
#pragma unroll
                        for (int c = 0; c < CPL; ++c) dm[r][c] += eq[r] * dy[c] * p.scale;
                    wave_reduce<S>(red);
                    float out_q = 0.f;
#pragma unroll
                    for (int r = 0; r < S; ++r)
                        if (lane == r) out_q = red[r] * p.scale;
                    if (lane < p.s_real)
                        p.rpart[((int64_t(tile) * p.nt * p.kr + slot) * p.heads + head) * p.s_real + lane] = out_q;
                }
            }
        }
    }
    // adjoint of the segment's initial state (FP32, per sequence)
    const int64_t off = ((bidx * p.banks + bank) * p.heads + head) * p.s_real * p.width + col0;
#pragma unroll
    for (int r = 0; r < S; ++r)
#pragma unroll
        for (int c = 0; c < CPL; ++c)
            if (r < p.s_real && col0 + c < p.width) p.dinit[off + int64_t(r) * p.width + c] = dm[r][c];
}


// ------------------------------------------------- S = 8, replay interval 16

// Sums over lane pairs l, l + 32: lanes 0..31 return a(l) + a(l + 32), lanes
// 32..63 return b(l - 32) + b(l) (v_permlane32_swap exchanges a's upper half
// with b's lower half).
__device__ __forceinline__ float half_pair_sum(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sums over 16-lane row pairs (0, 1) and (2, 3): rows 0 and 2 return a
// summed with the next row, rows 1 and 3 return b summed with the previous
// row (v_permlane16_swap exchanges a's odd rows with b's even rows).
__device__ __forceinline__ float row_pair_sum(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
    return x + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF,
                                                                     false));
}

// x of the lane CTRL (a DPP row_shr / row_shl) names inside the 16-lane row,
// 1 where that lane lies outside the row.
template <int CTRL>
__device__ __forceinline__ float row_shift(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, 1.f),
                                                                 __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// x * (x of the lane CTRL selects within the row), or x where that lane lies
// outside the row: one v_mul_f32 with a DPP source and bound_ctrl off (the
// lane without a source does not write).  CTRL: 0x111/0x112/0x114/0x118 are
// row_shr 1/2/4/8, 0x101/0x102/0x104/0x108 row_shl 1/2/4/8.  The s_nop gives
// the 2 wait states a DPP read of a VGPR needs after a VALU write of it.
template <int CTRL>
__device__ __forceinline__ float row_mul_step(float x) {
#define BDM_DPP_MUL(SEL) asm volatile("s_nop 1\n\tv_mul_f32_dpp %0, %0, %0 " SEL " row_mask:0xf bank_mask:0xf" : "+v"(x))
    if constexpr (CTRL == 0x111) BDM_DPP_MUL("row_shr:1");
    else if constexpr (CTRL == 0x112) BDM_DPP_MUL("row_shr:2");
    else if constexpr (CTRL == 0x114) BDM_DPP_MUL("row_shr:4");
    else if constexpr (CTRL == 0x118) BDM_DPP_MUL("row_shr:8");
    else if constexpr (CTRL == 0x101) BDM_DPP_MUL("row_shl:1");
    else if constexpr (CTRL == 0x102) BDM_DPP_MUL("row_shl:2");
    else if constexpr (CTRL == 0x104) BDM_DPP_MUL("row_shl:4");
    else if constexpr (CTRL == 0x108) BDM_DPP_MUL("row_shl:8");
    else static_assert(CTRL == 0x111, "row_mul_step: unsupported DPP control");
#undef BDM_DPP_MUL
    return x;
}

// Total of a 16-lane row in every lane of the row.
__device__ __forceinline__ float row_total(float x) {
    x = dpp_add<0xB1>(x);      // quad_perm [1,0,3,2]
    x = dpp_add<0x4E>(x);      // quad_perm [2,3,0,1]
    x = dpp_add<0x141>(x);     // row_half_mirror: quads 0 <-> 1, 2 <-> 3
    return dpp_add<0x140>(x);  // row_mirror: halves of the row
}

// Sums each of N values over the 64 lanes of the wave.  Value o = (N/4) * row
// + i (row = lane / 16) ends in the lanes of that row at position
// lane % 16 = i < N/4, which return it; other lanes return a partial sum.
template <int N>
__device__ __forceinline__ float reduce_scatter(const float (&x)[N], int lane) {
    static_assert(N % 4 == 0, "N");
    float y[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; ++i) y[i] = half_pair_sum(x[i], x[i + N / 2]);
    float z[N / 4];
#pragma unroll
    for (int i = 0; i < N / 4; ++i) z[i] = row_total(row_pair_sum(y[i], y[i + N / 4]));
    const int pos = lane & 15;
    float out = z[0];
#pragma unroll
    for (int i = 1; i < N / 4; ++i) out = pos == i ? z[i] : out;
    // computed in every lane: keeps the DPP adds fused when the caller stores
    // from a subset of lanes
    asm volatile("" : "+v"(out));
    return out;
}

// Two adjacent columns of T as loaded (BF16 pairs stay packed).
template <typename T>
struct Pair;
template <>
struct Pair<bf16_t> {
    using raw = uint32_t;
    static __device__ __forceinline__ raw load(const bf16_t *p) { return *reinterpret_cast<const uint32_t *>(p); }
    static __device__ __forceinline__ float lo(raw r) { return __uint_as_float(r << 16); }
    static __device__ __forceinline__ float hi(raw r) { return __uint_as_float(r & 0xffff0000u); }
    // bf(x*p) of both halves, packed
    static __device__ __forceinline__ raw scaled(raw r, float pw) { return pack_bf16x2(lo(r) * pw, hi(r) * pw); }
    static __device__ __forceinline__ raw zero() { return 0u; }
};
template <>
struct Pair<float> {
    using raw = float2;
    static __device__ __forceinline__ raw load(const float *p) { return *reinterpret_cast<const float2 *>(p); }
    static __device__ __forceinline__ float lo(raw r) { return r.x; }
    static __device__ __forceinline__ float hi(raw r) { return r.y; }
    static __device__ __forceinline__ raw scaled(raw r, float pw) { return make_float2(r.x * pw, r.y * pw); }
    static __device__ __forceinline__ raw zero() { return make_float2(0.f, 0.f); }
};

// One entry per event of the packed order: token, route slot, is_read and
// the route weight (FP32 bits), shared by every head.
template <typename T>
__global__ __launch_bounds__(256) void event_meta_kernel(const int64_t *order, int64_t events, int64_t write_events,
                                                         int kw, int kr, const T *ww, const T *rw, int4 *meta) {
    const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= events) return;
    int64_t o = order[e];
    o = o < 0 ? 0 : (o >= events ? events - 1 : o);
    const bool rd = o >= write_events;
    const int64_t route = rd ? o - write_events : o;
    const int64_t token = rd ? route / kr : route / kw;
    const float weight = to_f32(rd ? rw[route] : ww[route]);
    meta[e] = make_int4(int(token), int(route), rd ? 1 : 0, __float_as_int(weight));
}

template <typename T, typename SNAP>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void chunk_backward_kernel(
    BackwardParams<T> p) {
    constexpr int S = 8, CPL = 2, C = 16, HALF = 8;
    // Per-event operand row (64 floats).  Write: the adjoint's k*sigma,
    // erase coefficient a*decay*s, update a/sigma, replay k/s', the output
    // scales of U, X, P and the decay; read: eq*scale/sigma and dq's scale.
    constexpr int kKey = 0, kErase = 8, kUpd = 16, kRep = 24, kScale = 32, kDecay = 56;
    using P2 = Pair<T>;
    using Raw = typename P2::raw;
    using SnapRaw = typename Pair<SNAP>::raw;
    struct ColSlot {
        Raw a, b;  // write: v, bf(w p); read: dy, unused
    };
    struct Staged {
        Raw a[C], b[C];
        Raw kq, bb;
        float2 g;
        SnapRaw m0[S];  // snapshot rows (chunks > 0)
    };
    __shared__ int4 s_meta[2][C];
    __shared__ float4 s_rows[C][16];
    __shared__ ColSlot s_cols[C][kLanes];
    __shared__ float2 s_m0[S][kLanes];  // the chunk's start state, lane's column pair per row
    __shared__ float s_fold[S];         // product of the chunk's decays per row (lazy chunks) or 1
    __shared__ int s_eager;

    int seg, head, tile;
    block_item(p, seg, head, tile);
    const int bank = seg % p.banks;
    const int64_t bidx = seg / p.banks;
    const int lane = threadIdx.x;
    const int col0 = (tile * kLanes + lane) * CPL;
    const bool live = col0 < p.width;
    const int colc = live ? col0 : p.width - CPL;  // lanes past the width load a valid pair and zero it
    const int64_t start = p.cu[seg], end = p.cu[seg + 1];
    const int count = int((end - start + C - 1) / C);
    const uint32_t hw = uint32_t(p.heads) * uint32_t(p.width);
    const int lane_col = head * p.width + colc;  // offset of the lane's pair in a [token] row of H*v
    // event-uniform bases: x[slot] + per-lane offset
    float *du_lane = p.du + head * p.width + col0;
    float *wp_tile = p.wpart + (int64_t(tile) * p.nt * p.kw * p.heads + head) * 3 * S;
    float *rp_tile = p.rpart + (int64_t(tile) * p.nt * p.kr * p.heads + head) * S;

    auto chunk_len = [&](int c) { return int(min(int64_t(C), end - (start + int64_t(c) * C))); };
    auto load_meta = [&](int c) {
        const int len = chunk_len(c);
        return p.meta[start + int64_t(c) * C + (lane < len ? lane : len - 1)];
    };
    auto store_meta = [&](int c, const int4 &m) {
        if (lane < C) s_meta[c & 1][lane] = m;
    };
    // Loads of chunk c's operands and start state (its meta is in LDS).
    auto issue_stage = [&](int c, Staged &sg) {
        const int len = chunk_len(c);
        const int4 *mt = s_meta[c & 1];
#pragma unroll
        for (int e = 0; e < C; ++e) {
            const int4 m = mt[e < len ? e : len - 1];
            const uint64_t row = uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(m.x))) * hw;
            const bool rd = __builtin_amdgcn_readfirstlane(m.z) != 0;
            sg.a[e] = P2::load((rd ? p.dy : p.v) + row + lane_col);
            sg.b[e] = P2::load((rd ? p.dy : p.w) + row + lane_col);
        }
        {
            const int e = lane & (C - 1), rp = (lane >> 4) * 2;
            const int4 m = mt[e < len ? e : len - 1];
            const int64_t at = (int64_t(m.x) * p.heads + head) * S + rp;
            sg.kq = P2::load((m.z ? p.q : p.k) + at);
            sg.bb = P2::load(p.b + at);
            sg.g = *reinterpret_cast<const float2 *>(p.g + at);
        }
        if (c > 0) {
            const SNAP *snap = static_cast<const SNAP *>(p.snap) +
                               (((start + int64_t(c) * C) / C - 1) * p.heads + head) * S * p.width + colc;
#pragma unroll
            for (int r = 0; r < S; ++r) sg.m0[r] = Pair<SNAP>::load(snap + r * p.width);
        }
    };
    // Operand rows, columns and the start state of chunk c into LDS.
    auto finish_stage = [&](int c, const Staged &sg) {
        const int len = chunk_len(c);
        const int4 *mt = s_meta[c & 1];
#pragma unroll
        for (int e = 0; e < C; ++e) {
            const int4 m = mt[e < len ? e : len - 1];
            const bool rd = __builtin_amdgcn_readfirstlane(m.z) != 0;
            const float pw = __int_as_float(__builtin_amdgcn_readfirstlane(m.w));
            ColSlot cs;
            cs.a = live ? sg.a[e] : P2::zero();
            cs.b = (live && !rd) ? P2::scaled(sg.b[e], pw) : P2::zero();
            s_cols[e][lane] = cs;
        }
        {
            // lane = 16 j + e holds rows 2j, 2j+1 of event e: the scans over a
            // chunk's events run inside 16-lane rows (DPP row shifts)
            const int e = lane & (C - 1), rp = (lane >> 4) * 2;
            const int4 m = mt[e < len ? e : len - 1];
            const bool valid = e < len;
            const bool wr = valid && m.z == 0;
            const float pw = __int_as_float(m.w);
            const float x[2] = {P2::lo(sg.kq), P2::hi(sg.kq)};  // k of a write, q of a read
            const float bv[2] = {P2::lo(sg.bb), P2::hi(sg.bb)};
            const float gv[2] = {sg.g.x, sg.g.y};
            float d[2], a[2], pre[2], suf[2], pre_x[2], suf_x[2];
            bool bad = false;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                // decay = exp(g p), a = bf(b p) k (prepare_write_rows); 1 for reads
                d[i] = wr ? __expf(p.routed_decay ? gv[i] * pw : gv[i]) : 1.f;
                a[i] = round_to<T>(bv[i] * pw) * x[i];
                // inclusive prefix and suffix products of the decays over the chunk's events
                pre[i] = row_mul_step<0x118>(row_mul_step<0x114>(row_mul_step<0x112>(row_mul_step<0x111>(d[i]))));
                suf[i] = row_mul_step<0x108>(row_mul_step<0x104>(row_mul_step<0x102>(row_mul_step<0x101>(d[i]))));
                pre_x[i] = row_shift<0x111>(pre[i]);
                suf_x[i] = row_shift<0x101>(suf[i]);
                const float lo = 0x1p-40f, hi = 0x1p40f;
                bad |= !(pre[i] >= lo && pre[i] <= hi && suf[i] >= lo && suf[i] <= hi);
            }
            // Lazy chunk: state diag(s) Mh with s = the decays of the chunk's earlier
            // writes, adjoint diag(sigma) dMh with sigma = those of its later writes.
            // Eager chunk (a product out of range): s = sigma = 1 and both are
            // multiplied by the decay after each write.
            const bool eager = __ballot(bad) != 0;
            float *row = reinterpret_cast<float *>(&s_rows[e][0]);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = rp + i;
                const float s = eager ? 1.f : pre_x[i];                // before the event
                const float s1 = eager ? fmaxf(d[i], 0x1p-40f) : pre[i];  // after a write
                const float sg_ = eager ? 1.f : suf_x[i];
                const float inv_sg = __builtin_amdgcn_rcpf(sg_);
                if (m.z) {
                    const float eqs = round_to<T>(x[i] * pw) * p.scale;
                    row[kKey + r] = eqs * inv_sg;
                    row[kScale + r] = p.scale * s;
                } else {
                    row[kKey + r] = x[i] * sg_;
                    row[kErase + r] = a[i] * d[i] * s;
                    row[kUpd + r] = a[i] * inv_sg;
                    row[kRep + r] = x[i] * __builtin_amdgcn_rcpf(s1);
                    row[kScale + r] = sg_;
                    row[kScale + S + r] = d[i] * s;
                    row[kScale + 2 * S + r] = d[i] * s * sg_;
                    row[kDecay + r] = s1;
                }
                if (e == 0) s_fold[r] = eager ? 1.f : suf[i];
            }
            if (lane == 0) s_eager = eager ? 1 : 0;
        }
        float m0[S][CPL];
        if (c > 0) {
#pragma unroll
            for (int r = 0; r < S; ++r) {
                m0[r][0] = live ? Pair<SNAP>::lo(sg.m0[r]) : 0.f;
                m0[r][1] = live ? Pair<SNAP>::hi(sg.m0[r]) : 0.f;
            }
        } else {
            // the segment's initial state (rounded to BF16 under the rounding policy)
            const int64_t off = bidx * p.init_bstride + (int64_t(bank) * p.heads + head) * S * p.width + colc;
            float lo[S], hi[S];
            if (p.init_dtype == BDM_BF16) {
                uint32_t x[S];
#pragma unroll
                for (int r = 0; r < S; ++r)
                    x[r] = Pair<bf16_t>::load(static_cast<const bf16_t *>(p.initial) + off + r * p.width);
#pragma unroll
                for (int r = 0; r < S; ++r) lo[r] = Pair<bf16_t>::lo(x[r]), hi[r] = Pair<bf16_t>::hi(x[r]);
            } else {
                float2 x[S];
#pragma unroll
                for (int r = 0; r < S; ++r)
                    x[r] = Pair<float>::load(static_cast<const float *>(p.initial) + off + r * p.width);
#pragma unroll
                for (int r = 0; r < S; ++r) {
                    lo[r] = x[r].x, hi[r] = x[r].y;
                    if (p.rounding) round_pair<bf16_t>(lo[r], hi[r]);
                }
            }
#pragma unroll
            for (int r = 0; r < S; ++r) {
                m0[r][0] = live ? lo[r] : 0.f;
                m0[r][1] = live ? hi[r] : 0.f;
            }
        }
#pragma unroll
        for (int r = 0; r < S; ++r) s_m0[r][lane] = make_float2(m0[r][0], m0[r][1]);
    };
    auto load_m0 = [&](float (&m)[S][CPL]) {
#pragma unroll
        for (int r = 0; r < S; ++r) {
            const float2 x = s_m0[r][lane];
            m[r][0] = x.x;
            m[r][1] = x.y;
        }
    };
    auto rows8 = [&](int e, int at, float (&x)[S]) {
        const float4 lo = s_rows[e][at / 4], hi = s_rows[e][at / 4 + 1];
        x[0] = lo.x, x[1] = lo.y, x[2] = lo.z, x[3] = lo.w, x[4] = hi.x, x[5] = hi.y, x[6] = hi.z, x[7] = hi.w;
    };
    // Replay of write e: u = bf(w p) v - sum_r (a decay s)_r Mh_r ; Mh += (k / s') u.
    auto apply = [&](int e, float (&m)[S][CPL]) {
        float ce[S], kt[S];
        rows8(e, kErase, ce);
        rows8(e, kRep, kt);
        const ColSlot cs = s_cols[e][lane];
        const float v[CPL] = {P2::lo(cs.a), P2::hi(cs.a)}, ew[CPL] = {P2::lo(cs.b), P2::hi(cs.b)};
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            float erase = 0.f;
#pragma unroll
            for (int r = 0; r < S; ++r) erase = fmaf(ce[r], m[r][c], erase);
            const float u = fmaf(ew[c], v[c], -erase);
#pragma unroll
            for (int r = 0; r < S; ++r) m[r][c] = fmaf(kt[r], u, m[r][c]);
        }
    };
    // Eager chunks: multiply by the decay after a write.
    auto fold = [&](int e, float (&m)[S][CPL]) {
        float dd[S];
        rows8(e, kDecay, dd);
#pragma unroll
        for (int r = 0; r < S; ++r)
#pragma unroll
            for (int c = 0; c < CPL; ++c) m[r][c] *= dd[r];
    };

    float dm[S][CPL];
#pragma unroll
    for (int r = 0; r < S; ++r)
#pragma unroll
        for (int c = 0; c < CPL; ++c) dm[r][c] = 0.f;

    // Adjoint of write e, pre-event state st = diag(s) Mh, dm = diag(sigma) dMh:
    //   du = dMh^T (k sigma); u = x - Mh^T (a decay s)
    //   U = sigma (dMh u); X = decay s (Mh du); P = decay s sigma rowsum(dMh o Mh)
    //   dMh -= (a / sigma) du^T                      (role_bank_kernel.py:128-138)
    auto write_back = [&](int e, int buf, const float (&st)[S][CPL]) {
        float kk[S], ce[S], au[S];
        rows8(e, kKey, kk);
        rows8(e, kErase, ce);
        rows8(e, kUpd, au);
        const ColSlot cs = s_cols[e][lane];
        const float v[CPL] = {P2::lo(cs.a), P2::hi(cs.a)}, ew[CPL] = {P2::lo(cs.b), P2::hi(cs.b)};
        float u[CPL], du[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            float erase = 0.f, acc = 0.f;
#pragma unroll
            for (int r = 0; r < S; ++r) {
                erase = fmaf(ce[r], st[r][c], erase);
                acc = fmaf(dm[r][c], kk[r], acc);
            }
            u[c] = fmaf(ew[c], v[c], -erase);
            du[c] = acc;
        }
        const uint32_t slot = uint32_t(__builtin_amdgcn_readfirstlane(s_meta[buf][e].y));
        if (live) *reinterpret_cast<float2 *>(du_lane + uint64_t(slot) * hw) = make_float2(du[0], du[1]);
        float *wp = wp_tile + uint64_t(slot) * uint32_t(p.heads * 3 * S);
        // rows 0..3, then 4..7: red = U[4], X[4], P[4] of the group
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            float red[12];
#pragma unroll
            for (int i = 0; i < 12; ++i) red[i] = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 4 * g + i;
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    red[i] = fmaf(dm[r][c], u[c], red[i]);
                    red[4 + i] = fmaf(st[r][c], du[c], red[4 + i]);
                    red[8 + i] = fmaf(dm[r][c], st[r][c], red[8 + i]);
                    dm[r][c] = fmaf(-au[r], du[c], dm[r][c]);
                }
            }
            const int pos = lane & 15;
            const int at = 3 * (lane >> 4) + (pos < 3 ? pos : 0);  // kind = at / 4, row 4g + at % 4
            const int kind = at >> 2, r = 4 * g + (at & 3);
            const float o =
                reduce_scatter<12>(red, lane) * reinterpret_cast<const float *>(&s_rows[e][0])[kScale + kind * S + r];
            if (pos < 3) wp[kind * S + r] = o;
        }
    };
    // Adjoint of read e with state st = diag(s) Mh: dq = scale s (Mh dy); dMh += (eq scale / sigma) dy^T.
    auto read_back = [&](int e, int buf, const float (&st)[S][CPL]) {
        float eq[S];
        rows8(e, kKey, eq);
        const ColSlot cs = s_cols[e][lane];
        const float dy[CPL] = {P2::lo(cs.a), P2::hi(cs.a)};
        float red[S];
#pragma unroll
        for (int r = 0; r < S; ++r) {
            red[r] = 0.f;
#pragma unroll
            for (int c = 0; c < CPL; ++c) red[r] = fmaf(st[r][c], dy[c], red[r]);
        }
#pragma unroll
        for (int r = 0; r < S; ++r)
#pragma unroll
            for (int c = 0; c < CPL; ++c) dm[r][c] = fmaf(eq[r], dy[c], dm[r][c]);
        const uint32_t slot = uint32_t(__builtin_amdgcn_readfirstlane(s_meta[buf][e].y));
        const int pos = lane & 15;
        const int at = (S / 4) * (lane >> 4) + (pos < S / 4 ? pos : 0);
        const float o = reduce_scatter<S>(red, lane) * reinterpret_cast<const float *>(&s_rows[e][0])[kScale + at];
        if (pos < S / 4) rp_tile[uint64_t(slot) * uint32_t(p.heads * S) + at] = o;
    };

    if (count > 0) {
        store_meta(count - 1, load_meta(count - 1));
        int4 prev = make_int4(0, 0, 0, 0);
        if (count > 1) prev = load_meta(count - 2);
        __syncthreads();
        Staged sg;
        issue_stage(count - 1, sg);
        if (count > 1) store_meta(count - 2, prev);
        __syncthreads();
        finish_stage(count - 1, sg);
    }

#pragma unroll 1
    for (int c = count - 1; c >= 0; --c) {
        __syncthreads();
        const int buf = c & 1;
        const int len = chunk_len(c);
        const int4 mine = s_meta[buf][lane & (C - 1)];
        const uint32_t wmask = uint32_t(__ballot(lane < len && mine.z == 0)) & 0xffffu;
        const uint32_t rmask = uint32_t(__ballot(lane < len && mine.z != 0)) & 0xffffu;
        const uint32_t fmask = __builtin_amdgcn_readfirstlane(s_eager) ? wmask : 0u;
        float st[HALF][S][CPL];
        if (len > HALF) {
            float m[S][CPL];
            load_m0(m);
#pragma unroll
            for (int e = 0; e < C - 1; ++e) {
                if (e >= HALF) {
#pragma unroll
                    for (int r = 0; r < S; ++r)
#pragma unroll
                        for (int cc = 0; cc < CPL; ++cc) st[e - HALF][r][cc] = m[r][cc];
                }
                if (wmask & (1u << e)) apply(e, m);
                if (fmask & (1u << e)) fold(e, m);
            }
#pragma unroll
            for (int r = 0; r < S; ++r)
#pragma unroll
                for (int cc = 0; cc < CPL; ++cc) st[HALF - 1][r][cc] = m[r][cc];
#pragma unroll
            for (int e = C - 1; e >= HALF; --e) {
                if (wmask & (1u << e)) write_back(e, buf, st[e - HALF]);
                else if (rmask & (1u << e)) read_back(e, buf, st[e - HALF]);
                if (fmask & (1u << e)) fold(e, dm);
            }
        }
        {
            float m[S][CPL];
            load_m0(m);
#pragma unroll
            for (int e = 0; e < HALF; ++e) {
#pragma unroll
                for (int r = 0; r < S; ++r)
#pragma unroll
                    for (int cc = 0; cc < CPL; ++cc) st[e][r][cc] = m[r][cc];
                if (e + 1 < HALF) {
                    if (wmask & (1u << e)) apply(e, m);
                    if (fmask & (1u << e)) fold(e, m);
                }
            }
        }
        // the next chunk's loads, in flight while events 7..0 are differentiated
        int4 meta2 = make_int4(0, 0, 0, 0);
        Staged sg;
        if (c >= 2) meta2 = load_meta(c - 2);
        if (c >= 1) issue_stage(c - 1, sg);
#pragma unroll
        for (int e = HALF - 1; e >= 0; --e) {
            if (wmask & (1u << e)) write_back(e, buf, st[e]);
            else if (rmask & (1u << e)) read_back(e, buf, st[e]);
            if (fmask & (1u << e)) fold(e, dm);
        }
        // the adjoint leaves the chunk in eager form: dm = diag(sigma) dMh
        if (!fmask) {
#pragma unroll
            for (int r = 0; r < S; ++r) {
                const float f = s_fold[r];
#pragma unroll
                for (int cc = 0; cc < CPL; ++cc) dm[r][cc] *= f;
            }
        }
        __syncthreads();
        if (c >= 2) store_meta(c - 2, meta2);
        if (c >= 1) finish_stage(c - 1, sg);
    }
    // adjoint of the segment's initial state (FP32, per sequence)
    if (live) {
        const int64_t off = ((bidx * p.banks + bank) * p.heads + head) * S * p.width + col0;
#pragma unroll
        for (int r = 0; r < S; ++r)
            *reinterpret_cast<float2 *>(p.dinit + off + int64_t(r) * p.width) = make_float2(dm[r][0], dm[r][1]);
    }
}


template <typename T>
struct VjpParams {
    const T *q, *k, *b;
    const float *g;
    const T *v, *w;
    const T *ww, *rw;
    const float *du, *wpart, *rpart;
    T *dq, *dk, *db, *dv, *dw, *dww, *drw;
    float *dg;
    int64_t nt;
    int heads, s_real, width, kw, kr, tiles;
    int wph;  // token_grad_kernel: waves per head (each owns 64 * CPL value columns)
    int routed_decay;
};

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int m = kLanes / 2; m >= 1; m >>= 1) x += __shfl_xor(x, m, kLanes);
    return x;
}

// Sum over the 8 lanes of an 8-lane group (lane % 8 varies), in every lane.
__device__ __forceinline__ float group8_sum(float x) {
    x += __shfl_xor(x, 1, kLanes);
    x += __shfl_xor(x, 2, kLanes);
    return x + __shfl_xor(x, 4, kLanes);
}

// Sum over the 8 lanes of equal lane % 8 (lane / 8 varies), in every lane.
__device__ __forceinline__ float stride8_sum(float x) {
    x += __shfl_xor(x, 8, kLanes);
    x += __shfl_xor(x, 16, kLanes);
    return x + __shfl_xor(x, 32, kLanes);
}

// One workgroup per token, one wave per head (heads <= 16); S <= 8, KW, KR
// <= 8 and width <= 64 * CPL.  Lane (j, r) = (lane / 8, lane % 8) holds the
// S-side gradients of route slot j, row r; lane l owns value columns
// l*CPL .. l*CPL + CPL - 1.  The rounding points follow
// role_bank_dispatch.py:99-131; sums over slots and rows are in FP32.
template <typename T, int CPL>
__global__ __launch_bounds__(1024) void token_grad_kernel(VjpParams<T> p) {
    constexpr int MAXH = 16, MAXK = 8, MAXW = 16;
    __shared__ float s_route[MAXH][2 * MAXK];  // per head: d(ww) of each write slot, then d(rw)
    __shared__ float s_wv[MAXW][MAXK];         // per wave: its columns' part of d(ww)
    const int64_t token = blockIdx.x;
    const int wave = threadIdx.x / kLanes, lane = threadIdx.x % kLanes;
    // a head's columns are split over p.wph waves; every wave of a head
    // computes the head's S-side terms, its first wave stores them
    const int head = wave / p.wph, hw = wave % p.wph;
    const int64_t row = token * p.heads + head;
    const int64_t wslots = p.nt * p.kw, rslots = p.nt * p.kr;
    const int j = lane >> 3, r = lane & 7;
    const bool srow = r < p.s_real;
    const bool wl = srow && j < p.kw, rl = srow && j < p.kr;
    const int64_t wslot = token * p.kw + (j < p.kw ? j : p.kw - 1);
    const int64_t rslot = token * p.kr + (j < p.kr ? j : p.kr - 1);
    const int rr = srow ? r : 0;

    // ---- every load first: the S side (slot j, row r), then the value columns
    const float q0 = to_f32(p.q[row * p.s_real + rr]);
    const float k0 = to_f32(p.k[row * p.s_real + rr]);
    const float b0 = to_f32(p.b[row * p.s_real + rr]);
    const float g0 = p.g[row * p.s_real + rr];
    const float pw = to_f32(p.ww[wslot]), pr = to_f32(p.rw[rslot]);
    const float *wp0 = p.wpart + (wslot * p.heads + head) * 3 * p.s_real + rr;
    float su = wp0[0], sx = wp0[p.s_real], sp = wp0[2 * p.s_real];
    float sq = p.rpart[(rslot * p.heads + head) * p.s_real + rr];
    const int c0 = (hw * kLanes + lane) * CPL;
    bool live[CPL];
    float v0[CPL], w0[CPL], vwsum[CPL], wsum[CPL], wv[MAXK];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        live[c] = c0 + c < p.width;
        const int cc = min(c0 + c, p.width - 1);
        const float vx = to_f32(p.v[row * p.width + cc]), wx = to_f32(p.w[row * p.width + cc]);
        v0[c] = live[c] ? vx : 0.f;
        w0[c] = live[c] ? wx : 0.f;
        vwsum[c] = wsum[c] = 0.f;
    }
    // every slot's du and weight requested up front (slots >= KW re-read slot
    // KW-1: straight-line loads, all in flight together)
    float dus[MAXK][CPL], pws[MAXK];
    int cols[CPL];  // clamped columns: lanes past the width re-read the last one and drop it
#pragma unroll
    for (int c = 0; c < CPL; ++c) cols[c] = min(c0 + c, p.width - 1);
#pragma unroll
    for (int jj = 0; jj < MAXK; ++jj) {
        const int64_t slot = token * p.kw + (jj < p.kw ? jj : p.kw - 1);
        pws[jj] = to_f32(p.ww[slot]);
        const float *du = p.du + (slot * p.heads + head) * p.width;
#pragma unroll
        for (int c = 0; c < CPL; ++c) dus[jj][c] = du[cols[c]];
    }
    for (int t = 1; t < p.tiles; ++t) {  // column tiles past the first
        const float *wp = p.wpart + ((int64_t(t) * wslots + wslot) * p.heads + head) * 3 * p.s_real + rr;
        su += wp[0];
        sx += wp[p.s_real];
        sp += wp[2 * p.s_real];
        sq += p.rpart[((int64_t(t) * rslots + rslot) * p.heads + head) * p.s_real + rr];
    }
    // dk = U - eb X ; db = -k X ; dg = P - a X (role_bank_kernel.py:128-135)
    const float eb = round_to<T>(b0 * pw);
    const float dk = round_to<T>(su - eb * sx);
    const float db = round_to<T>(-k0 * sx);
    const float dg = sp - eb * k0 * sx;
    // routed decay: the packed gate was g*p (routed_update.py:43-47)
    const float k_term = wl ? dk : 0.f;
    const float g_term = wl ? (p.routed_decay ? dg * pw : dg) : 0.f;
    const float b_term = wl ? round_to<T>(db * pw) : 0.f;
    const float wb = round_to<T>(group8_sum(wl ? round_to<T>(db * b0) : 0.f));
    const float dec = group8_sum(wl ? dg * g0 : 0.f);
    const float dq = round_to<T>(sq);
    const float q_term = rl ? round_to<T>(dq * pr) : 0.f;
    const float wr = round_to<T>(group8_sum(rl ? round_to<T>(dq * q0) : 0.f));
    const float kwsum = stride8_sum(k_term), gsum = stride8_sum(g_term), bsum = stride8_sum(b_term);
    const float qsum = stride8_sum(q_term);
    if (hw == 0 && j == 0 && srow) {
        const int64_t at = row * p.s_real + r;
        p.dq[at] = from_f32<T>(qsum);
        p.dk[at] = from_f32<T>(kwsum);
        p.dg[at] = gsum;
        p.db[at] = from_f32<T>(bsum);
    }

    // ---- value columns: the token's write events in route order
#pragma unroll
    for (int jj = 0; jj < MAXK; ++jj) {
        wv[jj] = 0.f;
        if (jj < p.kw) {
            const float pj = pws[jj];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const float d = live[c] ? dus[jj][c] : 0.f;
                const float ew = round_to<T>(w0[c] * pj);
                const float dv = round_to<T>(d * ew);
                const float dw = round_to<T>(d * v0[c]);
                vwsum[c] = round_to<T>(vwsum[c] + dv);
                wsum[c] = round_to<T>(wsum[c] + round_to<T>(dw * pj));
                wv[jj] += round_to<T>(dw * w0[c]);
            }
        }
    }
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        if (live[c]) {
            p.dv[row * p.width + c0 + c] = from_f32<T>(vwsum[c]);
            p.dw[row * p.width + c0 + c] = from_f32<T>(wsum[c]);
        }
    }
    const float wv_total = reduce_scatter<MAXK>(wv, lane);
    if ((lane & 15) < MAXK / 4) s_wv[wave][(MAXK / 4) * (lane >> 4) + (lane & 15)] = wv_total;
    __syncthreads();
    if (hw == 0 && r == 0) {
        if (j < p.kw) {
            float cols = 0.f;  // the head's waves in column order
            for (int w = 0; w < p.wph; ++w) cols += s_wv[wave + w][j];
            float dww = round_to<T>(wb + round_to<T>(cols));
            if (p.routed_decay) dww = round_to<T>(dww + dec);
            s_route[head][j] = dww;
        }
        if (j < p.kr) s_route[head][MAXK + j] = wr;
    }
    __syncthreads();
    // route-weight gradients: the heads' contributions added in head order
    if (threadIdx.x < unsigned(p.kw + p.kr)) {
        const int jj = threadIdx.x;
        const bool wr_ = jj < p.kw;
        const int col = wr_ ? jj : MAXK + jj - p.kw;
        float total = 0.f;
        for (int h = 0; h < p.heads; ++h) total += s_route[h][col];
        if (wr_) p.dww[token * p.kw + jj] = from_f32<T>(total);
        else p.drw[token * p.kr + (jj - p.kw)] = from_f32<T>(total);
    }
}


// One workgroup (4 waves) per token.  VPL = value columns per lane.
template <typename T, int VPL>
__global__ __launch_bounds__(256) void token_vjp_kernel(VjpParams<T> p) {
    extern __shared__ float s_route[];  // [H][KW] d(ww) then [H][KR] d(rw), per head
    const int64_t token = blockIdx.x;
    const int wave = threadIdx.x / kLanes, lane = threadIdx.x % kLanes;
    const int nwaves = blockDim.x / kLanes;
    const int64_t wslots = p.nt * p.kw, rslots = p.nt * p.kr;
    const int64_t hs = int64_t(p.heads) * p.s_real;
    for (int head = wave; head < p.heads; head += nwaves) {
        const int64_t row = token * p.heads + head;
        const bool srow = lane < p.s_real;
        const float q0 = srow ? to_f32(p.q[row * p.s_real + lane]) : 0.f;
        const float k0 = srow ? to_f32(p.k[row * p.s_real + lane]) : 0.f;
        const float b0 = srow ? to_f32(p.b[row * p.s_real + lane]) : 0.f;
        const float g0 = srow ? p.g[row * p.s_real + lane] : 0.f;
        float v0[VPL], w0[VPL], vwsum[VPL], wsum[VPL];
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int c = lane + i * kLanes;
            v0[i] = c < p.width ? to_f32(p.v[row * p.width + c]) : 0.f;
            w0[i] = c < p.width ? to_f32(p.w[row * p.width + c]) : 0.f;
            vwsum[i] = wsum[i] = 0.f;
        }
        float kwsum = 0.f, gsum = 0.f, bsum = 0.f, qsum = 0.f;
        // write events in route order (role_bank_dispatch.py:99-115)
        for (int j = 0; j < p.kw; ++j) {
            const int64_t slot = token * p.kw + j;
            const float pw = to_f32(p.ww[slot]);
            float wb_part = 0.f, dec_part = 0.f;
            if (srow) {
                float su = 0.f, sx = 0.f, sp = 0.f;
                for (int t = 0; t < p.tiles; ++t) {
                    const float *wp = p.wpart + ((int64_t(t) * wslots + slot) * p.heads + head) * 3 * p.s_real;
                    su += wp[lane];
                    sx += wp[p.s_real + lane];
                    sp += wp[2 * p.s_real + lane];
                }
                // dk = U - eb X ; db = -k X ; dg = P - a X (role_bank_kernel.py:128-135)
                const float eb = round_to<T>(b0 * pw);
                const float dk = round_to<T>(su - eb * sx);
                const float db = round_to<T>(-k0 * sx);
                const float dg = sp - eb * k0 * sx;
                kwsum += dk;
                // routed decay: the packed gate was g*p (routed_update.py:43-47)
                gsum += p.routed_decay ? dg * pw : dg;
                dec_part = dg * g0;
                bsum += round_to<T>(db * pw);
                wb_part = round_to<T>(db * b0);
            }
            float wv_part = 0.f;
            const float *du = p.du + (slot * p.heads + head) * p.width;
#pragma unroll
            for (int i = 0; i < VPL; ++i) {
                const int c = lane + i * kLanes;
                if (c < p.width) {
                    const float ew = round_to<T>(w0[i] * pw);
                    const float dv = round_to<T>(du[c] * ew);
                    const float dw = round_to<T>(du[c] * v0[i]);
                    vwsum[i] = round_to<T>(vwsum[i] + dv);
                    wsum[i] = round_to<T>(wsum[i] + round_to<T>(dw * pw));
                    wv_part += round_to<T>(dw * w0[i]);
                }
            }
            const float wb = round_to<T>(wave_sum(wb_part));
            const float wv = round_to<T>(wave_sum(wv_part));
            float dww = round_to<T>(wb + wv);
            if (p.routed_decay) dww = round_to<T>(dww + wave_sum(dec_part));
            if (lane == 0) s_route[head * p.kw + j] = dww;
        }
        // read events in route order (:116-125)
        for (int j = 0; j < p.kr; ++j) {
            const int64_t slot = token * p.kr + j;
            const float pr = to_f32(p.rw[slot]);
            float wr_part = 0.f;
            if (srow) {
                float dq = 0.f;
                for (int t = 0; t < p.tiles; ++t) dq += p.rpart[(int64_t(t) * rslots + slot) * hs + head * p.s_real + lane];
                dq = round_to<T>(dq);
                qsum += round_to<T>(dq * pr);
                wr_part = round_to<T>(dq * q0);
            }
            const float wr = round_to<T>(wave_sum(wr_part));
            if (lane == 0) s_route[p.heads * p.kw + head * p.kr + j] = wr;
        }
        if (srow) {
            const int64_t at = row * p.s_real + lane;
            p.dq[at] = from_f32<T>(qsum);
            p.dk[at] = from_f32<T>(kwsum);
            p.dg[at] = gsum;
            p.db[at] = from_f32<T>(bsum);
        }
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int c = lane + i * kLanes;
            if (c < p.width) {
                p.dv[row * p.width + c] = from_f32<T>(vwsum[i]);
                p.dw[row * p.width + c] = from_f32<T>(wsum[i]);
            }
        }
    }
    __syncthreads();
    // route-weight gradients: the heads' contributions added in head order
    for (int j = threadIdx.x; j < p.kw + p.kr; j += blockDim.x) {
        float total = 0.f;
        if (j < p.kw) {
            for (int h = 0; h < p.heads; ++h) total += s_route[h * p.kw + j];
            p.dww[token * p.kw + j] = from_f32<T>(total);
        } else {
            const int jr = j - p.kw;
            for (int h = 0; h < p.heads; ++h) total += s_route[p.heads * p.kw + h * p.kr + jr];
            p.drw[token * p.kr + jr] = from_f32<T>(total);
        }
    }
}

struct Workspace {
    float *du, *wpart, *rpart;
    int4 *meta;  // per-event meta of the S = 8 chunk kernel (null otherwise)
    int *seg_order;  // the chunk kernel's segment order (null: bank order)
    size_t bytes;
};

constexpr size_t align256(size_t x) { return (x + 255) / 256 * 256; }

int column_lanes_per_tile(int bank_size) { return bank_size <= 8 ? 2 : 1; }

int replay_interval(const bdm_backward_args &a) {
    return a.round_interval > 0 ? a.round_interval : a.snapshot_interval;
}

// The S = 8, interval-16 chunk kernel: even head width (column pairs) and
// token and route indices in 32 bits.
bool chunk_path(const bdm_backward_args &a) {
    const int64_t nt = a.batch * a.time;
    const int64_t k = a.write_banks > a.read_banks ? a.write_banks : a.read_banks;
    return a.bank_size == 8 && replay_interval(a) == 16 && a.head_width % 2 == 0 && a.write_banks >= 1 &&
           a.read_banks >= 1 && nt * k < INT32_MAX;
}

// The per-token gradient kernel: one wave per head and one lane per (slot, row).
// A head wider than 256 columns takes ceil(width / 256) waves (4 columns per
// lane); the workgroup holds at most 16 waves.
int token_grad_waves(const bdm_backward_args &a) {
    return a.head_width <= 256 ? 1 : (a.head_width + 255) / 256;
}

bool token_grad_path(const bdm_backward_args &a) {
    return a.bank_size <= 8 && a.write_banks >= 1 && a.write_banks <= 8 && a.read_banks >= 1 && a.read_banks <= 8 &&
           a.heads * token_grad_waves(a) <= 16;
}

Workspace carve(const bdm_backward_args &a, void *base) {
    const size_t nt = size_t(a.batch) * size_t(a.time);
    const size_t hs = size_t(a.heads) * size_t(a.bank_size);
    const int cpl = column_lanes_per_tile(a.bank_size);
    const size_t tiles = (size_t(a.head_width) + kLanes * cpl - 1) / (kLanes * cpl);
    const size_t du = align256(nt * a.write_banks * a.heads * size_t(a.head_width) * sizeof(float));
    const size_t wp = align256(tiles * 3 * nt * a.write_banks * hs * sizeof(float));
    const size_t rp = align256(tiles * nt * a.read_banks * hs * sizeof(float));
    const size_t mt = chunk_path(a) ? align256(nt * size_t(a.write_banks + a.read_banks) * sizeof(int4)) : 0;
    const int64_t nseg = int64_t(a.batch) * a.bank_count;
    const size_t so = chunk_path(a) && order_geometry(nseg) ? align256(size_t(nseg) * sizeof(int)) : 0;
    char *c = static_cast<char *>(base);
    Workspace w{};
    w.du = reinterpret_cast<float *>(c);
    w.wpart = reinterpret_cast<float *>(c ? c + du : nullptr);
    w.rpart = reinterpret_cast<float *>(c ? c + du + wp : nullptr);
    w.meta = reinterpret_cast<int4 *>(c && mt ? c + du + wp + rp : nullptr);
    w.seg_order = reinterpret_cast<int *>(c && so && order_enabled() ? c + du + wp + rp + mt : nullptr);
    w.bytes = du + wp + rp + mt + so;
    return w;
}

template <typename T, int S, int CPL, int C>
int launch_backward(const bdm_backward_args &a, const Workspace &ws, hipStream_t stream) {
    BackwardParams<T> p{};
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
    p.snap = a.snapshots;
    p.dy = static_cast<const T *>(a.grad_output);
    p.du = ws.du;
    p.wpart = ws.wpart;
    p.rpart = ws.rpart;
    p.dinit = a.grad_initial;
    p.init_bstride = a.initial_batch_stride;
    p.nt = a.batch * a.time;
    p.heads = a.heads;
    p.s_real = a.bank_size;
    p.width = a.head_width;
    p.banks = a.bank_count;
    p.kw = a.write_banks;
    p.kr = a.read_banks;
    p.tiles = (a.head_width + kLanes * CPL - 1) / (kLanes * CPL);
    p.init_dtype = a.initial_dtype;
    p.snap_dtype = a.snapshot_dtype;
    p.routed_decay = a.routed_decay;
    p.rounding = a.round_interval > 0;
    p.scale = a.scale;
    const int64_t nseg = a.batch * a.bank_count;
    p.xcd_remap = (nseg % 8 == 0) ? 1 : 0;
    const dim3 grid(unsigned(nseg), unsigned(a.heads), unsigned(p.tiles));
    if constexpr (S == 8 && C == 16) {
        if (chunk_path(a)) {
            const int64_t events = p.nt * (p.kw + p.kr);
            const unsigned blocks = unsigned((events + 255) / 256);
            event_meta_kernel<T><<<blocks, 256, 0, stream>>>(p.order, events, p.nt * p.kw, p.kw, p.kr, p.ww, p.rw,
                                                            ws.meta);
            if (int rc = check_launch("event_meta_kernel")) return rc;
            p.meta = ws.meta;
            if (ws.seg_order) {
                launch_segment_order(p.cu, nseg, ws.seg_order, stream);
                if (int rc = check_launch("segment_order_kernel")) return rc;
                p.seg_order = ws.seg_order;
                const void *kernel = a.snapshot_dtype == BDM_BF16
                                         ? reinterpret_cast<const void *>(&chunk_backward_kernel<T, bf16_t>)
                                         : reinterpret_cast<const void *>(&chunk_backward_kernel<T, float>);
                p.order_gpr = order_groups_per_round(kernel, kLanes, nseg, int(grid.y * grid.z));
            }
            if (a.snapshot_dtype == BDM_BF16)
                chunk_backward_kernel<T, bf16_t><<<grid, kLanes, 0, stream>>>(p);
            else
                chunk_backward_kernel<T, float><<<grid, kLanes, 0, stream>>>(p);
            if (int rc = check_launch("chunk_backward_kernel")) return rc;
        } else {
            routed_backward_kernel<T, S, CPL, C><<<grid, kLanes, 0, stream>>>(p);
            if (int rc = check_launch("routed_backward_kernel")) return rc;
        }
    } else {
        routed_backward_kernel<T, S, CPL, C><<<grid, kLanes, 0, stream>>>(p);
        if (int rc = check_launch("routed_backward_kernel")) return rc;
    }

    VjpParams<T> v{};
    v.q = p.q;
    v.k = p.k;
    v.b = p.b;
    v.g = p.g;
    v.v = p.v;
    v.w = p.w;
    v.ww = p.ww;
    v.rw = p.rw;
    v.du = ws.du;
    v.wpart = ws.wpart;
    v.rpart = ws.rpart;
    v.dq = static_cast<T *>(a.grad_q);
    v.dk = static_cast<T *>(a.grad_k);
    v.db = static_cast<T *>(a.grad_b);
    v.dv = static_cast<T *>(a.grad_v);
    v.dw = static_cast<T *>(a.grad_w);
    v.dww = static_cast<T *>(a.grad_write_weights);
    v.drw = static_cast<T *>(a.grad_read_weights);
    v.dg = a.grad_g;
    v.nt = p.nt;
    v.heads = a.heads;
    v.s_real = a.bank_size;
    v.width = a.head_width;
    v.kw = a.write_banks;
    v.kr = a.read_banks;
    v.tiles = p.tiles;
    v.routed_decay = a.routed_decay;
    v.wph = token_grad_waves(a);
    const unsigned blocks = unsigned(p.nt);
    if (token_grad_path(a)) {
        const unsigned threads = unsigned(a.heads * v.wph) * kLanes;
        if (v.wph > 1)
            token_grad_kernel<T, 4><<<blocks, threads, 0, stream>>>(v);
        else if (a.head_width <= kLanes)
            token_grad_kernel<T, 1><<<blocks, threads, 0, stream>>>(v);
        else if (a.head_width <= 2 * kLanes)
            token_grad_kernel<T, 2><<<blocks, threads, 0, stream>>>(v);
        else
            token_grad_kernel<T, 4><<<blocks, threads, 0, stream>>>(v);
        return check_launch("token_grad_kernel");
    }
    const size_t lds = size_t(a.heads) * size_t(a.write_banks + a.read_banks) * sizeof(float);
    if (a.head_width <= kLanes)
        token_vjp_kernel<T, 1><<<blocks, 256, lds, stream>>>(v);
    else if (a.head_width <= 2 * kLanes)
        token_vjp_kernel<T, 2><<<blocks, 256, lds, stream>>>(v);
    else if (a.head_width <= 4 * kLanes)
        token_vjp_kernel<T, 4><<<blocks, 256, lds, stream>>>(v);
    else if (a.head_width <= 8 * kLanes)
        token_vjp_kernel<T, 8><<<blocks, 256, lds, stream>>>(v);
    else if (a.head_width <= 16 * kLanes)
        token_vjp_kernel<T, 16><<<blocks, 256, lds, stream>>>(v);
    else
        token_vjp_kernel<T, 32><<<blocks, 256, lds, stream>>>(v);
    return check_launch("token_vjp_kernel");
}

template <typename T>
int dispatch_backward(const bdm_backward_args &a, const Workspace &ws, hipStream_t stream) {
    const int c = a.round_interval > 0 ? a.round_interval : a.snapshot_interval;
    if (a.bank_size <= 8) {
        if (c == 16) return launch_backward<T, 8, 2, 16>(a, ws, stream);
        if (c == 8) return launch_backward<T, 8, 2, 8>(a, ws, stream);
        if (c == 4) return launch_backward<T, 8, 2, 4>(a, ws, stream);
    } else if (a.bank_size <= 16) {
        if (c == 8) return launch_backward<T, 16, 1, 8>(a, ws, stream);
        if (c == 4) return launch_backward<T, 16, 1, 4>(a, ws, stream);
    } else if (a.bank_size <= 32) {
        if (c == 4) return launch_backward<T, 32, 1, 4>(a, ws, stream);
    }
    return fail(BDM_ERR_UNSUPPORTED, "backward: bank_size %d with replay interval %d", a.bank_size, c);
}

}  // namespace
}  // namespace bdm

extern "C" size_t bdm_backward_workspace_size(const bdm_backward_args *a) {
    if (!a || a->batch <= 0 || a->time <= 0 || a->heads <= 0 || a->head_width <= 0 || a->bank_size <= 0 ||
        a->write_banks < 0 || a->read_banks < 0)
        return 0;
    return bdm::carve(*a, nullptr).bytes;
}

extern "C" int bdm_backward(const bdm_backward_args *a, void *workspace, size_t workspace_bytes, void *stream) {
    using namespace bdm;
    if (!a) return fail(BDM_ERR_INVALID, "backward: null args");
    if (a->batch <= 0 || a->time <= 0 || a->heads <= 0 || a->bank_size <= 0 || a->head_width <= 0 ||
        a->bank_count <= 0 || a->write_banks < 0 || a->read_banks < 0 || a->write_banks + a->read_banks == 0)
        return fail(BDM_ERR_INVALID, "backward: bad geometry");
    if (a->head_width > 32 * kLanes) return fail(BDM_ERR_UNSUPPORTED, "backward: head_width %d > 2048", a->head_width);
    if (a->ctrl_dtype != BDM_BF16 && a->ctrl_dtype != BDM_F32)
        return fail(BDM_ERR_INVALID, "backward: ctrl dtype %d", a->ctrl_dtype);
    if ((a->initial_dtype != BDM_BF16 && a->initial_dtype != BDM_F32) ||
        (a->snapshot_dtype != BDM_BF16 && a->snapshot_dtype != BDM_F32))
        return fail(BDM_ERR_INVALID, "backward: state dtype");
    if (a->round_interval > 0 && a->snapshot_interval != a->round_interval)
        return fail(BDM_ERR_INVALID, "backward: snapshot interval must equal the rounding interval");
    if (a->round_interval == 0 && a->snapshot_dtype != BDM_F32)
        return fail(BDM_ERR_INVALID, "backward: an unrounded state needs FP32 snapshots");
    if (a->batch * a->bank_count > int64_t(INT32_MAX) || a->heads > 65535 ||
        a->batch * a->time > int64_t(INT32_MAX))
        return fail(BDM_ERR_UNSUPPORTED, "backward: grid too large");
    if (!a->q || !a->k || !a->g || !a->b || !a->v || !a->w || !a->write_weights || !a->read_weights ||
        !a->order || !a->cu_seqlens || !a->initial || !a->snapshots || !a->grad_output || !a->grad_q ||
        !a->grad_k || !a->grad_g || !a->grad_b || !a->grad_v || !a->grad_w || !a->grad_write_weights ||
        !a->grad_read_weights || !a->grad_initial)
        return fail(BDM_ERR_INVALID, "backward: null pointer");
    const Workspace need = carve(*a, nullptr);
    if (!workspace || workspace_bytes < need.bytes)
        return fail(BDM_ERR_WORKSPACE, "backward: workspace %zu < %zu bytes", workspace_bytes, need.bytes);
    if (!aligned(workspace, 256)) return fail(BDM_ERR_INVALID, "backward: workspace must be 256-byte aligned");
    const Workspace ws = carve(*a, workspace);
    hipStream_t s = as_stream(stream);
    if (a->ctrl_dtype == BDM_BF16) return dispatch_backward<bf16_t>(*a, ws, s);
    return dispatch_backward<float>(*a, ws, s);
}

// Backward of the routed GDN2 bank recurrence and the token-level VJP.
//
// Reference: _role_backward (role_bank_kernel.py:76-150, launched by
// backward() at :205-228), RoutedUpdate.backward (routed_update.py:31-49:
// the decay term of d(ww) and dg scaled by p) and _vjp
// (role_bank_dispatch.py:76-132, with its BF16 rounding points).
//
// routed_backward_kernel: one wave per (segment, head, column tile).  A lane
// owns CPL value columns and all S rows of them, as in the forward.  Chunks
// of C events (the snapshot interval) are visited in reverse.  A chunk's
// states are rebuilt exactly from its snapshot (or the initial state) by the
// forward's own write update: for each SUB-event piece, in reverse, the
// chunk's writes before the piece are replayed from the chunk's start state
// and the piece's pre-event states are kept in registers, so the reverse pass
// reads every pre-event state from registers (about 2.5x the forward's
// writes for C = 16, no LDS or HBM history).  Per event the adjoint dM (S x CPL per lane) is
// updated in-lane; the reductions over value columns that produce the
// event's S-wide gradients (dk, db, dg for a write, dq for a read) do not feed
// back into dM, so they are reduced across the wave and stored per event.
// The write's du (one value per column) is stored in FP32; the token kernel
// forms dv = bf(du*ew) and dw = bf(du*v) from it exactly as the reference's
// stored BF16 products.
//
// token_vjp_kernel: one workgroup per token; each wave handles heads
// wave, wave+4, ...  It folds a token's KW write events and KR read events
// in route order with the reference's rounding (role_bank_dispatch.py:99-131)
// and produces the token gradients of q,k,v,g,b,w and of both route weights.
// Heads' route-weight gradients are added in head order in FP32.
#include "bdm_common.h"
#include "recurrence_ops.h"

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
    float *wpart;   // [tiles, 3, NT*KW, H, S]: dk, db, dg of each write slot
    float *rpart;   // [tiles, NT*KR, H, S]: dq of each read slot
    float *dinit;   // [batch, J, H, S, v]
    int64_t init_bstride, nt;
    int heads, s_real, width, banks, kw, kr, tiles;
    int init_dtype, snap_dtype, routed_decay, rounding;
    int xcd_remap;
    float scale;
};

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

    const int nseg = gridDim.x;
    const int seg = p.xcd_remap ? int((blockIdx.x % 8) * (nseg / 8) + blockIdx.x / 8) : int(blockIdx.x);
    const int bank = seg % p.banks;
    const int64_t bidx = seg / p.banks;
    const int head = blockIdx.y;
    const int tile = blockIdx.z;
    const int lane = threadIdx.x;
    const int col0 = (tile * kLanes + lane) * CPL;
    const int64_t start = p.cu[seg], end = p.cu[seg + 1];
    const int64_t write_events = p.nt * p.kw;
    const int64_t events = p.nt * (p.kw + p.kr);
    const int64_t hs = int64_t(p.heads) * p.s_real;

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
                    // dk = sum(dh*u) - eb*X ; db = -k*X ; dg = sum(dh*hd) - a*X
                    // (role_bank_kernel.py:128-135, X = the contraction hd.du)
                    float out_k = 0.f, out_b = 0.f, out_g = 0.f;
#pragma unroll
                    for (int r = 0; r < S; ++r) {
                        if (lane == r) {
                            const float x = red[S + r];
                            out_k = red[r] - ev.rows.eb[r] * x;
                            out_b = -ev.rows.key[r] * x;
                            out_g = red[2 * S + r] - ev.rows.a[r] * x;
                        }
                    }
                    if (lane < p.s_real) {
                        const int64_t nslots = p.nt * p.kw;
                        const int64_t at = (slot * p.heads + head) * p.s_real + lane;
                        const int64_t plane = nslots * hs;
                        float *wp = p.wpart + int64_t(tile) * 3 * plane;
                        wp[at] = out_k;
                        wp[plane + at] = out_b;
                        wp[2 * plane + at] = out_g;
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


template <typename T>
struct VjpParams {
    const T *q, *b;
    const float *g;
    const T *v, *w;
    const T *ww, *rw;
    const float *du, *wpart, *rpart;
    T *dq, *dk, *db, *dv, *dw, *dww, *drw;
    float *dg;
    int64_t nt;
    int heads, s_real, width, kw, kr, tiles;
    int routed_decay;
};

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int m = kLanes / 2; m >= 1; m >>= 1) x += __shfl_xor(x, m, kLanes);
    return x;
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
                const int64_t at = (slot * p.heads + head) * p.s_real + lane;
                float dk = 0.f, db = 0.f, dg = 0.f;
                for (int t = 0; t < p.tiles; ++t) {
                    const float *wp = p.wpart + int64_t(t) * 3 * wslots * hs;
                    dk += wp[at];
                    db += wp[wslots * hs + at];
                    dg += wp[2 * wslots * hs + at];
                }
                dk = round_to<T>(dk);
                db = round_to<T>(db);
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
    size_t bytes;
};

constexpr size_t align256(size_t x) { return (x + 255) / 256 * 256; }

int column_lanes_per_tile(int bank_size) { return bank_size <= 8 ? 2 : 1; }

Workspace carve(const bdm_backward_args &a, void *base) {
    const size_t nt = size_t(a.batch) * size_t(a.time);
    const size_t hs = size_t(a.heads) * size_t(a.bank_size);
    const int cpl = column_lanes_per_tile(a.bank_size);
    const size_t tiles = (size_t(a.head_width) + kLanes * cpl - 1) / (kLanes * cpl);
    const size_t du = align256(nt * a.write_banks * a.heads * size_t(a.head_width) * sizeof(float));
    const size_t wp = align256(tiles * 3 * nt * a.write_banks * hs * sizeof(float));
    const size_t rp = align256(tiles * nt * a.read_banks * hs * sizeof(float));
    char *c = static_cast<char *>(base);
    Workspace w{};
    w.du = reinterpret_cast<float *>(c);
    w.wpart = reinterpret_cast<float *>(c ? c + du : nullptr);
    w.rpart = reinterpret_cast<float *>(c ? c + du + wp : nullptr);
    w.bytes = du + wp + rp;
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
    routed_backward_kernel<T, S, CPL, C><<<grid, kLanes, 0, stream>>>(p);
    if (int rc = check_launch("routed_backward_kernel")) return rc;

    VjpParams<T> v{};
    v.q = p.q;
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
    const size_t lds = size_t(a.heads) * size_t(a.write_banks + a.read_banks) * sizeof(float);
    const unsigned blocks = unsigned(p.nt);
    if (a.head_width <= kLanes)
        token_vjp_kernel<T, 1><<<blocks, 256, lds, stream>>>(v);
    else if (a.head_width <= 2 * kLanes)
        token_vjp_kernel<T, 2><<<blocks, 256, lds, stream>>>(v);
    else
        token_vjp_kernel<T, 4><<<blocks, 256, lds, stream>>>(v);
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
    if (a->head_width > 4 * kLanes) return fail(BDM_ERR_UNSUPPORTED, "backward: head_width %d > 256", a->head_width);
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

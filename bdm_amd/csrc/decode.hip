// Single-token decode against resident bank states.
//
// Reference: inference.step (implementation/bdm/inference.py:161-194) and its
// kernels _decode_write (:21-34), _decode_read (:37-50), _decode_sum (:53-67);
// the reference supports one head with eight rows only (:88-104), this kernel
// any head count and bank size <= 32.
//
// One workgroup per (sequence, head, column span).  Value columns are
// independent in both the write rule and the read, so a wide head is split
// into spans that keep a workgroup within 512 lanes and 64 KiB of LDS.  Lane
// group j (span / CPL lanes) owns write slot j and read slot j.  A step makes two dependent trips to HBM:
// first the bank indices and controller rows (all independent of a bank id,
// issued together, with no barrier behind them), then every bank state the
// step touches — the write banks and the read banks that are not also
// written — requested at once.  Writes are applied and stored (rounded
// to the state dtype), and also kept in LDS, so a read of a bank written by the
// same token sees the stored value without another trip to HBM.  The reads are
// then combined in increasing bank id with a rounding after every add.
#include <type_traits>

#include "bdm_common.h"
#include "epilogue_ops.h"
#include "recurrence_ops.h"
#include "router_ops.h"

namespace bdm {
namespace {

constexpr int kMaxSlots = 16;

// One token's S-element controller row: whole 16-byte vectors when the row is
// full width and aligned, else element by element (rows >= s_real are 0).
template <int S, bool VEC, typename E>
__device__ __forceinline__ void load_ctrl_row(const E *p, int s_real, float (&out)[S]) {
    if constexpr (VEC) {
        load_row<S>(p, out);  // the launcher checked s_real == S and the alignment
    } else {
#pragma unroll
        for (int r = 0; r < S; ++r) out[r] = r < s_real ? to_f32(p[r]) : 0.f;
    }
}

template <typename T>
struct DecodeParams {
    const T *q, *k, *b;
    const float *g;
    const T *v, *w;
    const T *ww, *rw;
    const int64_t *wi, *ri;
    void *state;
    T *out;
    int heads, s_real, width, banks, kw, kr;
    int span, spans;  // columns per workgroup and workgroups per (sequence, head)
    int lanes_per_slot;
    int vec_rows;  // q, k, b, g rows of S elements can be read as 16-byte vectors
    int state_dtype, routed_decay;
    float scale;
    // fused step (bdm_decode_fused): the controllers and routes come from the
    // projection row proj[seq] (column offsets below) and the f_proj output
    const T *proj, *f;
    const void *a_log, *dt_bias;
    int64_t proj_stride, f_stride;
    int q_col, k_col, v_col, b_col, w_col, read_col, write_col;
    int j1, j2, param_dtype, qk_norm;
    // f formed in the launch (f_weight set): f_proj's second factor [H*S, f_width]
    const T *f_weight;
    T *f_out;
    int f_col, f_width;
};

// SE: the state element type (bf16_t or float, the state_dtype argument);
// KMAX >= the selected banks per role, KFIX: exactly KMAX banks in both roles.
// FUSED: the step starts from the projection outputs (bdm_decode_fused):
// waves 0 and 1 route the write and read scores of the sequence (the wave
// router of router_ops.h), lanes 0..3 of wave 2 form the head's q, k, b, g
// rows and every lane its own v, w columns (the controller epilogue's
// helpers of epilogue_ops.h), so the inputs equal those the separate kernels
// would have stored, bit for bit.
template <typename T, typename SE, int S, int CPL, bool VEC, int KMAX, bool KFIX, bool FUSED = false>
__global__ __launch_bounds__(512) void decode_kernel(DecodeParams<T> p) {
    extern __shared__ float smem[];
    // smem layout: written states [kw][S][span], read values [kr][span]
    float *written = smem;
    float *reads = smem + p.kw * S * p.span;
    __shared__ int s_rank_slot[kMaxSlots];

    const int64_t seq = blockIdx.x / (p.heads * p.spans);
    const int head = (blockIdx.x / p.spans) % p.heads;
    const int span0 = (blockIdx.x % p.spans) * p.span;
    const int slot = threadIdx.x / p.lanes_per_slot;
    const int lc = (threadIdx.x % p.lanes_per_slot) * CPL;  // column within the span
    const int col0 = span0 + lc;
    const int64_t row = seq * p.heads + head;
    const bool has_write = slot < p.kw;
    const bool has_read = slot < p.kr;
    auto clamp_bank = [&](int64_t bank) { return bank < 0 ? int64_t(0) : (bank >= p.banks ? int64_t(p.banks - 1) : bank); };

    int64_t wbank[KMAX], rbank[KMAX];
    float wwt[KMAX], rwt[KMAX];
    float kk[S], gg[S], bb[S], qq[S];
    float vv[CPL], wv[CPL];
    if constexpr (FUSED) {
        static_assert(KFIX && VEC && KMAX == 8 && S == 8 && std::is_same<T, bf16_t>::value, "fused geometry");
        __shared__ int64_t s_bank[2][KMAX];
        __shared__ float s_wt[2][KMAX];
        __shared__ float s_ctrl[4][S];
        const T *prow = p.proj + seq * p.proj_stride;
        const int wave = int(threadIdx.x) / kWave, lane = int(threadIdx.x) % kWave;
        if (wave < 2) {
            // routes of both roles (gdn2_banks.py:74-114): wave 0 writes, wave 1 reads
            float wt;
            int64_t bk;
            route_row_wave(prow + (wave == 0 ? p.write_col : p.read_col), p.j1, p.j2, KMAX, lane, wt, bk);
            if (lane < KMAX) {
                s_bank[wave][lane] = bk;
                s_wt[wave][lane] = wt;
            }
        } else if (wave == 2 && (lane < 3 || (lane == 3 && !p.f_weight))) {
            // the head's controller rows (heads.py:11-22): q, k, b rounded to T, g FP32
            float y[S];
            if (lane < 2)
                qk_row<T, S, true>(prow + (lane == 0 ? p.q_col : p.k_col) + head * S, p.qk_norm, y);
            else if (lane == 2)
                sigmoid_row<T, S, true>(prow + p.b_col + head * S, y);
            else
                decay_row<T, S, true>(p.f + seq * p.f_stride + head * S, p.a_log, p.dt_bias, p.param_dtype, head, y);
#pragma unroll
            for (int r = 0; r < S; ++r) s_ctrl[lane][r] = lane == 3 ? y[r] : round_to<T>(y[r]);
        } else if (wave == 3 && p.f_weight) {
            // f = f_proj[1](f_proj[0] slice) for this head's S rows: lane
            // (r, part) sums elements part*8 + 64*i .. +7 of row r in FP32, in
            // increasing order, then the 8 parts add in a fixed butterfly and
            // the sum is rounded to T (the GEMM's output dtype)
            const int r = lane / 8, part = lane % 8;
            const T *x = prow + p.f_col;
            const T *wrow = p.f_weight + int64_t(head * S + r) * p.f_width;
            float acc = 0.f;
            for (int i0 = part * 8; i0 < p.f_width; i0 += 64) {
                float xa[8], wb[8];
                load_row<8>(x + i0, xa);
                load_row<8>(wrow + i0, wb);
#pragma unroll
                for (int j = 0; j < 8; ++j) acc = fmaf(xa[j], wb[j], acc);
            }
            acc += __shfl_xor(acc, 1, 8);
            acc += __shfl_xor(acc, 2, 8);
            acc += __shfl_xor(acc, 4, 8);
            const float f = round_to<T>(acc);
            if (part == 0) {
                // decay_row's element: g = -exp(A_log[h]) * softplus(f + dt_bias)
                const float a = -expf(param_at(p.a_log, p.param_dtype, head));
                s_ctrl[3][r] = a * softplus_f(f + param_at(p.dt_bias, p.param_dtype, int64_t(head) * S + r));
                if (p.f_out) p.f_out[seq * int64_t(p.heads) * S + head * S + r] = from_f32<T>(f);
            }
        }
        {
            // this lane's value columns: v = silu, w = sigmoid, rounded to T
            float tv[CPL], tw[CPL];
            load_row<CPL>(prow + p.v_col + int64_t(head) * p.width + col0, tv);
            load_row<CPL>(prow + p.w_col + int64_t(head) * p.width + col0, tw);
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                vv[c] = round_to<T>(silu_f(tv[c]));
                wv[c] = round_to<T>(sigmoid_f(tw[c]));
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
            wbank[j] = clamp_bank(s_bank[0][j]);
            rbank[j] = clamp_bank(s_bank[1][j]);
            wwt[j] = s_wt[0][j];
            rwt[j] = s_wt[1][j];
        }
#pragma unroll
        for (int r = 0; r < S; ++r) {
            qq[r] = s_ctrl[0][r];
            kk[r] = s_ctrl[1][r];
            bb[r] = s_ctrl[2][r];
            gg[r] = s_ctrl[3][r];
        }
    } else {
        // ---- round trip 1: everything that does not depend on a bank index,
        // issued together with no barrier behind it.  The token's bank indices,
        // route weights and controller rows have workgroup-uniform addresses and
        // are read by scalar loads (entry j >= K re-reads entry K-1, so every
        // address is in bounds and the loads are unconditional); each lane group
        // selects its own slot's entries.  The lane's value columns are vector loads.
        const int64_t *wi = p.wi + seq * p.kw;
        const int64_t *ri = p.ri + seq * p.kr;
        const T *wwp = p.ww + seq * p.kw;
        const T *rwp = p.rw + seq * p.kr;
        if constexpr (KFIX) {
            // exactly KMAX banks per role: straight-line loads of whole rows
#pragma unroll
            for (int j = 0; j < KMAX; ++j) {
                wbank[j] = clamp_bank(wi[j]);
                rbank[j] = clamp_bank(ri[j]);
            }
            load_row<KMAX>(wwp, wwt);
            load_row<KMAX>(rwp, rwt);
        } else {
#pragma unroll
            for (int j = 0; j < KMAX; ++j) {
                const int jw = min(j, max(p.kw - 1, 0)), jr = min(j, max(p.kr - 1, 0));
                wbank[j] = p.kw > 0 ? clamp_bank(wi[jw]) : 0;
                wwt[j] = p.kw > 0 ? to_f32(wwp[jw]) : 0.f;
                rbank[j] = p.kr > 0 ? clamp_bank(ri[jr]) : 0;
                rwt[j] = p.kr > 0 ? to_f32(rwp[jr]) : 0.f;
            }
        }
        {
            const int64_t at = row * p.s_real;
            load_ctrl_row<S, VEC>(p.k + at, p.s_real, kk);
            load_ctrl_row<S, VEC>(p.g + at, p.s_real, gg);
            load_ctrl_row<S, VEC>(p.b + at, p.s_real, bb);
            load_ctrl_row<S, VEC>(p.q + at, p.s_real, qq);
        }
        load_row<CPL>(p.v + row * p.width + col0, vv);
        load_row<CPL>(p.w + row * p.width + col0, wv);
    }
    int64_t my_w = 0, my_r = 0;
    float pw = 0.f, pr = 0.f;
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
        if (j == slot) {
            my_w = wbank[j];
            my_r = rbank[j];
            pw = wwt[j];
            pr = rwt[j];
        }
    }
    if (!has_write) pw = 0.f;
    // a read of a bank written by the same token is served from the stored
    // post-write value in LDS
    int read_from_write = -1;
#pragma unroll
    for (int j = 0; j < KMAX; ++j)
        if (j < p.kw && wbank[j] == my_r) read_from_write = j;
    if (!has_read) read_from_write = -1;

    // ---- round trip 2: the bank states this step touches
    const int64_t bank_stride = int64_t(p.heads) * p.s_real * p.width;  // elements per bank
    const int64_t seq_base = seq * p.banks * bank_stride + int64_t(head) * p.s_real * p.width + col0;
    float hw[S][CPL], hr[S][CPL];
#pragma unroll
    for (int r = 0; r < S; ++r)
#pragma unroll
        for (int c = 0; c < CPL; ++c) hw[r][c] = hr[r][c] = 0.f;
    // Unconditional, branch-free loads (a conditional load under divergent
    // control makes the compiler wait at the join): a lane group without a
    // write loads bank 0, a read served from a same-step write re-reads the
    // write bank's lines, already requested by the write load.
    const bool load_read = has_read && read_from_write < 0;
    {
        const int64_t wbase = seq_base + my_w * bank_stride;
        const int64_t rbase = load_read ? seq_base + my_r * bank_stride : wbase;
        const SE *st = static_cast<const SE *>(p.state);
#pragma unroll
        for (int r = 0; r < S; ++r) {
            if (VEC || r < p.s_real) {
                load_row<CPL>(st + wbase + int64_t(r) * p.width, hw[r]);
                load_row<CPL>(st + rbase + int64_t(r) * p.width, hr[r]);
            }
        }
    }
    // thread t < KR ranks read slot t by (bank id, slot)
    if (int(threadIdx.x) < p.kr) {
        const int t = threadIdx.x;
        int64_t mine = rbank[0];
#pragma unroll
        for (int j = 1; j < KMAX; ++j)
            if (j == t) mine = rbank[j];
        int rank = 0;
#pragma unroll
        for (int j = 0; j < KMAX; ++j)
            if (j < p.kr) rank += (rbank[j] < mine) || (rbank[j] == mine && j < t);
        s_rank_slot[rank] = t;
    }

    // ---- writes (inference.py:21-34 with the write rule of role_bank_kernel.py:40-43)
    if (has_write) {
        WriteRows<S> rows;
        prepare_write_rows<T, S>(kk, gg, bb, pw, p.routed_decay, rows);
        float ew[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) ew[c] = round_to<T>(wv[c] * pw);
        apply_write<S, CPL>(hw, rows, ew, vv);
        const int64_t base = seq_base + my_w * bank_stride;
#pragma unroll
        for (int r = 0; r < S; ++r) {
            if (!VEC && r >= p.s_real) continue;
            if constexpr (std::is_same<SE, bf16_t>::value) {
#pragma unroll
                for (int c = 0; c < CPL; ++c) hw[r][c] = round_bf16(hw[r][c]);
            }
            store_row<CPL>(static_cast<SE *>(p.state) + base + int64_t(r) * p.width, hw[r]);
#pragma unroll
            for (int c = 0; c < CPL; ++c) written[(slot * S + r) * p.span + lc + c] = hw[r][c];
        }
    }
    __syncthreads();

    // ---- reads of the post-write states (inference.py:37-50)
    if (has_read) {
        if (read_from_write >= 0) {
#pragma unroll
            for (int r = 0; r < S; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c)
                    hr[r][c] = r < p.s_real ? written[(read_from_write * S + r) * p.span + lc + c] : 0.f;
        }
        float qr[S];
#pragma unroll
        for (int r = 0; r < S; ++r) qr[r] = round_to<T>(qq[r] * pr);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            float acc = 0.f;
#pragma unroll
            for (int r = 0; r < S; ++r) acc = fmaf(qr[r], hr[r][c], acc);
            reads[slot * p.span + lc + c] = round_to<T>(acc * p.scale);
        }
    }
    __syncthreads();

    // ---- ordered sum (inference.py:53-67)
    T *out = p.out + seq * int64_t(p.heads) * p.width + int64_t(head) * p.width + span0;
    for (int c = threadIdx.x; c < p.span; c += blockDim.x) {
        float v[kMaxSlots];
#pragma unroll
        for (int j = 0; j < kMaxSlots; ++j) v[j] = j < p.kr ? reads[s_rank_slot[j] * p.span + c] : 0.f;
        float total = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxSlots; ++j)
            if (j < p.kr) total = round_to<T>(total + v[j]);
        out[c] = from_f32<T>(total);
    }
}

template <typename T, int S, int CPL>
int launch_decode(const bdm_decode_args &a, hipStream_t stream) {
    DecodeParams<T> p{};
    p.q = static_cast<const T *>(a.q);
    p.k = static_cast<const T *>(a.k);
    p.b = static_cast<const T *>(a.b);
    p.g = a.g;
    p.v = static_cast<const T *>(a.v);
    p.w = static_cast<const T *>(a.w);
    p.ww = static_cast<const T *>(a.write_weights);
    p.rw = static_cast<const T *>(a.read_weights);
    p.wi = a.write_indices;
    p.ri = a.read_indices;
    p.state = a.state;
    p.out = static_cast<T *>(a.output);
    p.heads = a.heads;
    p.s_real = a.bank_size;
    p.width = a.head_width;
    p.banks = a.bank_count;
    p.kw = a.write_banks;
    p.kr = a.read_banks;
    // the widest span (a divisor of the head width, a multiple of CPL) that
    // fits 512 lanes and 64 KiB of LDS
    const int slots = a.write_banks > a.read_banks ? a.write_banks : a.read_banks;
    auto lds_bytes = [&](int span) {
        return (size_t(a.write_banks) * S * span + size_t(a.read_banks) * span) * sizeof(float);
    };
    int span = a.head_width;
    while ((slots * (span / CPL) > 512 || lds_bytes(span) > 64 * 1024) && span % 2 == 0 && (span / 2) % CPL == 0)
        span /= 2;
    p.span = span;
    p.spans = a.head_width / span;
    p.lanes_per_slot = span / CPL;
    // vector row loads need the S-element rows at 16-byte boundaries
    p.vec_rows = (a.bank_size == S && aligned(a.q, 16) && aligned(a.k, 16) && aligned(a.b, 16) && aligned(a.g, 16) &&
                  (S * sizeof(T)) % 16 == 0)
                     ? 1
                     : 0;
    p.state_dtype = a.state_dtype;
    p.routed_decay = a.routed_decay;
    p.scale = a.scale;
    const int threads = ((slots * p.lanes_per_slot + kWave - 1) / kWave) * kWave;
    if (threads > 512) return fail(BDM_ERR_UNSUPPORTED, "decode: %d lanes per workgroup", threads);
    const size_t lds = lds_bytes(span);
    if (lds > 64 * 1024) return fail(BDM_ERR_UNSUPPORTED, "decode: %zu bytes of LDS", lds);
    if (a.batch * a.heads * p.spans > int64_t(UINT32_MAX)) return fail(BDM_ERR_UNSUPPORTED, "decode: grid too large");
    const unsigned grid = unsigned(a.batch * a.heads * p.spans);
    // the production geometry (8 banks per role, full-width aligned rows) gets
    // straight-line loads; anything else the general form
    const bool fast = p.vec_rows && a.write_banks == 8 && a.read_banks == 8 && aligned(a.write_weights, 16) &&
                      aligned(a.read_weights, 16) && aligned(a.write_indices, 16) && aligned(a.read_indices, 16);
    if (a.state_dtype == BDM_BF16) {
        if (fast)
            decode_kernel<T, bf16_t, S, CPL, true, 8, true><<<grid, threads, lds, stream>>>(p);
        else
            decode_kernel<T, bf16_t, S, CPL, false, kMaxSlots, false><<<grid, threads, lds, stream>>>(p);
    } else {
        if (fast)
            decode_kernel<T, float, S, CPL, true, 8, true><<<grid, threads, lds, stream>>>(p);
        else
            decode_kernel<T, float, S, CPL, false, kMaxSlots, false><<<grid, threads, lds, stream>>>(p);
    }
    return check_launch("decode_kernel");
}

// The fused step (bdm_decode_fused): BF16 controllers, S = 8, 8 banks per
// role, two columns per lane, spans of 128 columns at most; at least three
// waves per workgroup (two routers and the controller rows).
int launch_decode_fused(const bdm_decode_fused_args &a, hipStream_t stream) {
    constexpr int S = 8, CPL = 2, K = 8;
    DecodeParams<bf16_t> p{};
    p.proj = static_cast<const bf16_t *>(a.proj);
    p.f = static_cast<const bf16_t *>(a.f);
    p.a_log = a.a_log;
    p.dt_bias = a.dt_bias;
    p.proj_stride = a.proj_stride;
    p.f_stride = a.f_stride;
    p.q_col = a.q_col, p.k_col = a.k_col, p.v_col = a.v_col, p.b_col = a.b_col, p.w_col = a.w_col;
    p.read_col = a.read_col, p.write_col = a.write_col;
    p.j1 = a.factor_first, p.j2 = a.factor_second;
    p.f_weight = static_cast<const bf16_t *>(a.f_weight);
    p.f_out = static_cast<bf16_t *>(a.f_out);
    p.f_col = a.f_col;
    p.f_width = a.f_width;
    p.param_dtype = a.param_dtype;
    p.qk_norm = a.qk_norm;
    p.state = a.state;
    p.out = static_cast<bf16_t *>(a.output);
    p.heads = a.heads;
    p.s_real = S;
    p.width = a.head_width;
    p.banks = a.factor_first * a.factor_second;
    p.kw = p.kr = K;
    int span = a.head_width;
    while (span > 128 && span % 2 == 0) span /= 2;
    p.span = span;
    p.spans = a.head_width / span;
    p.lanes_per_slot = span / CPL;
    p.vec_rows = 1;
    p.state_dtype = a.state_dtype;
    p.routed_decay = a.routed_decay;
    p.scale = a.scale;
    const int threads = K * p.lanes_per_slot;
    const size_t lds = (size_t(K) * S * span + size_t(K) * span) * sizeof(float);
    const unsigned grid = unsigned(a.batch * a.heads * p.spans);
    if (a.state_dtype == BDM_BF16)
        decode_kernel<bf16_t, bf16_t, S, CPL, true, K, true, true><<<grid, threads, lds, stream>>>(p);
    else
        decode_kernel<bf16_t, float, S, CPL, true, K, true, true><<<grid, threads, lds, stream>>>(p);
    return check_launch("decode_kernel (fused step)");
}

template <typename T>
int dispatch_decode(const bdm_decode_args &a, hipStream_t stream) {
    if (a.bank_size <= 8) {
        // two columns per lane: 64 lanes per slot, more loads in flight per
        // step (wide heads run as spans of 128 columns)
        if (a.head_width % 2 == 0 && (a.head_width / 2 <= 64 || a.head_width % 128 == 0))
            return launch_decode<T, 8, 2>(a, stream);
        if (a.head_width % 4 == 0 && a.head_width / 4 <= 64) return launch_decode<T, 8, 4>(a, stream);
        if (a.head_width % 8 == 0) return launch_decode<T, 8, 8>(a, stream);
        return launch_decode<T, 8, 1>(a, stream);
    }
    if (a.bank_size <= 16) {
        if (a.head_width % 4 == 0) return launch_decode<T, 16, 4>(a, stream);
        return launch_decode<T, 16, 1>(a, stream);
    }
    if (a.head_width % 2 == 0) return launch_decode<T, 32, 2>(a, stream);
    return launch_decode<T, 32, 1>(a, stream);
}

}  // namespace
}  // namespace bdm

extern "C" int bdm_decode(const bdm_decode_args *a, void *stream) {
    using namespace bdm;
    if (!a) return fail(BDM_ERR_INVALID, "decode: null args");
    if (a->batch <= 0 || a->heads <= 0 || a->bank_size <= 0 || a->head_width <= 0 || a->bank_count <= 0 ||
        a->write_banks < 0 || a->read_banks < 0 || a->write_banks + a->read_banks == 0)
        return fail(BDM_ERR_INVALID, "decode: bad geometry");
    if (a->bank_size > 32) return fail(BDM_ERR_UNSUPPORTED, "decode: bank_size %d > 32", a->bank_size);
    if (a->write_banks > kMaxSlots || a->read_banks > kMaxSlots)
        return fail(BDM_ERR_UNSUPPORTED, "decode: more than %d selected banks", kMaxSlots);
    if (a->ctrl_dtype != BDM_BF16 && a->ctrl_dtype != BDM_F32) return fail(BDM_ERR_INVALID, "decode: ctrl dtype");
    if (a->state_dtype != BDM_BF16 && a->state_dtype != BDM_F32) return fail(BDM_ERR_INVALID, "decode: state dtype");
    if (a->batch * a->heads > int64_t(INT32_MAX)) return fail(BDM_ERR_UNSUPPORTED, "decode: grid too large");
    if (!a->q || !a->k || !a->g || !a->b || !a->v || !a->w || !a->state || !a->output ||
        (a->write_banks && (!a->write_weights || !a->write_indices)) ||
        (a->read_banks && (!a->read_weights || !a->read_indices)))
        return fail(BDM_ERR_INVALID, "decode: null pointer");
    const void *ptrs[] = {a->v, a->w, a->state, a->output};
    for (const void *ptr : ptrs)
        if (!aligned(ptr, 16)) return fail(BDM_ERR_INVALID, "decode: tensors must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    if (a->ctrl_dtype == BDM_BF16) return dispatch_decode<bf16_t>(*a, s);
    return dispatch_decode<float>(*a, s);
}

extern "C" int bdm_decode_fused_supported(const bdm_decode_fused_args *a) {
    if (!a) return 0;
    const int j1 = a->factor_first, j2 = a->factor_second;
    const int s = a->selected_banks < j1 ? (a->selected_banks < j2 ? a->selected_banks : j2) : (j1 < j2 ? j1 : j2);
    const int count = a->selected_banks < s * s ? a->selected_banks : s * s;
    int span = a->head_width;
    while (span > 128 && span % 2 == 0) span /= 2;
    const bool cols8 = a->q_col % 8 == 0 && a->k_col % 8 == 0 && a->v_col % 8 == 0 && a->b_col % 8 == 0 &&
                       a->w_col % 8 == 0 && a->read_col % 8 == 0 && a->write_col % 8 == 0;
    // f formed in the launch: a fourth wave (64-column spans at least) and 16-byte aligned rows
    const bool f_ok = !a->f_weight || (span >= 64 && a->f_width > 0 && a->f_width % 8 == 0 && a->f_col % 8 == 0 &&
                                       a->f_col >= 0);
    return f_ok && a->batch > 0 && a->heads > 0 && a->ctrl_dtype == BDM_BF16 && a->bank_size == 8 &&
           a->selected_banks == 8 && count == 8 && j1 >= 1 && j2 >= 1 && j1 <= 64 && j2 <= 64 &&
           a->head_width % 2 == 0 && span <= 128 && span >= 48 && a->head_width % span == 0 &&
           (a->state_dtype == BDM_BF16 || a->state_dtype == BDM_F32) &&
           (a->param_dtype == BDM_BF16 || a->param_dtype == BDM_F32) && a->proj_stride % 8 == 0 &&
           a->f_stride % 8 == 0 && cols8 && a->q_col >= 0 && a->k_col >= 0 && a->v_col >= 0 && a->b_col >= 0 &&
           a->w_col >= 0 && a->read_col >= 0 && a->write_col >= 0;
}

extern "C" int bdm_decode_fused(const bdm_decode_fused_args *a, void *stream) {
    using namespace bdm;
    if (!a) return fail(BDM_ERR_INVALID, "decode_fused: null args");
    if (!bdm_decode_fused_supported(a))
        return fail(BDM_ERR_UNSUPPORTED, "decode_fused: geometry outside the fused step (BF16, S = 8, 8 banks per "
                                         "role, J1, J2 <= 64, aligned column offsets, head spans of 48..128)");
    if (a->batch * a->heads > int64_t(INT32_MAX) / 16) return fail(BDM_ERR_UNSUPPORTED, "decode_fused: grid too large");
    if (!a->proj || (!a->f && !a->f_weight) || !a->a_log || !a->dt_bias || !a->state || !a->output)
        return fail(BDM_ERR_INVALID, "decode_fused: null pointer");
    const void *ptrs[] = {a->proj, a->f, a->a_log, a->dt_bias, a->state, a->output, a->f_weight, a->f_out};
    for (const void *ptr : ptrs)
        if (ptr && !aligned(ptr, 16)) return fail(BDM_ERR_INVALID, "decode_fused: tensors must be 16-byte aligned");
    return launch_decode_fused(*a, as_stream(stream));
}

// Single-token decode against resident bank states.
//
// Reference: inference.step (implementation/bdm/inference.py:161-194) and its
// kernels _decode_write (:21-34), _decode_read (:37-50), _decode_sum (:53-67);
// the reference supports one head with eight rows only (:88-104), this kernel
// any head count and bank size <= 32.
//
// One workgroup per (sequence, head).  Lane group j (head_width / CPL lanes)
// owns write slot j and read slot j.  A step makes two dependent trips to HBM:
// first the bank indices and controller rows (all independent of a bank id),
// then every bank state the step touches — the write banks and the read banks
// that are not also written — requested at once.  Writes are applied and stored (rounded
// to the state dtype), and also kept in LDS, so a read of a bank written by the
// same token sees the stored value without another trip to HBM.  The reads are
// then combined in increasing bank id with a rounding after every add.
#include "bdm_common.h"
#include "recurrence_ops.h"

namespace bdm {
namespace {

constexpr int kMaxSlots = 16;

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
    int lanes_per_slot;
    int state_dtype, routed_decay;
    float scale;
};

template <typename T, int S, int CPL>
__global__ __launch_bounds__(512) void decode_kernel(DecodeParams<T> p) {
    extern __shared__ float smem[];
    // smem layout: written states [kw][S][width], read values [kr][width]
    float *written = smem;
    float *reads = smem + p.kw * S * p.width;
    __shared__ int s_rank_slot[kMaxSlots];

    const int64_t seq = blockIdx.x / p.heads;
    const int head = blockIdx.x % p.heads;
    const int slot = threadIdx.x / p.lanes_per_slot;
    const int col0 = (threadIdx.x % p.lanes_per_slot) * CPL;
    const int64_t row = seq * p.heads + head;
    const bool has_write = slot < p.kw;
    const bool has_read = slot < p.kr;

    // ---- round trip 1: everything that does not depend on a bank index.  The
    // per-token values are loaded once for the workgroup, one element per lane
    // of the first wave(s), and shared through LDS (a conditional scalar load
    // per value would serialise them).
    __shared__ int64_t s_wbank[kMaxSlots], s_rbank[kMaxSlots];
    __shared__ float s_pw[kMaxSlots], s_pr[kMaxSlots];
    __shared__ float s_ctrl[4][32];  // k, g, b, q rows (S <= 32)
    {
        const int nk = p.kw + p.kr;
        for (int t = threadIdx.x; t < nk + 4 * S; t += blockDim.x) {
            if (t < p.kw) {
                const int64_t bank = p.wi[seq * p.kw + t];
                s_wbank[t] = bank < 0 ? 0 : (bank >= p.banks ? p.banks - 1 : bank);
                s_pw[t] = to_f32(p.ww[seq * p.kw + t]);
            } else if (t < nk) {
                const int j = t - p.kw;
                const int64_t bank = p.ri[seq * p.kr + j];
                s_rbank[j] = bank < 0 ? 0 : (bank >= p.banks ? p.banks - 1 : bank);
                s_pr[j] = to_f32(p.rw[seq * p.kr + j]);
            } else {
                const int e = t - nk, which = e / S, r = e % S;
                float x = 0.f;
                if (r < p.s_real) {
                    const int64_t at = row * p.s_real + r;
                    x = which == 0 ? to_f32(p.k[at])
                                   : which == 1 ? p.g[at] : which == 2 ? to_f32(p.b[at]) : to_f32(p.q[at]);
                }
                s_ctrl[which][r] = x;
            }
        }
    }
    float vv[CPL], wv[CPL];
    load_row<CPL>(p.v + row * p.width + col0, vv);
    load_row<CPL>(p.w + row * p.width + col0, wv);
    __syncthreads();
    float kk[S], gg[S], bb[S], qq[S];
#pragma unroll
    for (int r = 0; r < S; ++r) {
        kk[r] = s_ctrl[0][r];
        gg[r] = s_ctrl[1][r];
        bb[r] = s_ctrl[2][r];
        qq[r] = s_ctrl[3][r];
    }
    const float pw = has_write ? s_pw[slot] : 0.f;
    const float pr = has_read ? s_pr[slot] : 0.f;
    // this lane group's write bank and read bank; a read of a bank written by
    // the same token is served from the stored post-write value in LDS
    const int64_t my_w = has_write ? s_wbank[slot] : 0;
    const int64_t my_r = has_read ? s_rbank[slot] : 0;
    int read_from_write = -1;
    if (has_read) {
        for (int j = 0; j < p.kw; ++j)
            if (s_wbank[j] == my_r) read_from_write = j;
    }
    // thread t < KR ranks read slot t by (bank id, slot)
    if (int(threadIdx.x) < p.kr) {
        const int t = threadIdx.x;
        const int64_t mine = s_rbank[t];
        int rank = 0;
        for (int j = 0; j < p.kr; ++j) rank += (s_rbank[j] < mine) || (s_rbank[j] == mine && j < t);
        s_rank_slot[rank] = t;
    }

    // ---- round trip 2: the bank states this step touches
    const int64_t bank_stride = int64_t(p.heads) * p.s_real * p.width;  // elements per bank
    const int64_t seq_base = seq * p.banks * bank_stride + int64_t(head) * p.s_real * p.width + col0;
    float hw[S][CPL], hr[S][CPL];
#pragma unroll
    for (int r = 0; r < S; ++r)
#pragma unroll
        for (int c = 0; c < CPL; ++c) hw[r][c] = hr[r][c] = 0.f;
    if (has_write) {
        const int64_t base = seq_base + my_w * bank_stride;
#pragma unroll
        for (int r = 0; r < S; ++r) {
            if (r >= p.s_real) continue;
            if (p.state_dtype == BDM_BF16)
                load_row<CPL>(static_cast<const bf16_t *>(p.state) + base + int64_t(r) * p.width, hw[r]);
            else
                load_row<CPL>(static_cast<const float *>(p.state) + base + int64_t(r) * p.width, hw[r]);
        }
    }
    if (has_read && read_from_write < 0) {
        const int64_t base = seq_base + my_r * bank_stride;
#pragma unroll
        for (int r = 0; r < S; ++r) {
            if (r >= p.s_real) continue;
            if (p.state_dtype == BDM_BF16)
                load_row<CPL>(static_cast<const bf16_t *>(p.state) + base + int64_t(r) * p.width, hr[r]);
            else
                load_row<CPL>(static_cast<const float *>(p.state) + base + int64_t(r) * p.width, hr[r]);
        }
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
            if (r >= p.s_real) continue;
            if (p.state_dtype == BDM_BF16) {
#pragma unroll
                for (int c = 0; c < CPL; ++c) hw[r][c] = round_bf16(hw[r][c]);
                store_row<CPL>(static_cast<bf16_t *>(p.state) + base + int64_t(r) * p.width, hw[r]);
            } else {
                store_row<CPL>(static_cast<float *>(p.state) + base + int64_t(r) * p.width, hw[r]);
            }
#pragma unroll
            for (int c = 0; c < CPL; ++c) written[(slot * S + r) * p.width + col0 + c] = hw[r][c];
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
                    hr[r][c] = r < p.s_real ? written[(read_from_write * S + r) * p.width + col0 + c] : 0.f;
        }
        float qr[S];
#pragma unroll
        for (int r = 0; r < S; ++r) qr[r] = round_to<T>(qq[r] * pr);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            float acc = 0.f;
#pragma unroll
            for (int r = 0; r < S; ++r) acc = fmaf(qr[r], hr[r][c], acc);
            reads[slot * p.width + col0 + c] = round_to<T>(acc * p.scale);
        }
    }
    __syncthreads();

    // ---- ordered sum (inference.py:53-67)
    T *out = p.out + seq * int64_t(p.heads) * p.width + int64_t(head) * p.width;
    for (int c = threadIdx.x; c < p.width; c += blockDim.x) {
        float total = 0.f;
        for (int j = 0; j < p.kr; ++j) total = round_to<T>(total + reads[s_rank_slot[j] * p.width + c]);
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
    p.lanes_per_slot = a.head_width / CPL;
    p.state_dtype = a.state_dtype;
    p.routed_decay = a.routed_decay;
    p.scale = a.scale;
    const int slots = a.write_banks > a.read_banks ? a.write_banks : a.read_banks;
    const int threads = ((slots * p.lanes_per_slot + kWave - 1) / kWave) * kWave;
    if (threads > 512) return fail(BDM_ERR_UNSUPPORTED, "decode: %d lanes per workgroup", threads);
    const size_t lds = (size_t(a.write_banks) * S * a.head_width + size_t(a.read_banks) * a.head_width) * sizeof(float);
    if (lds > 64 * 1024) return fail(BDM_ERR_UNSUPPORTED, "decode: %zu bytes of LDS", lds);
    decode_kernel<T, S, CPL><<<unsigned(a.batch * a.heads), threads, lds, stream>>>(p);
    return check_launch("decode_kernel");
}

template <typename T>
int dispatch_decode(const bdm_decode_args &a, hipStream_t stream) {
    if (a.bank_size <= 8) {
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

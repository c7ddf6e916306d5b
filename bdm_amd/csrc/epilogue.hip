// Controller and output epilogues of the inference path: the elementwise and
// per-head work around the projection GEMMs, one pass each over the GEMM
// outputs instead of a dozen elementwise kernels.
//
// Reference: heads.controllers (implementation/bdm/heads.py:11-22) with
// _normalize_qk (_parameters.py:214-220), and _project_bank_output
// (_parameters.py:222-232).  Every intermediate that torch materialises in
// the controller dtype is rounded to it at the same point here (silu before
// the l2 normalization, sigmoid of the gate before the product, ...); the
// arithmetic between those points is FP32 as in torch's opmath.
//
// The language-model shell around the layer adds two more: the residual add
// fused with RMSNorm (_shell.py:10-35) and the SwiGLU product
// silu(w1 x) * (w3 x) (_shell.py:86-91) over one GEMM of the concatenated
// w1 | w3 weights.
#include <type_traits>

#include "epilogue_ops.h"

namespace bdm {
namespace {

template <typename T>
struct ControllerParams {
    const T *proj, *f;
    const void *a_log, *dt_bias;
    T *q, *k, *v, *b, *w;
    float *g;
    int64_t tokens, proj_stride, f_stride;
    int q_col, k_col, v_col, b_col, w_col;
    int heads, hv, param_dtype, qk_norm;
};

// One thread per (token, item): items 0..4H-1 are the q, k, b, g rows of one
// head (S values, 8 at a time), the rest 8-column chunks of v then w.  VEC:
// every 8-element group of the inputs and outputs is 16-byte aligned.
template <typename T, int S, bool VEC>
__global__ __launch_bounds__(64) void controller_epilogue_kernel(ControllerParams<T> p) {
    static_assert(S % 8 == 0, "S");
    const int chunks = p.heads * p.hv / 8;
    const int items = 4 * p.heads + 2 * chunks;
    const int64_t token = blockIdx.x;  // grid: (tokens, item blocks of 64)
    const int it = int(blockIdx.y) * 64 + int(threadIdx.x);
    if (it >= items) return;
    const T *row = p.proj + token * p.proj_stride;
    const int64_t hs = int64_t(p.heads) * S;
    // the row helpers are shared with the fused decode step (decode.hip)
    auto store = [&](auto *dst, const float (&y)[S]) {
#pragma unroll
        for (int r0 = 0; r0 < S; r0 += 8) {
            float t[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) t[j] = y[r0 + j];
            if constexpr (VEC)
                store_row<8>(dst + r0, t);
            else
#pragma unroll
                for (int j = 0; j < 8; ++j) dst[r0 + j] = from_f32<std::remove_pointer_t<decltype(dst)>>(t[j]);
        }
    };
    if (it < 2 * p.heads) {
        // q or k: silu, rounded, then the l2 normalization over the head's S values
        const int h = it % p.heads;
        float y[S];
        qk_row<T, S, VEC>(row + (it < p.heads ? p.q_col : p.k_col) + h * S, p.qk_norm, y);
        store((it < p.heads ? p.q : p.k) + token * hs + h * S, y);
    } else if (it < 3 * p.heads) {
        const int h = it - 2 * p.heads;
        float y[S];
        sigmoid_row<T, S, VEC>(row + p.b_col + h * S, y);
        store(p.b + token * hs + h * S, y);
    } else if (it < 4 * p.heads) {
        // g = -exp(A_log[h]) * softplus(f + dt_bias), FP32
        const int h = it - 3 * p.heads;
        float y[S];
        decay_row<T, S, VEC>(p.f + token * p.f_stride + h * S, p.a_log, p.dt_bias, p.param_dtype, h, y);
        store(p.g + token * hs + h * S, y);
    } else {
        const int c = it - 4 * p.heads;
        const bool is_v = c < chunks;
        const int col = (is_v ? c : c - chunks) * 8;
        const T *src = row + (is_v ? p.v_col : p.w_col) + col;
        T *dst = (is_v ? p.v : p.w) + token * int64_t(p.heads) * p.hv + col;
        float x[8];
        load8<T, VEC>(src, x);
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = is_v ? silu_f(x[j]) : sigmoid_f(x[j]);
        store_row<8>(dst, x);
    }
}

template <typename T>
struct OutputParams {
    const T *raw, *gate;
    const void *weight, *bias;
    T *out;
    int64_t tokens, gate_stride;
    int width, param_dtype, norm_kind;
    float eps;
};

// One wave per token; a lane owns 8-column chunks lane*8, lane*8 + 512, ...
// VEC: raw, gate and the parameters are read as 16-byte groups.
template <typename T, int MAXC, bool VEC>
__global__ __launch_bounds__(256) void output_epilogue_kernel(OutputParams<T> p) {
    const int lane = threadIdx.x % kWave;
    const int64_t token = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (token >= p.tokens) return;
    const T *raw = p.raw + token * p.width;
    const T *gate = p.gate + token * p.gate_stride;
    float x[MAXC][8], gs[MAXC][8];
    float sum = 0.f, sq = 0.f;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        const int c = min((lane + i * kWave) * 8, p.width - 8);  // chunks past the width re-read the last
        load8<T, VEC>(raw + c, x[i]);
        load8<T, VEC>(gate + c, gs[i]);
        const bool live = (lane + i * kWave) * 8 < p.width;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            x[i][j] = live ? x[i][j] : 0.f;
            sum += x[i][j];
            sq = fmaf(x[i][j], x[i][j], sq);
        }
    }
    const float inv_n = 1.f / float(p.width);
    float mean = 0.f, scale = 0.f;
    if (p.norm_kind == 1) {
        // layer norm: mean, then the centred second moment
        mean = wave_total<kWave>(sum) * inv_n;
        float var = 0.f;
#pragma unroll
        for (int i = 0; i < MAXC; ++i) {
            const bool live = (lane + i * kWave) * 8 < p.width;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float d = x[i][j] - mean;
                var = live ? fmaf(d, d, var) : var;
            }
        }
        scale = rsqrtf(fmaf(wave_total<kWave>(var), inv_n, p.eps));
    } else {
        scale = round_to<T>(rsqrtf(fmaf(wave_total<kWave>(sq), inv_n, p.eps)));
    }
    T *out = p.out + token * p.width;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        const int c = (lane + i * kWave) * 8;
        if (c >= p.width) continue;
        float wt[8], bs[8], y[8];
        param8<VEC>(p.weight, p.param_dtype, c, wt);
        if (p.norm_kind == 1) param8<VEC>(p.bias, p.param_dtype, c, bs);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float n;
            if (p.norm_kind == 1) {
                // the multiply-adds spelled out: the fused GEMV prologue rounds identically
                n = round_to<T>(fmaf((x[i][j] - mean) * scale, wt[j], bs[j]));
            } else {
                n = round_to<T>(x[i][j] * scale);
                n = round_to<T>(n * round_to<T>(wt[j]));
            }
            y[j] = n * round_to<T>(sigmoid_f(gs[i][j]));
        }
        store_row<8>(out + c, y);
    }
}

template <typename T>
int launch_controller(const bdm_controller_args &a, hipStream_t stream) {
    ControllerParams<T> p{};
    p.proj = static_cast<const T *>(a.proj);
    p.f = static_cast<const T *>(a.f);
    p.a_log = a.a_log;
    p.dt_bias = a.dt_bias;
    p.q = static_cast<T *>(a.q);
    p.k = static_cast<T *>(a.k);
    p.v = static_cast<T *>(a.v);
    p.b = static_cast<T *>(a.b);
    p.w = static_cast<T *>(a.w);
    p.g = a.g;
    p.tokens = a.tokens;
    p.proj_stride = a.proj_stride;
    p.f_stride = a.f_stride;
    p.q_col = a.q_col;
    p.k_col = a.k_col;
    p.v_col = a.v_col;
    p.b_col = a.b_col;
    p.w_col = a.w_col;
    p.heads = a.heads;
    p.hv = a.head_width;
    p.param_dtype = a.param_dtype;
    p.qk_norm = a.qk_norm;
    const int64_t items = 4 * int64_t(a.heads) + 2 * (int64_t(a.heads) * a.head_width / 8);
    const dim3 blocks(unsigned(a.tokens), unsigned((items + 63) / 64));
    // 16-byte groups everywhere: aligned bases, strides and column offsets in multiples of 8 elements
    const bool vec = aligned(a.proj, 16) && aligned(a.f, 16) && aligned(a.q, 16) && aligned(a.k, 16) &&
                     aligned(a.b, 16) && aligned(a.g, 16) && aligned(a.dt_bias, 16) && a.proj_stride % 8 == 0 &&
                     a.f_stride % 8 == 0 && a.q_col % 8 == 0 && a.k_col % 8 == 0 && a.v_col % 8 == 0 &&
                     a.b_col % 8 == 0 && a.w_col % 8 == 0;
#define BDM_CTRL(S) (vec ? (controller_epilogue_kernel<T, S, true><<<blocks, 64, 0, stream>>>(p), 0) \
                         : (controller_epilogue_kernel<T, S, false><<<blocks, 64, 0, stream>>>(p), 0))
    switch (a.bank_size) {
        case 8: BDM_CTRL(8); break;
        case 16: BDM_CTRL(16); break;
        case 32: BDM_CTRL(32); break;
        default: return fail(BDM_ERR_UNSUPPORTED, "controller epilogue: bank_size %d", a.bank_size);
    }
#undef BDM_CTRL
    return check_launch("controller_epilogue_kernel");
}

template <typename T>
int launch_output(const bdm_output_args &a, hipStream_t stream) {
    OutputParams<T> p{};
    p.raw = static_cast<const T *>(a.raw);
    p.gate = static_cast<const T *>(a.gate);
    p.weight = a.norm_weight;
    p.bias = a.norm_bias;
    p.out = static_cast<T *>(a.out);
    p.tokens = a.tokens;
    p.gate_stride = a.gate_stride;
    p.width = a.width;
    p.param_dtype = a.param_dtype;
    p.norm_kind = a.norm_kind;
    p.eps = a.eps;
    const unsigned blocks = unsigned((a.tokens + 3) / 4);
    const int chunks = (a.width / 8 + kWave - 1) / kWave;  // 8-column chunks per lane
    const bool vec = aligned(a.raw, 16) && aligned(a.gate, 16) && aligned(a.norm_weight, 16) &&
                     (!a.norm_bias || aligned(a.norm_bias, 16)) && a.gate_stride % 8 == 0;
#define BDM_OUT(C) (vec ? (output_epilogue_kernel<T, C, true><<<blocks, 256, 0, stream>>>(p), 0) \
                        : (output_epilogue_kernel<T, C, false><<<blocks, 256, 0, stream>>>(p), 0))
    if (chunks <= 1)
        BDM_OUT(1);
    else if (chunks <= 2)
        BDM_OUT(2);
    else if (chunks <= 4)
        BDM_OUT(4);
    else if (chunks <= 8)
        BDM_OUT(8);
    else
        return fail(BDM_ERR_UNSUPPORTED, "output epilogue: width %d > 4096", a.width);
#undef BDM_OUT
    return check_launch("output_epilogue_kernel");
}

// RMSNorm of the shell (_shell.py:29-35): out = (x * rsqrt(mean(x^2) + eps))
// * weight in FP32, rounded once to T.  With a residual, x = round(a + r) is
// the block's new hidden state: written to sum_out and normalized.  One wave
// per row; lane l owns the 8-column chunks l*8, l*8 + 512, ...
template <typename T, int MAXC, bool VEC>
__global__ __launch_bounds__(256) void rms_norm_kernel(const T *__restrict__ x, const T *__restrict__ residual,
                                                       const void *__restrict__ weight, int weight_dtype,
                                                       T *__restrict__ sum_out, T *__restrict__ out, int64_t rows,
                                                       int width, float eps) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = int64_t(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;
    const int64_t base = row * width;
    float h[MAXC][8];
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        const int c = min((lane + i * kWave) * 8, width - 8);  // chunks past the width re-read the last
        const bool live = (lane + i * kWave) * 8 < width;
        load8<T, VEC>(x + base + c, h[i]);
        if (residual) {
            float r[8];
            load8<T, VEC>(residual + base + c, r);
#pragma unroll
            for (int j = 0; j < 8; ++j) h[i][j] = round_to<T>(h[i][j] + r[j]);
            if (live) store_row<8>(sum_out + base + c, h[i]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) sq = live ? fmaf(h[i][j], h[i][j], sq) : sq;
    }
    const float scale = rsqrtf(wave_total<kWave>(sq) / float(width) + eps);
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        const int c = (lane + i * kWave) * 8;
        if (c >= width) continue;
        float wt[8], y[8];
        param8<VEC>(weight, weight_dtype, c, wt);
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = h[i][j] * scale * wt[j];
        store_row<8>(out + base + c, y);
    }
}

// Gradients of rms_norm_kernel's normalization (no residual) for training.
// With xh = x * s, s = rsqrt(mean(x^2) + eps) and y = xh * w in FP32:
//   dxh = dy * w,  dx = dxh * s - x * s^3 * sum(dxh * x) / width,
//   dw = sum over rows of dy * xh,
// the derivative of the FP32 chain of RMSNorm.forward (_shell.py:29-35) that
// autograd forms op by op.  One wave per row; the 4 waves of a workgroup take
// kRmsRowsPerBlock consecutive rows and each wave keeps an FP32 partial of dw
// for its columns; the workgroup adds its waves' partials in LDS and stores
// one partial row, and rms_norm_weight_grad_kernel sums the partial rows.
constexpr int kRmsRowsPerBlock = 32;

template <typename T, int MAXC, bool VEC>
__global__ __launch_bounds__(256) void rms_norm_backward_kernel(const T *__restrict__ x, const T *__restrict__ dy,
                                                                const void *__restrict__ weight, int weight_dtype,
                                                                T *__restrict__ dx, float *__restrict__ dw_part,
                                                                int64_t rows, int width, float eps) {
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int64_t first = int64_t(blockIdx.x) * kRmsRowsPerBlock;
    const int64_t last = min(rows, first + kRmsRowsPerBlock);
    float acc[MAXC][8];
#pragma unroll
    for (int i = 0; i < MAXC; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.f;
    for (int64_t row = first + wave; row < last; row += blockDim.x / kWave) {
        const int64_t base = row * width;
        float h[MAXC][8], g[MAXC][8];
        float sq = 0.f;
#pragma unroll
        for (int i = 0; i < MAXC; ++i) {
            const int c = min((lane + i * kWave) * 8, width - 8);
            const bool live = (lane + i * kWave) * 8 < width;
            load8<T, VEC>(x + base + c, h[i]);
            load8<T, VEC>(dy + base + c, g[i]);
#pragma unroll
            for (int j = 0; j < 8; ++j) sq = live ? fmaf(h[i][j], h[i][j], sq) : sq;
        }
        const float s = rsqrtf(wave_total<kWave>(sq) / float(width) + eps);
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < MAXC; ++i) {
            const int c = (lane + i * kWave) * 8;
            if (c >= width) continue;
            float wt[8];
            param8<VEC>(weight, weight_dtype, c, wt);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc[i][j] = fmaf(g[i][j], h[i][j] * s, acc[i][j]);
                g[i][j] *= wt[j];  // dxh
                dot = fmaf(g[i][j], h[i][j], dot);
            }
        }
        const float coef = wave_total<kWave>(dot) * s * s * s / float(width);
#pragma unroll
        for (int i = 0; i < MAXC; ++i) {
            const int c = (lane + i * kWave) * 8;
            if (c >= width) continue;
            float d[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) d[j] = g[i][j] * s - h[i][j] * coef;
            store_row<8>(dx + base + c, d);
        }
    }
    // the workgroup's partial row: its waves' partials added in wave order
    extern __shared__ float red[];  // [waves][width]
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        const int c = (lane + i * kWave) * 8;
        if (c < width)
#pragma unroll
            for (int j = 0; j < 8; ++j) red[wave * width + c + j] = acc[i][j];
    }
    __syncthreads();
    float *part = dw_part + int64_t(blockIdx.x) * width;
    for (int c = threadIdx.x; c < width; c += blockDim.x) {
        float total = red[c];
        for (int w = 1; w < int(blockDim.x / kWave); ++w) total += red[w * width + c];
        part[c] = total;
    }
}

// dw[c] = sum of the partial rows' column c, rounded once to the weight's
// dtype.  A workgroup of 16 waves owns 64 columns: wave k sums the partial
// rows k, k + 16, ... (loads unrolled, many in flight), and the 16 wave sums
// are added in wave order, so the result repeats bit for bit.
constexpr int kRmsSumWaves = 16;

__global__ __launch_bounds__(kRmsSumWaves * 64) void rms_norm_weight_grad_kernel(const float *__restrict__ dw_part,
                                                                                 int64_t parts, int width,
                                                                                 void *__restrict__ dw, int dw_dtype) {
    __shared__ float slice[kRmsSumWaves][64];
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int c = int(blockIdx.x) * 64 + lane;
    float total = 0.f;
    if (c < width) {
#pragma unroll 8
        for (int64_t p = wave; p < parts; p += kRmsSumWaves) total += dw_part[p * width + c];
    }
    slice[wave][lane] = total;
    __syncthreads();
    if (wave != 0 || c >= width) return;
    float sum = slice[0][lane];
    for (int k = 1; k < kRmsSumWaves; ++k) sum += slice[k][lane];
    if (dw_dtype == BDM_BF16)
        static_cast<bf16_t *>(dw)[c] = from_f32<bf16_t>(sum);
    else
        static_cast<float *>(dw)[c] = sum;
}

// SwiGLU of the shell's feed-forward (_shell.py:86-91) over the output of one
// GEMM with the concatenated w1 | w3 weights: row r holds x1 = w1 x in columns
// [0, hidden) and x3 = w3 x in [hidden, 2 hidden).  out = round(round(silu(x1))
// * x3), the two roundings torch makes in the module's dtype; silu is
// x / (1 + exp(-x)) with IEEE division, as torch evaluates it.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void swiglu_kernel(const T *__restrict__ gate_up, T *__restrict__ out,
                                                     int64_t rows, int hidden) {
    const int64_t groups = int64_t(hidden) / 8;
    const int64_t item = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (item >= rows * groups) return;
    const int64_t row = item / groups;
    const int c = int(item % groups) * 8;
    const T *in = gate_up + row * 2 * hidden;
    float a[8], b[8], y[8];
    load8<T, VEC>(in + c, a);
    load8<T, VEC>(in + hidden + c, b);
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = swiglu_value<T>(a[j], b[j]);
    store_row<8>(out + row * hidden + c, y);
}

// The SwiGLU element over two separate tensors (the training path's w1 x and
// w3 x, _shell.py:86-91), 8 consecutive elements per thread.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void swiglu_pair_kernel(const T *__restrict__ a, const T *__restrict__ b,
                                                          T *__restrict__ out, int64_t n) {
    const int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
    if (i >= n) return;
    if (VEC && i + 8 <= n) {
        float x[8], y[8], z[8];
        load8<T, true>(a + i, x);
        load8<T, true>(b + i, y);
#pragma unroll
        for (int j = 0; j < 8; ++j) z[j] = swiglu_value<T>(x[j], y[j]);
        store_row<8>(out + i, z);
    } else {
        for (int64_t e = i; e < min(n, i + 8); ++e) out[e] = from_f32<T>(swiglu_value<T>(to_f32(a[e]), to_f32(b[e])));
    }
}

// Gradients of h = round(silu(a)) * b in the order and dtype autograd forms
// them for F.silu(a) * b: s = round(silu(a)), db = round(dy * s),
// ds = round(dy * b), da = round(ds * sig * (1 + a * (1 - sig))) with
// sig = 1 / (1 + exp(-a)) in FP32 (silu's backward).
__device__ __forceinline__ void swiglu_grad(float a, float b, float dy, float &da, float &db, bool bf16) {
    const float sig = 1.f / (1.f + expf(-a));
    const float s = a / (1.f + expf(-a));
    const float sr = bf16 ? round_bf16(s) : s;
    const float ds = bf16 ? round_bf16(dy * b) : dy * b;
    db = dy * sr;
    da = ds * sig * (1.f + a * (1.f - sig));
}

template <typename T, bool VEC>
__global__ __launch_bounds__(256) void swiglu_backward_kernel(const T *__restrict__ a, const T *__restrict__ b,
                                                              const T *__restrict__ dy, T *__restrict__ da,
                                                              T *__restrict__ db, int64_t n) {
    constexpr bool kBf16 = sizeof(T) == 2;
    const int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
    if (i >= n) return;
    if (VEC && i + 8 <= n) {
        float x[8], y[8], g[8], ga[8], gb[8];
        load8<T, true>(a + i, x);
        load8<T, true>(b + i, y);
        load8<T, true>(dy + i, g);
#pragma unroll
        for (int j = 0; j < 8; ++j) swiglu_grad(x[j], y[j], g[j], ga[j], gb[j], kBf16);
        store_row<8>(da + i, ga);
        store_row<8>(db + i, gb);
    } else {
        for (int64_t e = i; e < min(n, i + 8); ++e) {
            float ga, gb;
            swiglu_grad(to_f32(a[e]), to_f32(b[e]), to_f32(dy[e]), ga, gb, kBf16);
            da[e] = from_f32<T>(ga);
            db[e] = from_f32<T>(gb);
        }
    }
}

}  // namespace
}  // namespace bdm

extern "C" int bdm_controller_epilogue(const bdm_controller_args *a, void *stream) {
    using namespace bdm;
    if (!a) return fail(BDM_ERR_INVALID, "controller epilogue: null args");
    if (a->tokens < 0 || a->heads <= 0 || a->bank_size <= 0 || a->head_width <= 0)
        return fail(BDM_ERR_INVALID, "controller epilogue: bad geometry");
    if ((int64_t(a->heads) * a->head_width) % 8 != 0)
        return fail(BDM_ERR_UNSUPPORTED, "controller epilogue: value width not a multiple of 8");
    if (a->tokens > int64_t(INT32_MAX) || 4 * int64_t(a->heads) + 2 * int64_t(a->heads) * a->head_width / 8 > 64 * 65535)
        return fail(BDM_ERR_UNSUPPORTED, "controller epilogue: grid too large");
    if (a->ctrl_dtype != BDM_BF16 && a->ctrl_dtype != BDM_F32) return fail(BDM_ERR_INVALID, "controller: dtype");
    if (a->param_dtype != BDM_BF16 && a->param_dtype != BDM_F32) return fail(BDM_ERR_INVALID, "controller: params");
    const int64_t hs = int64_t(a->heads) * a->bank_size, vw = int64_t(a->heads) * a->head_width;
    const int64_t cols[5] = {a->q_col, a->k_col, a->b_col, a->v_col, a->w_col};
    const int64_t widths[5] = {hs, hs, hs, vw, vw};
    for (int i = 0; i < 5; ++i)
        if (cols[i] < 0 || cols[i] + widths[i] > a->proj_stride)
            return fail(BDM_ERR_INVALID, "controller epilogue: slice %d outside the projection row", i);
    if (a->f_stride < hs) return fail(BDM_ERR_INVALID, "controller epilogue: f row shorter than H*S");
    if (a->tokens == 0) return BDM_OK;
    if (!a->proj || !a->f || !a->a_log || !a->dt_bias || !a->q || !a->k || !a->v || !a->b || !a->w || !a->g)
        return fail(BDM_ERR_INVALID, "controller epilogue: null pointer");
    if (!aligned(a->v, 16) || !aligned(a->w, 16))
        return fail(BDM_ERR_INVALID, "controller epilogue: v and w must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    if (a->ctrl_dtype == BDM_BF16) return launch_controller<bf16_t>(*a, s);
    return launch_controller<float>(*a, s);
}

extern "C" int bdm_output_epilogue(const bdm_output_args *a, void *stream) {
    using namespace bdm;
    if (!a) return fail(BDM_ERR_INVALID, "output epilogue: null args");
    if (a->tokens < 0 || a->width <= 0 || a->width % 8 != 0 || a->gate_stride < a->width)
        return fail(BDM_ERR_INVALID, "output epilogue: bad geometry");
    if (a->norm_kind != 0 && a->norm_kind != 1) return fail(BDM_ERR_INVALID, "output epilogue: norm kind");
    if (a->ctrl_dtype != BDM_BF16 && a->ctrl_dtype != BDM_F32) return fail(BDM_ERR_INVALID, "output: dtype");
    if (a->param_dtype != BDM_BF16 && a->param_dtype != BDM_F32) return fail(BDM_ERR_INVALID, "output: params");
    if (a->tokens == 0) return BDM_OK;
    if (!a->raw || !a->gate || !a->norm_weight || !a->out || (a->norm_kind == 1 && !a->norm_bias))
        return fail(BDM_ERR_INVALID, "output epilogue: null pointer");
    if (!aligned(a->out, 16)) return fail(BDM_ERR_INVALID, "output epilogue: out must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    if (a->ctrl_dtype == BDM_BF16) return launch_output<bf16_t>(*a, s);
    return launch_output<float>(*a, s);
}

extern "C" int bdm_rms_norm(const void *x, const void *residual, const void *weight, void *sum_out, void *out,
                            int64_t rows, int32_t width, int32_t dtype, int32_t weight_dtype, float eps,
                            void *stream) {
    using namespace bdm;
    if (rows < 0 || width <= 0 || width % 8 != 0) return fail(BDM_ERR_INVALID, "rms_norm: bad geometry");
    if (width > 8192) return fail(BDM_ERR_UNSUPPORTED, "rms_norm: width %d > 8192", width);
    if (dtype != BDM_BF16 && dtype != BDM_F32) return fail(BDM_ERR_INVALID, "rms_norm: dtype");
    if (weight_dtype != BDM_BF16 && weight_dtype != BDM_F32) return fail(BDM_ERR_INVALID, "rms_norm: weight dtype");
    if (rows == 0) return BDM_OK;
    if (!x || !weight || !out || (residual && !sum_out)) return fail(BDM_ERR_INVALID, "rms_norm: null pointer");
    if ((rows + 3) / 4 > int64_t(INT32_MAX)) return fail(BDM_ERR_UNSUPPORTED, "rms_norm: too many rows");
    const bool vec = aligned(x, 16) && aligned(weight, 16) && aligned(out, 16) &&
                     (!residual || (aligned(residual, 16) && aligned(sum_out, 16)));
    const unsigned blocks = unsigned((rows + 3) / 4);
    const int chunks = (width / 8 + kWave - 1) / kWave;
    hipStream_t s = as_stream(stream);
    auto go = [&](auto tag) {
        using T = decltype(tag);
        const T *xp = static_cast<const T *>(x), *rp = static_cast<const T *>(residual);
        T *sp = static_cast<T *>(sum_out), *op = static_cast<T *>(out);
#define BDM_RMS(C)                                                                                           \
    (vec ? (rms_norm_kernel<T, C, true><<<blocks, 256, 0, s>>>(xp, rp, weight, weight_dtype, sp, op, rows, width, eps), 0) \
         : (rms_norm_kernel<T, C, false><<<blocks, 256, 0, s>>>(xp, rp, weight, weight_dtype, sp, op, rows, width, eps), 0))
        if (chunks <= 1)
            BDM_RMS(1);
        else if (chunks <= 2)
            BDM_RMS(2);
        else if (chunks <= 4)
            BDM_RMS(4);
        else if (chunks <= 8)
            BDM_RMS(8);
        else
            BDM_RMS(16);
#undef BDM_RMS
    };
    if (dtype == BDM_BF16)
        go(bf16_t{});
    else
        go(0.f);
    return check_launch("rms_norm_kernel");
}

extern "C" int64_t bdm_rms_norm_backward_partials(int64_t rows) {
    return rows <= 0 ? 0 : (rows + bdm::kRmsRowsPerBlock - 1) / bdm::kRmsRowsPerBlock;
}

extern "C" int bdm_rms_norm_backward(const void *x, const void *grad_out, const void *weight, void *grad_x,
                                     void *grad_weight, float *partials, int64_t rows, int32_t width, int32_t dtype,
                                     int32_t weight_dtype, float eps, void *stream) {
    using namespace bdm;
    if (rows < 0 || width <= 0 || width % 8 != 0) return fail(BDM_ERR_INVALID, "rms_norm_backward: bad geometry");
    if (width > 4096) return fail(BDM_ERR_UNSUPPORTED, "rms_norm_backward: width %d > 4096", width);
    if (dtype != BDM_BF16 && dtype != BDM_F32) return fail(BDM_ERR_INVALID, "rms_norm_backward: dtype");
    if (weight_dtype != BDM_BF16 && weight_dtype != BDM_F32)
        return fail(BDM_ERR_INVALID, "rms_norm_backward: weight dtype");
    if (!x || !grad_out || !weight || !grad_x || !grad_weight || (rows > 0 && !partials))
        return fail(BDM_ERR_INVALID, "rms_norm_backward: null pointer");
    const int64_t parts = bdm_rms_norm_backward_partials(rows);
    if (parts > int64_t(INT32_MAX)) return fail(BDM_ERR_UNSUPPORTED, "rms_norm_backward: too many rows");
    hipStream_t s = as_stream(stream);
    if (rows > 0) {
        const bool vec = aligned(x, 16) && aligned(grad_out, 16) && aligned(weight, 16) && aligned(grad_x, 16) &&
                         aligned(partials, 16);
        const int chunks = (width / 8 + kWave - 1) / kWave;
        const size_t lds = size_t(4) * width * sizeof(float);
        auto go = [&](auto tag) {
            using T = decltype(tag);
            const T *xp = static_cast<const T *>(x), *gp = static_cast<const T *>(grad_out);
            T *dp = static_cast<T *>(grad_x);
#define BDM_RMS_BWD(C)                                                                                        \
    (vec ? (rms_norm_backward_kernel<T, C, true><<<unsigned(parts), 256, lds, s>>>(xp, gp, weight, weight_dtype, dp, \
                                                                                   partials, rows, width, eps), \
            0)                                                                                                 \
         : (rms_norm_backward_kernel<T, C, false><<<unsigned(parts), 256, lds, s>>>(                          \
                xp, gp, weight, weight_dtype, dp, partials, rows, width, eps),                                 \
            0))
            if (chunks <= 1)
                BDM_RMS_BWD(1);
            else if (chunks <= 2)
                BDM_RMS_BWD(2);
            else if (chunks <= 4)
                BDM_RMS_BWD(4);
            else
                BDM_RMS_BWD(8);
#undef BDM_RMS_BWD
        };
        if (dtype == BDM_BF16)
            go(bf16_t{});
        else
            go(0.f);
        if (int rc = check_launch("rms_norm_backward_kernel")) return rc;
        rms_norm_weight_grad_kernel<<<unsigned((width + 63) / 64), kRmsSumWaves * 64, 0, s>>>(
            partials, parts, width, grad_weight, weight_dtype);
    } else {
        // no rows: the weight gradient is zero
        rms_norm_weight_grad_kernel<<<unsigned((width + 63) / 64), kRmsSumWaves * 64, 0, s>>>(
            nullptr, 0, width, grad_weight, weight_dtype);
    }
    return check_launch("rms_norm_weight_grad_kernel");
}

extern "C" int bdm_swiglu(const void *gate_up, void *out, int64_t rows, int32_t hidden, int32_t dtype,
                          void *stream) {
    using namespace bdm;
    if (rows < 0 || hidden <= 0 || hidden % 8 != 0) return fail(BDM_ERR_INVALID, "swiglu: bad geometry");
    if (dtype != BDM_BF16 && dtype != BDM_F32) return fail(BDM_ERR_INVALID, "swiglu: dtype");
    if (rows == 0) return BDM_OK;
    if (!gate_up || !out) return fail(BDM_ERR_INVALID, "swiglu: null pointer");
    const int64_t items = rows * (hidden / 8);
    if ((items + 255) / 256 > int64_t(INT32_MAX)) return fail(BDM_ERR_UNSUPPORTED, "swiglu: too many rows");
    const bool vec = aligned(gate_up, 16) && aligned(out, 16);
    const unsigned blocks = unsigned((items + 255) / 256);
    hipStream_t s = as_stream(stream);
    if (dtype == BDM_BF16) {
        auto *in = static_cast<const bf16_t *>(gate_up);
        auto *o = static_cast<bf16_t *>(out);
        if (vec)
            swiglu_kernel<bf16_t, true><<<blocks, 256, 0, s>>>(in, o, rows, hidden);
        else
            swiglu_kernel<bf16_t, false><<<blocks, 256, 0, s>>>(in, o, rows, hidden);
    } else {
        auto *in = static_cast<const float *>(gate_up);
        auto *o = static_cast<float *>(out);
        if (vec)
            swiglu_kernel<float, true><<<blocks, 256, 0, s>>>(in, o, rows, hidden);
        else
            swiglu_kernel<float, false><<<blocks, 256, 0, s>>>(in, o, rows, hidden);
    }
    return check_launch("swiglu_kernel");
}

extern "C" int bdm_swiglu_pair(const void *a, const void *b, void *out, int64_t n, int32_t dtype, void *stream) {
    using namespace bdm;
    if (n < 0) return fail(BDM_ERR_INVALID, "swiglu_pair: bad size");
    if (dtype != BDM_BF16 && dtype != BDM_F32) return fail(BDM_ERR_INVALID, "swiglu_pair: dtype");
    if (n == 0) return BDM_OK;
    if (!a || !b || !out) return fail(BDM_ERR_INVALID, "swiglu_pair: null pointer");
    const int64_t blocks = (n + 8 * 256 - 1) / (8 * 256);
    if (blocks > int64_t(INT32_MAX)) return fail(BDM_ERR_UNSUPPORTED, "swiglu_pair: too many elements");
    const bool vec = aligned(a, 16) && aligned(b, 16) && aligned(out, 16);
    hipStream_t s = as_stream(stream);
    auto go = [&](auto tag) {
        using T = decltype(tag);
        auto *pa = static_cast<const T *>(a), *pb = static_cast<const T *>(b);
        auto *po = static_cast<T *>(out);
        if (vec)
            swiglu_pair_kernel<T, true><<<unsigned(blocks), 256, 0, s>>>(pa, pb, po, n);
        else
            swiglu_pair_kernel<T, false><<<unsigned(blocks), 256, 0, s>>>(pa, pb, po, n);
    };
    if (dtype == BDM_BF16)
        go(bf16_t{});
    else
        go(0.f);
    return check_launch("swiglu_pair_kernel");
}

extern "C" int bdm_swiglu_backward(const void *a, const void *b, const void *grad_out, void *grad_a, void *grad_b,
                                   int64_t n, int32_t dtype, void *stream) {
    using namespace bdm;
    if (n < 0) return fail(BDM_ERR_INVALID, "swiglu_backward: bad size");
    if (dtype != BDM_BF16 && dtype != BDM_F32) return fail(BDM_ERR_INVALID, "swiglu_backward: dtype");
    if (n == 0) return BDM_OK;
    if (!a || !b || !grad_out || !grad_a || !grad_b) return fail(BDM_ERR_INVALID, "swiglu_backward: null pointer");
    const int64_t blocks = (n + 8 * 256 - 1) / (8 * 256);
    if (blocks > int64_t(INT32_MAX)) return fail(BDM_ERR_UNSUPPORTED, "swiglu_backward: too many elements");
    const bool vec = aligned(a, 16) && aligned(b, 16) && aligned(grad_out, 16) && aligned(grad_a, 16) &&
                     aligned(grad_b, 16);
    hipStream_t s = as_stream(stream);
    auto go = [&](auto tag) {
        using T = decltype(tag);
        auto *pa = static_cast<const T *>(a), *pb = static_cast<const T *>(b), *pg = static_cast<const T *>(grad_out);
        auto *da = static_cast<T *>(grad_a), *db = static_cast<T *>(grad_b);
        if (vec)
            swiglu_backward_kernel<T, true><<<unsigned(blocks), 256, 0, s>>>(pa, pb, pg, da, db, n);
        else
            swiglu_backward_kernel<T, false><<<unsigned(blocks), 256, 0, s>>>(pa, pb, pg, da, db, n);
    };
    if (dtype == BDM_BF16)
        go(bf16_t{});
    else
        go(0.f);
    return check_launch("swiglu_backward_kernel");
}

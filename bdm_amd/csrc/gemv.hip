// Skinny linear maps of the decode step: y[m] = W x'[m] + bias for a few rows
// m (one per sequence of a decode batch), W [N, K] row-major as nn.Linear
// stores it, x' the input row after an optional prologue.
//
// At one to four rows every weight byte is read once and used M times, so
// the map is a stream over W at HBM bandwidth, not a matrix product: the
// GEMM libraries' tiles for M = 1 leave most of that bandwidth unused.  Each
// wave owns R consecutive output rows; lane l reads the 16-byte groups
// l, l + 64, ... of each of its rows (coalesced 1 KiB per row and load), all
// of them issued before the first FMA, and keeps one FP32 sum per (m, row).
// The sums are reduced across the wave and lane (m, row) adds the bias and
// stores the output, rounded once to the output dtype as torch's F.linear
// does (FP32 accumulation, bias added in FP32).
//
// Prologues.  At one row, the elementwise kernel that produces a GEMV's input
// costs a launch (~5 us) for microseconds of work, so the GEMV forms its input
// itself (K <= 6144): every wave issues all its weight loads, then reads the
// input row (from L2) into registers and applies
//   RMS:     the shell's RMSNorm, after the residual add when one is given
//            (the sum, the block's new hidden state, is stored by one wave);
//   SWIGLU:  round(round(silu(a)) * b) of a [2K] row (a | b);
//   OUT_LAYER / OUT_RMS: the layer's output interface, norm(raw) * sigmoid(gate).
// Each prologue visits the row in the lane order of the standalone kernel it
// replaces (rms_norm_kernel, swiglu_kernel, output_epilogue_kernel) with the
// same sums and rounding points, so the fused result is bit-identical to the
// unfused pair of kernels (FP32 layer norm: the row mean can differ in its
// last bit, the result within an FP32 ulp).
#include <type_traits>

#include "epilogue_ops.h"

namespace bdm {
namespace {

enum Prologue { kPlain = 0, kRms = 1, kSwiglu = 2, kOutLayer = 3, kOutRms = 4 };

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Eight consecutive weights from a 16-byte aligned address, widened to FP32:
// streamed once, so BF16 rows are read nontemporal.
__device__ __forceinline__ void stream8(const bf16_t *p, float (&x)[8]) {
    const u32x4_t r = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        x[2 * q] = __uint_as_float(w[q] << 16);
        x[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
    }
}
__device__ __forceinline__ void stream8(const float *p, float (&x)[8]) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
    x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
}

template <typename T>
struct GemvParams {
    const T *x, *w, *bias;
    T *y;
    const T *residual;     // kRms: [M, K] or null
    T *sum_out;            // kRms with a residual: [M, K] <- round(x + residual)
    const void *norm_w;    // kRms, kOut*: [K] of param_dtype
    const void *norm_b;    // kOutLayer: [K]
    const T *gate;         // kOut*: [M, gate_stride]
    int64_t n, gate_stride;
    int k, param_dtype;
    float eps;
};

// Row m's GEMV input x' for the lane's groups lane + 64 i (i < NCH), held in
// registers, after the prologue.  The statistics are summed in the lane order
// of the standalone kernel (lane l: groups l, l + 64, ...) with its rounding
// points; groups past the row are zero and take no part in the sums.
template <typename T, int NCH, int PRO>
__device__ __forceinline__ void prologue_row(const GemvParams<T> &p, int m, int lane, bool store_sum,
                                             float (&xr)[NCH][8]) {
    const int groups = p.k / 8;
    bool live[NCH];
    int gs[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        live[i] = lane + i * kWave < groups;
        gs[i] = min(lane + i * kWave, groups - 1);
    }
    if constexpr (PRO == kRms) {
        float wt[NCH][8];
        const T *x = p.x + int64_t(m) * p.k;
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            load8<T, true>(x + gs[i] * 8, xr[i]);
            param8<true>(p.norm_w, p.param_dtype, int64_t(gs[i]) * 8, wt[i]);
        }
        if (p.residual) {
            const T *res = p.residual + int64_t(m) * p.k;
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                float r[8];
                load8<T, true>(res + gs[i] * 8, r);
#pragma unroll
                for (int j = 0; j < 8; ++j) xr[i][j] = round_to<T>(xr[i][j] + r[j]);
                if (store_sum && live[i]) store_row<8>(p.sum_out + int64_t(m) * p.k + gs[i] * 8, xr[i]);
            }
        }
        float sq = 0.f;
#pragma unroll
        for (int i = 0; i < NCH; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) sq = live[i] ? fmaf(xr[i][j], xr[i][j], sq) : sq;
        const float scale = rsqrtf(wave_total<kWave>(sq) / float(p.k) + p.eps);
#pragma unroll
        for (int i = 0; i < NCH; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) xr[i][j] = round_to<T>(xr[i][j] * scale * wt[i][j]);
    } else if constexpr (PRO == kSwiglu) {
        const T *row = p.x + int64_t(m) * 2 * p.k;
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            float a[8], b[8];
            load8<T, true>(row + gs[i] * 8, a);
            load8<T, true>(row + p.k + gs[i] * 8, b);
#pragma unroll
            for (int j = 0; j < 8; ++j) xr[i][j] = swiglu_value<T>(a[j], b[j]);
        }
    } else {
        float gt[NCH][8];
        const T *x = p.x + int64_t(m) * p.k;
        const T *gate = p.gate + int64_t(m) * p.gate_stride;
        float sum = 0.f, sq = 0.f;
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            load8<T, true>(x + gs[i] * 8, xr[i]);
            load8<T, true>(gate + gs[i] * 8, gt[i]);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                sum += live[i] ? xr[i][j] : 0.f;
                sq = live[i] ? fmaf(xr[i][j], xr[i][j], sq) : sq;
            }
        }
        const float inv_n = 1.f / float(p.k);
        float mean = 0.f, scale;
        if constexpr (PRO == kOutLayer) {
            mean = wave_total<kWave>(sum) * inv_n;
            float var = 0.f;
#pragma unroll
            for (int i = 0; i < NCH; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float d = xr[i][j] - mean;
                    var = live[i] ? fmaf(d, d, var) : var;
                }
            scale = rsqrtf(fmaf(wave_total<kWave>(var), inv_n, p.eps));
        } else {
            scale = round_to<T>(rsqrtf(fmaf(wave_total<kWave>(sq), inv_n, p.eps)));
        }
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            float wt[8], bs[8];
            param8<true>(p.norm_w, p.param_dtype, int64_t(gs[i]) * 8, wt);
            if constexpr (PRO == kOutLayer) param8<true>(p.norm_b, p.param_dtype, int64_t(gs[i]) * 8, bs);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float n;
                if constexpr (PRO == kOutLayer) {
                    n = round_to<T>(fmaf((xr[i][j] - mean) * scale, wt[j], bs[j]));
                } else {
                    n = round_to<T>(xr[i][j] * scale);
                    n = round_to<T>(n * round_to<T>(wt[j]));
                }
                xr[i][j] = round_to<T>(n * round_to<T>(sigmoid_f(gt[i][j])));
            }
        }
    }
}

// The GEMV with a prologue: one pass over a row of at most NCH * 512
// elements.  Every weight load of the wave's R rows is issued first; the
// input rows are formed in registers while they are in flight.
template <typename T, int M, int R, int NCH, int PRO>
__global__ __launch_bounds__(256) void gemv_prologue_kernel(GemvParams<T> p) {
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int64_t row0 = (int64_t(blockIdx.x) * (blockDim.x / kWave) + wave) * R;
    if (row0 >= p.n) return;
    const int groups = p.k / 8;
    float wv[NCH][R][8];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int g = min(lane + i * kWave, groups - 1);  // past the end: re-read the last group
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t row = min(row0 + r, p.n - 1);
            stream8(p.w + row * p.k + int64_t(g) * 8, wv[i][r]);
        }
    }
    const bool store_sum = blockIdx.x == 0 && wave == 0;
#pragma unroll 1
    for (int m = 0; m < M; ++m) {
        float xr[NCH][8];
        prologue_row<T, NCH, PRO>(p, m, lane, store_sum, xr);
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const bool live = lane + i * kWave < groups;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float s = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) s = fmaf(wv[i][r][j], xr[i][j], s);
                acc[r] += live ? s : 0.f;
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = wave_total<kWave>(acc[r]);
            const int64_t row = row0 + r;
            if (lane == r && row < p.n) {
                const float out = p.bias ? v + to_f32(p.bias[row]) : v;
                p.y[int64_t(m) * p.n + row] = from_f32<T>(out);
            }
        }
    }
}

// M rows of x, R output rows per wave, KC 512-element chunks of K unrolled
// per pass (all weight loads of a pass in flight together).
template <typename T, int M, int R, int KC>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams<T> p) {
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int64_t row0 = (int64_t(blockIdx.x) * (blockDim.x / kWave) + wave) * R;
    if (row0 >= p.n) return;
    float acc[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.f;
    const int groups = p.k / 8;  // 16-byte groups per row
    for (int g0 = 0; g0 < groups; g0 += KC * kWave) {
        float wv[KC][R][8];
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int g = min(g0 + c * kWave + lane, groups - 1);  // past the end: re-read the last group
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int64_t row = min(row0 + r, p.n - 1);
                stream8(p.w + row * p.k + int64_t(g) * 8, wv[c][r]);
            }
        }
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const int gi = g0 + c * kWave + lane;
            const bool live = gi < groups;
            const int g = min(gi, groups - 1);
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float xv[8];
                load8<T, true>(p.x + int64_t(m) * p.k + g * 8, xv);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float s = 0.f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) s = fmaf(wv[c][r][j], xv[j], s);
                    acc[m][r] += live ? s : 0.f;
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = wave_total<kWave>(acc[m][r]);
    // lane m*R + r stores output (m, row0 + r)
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t row = row0 + r;
            if (lane == m * R + r && row < p.n) {
                float v = acc[m][r];
                if (p.bias) v += to_f32(p.bias[row]);
                p.y[int64_t(m) * p.n + row] = from_f32<T>(v);
            }
        }
}

template <typename T, int M>
int launch_plain(const GemvParams<T> &p, hipStream_t s) {
    // enough waves to keep HBM busy: 4 rows per wave once there are >= 8192
    // rows, fewer (more waves) below that
    const int groups = p.k / 8;
    const int kc = groups >= 4 * kWave ? 4 : (groups >= 2 * kWave ? 2 : 1);
    auto go = [&](auto r_tag) {
        constexpr int R = decltype(r_tag)::value;
        const int64_t waves = (p.n + R - 1) / R;
        const unsigned blocks = unsigned((waves + 3) / 4);
        if (kc == 4)
            gemv_kernel<T, M, R, 4><<<blocks, 256, 0, s>>>(p);
        else if (kc == 2)
            gemv_kernel<T, M, R, 2><<<blocks, 256, 0, s>>>(p);
        else
            gemv_kernel<T, M, R, 1><<<blocks, 256, 0, s>>>(p);
    };
    if (p.n >= 8192)
        go(std::integral_constant<int, 4>{});
    else if (p.n >= 2048)
        go(std::integral_constant<int, 2>{});
    else
        go(std::integral_constant<int, 1>{});
    return check_launch("gemv_kernel");
}

// Chunks of 512 elements per lane: 4 (K <= 2048) or 12 (K <= 6144); the
// weight groups in flight per lane, NCH * R, stay at 16 or fewer.
template <typename T, int M, int PRO>
int launch_prologue(const GemvParams<T> &p, hipStream_t s) {
    const int chunks = (p.k / 8 + kWave - 1) / kWave;
    const int want_r = p.n >= 8192 ? 4 : (p.n >= 2048 ? 2 : 1);
    auto go = [&](auto nch_tag, auto r_tag) {
        constexpr int NCH = decltype(nch_tag)::value, R = decltype(r_tag)::value;
        const int64_t waves = (p.n + R - 1) / R;
        gemv_prologue_kernel<T, M, R, NCH, PRO><<<unsigned((waves + 3) / 4), 256, 0, s>>>(p);
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    if (chunks <= 4) {
        if (want_r == 4) go(I4{}, I4{});
        else if (want_r == 2) go(I4{}, I2{});
        else go(I4{}, I1{});
    } else if (chunks <= 12) {
        go(std::integral_constant<int, 12>{}, I1{});
    } else {
        return fail(BDM_ERR_UNSUPPORTED, "gemv: a prologue takes K <= 6144 (K = %d)", p.k);
    }
    return check_launch("gemv_prologue_kernel");
}

template <typename T, int PRO>
int launch_gemv_pro(const GemvParams<T> &p, int64_t m, hipStream_t s) {
    if constexpr (PRO == kPlain) {
        switch (m) {
            case 1: return launch_plain<T, 1>(p, s);
            case 2: return launch_plain<T, 2>(p, s);
            case 3: return launch_plain<T, 3>(p, s);
            case 4: return launch_plain<T, 4>(p, s);
            default: break;
        }
    } else {
        switch (m) {
            case 1: return launch_prologue<T, 1, PRO>(p, s);
            case 2: return launch_prologue<T, 2, PRO>(p, s);
            case 3: return launch_prologue<T, 3, PRO>(p, s);
            case 4: return launch_prologue<T, 4, PRO>(p, s);
            default: break;
        }
    }
    return fail(BDM_ERR_UNSUPPORTED, "gemv: %lld rows (at most 4)", (long long)m);
}

// ---- 5 to 64 rows (a decode batch): matrix-core tiles
//
// y = x W^T + bias for BF16 x [M, K] and W [N, K] with M <= 64.  A workgroup
// owns 16 output columns for every row; its four waves each take a quarter of
// K and accumulate all M rows in v_mfma_f32_16x16x32_bf16 tiles (16 rows by
// 16 columns by 32 k), so the workgroup streams its 16 weight rows once and
// the rows of x, shared by every workgroup, come from L2.  The quarters'
// FP32 partials are added through LDS in wave order, the bias added in FP32
// and the sum rounded once, as F.linear does (the summation order differs
// from the library GEMM's, so results agree to FP32 rounding before the BF16
// one).  Against the library GEMM at the decode shapes (M = 64,
// graph-replayed): about equal with the weights in cache, ~1 µs faster with
// them coming from HBM, ~1 µs faster at M = 16; 64-column workgroups (x read
// from L2 a quarter as often) were twice as slow.
// Operand fragments: lane l supplies row (or column) l % 16 and the 8
// consecutive k at 8 * (l / 16) of the 32; A and B use the same lane-to-k
// assignment, so every product pairs equal k.  The 16 x 16 FP32 result holds
// rows 4 * (l / 16) .. + 3 of column l % 16 in lane l.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kSkinnyWaves = 4;
constexpr int kSkinnyMaxRows = 64;  // above 64 rows the library GEMM is faster (8.3 against 12 us at 128)

template <int MT>
__global__ __launch_bounds__(kSkinnyWaves * kWave) void skinny_gemm_kernel(const bf16_t *__restrict__ x,
                                                                           const bf16_t *__restrict__ w,
                                                                           const bf16_t *__restrict__ bias,
                                                                           bf16_t *__restrict__ y, int m, int n,
                                                                           int k) {
    __shared__ float part[kSkinnyWaves][MT * 256];  // each wave's partial tile
    __shared__ float bcol[16];                       // the workgroup's 16 biases
    const int wave = int(threadIdx.x) / kWave, lane = int(threadIdx.x) % kWave;
    const int col = lane % 16, kg = lane / 16;
    const int c = int(blockIdx.x) * 16 + col;  // this lane's output column
    // rows and columns past the matrix read the last one; their results are not stored
    const bf16_t *wrow = w + int64_t(min(c, n - 1)) * k + kg * 8;
    const bf16_t *xrow[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) xrow[t] = x + int64_t(min(t * 16 + col, m - 1)) * k + kg * 8;
    const float bc = bias ? to_f32(bias[min(c, n - 1)]) : 0.f;  // loaded before the products
    f32x4_t acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int steps = k / 32;
    const int per = (steps + kSkinnyWaves - 1) / kSkinnyWaves;
    const int s0 = min(steps, wave * per), s1 = min(steps, s0 + per);
    // CH steps of 32 k at a time, every load of a chunk issued before its
    // products (K = 1024: the wave's whole quarter in one chunk)
    constexpr int CH = 8;
    for (int base = s0; base < s1; base += CH) {
        u32x4_t b[CH], a[CH][MT];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int kk = min(base + j, s1 - 1) * 32;
            b[j] = *reinterpret_cast<const u32x4_t *>(wrow + kk);
#pragma unroll
            for (int t = 0; t < MT; ++t) a[j][t] = *reinterpret_cast<const u32x4_t *>(xrow[t] + kk);
        }
        // (the scheduler would interleave loads and products to save
        // registers, leaving 2 or 3 loads in flight; the latency is the cost)
        __builtin_amdgcn_sched_barrier(0);
        // steps past the range multiply a zero weight fragment: the products
        // stay unconditional, so no load is sunk behind a branch
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            if (base + j >= s1) b[j] = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
            for (int t = 0; t < MT; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a[j][t]),
                                                                __builtin_bit_cast(bf16x8_t, b[j]), acc[t], 0, 0, 0);
        }
    }
    // partial tiles to LDS as [tile][row][column]; then every thread adds the
    // four quarters of its outputs in wave order
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[wave][t * 256 + (4 * kg + i) * 16 + col] = acc[t][i];
    bcol[lane % 16] = bc;  // (every wave writes the same 16 values)
    __syncthreads();
    for (int o = int(threadIdx.x); o < MT * 256; o += kSkinnyWaves * kWave) {
        float sum = 0.f;
#pragma unroll
        for (int q = 0; q < kSkinnyWaves; ++q) sum += part[q][o];
        const int row = (o / 256) * 16 + (o % 256) / 16, cn = int(blockIdx.x) * 16 + o % 16;
        if (row < m && cn < n) y[int64_t(row) * n + cn] = from_f32<bf16_t>(sum + bcol[o % 16]);
    }
}

int launch_skinny(const bdm_gemv_args &a, hipStream_t s) {
    const auto *x = static_cast<const bf16_t *>(a.x);
    const auto *w = static_cast<const bf16_t *>(a.weight);
    const auto *bias = static_cast<const bf16_t *>(a.bias);
    auto *y = static_cast<bf16_t *>(a.y);
    const int m = int(a.rows), n = int(a.n), k = int(a.k);
    const unsigned grid = unsigned((a.n + 15) / 16);
    const int threads = kSkinnyWaves * kWave;
    if (m <= 16)
        skinny_gemm_kernel<1><<<grid, threads, 0, s>>>(x, w, bias, y, m, n, k);
    else if (m <= 32)
        skinny_gemm_kernel<2><<<grid, threads, 0, s>>>(x, w, bias, y, m, n, k);
    else
        skinny_gemm_kernel<4><<<grid, threads, 0, s>>>(x, w, bias, y, m, n, k);
    return check_launch("skinny_gemm_kernel");
}

template <typename T>
int launch_gemv(const bdm_gemv_args &a, hipStream_t s) {
    GemvParams<T> p{};
    p.x = static_cast<const T *>(a.x);
    p.w = static_cast<const T *>(a.weight);
    p.bias = static_cast<const T *>(a.bias);
    p.y = static_cast<T *>(a.y);
    p.residual = static_cast<const T *>(a.residual);
    p.sum_out = static_cast<T *>(a.sum_out);
    p.norm_w = a.norm_weight;
    p.norm_b = a.norm_bias;
    p.gate = static_cast<const T *>(a.gate);
    p.n = a.n;
    p.gate_stride = a.gate_stride;
    p.k = int(a.k);
    p.param_dtype = a.param_dtype;
    p.eps = a.eps;
    switch (a.prologue) {
        case BDM_GEMV_PLAIN: return launch_gemv_pro<T, kPlain>(p, a.rows, s);
        case BDM_GEMV_RMS: return launch_gemv_pro<T, kRms>(p, a.rows, s);
        case BDM_GEMV_SWIGLU: return launch_gemv_pro<T, kSwiglu>(p, a.rows, s);
        case BDM_GEMV_OUT_LAYER: return launch_gemv_pro<T, kOutLayer>(p, a.rows, s);
        case BDM_GEMV_OUT_RMS: return launch_gemv_pro<T, kOutRms>(p, a.rows, s);
        default: return fail(BDM_ERR_INVALID, "gemv: prologue %d", a.prologue);
    }
}

}  // namespace
}  // namespace bdm

extern "C" int bdm_gemv_ex(const bdm_gemv_args *a, void *stream) {
    using namespace bdm;
    if (!a) return fail(BDM_ERR_INVALID, "gemv: null args");
    if (a->rows <= 0 || a->n <= 0 || a->k <= 0 || a->k % 8 != 0) return fail(BDM_ERR_INVALID, "gemv: bad geometry");
    if (a->k > INT32_MAX / 2) return fail(BDM_ERR_UNSUPPORTED, "gemv: K too large");
    if (a->dtype != BDM_BF16 && a->dtype != BDM_F32) return fail(BDM_ERR_INVALID, "gemv: dtype");
    if (!a->x || !a->weight || !a->y) return fail(BDM_ERR_INVALID, "gemv: null pointer");
    const bool norm = a->prologue == BDM_GEMV_RMS || a->prologue == BDM_GEMV_OUT_LAYER ||
                      a->prologue == BDM_GEMV_OUT_RMS;
    if (norm && a->param_dtype != BDM_BF16 && a->param_dtype != BDM_F32)
        return fail(BDM_ERR_INVALID, "gemv: norm parameter dtype");
    if (norm && !a->norm_weight) return fail(BDM_ERR_INVALID, "gemv: the prologue needs its norm weight");
    if (a->prologue == BDM_GEMV_RMS && a->residual && !a->sum_out)
        return fail(BDM_ERR_INVALID, "gemv: a residual needs sum_out");
    if (a->prologue == BDM_GEMV_OUT_LAYER && !a->norm_bias) return fail(BDM_ERR_INVALID, "gemv: layer norm bias");
    if ((a->prologue == BDM_GEMV_OUT_LAYER || a->prologue == BDM_GEMV_OUT_RMS) &&
        (!a->gate || a->gate_stride < a->k || a->gate_stride % 8 != 0))
        return fail(BDM_ERR_INVALID, "gemv: the output prologue needs gate rows of at least K (stride % 8 == 0)");
    const void *ptrs[] = {a->x, a->weight, a->residual, a->sum_out, a->norm_weight, a->norm_bias, a->gate};
    for (const void *ptr : ptrs)
        if (ptr && !aligned(ptr, 16)) return fail(BDM_ERR_INVALID, "gemv: operands must be 16-byte aligned");
    if ((a->n + 3) / 4 > int64_t(UINT32_MAX)) return fail(BDM_ERR_UNSUPPORTED, "gemv: too many rows");
    hipStream_t s = as_stream(stream);
    if (a->rows > 4) {
        // a decode batch: matrix-core tiles (BF16, no prologue, K a multiple of 32)
        if (a->dtype != BDM_BF16 || a->prologue != BDM_GEMV_PLAIN || a->rows > kSkinnyMaxRows || a->k % 32 != 0 ||
            a->n > INT32_MAX || (a->bias && !aligned(a->bias, 2)))
            return fail(BDM_ERR_UNSUPPORTED, "gemv: %lld rows take BF16 operands without a prologue, K %% 32 == 0 and "
                                             "at most %d rows", (long long)a->rows, kSkinnyMaxRows);
        return launch_skinny(*a, s);
    }
    if (a->dtype == BDM_BF16) return launch_gemv<bf16_t>(*a, s);
    return launch_gemv<float>(*a, s);
}

extern "C" int bdm_gemv(const void *x, const void *weight, const void *bias, void *y, int64_t rows, int64_t n,
                        int64_t k, int32_t dtype, void *stream) {
    bdm_gemv_args a{};
    a.x = x;
    a.weight = weight;
    a.bias = bias;
    a.y = y;
    a.rows = rows;
    a.n = n;
    a.k = k;
    a.dtype = dtype;
    a.param_dtype = BDM_F32;
    a.prologue = BDM_GEMV_PLAIN;
    return bdm_gemv_ex(&a, stream);
}

// Routed GDN2 forward on matrix cores: S = 8, state rounded to BF16 every 16
// packed events.
//
// Reference semantics: _role_forward with ROUND_STATE (role_bank_kernel.py:
// 32-73, chunk 16 for S = 8, :153-165), which the module forward runs per head
// at H > 1 with training_state_dtype='bfloat16' (heads.py:40-46); packing and
// the decay transform as in _pack (role_bank_dispatch.py:41-73) and
// decay_transform (routed_update.py:5-13).  Per (segment, head), events in
// packed order on an 8 x v FP32 state M:
//   write (weight p): hd = diag(exp(g p)) M;  u = bf(w p) v - (bf(b p) k)^T hd;
//                     M = hd + k u^T
//   read  (weight r): z = scale * bf(q r)^T M
// and M is rounded to BF16 at the segment start and before every event whose
// offset in the segment is a positive multiple of 16.
//
// Chunked form.  The segment runs in chunks of 16 events, so every chunk
// starts from a state M0 that is exact in BF16.  Within a chunk the end state
// and every read are linear in M0 and in the gated values x_j = bf(w p_j) v_j
// of the chunk's writes:
//     [M_end; z_1 .. z_R] = Phi M0 + Psi [x_1; ..; x_W]
// Phi ((8 + R) x 8) and Psi ((8 + R) x W) depend on the chunk's keys, decays
// and gates only, not on the value columns.  They are computed by running the
// recurrence itself on a 24-column basis (the 8 rows of M0 and the W <= 16
// write values; 4 rows per lane, the erase sum over rows completed across the
// half-waves).  The value columns then cost 4 + ceil(W / 2)
// v_mfma_f32_32x32x2_f32 per 32 columns, K = 8 + W in steps of 2:
//     steps 0..3:   Phi . M0          (basis rows 0..7)
//     steps 4..11:  Psi . [x_1; ..]   (basis row 8 + j: write j)
// all in FP32: Phi and Psi are the FP32 coefficients themselves, M0 is exact
// in BF16, and x = bf(w p) v, a product of two BF16 values, is exact in FP32,
// so every product is formed and accumulated at FP32 precision, as the
// sequential form's FMAs are (only the order of the sums differs).  A form
// on BF16 matrix cores with two-part (high/low BF16) coefficients was
// measured first: their relative error of ~2^-16 flipped the BF16 roundings
// of the state and of the read fold often enough to leave tokens 1.08 % off
// the oracle at the full C2 size.
//
// Accumulator layout of a 32 x 32 tile (lane l, value i): row 8(i/4) +
// 4(l/32) + i%4, column l%32.  Rows are assigned so that every lane's values
// 0..7 are the 8 state rows of its column (tile rows 0-3, 8-11 are state rows
// 0-7 and rows 4-7, 12-15 repeat them for the upper half-wave) and values
// 8..15 are reads (0-7 in the lower half-wave, 8-15 in the upper).  A step's
// operands: lane l gives A[row l%32][k = 2 step + l/32] and B[k][column
// l%32], so the next chunk's state rows come from the lane's own values 0..7
// (rounded to BF16): no data crosses lanes between chunks.  Column n of tile
// t is value column TILES*n + t, so a lane owns TILES adjacent columns and
// moves them with one vector access.

#include "chunk_forward.h"

namespace bdm {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kChunk = 16;    // events per chunk: the rounding interval
constexpr int kBasis = 24;    // coefficient columns: M0 rows 0-7, even writes, odd writes
constexpr int kGStride = 28;  // floats per coefficient row in LDS (16-byte aligned rows)

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// a(l) + a(l ^ 32): v_permlane32_swap exchanges the half-waves.
__device__ __forceinline__ float half_wave_sum(float a) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// TILES adjacent BF16 columns in 32-bit words.
template <int TILES>
struct ColWords {
    static_assert(TILES == 2 || TILES == 4 || TILES == 8, "tiles");
    uint32_t u[TILES / 2];
    __device__ __forceinline__ void load(const bf16_t *p) {
        if constexpr (TILES == 2) {
            u[0] = *reinterpret_cast<const uint32_t *>(p);
        } else if constexpr (TILES == 4) {
            const uint2 x = *reinterpret_cast<const uint2 *>(p);
            u[0] = x.x;
            u[1] = x.y;
        } else {
            const uint4 x = *reinterpret_cast<const uint4 *>(p);
            u[0] = x.x;
            u[1] = x.y;
            u[2] = x.z;
            u[3] = x.w;
        }
    }
    __device__ __forceinline__ float at(int t) const { return (t & 1) ? bf16_hi(u[t / 2]) : bf16_lo(u[t / 2]); }
};

// Row g of the chunk's coefficient matrix that tile row m holds: rows 0..7
// are the state rows, 8 + i read i.
__device__ __forceinline__ int coefficient_row(int m) {
    if (m < 16) return (m & 3) + (((m >> 3) & 1) << 2);
    const int mm = m - 16;
    return 8 + (mm & 3) + (((mm >> 3) & 1) << 2) + (((mm >> 2) & 1) << 3);
}

// Token of a route: routes are token * K + j.
__device__ __forceinline__ int route_token(int route, int k, int kshift) {
    return kshift >= 0 ? route >> kshift : route / k;
}

template <int TILES>
__global__ __launch_bounds__(64) void chunk_forward_kernel(ChunkForwardParams p) {
    __shared__ __attribute__((aligned(16))) float s_prm[kChunk][3][8];  // write: a, k, d; read: [0] gamma
    __shared__ __attribute__((aligned(16))) float s_g[8 + kChunk][kGStride];
    __shared__ int s_wrow[kChunk];   // element offset of write j's v and w rows (this head)
    __shared__ float s_wp[kChunk];   // route weight of write j
    __shared__ int s_zrow[kChunk];   // read buffer row of read i

    const int lane = int(threadIdx.x);
    const int c32 = lane & 31, half = lane >> 5;
    const int block = int(blockIdx.x);
    const int seg = p.xcd_remap ? (block % 8) * (p.nseg / 8) + block / 8 : block;
    const int head = int(blockIdx.y);
    const int rhead = head / p.split;
    const int bank = seg % p.banks;
    const int64_t bidx = seg / p.banks;
    const int64_t start = p.cu[seg], end = p.cu[seg + 1];
    const int nchunks = int((end - start + kChunk - 1) / kChunk);
    const int write_events = int(p.nt * p.kw);
    const int col0 = TILES * c32;
    const int64_t vcol = int64_t(head % p.split) * p.width + col0;  // this lane's columns in a real-head row
    const int64_t head_cols = int64_t(rhead) * 8 * p.row_stride + vcol;
    const int64_t state_offset = int64_t(bank) * p.s_heads * 8 * p.row_stride + head_cols;
    const int64_t hw = int64_t(p.heads) * p.width;
    const int64_t zcol = int64_t(head) * p.width + col0;
    const int vrow = p.s_heads * int(p.row_stride);  // elements of one token's v or w row
    const int vhead = rhead * int(p.row_stride);

    // The state, in accumulator values 0..7 of every tile, rounded to BF16
    // (the segment start is a rounding point).
    f32x16_t acc[TILES];
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[t][i] = 0.f;
    {
        const int64_t off = bidx * p.init_bstride + state_offset;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            float row[TILES];
            if (p.init_dtype == BDM_BF16)
                load_row<TILES>(static_cast<const bf16_t *>(p.initial) + off + int64_t(r) * p.row_stride, row);
            else
                load_row<TILES>(static_cast<const float *>(p.initial) + off + int64_t(r) * p.row_stride, row);
#pragma unroll
            for (int t = 0; t < TILES; ++t) acc[t][r] = round_bf16(row[t]);
        }
    }

#pragma unroll 1
    for (int ch = 0; ch < nchunks; ++ch) {
        const int64_t e0 = start + int64_t(ch) * kChunk;
        const int n = int(min(int64_t(kChunk), end - e0));

        // ---- metadata: lane e < n holds event e of the chunk
        int o = 0;
        if (lane < n) o = int(p.order[e0 + lane]);
        const bool live = lane < n;
        const bool rd = live && o >= write_events;
        const uint32_t rmask = uint32_t(__ballot(rd));
        const uint32_t wmask = uint32_t(__ballot(live && !rd));
        const int nr = __popc(rmask), nw = __popc(wmask);
        if (live) {
            const uint32_t below = (1u << lane) - 1u;
            if (rd) {
                const int route = o - write_events;
                s_zrow[__popc(rmask & below)] = route;  // a read's row of zbuf: its route
            } else {
                const int j = __popc(wmask & below);
                s_wrow[j] = route_token(o, p.kw, p.kw_shift) * vrow + vhead;
                s_wp[j] = to_f32(p.ww[o]);
            }
        }
        // ---- row operands: lane (event e, rows 2rp, 2rp + 1)
        {
            const int e = lane & 15, rp = lane >> 4;
            const int oe = __shfl(o, e);
            if (e < n) {
                const bool erd = oe >= write_events;
                const int route = erd ? oe - write_events : oe;
                const int tok = erd ? route_token(route, p.kr, p.kr_shift) : route_token(route, p.kw, p.kw_shift);
                const int64_t row = (int64_t(tok) * p.s_heads + rhead) * 8 + 2 * rp;
                if (erd) {
                    const uint32_t qq = *reinterpret_cast<const uint32_t *>(p.q + row);
                    const float r = to_f32(p.rw[route]);
                    s_prm[e][0][2 * rp] = p.scale * round_bf16(bf16_lo(qq) * r);
                    s_prm[e][0][2 * rp + 1] = p.scale * round_bf16(bf16_hi(qq) * r);
                } else {
                    const uint32_t kk = *reinterpret_cast<const uint32_t *>(p.k + row);
                    const uint32_t bb = *reinterpret_cast<const uint32_t *>(p.b + row);
                    const float2 gg = *reinterpret_cast<const float2 *>(p.g + row);
                    const float pw = to_f32(p.ww[route]);
                    const float k0 = bf16_lo(kk), k1 = bf16_hi(kk);
                    s_prm[e][0][2 * rp] = round_bf16(bf16_lo(bb) * pw) * k0;
                    s_prm[e][0][2 * rp + 1] = round_bf16(bf16_hi(bb) * pw) * k1;
                    s_prm[e][1][2 * rp] = k0;
                    s_prm[e][1][2 * rp + 1] = k1;
                    s_prm[e][2][2 * rp] = __expf(p.routed_decay ? gg.x * pw : gg.x);
                    s_prm[e][2][2 * rp + 1] = __expf(p.routed_decay ? gg.y * pw : gg.y);
                }
            }
        }
        __syncthreads();

        // ---- this lane's writes: slot s holds write 2s + half, the B operand
        //      of step 4 + s in this half-wave
        ColWords<TILES> vraw[8], wraw[8];
        float wp[8];
        const int nslots = (nw + 1) >> 1;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int j = 2 * s + half;
            wp[s] = 0.f;
            if (s < nslots && j < nw) {
                const int base = s_wrow[j] + int(vcol);
                vraw[s].load(p.v + base);
                wraw[s].load(p.w + base);
                wp[s] = s_wp[j];
            } else {
#pragma unroll
                for (int i = 0; i < TILES / 2; ++i) vraw[s].u[i] = wraw[s].u[i] = 0u;
            }
        }

        // ---- coefficients: the recurrence on the basis [M0 rows | writes],
        //      lane (column c32, rows 4 half .. 4 half + 3)
        {
            float nrow[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) nrow[r] = (c32 == 4 * half + r) ? 1.f : 0.f;
            int wj = 0, ri = 0;
#pragma unroll 1
            for (int e = 0; e < n; ++e) {
                if ((rmask >> e) & 1u) {
                    const float4 gm = *reinterpret_cast<const float4 *>(&s_prm[e][0][4 * half]);
                    float part = gm.x * nrow[0];
                    part = fmaf(gm.y, nrow[1], part);
                    part = fmaf(gm.z, nrow[2], part);
                    part = fmaf(gm.w, nrow[3], part);
                    const float tot = half_wave_sum(part);
                    if (half == 0 && c32 < kBasis) s_g[8 + ri][c32] = tot;
                    ++ri;
                } else {
                    const float4 a4 = *reinterpret_cast<const float4 *>(&s_prm[e][0][4 * half]);
                    const float4 k4 = *reinterpret_cast<const float4 *>(&s_prm[e][1][4 * half]);
                    const float4 d4 = *reinterpret_cast<const float4 *>(&s_prm[e][2][4 * half]);
                    const float hd0 = d4.x * nrow[0], hd1 = d4.y * nrow[1], hd2 = d4.z * nrow[2],
                                hd3 = d4.w * nrow[3];
                    float part = a4.x * hd0;
                    part = fmaf(a4.y, hd1, part);
                    part = fmaf(a4.z, hd2, part);
                    part = fmaf(a4.w, hd3, part);
                    const float tot = half_wave_sum(part);
                    const int col = 8 + wj;
                    const float u = (c32 == col ? 1.f : 0.f) - tot;
                    nrow[0] = fmaf(k4.x, u, hd0);
                    nrow[1] = fmaf(k4.y, u, hd1);
                    nrow[2] = fmaf(k4.z, u, hd2);
                    nrow[3] = fmaf(k4.w, u, hd3);
                    ++wj;
                }
            }
            if (c32 < kBasis) {
#pragma unroll
                for (int r = 0; r < 4; ++r) s_g[4 * half + r][c32] = nrow[r];
            }
        }
        __syncthreads();

        // ---- A operands: lane (tile row m = c32, K half): coefficient row
        //      coefficient_row(m), basis column 2 step + half, for the four
        //      state steps and the live write steps (0 in rows past the reads)
        float a_op[12];
        {
            const int gr = coefficient_row(c32);
            const bool row_live = c32 < 16 || gr - 8 < nr;
#pragma unroll
            for (int st = 0; st < 12; ++st) a_op[st] = row_live ? s_g[gr][2 * st + half] : 0.f;
        }

        // ---- B operands and the products, one 32-column tile at a time
        const bool snap = p.snap && ch > 0;
        const int64_t snap_offset = (start / kChunk + ch - 1) * p.s_heads * 8 * p.row_stride + head_cols;
#pragma unroll
        for (int t = 0; t < TILES; ++t) {
            // the chunk's start state, rounded to BF16 (a rounding point)
            float m0[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) m0[r] = round_bf16(acc[t][r]);
            if (snap) {
                // the state at this chunk's start, as rounded (a replay boundary)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int rr = 4 * half + r;
                    reinterpret_cast<uint16_t *>(p.snap)[snap_offset + int64_t(rr) * p.row_stride + t] =
                        uint16_t(__float_as_uint(m0[rr]) >> 16);
                }
            }
            f32x16_t d;
#pragma unroll
            for (int i = 0; i < 16; ++i) d[i] = 0.f;
            // state row 2 st + half: a bit-mask select (a plain select of two
            // array slots becomes a per-lane index into a scratch copy)
            const uint32_t upper = half ? ~0u : 0u;
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const uint32_t b = (__float_as_uint(m0[2 * st + 1]) & upper) | (__float_as_uint(m0[2 * st]) & ~upper);
                d = __builtin_amdgcn_mfma_f32_32x32x2f32(a_op[st], __uint_as_float(b), d, 0, 0, 0);
            }
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                if (s < nslots) {  // wave-uniform
                    const float x = round_bf16(wraw[s].at(t) * wp[s]) * vraw[s].at(t);
                    d = __builtin_amdgcn_mfma_f32_32x32x2f32(a_op[4 + s], x, d, 0, 0, 0);
                }
            }
            acc[t] = d;
        }

        // ---- the chunk's reads: values 8..15, read s + 8 half
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int i = s + 8 * half;
            if (i < nr) {
                float z[TILES];
#pragma unroll
                for (int t = 0; t < TILES; ++t) z[t] = acc[t][8 + s];
                store_row<TILES>(p.zbuf + int64_t(s_zrow[i]) * hw + zcol, z);
            }
        }
        __syncthreads();  // the chunk's LDS tables are rewritten by the next one
    }

    if (p.final_state) {
        const int64_t off = bidx * (int64_t(p.banks) * p.s_heads * 8 * p.row_stride) + state_offset;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rr = 4 * half + r;
            float row[TILES];
#pragma unroll
            for (int t = 0; t < TILES; ++t) row[t] = acc[t][rr];
            if (p.final_dtype == BDM_BF16)
                store_row<TILES>(static_cast<bf16_t *>(p.final_state) + off + int64_t(rr) * p.row_stride, row);
            else
                store_row<TILES>(static_cast<float *>(p.final_state) + off + int64_t(rr) * p.row_stride, row);
        }
    }
}

}  // namespace

// Matrix-core path: S = 8, BF16 controllers, the state rounded every 16
// events (snapshots, when asked, at the same boundaries in BF16), heads (or
// 128-column virtual heads of wider ones) of 64, 128 or 256 columns, 16-byte
// aligned rows, and event indices in 32 bits.
bool chunk_path(const bdm_forward_args &a) {
    if (a.ctrl_dtype != BDM_BF16 || a.bank_size != 8 || a.round_interval != kChunk) return false;
    if (a.snapshots && (a.snapshot_interval != kChunk || a.snapshot_dtype != BDM_BF16)) return false;
    const int w = a.head_width;
    if (!(w == 64 || w == 128 || w == 256 || (w > 256 && w % 128 == 0))) return false;
    if (a.initial_batch_stride % 8 != 0) return false;
    const int64_t events = a.batch * a.time * (int64_t(a.write_banks) + a.read_banks);
    // value rows are addressed with 32-bit element offsets
    const int64_t value_elements = a.batch * a.time * int64_t(a.heads) * a.head_width;
    return events < INT32_MAX && a.batch * a.bank_count <= INT32_MAX && value_elements < INT32_MAX;
}

int launch_chunk_forward(const ChunkForwardParams &p, int tiles, hipStream_t stream) {
    const dim3 grid(unsigned(p.nseg), unsigned(p.heads));
    switch (tiles) {
        case 2: chunk_forward_kernel<2><<<grid, 64, 0, stream>>>(p); break;
        case 4: chunk_forward_kernel<4><<<grid, 64, 0, stream>>>(p); break;
        case 8: chunk_forward_kernel<8><<<grid, 64, 0, stream>>>(p); break;
        default: return fail(BDM_ERR_UNSUPPORTED, "chunk forward: %d tiles", tiles);
    }
    return check_launch("chunk_forward_kernel");
}

}  // namespace bdm

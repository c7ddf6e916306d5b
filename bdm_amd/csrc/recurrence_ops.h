// Per-event operand preparation and the write update of the routed GDN2
// recurrence, shared by the forward kernel and the backward replay so both
// execute the identical FP32 operation sequence (the backward replays the
// forward trajectory exactly from its snapshots).
//
// Reference: _pack (role_bank_dispatch.py:47-73: eb = b*p and ew = w*p rounded
// to the source dtype once), decay_transform (routed_update.py:5-13: eg = g*p
// in FP32) and _write (role_bank_kernel.py:35-43):
//   hd = diag(exp(eg)) M;  a = eb * k;  u = ew * v - a^T hd;  M' = hd + k u^T
#pragma once

#include "bdm_common.h"

namespace bdm {

// Row-side operands of one write event (one token, one head).
template <int S>
struct WriteRows {
    float key[S];    // k
    float decay[S];  // exp(eg)
    float eb[S];     // bf(b*p)
    float a[S];      // eb * k
};

// eg = g*p (routed decay) or g; eb = bf(b*p) in the controller dtype T.
template <typename T, int S>
__device__ __forceinline__ void prepare_write_rows(const float (&k)[S], const float (&g)[S], const float (&b)[S],
                                                   float pw, bool routed_decay, WriteRows<S> &w) {
#pragma unroll
    for (int r = 0; r < S; ++r) {
        const float eg = routed_decay ? g[r] * pw : g[r];
        w.key[r] = k[r];
        w.decay[r] = __expf(eg);
        w.eb[r] = round_to<T>(b[r] * pw);
        w.a[r] = w.eb[r] * k[r];
    }
}

// Apply one write to the CPL columns a lane owns.  ew = bf(w*p) per column.
template <int S, int CPL>
__device__ __forceinline__ void apply_write(float (&h)[S][CPL], const WriteRows<S> &w, const float (&ew)[CPL],
                                            const float (&value)[CPL]) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        float erase = 0.f;
#pragma unroll
        for (int r = 0; r < S; ++r) {
            h[r][c] *= w.decay[r];
            erase = fmaf(w.a[r], h[r][c], erase);
        }
        const float u = fmaf(ew[c], value[c], -erase);
#pragma unroll
        for (int r = 0; r < S; ++r) h[r][c] = fmaf(w.key[r], u, h[r][c]);
    }
}

}  // namespace bdm

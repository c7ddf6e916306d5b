/*
 * bdm_hip.h — C ABI of the MI355X (gfx950) routed-memory path of the BDM layer.
 *
 * Every entry point takes device pointers, element counts and a HIP stream
 * (passed as void *, a hipStream_t; NULL is the default stream), enqueues its
 * kernels on that stream and returns without synchronising the host.  No
 * entry point allocates device memory: scratch space is passed in as a
 * workspace whose size the matching *_workspace_size function reports.
 *
 * Return value: BDM_OK (0) on success, a negative BDM_ERR_* code otherwise;
 * bdm_last_error_string() then describes the failure (per calling thread).
 *
 * Layouts are token-major with token = batch_index * time + t, matching the
 * reference tensors [batch, time, ...] in row-major order.
 */
#ifndef BDM_HIP_H
#define BDM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum bdm_dtype { BDM_F32 = 0, BDM_BF16 = 1 };

enum bdm_status {
    BDM_OK = 0,
    BDM_ERR_INVALID = -1,     /* bad pointer, shape or dtype */
    BDM_ERR_UNSUPPORTED = -2, /* geometry outside what the kernels implement */
    BDM_ERR_WORKSPACE = -3,   /* workspace missing or too small */
    BDM_ERR_LAUNCH = -4       /* the HIP runtime rejected a launch */
};

/* Bits of the int32 status word that bdm_dispatch_build can raise on device. */
enum bdm_route_flags {
    BDM_ROUTE_OUT_OF_RANGE = 1, /* a bank index outside [0, bank_count) (clamped) */
    BDM_ROUTE_DUPLICATE = 2     /* one token selected the same bank twice in one role */
};

int bdm_version(void);
const char *bdm_last_error_string(void);

/*
 * Product-key router.  Replaces product_key_route
 * (implementation/bdm/gdn2_banks.py:74-114, including the batch_factors
 * variant at :93-102, whose selection is identical).
 *
 * scores   [rows, row_stride] of score_dtype; columns [0, J1) are the first
 *          factor and [J1, J1+J2) the second, J1*J2 = bank_count.
 * weights  [rows, C] of score_dtype: softmax (FP32) of the selected pair
 *          sums, cast to score_dtype.  C = min(selected, s*s) with
 *          s = min(selected, J1, J2) (gdn2_banks.py:92,107); C = selected
 *          whenever selected <= min(J1, J2), as BDMConfig requires.
 * indices  [rows, C] int64: row*J2 + col, in descending pair-sum order.
 * Pair sums are rounded to score_dtype.  Equal values keep the lower index
 * first (stable descending order), both within a factor and among pairs.
 */
int bdm_router_select(const void *scores, int32_t score_dtype, int64_t rows, int64_t row_stride,
                      int32_t factor_first, int32_t factor_second, int32_t selected,
                      void *weights, int64_t *indices, void *stream);
/* Two routers of one geometry in one launch (a layer's write and read roles,
 * `_route(write_routes, num_writes)` and `_route(read_routes, num_reads)`,
 * implementation/bdm/model.py:96-97): the results of two bdm_router_select
 * calls, role a to weights_a/indices_a and role b to weights_b/indices_b. */
int bdm_router_select_pair(const void *scores_a, int64_t row_stride_a, const void *scores_b, int64_t row_stride_b,
                           int32_t score_dtype, int64_t rows, int32_t factor_first, int32_t factor_second,
                           int32_t selected, void *weights_a, int64_t *indices_a, void *weights_b,
                           int64_t *indices_b, void *stream);

/*
 * Causal bank dispatch.  Replaces metadata + the INVERSE/TOKENS outputs of
 * _pack (implementation/bdm/role_bank_dispatch.py:143-153, :15-38, :72-73).
 *
 * Events in original order are the writes (token*KW + j) followed by the reads
 * (NT*KW + token*KR + j), NT = batch*time.  They are bucketed by segment
 * (batch*bank_count + bank), stably, so a segment lists its events in
 * (time, write-before-read) order: the permutation that sorts the reference
 * keys ((b*J + bank)*T + t)*2 + is_read.
 *
 * order      [E] int64  original event index of each packed slot
 * inverse    [E] int64  packed slot of each original event
 * tokens     [E] int64  token of each packed slot
 * cu_seqlens [batch*bank_count + 1] int64  segment bounds
 * status     one int32 on device: cleared by the call, then OR-ed with
 *            bdm_route_flags (the caller need not clear it)
 * E = NT*(KW+KR) < 2^31.  bank_count <= 8192 runs the LDS-mask counting sort;
 * larger bank counts radix-sort the keys (same permutation).
 */
size_t bdm_dispatch_workspace_size(int64_t batch, int64_t time, int32_t bank_count);
/* Workspace of bdm_dispatch_build for any bank_count: the bucket counts of
 * the LDS-mask path for bank_count <= 8192 (bdm_dispatch_workspace_size,
 * which returns 0 above that), else the radix-sort path's keys, values and
 * sort scratch. */
size_t bdm_dispatch_workspace_size_ex(int64_t batch, int64_t time, int32_t bank_count, int32_t write_banks,
                                      int32_t read_banks);
int bdm_dispatch_build(const int64_t *write_indices, const int64_t *read_indices, int64_t batch,
                       int64_t time, int32_t write_banks, int32_t read_banks, int32_t bank_count,
                       int64_t *order, int64_t *inverse, int64_t *tokens, int64_t *cu_seqlens,
                       int32_t *status, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Both routers and the dispatch of one layer step in one call: the results of
 * bdm_router_select_pair (write role to write_*, read role to read_*, the
 * selected count per role) followed by bdm_dispatch_build on those routes
 * (model.py:96-97 routing, then role_bank_dispatch.py:143-153).  Where the
 * geometry allows (BF16 scores, 8 banks per role from factors of 8..32, the
 * alignment of bdm_router_select_pair's two-lanes-per-row kernel) the routing
 * launch also counts the dispatch tiles.  inverse and tokens may be NULL (not
 * stored; bdm_forward and bdm_backward do not read them).
 * segment_order: NULL, or [batch*bank_count] int32 receiving the longest-first
 * order bdm_forward would compute itself (pass it in bdm_forward_args); it is
 * written where that order applies (batch*bank_count a multiple of 8, ranges
 * of at most 1024 segments).
 */
typedef struct bdm_route_dispatch_args {
    const void *write_scores;  /* [rows, write_stride] score_dtype, rows = batch*time */
    int64_t write_stride;
    const void *read_scores;   /* [rows, read_stride] */
    int64_t read_stride;
    int32_t score_dtype;
    int64_t batch, time;
    int32_t factor_first, factor_second, selected;
    void *write_weights;       /* [rows, selected] score_dtype */
    int64_t *write_indices;    /* [rows, selected] */
    void *read_weights;
    int64_t *read_indices;
    int64_t *order, *inverse, *tokens, *cu_seqlens;
    int32_t *status;
    int32_t *segment_order;
} bdm_route_dispatch_args;
size_t bdm_route_dispatch_workspace_size(const bdm_route_dispatch_args *args);
int bdm_route_dispatch(const bdm_route_dispatch_args *args, void *workspace, size_t workspace_bytes, void *stream);

/*
 * bdm_dispatch_build without a workspace, for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  It has no counterpart in the reference.  Same arguments,
 * outputs and errors as bdm_dispatch_build, minus the workspace; it allocates
 * nothing and calls no allocating routine.  Its scratch is a static device
 * buffer of BDM_DISPATCH_STATIC_SCRATCH_BYTES per GPU (held until the process
 * ends), so it takes the LDS-mask path only: bank_count <= 8192 and
 * bdm_dispatch_workspace_size(batch, time, bank_count) <= that size (C2:
 * 1.06 MB, C4: 8.4 MB); larger geometries return BDM_ERR_UNSUPPORTED with a
 * message.  Every call on one GPU shares that buffer: calls that overlap on
 * one GPU (concurrent streams or threads) race and must be serialised by the
 * caller.
 */
#define BDM_DISPATCH_STATIC_SCRATCH_BYTES (16u << 20)
int bdm_dispatch_build_static(const int64_t *write_indices, const int64_t *read_indices, int64_t batch,
                              int64_t time, int32_t write_banks, int32_t read_banks, int32_t bank_count,
                              int64_t *order, int64_t *inverse, int64_t *tokens, int64_t *cu_seqlens,
                              int32_t *status, void *stream);

/*
 * Routed GDN2 bank recurrence with the r-weighted read combine.  Replaces, for
 * all heads at once: pack (role_bank_dispatch.py:156-185), decay_transform
 * (routed_update.py:5-13), _role_forward (role_bank_kernel.py:46-73, and the
 * stateful forward_rows variants, forward_rows.py:10-194), _readout
 * (role_bank_dispatch.py:201-231) and _compact_readout (inference.py:70-85).
 *
 * Per segment and head, events in packed order on an S x v FP32 state M:
 *   write (route weight p):  hd = diag(exp(eg)) M,  eg = g*p (routed_decay) or g
 *                            u  = bf(w*p) * v - (bf(b*p) * k)^T hd
 *                            M  = hd + k u^T
 *   read  (route weight r):  z  = scale * bf(q*r)^T M, stored in ctrl_dtype
 * bf() rounds to ctrl_dtype.  With round_interval > 0 the state is rounded to
 * BF16 at the segment start and before every event whose in-segment offset is
 * a positive multiple of round_interval (the training path's storage cadence).
 * y[token, h*v + c] adds the token's reads in increasing bank id, rounding to
 * ctrl_dtype after each add.
 *
 * Snapshots for the backward (role_bank_kernel.py:57-66): when `snapshots` is
 * not NULL the state before every event whose in-segment offset is a positive
 * multiple of snapshot_interval (after the rounding above, which must then use
 * the same interval) is stored at row (packed position / interval - 1) of
 * snapshots [bdm_snapshot_rows(E, interval), H, S, v] in snapshot_dtype.
 * Rows that no boundary maps to are left untouched.
 */
typedef struct bdm_forward_args {
    const void *q;             /* [NT, H, S] ctrl_dtype */
    const void *k;             /* [NT, H, S] ctrl_dtype */
    const float *g;            /* [NT, H, S] FP32 log decay */
    const void *b;             /* [NT, H, S] ctrl_dtype erase gate */
    const void *v;             /* [NT, H, v] ctrl_dtype */
    const void *w;             /* [NT, H, v] ctrl_dtype write gate */
    const void *write_weights; /* [NT, KW] ctrl_dtype */
    const void *read_weights;  /* [NT, KR] ctrl_dtype */
    const int64_t *read_indices; /* [NT, KR] */
    const int64_t *order;      /* [E] from bdm_dispatch_build */
    const int64_t *cu_seqlens; /* [batch*J + 1] */
    const void *initial;       /* [J, H, S, v] (+ batch stride) of initial_dtype */
    void *final_state;         /* NULL or [batch, J, H, S, v] of final_dtype; may alias initial */
    void *output;              /* [NT, H*v] ctrl_dtype */
    int64_t initial_batch_stride; /* elements between batches of `initial`; 0 = shared */
    int64_t batch, time;
    int32_t heads, bank_size, head_width, bank_count, write_banks, read_banks;
    int32_t ctrl_dtype, initial_dtype, final_dtype;
    int32_t routed_decay;
    int32_t round_interval;
    float scale;
    void *snapshots;           /* NULL or [rows, H, S, v] of snapshot_dtype (see above) */
    int32_t snapshot_interval;
    int32_t snapshot_dtype;    /* BDM_BF16 only with round_interval == snapshot_interval */
    /* Profiling: NULL, or three hipEvent_t the call records: before the
     * recurrence kernels, after the last recurrence launch (the last head-group
     * round, whose read combine follows it; the earlier rounds' combines run
     * beside the later rounds on an auxiliary stream) and after the combine,
     * so a caller can time the recurrence and the combine left after it. */
    void *phase_events[3];
    /* NULL, or the longest-first segment order bdm_route_dispatch wrote for
     * this dispatch ([batch*J] int32); the call computes it itself otherwise. */
    const int32_t *segment_order;
} bdm_forward_args;

/* Rows of the snapshot buffer for E packed events: E / interval. */
int64_t bdm_snapshot_rows(int64_t events, int32_t interval);

size_t bdm_forward_workspace_size(const bdm_forward_args *args);
int bdm_forward(const bdm_forward_args *args, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Backward of bdm_forward.  Replaces RoutedUpdate.backward / RoleBankTraining
 * .backward (implementation/bdm/routed_update.py:31-49,
 * role_bank_kernel.py:231-256): the chunk replay and reverse adjoint of
 * _role_backward (role_bank_kernel.py:76-150) and the token-level VJP _vjp
 * (role_bank_dispatch.py:76-132), with its BF16 rounding points, plus the
 * routed-decay term of d(ww) (routed_update.py:43-47).
 *
 * Inputs are those of the forward (same layouts), its snapshots (taken with
 * snapshot_interval = C: 16 for S <= 8, 8 for S <= 16, 4 for S <= 32 — the
 * reference replay chunk, role_bank_kernel.py:153-154) and grad_output
 * [NT, H*v] in ctrl_dtype.  Outputs, token-major like the inputs:
 *   grad_q, grad_k, grad_b [NT, H, S] ctrl_dtype;  grad_g [NT, H, S] FP32;
 *   grad_v, grad_w [NT, H, v] ctrl_dtype;
 *   grad_write_weights [NT, KW], grad_read_weights [NT, KR] ctrl_dtype, the
 *     heads' contributions summed;
 *   grad_initial [batch, J, H, S, v] FP32: the adjoint of each sequence's
 *     initial bank state (sum over the batch for a shared initial state).
 * Every output element is written.  Route order within a token (j = 0..K-1)
 * is the order the reference folds the token's events in.
 */
typedef struct bdm_backward_args {
    const void *q, *k;         /* [NT, H, S] ctrl_dtype */
    const float *g;            /* [NT, H, S] */
    const void *b;             /* [NT, H, S] ctrl_dtype */
    const void *v, *w;         /* [NT, H, v] ctrl_dtype */
    const void *write_weights, *read_weights; /* [NT, KW], [NT, KR] ctrl_dtype */
    const int64_t *order, *cu_seqlens;        /* from bdm_dispatch_build */
    const void *initial;       /* as in bdm_forward_args */
    const void *snapshots;     /* written by bdm_forward */
    const void *grad_output;   /* [NT, H*v] ctrl_dtype */
    void *grad_q, *grad_k;
    float *grad_g;
    void *grad_b, *grad_v, *grad_w;
    void *grad_write_weights, *grad_read_weights;
    float *grad_initial;
    int64_t initial_batch_stride, batch, time;
    int32_t heads, bank_size, head_width, bank_count, write_banks, read_banks;
    int32_t ctrl_dtype, initial_dtype, snapshot_dtype, routed_decay, round_interval, snapshot_interval;
    float scale;
} bdm_backward_args;

/* Scratch of bdm_backward: per-event du (FP32, NT*KW*H*v), per-event S-wide
 * partials (U, X, P of each write and dq of each read, per 128-column tile)
 * and, for S = 8 with replay interval 16, a 16-byte meta entry per event; the
 * workspace must be 256-byte aligned. */
size_t bdm_backward_workspace_size(const bdm_backward_args *args);
int bdm_backward(const bdm_backward_args *args, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Single-token decode against resident bank states.  Replaces
 * _decode_write/_decode_read/_decode_sum (implementation/bdm/inference.py:21-67,
 * step at :161-194) and generalises them to any head count.
 *
 * state [batch, J, H, S, v] of state_dtype is updated in place: each of the
 * token's KW write banks is advanced by the write rule above and stored
 * (rounded to state_dtype); then each of the KR read banks is read from the
 * stored state; the reads are added in increasing bank id with a rounding to
 * ctrl_dtype after each add into output [batch, H*v].
 * The write banks of one token must be distinct (as the router guarantees).
 */
typedef struct bdm_decode_args {
    const void *q, *k, *b;     /* [batch, H, S] ctrl_dtype */
    const float *g;            /* [batch, H, S] */
    const void *v, *w;         /* [batch, H, v] ctrl_dtype */
    const void *write_weights, *read_weights; /* [batch, KW], [batch, KR] */
    const int64_t *write_indices, *read_indices;
    void *state;
    void *output;              /* [batch, H*v] ctrl_dtype */
    int64_t batch;
    int32_t heads, bank_size, head_width, bank_count, write_banks, read_banks;
    int32_t ctrl_dtype, state_dtype, routed_decay;
    float scale;
} bdm_decode_args;

int bdm_decode(const bdm_decode_args *args, void *stream);

/*
 * The decode step of the inference path from the projection outputs, in one
 * launch: the controller epilogue (bdm_controller_epilogue, heads.py:11-22),
 * both routers (bdm_router_select_pair, gdn2_banks.py:74-114) and bdm_decode
 * (inference.py:161-194).  Replaces the three calls of a step.  Given f (the
 * f pointer), every input the decode sees equals, bit for bit, what those
 * kernels would have stored; with f_weight (below) f is formed in another
 * summation order, and results match the separate kernels within tolerance.
 * proj is [batch, proj_stride] ctrl_dtype with the q, k, v, b, w slices and
 * the read and write route scores (J1 + J2 each) at the given column offsets;
 * f is the f_proj output [batch, f_stride]; a_log [H] and dt_bias [H*S] in
 * param_dtype.  The state [batch, J1*J2, H, S, v] is updated in place and y
 * [batch, H*v] written.  Geometry: BF16 controllers, S = 8, 8 banks per role
 * from J1, J2 <= 64, column offsets and strides multiples of 8 elements,
 * head_width even with spans of 48..128 columns
 * (bdm_decode_fused_supported); anything else returns BDM_ERR_UNSUPPORTED.
 * With f_weight set (f_proj's second factor [H*S, f_width] ctrl_dtype, rows
 * contiguous), f is formed in the launch from the f_proj first-factor slice
 * of proj at f_col instead of read from f: FP32 dot products in a fixed order,
 * rounded to ctrl_dtype as the GEMM output is (spans of 64..128 columns);
 * f_out, when set, receives that f [batch, H*S].
 */
typedef struct bdm_decode_fused_args {
    const void *proj;
    const void *f;
    const void *a_log;         /* [H], param_dtype */
    const void *dt_bias;       /* [H*S], param_dtype */
    void *state;
    void *output;              /* [batch, H*v] ctrl_dtype */
    int64_t batch, proj_stride, f_stride;
    int32_t q_col, k_col, v_col, b_col, w_col, read_col, write_col;
    int32_t heads, bank_size, head_width, factor_first, factor_second, selected_banks;
    int32_t ctrl_dtype, param_dtype, state_dtype, qk_norm, routed_decay;
    float scale;
    const void *f_weight;      /* optional: f_proj's second factor [H*S, f_width] */
    void *f_out;               /* optional: [batch, H*S] ctrl_dtype */
    int32_t f_col, f_width;
} bdm_decode_fused_args;

int bdm_decode_fused(const bdm_decode_fused_args *args, void *stream);
/* 1 when bdm_decode_fused takes this geometry, else 0 (no launch). */
int bdm_decode_fused_supported(const bdm_decode_fused_args *args);

/*
 * Controller epilogue of the inference path.  Replaces the activations of
 * heads.controllers (implementation/bdm/heads.py:11-22) applied to the
 * outputs of one concatenated projection GEMM:
 *   q = l2norm(silu(P_q)), k = l2norm(silu(P_k)) per head of S values
 *     (qk_norm 1: x * rsqrt(sum x^2 + 1e-6); 0: x / max(|x|_2, 1e-12),
 *      _parameters.py:214-220), rounded to ctrl_dtype after silu and after
 *     the normalization;
 *   v = silu(P_v), b = sigmoid(P_b), w = sigmoid(P_w), rounded to ctrl_dtype;
 *   g = -exp(A_log[h]) * softplus(f + dt_bias) in FP32, f the f_proj output.
 * proj is [tokens, proj_stride] ctrl_dtype with the q, k, v, b, w slices at
 * the given column offsets; f is [tokens, f_stride].  Outputs are contiguous
 * [tokens, H, S] (q, k, b; g FP32) and [tokens, H, head_width] (v, w).
 */
typedef struct bdm_controller_args {
    const void *proj;
    const void *f;
    const void *a_log;         /* [H], param_dtype */
    const void *dt_bias;       /* [H*S], param_dtype */
    void *q, *k, *v, *b, *w;
    float *g;
    int64_t tokens, proj_stride, f_stride;
    int32_t q_col, k_col, v_col, b_col, w_col;
    int32_t heads, bank_size, head_width;
    int32_t ctrl_dtype, param_dtype, qk_norm;
} bdm_controller_args;

int bdm_controller_epilogue(const bdm_controller_args *args, void *stream);

/*
 * Output epilogue of the inference path: the normalization and gate of
 * _project_bank_output (_parameters.py:222-232) before o_proj.
 *   norm_kind 1 (layer): layer_norm(raw, weight, bias, eps) in FP32, rounded;
 *   norm_kind 0 (rms):   raw * bf(rsqrt(mean(raw^2) + eps)), rounded, then
 *                        times bf(weight), rounded;
 * then times bf(sigmoid(gate)), rounded to ctrl_dtype.  raw is [tokens, width],
 * gate [tokens, gate_stride] (the output_gate projection with its bias), out
 * [tokens, width]; norm_bias may be null for rms.
 */
typedef struct bdm_output_args {
    const void *raw;
    const void *gate;
    const void *norm_weight, *norm_bias;   /* [width], param_dtype */
    void *out;
    int64_t tokens, gate_stride;
    int32_t width, ctrl_dtype, param_dtype, norm_kind;
    float eps;
} bdm_output_args;

int bdm_output_epilogue(const bdm_output_args *args, void *stream);

/*
 * Bank occupancy of a write-route table: the Elastic-SDM final-union
 * regularizer applied to banks (reproduction/experiments/
 * elastic_bank_regularizer.py:10-25), reduced over the (sequence, bank)
 * segments of a write-only dispatch (bdm_dispatch_build with read_banks = 0)
 * instead of a scatter over [batch, J].  For segment s = b*J + bank:
 *   totals[s] = sum over its writes of valid tokens of
 *               log1p(-clamp(p, 0, 1 - 1e-6)) in FP32,
 *   counts[s] = the number of those writes,
 *   first_write[s] = the first position t of such a write, or INT32_MAX
 *               when the bank is never written (first_write may be null).
 * valid ([batch*time] bytes, nonzero = valid) may be null.  write_weights
 * may be null when only counts and first writes are wanted (totals are then
 * 0).  The sum of a segment is a fixed wave reduction: deterministic.
 */
int bdm_bank_occupancy(const void *write_weights, int32_t weight_dtype, const uint8_t *valid,
                       const int64_t *order, const int64_t *cu_seqlens, int64_t batch, int64_t time,
                       int32_t write_banks, int32_t bank_count, float *totals, int32_t *counts,
                       int32_t *first_write, void *stream);

/* Written banks at nested prefixes: the copy-on-write state count of the
 * reference's memory study (APPENDIX.md:511-584; the byte arithmetic is
 * checked by scripts/verify_results.py:190-235).  A bank holds private state
 * from its first write on, so after the first t positions of sequence b
 *   written[b*prefix_count + i] = #{bank : first_write[b*J + bank] < prefixes[i]}
 * first_write [batch, J] int32 from bdm_bank_occupancy; prefixes [prefix_count]
 * int64 on the device. */
int bdm_written_bank_curve(const int32_t *first_write, int64_t batch, int32_t bank_count,
                           const int64_t *prefixes, int32_t prefix_count, int32_t *written, void *stream);

/* RMSNorm of the language-model shell (implementation/bdm/_shell.py:29-35,
 * RMSNorm.forward): out = (x * rsqrt(mean(x^2) + eps)) * weight, in FP32,
 * rounded once to dtype.  x, out [rows, width] of dtype (BDM_BF16 or
 * BDM_F32); weight [width] of weight_dtype.  With residual non-null the
 * block's residual add comes first (model.py:174-176): sum_out = round(x +
 * residual) is written and normalized.  width: a multiple of 8, at most 8192. */
int bdm_rms_norm(const void *x, const void *residual, const void *weight, void *sum_out, void *out,
                 int64_t rows, int32_t width, int32_t dtype, int32_t weight_dtype, float eps, void *stream);

/* SwiGLU of the shell's feed-forward (_shell.py:86-91, FeedForward._forward:
 * silu(w1 x) * w3 x) applied to the output of one GEMM with the concatenated
 * weights [w1; w3]: gate_up [rows, 2*hidden] (x1 in the first hidden columns,
 * x3 in the rest), out [rows, hidden] = round(round(silu(x1)) * x3), the
 * roundings torch makes in dtype.  hidden: a multiple of 8. */
int bdm_swiglu(const void *gate_up, void *out, int64_t rows, int32_t hidden, int32_t dtype, void *stream);

/* Gradients of bdm_rms_norm without a residual, for training: the derivative
 * of the FP32 chain of RMSNorm.forward (_shell.py:29-35) that autograd forms.
 * grad_x [rows, width] of dtype, grad_weight [width] of weight_dtype (FP32
 * sum over rows, one rounding).  partials: FP32 scratch of
 * bdm_rms_norm_backward_partials(rows) * width elements, 16-byte aligned.
 * width: a multiple of 8, at most 4096. */
/* The SwiGLU product of the training path, whose two inputs come from
 * separate GEMMs (_shell.py:86-91, FeedForward._forward: F.silu(w1 x) * w3 x):
 * out[i] = round(round(silu(a[i])) * b[i]) over n elements of dtype, the
 * element of bdm_swiglu.  bdm_swiglu_backward forms autograd's gradients of
 * that product in the same dtype: s = round(silu(a)), grad_b =
 * round(grad_out * s), grad_a = round(round(grad_out * b) * silu'(a)), silu'
 * in FP32. */
int bdm_swiglu_pair(const void *a, const void *b, void *out, int64_t n, int32_t dtype, void *stream);
int bdm_swiglu_backward(const void *a, const void *b, const void *grad_out, void *grad_a, void *grad_b, int64_t n,
                        int32_t dtype, void *stream);

int64_t bdm_rms_norm_backward_partials(int64_t rows);
int bdm_rms_norm_backward(const void *x, const void *grad_out, const void *weight, void *grad_x, void *grad_weight,
                          float *partials, int64_t rows, int32_t width, int32_t dtype, int32_t weight_dtype,
                          float eps, void *stream);

/* y[m] = W x[m] + bias for the rows of a decode step: torch's F.linear
 * (nn.Linear.forward, used by every projection of implementation/bdm/
 * _parameters.py:189-232 and _shell.py:86-91).  x [rows, k], W [n, k]
 * row-major, bias [n] or null, y [rows, n], all of dtype; FP32 accumulation,
 * bias added in FP32, one rounding; x and W 16-byte aligned.  1 to 4 rows:
 * BDM_BF16 or BDM_F32, k a multiple of 8 (a stream over W).  5 to 64 rows:
 * BDM_BF16, k a multiple of 32 (matrix-core tiles); other shapes return
 * BDM_ERR_UNSUPPORTED. */
int bdm_gemv(const void *x, const void *weight, const void *bias, void *y, int64_t rows, int64_t n, int64_t k,
             int32_t dtype, void *stream);

/* bdm_gemv with an input prologue: the elementwise kernel that would produce
 * the GEMV's input row, fused (no counterpart of its own in the reference; it
 * replaces the pair "elementwise kernel, then F.linear" of a decode step with
 * bit-identical results):
 *   BDM_GEMV_RMS        x' = RMSNorm(x [+ residual]) * norm_weight, the shell's
 *                       RMSNorm (_shell.py:29-35); with a residual,
 *                       sum_out = round(x + residual) is also stored
 *                       (model.py:174-176);
 *   BDM_GEMV_SWIGLU     x [rows, 2k] = (a | b), x' = silu(a) * b (_shell.py:86-91);
 *   BDM_GEMV_OUT_LAYER  x' = LayerNorm(x; norm_weight, norm_bias) * sigmoid(gate)
 *   BDM_GEMV_OUT_RMS    x' = RMSNorm(x) * norm_weight * sigmoid(gate)
 *                       (_project_bank_output, _parameters.py:222-232), the
 *                       rounding points of bdm_output_epilogue.
 * A prologue takes k <= 6144.  sum_out must not alias x or residual. */
#define BDM_GEMV_PLAIN 0
#define BDM_GEMV_RMS 1
#define BDM_GEMV_SWIGLU 2
#define BDM_GEMV_OUT_LAYER 3
#define BDM_GEMV_OUT_RMS 4

typedef struct bdm_gemv_args {
    const void *x;            /* [rows, k] ([rows, 2k] for BDM_GEMV_SWIGLU) of dtype */
    const void *weight;       /* [n, k] of dtype, row-major */
    const void *bias;         /* [n] of dtype or NULL */
    void *y;                  /* [rows, n] of dtype */
    const void *residual;     /* BDM_GEMV_RMS: [rows, k] or NULL */
    void *sum_out;            /* BDM_GEMV_RMS with a residual: [rows, k] */
    const void *norm_weight;  /* [k] of param_dtype (norm prologues) */
    const void *norm_bias;    /* [k] of param_dtype (BDM_GEMV_OUT_LAYER) */
    const void *gate;         /* [rows, gate_stride] of dtype (output prologues) */
    int64_t rows, n, k, gate_stride;
    int32_t dtype, param_dtype;
    int32_t prologue;
    float eps;
} bdm_gemv_args;

int bdm_gemv_ex(const bdm_gemv_args *args, void *stream);

/* One AdamW step of the shell's training recipe with FP32 masters
 * (reproduction/experiments/optim.py:30-50, AdamW.step for "wiki"): the
 * gradient-clipping scale, torch's fused AdamW update of the masters and both
 * moments, and the masters' copy back into the BF16 weights, fused into one
 * pass.  Tensor i's master and moments are elements [offset, offset + numel)
 * of the flat FP32 buffers master, exp_avg, exp_avg_sq (16-byte aligned).
 * Each of the `blocks` workgroups updates elements [block_start[b],
 * block_start[b] + chunk) of tensor block_tensor[b] (chunk a multiple of 4).
 * grad_scale (device, may be NULL) multiplies every gradient, rounded to
 * BF16 as clip_grad_norm_'s in-place scaling rounds it; the gradients
 * themselves are not written.  step: the step count after this update's
 * increment (>= 1).  tensors, block_tensor and block_start are device
 * arrays. */
typedef struct bdm_adamw_tensor {
    void *param;          /* [numel] BF16 weight, overwritten with round(master) */
    const void *grad;     /* [numel] BF16 gradient */
    int64_t offset;       /* first element in the flat FP32 buffers */
    int64_t numel;
    double weight_decay;  /* 0 for the no-decay group */
} bdm_adamw_tensor;

typedef struct bdm_adamw_args {
    const bdm_adamw_tensor *tensors;
    const int32_t *block_tensor;
    const int64_t *block_start;
    int64_t tensor_count, blocks, chunk;
    float *master, *exp_avg, *exp_avg_sq;
    const float *grad_scale;
    double lr, beta1, beta2, eps, step;
} bdm_adamw_args;

int bdm_adamw_step(const bdm_adamw_args *args, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* BDM_HIP_H */

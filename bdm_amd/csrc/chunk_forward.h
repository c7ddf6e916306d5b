// The S = 8 routed recurrence on matrix cores (training policy: BF16 state
// rounded every 16 packed events).  See chunk_forward.hip.
#pragma once

#include "bdm_common.h"

namespace bdm {

struct ChunkForwardParams {
    const bf16_t *q, *k, *b;      // [NT, s_heads, 8]
    const float *g;               // [NT, s_heads, 8]
    const bf16_t *v, *w;          // [NT, s_heads, row_stride]
    const bf16_t *ww, *rw;        // [NT, KW], [NT, KR]
    const int64_t *order, *cu;    // dispatch
    const void *initial;          // [J, s_heads, 8, row_stride] (+ init_bstride per batch)
    void *final_state;            // NULL or [batch, J, s_heads, 8, row_stride]
    bf16_t *snap;                 // NULL or [rows, s_heads, 8, row_stride] BF16
    bf16_t *zbuf;                 // [NT*KR, heads * width] read rows
    int64_t init_bstride;
    int64_t nt;
    int heads;        // virtual heads: s_heads * split
    int width;        // columns of a virtual head: 32 * TILES
    int split;        // virtual heads per real head
    int s_heads;      // real heads
    int64_t row_stride;  // columns of a real head
    int banks, kw, kr;
    int kw_shift, kr_shift;  // log2 of kw, kr when powers of two, else -1
    int routed_decay;
    int init_dtype, final_dtype;
    int xcd_remap;
    int nseg;
    float scale;
};

// Whether the matrix-core path takes this forward, and its launch.
bool chunk_path(const bdm_forward_args &a);
int launch_chunk_forward(const ChunkForwardParams &p, int tiles, hipStream_t stream);

}  // namespace bdm

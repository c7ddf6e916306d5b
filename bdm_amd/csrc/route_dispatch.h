// Routing fused with the dispatch's tile count (router.hip), for
// bdm_route_dispatch (dispatch.hip).
#pragma once

#include "bdm_common.h"

namespace bdm {

bool route_tile_count_supported(const void *const *scores, const int64_t *strides, void *const *weights,
                                int64_t *const *indices, int32_t score_dtype, int32_t j1, int32_t j2,
                                int32_t selected);
int launch_route_tile_count(const void *const *scores, const int64_t *strides, void *const *weights,
                            int64_t *const *indices, int64_t batch, int64_t time, int32_t j1, int32_t j2,
                            int32_t *tile_counts, int32_t *status, hipStream_t stream);

}  // namespace bdm

// Launchers of the exact k-nearest-neighbour kernels (gann_knn.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace gann {

int knn_queries_per_block();
size_t knn_smem_bytes(int dtype, int dim, int k);

// x - 128 as int8 rows of dp bytes (zero padded) and |x - 128|^2 per point.
hipError_t launch_knn_prep_u8(const uint8_t* x, int64_t n, int dim, int dp, int8_t* xs, int32_t* xn,
                              hipStream_t stream);

// Per (32-query block, slice of slice_len points): the k best (dist, id + id_base)
// of each query, sorted, into part_d/part_i [slices][nq][k] (padding +inf / -1).
// qs/qn hold nq rounded up to 32 query rows.
hipError_t launch_knn_u8(const int8_t* xs, const int32_t* xn, int64_t n, int dp, const int8_t* qs,
                         const int32_t* qn, int nq, int k, int64_t slices, int64_t slice_len,
                         int64_t id_base, float* part_d, int32_t* part_i, hipStream_t stream);
// Folds slots [0, slots) of part_d/part_i [slots][nq][k] into slot 0, per
// query the k best of all of them in (dist, id) order (a tree of pairwise
// merges, log2(slots) launches).  k <= 128.
hipError_t launch_knn_merge(float* part_d, int32_t* part_i, int nq, int k, int64_t slots,
                            hipStream_t stream);
hipError_t launch_knn_f32(const float* x, int64_t n, int dim, const float* q, int nq, int k,
                          int64_t slices, int64_t slice_len, int64_t id_base, float* part_d,
                          int32_t* part_i, hipStream_t stream);

}  // namespace gann

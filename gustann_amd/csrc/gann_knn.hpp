// Launchers of the exact k-nearest-neighbour kernels (gann_knn.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace gann {

// The uint8 kernel form of a call: queries per wavefront qb (32: one 32x32
// block of products per tile; 16: two 16x16 blocks, half the candidate
// buffers and twice the point reads), the width dp of the int8 rows (dim
// rounded up to the form's 1024 / qb bytes per product step) and the
// kernel's resident wavefronts per CU.
struct KnnU8Form {
  int qb, dp, blocks_per_cu;
};
// The form with more resident queries per CU (qb x blocks_per_cu) for this
// dim and k, the 32-query form on a tie.
KnnU8Form knn_u8_form(int dim, int k);
constexpr int kKnnF32Queries = 32;  // float: queries per wavefront
int knn_f32_blocks_per_cu(int dim, int k);
// LDS bytes per wavefront (dtype 0: uint8 with qb queries, rows of dim
// bytes; 1: float).
size_t knn_smem_bytes(int dtype, int qb, int dim, int k);

// x - 128 as int8 rows of dp bytes (zero padded) and |x - 128|^2 per point.
hipError_t launch_knn_prep_u8(const uint8_t* x, int64_t n, int dim, int dp, int8_t* xs, int32_t* xn,
                              hipStream_t stream);

// Per (query block, slice of slice_len points): the k best (dist, id + id_base)
// of each query, sorted, into part_d/part_i [slices][nq][k] (padding +inf / -1).
// xs holds rows of form.dp bytes; qs/qn hold nq rounded up to form.qb query
// rows of form.dp bytes.
hipError_t launch_knn_u8(const KnnU8Form& form, const int8_t* xs, const int32_t* xn, int64_t n,
                         const int8_t* qs, const int32_t* qn, int nq, int k, int64_t slices,
                         int64_t slice_len, int64_t id_base, float* part_d, int32_t* part_i,
                         hipStream_t stream);
// Folds slots [0, slots) of part_d/part_i [slots][nq][k] into slot 0, per
// query the k best of all of them in (dist, id) order (a tree of pairwise
// merges, log2(slots) launches).  k <= 128.
hipError_t launch_knn_merge(float* part_d, int32_t* part_i, int nq, int k, int64_t slots,
                            hipStream_t stream);
hipError_t launch_knn_f32(const float* x, int64_t n, int dim, const float* q, int nq, int k,
                          int64_t slices, int64_t slice_len, int64_t id_base, float* part_d,
                          int32_t* part_i, hipStream_t stream);

}  // namespace gann

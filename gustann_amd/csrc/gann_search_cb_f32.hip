// The fused shared-codebook search kernels (search_cb_kernel, every shape
// and pivot-table form) for float coordinates.
#include "gann_search.hpp"

namespace gann {

hipError_t launch_search_cb_f32(GANN_CB_ARGS) {
  return launch_search_cb_t<float>(ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, queue, order,
                                qs_all, waves, blocks, global_pivots, lds_groups, smem, stream);
}

}  // namespace gann

// The beam-width search kernels (search_beam_kernel, every shape and pivot
// placement) for float coordinates.
#include "gann_search.hpp"

namespace gann {

hipError_t launch_search_beam_f32(GANN_BEAM_ARGS) {
  return launch_search_beam_t<float>(ix, pq, q, nq, entries, topk, L, bw, nns, dists, found, n_exp, n_adc,
                                  queue, order, qs_all, waves, blocks, global_pivots, smem, stream);
}

}  // namespace gann

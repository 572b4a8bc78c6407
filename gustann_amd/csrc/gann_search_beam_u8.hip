// The beam-width search kernels (search_beam_kernel, every shape and pivot
// placement) for uint8_t coordinates.
#include "gann_search.hpp"

namespace gann {

hipError_t launch_search_beam_u8(GANN_BEAM_ARGS) {
  return launch_search_beam_t<uint8_t>(ix, pq, q, nq, entries, topk, L, bw, nns, dists, found, n_exp, n_adc,
                                  queue, order, qs_all, waves, blocks, global_pivots, smem, stream);
}

}  // namespace gann

// The per-query-LUT fused search kernel (search_kernel) and the step-wise
// round kernel (step_round_kernel) for uint8 and float coordinates.
#include "gann_search.hpp"

namespace gann {

hipError_t launch_search_lut_u8(GANN_LUT_ARGS) {
  return launch_search_lut_t<uint8_t>(ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc,
                                      stream);
}
hipError_t launch_search_lut_f32(GANN_LUT_ARGS) {
  return launch_search_lut_t<float>(ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, stream);
}
hipError_t launch_round_u8(GANN_ROUND_ARGS) {
  return launch_round_t<uint8_t>(ix, pq, q, nq, luts, topk, L, lists, st, nns, dists, active, slots, stream);
}
hipError_t launch_round_f32(GANN_ROUND_ARGS) {
  return launch_round_t<float>(ix, pq, q, nq, luts, topk, L, lists, st, nns, dists, active, slots, stream);
}

}  // namespace gann

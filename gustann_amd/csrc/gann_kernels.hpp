// Host-side launchers of the GustANN HIP kernels (defined in gann_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "gann_device.hpp"

namespace gann {

size_t search_smem_bytes(int M, int dim, int L, int R, int topk);
size_t adc_smem_bytes(int M, int dim);
size_t step_state_bytes();
// Diagnostic: the ADC scan's row reads alone (row_bytes 16, 32, 48 or 64).
hipError_t launch_gather_rows(const uint8_t* rows, int64_t num_rows, int row_bytes,
                              const int32_t* ids, int64_t n, uint32_t* out, hipStream_t stream);
// The node query i expands next (-1: done), read from a host copy of the
// step-wise state array.
int32_t step_state_node(const void* host_states, int64_t i);

hipError_t launch_pq_lut(const PQDev& pq, const float* q, int nq, float* lut_out,
                         hipStream_t stream);
hipError_t launch_pq_adc_scan(const PQDev& pq, const float* q, int nq, const int32_t* ids, int S,
                              float* out, hipStream_t stream);
hipError_t launch_nav_entry(const NavDev& nav, int dtype, int64_t medoid, int64_t num_pts, int dim,
                            const float* q, int nq, int32_t* entries, int32_t* local_out,
                            int32_t* fallback_count, hipStream_t stream);
// order[0..nq): the queries by their squared distance to their entry point
// (into entry_dist[nq]), largest first (approximately: 4096 buckets), the
// order in which the fused search kernels take them.
hipError_t launch_query_order(const IndexDev& ix, int dtype, const float* q, int nq, const int32_t* entries,
                              float* entry_dist, int32_t* order, hipStream_t stream);
hipError_t launch_search(const IndexDev& ix, const PQDev& pq, int dtype, const float* q, int nq,
                         const int32_t* entries, int topk, int L, int32_t* nns, float* dists,
                         int32_t* found, int32_t* n_exp, int32_t* n_adc, hipStream_t stream);
// Shared-codebook search: waves per workgroup that fit the LDS (0 = does not
// fit) and the kernel's register budget, with the pivot table in LDS or
// (global_pivots) read from pq.piv_cb, the first lds_groups groups of 8
// chunks (chunk_w dims each) still in LDS.
int search_cb_waves(int dim, int M, int chunk_w, int L, int topk, size_t lds_limit, bool global_pivots,
                    int lds_groups);
// Groups of 8 chunks of the pivot table (0: the split forms are not
// available); the split forms keep all but the last group, or the first
// half of the groups, in LDS (lds_groups = groups - 1 or groups / 2).
int search_cb_split_groups(int M, int chunk_w);
// lds_groups value (with global_pivots) of the wide form: the whole table
// read through the caches with every pivot row of a lookup requested at
// once, in workgroups of at most 8 waves; served where search_cb_wide_ok
// (16, 32 or 64 chunks of 2 or 4 dims, at most 128 dims).
constexpr int kCbGpWide = -1;
bool search_cb_wide_ok(int M, int chunk_w, int dim);
// The wide form can also keep its first G chunks (1 <= G <= kCbMaxWideLds,
// graph degree <= 64) in a partial pivot table in LDS, in the LDS the lists
// leave: lds_groups = kCbGpWide - G.
constexpr int kCbMaxWideLds = 3;
__host__ __device__ constexpr bool cb_is_wide(int lds_groups) {
  return lds_groups <= kCbGpWide && lds_groups >= kCbGpWide - kCbMaxWideLds;
}
__host__ __device__ constexpr int cb_wide_lds(int lds_groups) {
  return cb_is_wide(lds_groups) ? kCbGpWide - lds_groups : 0;
}
// LDS bytes of the wide form's partial table of G chunks of chunk_w dims.
__host__ __device__ constexpr size_t cb_wide_lds_bytes(int G, int chunk_w) {
  return (size_t)256 * G * chunk_w * 4;
}
// The most chunks (<= kCbMaxWideLds) that fit beside `waves` lists.
int search_cb_wide_lds_chunks(int chunk_w, int L, int topk, size_t lds_limit, int waves, int R);
// Size and contents of pq.piv_cb: the pivots [256][dim] in the kernel's row layout.
size_t search_cb_pivot_bytes(int dim);
void search_cb_pivot_layout(const float* pivots, int dim, uint8_t* out);
hipError_t launch_search_cb(const IndexDev& ix, const PQDev& pq, int dtype, const float* q, int nq,
                            const int32_t* entries, int topk, int L, int32_t* nns, float* dists,
                            int32_t* found, int32_t* n_exp, int32_t* n_adc, int32_t* queue,
                            const int32_t* order, float* qs_all, int waves, int blocks, bool global_pivots,
                            int lds_groups, hipStream_t stream);
// Beam search with beam width bw in [2, max_beam_width()] (same LDS layout,
// pivot placement and launch shape as launch_search_cb).
hipError_t launch_search_beam(const IndexDev& ix, const PQDev& pq, int dtype, const float* q, int nq,
                              const int32_t* entries, int topk, int L, int bw, int32_t* nns,
                              float* dists, int32_t* found, int32_t* n_exp, int32_t* n_adc,
                              int32_t* queue, const int32_t* order, float* qs_all, int waves, int blocks,
                              bool global_pivots, hipStream_t stream);
int max_beam_width();
hipError_t launch_step_init(const PQDev& pq, const float* q, int nq, const int32_t* entries,
                            float* luts, void* st, hipStream_t stream);
hipError_t launch_step_round(const IndexDev& ix, const PQDev& pq, int dtype, const float* q, int nq,
                             const float* luts, int topk, int L, uint64_t* lists, void* st,
                             int32_t* nns, float* dists, int32_t* active, const uint8_t* slots,
                             hipStream_t stream);
hipError_t launch_step_finish(int nq, int topk, const void* st, int32_t* nns, float* dists,
                              int32_t* found, int32_t* n_exp, int32_t* n_adc, hipStream_t stream);
hipError_t launch_fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t stream);

// Fixed device scratch of the allocation-free search entry point
// (gann_search_device_noalloc): kNoAllocCounterBytes of counters, then
// q - centroid of every query from byte kNoAllocCounterBytes on.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
constexpr size_t kNoAllocCounterBytes = 256;
// The device address of the current device's copy of that scratch, resolved
// once per device (hipGetSymbolAddress) and cached; call with `device`
// current.
hipError_t noalloc_scratch_setup(int device, void** out);

}  // namespace gann

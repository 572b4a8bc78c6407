// Launchers of the GPU Vamana graph builder for uint8 points (gann_build.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace gann {

// Expanded nodes kept per build search and prune candidates per node.
constexpr int kBuildPoolMax = 128;
constexpr int kBuildCandMax = 224;

// Points resident in HBM with the graph under construction.
struct BuildDev {
  const uint8_t* x;   // [n][dp] coordinates, rows zero padded to dp bytes
  const int32_t* xn;  // [n] squared norms
  uint32_t* nbr;      // [n][C] out-neighbours, the first deg[i] valid
  uint32_t* deg;      // [n]
  int64_t n;
  int32_t dp;         // row bytes: 32, 64, 96, 128, 192 or 256
  int32_t R;          // degree a prune keeps
  int32_t C;          // list capacity (R <= C <= kBuildSlackMax): reverse edges are
                      // appended up to C before the list is pruned back to R
};

// List capacity with DiskANN's graph slack, ceil(1.3 R).
constexpr int kBuildSlackMax = 84;
constexpr int build_capacity(int R) { return (R * 13 + 9) / 10; }

// Row bytes the builder stores for dim coordinates (0: dim unsupported).
int build_row_bytes(int dim);

// Squared norms of the rows of x ([n][dp]).
hipError_t launch_build_norms(const uint8_t* x, int64_t n, int dp, int32_t* xn, hipStream_t stream);

// Per-dimension sums of the rows of x into sums[dp] (zeroed by the caller).
hipError_t launch_build_col_sums(const uint8_t* x, int64_t n, int dp, unsigned long long* sums,
                                 hipStream_t stream);

// Point closest to mean ([dim] f32, squared L2 summed over dims in order,
// ties by the smaller id) as (float bits << 32 | id) in *best (set to ~0 by
// the caller).
hipError_t launch_build_medoid(const uint8_t* x, int64_t n, int dim, int dp, const float* mean,
                               unsigned long long* best, hipStream_t stream);

// Prunes every list longer than R back to R (the end of the build).
hipError_t launch_build_final_prune(BuildDev g, float alpha, int32_t* queue, int cus, size_t lds_limit,
                                    hipStream_t stream);

// Copies the first R entries of every list into out ([n][R], device).
hipError_t launch_build_compact(BuildDev g, uint32_t* out, hipStream_t stream);

// Random initial graph: init_deg distinct random out-edges per node, no
// self loops (the host builder's stream per node).
hipError_t launch_build_random_graph(BuildDev g, int init_deg, uint64_t seed, hipStream_t stream);

// Greedy search from `start` for each point pts[0..npts) over the current
// graph with exact distances and a list of L; the best kBuildPoolMax
// expanded nodes per point go to pool_id / pool_d ([npts][kBuildPoolMax],
// sorted by distance) and their count to pool_n.  queue: one zeroed int.
size_t build_search_smem_bytes(int L, int waves);
hipError_t launch_build_search(BuildDev g, const uint32_t* pts, int npts, uint32_t start, int L,
                               uint32_t* pool_id, float* pool_d, int32_t* pool_n, int32_t* queue,
                               int cus, hipStream_t stream);

// RobustPrune of every point of the batch over pool + current neighbours;
// writes the new lists and the reverse-edge requests
// pairs[i*R + j] = target << 32 | source (~0 for unused slots).
int build_prune_waves(int dp, size_t lds_limit);
hipError_t launch_build_prune_fwd(BuildDev g, const uint32_t* pts, int npts, const uint32_t* pool_id,
                                  const float* pool_d, const int32_t* pool_n, float alpha,
                                  unsigned long long* pairs, int32_t* queue, int cus,
                                  size_t lds_limit, hipStream_t stream);

// Sorts npairs 64-bit requests and lists the first index of every run of
// equal targets into seg_start, the run count into *n_seg.  temp: scratch
// of the size build_segments_temp_bytes gives for npairs.
hipError_t build_segments_temp_bytes(int64_t npairs, size_t* bytes);
hipError_t launch_build_segments(void* temp, size_t temp_bytes, const unsigned long long* pairs_in,
                                 unsigned long long* pairs_out, int64_t npairs, uint8_t* flags,
                                 int32_t* seg_start, int32_t* n_seg, hipStream_t stream);

// Adds the reverse edges of every run to its target: appended while the
// list has room, else the list and the new sources are pruned back to R.
hipError_t launch_build_reverse(BuildDev g, const unsigned long long* pairs, int64_t npairs,
                                const int32_t* seg_start, const int32_t* n_seg, float alpha,
                                int32_t* queue, int cus, size_t lds_limit, hipStream_t stream);

// PQ codes of n points ([n][dim], uint8 (dtype 0) or f32) with pivots
// [256][dim], centroid [dim] and chunk offsets [M+1] on the device; chunks of
// at most kPqEncodeMaxW dims.
constexpr int kPqEncodeMaxW = 16;
hipError_t launch_pq_encode(const void* x, int dtype, int64_t n, int dim, const float* pivots,
                            const float* centroid, const int32_t* chunk_off, int M, uint8_t* codes,
                            hipStream_t stream);

// RobustPrune of point p over cand[0..ncand) on the device (diagnostic
// entry): out[0..*nout).
hipError_t launch_build_prune_one(BuildDev g, uint32_t p, const uint32_t* cand, int ncand, float alpha,
                                  uint32_t* out, int32_t* nout, size_t lds_limit, hipStream_t stream);

}  // namespace gann

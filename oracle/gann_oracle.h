/* CPU oracle for GustANN's in-memory search path: TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference algorithm (1799364931/GustANN),
 * function by function, used as the parity checker of the HIP kernels and as
 * the timed CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path never does.
 *
 * Arithmetic contract shared with the HIP kernels (both are built with
 * floating-point contraction disabled and spell every fused multiply-add out):
 *  - LUT accumulation  acc = fma(d, d, acc)        (src/impl/pq.cuh:38-40)
 *  - exact L2 partials v   = fma(d, d, v)          (src/impl/util.cuh:36-39)
 *  - ADC sum            s  = s + LUT[j][c_j]       (src/impl/pure_mem.cuh:306-308)
 * nvcc's default --fmad=true contracts both multiply-adds above into FFMA; the
 * oracle therefore defines them as fused.  No reference binary can pin this
 * choice (no CUDA compiler here); see the pinning tests in tests/.
 */
#ifndef GANN_ORACLE_H
#define GANN_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_NUM_PIVOTS 256
#define ORC_NAV_KEEP 4   /* src/impl/nav.cuh:11 */
#define ORC_NAV_EXPAND 28 /* src/impl/nav.cuh:12 */

typedef struct {
  /* disk index (sectors 1.. of <prefix>_disk.index, loaded contiguously) */
  const uint8_t* pages;
  int64_t num_pts, dim, medoid, node_len, nodes_per_page, max_m;
  int32_t dtype; /* 0 = uint8 coords, 1 = float32 coords */
  /* product quantizer */
  const float* pivots;          /* [256][dim] */
  const float* centroid;        /* [dim] */
  const int32_t* chunk_offsets; /* [num_chunks + 1] */
  int32_t num_chunks;
  const uint8_t* codes;         /* [num_pts][num_chunks] */
  /* pivot ("nav") graph; nav_num_node == 0 means none */
  const void* nav_data;         /* [nav_num_node][dim] of the coordinate type */
  const int32_t* nav_graph;     /* [nav_num_node][nav_max_m], -1 padded */
  const int32_t* nav_map;       /* [nav_num_node] base ids */
  int64_t nav_num_node;
  int32_t nav_max_m, nav_start;
} orc_index;

/* LUT[m][k] = sum over dims i of chunk m (ascending) of (q_i - mu_i - P[k][i])^2,
 * accumulated as fma from 0 (src/impl/pq.cuh:8-59). */
void orc_lut_build(const float* pivots, const float* centroid, const int32_t* chunk_offsets,
                   int32_t dim, int32_t num_chunks, const float* q, float* lut);

/* The query as the reference's rerank sees it after init_query restores it in
 * place: fl(fl(q_i - mu_i) + mu_i) (src/impl/pq.cuh:22-24, 54-56). */
void orc_query_restore(const float* centroid, int32_t dim, const float* q, float* q_out);

/* Sequential f32 ADC sum from 0 (src/impl/pure_mem.cuh:300-310). */
float orc_adc(const float* lut, int32_t num_chunks, const uint8_t* code);

/* ADC microbenchmark: out[q][s] = ADC(LUT(q), codes[ids[q][s]]). */
void orc_adc_scan(const float* pivots, const float* centroid, const int32_t* chunk_offsets,
                  int32_t dim, int32_t num_chunks, const uint8_t* codes, int64_t num_pts,
                  const float* q, int32_t nq, const int32_t* ids, int32_t ids_per_q, float* out,
                  int32_t nthreads);

/* Exact squared L2 in square_sum_32 order: 32 lane partials over dims
 * lane, lane+32, ..., then the shfl_down tree 16/8/4/2/1 read at lane 0
 * (src/impl/util.cuh:26-46).  dtype 0 = uint8 x, 1 = float x. */
float orc_l2(const float* q, const void* x, int32_t dtype, int32_t dim);

/* Pivot-graph greedy entry search (src/impl/nav.cuh:13-135); returns the
 * pivot-local id left in slot 0 (masked). *iters receives the expansion count. */
int32_t orc_nav_entry_local(const orc_index* ix, const float* q, int32_t* iters);

/* Base-graph entry for one query: nav entry translated through map.txt
 * (src/nav_graph.cu:104-109) or the medoid without a nav graph
 * (src/pure_mem.cu:119-123).  A pivot id outside the map falls back to the
 * medoid and sets *fallback. */
int32_t orc_entry(const orc_index* ix, const float* q, int32_t* fallback);

/* Beam search of the fused kernel (src/impl/pure_mem.cuh:243-432) for nq
 * queries, entries precomputed (entries == NULL: computed with orc_entry).
 * nns/dists: [nq][topk], found: [nq]; unfilled result slots are 0 as in the
 * reference's zero-initialised device vectors (src/pure_mem.cu:84-87).
 * n_expansions (nullable): per-query expansion counts.  check != 0 verifies
 * list invariants after every expansion; returns the number of violations. */
int64_t orc_search(const orc_index* ix, const float* q, int32_t nq, const int32_t* entries,
                   int32_t topk, int32_t L, int32_t* nns, float* dists, int32_t* found,
                   int32_t* n_expansions, int32_t nthreads, int32_t check);

/* Beam search with beam width bw >= 1, a mode of this library with no
 * counterpart in the reference (which expands one node per iteration).  The
 * list holds at most L entries sorted by (dist, id), each id once, with a
 * visited flag.  Each round takes the first bw unvisited entries in list
 * order (the entry node alone in the first round), marks them visited and
 * expands them in that order: the PQ (ADC) keys of the node's neighbours
 * whose ids are not listed are inserted at their lower bounds, the list is
 * cut back to L, and the node's exact distance is pushed into the top-k
 * (retset_push_32).  The search ends when no unvisited entry is left.
 * Arguments as orc_search. */
int64_t orc_search_beam(const orc_index* ix, const float* q, int32_t nq, const int32_t* entries,
                        int32_t topk, int32_t L, int32_t bw, int32_t* nns, float* dists,
                        int32_t* found, int32_t* n_expansions, int32_t nthreads);

/* on != 0: every later call's worker t runs pinned to the (t mod n)-th of
 * the n CPUs the process may use (the CPU baseline's one thread per core). */
void orc_set_pin_threads(int32_t on);

/* calc_recall (bin/utils.hpp:104-116): hits of res[i][0..k) in the set of the
 * first k ground-truth ids, over `num` queries, divided by num*k. */
double orc_recall(const int32_t* res, const int32_t* gt, int32_t num, int32_t gt_dim, int32_t k);

#ifdef __cplusplus
}
#endif
#endif

/* gustann.h — C ABI of libgustann_hip.so, the MI355X (gfx950) implementation
 * of GustANN's in-GPU search path.
 *
 * Every entry point returns an int status (GANN_OK == 0); on failure
 * gann_last_error() describes the cause (thread-local).  No C++ exception
 * crosses this boundary.  Handles are not thread-safe: one thread per handle,
 * or external locking.  Each handle owns one HIP stream on its device.
 *
 * Reference interfaces replaced (1799364931/GustANN):
 *   GustANN::GustANN(DataType)                 src/ssd_search.hpp:70
 *   GustANN::init_pure_mem(cfg, use_gpu_mem)   src/ssd_search.hpp:76, src/ssd_search.cu:108-112
 *   GustANN::search(q, nq, topk, L, nns, dists, found_cnt, stats)
 *                                              src/ssd_search.hpp:78-80, src/pure_mem.cu:71-199
 *   GustANN::~GustANN()                        src/ssd_search.cu:28-53
 *   PQSearch::read_data / init_device          src/pq_search.cu:56-185
 *   PQSearchData::init_query (LUT build)       src/impl/pq.cuh:8-59
 *   ADC scan                                   src/impl/pure_mem.cuh:300-310
 *   get_entry_kernel + NavGraph::translate     src/impl/nav.cuh:13-147, src/nav_graph.cu:104-109
 */
#ifndef GUSTANN_H
#define GUSTANN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes */
#define GANN_OK 0
#define GANN_ERR_INVALID 1     /* bad argument (the reference asserted or threw) */
#define GANN_ERR_IO 2          /* file missing / unreadable (the reference called exit(-1)) */
#define GANN_ERR_FORMAT 3      /* malformed index file */
#define GANN_ERR_HIP 4         /* HIP runtime failure (the reference's CHECK_CUDA threw) */
#define GANN_ERR_NOMEM 5       /* device or pinned host allocation failed */
#define GANN_ERR_UNSUPPORTED 6 /* valid request outside what this build implements */

/* ---- enums */
#define GANN_UINT8 0 /* DataType UINT8, src/common.hpp:22-25 */
#define GANN_FLOAT 1 /* DataType FLOAT */

#define GANN_PLACEMENT_HBM 0         /* search_mem -G: index pages copied to HBM */
#define GANN_PLACEMENT_HOST_PINNED 1 /* search_mem without -G: pages read zero-copy from pinned host memory */

#define GANN_MODE_FUSED 0     /* one kernel per search (src/impl/pure_mem.cuh:243-432); picks the
                                 shared-codebook kernel with the pivot table in LDS while at least
                                 8 lists fit beside it, else the same kernel reading the pivot
                                 table through the caches (GANN_MODE_FUSED_GP) */
#define GANN_MODE_STEPWISE 1  /* one launch per expansion round, list in HBM (src/impl/hyd_search_v2.cuh) */
#define GANN_MODE_FUSED_LUT 2 /* the fused kernel with a per-query LUT in LDS, forced */
#define GANN_MODE_STEPWISE_PAGED 3 /* step-wise with a page-fetch stage: each round the host copies
                                      every query's next page into a pinned slot the kernel reads
                                      (src/hyd_task_runner.cu:200-275, src/io/mem_io.cpp:11-44);
                                      pages come from host memory (pinned placement) or the index
                                      file */
#define GANN_MODE_STEPWISE_URING 5 /* GANN_MODE_STEPWISE_PAGED with every query's whole page read
                                      from the index file through io_uring each round (O_DIRECT
                                      where the file system allows; src/io/io_uring.cpp);
                                      GANN_ERR_UNSUPPORTED where the kernel refuses io_uring */
#define GANN_MODE_FUSED_GP 4  /* the shared-codebook fused kernel with the pivot table read from HBM
                                 through the caches and only the lists in LDS, forced (more lists
                                 per CU at large L) */

/* OR'ed into the mode of gann_search_device_ex / gann_search_device_noalloc:
 * entries_dev holds each query's entry node on input and entry selection is
 * skipped (a caller that already has entry points, e.g. from another
 * shard's search, or that times the search kernel alone).  An entry outside
 * [0, num_pts) gives that query an empty result.  The reference always
 * selects entries itself (src/pure_mem.cu:104-124). */
#define GANN_SEARCH_ENTRIES_GIVEN 0x100

typedef struct gann_handle gann_handle;
typedef struct gann_pq gann_pq;

/* GustANNConfig (src/ssd_search.hpp:18-23) plus the data type, placement and
 * device that the reference took from its constructor, -G flag and
 * CUDA_VISIBLE_DEVICES. */
typedef struct gann_config {
  const char* index_file; /* <prefix>_disk.index */
  const char* pq_prefix;  /* <pq>_pivots.bin, <pq>_compressed.bin (required) */
  const char* nav_prefix; /* directory with nav_index, nav_index.data, map.txt; NULL or "" = none */
  int32_t dtype;          /* GANN_UINT8 / GANN_FLOAT */
  int32_t placement;      /* GANN_PLACEMENT_* */
  int32_t device_id;
} gann_config;

/* GustANNStats (src/ssd_search.hpp:25-27) extended with device counters. */
typedef struct gann_stats {
  double run_time_s;      /* wall clock of entry selection + search, the scope of src/pure_mem.cu:101-187 */
  double entry_time_s;    /* wall clock of entry selection alone */
  int64_t n_expansions;   /* node expansions summed over queries */
  int64_t n_adc;          /* ADC evaluations summed over queries */
  double alg_bytes;       /* algorithmic bytes: per expansion record + deg*M codes, per query q + results */
  int64_t n_nav_fallback; /* queries whose pivot entry fell outside map.txt (entry = medoid) */
} gann_stats;

typedef struct gann_index_info {
  int64_t num_pts, dim, medoid, max_m, node_len, nodes_per_page, num_pages;
  int32_t dtype, num_chunks;
  int64_t nav_num_node;
  int32_t nav_max_m, nav_start;
} gann_index_info;

const char* gann_last_error(void);
const char* gann_version(void);

/* ---- index handle (GustANN facade, PURE_MEM executor) */

/* GustANN(dtype) + init_pure_mem(cfg, placement == HBM). Loads the disk
 * index, the PQ tables and the optional pivot graph, validates every node
 * record (deg <= R, neighbour ids < num_pts, no repeated id in a list) and
 * makes the index resident on the device. */
int gann_open(const gann_config* cfg, gann_handle** out);
int gann_close(gann_handle* h);
int gann_get_info(const gann_handle* h, gann_index_info* info);

/* GustANN::search (src/ssd_search.hpp:78-80, src/pure_mem.cu:71-199).
 * Synchronous; q is [nq][dim] f32 row-major on the host; nns/dists are
 * [nq][topk], found_cnt [nq] on the host.  Requires L >= topk
 * (bin/search_disk.cpp:189-192).  beam_width 1 is the reference's one node
 * per iteration (results identical to the reference); 2..4 selects the beam
 * search of this library (the first beam_width unvisited entries are expanded
 * per round; GANN_MODE_FUSED or GANN_MODE_FUSED_GP only), which the reference does not have.
 * st may be NULL. */
int gann_search(gann_handle* h, const float* q, int32_t nq, int32_t topk, int32_t L,
                int32_t beam_width, int32_t* nns, float* dists, int32_t* found_cnt,
                gann_stats* st);

/* gann_search with an explicit execution mode (GANN_MODE_*); n_exp (nullable,
 * [nq]) receives each query's expansion count. */
int gann_search_ex(gann_handle* h, const float* q, int32_t nq, int32_t topk, int32_t L,
                   int32_t beam_width, int32_t mode, int32_t* nns, float* dists,
                   int32_t* found_cnt, int32_t* n_exp, gann_stats* st);

/* Asynchronous fused search on device buffers already resident in HBM,
 * enqueued on `stream` (a hipStream_t; 0 = the default stream).
 * entries_dev: [nq] device scratch for the entry ids.  n_exp_dev/n_adc_dev
 * nullable [nq].  The kernels also use scratch owned by the handle (the
 * query queue counter, q - centroid of every query, the order in which the
 * fused kernels take the queries, and the step-wise modes' LUTs, lists and
 * states), so at most one call per handle may be in flight: a caller that
 * enqueues calls of one handle on different streams orders them itself (or
 * uses one handle per stream).  The fused kernels take the queries farthest
 * from their entry point first; every result is the same in any order. */
int gann_search_device(gann_handle* h, const float* q_dev, int32_t nq, int32_t topk, int32_t L,
                       int32_t* entries_dev, int32_t* nns_dev, float* dists_dev,
                       int32_t* found_dev, int32_t* n_exp_dev, int32_t* n_adc_dev, void* stream);

/* gann_search_device with a beam width and an execution mode (as in
 * gann_search_ex).  No counterpart in the reference, whose search takes host
 * arrays only; it is the device-resident form of gann_search_ex. */
int gann_search_device_ex(gann_handle* h, const float* q_dev, int32_t nq, int32_t topk, int32_t L,
                          int32_t beam_width, int32_t mode, int32_t* entries_dev, int32_t* nns_dev,
                          float* dists_dev, int32_t* found_dev, int32_t* n_exp_dev,
                          int32_t* n_adc_dev, void* stream);

/* gann_search_device_ex without any allocation, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * kernels' scratch (counters and q - centroid of every query) lives in a
 * fixed device array of 64 MiB that each GPU holds until the process ends,
 * so nq * dim * 4 must not exceed 64 MiB - 256 B (131071 queries at dim
 * 128); larger calls return GANN_ERR_INVALID.  Fused modes only
 * (GANN_MODE_FUSED, GANN_MODE_FUSED_GP, GANN_MODE_FUSED_LUT; the step-wise
 * modes return GANN_ERR_UNSUPPORTED).  Every call on one GPU shares that
 * array, whichever handle it comes from: calls that overlap on one GPU race,
 * so the caller orders them.  Arguments and results as gann_search_device_ex
 * (the queries are taken in queue order: the fixed array holds no order,
 * which changes the time, not the results). */
int gann_search_device_noalloc(gann_handle* h, const float* q_dev, int32_t nq, int32_t topk, int32_t L,
                               int32_t beam_width, int32_t mode, int32_t* entries_dev, int32_t* nns_dev,
                               float* dists_dev, int32_t* found_dev, int32_t* n_exp_dev,
                               int32_t* n_adc_dev, void* stream);

/* get_entry_kernel + NavGraph::translate: base-graph entry per query (the
 * medoid when the handle has no pivot graph).  local_out (nullable) receives
 * the pivot-local ids. */
int gann_nav_entry(gann_handle* h, const float* q, int32_t nq, int32_t* entries_out,
                   int32_t* local_out);

/* ---- PQ tables */

/* PQSearch::read_data + init_device for a standalone PQ (no graph). */
int gann_pq_open(const char* pq_prefix, int32_t device_id, gann_pq** out);
/* PQ from arrays: pivots [256][dim], centroid [dim], chunk_offsets [M+1]
 * (0 .. dim, non-decreasing), codes [num_pts][M].  codes_on_device != 0
 * borrows a device pointer (the caller keeps it alive); otherwise the codes
 * are copied to HBM. */
int gann_pq_create(const float* pivots, const float* centroid, const int32_t* chunk_offsets,
                   int32_t dim, int32_t num_chunks, const uint8_t* codes, int64_t num_pts,
                   int32_t codes_on_device, int32_t device_id, gann_pq** out);
int gann_pq_close(gann_pq* pq);
/* The PQ tables of an open handle (borrowed; valid until gann_close). */
int gann_handle_pq(gann_handle* h, gann_pq** out);

/* LUT build (src/impl/pq.cuh:8-59): lut_out [nq][M][256] on the host. */
int gann_pq_lut_build(gann_pq* pq, const float* q, int32_t nq, float* lut_out);
/* LUT + ADC gather-scan: out[i][s] = ADC(LUT(q_i), codes[ids[i][s]]); ids
 * [nq][ids_per_q] on the host, each in [0, num_pts). */
int gann_pq_adc_scan(gann_pq* pq, const float* q, int32_t nq, const int32_t* ids,
                     int32_t ids_per_q, float* out);
/* Asynchronous LUT + ADC gather-scan on device buffers, enqueued on `stream`
 * (a hipStream_t; 0 = the default stream).  Ids outside [0, num_pts) give NaN. */
int gann_pq_adc_scan_device(gann_pq* pq, const float* q_dev, int32_t nq, const int32_t* ids_dev,
                            int32_t ids_per_q, float* out_dev, void* stream);

/* ---- exact nearest neighbours (ground truth) */

/* Exact k nearest neighbours of each query by squared L2, ties broken by the
 * smaller id: the ground truth that calc_recall (bin/utils.hpp:104-116)
 * scores against, stored by callers as ivecs.  No counterpart in the
 * reference, whose ground truth comes from external tools; it serves
 * dataset builders and tests.  base: [n][dim] on the host, uint8
 * (GANN_UINT8; queries must then hold integers in [0, 255]; distances exact)
 * or f32 (GANN_FLOAT; each distance sums fma((q - x)^2) over the dims in
 * ascending order); queries [nq][dim] f32 on the host; ids/dists [nq][k] on
 * the host, id -1 and +inf past n.  dim <= 256, k <= 128, n < 2^31. */
int gann_knn_exact(const void* base, int64_t n, int32_t dim, int32_t dtype, const float* queries,
                   int32_t nq, int32_t k, int32_t device_id, int32_t* ids, float* dists);

/* ---- index construction */

/* PQ codes of n points on the GPU: for every chunk m, the first of the 256
 * pivots with the smallest distance, accumulated as fma(t, t, d) over the
 * chunk's dims in order with t = (x - centroid) - pivot -- the operations of
 * a LUT entry (src/impl/pq.cuh:35-43), so a point's code is the argmin of the
 * LUT the search would build for that point.  Replaces the encoding step of
 * DiskANN's PQ build (external to the reference, scripts/build_diskann_index.sh:7);
 * no counterpart in the reference's own code.  data [n][dim] on the host,
 * GANN_UINT8 or GANN_FLOAT; pivots [256][dim], centroid [dim], chunk_offsets
 * [M+1] (tiling [0, dim), chunks of at most 16 dims) and codes [n][M] on
 * the host. */
int gann_pq_encode(const void* data, int64_t n, int32_t dim, int32_t dtype, const float* pivots,
                   const float* centroid, const int32_t* chunk_offsets, int32_t M, int32_t device_id,
                   uint8_t* codes);


/* Vamana graph of uint8 points built on the GPU.  Replaces the external
 * DiskANN build the reference runs before searching
 * (scripts/build_diskann_index.sh:7 for the base graph,
 * scripts/gen_pivot_graph.sh:13 for the pivot graph); no counterpart in the
 * reference's own code.  Same steps as a sequential Vamana build: medoid
 * start, random initial graph of R/2 edges per node, a pass with alpha = 1
 * then one with `alpha`, each inserting every point in a seeded random order
 * by greedy search (list L), RobustPrune and reverse edges (lists grow to
 * ceil(1.3 R) before a prune, DiskANN's slack, and are pruned back to R at
 * the end); points are inserted in batches of at most max_batch (doubling
 * from 1 in the first pass) that see the graph as of the batch start.  data: [n][dim] on the
 * host; out_nbr [n][R] and out_deg [n] on the host (row i: the first
 * out_deg[i] entries valid), *out_medoid the start node.  dim <= 256,
 * R <= 64, L <= 1024, n < 2^31 - 1.  verbose: progress lines on stderr. */
int gann_build_vamana(const uint8_t* data, int64_t n, int32_t dim, int32_t R, int32_t L, float alpha,
                      uint64_t seed, int64_t max_batch, int32_t device_id, int32_t verbose,
                      uint32_t* out_nbr, uint32_t* out_deg, int64_t* out_medoid);

/* ---- diagnostics */

/* The memory access of gann_pq_adc_scan_device alone: reads the row of every
 * id (row_bytes of 16, 32, 48 or 64 at rows_dev + id * row_bytes, device
 * memory, 16-byte aligned) with the same vector loads and folds it to one
 * word in out_dev[i]; ids outside [0, num_rows) read row 0.  No counterpart
 * in the reference: its time is the random-gather ceiling the ADC scan's
 * roofline is read against.  Asynchronous on `stream`. */
int gann_diag_gather_rows(const uint8_t* rows_dev, int64_t num_rows, int32_t row_bytes,
                          const int32_t* ids_dev, int64_t n_ids, uint32_t* out_dev, void* stream);

/* One RobustPrune of the graph builder on the device: point p of data
 * ([n][dim] uint8, host) over the candidate ids cand[0..ncand) (host,
 * ncand <= 224): candidates sorted by (exact squared L2 to p, id), repeated
 * ids and p dropped, each kept candidate occludes a later one j when
 * d(p, j) / d(kept, j) > alpha; at most R kept, in order, into out (host,
 * R entries), their count into *nout.  No counterpart in the reference; it
 * lets tests check the builder's pruning step exactly. */
int gann_diag_robust_prune(const uint8_t* data, int64_t n, int32_t dim, int64_t p, const uint32_t* cand,
                           int32_t ncand, float alpha, int32_t R, int32_t device_id, uint32_t* out,
                           int32_t* nout);

#ifdef __cplusplus
}
#endif
#endif /* GUSTANN_H */

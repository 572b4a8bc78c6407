// GustANN kernels for MI355X (gfx950, wave64), except the beam-search
// kernels themselves (gann_search.hpp and its per-type translation units):
//
//  * pq_lut_kernel      : LUT build only (src/impl/pq.cuh:8-59), one
//                         workgroup per query, LUT written to HBM.
//  * pq_adc_scan_kernel : LUT build staged in LDS + ADC gather-scan over a
//                         list of candidate ids per query
//                         (src/impl/pure_mem.cuh:300-310 applied to an id list).
//  * nav_entry_kernel   : pivot-graph entry selection (src/impl/nav.cuh:13-135)
//                         with the map.txt translation (src/nav_graph.cu:104-109)
//                         done on the device.
//  * query_centre_kernel, step_init_kernel, step_finish_kernel: the set-up
//                         and tear-down of the search kernels;
//  * the launchers, which dispatch on the coordinate type.
#include "gann_kernels.hpp"

#include <hip/hip_runtime.h>

#include <climits>
#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

#include "gann_device.hpp"
#include "gann_list.hpp"
#include "gann_search.hpp"

namespace gann {

// ------------------------------------------------------------------ LUT only

template <int W>
__global__ __launch_bounds__(256) void pq_lut_kernel(PQDev pq, const float* __restrict__ q,
                                                     int nq, float* __restrict__ lut_out) {
  extern __shared__ float qs_smem[];
  const int qi = blockIdx.x;
  if (qi >= nq) return;
  for (int i = threadIdx.x; i < pq.dim; i += blockDim.x)
    qs_smem[i] = q[(int64_t)qi * pq.dim + i] - pq.centroid[i];
  __syncthreads();
  lut_build<W>(pq, qs_smem, lut_out + (int64_t)qi * pq.M * kPivots, threadIdx.x, blockDim.x);
}

// ------------------------------------------------------------------ ADC scan

// One workgroup (256 lanes) per query.  LDS: LUT [M][256] f32 then q - mu.
// Each lane scores ids tid, tid+256, ... in batches of kBatch rows.  The
// first batch of ids and code rows is requested before the LUT is built, and
// each following batch right after the previous one is summed, so the random
// row gathers (the bound of this kernel) overlap the LUT build and the LDS
// lookups.  Code rows use ordinary cached loads: on gfx950 nontemporal loads
// cut the random-row request rate by about a fifth.
template <int MW, int W, int kBatch>
__global__ __launch_bounds__(256) void pq_adc_scan_kernel(PQDev pq, const float* __restrict__ q,
                                                          int nq, const int32_t* __restrict__ ids,
                                                          int S, float* __restrict__ out) {
  extern __shared__ float smem[];
  float* lut = smem;
  float* qs = smem + pq.M * kPivots;
  const int qi = blockIdx.x;
  if (qi >= nq) return;
  const int tid = threadIdx.x;
  const int nt = blockDim.x;
  const int M = pq.M;
  const int32_t* qids = ids + (int64_t)qi * S;
  float* qout = out + (int64_t)qi * S;

  int32_t id[kBatch];
  CodeRow<MW> row[kBatch];
  auto request = [&](int s0) {
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int s = s0 + b * nt + tid;
      const int32_t x = s < S ? qids[s] : -1;
      id[b] = (x >= 0 && (int64_t)x < pq.num_pts) ? x : -1;
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
      if (id[b] >= 0) row[b].load(pq.codes + (int64_t)id[b] * M, M);
  };
  request(0);

  for (int i = tid; i < pq.dim; i += nt) qs[i] = q[(int64_t)qi * pq.dim + i] - pq.centroid[i];
  __syncthreads();
  lut_build<W>(pq, qs, lut, tid, nt);
  __syncthreads();

  for (int s0 = 0; s0 < S; s0 += kBatch * nt) {
    float d[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
      d[b] = id[b] >= 0 ? row[b].adc(lut, pq.codes + (int64_t)id[b] * M, M) : __builtin_nanf("");
    if (s0 + kBatch * nt < S) request(s0 + kBatch * nt);
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int s = s0 + b * nt + tid;
      if (s < S) __builtin_nontemporal_store(d[b], qout + s);
    }
  }
}

// ------------------------------------------------------------------ nav entry

// One wavefront per query; lanes 0..31 hold the 32-slot pool of the
// reference's warp (slot t in lane t), lanes 0..27 score the expanded node's
// neighbours, each computing its full square_sum_32 value in-lane.
template <typename T>
__global__ __launch_bounds__(64) void nav_entry_kernel(NavDev nav, int64_t medoid, int64_t num_pts,
                                                       int dim, const float* __restrict__ q,
                                                       int nq, int32_t* __restrict__ entries,
                                                       int32_t* __restrict__ local_out,
                                                       int32_t* __restrict__ fallback_count) {
  extern __shared__ float qv[];
  const int qi = blockIdx.x;
  if (qi >= nq) return;
  const int lane = lane_id();
  for (int i = lane; i < dim; i += kWave) qv[i] = q[(int64_t)qi * dim + i];
  __syncthreads();
  const T* data = reinterpret_cast<const T*>(nav.data);
  constexpr int kKeep = 4, kExpand = 28;  // src/impl/nav.cuh:11-12
  const int64_t total = nav.n * (int64_t)nav.max_m;

  uint32_t pid = 0xffffffffu;
  float pd = INFINITY;
  {
    float d0 = l2_square_sum_32<T>(qv, data + (int64_t)nav.start * dim, dim);
    if (lane == 0) {
      pid = (uint32_t)nav.start;
      pd = d0;
    }
  }
  int idx = 0;
  const int64_t cap = 4 * nav.n + 64;
  for (int64_t it = 0; idx != -1 && it < cap; ++it) {
    const uint32_t u = (uint32_t)__shfl((int)pid, idx, kWave) & kMask31;
    if (lane == idx) pid |= kVisited;
    // neighbours: first <= 28 entries of the flat -1-padded array from u*max_m
    const int64_t flat = (int64_t)u * nav.max_m + lane;
    int32_t v = -1;
    if (lane < kExpand && flat < total) v = nav.graph[flat];
    const uint64_t stop = ballot64(lane >= kExpand || v == -1);
    const int cnt = (int)__builtin_ctzll(stop);  // lanes < cnt hold neighbours
    float dv = INFINITY;
    if (lane < cnt) dv = l2_square_sum_32_inlane<T>(qv, data + (int64_t)v * dim, dim);
    // neighbour t -> slot t + 4
    const int src = lane - kKeep;
    const int32_t v_sh = __shfl(v, src < 0 ? 0 : src, kWave);
    const float d_sh = __shfl(dv, src < 0 ? 0 : src, kWave);
    if (lane >= kKeep && lane < 32 && src < cnt) {
      pid = (uint32_t)v_sh;
      pd = d_sh;
    }
    // four selection steps (src/impl/nav.cuh:84-119)
#pragma unroll
    for (int i = 0; i < kKeep; ++i) {
      float d = pd;
      int pos = lane;
      if (i != 0) {
        const uint32_t prev = (uint32_t)__shfl((int)pid, i - 1, kWave);
        const bool fold = lane < 32 && lane >= i && ((pid ^ prev) & kMask31) == 0;
        const bool fold_vis = ballot64(fold && (pid & kVisited)) != 0;
        if (fold) pd = INFINITY;
        if (lane == i - 1 && fold_vis) pid |= kVisited;
        d = fold ? INFINITY : pd;
      }
      if (lane < i) d = INFINITY;
#pragma unroll
      for (int off = 16; off > 0; off >>= 1) {
        const float od = __shfl_down(d, off, 32);
        const int op = __shfl_down(pos, off, 32);
        if (od < d) {
          d = od;
          pos = op;
        }
      }
      pos = __shfl(pos, 0, kWave);
      if (i != pos) {
        const float tv = __shfl(pd, i, kWave), yv = __shfl(pd, pos, kWave);
        const uint32_t ti = (uint32_t)__shfl((int)pid, i, kWave);
        const uint32_t yi = (uint32_t)__shfl((int)pid, pos, kWave);
        if (tv != yv) {
          if (lane == i) {
            pd = yv;
            pid = yi;
          } else if (lane == pos) {
            pd = tv;
            pid = ti;
          }
        }
      }
    }
    const uint64_t unv = ballot64(lane < 32 && !(pid & kVisited));
    const int x = unv ? (int)__builtin_ctzll(unv) : 32;
    idx = x < kKeep ? x : -1;
  }
  if (lane == 0) {
    const int32_t local = (int32_t)(pid & kMask31);
    int32_t base = -1;
    if (local >= 0 && local < nav.n) base = nav.map[local];
    if (base < 0 || base >= num_pts) {
      base = (int32_t)medoid;
      atomicAdd(fallback_count, 1);
    }
    entries[qi] = base;
    if (local_out) local_out[qi] = local;
  }
}

// Squared distance of each query to its entry point (the order key of
// query_order_kernel); entries outside the index give 0.
template <typename T>
__global__ void entry_dist_kernel(IndexDev ix, const float* __restrict__ q, int nq,
                                  const int32_t* __restrict__ entries, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nq) return;
  const int32_t u = entries[i];
  float s = 0.0f;
  if (u >= 0 && u < ix.num_pts) {
    const T* x = reinterpret_cast<const T*>(record_of(ix, u));
    const float* qq = q + (int64_t)i * ix.dim;
    for (int d = 0; d < ix.dim; ++d) {
      const float t = qq[d] - to_f(x[d]);
      s = fma_f(t, t, s);
    }
  }
  out[i] = s;
}

// The order in which the persistent search kernels take the queries: the
// farthest from its entry point first.  Expansions per query vary (2,577 to
// 6,994 at L = 2576 on a 100M mixture, mean 3,044) and grow with that
// distance, so long searches start early and the last queries taken are
// short ones, instead of a long one holding the kernel open while most lists
// are idle.  A counting sort on 4096 buckets of the distance's bit pattern
// (a non-negative float's bits order like its value; exponent and 4
// mantissa bits), in one workgroup; order within a bucket is arbitrary.  No
// result depends on the order: each query's search is independent.
constexpr int kOrderBuckets = 4096, kOrderThreads = 1024;

__device__ __forceinline__ int order_bucket(float d) {
  const uint32_t b = __float_as_uint(d) >> 19;
  return kOrderBuckets - 1 - (int)min(b, (uint32_t)(kOrderBuckets - 1));
}

__global__ __launch_bounds__(kOrderThreads) void query_order_kernel(const float* __restrict__ d, int nq,
                                                                    int32_t* __restrict__ order) {
  __shared__ int cnt[kOrderBuckets];
  __shared__ int wave_sum[kOrderThreads / kWave];
  constexpr int kPer = kOrderBuckets / kOrderThreads;
  const int t = threadIdx.x, wave = t / kWave;
  for (int b = t; b < kOrderBuckets; b += kOrderThreads) cnt[b] = 0;
  __syncthreads();
  for (int i = t; i < nq; i += kOrderThreads) atomicAdd(&cnt[order_bucket(d[i])], 1);
  __syncthreads();
  // exclusive scan of the counts: thread t owns buckets kPer t .. kPer t + kPer - 1
  int c[kPer], s = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) s += (c[j] = cnt[kPer * t + j]);
  const int incl = wave_incl_scan(s);
  if (lane_id() == kWave - 1) wave_sum[wave] = incl;
  __syncthreads();
  int off = incl - s;
  for (int w = 0; w < wave; ++w) off += wave_sum[w];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    cnt[kPer * t + j] = off;
    off += c[j];
  }
  __syncthreads();
  for (int i = t; i < nq; i += kOrderThreads) order[atomicAdd(&cnt[order_bucket(d[i])], 1)] = i;
}

// q - mu of every query (src/impl/pq.cuh:22-24), read back with uniform
// (scalar) loads by the shared-codebook ADC.
__global__ void query_centre_kernel(const float* __restrict__ q, const float* __restrict__ centroid,
                                    int64_t n, int dim, float* __restrict__ qs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) qs[i] = q[i] - centroid[i % dim];
}


// Builds each query's LUT into HBM (the role of init_search,
// src/hyd_task_runner.cu:12-15) and initialises its state.
template <int W>
__global__ __launch_bounds__(64) void step_init_kernel(PQDev pq, const float* __restrict__ q,
                                                       int nq, int64_t num_pts,
                                                       const int32_t* __restrict__ entries,
                                                       float* __restrict__ luts,
                                                       StepState* __restrict__ st) {
  extern __shared__ float qs[];
  const int qi = blockIdx.x;
  if (qi >= nq) return;
  const int lane = lane_id();
  for (int i = lane; i < pq.dim; i += kWave) qs[i] = q[(int64_t)qi * pq.dim + i] - pq.centroid[i];
  __syncthreads();
  lut_build<W>(pq, qs, luts + (int64_t)qi * pq.M * kPivots, lane, kWave);
  if (lane == 0) {
    const int32_t e = entries[qi];
    st[qi] = StepState{e < num_pts ? e : -1, 0, 0, 0, 0, 0};
  }
}


// Finalises the step-wise results: zero the unfilled slots, counts out.
__global__ void step_finish_kernel(int nq, int topk, const StepState* __restrict__ st,
                                   int32_t* __restrict__ nns, float* __restrict__ dists,
                                   int32_t* __restrict__ found_cnt, int32_t* __restrict__ n_exp,
                                   int32_t* __restrict__ n_adc) {
  const int qi = blockIdx.x;
  if (qi >= nq) return;
  const StepState s = st[qi];
  for (int j = threadIdx.x; j < topk; j += blockDim.x) {
    if (j >= s.found) {
      nns[(int64_t)qi * topk + j] = 0;
      dists[(int64_t)qi * topk + j] = 0.0f;
    }
  }
  if (threadIdx.x == 0) {
    found_cnt[qi] = s.found;
    if (n_exp) n_exp[qi] = s.exps;
    if (n_adc) n_adc[qi] = s.adcs;
  }
}

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ------------------------------------------------------------------ diagnostics

// The ADC scan's memory access alone: every id's row of row_words 16-byte
// words is read (plain vector loads, as CodeRow does) and folded to one word;
// no LUT and no arithmetic.  Its time is the ceiling the ADC scan is measured
// against.  Each thread keeps 8 ids in flight.  Ids outside [0, num_rows) read
// row 0.
template <int RW>
__global__ __launch_bounds__(256) void gather_rows_kernel(const u32x4* __restrict__ rows,
                                                          int64_t num_rows,
                                                          const int32_t* __restrict__ ids,
                                                          int64_t n, uint32_t* __restrict__ out) {
  constexpr int B = 8;
  const int64_t base = ((int64_t)blockIdx.x * blockDim.x) * B + threadIdx.x;
  int64_t id[B];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    const int64_t s = base + (int64_t)b * blockDim.x;
    const int32_t v = s < n ? ids[s] : 0;
    id[b] = (v >= 0 && v < num_rows) ? v : 0;
  }
  u32x4 w[B][RW];
#pragma unroll
  for (int b = 0; b < B; ++b)
#pragma unroll
    for (int r = 0; r < RW; ++r) w[b][r] = rows[id[b] * RW + r];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    const int64_t s = base + (int64_t)b * blockDim.x;
    uint32_t x = 0;
#pragma unroll
    for (int r = 0; r < RW; ++r) x ^= w[b][r].x ^ w[b][r].y ^ w[b][r].z ^ w[b][r].w;
    if (s < n) out[s] = x;
  }
}

// ------------------------------------------------------------------ launchers

size_t search_smem_bytes(int M, int dim, int L, int R, int topk) {
  (void)R;
  return SearchSmem::bytes(M, dim, L, topk);
}

size_t adc_smem_bytes(int M, int dim) { return (size_t)M * kPivots * 4 + (size_t)dim * 4; }

hipError_t launch_pq_lut(const PQDev& pq, const float* q, int nq, float* lut_out,
                         hipStream_t stream) {
  return with_w(pq.chunk_w, [&](auto w) {
    hipLaunchKernelGGL((pq_lut_kernel<decltype(w)::value>), dim3(nq), dim3(256),
                       (size_t)pq.dim * 4, stream, pq, q, nq, lut_out);
    return hipGetLastError();
  });
}

hipError_t launch_pq_adc_scan(const PQDev& pq, const float* q, int nq, const int32_t* ids, int S,
                              float* out, hipStream_t stream) {
  const size_t smem = adc_smem_bytes(pq.M, pq.dim);
  return with_mw(pq.M, [&](auto mw) {
    return with_w(pq.chunk_w, [&](auto w) {
      constexpr int MW = decltype(mw)::value;
      constexpr int kBatch = MW == 0 ? 4 : (MW <= 2 ? 8 : 4);
      hipLaunchKernelGGL((pq_adc_scan_kernel<MW, decltype(w)::value, kBatch>), dim3(nq), dim3(256),
                         smem, stream, pq, q, nq, ids, S, out);
      return hipGetLastError();
    });
  });
}

hipError_t launch_nav_entry(const NavDev& nav, int dtype, int64_t medoid, int64_t num_pts, int dim,
                            const float* q, int nq, int32_t* entries, int32_t* local_out,
                            int32_t* fallback_count, hipStream_t stream) {
  size_t smem = (size_t)dim * 4;
  if (dtype == 0)
    hipLaunchKernelGGL(nav_entry_kernel<uint8_t>, dim3(nq), dim3(64), smem, stream, nav, medoid,
                       num_pts, dim, q, nq, entries, local_out, fallback_count);
  else
    hipLaunchKernelGGL(nav_entry_kernel<float>, dim3(nq), dim3(64), smem, stream, nav, medoid,
                       num_pts, dim, q, nq, entries, local_out, fallback_count);
  return hipGetLastError();
}

hipError_t launch_query_order(const IndexDev& ix, int dtype, const float* q, int nq, const int32_t* entries,
                              float* entry_dist, int32_t* order, hipStream_t stream) {
  if (nq <= 0) return hipSuccess;
  const dim3 grid((unsigned)((nq + 255) / 256));
  if (dtype == 0)
    hipLaunchKernelGGL(entry_dist_kernel<uint8_t>, grid, dim3(256), 0, stream, ix, q, nq, entries, entry_dist);
  else
    hipLaunchKernelGGL(entry_dist_kernel<float>, grid, dim3(256), 0, stream, ix, q, nq, entries, entry_dist);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(query_order_kernel, dim3(1), dim3(kOrderThreads), 0, stream, entry_dist, nq, order);
  return hipGetLastError();
}

hipError_t launch_search(const IndexDev& ix, const PQDev& pq, int dtype, const float* q, int nq,
                         const int32_t* entries, int topk, int L, int32_t* nns, float* dists,
                         int32_t* found, int32_t* n_exp, int32_t* n_adc, hipStream_t stream) {
  if (dtype == 0)
    return launch_search_lut_u8(ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, stream);
  return launch_search_lut_f32(ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, stream);
}

int search_cb_waves(int dim, int M, int chunk_w, int L, int topk, size_t lds_limit, bool global_pivots,
                    int lds_groups) {
  const size_t piv = global_pivots ? split_pivot_bytes(lds_groups, chunk_w) : CbSmem::pivot_bytes(dim);
  const size_t w = CbSmem::wave_bytes(L, topk);
  if (piv + w > lds_limit) return 0;
  const int cap = cb_block_threads(cb_rerank_regs(M, chunk_w, dim), global_pivots ? lds_groups : 0) / kWave;
  return (int)std::min<size_t>((size_t)cap, (lds_limit - piv) / w);
}

int search_cb_split_groups(int M, int chunk_w) {
  return (mw_of(M) > 0 && (chunk_w == 2 || chunk_w == 4)) ? M / 8 : 0;
}

int search_cb_wide_lds_chunks(int chunk_w, int L, int topk, size_t lds_limit, int waves, int R) {
  if (R > kWave || chunk_w <= 0) return 0;
  const size_t used = (size_t)waves * CbSmem::wave_bytes(L, topk);
  if (used >= lds_limit) return 0;
  return (int)std::min<size_t>((size_t)kCbMaxWideLds, (lds_limit - used) / cb_wide_lds_bytes(1, chunk_w));
}

bool search_cb_wide_ok(int M, int chunk_w, int dim) {
  const int mw = mw_of(M);
  return mw > 0 && (chunk_w == 2 || chunk_w == 4) && 16 * mw * chunk_w <= 128 && dim == M * chunk_w;
}

size_t search_cb_pivot_bytes(int dim) { return CbSmem::pivot_bytes(dim); }

void search_cb_pivot_layout(const float* pivots, int dim, uint8_t* out) {
  const uint32_t rowb = cb_stride(4 * dim);
  std::fill(out, out + CbSmem::pivot_bytes(dim), (uint8_t)0);
  for (uint32_t c = 0; c < (uint32_t)kPivots; ++c)
    std::copy(reinterpret_cast<const uint8_t*>(pivots + (size_t)c * dim),
              reinterpret_cast<const uint8_t*>(pivots + (size_t)(c + 1) * dim), out + (size_t)c * rowb);
}

namespace {
// Queue counter to 0 and q - mu of every query, the set-up of the
// shared-codebook kernels.
hipError_t prepare_cb(const IndexDev& ix, const PQDev& pq, const float* q, int nq, int32_t* queue,
                      float* qs_all, hipStream_t stream) {
  hipError_t e = launch_fill_i32(queue, 1, 0, stream);
  if (e != hipSuccess) return e;
  const int64_t n = (int64_t)nq * ix.dim;
  hipLaunchKernelGGL(query_centre_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, q,
                     pq.centroid, n, ix.dim, qs_all);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_search_cb(const IndexDev& ix, const PQDev& pq, int dtype, const float* q, int nq,
                            const int32_t* entries, int topk, int L, int32_t* nns, float* dists,
                            int32_t* found, int32_t* n_exp, int32_t* n_adc, int32_t* queue,
                            const int32_t* order, float* qs_all, int waves, int blocks, bool global_pivots, int lds_groups,
                            hipStream_t stream) {
  if (global_pivots && !pq.piv_cb) return hipErrorInvalidValue;
  const int split = search_cb_split_groups(pq.M, pq.chunk_w);
  if (cb_is_wide(lds_groups)) {
    if (!global_pivots || !search_cb_wide_ok(pq.M, pq.chunk_w, ix.dim)) return hipErrorInvalidValue;
    if (cb_wide_lds(lds_groups) > 0 && ix.R > kWave) return hipErrorInvalidValue;
  } else if (lds_groups != 0 && (!global_pivots || (lds_groups != split - 1 && lds_groups != split / 2))) {
    return hipErrorInvalidValue;
  }
  const size_t smem = (global_pivots ? split_pivot_bytes(lds_groups, pq.chunk_w) : CbSmem::pivot_bytes(ix.dim)) +
                      cb_wide_lds_bytes(cb_wide_lds(lds_groups), pq.chunk_w) +
                      (size_t)waves * CbSmem::wave_bytes(L, topk);
  hipError_t e = prepare_cb(ix, pq, q, nq, queue, qs_all, stream);
  if (e != hipSuccess) return e;
  if (dtype == 0)
    return launch_search_cb_u8(ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, queue, order, qs_all,
                               waves, blocks, global_pivots, lds_groups, smem, stream);
  return launch_search_cb_f32(ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, queue, order, qs_all,
                              waves, blocks, global_pivots, lds_groups, smem, stream);
}

hipError_t launch_search_beam(const IndexDev& ix, const PQDev& pq, int dtype, const float* q, int nq,
                              const int32_t* entries, int topk, int L, int bw, int32_t* nns,
                              float* dists, int32_t* found, int32_t* n_exp, int32_t* n_adc,
                              int32_t* queue, const int32_t* order, float* qs_all, int waves, int blocks,
                              bool global_pivots, hipStream_t stream) {
  if (bw < 2 || bw > kMaxBeam) return hipErrorInvalidValue;
  if (global_pivots && !pq.piv_cb) return hipErrorInvalidValue;
  const size_t smem = (global_pivots ? 0 : CbSmem::pivot_bytes(ix.dim)) +
                      (size_t)waves * CbSmem::wave_bytes(L, topk);
  hipError_t e = prepare_cb(ix, pq, q, nq, queue, qs_all, stream);
  if (e != hipSuccess) return e;
  if (dtype == 0)
    return launch_search_beam_u8(ix, pq, q, nq, entries, topk, L, bw, nns, dists, found, n_exp, n_adc, queue, order,
                                 qs_all, waves, blocks, global_pivots, smem, stream);
  return launch_search_beam_f32(ix, pq, q, nq, entries, topk, L, bw, nns, dists, found, n_exp, n_adc, queue, order,
                                qs_all, waves, blocks, global_pivots, smem, stream);
}

int max_beam_width() { return kMaxBeam; }

hipError_t launch_gather_rows(const uint8_t* rows, int64_t num_rows, int row_bytes,
                              const int32_t* ids, int64_t n, uint32_t* out, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 256 * 8 - 1) / (256 * 8)));
  const u32x4* r = reinterpret_cast<const u32x4*>(rows);
  switch (row_bytes) {
    case 16:
      hipLaunchKernelGGL(gather_rows_kernel<1>, grid, dim3(256), 0, stream, r, num_rows, ids, n, out);
      break;
    case 32:
      hipLaunchKernelGGL(gather_rows_kernel<2>, grid, dim3(256), 0, stream, r, num_rows, ids, n, out);
      break;
    case 48:
      hipLaunchKernelGGL(gather_rows_kernel<3>, grid, dim3(256), 0, stream, r, num_rows, ids, n, out);
      break;
    case 64:
      hipLaunchKernelGGL(gather_rows_kernel<4>, grid, dim3(256), 0, stream, r, num_rows, ids, n, out);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

size_t step_state_bytes() { return sizeof(StepState); }
int32_t step_state_node(const void* host_states, int64_t i) {
  return reinterpret_cast<const StepState*>(host_states)[i].u;
}

hipError_t launch_step_init(const PQDev& pq, const float* q, int nq, const int32_t* entries,
                            float* luts, void* st, hipStream_t stream) {
  return with_w(pq.chunk_w, [&](auto w) {
    hipLaunchKernelGGL((step_init_kernel<decltype(w)::value>), dim3(nq), dim3(64),
                       (size_t)pq.dim * 4, stream, pq, q, nq, pq.num_pts, entries, luts,
                       reinterpret_cast<StepState*>(st));
    return hipGetLastError();
  });
}

hipError_t launch_step_round(const IndexDev& ix, const PQDev& pq, int dtype, const float* q, int nq,
                             const float* luts, int topk, int L, uint64_t* lists, void* st,
                             int32_t* nns, float* dists, int32_t* active, const uint8_t* slots,
                             hipStream_t stream) {
  StepState* s = reinterpret_cast<StepState*>(st);
  if (dtype == 0)
    return launch_round_u8(ix, pq, q, nq, luts, topk, L, lists, s, nns, dists, active, slots, stream);
  return launch_round_f32(ix, pq, q, nq, luts, topk, L, lists, s, nns, dists, active, slots, stream);
}

hipError_t launch_step_finish(int nq, int topk, const void* st, int32_t* nns, float* dists,
                              int32_t* found, int32_t* n_exp, int32_t* n_adc, hipStream_t stream) {
  hipLaunchKernelGGL(step_finish_kernel, dim3(nq), dim3(64), 0, stream, nq, topk,
                     reinterpret_cast<const StepState*>(st), nns, dists, found, n_exp, n_adc);
  return hipGetLastError();
}

hipError_t launch_fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p,
                     n, v);
  return hipGetLastError();
}

// ------------------------------------------------------------------ fixed scratch

// Scratch of the allocation-free search entry point: its counters (entry
// fallback count, query queue) and q - centroid of every query.  Each GPU
// that loads this library holds its own copy until the process ends.  In
// host code the name `scratch` is not a device address: the copy of the
// current device is resolved below with hipGetSymbolAddress, and only that
// pointer is handed to kernels and fills.
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_dev;  // per device id
}  // namespace

hipError_t noalloc_scratch_setup(int device, void** out) {
  if (device < 0 || !out) return hipErrorInvalidValue;
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if ((size_t)device >= g_scratch_dev.size()) g_scratch_dev.resize((size_t)device + 1, nullptr);
  if (!g_scratch_dev[(size_t)device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_dev[(size_t)device] = p;
  }
  *out = g_scratch_dev[(size_t)device];
  return hipSuccess;
}

}  // namespace gann

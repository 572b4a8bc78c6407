// GustANN search kernels for MI355X (gfx950, wave64).
//
//  * pq_lut_kernel      : LUT build only (src/impl/pq.cuh:8-59), one
//                         workgroup per query, LUT written to HBM.
//  * pq_adc_scan_kernel : LUT build staged in LDS + ADC gather-scan over a
//                         list of candidate ids per query
//                         (src/impl/pure_mem.cuh:300-310 applied to an id list).
//  * nav_entry_kernel   : pivot-graph entry selection (src/impl/nav.cuh:13-135)
//                         with the map.txt translation (src/nav_graph.cu:104-109)
//                         done on the device.
//  * search_kernel      : the fused beam search of
//                         src/impl/pure_mem.cuh:243-432, one wavefront per
//                         query, LUT + candidate list + top-k in LDS.
//  * step_round_kernel  : one expansion round of the step-wise form
//                         (src/impl/hyd_search_v2.cuh:8-472) with the list in HBM.
#include "gann_kernels.hpp"

#include <hip/hip_runtime.h>

#include <climits>
#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

#include "gann_device.hpp"
#include "gann_list.hpp"

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

// ------------------------------------------------------------------ beam search

__device__ __forceinline__ const uint8_t* record_of(const IndexDev& ix, int64_t u) {
  return ix.pages + (u / ix.nodes_per_page) * 4096 + (u % ix.nodes_per_page) * ix.node_len;
}

// One node record held in registers: its degree, this lane's neighbour id
// and, in lanes 0..31, the coordinates l, l+32, ... that the exact rerank of
// lane l reads (square_sum_32's lane roles).  Loads are issued by load() and
// consumed one expansion later, so their latency overlaps the list update.
template <typename T, int kPer>
struct RecRegs {
  int deg_raw;
  uint32_t v;
  T x[kPer];
  __device__ __forceinline__ void load(const IndexDev& ix, int64_t u) { load_at(ix, record_of(ix, u)); }
  __device__ __forceinline__ void load_at(const IndexDev& ix, const uint8_t* rec) {
    const int lane = lane_id();
    deg_raw = *reinterpret_cast<const int32_t*>(rec + ix.data_len);
    const uint32_t* edge = reinterpret_cast<const uint32_t*>(rec + ix.data_len + 4);
    v = lane < ix.R ? edge[lane] : 0u;
    const T* xs = reinterpret_cast<const T*>(rec);
    const int l = lane & 31;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = l + 32 * k;
      x[k] = i < ix.dim ? xs[i] : T(0);
    }
  }
  // square_sum_32 (src/impl/util.cuh:26-46) from the registers: lane l's
  // partial over dims l, l+32, ... then the 16/8/4/2/1 tree read at lane 0.
  // qv[k] holds the restored query at dim l + 32k.
  __device__ __forceinline__ float l2(const float (&qv)[kPer], int dim) const {
    const int l = lane_id() & 31;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = l + 32 * k;
      if (i < dim) {
        const float d = qv[k] - to_f(x[k]);
        acc = fma_f(d, d, acc);
      }
    }
    return square_sum_tree(acc);
  }
};

// LDS carve-up of the fused kernel (bytes): LUT | qr | list A (L) | list
// scratch | top-k dists | top-k ids.
struct SearchSmem {
  static __host__ __device__ size_t bytes(int M, int dim, int L, int R, int k) {
    (void)R;
    return (size_t)M * kPivots * 4 + (size_t)((dim + 1) & ~1) * 4 + (size_t)L * 8 +
           (size_t)list_scratch_words(L) * 4 + (size_t)k * 8;
  }
};

constexpr int kMaxDimRegs = 8;  // rerank coordinates per lane: dim <= 256

// The restored query fl(fl(q - mu) + mu) (src/impl/pq.cuh:22-24, 54-56) in
// the rerank lane roles: lane l holds dims l, l+32, ...
template <int N>
__device__ __forceinline__ void restored_query_regs(const float* q, const float* centroid, int dim,
                                                    float (&qv)[N]) {
  const int l = lane_id() & 31;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const int i = l + 32 * k;
    float v = 0.0f;
    if (i < dim) {
      const float t = q[i] - centroid[i];
      v = t + centroid[i];
    }
    qv[k] = v;
  }
}

template <typename T, int MW, int W>
__global__ __launch_bounds__(64) void search_kernel(IndexDev ix, PQDev pq,
                                                    const float* __restrict__ q, int nq,
                                                    const int32_t* __restrict__ entries, int topk,
                                                    int L, int32_t* __restrict__ nns,
                                                    float* __restrict__ dists,
                                                    int32_t* __restrict__ found_cnt,
                                                    int32_t* __restrict__ n_exp,
                                                    int32_t* __restrict__ n_adc) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  const int qi = blockIdx.x;
  if (qi >= nq) return;
  const int lane = lane_id();
  const int dim = ix.dim, M = pq.M, R = ix.R;
  float* lut = reinterpret_cast<float*>(smem_raw);
  float* qr = lut + M * kPivots;
  uint64_t* A = reinterpret_cast<uint64_t*>(qr + ((dim + 1) & ~1));
  uint32_t* BM = reinterpret_cast<uint32_t*>(A + L);
  float* td = reinterpret_cast<float*>(BM + list_scratch_words(L));
  int32_t* ti = reinterpret_cast<int32_t*>(td + topk);

  int32_t u = __builtin_amdgcn_readfirstlane(entries[qi]);
  if (u >= ix.num_pts) u = -1;  // caller-given entries outside the index: empty result
  RecRegs<T, kMaxDimRegs> cur;
  if (u >= 0) cur.load(ix, u);

  // q - mu for the LUT build (src/impl/pq.cuh:22-24) and the restored query
  // the rerank reads
  const float* qq = q + (int64_t)qi * dim;
  for (int i = lane; i < dim; i += kWave) qr[i] = qq[i] - pq.centroid[i];
  float qv[kMaxDimRegs];
  restored_query_regs(qq, pq.centroid, dim, qv);
  __syncthreads();
  lut_build<W>(pq, qr, lut, lane, kWave);
  __syncthreads();

  int sz = 0, fu = 0;
  TopK top(td, ti, topk);
  int32_t exps = 0, adcs = 0;
  const int64_t cap = ix.num_pts + 2;
  while (u >= 0 && exps < cap) {
    ++exps;
    const int deg = __builtin_amdgcn_readfirstlane(min(max(cur.deg_raw, 0), R));
    adcs += deg;
    uint64_t key = ~(uint64_t)0;  // padding sorts last
    if (lane < deg) {
      CodeRow<MW> row;
      const uint8_t* crow = pq.codes + (int64_t)cur.v * M;
      row.load(crow, M);
      key = make_key(row.adc(lut, crow, M), cur.v);
    }
    // exact rerank of u (independent of the list update; :420-423)
    const float du = cur.l2(qv, dim);
    const ListPlan P = list_plan(A, L, key, deg, sz, fu);
    const int32_t next =
        __builtin_amdgcn_readfirstlane(P.cand >= 0 ? (int32_t)entry_id(P.sel) : -1);
    RecRegs<T, kMaxDimRegs> nxt;
    if (next >= 0) nxt.load(ix, next);
    fu = list_apply(A, BM, P);
    sz = P.nsz;
    top.push(du, u);
    u = next;
    cur = nxt;
  }
  top.store(nns, dists, qi);
  if (lane == 0) {
    found_cnt[qi] = top.found;
    if (n_exp) n_exp[qi] = exps;
    if (n_adc) n_adc[qi] = adcs;
  }
}

// ------------------------------------------------------------------ beam search, shared codebook

// The same search with no per-query LUT: the 256 x dim pivot table sits once
// in each CU's LDS, shared by up to 16 wavefronts (one query each), and every
// neighbour's ADC distance is computed directly from the pivots.  For chunk
// m and code c it accumulates fma((q_i - mu_i) - P[c][i])^2 over the chunk's
// dims in ascending order from 0 -- exactly the operations that build
// LUT[m][c] (src/impl/pq.cuh:35-43) -- then sums the chunks in order
// (src/impl/pure_mem.cuh:306-308), so the distances are bit-identical to the
// LUT path while a query needs only its list, query vector and top-k in LDS.
//
// Pivot row c (the dim floats of code c) starts at byte c*(4*dim + 16): the
// 16 bytes of padding per row move consecutive rows 4 banks apart, which
// spreads the lanes of a wave (random rows, same chunk) over the LDS banks;
// a row address is one 24-bit multiply of the code byte (the compiler folds
// the byte select into it), and a chunk's offset inside its row stays a
// compile-time immediate of the LDS read.

// Row stride of the shared-codebook pivot layout for rows of `row_bytes`
// bytes of floats.
__host__ __device__ constexpr uint32_t cb_stride(int row_bytes) { return (uint32_t)row_bytes + 16u; }

struct CbSmem {
  // per-wave bytes: list (L) | list scratch | top-k d, top-k id (LDS only
  // when k > 64; smaller top-k lists live in registers)
  static __host__ __device__ size_t wave_bytes(int dim, int L, int k) {
    (void)dim;
    size_t b = (size_t)L * 8 + (size_t)list_scratch_words(L) * 4 + (k > kWave ? (size_t)k * 8 : 0);
    return (b + 15) & ~(size_t)15;
  }
  static __host__ __device__ size_t pivot_bytes(int dim) { return (size_t)kPivots * cb_stride(4 * dim); }
};

// LDS bytes of the first g groups of 8 chunks of W dims, in the cb_row layout.
__host__ __device__ constexpr size_t split_pivot_bytes(int g, int W) {
  return g > 0 ? (size_t)kPivots * cb_stride(g * 8 * W * 4) : 0;
}

// Byte offset of pivot row c in a table whose rows are `stride` bytes apart
// (stride = cb_stride(bytes of the row's floats)).
__device__ __forceinline__ uint32_t cb_row(uint32_t c, uint32_t stride) {
  return __umul24(c, stride);
}

// q - mu of every query (src/impl/pq.cuh:22-24), read back with uniform
// (scalar) loads by the shared-codebook ADC.
__global__ void query_centre_kernel(const float* __restrict__ q, const float* __restrict__ centroid,
                                    int64_t n, int dim, float* __restrict__ qs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) qs[i] = q[i] - centroid[i % dim];
}

// Chunk distance of pivot vector p against q - mu, accumulated over the
// chunk's dims in ascending order from 0 as the LUT build does.
template <int W>
__device__ __forceinline__ float cb_chunk(const float* qc, const float* p) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < W; ++i) {
    const float d = qc[i] - p[i];
    acc = fma_f(d, d, acc);
  }
  return acc;
}

template <int W>
struct PivotVec;
template <>
struct PivotVec<4> {
  typedef float __attribute__((ext_vector_type(4))) type;
};
template <>
struct PivotVec<2> {
  typedef float __attribute__((ext_vector_type(2))) type;
};

// ADC distance of one code row from the pivots in LDS (piv: byte base of the
// table, rowb = cb_stride(4*dim)).  The pivot reads of 8 chunks are issued together;
// q - mu is read 8 chunks at a time with uniform loads from qs, whose
// address is made opaque per group so the compiler does not keep all of it
// in scalar registers across expansions.
// kSplitG > 0: groups of 8 chunks below kSplitG come from the partial
// table pivl in LDS (rows of kSplitG * 8 * W floats), the others from piv.
// kSplitLds: read the partial table from LDS address 0 as well (pivl is the
// start of the dynamic LDS).  The compiler then keeps more reads in flight;
// with 8 rerank slots per lane that spills registers (1024-lane workgroups
// cap a kernel at 128 VGPRs), so only the 4-slot kernels (dim <= 128) do.
// kPivLds: piv is the whole table in LDS, at the beginning of the dynamic
// LDS, which is LDS address 0: the kernels that call this declare no static
// LDS, and their launchers check that with hipFuncGetAttributes.  Reading
// LDS rows by their address from 0 leaves the row address as one 24-bit
// multiply of the code byte (the compiler folds the byte select into it); an
// offset from the dynamic LDS symbol costs a second VALU operation per chunk.
template <typename PV>
__device__ __forceinline__ PV lds_at(uint32_t a) {
  return *reinterpret_cast<const __attribute__((address_space(3))) PV*>((size_t)a);
}

template <int W, int MW, int kSplitG = 0, bool kPivLds = false, bool kSplitLds = false>
__device__ __forceinline__ float cb_adc(const uint8_t* piv, const float* qs, uint32_t rowb,
                                        const PQDev& pq, const CodeRow<MW>& row,
                                        const uint8_t* crow, const uint8_t* pivl = nullptr) {
  float dist = 0.0f;
  if constexpr (MW > 0 && (W == 4 || W == 2)) {
    typedef typename PivotVec<W>::type PV;
#pragma unroll
    for (int k = 0; k < MW; ++k) {
      const uint32_t ws[4] = {row.w[k].x, row.w[k].y, row.w[k].z, row.w[k].w};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        PV p[8];
        const bool from_lds = 2 * k + h < kSplitG;  // compile-time
        const uint32_t stride = from_lds ? cb_stride(kSplitG * 8 * W * 4) : rowb;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const int bb = 8 * h + b;
          const uint32_t c = (ws[bb >> 2] >> (8 * (bb & 3))) & 0xffu;
          const uint32_t off = cb_row(c, stride) + (16 * k + bb) * W * 4;
          if (kPivLds || (from_lds && kSplitLds))
            p[b] = lds_at<PV>(off);  // a table at LDS address 0 (whole, or partial)
          else
            p[b] = *reinterpret_cast<const PV*>((from_lds ? pivl : piv) + off);
        }
        // uniform address in the constant address space: scalar loads
        uint64_t qa = (uint64_t)(qs + (16 * k + 8 * h) * W);
        asm volatile("" : "+s"(qa));
        const __attribute__((address_space(4))) float* qg =
            (const __attribute__((address_space(4))) float*)qa;
        float qv[8 * W];
#pragma unroll
        for (int i = 0; i < 8 * W; ++i) qv[i] = qg[i];
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          float pv[W];
#pragma unroll
          for (int i = 0; i < W; ++i) pv[i] = p[b][i];
          dist = dist + cb_chunk<W>(qv + b * W, pv);
        }
      }
    }
  } else {
    const float* pf = reinterpret_cast<const float*>(piv);
    for (int m = 0; m < pq.M; ++m) {
      const uint32_t base = cb_row(crow[m], rowb) / 4;
      float acc = 0.0f;
      for (int i = pq.chunk_off[m]; i < pq.chunk_off[m + 1]; ++i) {
        const float d = qs[i] - pf[base + i];
        acc = fma_f(d, d, acc);
      }
      dist = dist + acc;
    }
  }
  return dist;
}

// kGP: the pivot table is read from pq.piv_cb (HBM, through the caches)
// instead of a copy in LDS, which then holds only the per-wave lists: the
// form for large L, where lists beside a 128 KB table leave few waves.
// KP: rerank coordinates per lane (dim <= 32 * KP).
template <typename T, int MW, int W, bool kGP, int kSplitG = 0, int KP = kMaxDimRegs>
__global__ __launch_bounds__(1024) void search_cb_kernel(IndexDev ix, PQDev pq,
                                                         const float* __restrict__ q, int nq,
                                                         const int32_t* __restrict__ entries,
                                                         int topk, int L, int32_t* __restrict__ nns,
                                                         float* __restrict__ dists,
                                                         int32_t* __restrict__ found_cnt,
                                                         int32_t* __restrict__ n_exp,
                                                         int32_t* __restrict__ n_adc,
                                                         int32_t* __restrict__ queue,
                                                         const float* __restrict__ qs_all) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  const int dim = ix.dim, M = pq.M, R = ix.R;
  const uint32_t rowb = cb_stride(4 * dim);
  const uint8_t* piv;
  size_t lists_at = 0;
  if constexpr (kGP) {
    piv = (const uint8_t*)((const __attribute__((address_space(1))) uint8_t*)pq.piv_cb);
    if constexpr (kSplitG > 0) {
      // the first kSplitG groups of 8 chunks also in LDS
      constexpr int per_row = kSplitG * 8 * W;
      for (int idx = threadIdx.x; idx < kPivots * per_row; idx += blockDim.x) {
        const int c = idx / per_row, i = idx - c * per_row;
        *reinterpret_cast<float*>(smem_raw + cb_row((uint32_t)c, cb_stride(per_row * 4)) + 4 * i) = pq.pivots[c * dim + i];
      }
      __syncthreads();
      lists_at = split_pivot_bytes(kSplitG, W);
    }
  } else {
    piv = smem_raw;
    lists_at = CbSmem::pivot_bytes(dim);
    // pivot table (whole workgroup), the only workgroup barrier
    for (int idx = threadIdx.x; idx < kPivots * dim; idx += blockDim.x) {
      const int c = idx / dim, i = idx - c * dim;
      *reinterpret_cast<float*>(smem_raw + cb_row((uint32_t)c, rowb) + 4 * i) = pq.pivots[idx];
    }
    __syncthreads();
  }

  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  uint8_t* wbase = smem_raw + lists_at + (size_t)wave * CbSmem::wave_bytes(dim, L, topk);
  uint64_t* A = reinterpret_cast<uint64_t*>(wbase);
  uint32_t* BM = reinterpret_cast<uint32_t*>(A + L);
  float* td = reinterpret_cast<float*>(BM + list_scratch_words(L));
  int32_t* ti = reinterpret_cast<int32_t*>(td + topk);
  const int64_t cap = ix.num_pts + 2;

  for (;;) {
    int qi = 0;
    if (lane == 0) qi = atomicAdd(queue, 1);
    qi = __builtin_amdgcn_readfirstlane(__shfl(qi, 0, kWave));
    if (qi >= nq) break;
    int32_t u = __builtin_amdgcn_readfirstlane(entries[qi]);
    if (u >= ix.num_pts) u = -1;  // caller-given entries outside the index: empty result
    RecRegs<T, KP> cur;
    if (u >= 0) cur.load(ix, u);
    const float* qs = qs_all + (int64_t)qi * dim;  // q - mu, uniform reads
    float qv[KP];
    restored_query_regs(q + (int64_t)qi * dim, pq.centroid, dim, qv);
    int sz = 0, fu = 0;
    TopK top(td, ti, topk);
    int32_t exps = 0, adcs = 0;
    while (u >= 0 && exps < cap) {
      ++exps;
      const int deg = __builtin_amdgcn_readfirstlane(min(max(cur.deg_raw, 0), R));
      adcs += deg;
      uint64_t key = ~(uint64_t)0;  // padding sorts last
      if (lane < deg) {
        CodeRow<MW> row;
        const uint8_t* crow = pq.codes + (int64_t)cur.v * M;
        row.load(crow, M);
        key = make_key(cb_adc<W, MW, kSplitG, !kGP, (KP <= 4)>(piv, qs, rowb, pq, row, crow, smem_raw), cur.v);
      }
      const float du = cur.l2(qv, dim);
      const ListPlan P = list_plan(A, L, key, deg, sz, fu);
      const int32_t next =
          __builtin_amdgcn_readfirstlane(P.cand >= 0 ? (int32_t)entry_id(P.sel) : -1);
      RecRegs<T, KP> nxt;
      if (next >= 0) nxt.load(ix, next);
      fu = list_apply(A, BM, P);
      sz = P.nsz;
      top.push(du, u);
      u = next;
      cur = nxt;
    }
    top.store(nns, dists, qi);
    if (lane == 0) {
      found_cnt[qi] = top.found;
      if (n_exp) n_exp[qi] = exps;
      if (n_adc) n_adc[qi] = adcs;
    }
    wave_sync();
  }
}

// ------------------------------------------------------------------ beam search, beam width > 1

// Beam search with beam width bw (2..kMaxBeam), a mode the reference does not
// have (it expands one node per iteration; this mode is reported beside it
// with its own recall).  Each round takes the first bw unvisited list entries
// at once, marks them visited and loads their records together, then expands
// them in list order: every expansion merges its neighbours into the list
// with the same rank / sort / gather update as search_cb_kernel and pushes
// the node's exact distance into the top-k.  The code rows of the next node
// of the round are fetched while the current one is merged.  The search ends
// when no unvisited entry is left.  LDS layout and query queue as in
// search_cb_kernel; KP rerank coordinates per lane (dim <= 32 * KP).
constexpr int kMaxBeam = 4;

template <typename T, int MW, int W, int KP, bool kGP>
__global__ __launch_bounds__(1024) void search_beam_kernel(IndexDev ix, PQDev pq,
                                                           const float* __restrict__ q, int nq,
                                                           const int32_t* __restrict__ entries,
                                                           int topk, int L, int bw,
                                                           int32_t* __restrict__ nns,
                                                           float* __restrict__ dists,
                                                           int32_t* __restrict__ found_cnt,
                                                           int32_t* __restrict__ n_exp,
                                                           int32_t* __restrict__ n_adc,
                                                           int32_t* __restrict__ queue,
                                                           const float* __restrict__ qs_all) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  const int dim = ix.dim, M = pq.M, R = ix.R;
  const uint32_t rowb = cb_stride(4 * dim);
  const uint8_t* piv;
  size_t lists_at = 0;
  if constexpr (kGP) {
    piv = (const uint8_t*)((const __attribute__((address_space(1))) uint8_t*)pq.piv_cb);
  } else {
    piv = smem_raw;
    lists_at = CbSmem::pivot_bytes(dim);
    for (int idx = threadIdx.x; idx < kPivots * dim; idx += blockDim.x) {
      const int c = idx / dim, i = idx - c * dim;
      *reinterpret_cast<float*>(smem_raw + cb_row((uint32_t)c, rowb) + 4 * i) = pq.pivots[idx];
    }
    __syncthreads();
  }

  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  uint8_t* wbase = smem_raw + lists_at + (size_t)wave * CbSmem::wave_bytes(dim, L, topk);
  uint64_t* A = reinterpret_cast<uint64_t*>(wbase);
  uint32_t* BM = reinterpret_cast<uint32_t*>(A + L);
  float* td = reinterpret_cast<float*>(BM + list_scratch_words(L));
  int32_t* ti = reinterpret_cast<int32_t*>(td + topk);
  const int64_t cap = ix.num_pts + 2;

  for (;;) {
    int qi = 0;
    if (lane == 0) qi = atomicAdd(queue, 1);
    qi = __builtin_amdgcn_readfirstlane(__shfl(qi, 0, kWave));
    if (qi >= nq) break;
    const float* qs = qs_all + (int64_t)qi * dim;
    float qv[KP];
    restored_query_regs(q + (int64_t)qi * dim, pq.centroid, dim, qv);
    int sz = 0, fu = 0;
    TopK top(td, ti, topk);
    int32_t exps = 0, adcs = 0;
    int32_t sel[kMaxBeam];
#pragma unroll
    for (int b = 0; b < kMaxBeam; ++b) sel[b] = -1;
    sel[0] = __builtin_amdgcn_readfirstlane(entries[qi]);
    int nsel = sel[0] >= 0 && sel[0] < ix.num_pts ? 1 : 0;
    while (nsel > 0) {
      RecRegs<T, KP> rec[kMaxBeam];
#pragma unroll
      for (int b = 0; b < kMaxBeam; ++b)
        if (b < nsel) rec[b].load(ix, sel[b]);
      CodeRow<MW> rows[2];
      {
        const int d0 = __builtin_amdgcn_readfirstlane(min(max(rec[0].deg_raw, 0), R));
        if (lane < d0) rows[0].load(pq.codes + (int64_t)rec[0].v * M, M);
      }
#pragma unroll
      for (int b = 0; b < kMaxBeam; ++b) {
        if (b < nsel && exps < cap) {
          ++exps;
          const int deg = __builtin_amdgcn_readfirstlane(min(max(rec[b].deg_raw, 0), R));
          adcs += deg;
          if (b + 1 < kMaxBeam && b + 1 < nsel) {
            const int dn = __builtin_amdgcn_readfirstlane(min(max(rec[b + 1].deg_raw, 0), R));
            if (lane < dn) rows[(b + 1) & 1].load(pq.codes + (int64_t)rec[b + 1].v * M, M);
          }
          uint64_t key = ~(uint64_t)0;
          if (lane < deg) {
            const uint8_t* crow = pq.codes + (int64_t)rec[b].v * M;
            key = make_key(cb_adc<W, MW, 0, !kGP>(piv, qs, rowb, pq, rows[b & 1], crow), rec[b].v);
          }
          const float du = rec[b].l2(qv, dim);
          const ListPlan P = list_plan(A, L, key, deg, sz, fu);
          fu = list_apply<false>(A, BM, P);
          sz = P.nsz;
          top.push(du, sel[b]);
        }
      }
      // next round: the first bw unvisited entries at or after fu (every
      // entry before fu is visited)
      nsel = 0;
      if (exps < cap) {
        for (int base = fu; base < sz && nsel < bw; base += kWave) {
          const int i = base + lane;
          const uint64_t e = i < sz ? A[i] : kListVisited;
          uint64_t m = ballot64(!entry_visited(e));
          bool take = false;
          int last = -1;
          while (m != 0 && nsel < bw) {
            const int l = (int)__builtin_ctzll(m);
            m &= m - 1;
            const int32_t id = (int32_t)__builtin_amdgcn_readlane((int)entry_id(e), l);
#pragma unroll
            for (int t = 0; t < kMaxBeam; ++t)
              if (t == nsel) sel[t] = id;
            take |= lane == l;
            last = l;
            ++nsel;
          }
          if (take) A[i] = e | kListVisited;
          fu = nsel < bw ? min(base + kWave, sz) : base + last + 1;
        }
        wave_sync();
      }
    }
    top.store(nns, dists, qi);
    if (lane == 0) {
      found_cnt[qi] = top.found;
      if (n_exp) n_exp[qi] = exps;
      if (n_adc) n_adc[qi] = adcs;
    }
    wave_sync();
  }
}

// ------------------------------------------------------------------ step-wise

// Per-query state of the step-wise form, kept in HBM between rounds
// (the role of Data{visited_cnt,size} + request[] in src/impl/hyd.cuh:6-9,
// src/impl/hyd_search_v2.cuh:35, :450-458).
constexpr int64_t kStepSlotBytes = 4096;  // one index page per query slot

struct StepState {
  int32_t u;      // node to expand this round, -1 when done
  int32_t sz;     // list size
  int32_t fu;     // index of the first unvisited list entry (sz if none)
  int32_t found;  // top-k fill
  int32_t exps;   // expansions so far
  int32_t adcs;   // ADC evaluations so far
};

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

// One expansion per active query: the work of merge_data_kernel followed by
// unify_kernel (src/impl/hyd_search_v2.cuh:8-351, 353-472) in one launch;
// the candidate list and the top-k travel through HBM between rounds.
template <typename T, int MW>
__global__ __launch_bounds__(64) void step_round_kernel(IndexDev ix, PQDev pq,
                                                        const float* __restrict__ q, int nq,
                                                        const float* __restrict__ luts, int topk,
                                                        int L, uint64_t* __restrict__ lists,
                                                        StepState* __restrict__ st,
                                                        int32_t* __restrict__ nns,
                                                        float* __restrict__ dists,
                                                        int32_t* __restrict__ active,
                                                        const uint8_t* __restrict__ slots) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  const int qi = blockIdx.x;
  if (qi >= nq) return;
  StepState s = st[qi];
  if (s.u < 0) return;
  const int lane = lane_id();
  const int dim = ix.dim, M = pq.M, R = ix.R;
  float* qr = reinterpret_cast<float*>(smem_raw);
  uint64_t* A = reinterpret_cast<uint64_t*>(qr + ((dim + 1) & ~1));
  uint32_t* BM = reinterpret_cast<uint32_t*>(A + L);
  float* td = reinterpret_cast<float*>(BM + list_scratch_words(L));
  int32_t* ti = reinterpret_cast<int32_t*>(td + topk);
  const float* lut = luts + (int64_t)qi * M * kPivots;
  uint64_t* glist = lists + (int64_t)qi * L;

  const int32_t u = __builtin_amdgcn_readfirstlane(s.u);
  RecRegs<T, kMaxDimRegs> cur;
  // the record comes from the index pages, or from this query's 4096-byte
  // slot that the host filled with u's page (src/hyd_task_runner.cu:216-240)
  if (slots)
    cur.load_at(ix, slots + (int64_t)qi * kStepSlotBytes + (u % ix.nodes_per_page) * ix.node_len);
  else
    cur.load(ix, u);
  float qv[kMaxDimRegs];
  restored_query_regs(q + (int64_t)qi * dim, pq.centroid, dim, qv);
  for (int i = lane; i < s.sz; i += kWave) A[i] = glist[i];
  for (int j = lane; j < s.found; j += kWave) {
    td[j] = dists[(int64_t)qi * topk + j];
    ti[j] = nns[(int64_t)qi * topk + j];
  }
  __syncthreads();

  const int deg = __builtin_amdgcn_readfirstlane(min(max(cur.deg_raw, 0), R));
  uint64_t key = ~(uint64_t)0;
  if (lane < deg) {
    CodeRow<MW> row;
    const uint8_t* crow = pq.codes + (int64_t)cur.v * M;
    row.load(crow, M);
    key = make_key(row.adc(lut, crow, M), cur.v);
  }
  const float du = cur.l2(qv, dim);
  const ListPlan P = list_plan(A, L, key, deg, s.sz, s.fu);
  const int32_t next = P.cand >= 0 ? (int32_t)entry_id(P.sel) : -1;
  const int fu = list_apply(A, BM, P);
  const int sz = P.nsz;
  int found = s.found;
  topk_push(td, ti, &found, topk, du, u);

  for (int i = lane; i < sz; i += kWave) glist[i] = A[i];
  for (int j = lane; j < found; j += kWave) {
    dists[(int64_t)qi * topk + j] = td[j];
    nns[(int64_t)qi * topk + j] = ti[j];
  }
  if (lane == 0) {
    const int32_t exps = s.exps + 1;
    const bool done = next < 0 || exps >= ix.num_pts + 2;
    st[qi] = StepState{done ? -1 : next, sz, fu, found, exps, s.adcs + deg};
    if (done) atomicSub(active, 1);
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

namespace {
int mw_of(int M) {
  if (M % 16 != 0) return 0;
  const int mw = M / 16;
  return (mw >= 1 && mw <= 4) ? mw : 0;
}
int w_of(int chunk_w) { return (chunk_w == 2 || chunk_w == 4) ? chunk_w : 0; }

// Calls f(std::integral_constant<int, MW>{}) for the runtime code-row shape.
template <class F>
hipError_t with_mw(int M, F&& f) {
  switch (mw_of(M)) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 3: return f(std::integral_constant<int, 3>{});
    case 4: return f(std::integral_constant<int, 4>{});
    default: return f(std::integral_constant<int, 0>{});
  }
}
// Calls f(std::integral_constant<int, W>{}) for the runtime chunk width.
template <class F>
hipError_t with_w(int chunk_w, F&& f) {
  switch (w_of(chunk_w)) {
    case 2: return f(std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, 4>{});
    default: return f(std::integral_constant<int, 0>{});
  }
}
}  // namespace

size_t search_smem_bytes(int M, int dim, int L, int R, int topk) {
  return SearchSmem::bytes(M, dim, L, R, topk);
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

namespace {
template <typename T>
hipError_t launch_search_t(const IndexDev& ix, const PQDev& pq, const float* q, int nq,
                           const int32_t* entries, int topk, int L, int32_t* nns, float* dists,
                           int32_t* found, int32_t* n_exp, int32_t* n_adc, hipStream_t stream) {
  const size_t smem = SearchSmem::bytes(pq.M, ix.dim, L, ix.R, topk);
  return with_mw(pq.M, [&](auto mw) {
    return with_w(pq.chunk_w, [&](auto w) {
      hipLaunchKernelGGL((search_kernel<T, decltype(mw)::value, decltype(w)::value>), dim3(nq),
                         dim3(64), smem, stream, ix, pq, q, nq, entries, topk, L, nns, dists, found,
                         n_exp, n_adc);
      return hipGetLastError();
    });
  });
}

template <typename T>
hipError_t launch_round_t(const IndexDev& ix, const PQDev& pq, const float* q, int nq,
                          const float* luts, int topk, int L, uint64_t* lists, StepState* st,
                          int32_t* nns, float* dists, int32_t* active, const uint8_t* slots,
                          hipStream_t stream) {
  const size_t smem = (size_t)((ix.dim + 1) & ~1) * 4 + (size_t)L * 8 +
                      (size_t)list_scratch_words(L) * 4 + (size_t)topk * 8;
  return with_mw(pq.M, [&](auto mw) {
    hipLaunchKernelGGL((step_round_kernel<T, decltype(mw)::value>), dim3(nq), dim3(64), smem,
                       stream, ix, pq, q, nq, luts, topk, L, lists, st, nns, dists, active, slots);
    return hipGetLastError();
  });
}
}  // namespace

hipError_t launch_search(const IndexDev& ix, const PQDev& pq, int dtype, const float* q, int nq,
                         const int32_t* entries, int topk, int L, int32_t* nns, float* dists,
                         int32_t* found, int32_t* n_exp, int32_t* n_adc, hipStream_t stream) {
  if (dtype == 0)
    return launch_search_t<uint8_t>(ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp,
                                    n_adc, stream);
  return launch_search_t<float>(ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc,
                                stream);
}

int search_cb_waves(int dim, int L, int topk, size_t lds_limit, bool global_pivots, int lds_groups,
                    int chunk_w) {
  const size_t piv = global_pivots ? split_pivot_bytes(lds_groups, chunk_w) : CbSmem::pivot_bytes(dim);
  const size_t w = CbSmem::wave_bytes(dim, L, topk);
  if (piv + w > lds_limit) return 0;
  return (int)std::min<size_t>(16, (lds_limit - piv) / w);
}

int search_cb_split_groups(int M, int chunk_w) {
  return (mw_of(M) > 0 && (chunk_w == 2 || chunk_w == 4)) ? M / 8 : 0;
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
// The shared-codebook kernels address their LDS pivot tables (the whole
// table, or the partial table of a split form with 4 rerank slots per lane)
// from LDS address 0 (lds_at), which is where the dynamic LDS starts only
// when the kernel has no static LDS: refuse the launch otherwise (checked for
// every form, so that none gains static LDS unnoticed).
hipError_t check_dynamic_lds_at_zero(const void* fn) {
  hipFuncAttributes a{};
  const hipError_t e = hipFuncGetAttributes(&a, fn);
  if (e != hipSuccess) return e;
  return a.sharedSizeBytes == 0 ? hipSuccess : hipErrorInvalidDeviceFunction;
}

template <class K, class F>
hipError_t launch_checked(K* fn, F&& launch) {
  const hipError_t e = check_dynamic_lds_at_zero(reinterpret_cast<const void*>(fn));
  if (e != hipSuccess) return e;
  launch();
  return hipGetLastError();
}
}  // namespace

hipError_t launch_search_cb(const IndexDev& ix, const PQDev& pq, int dtype, const float* q, int nq,
                            const int32_t* entries, int topk, int L, int32_t* nns, float* dists,
                            int32_t* found, int32_t* n_exp, int32_t* n_adc, int32_t* queue,
                            float* qs_all, int waves, int blocks, bool global_pivots, int lds_groups,
                            hipStream_t stream) {
  if (global_pivots && !pq.piv_cb) return hipErrorInvalidValue;
  const int split = search_cb_split_groups(pq.M, pq.chunk_w);
  if (lds_groups != 0 && (!global_pivots || (lds_groups != split - 1 && lds_groups != split / 2)))
    return hipErrorInvalidValue;
  const size_t smem = (global_pivots ? split_pivot_bytes(lds_groups, pq.chunk_w) : CbSmem::pivot_bytes(ix.dim)) +
                      (size_t)waves * CbSmem::wave_bytes(ix.dim, L, topk);
  hipError_t e = launch_fill_i32(queue, 1, 0, stream);
  if (e != hipSuccess) return e;
  const int64_t n = (int64_t)nq * ix.dim;
  hipLaunchKernelGGL(query_centre_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, q,
                     pq.centroid, n, ix.dim, qs_all);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  auto go = [&](auto t, auto kp) {
    using T = decltype(t);
    constexpr int KPv = decltype(kp)::value;
    return with_mw(pq.M, [&](auto mw) {
      return with_w(pq.chunk_w, [&](auto w) {
        constexpr int MWv = decltype(mw)::value, Wv = decltype(w)::value;
        constexpr bool kCanSplit = MWv > 0 && (Wv == 2 || Wv == 4);
        constexpr int kSplit = kCanSplit ? 2 * MWv - 1 : 0, kHalf = kCanSplit ? MWv : 0;
        if (global_pivots && lds_groups > 0 && kCanSplit && lds_groups == kSplit)
          return launch_checked(&search_cb_kernel<T, MWv, Wv, true, kSplit, KPv>, [&] {
            hipLaunchKernelGGL((search_cb_kernel<T, MWv, Wv, true, kSplit, KPv>), dim3(blocks), dim3(waves * kWave),
                               smem, stream, ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc,
                               queue, qs_all);
          });
        if (global_pivots && lds_groups > 0 && kCanSplit && lds_groups == kHalf)
          return launch_checked(&search_cb_kernel<T, MWv, Wv, true, kHalf, KPv>, [&] {
            hipLaunchKernelGGL((search_cb_kernel<T, MWv, Wv, true, kHalf, KPv>), dim3(blocks), dim3(waves * kWave),
                               smem, stream, ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc,
                               queue, qs_all);
          });
        if (global_pivots)
          return launch_checked(&search_cb_kernel<T, MWv, Wv, true, 0, KPv>, [&] {
            hipLaunchKernelGGL((search_cb_kernel<T, MWv, Wv, true, 0, KPv>), dim3(blocks), dim3(waves * kWave), smem,
                               stream, ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, queue,
                               qs_all);
          });
        return launch_checked(&search_cb_kernel<T, MWv, Wv, false, 0, KPv>, [&] {
          hipLaunchKernelGGL((search_cb_kernel<T, MWv, Wv, false, 0, KPv>), dim3(blocks), dim3(waves * kWave), smem,
                             stream, ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, queue,
                             qs_all);
        });
      });
    });
  };
  // 4 rerank coordinates per lane cover dim <= 128 (fewer registers and no
  // idle rerank slots); larger dims take kMaxDimRegs
  const bool small = ix.dim <= 128;
  if (dtype == 0)
    return small ? go(uint8_t{}, std::integral_constant<int, 4>{})
                 : go(uint8_t{}, std::integral_constant<int, kMaxDimRegs>{});
  return small ? go(float{}, std::integral_constant<int, 4>{})
               : go(float{}, std::integral_constant<int, kMaxDimRegs>{});
}

hipError_t launch_search_beam(const IndexDev& ix, const PQDev& pq, int dtype, const float* q, int nq,
                              const int32_t* entries, int topk, int L, int bw, int32_t* nns,
                              float* dists, int32_t* found, int32_t* n_exp, int32_t* n_adc,
                              int32_t* queue, float* qs_all, int waves, int blocks,
                              bool global_pivots, hipStream_t stream) {
  if (bw < 2 || bw > kMaxBeam) return hipErrorInvalidValue;
  if (global_pivots && !pq.piv_cb) return hipErrorInvalidValue;
  const size_t smem = (global_pivots ? 0 : CbSmem::pivot_bytes(ix.dim)) +
                      (size_t)waves * CbSmem::wave_bytes(ix.dim, L, topk);
  hipError_t e = launch_fill_i32(queue, 1, 0, stream);
  if (e != hipSuccess) return e;
  const int64_t n = (int64_t)nq * ix.dim;
  hipLaunchKernelGGL(query_centre_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, q,
                     pq.centroid, n, ix.dim, qs_all);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  auto go = [&](auto t, auto kp) {
    using T = decltype(t);
    return with_mw(pq.M, [&](auto mw) {
      return with_w(pq.chunk_w, [&](auto w) {
        constexpr int MWv = decltype(mw)::value, Wv = decltype(w)::value, KPv = decltype(kp)::value;
        if (global_pivots)
          return launch_checked(&search_beam_kernel<T, MWv, Wv, KPv, true>, [&] {
            hipLaunchKernelGGL((search_beam_kernel<T, MWv, Wv, KPv, true>), dim3(blocks), dim3(waves * kWave),
                               smem, stream, ix, pq, q, nq, entries, topk, L, bw, nns, dists, found, n_exp,
                               n_adc, queue, qs_all);
          });
        return launch_checked(&search_beam_kernel<T, MWv, Wv, KPv, false>, [&] {
          hipLaunchKernelGGL((search_beam_kernel<T, MWv, Wv, KPv, false>), dim3(blocks), dim3(waves * kWave),
                             smem, stream, ix, pq, q, nq, entries, topk, L, bw, nns, dists, found, n_exp,
                             n_adc, queue, qs_all);
        });
      });
    });
  };
  const bool small = ix.dim <= 128;
  if (dtype == 0)
    return small ? go(uint8_t{}, std::integral_constant<int, 4>{})
                 : go(uint8_t{}, std::integral_constant<int, kMaxDimRegs>{});
  return small ? go(float{}, std::integral_constant<int, 4>{})
               : go(float{}, std::integral_constant<int, kMaxDimRegs>{});
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
    return launch_round_t<uint8_t>(ix, pq, q, nq, luts, topk, L, lists, s, nns, dists, active,
                                   slots, stream);
  return launch_round_t<float>(ix, pq, q, nq, luts, topk, L, lists, s, nns, dists, active, slots,
                               stream);
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

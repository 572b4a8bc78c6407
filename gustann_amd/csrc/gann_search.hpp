// The fused and step-wise beam-search kernels of the in-memory search
// (src/impl/pure_mem.cuh:243-432, src/impl/hyd_search_v2.cuh:8-472) and their
// launchers, as templates over the coordinate type.  Each of
// gann_search_{cb,beam}_{u8,f32}.hip and gann_search_lut.hip instantiates
// one family for one type, so the many shape specialisations compile in
// parallel.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <type_traits>

#include "gann_device.hpp"
#include "gann_kernels.hpp"
#include "gann_list.hpp"

namespace gann {

template <int V>
using ic = std::integral_constant<int, V>;

// Node u's record: page u / nodes_per_page, slot u % nodes_per_page (node ids
// are below 2^31; the page by the multiply of set_page_divisor).
__device__ __forceinline__ uint32_t page_of(const IndexDev& ix, uint32_t u) {
  return ix.npp_shift < 0 ? u : __umulhi(u, ix.npp_magic) >> ix.npp_shift;
}
__device__ __forceinline__ const uint8_t* record_of(const IndexDev& ix, int64_t u) {
  const uint32_t n = (uint32_t)u, page = page_of(ix, n);
  const uint32_t slot = n - page * (uint32_t)ix.nodes_per_page;
  return ix.pages + ((uint64_t)page << 12) + slot * (uint32_t)ix.node_len;
}

// Rerank coordinates per lane kept in registers by the kernels with one
// register layout for every dim (the LUT and step-wise forms, and the
// shared-codebook kernels' generic shape above dim 128): dims 0 .. 383.
constexpr int kMaxDimRegs = 12;

// One node record held in registers: its degree, this lane's neighbour ids
// (block b: neighbour 64b + lane, graph degree up to 64 kNB) and, in lanes
// 0..31, the coordinates l, l+32, ... that the exact rerank of lane l reads
// (square_sum_32's lane roles), for dims below 32 kPer; the coordinates of
// larger dims (kPer == kMaxDimRegs only) are read from the record when the
// rerank runs.  Loads are
// issued by load() and consumed one expansion later, so their latency
// overlaps the list update.
template <typename T, int kPer, int kNB>
struct RecRegs {
  int deg_raw;
  uint32_t v[kNB];
  T x[kPer];
  const T* xs;  // the record's coordinates
  __device__ __forceinline__ void load(const IndexDev& ix, int64_t u) { load_at(ix, record_of(ix, u)); }
  __device__ __forceinline__ void load_at(const IndexDev& ix, const uint8_t* rec) {
    const int lane = lane_id();
    deg_raw = *reinterpret_cast<const int32_t*>(rec + ix.data_len);
    const uint32_t* edge = reinterpret_cast<const uint32_t*>(rec + ix.data_len + 4);
#pragma unroll
    for (int b = 0; b < kNB; ++b) v[b] = lane + kWave * b < ix.R ? edge[lane + kWave * b] : 0u;
    xs = reinterpret_cast<const T*>(rec);
    const int l = lane & 31;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = l + 32 * k;
      x[k] = i < ix.dim ? xs[i] : T(0);
    }
  }
  // load() with every lane loading, at clamped addresses: a fixed number of
  // loads whatever the lane mask, so a later wait can count the loads issued
  // after them exactly.  Neighbours past R and coordinates past dim hold
  // copies of the last ones; every use is under lane < deg <= R or i < dim.
  __device__ __forceinline__ void load_fixed(const IndexDev& ix, int64_t u) {
    const uint8_t* rec = record_of(ix, u);
    const int lane = lane_id();
    deg_raw = *reinterpret_cast<const int32_t*>(rec + ix.data_len);
    const uint32_t* edge = reinterpret_cast<const uint32_t*>(rec + ix.data_len + 4);
#pragma unroll
    for (int b = 0; b < kNB; ++b) v[b] = edge[min(lane + kWave * b, ix.R - 1)];
    xs = reinterpret_cast<const T*>(rec);
    const int l = lane & 31;
#pragma unroll
    for (int k = 0; k < kPer; ++k) x[k] = xs[min(l + 32 * k, ix.dim - 1)];
  }
  // square_sum_32 (src/impl/util.cuh:26-46): lane l's partial over dims l,
  // l+32, ... in ascending order (registers first, then the record for dims
  // from 32 kPer, with the query restored from q and the centroid as
  // restored_query_regs does), then the 16/8/4/2/1 tree read at lane 0.
  // qv[k] holds the restored query at dim l + 32k.
  __device__ __forceinline__ float l2(const float (&qv)[kPer], int dim, const float* q,
                                      const float* centroid) const {
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
    if constexpr (kPer >= kMaxDimRegs) {
      // only the 12-slot layout serves dims past its registers; the others
      // are instantiated for dim <= 32 kPer
      for (int i = l + 32 * kPer; i < dim; i += 32) {
        const float t = q[i] - centroid[i];
        const float d = (t + centroid[i]) - to_f(xs[i]);
        acc = fma_f(d, d, acc);
      }
    }
    return square_sum_tree(acc);
  }
};

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

// LDS carve-up of the per-query-LUT kernel (bytes): LUT | qr | list A (L) |
// list scratch | top-k dists | top-k ids.
struct SearchSmem {
  static __host__ __device__ size_t bytes(int M, int dim, int L, int k) {
    return (size_t)M * kPivots * 4 + (size_t)((dim + 1) & ~1) * 4 + (size_t)list_capacity(L) * 8 +
           (size_t)list_scratch_words(L) * 4 + (size_t)k * 8;
  }
};

inline int mw_of(int M) {
  if (M % 16 != 0) return 0;
  const int mw = M / 16;
  return (mw >= 1 && mw <= 4) ? mw : 0;
}
inline int w_of(int chunk_w) { return (chunk_w == 2 || chunk_w == 4) ? chunk_w : 0; }

// Calls f(ic<MW>) for the runtime code-row shape (MW > 0: M == 16 MW and
// the rows are read as MW 16-byte words; 0: byte reads for any M).
template <class F>
hipError_t with_mw(int M, F&& f) {
  switch (mw_of(M)) {
    case 1: return f(ic<1>{});
    case 2: return f(ic<2>{});
    case 3: return f(ic<3>{});
    case 4: return f(ic<4>{});
    default: return f(ic<0>{});
  }
}
// Calls f(ic<W>) for the runtime chunk width (2 or 4 unrolled, 0: any).
template <class F>
hipError_t with_w(int chunk_w, F&& f) {
  switch (w_of(chunk_w)) {
    case 2: return f(ic<2>{});
    case 4: return f(ic<4>{});
    default: return f(ic<0>{});
  }
}
// Calls f(ic<NB>) for the graph degree: one 64-neighbour block up to R = 64,
// two up to 128.
template <class F>
hipError_t with_nb(int R, F&& f) {
  if (R <= kWave) return f(ic<1>{});
  return f(ic<2>{});
}

// ------------------------------------------------------------------ per-query LUT

template <typename T, int MW, int W, int NB>
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
  uint32_t* BM = reinterpret_cast<uint32_t*>(A + list_capacity(L));
  float* td = reinterpret_cast<float*>(BM + list_scratch_words(L));
  int32_t* ti = reinterpret_cast<int32_t*>(td + topk);

  int32_t u = __builtin_amdgcn_readfirstlane(entries[qi]);
  if (u >= ix.num_pts) u = -1;  // caller-given entries outside the index: empty result
  RecRegs<T, kMaxDimRegs, NB> cur;
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
    uint64_t key[NB];
    CodeRow<MW> row[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
      if (lane + kWave * b < deg) row[b].load(pq.codes + (int64_t)cur.v[b] * M, M);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      key[b] = ~(uint64_t)0;  // padding sorts last
      if (lane + kWave * b < deg)
        key[b] = make_key(row[b].adc(lut, pq.codes + (int64_t)cur.v[b] * M, M), cur.v[b]);
    }
    // exact rerank of u (independent of the list update; :420-423)
    const float du = cur.l2(qv, dim, qq, pq.centroid);
    const ListPlan P = list_plan_nb<NB>(A, BM, L, key, deg, sz, fu);
    const int32_t next =
        __builtin_amdgcn_readfirstlane(P.cand >= 0 ? (int32_t)entry_id(P.sel) : -1);
    RecRegs<T, kMaxDimRegs, NB> nxt;
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

// ------------------------------------------------------------------ shared codebook

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
  static __host__ __device__ size_t wave_bytes(int L, int k) {
    size_t b = (size_t)list_capacity(L) * 8 + (size_t)list_scratch_words(L) * 4 + (k > kWave ? (size_t)k * 8 : 0);
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
// cap a kernel at 128 VGPRs), so only the kernels with at most 4 rerank
// slots per lane (dim <= 128) do.
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

// The wide lookup in two steps: issue() requests the pivot rows of all 16 MW
// chunks of a code row (`piv` in HBM, `rowb` bytes per row), sum() adds the
// chunk distances in order 0 .. M-1 (the LUT's arithmetic, src/impl/pq.cuh:
// 35-43, and the ADC's order, src/impl/pure_mem.cuh:306-308).  Loads the
// caller issues between the two do not delay the rows sum() waits for.
// kWL > 0: the first kWL chunks come from a partial table at LDS address 0
// (rows of kWL * W floats, no padding), the others from piv.
template <int MW, int W, int kWL = 0>
struct WidePivots {
  static_assert(MW > 0 && (W == 4 || W == 2), "16 MW chunks of 2 or 4 dims");
  typedef typename PivotVec<W>::type PV;
  static constexpr int kM = 16 * MW;
  PV p[kM];
  __device__ __forceinline__ void issue(const uint8_t* piv, uint32_t rowb, const CodeRow<MW>& row) {
#pragma unroll
    for (int k = 0; k < MW; ++k) {
      const uint32_t ws[4] = {row.w[k].x, row.w[k].y, row.w[k].z, row.w[k].w};
#pragma unroll
      for (int b = 0; b < 16; ++b) {
        const uint32_t c = (ws[b >> 2] >> (8 * (b & 3))) & 0xffu;
        const int j = 16 * k + b;
        if (j < kWL)  // compile-time
          p[j] = lds_at<PV>(cb_row(c, kWL * W * 4) + j * W * 4);
        else
          p[j] = *reinterpret_cast<const PV*>(piv + cb_row(c, rowb) + j * W * 4);
      }
    }
  }
  __device__ __forceinline__ float sum(const float* qs) const {
    float dist = 0.0f;
#pragma unroll
    for (int g = 0; g < kM / 8; ++g) {
      uint64_t qa = (uint64_t)(qs + 8 * g * W);
      asm volatile("" : "+s"(qa));
      const __attribute__((address_space(4))) float* qg = (const __attribute__((address_space(4))) float*)qa;
      float qv[8 * W];
#pragma unroll
      for (int i = 0; i < 8 * W; ++i) qv[i] = qg[i];
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        float pv[W];
#pragma unroll
        for (int i = 0; i < W; ++i) pv[i] = p[8 * g + b][i];
        dist = dist + cb_chunk<W>(qv + b * W, pv);
      }
    }
    return dist;
  }
};

// kWide (pivot table read through the caches, none of it in LDS): the
// pivot rows of all 16 MW chunks are requested before the first is used, so
// a lookup waits for one cache round trip instead of one per 8 chunks; the
// 64 MW W-float rows need the register budget of 8-wave workgroups.
template <int W, int MW, int kSplitG = 0, bool kPivLds = false, bool kSplitLds = false, bool kWide = false>
__device__ __forceinline__ float cb_adc(const uint8_t* piv, const float* qs, uint32_t rowb,
                                        const PQDev& pq, const CodeRow<MW>& row,
                                        const uint8_t* crow, const uint8_t* pivl = nullptr) {
  float dist = 0.0f;
  if constexpr (kWide) {
    static_assert(kSplitG == 0 && !kPivLds, "wide form: whole table in HBM");
    WidePivots<MW, W> wp;
    wp.issue(piv, rowb, row);
    dist = wp.sum(qs);
  } else if constexpr (MW > 0 && (W == 4 || W == 2)) {
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

constexpr int kGpWide = kCbGpWide;

// Largest workgroup of the shared-codebook kernels: 16 waves, or 8 when a
// lane keeps more than 8 rerank coordinates or all pivot rows of a lookup
// (kGpWide) in flight (the 128-VGPR cap of 16-wave workgroups would spill
// them).
__host__ __device__ constexpr int cb_block_threads(int KP, int kSplitG = 0) {
  return (KP > 8 || cb_is_wide(kSplitG)) ? 512 : 1024;
}

// kGP: the pivot table is read from pq.piv_cb (HBM, through the caches)
// instead of a copy in LDS, which then holds only the per-wave lists: the
// form for large L, where lists beside a 128 KB table leave few waves.
// kSplitG > 0 (with kGP): that many groups of 8 chunks also in LDS;
// kSplitG == kGpWide - G (with kGP): the wide lookup of cb_adc in 8-wave
// workgroups, the first G chunks (one neighbour block only) from a partial
// table in LDS.  KP: rerank coordinates per lane held in registers; NB:
// neighbour blocks.
template <typename T, int MW, int W, bool kGP, int kSplitG, int KP, int NB>
__global__ __launch_bounds__(cb_block_threads(KP, kSplitG)) void search_cb_kernel(
    IndexDev ix, PQDev pq, const float* __restrict__ q, int nq, const int32_t* __restrict__ entries,
    int topk, int L, int32_t* __restrict__ nns, float* __restrict__ dists,
    int32_t* __restrict__ found_cnt, int32_t* __restrict__ n_exp, int32_t* __restrict__ n_adc,
    int32_t* __restrict__ queue, const int32_t* __restrict__ order, const float* __restrict__ qs_all) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  const int dim = ix.dim, M = pq.M, R = ix.R;
  const uint32_t rowb = cb_stride(4 * dim);
  const uint8_t* piv;
  size_t lists_at = 0;
  constexpr int kWL = cb_wide_lds(kSplitG);
  static_assert(kWL == 0 || NB == 1, "the wide form's LDS chunks serve one neighbour block");
  if constexpr (kGP) {
    piv = (const uint8_t*)((const __attribute__((address_space(1))) uint8_t*)pq.piv_cb);
    if constexpr (kWL > 0) {
      // the first kWL chunks (dims 0 .. kWL W - 1) at LDS address 0
      constexpr int per_row = kWL * W;
      for (int idx = threadIdx.x; idx < kPivots * per_row; idx += blockDim.x) {
        const int c = idx / per_row, i = idx - c * per_row;
        *reinterpret_cast<float*>(smem_raw + 4 * idx) = pq.pivots[c * dim + i];
      }
      __syncthreads();
      lists_at = cb_wide_lds_bytes(kWL, W);
    }
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
  uint8_t* wbase = smem_raw + lists_at + (size_t)wave * CbSmem::wave_bytes(L, topk);
  uint64_t* A = reinterpret_cast<uint64_t*>(wbase);
  uint32_t* BM = reinterpret_cast<uint32_t*>(A + list_capacity(L));
  float* td = reinterpret_cast<float*>(BM + list_scratch_words(L));
  int32_t* ti = reinterpret_cast<int32_t*>(td + topk);
  const int64_t cap = ix.num_pts + 2;

  for (;;) {
    int qi = 0;
    if (lane == 0) qi = atomicAdd(queue, 1);
    qi = __builtin_amdgcn_readfirstlane(__shfl(qi, 0, kWave));
    if (qi >= nq) break;
    if (order) qi = __builtin_amdgcn_readfirstlane(order[qi]);  // queue position -> query
    int32_t u = __builtin_amdgcn_readfirstlane(entries[qi]);
    if (u >= ix.num_pts) u = -1;  // caller-given entries outside the index: empty result
    RecRegs<T, KP, NB> cur;
    if (u >= 0) cur.load(ix, u);
    const float* qq = q + (int64_t)qi * dim;
    const float* qs = qs_all + (int64_t)qi * dim;  // q - mu, uniform reads
    float qv[KP];
    restored_query_regs(qq, pq.centroid, dim, qv);
    int sz = 0, fu = 0;
    TopK top(td, ti, topk);
    int32_t exps = 0, adcs = 0;
    // kSpec (the wide form, one neighbour block): the node after next is
    // guessed as the first unvisited entry once the list is updated (right
    // unless next's expansion inserts before it), and its record is
    // requested right after the next expansion's pivot reads, its code rows
    // right after that expansion's ADC.  A right guess finds record and rows
    // in flight or in registers; a wrong one loads them as the plain loop
    // does.  Only where data is fetched changes: every value used is the
    // one the plain loop loads.  The guess loads come after the loads the
    // expansion waits for, so they never hold those up.
    constexpr bool kSpec = cb_is_wide(kSplitG) && NB == 1;
    struct NoPivots {};
    std::conditional_t<kSpec, WidePivots<(kSpec ? MW : 1), (kSpec ? W : 4), kWL>, NoPivots> wp;  // cur's pivot rows
    bool piv_ok = false;    // wp already requested for cur (uniform)
    RecRegs<T, KP, NB> gs;  // the guessed next node's record
    CodeRow<MW> grows;      // and its code rows
    int32_t g_id = -1;      // the guess (-1: none)
    while (u >= 0 && exps < cap) {
      ++exps;
      const int deg = __builtin_amdgcn_readfirstlane(min(max(cur.deg_raw, 0), R));
      adcs += deg;
      uint64_t key[NB];
      if constexpr (kSpec) {
        if (!piv_ok) {
          CodeRow<MW> rows;  // cur's code rows (lanes past deg: all codes 0)
          if (lane < deg)
            rows.load(pq.codes + (int64_t)cur.v[0] * M, M);
          else
            rows.zero();
          wp.issue(piv, rowb, rows);
        }
        // the fences keep this order: pivot reads, guess record, the sum
        // (waiting for the pivot reads only), then the first use of the
        // guess record
        asm volatile("" ::: "memory");
        gs.load_fixed(ix, g_id >= 0 ? g_id : 0);
        float d = wp.sum(qs);
        asm volatile("" : "+v"(d));
        asm volatile("" : "+v"(gs.deg_raw));
        key[0] = lane < deg ? make_key(d, cur.v[0]) : ~(uint64_t)0;
        const int gdeg = __builtin_amdgcn_readfirstlane(min(max(gs.deg_raw, 0), R));
        if (lane < gdeg)
          grows.load(pq.codes + (int64_t)gs.v[0] * M, M);
        else
          grows.zero();
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if constexpr (kSpec) break;
        key[b] = ~(uint64_t)0;  // padding sorts last
        if (lane + kWave * b < deg) {
          CodeRow<MW> row;
          const uint8_t* crow = pq.codes + (int64_t)cur.v[b] * M;
          row.load(crow, M);
          key[b] = make_key(cb_adc<W, MW, (kSplitG > 0 ? kSplitG : 0), !kGP, (KP <= 4), cb_is_wide(kSplitG)>(
                                piv, qs, rowb, pq, row, crow, smem_raw),
                            cur.v[b]);
        }
      }
      const float du = cur.l2(qv, dim, qq, pq.centroid);
      const ListPlan P = list_plan_nb<NB>(A, BM, L, key, deg, sz, fu);
      const int32_t next =
          __builtin_amdgcn_readfirstlane(P.cand >= 0 ? (int32_t)entry_id(P.sel) : -1);
      RecRegs<T, KP, NB> nxt;
      piv_ok = false;
      // the guess's code rows (requested an expansion step ago) are waited
      // for on every path, before the branch: with a load still pending on
      // one path, the list update below would wait for it, and in issue
      // order that wait also covers the pivot reads issued early on the
      // other path
      if constexpr (kSpec) __builtin_amdgcn_s_waitcnt(kVmcntZero);
      if (kSpec && next >= 0 && next == g_id) {
        nxt = gs;
        if constexpr (kSpec) {
          // next's code rows are here: its pivot reads go out now and
          // arrive during the list update
          wp.issue(piv, rowb, grows);
          piv_ok = true;
          asm volatile("" ::: "memory");
        }
      } else if (!kSpec && next >= 0) {
        nxt.load(ix, next);
      }
      fu = list_apply(A, BM, P);
      // kSpec without early pivot reads (a wrong guess): next's record is
      // requested after the list update, so that the update has no pending
      // load on either path
      if constexpr (kSpec)
        if (next >= 0 && !piv_ok) nxt.load(ix, next);
      sz = P.nsz;
      top.push(du, u);
      if constexpr (kSpec)
        g_id = next >= 0 && fu < sz ? __builtin_amdgcn_readfirstlane((int32_t)entry_id(A[fu])) : -1;
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

// ------------------------------------------------------------------ beam width > 1

// Beam search with beam width bw (2..kMaxBeam), a mode the reference does not
// have (it expands one node per iteration; this mode is reported beside it
// with its own recall).  Each round takes the first bw unvisited list entries
// at once, marks them visited and loads their records together, then expands
// them in list order: every expansion merges its neighbours into the list
// with the same rank / sort / gather update as search_cb_kernel and pushes
// the node's exact distance into the top-k.  The code rows of the next node
// of the round are fetched while the current one is merged.  The search ends
// when no unvisited entry is left.  LDS layout and query queue as in
// search_cb_kernel; KP rerank coordinates per lane, NB neighbour blocks.
constexpr int kMaxBeam = 4;

template <typename T, int MW, int W, int KP, bool kGP, int NB>
__global__ __launch_bounds__(cb_block_threads(KP)) void search_beam_kernel(
    IndexDev ix, PQDev pq, const float* __restrict__ q, int nq, const int32_t* __restrict__ entries,
    int topk, int L, int bw, int32_t* __restrict__ nns, float* __restrict__ dists,
    int32_t* __restrict__ found_cnt, int32_t* __restrict__ n_exp, int32_t* __restrict__ n_adc,
    int32_t* __restrict__ queue, const int32_t* __restrict__ order, const float* __restrict__ qs_all) {
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
  uint8_t* wbase = smem_raw + lists_at + (size_t)wave * CbSmem::wave_bytes(L, topk);
  uint64_t* A = reinterpret_cast<uint64_t*>(wbase);
  uint32_t* BM = reinterpret_cast<uint32_t*>(A + list_capacity(L));
  float* td = reinterpret_cast<float*>(BM + list_scratch_words(L));
  int32_t* ti = reinterpret_cast<int32_t*>(td + topk);
  const int64_t cap = ix.num_pts + 2;

  for (;;) {
    int qi = 0;
    if (lane == 0) qi = atomicAdd(queue, 1);
    qi = __builtin_amdgcn_readfirstlane(__shfl(qi, 0, kWave));
    if (qi >= nq) break;
    if (order) qi = __builtin_amdgcn_readfirstlane(order[qi]);  // queue position -> query
    const float* qq = q + (int64_t)qi * dim;
    const float* qs = qs_all + (int64_t)qi * dim;
    float qv[KP];
    restored_query_regs(qq, pq.centroid, dim, qv);
    int sz = 0, fu = 0;
    TopK top(td, ti, topk);
    int32_t exps = 0, adcs = 0;
    int32_t sel[kMaxBeam];
#pragma unroll
    for (int b = 0; b < kMaxBeam; ++b) sel[b] = -1;
    sel[0] = __builtin_amdgcn_readfirstlane(entries[qi]);
    int nsel = sel[0] >= 0 && sel[0] < ix.num_pts ? 1 : 0;
    while (nsel > 0) {
      RecRegs<T, KP, NB> rec[kMaxBeam];
#pragma unroll
      for (int b = 0; b < kMaxBeam; ++b)
        if (b < nsel) rec[b].load(ix, sel[b]);
      CodeRow<MW> rows[2][NB];
      {
        const int d0 = __builtin_amdgcn_readfirstlane(min(max(rec[0].deg_raw, 0), R));
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          if (lane + kWave * nb < d0) rows[0][nb].load(pq.codes + (int64_t)rec[0].v[nb] * M, M);
      }
#pragma unroll
      for (int b = 0; b < kMaxBeam; ++b) {
        if (b < nsel && exps < cap) {
          ++exps;
          const int deg = __builtin_amdgcn_readfirstlane(min(max(rec[b].deg_raw, 0), R));
          adcs += deg;
          if (b + 1 < kMaxBeam && b + 1 < nsel) {
            const int dn = __builtin_amdgcn_readfirstlane(min(max(rec[b + 1].deg_raw, 0), R));
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
              if (lane + kWave * nb < dn)
                rows[(b + 1) & 1][nb].load(pq.codes + (int64_t)rec[b + 1].v[nb] * M, M);
          }
          uint64_t key[NB];
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            key[nb] = ~(uint64_t)0;
            if (lane + kWave * nb < deg) {
              const uint8_t* crow = pq.codes + (int64_t)rec[b].v[nb] * M;
              key[nb] = make_key(cb_adc<W, MW, 0, !kGP>(piv, qs, rowb, pq, rows[b & 1][nb], crow),
                                 rec[b].v[nb]);
            }
          }
          const float du = rec[b].l2(qv, dim, qq, pq.centroid);
          const ListPlan P = list_plan_nb<NB>(A, BM, L, key, deg, sz, fu);
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

// One expansion per active query: the work of merge_data_kernel followed by
// unify_kernel (src/impl/hyd_search_v2.cuh:8-351, 353-472) in one launch;
// the candidate list and the top-k travel through HBM between rounds.
template <typename T, int MW, int NB>
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
  uint32_t* BM = reinterpret_cast<uint32_t*>(A + list_capacity(L));
  float* td = reinterpret_cast<float*>(BM + list_scratch_words(L));
  int32_t* ti = reinterpret_cast<int32_t*>(td + topk);
  const float* lut = luts + (int64_t)qi * M * kPivots;
  uint64_t* glist = lists + (int64_t)qi * L;

  const int32_t u = __builtin_amdgcn_readfirstlane(s.u);
  RecRegs<T, kMaxDimRegs, NB> cur;
  // the record comes from the index pages, or from this query's 4096-byte
  // slot that the host filled with u's page (src/hyd_task_runner.cu:216-240)
  if (slots)
    cur.load_at(ix, slots + (int64_t)qi * kStepSlotBytes +
                        ((uint32_t)u - page_of(ix, (uint32_t)u) * (uint32_t)ix.nodes_per_page) * (uint32_t)ix.node_len);
  else
    cur.load(ix, u);
  const float* qq = q + (int64_t)qi * dim;
  float qv[kMaxDimRegs];
  restored_query_regs(qq, pq.centroid, dim, qv);
  for (int i = lane; i < s.sz; i += kWave) A[i] = glist[i];
  for (int j = lane; j < s.found; j += kWave) {
    td[j] = dists[(int64_t)qi * topk + j];
    ti[j] = nns[(int64_t)qi * topk + j];
  }
  __syncthreads();

  const int deg = __builtin_amdgcn_readfirstlane(min(max(cur.deg_raw, 0), R));
  uint64_t key[NB];
  CodeRow<MW> row[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
    if (lane + kWave * b < deg) row[b].load(pq.codes + (int64_t)cur.v[b] * M, M);
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    key[b] = ~(uint64_t)0;
    if (lane + kWave * b < deg)
      key[b] = make_key(row[b].adc(lut, pq.codes + (int64_t)cur.v[b] * M, M), cur.v[b]);
  }
  const float du = cur.l2(qv, dim, qq, pq.centroid);
  int sz = s.sz, fu = s.fu;
  const ListPlan P = list_plan_nb<NB>(A, BM, L, key, deg, sz, fu);
  const int32_t next = P.cand >= 0 ? (int32_t)entry_id(P.sel) : -1;
  fu = list_apply(A, BM, P);
  sz = P.nsz;
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

// ------------------------------------------------------------------ launchers

// Calls f(ic<MW>, ic<W>, ic<KP>) for the shared-codebook kernels: the
// specialised shapes (M = 16 MW bytes of code read as MW 16-byte words,
// uniform chunks of W = 2 or 4 dims, so dim = 16 MW W and KP = dim / 32
// rerank coordinates per lane), or the generic one (byte reads of the codes,
// chunk bounds from chunk_off; 4 coordinates per lane in registers up to dim
// 128, else 12 and the rest read from the record).
template <class F>
hipError_t with_cb_shape(int M, int chunk_w, int dim, F&& f) {
  const int mw = mw_of(M), w = w_of(chunk_w);
  if (mw > 0 && w > 0) {
    switch (mw * 8 + w) {
      case 1 * 8 + 2: return f(ic<1>{}, ic<2>{}, ic<1>{});  // dim 32
      case 1 * 8 + 4: return f(ic<1>{}, ic<4>{}, ic<2>{});  // dim 64
      case 2 * 8 + 2: return f(ic<2>{}, ic<2>{}, ic<2>{});  // dim 64
      case 2 * 8 + 4: return f(ic<2>{}, ic<4>{}, ic<4>{});  // dim 128
      case 3 * 8 + 2: return f(ic<3>{}, ic<2>{}, ic<3>{});  // dim 96
      case 3 * 8 + 4: return f(ic<3>{}, ic<4>{}, ic<6>{});  // dim 192
      case 4 * 8 + 2: return f(ic<4>{}, ic<2>{}, ic<4>{});  // dim 128
      case 4 * 8 + 4: return f(ic<4>{}, ic<4>{}, ic<8>{});  // dim 256
      default: break;
    }
  }
  if (dim <= 128) return f(ic<0>{}, ic<0>{}, ic<4>{});
  return f(ic<0>{}, ic<0>{}, ic<kMaxDimRegs>{});
}

// Rerank coordinates per lane that the shared-codebook kernels keep in
// registers for this shape (as with_cb_shape chooses).
inline int cb_rerank_regs(int M, int chunk_w, int dim) {
  int kp = 0;
  (void)with_cb_shape(M, chunk_w, dim, [&](auto, auto, auto k) {
    kp = decltype(k)::value;
    return hipSuccess;
  });
  return kp;
}

// The shared-codebook kernels address their LDS pivot tables (the whole
// table, or the partial table of a split form with 4 rerank slots per lane)
// from LDS address 0 (lds_at), which is where the dynamic LDS starts only
// when the kernel has no static LDS: refuse the launch otherwise (checked for
// every form, so that none gains static LDS unnoticed).
inline hipError_t check_dynamic_lds_at_zero(const void* fn) {
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

// The fused shared-codebook search kernel for coordinate type T (queue and
// q - mu already prepared by launch_search_cb).
template <typename T>
hipError_t launch_search_cb_t(const IndexDev& ix, const PQDev& pq, const float* q, int nq,
                              const int32_t* entries, int topk, int L, int32_t* nns, float* dists,
                              int32_t* found, int32_t* n_exp, int32_t* n_adc, int32_t* queue,
                              const int32_t* order, const float* qs_all, int waves, int blocks, bool global_pivots,
                              int lds_groups, size_t smem, hipStream_t stream) {
  return with_nb(ix.R, [&](auto nb) {
    constexpr int NBv = decltype(nb)::value;
    return with_cb_shape(pq.M, pq.chunk_w, ix.dim, [&](auto mw, auto w, auto kp) {
      constexpr int MWv = decltype(mw)::value, Wv = decltype(w)::value, KPv = decltype(kp)::value;
      if (waves * kWave > cb_block_threads(KPv, cb_is_wide(lds_groups) ? kGpWide : 0))
        return hipErrorInvalidConfiguration;
      // the split forms keep part of the table in LDS for one neighbour
      // block; with two the extra live registers would spill
      constexpr bool kCanSplit = MWv > 0 && NBv == 1;
      constexpr int kSplit = kCanSplit ? 2 * MWv - 1 : 0, kHalf = kCanSplit ? MWv : 0;
      const dim3 grid(blocks), block(waves * kWave);
      // the wide form: all 16 MW pivot rows of a lookup in at most 128 registers
      constexpr bool kCanWide = MWv > 0 && 16 * MWv * Wv <= 128;
      if constexpr (kCanWide) {
        if (global_pivots && cb_is_wide(lds_groups)) {
          auto wide = [&](auto g) {
            constexpr int kG = decltype(g)::value;
            return launch_checked(&search_cb_kernel<T, MWv, Wv, true, kG, KPv, NBv>, [&] {
              hipLaunchKernelGGL((search_cb_kernel<T, MWv, Wv, true, kG, KPv, NBv>), grid, block, smem, stream,
                                 ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, queue, order, qs_all);
            });
          };
          if (lds_groups == kGpWide) return wide(ic<kGpWide>{});
          if constexpr (NBv == 1) {
            static_assert(kCbMaxWideLds == 3, "one instantiation per partial-table size");
            if (lds_groups == kGpWide - 1) return wide(ic<kGpWide - 1>{});
            if (lds_groups == kGpWide - 2) return wide(ic<kGpWide - 2>{});
            if (lds_groups == kGpWide - 3) return wide(ic<kGpWide - 3>{});
          }
          return hipErrorInvalidValue;
        }
      }
      if constexpr (kCanSplit) {
        if (global_pivots && lds_groups > 0 && lds_groups == kSplit)
          return launch_checked(&search_cb_kernel<T, MWv, Wv, true, kSplit, KPv, NBv>, [&] {
            hipLaunchKernelGGL((search_cb_kernel<T, MWv, Wv, true, kSplit, KPv, NBv>), grid, block, smem, stream,
                               ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, queue, order, qs_all);
          });
        if (global_pivots && lds_groups > 0 && lds_groups == kHalf)
          return launch_checked(&search_cb_kernel<T, MWv, Wv, true, kHalf, KPv, NBv>, [&] {
            hipLaunchKernelGGL((search_cb_kernel<T, MWv, Wv, true, kHalf, KPv, NBv>), grid, block, smem, stream,
                               ix, pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, queue, order, qs_all);
          });
      }
      if (lds_groups != 0) return hipErrorInvalidValue;
      if (global_pivots)
        return launch_checked(&search_cb_kernel<T, MWv, Wv, true, 0, KPv, NBv>, [&] {
          hipLaunchKernelGGL((search_cb_kernel<T, MWv, Wv, true, 0, KPv, NBv>), grid, block, smem, stream, ix,
                             pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, queue, order, qs_all);
        });
      return launch_checked(&search_cb_kernel<T, MWv, Wv, false, 0, KPv, NBv>, [&] {
        hipLaunchKernelGGL((search_cb_kernel<T, MWv, Wv, false, 0, KPv, NBv>), grid, block, smem, stream, ix,
                           pq, q, nq, entries, topk, L, nns, dists, found, n_exp, n_adc, queue, order, qs_all);
      });
    });
  });
}

template <typename T>
hipError_t launch_search_beam_t(const IndexDev& ix, const PQDev& pq, const float* q, int nq,
                                const int32_t* entries, int topk, int L, int bw, int32_t* nns,
                                float* dists, int32_t* found, int32_t* n_exp, int32_t* n_adc,
                                int32_t* queue, const int32_t* order, const float* qs_all, int waves, int blocks,
                                bool global_pivots, size_t smem, hipStream_t stream) {
  return with_nb(ix.R, [&](auto nb) {
    constexpr int NBv = decltype(nb)::value;
    return with_cb_shape(pq.M, pq.chunk_w, ix.dim, [&](auto mw, auto w, auto kp) {
      constexpr int MWv = decltype(mw)::value, Wv = decltype(w)::value, KPv = decltype(kp)::value;
      if (waves * kWave > cb_block_threads(KPv)) return hipErrorInvalidConfiguration;
      const dim3 grid(blocks), block(waves * kWave);
      if (global_pivots)
        return launch_checked(&search_beam_kernel<T, MWv, Wv, KPv, true, NBv>, [&] {
          hipLaunchKernelGGL((search_beam_kernel<T, MWv, Wv, KPv, true, NBv>), grid, block, smem, stream, ix, pq,
                             q, nq, entries, topk, L, bw, nns, dists, found, n_exp, n_adc, queue, order, qs_all);
        });
      return launch_checked(&search_beam_kernel<T, MWv, Wv, KPv, false, NBv>, [&] {
        hipLaunchKernelGGL((search_beam_kernel<T, MWv, Wv, KPv, false, NBv>), grid, block, smem, stream, ix, pq,
                           q, nq, entries, topk, L, bw, nns, dists, found, n_exp, n_adc, queue, order, qs_all);
      });
    });
  });
}

template <typename T>
hipError_t launch_search_lut_t(const IndexDev& ix, const PQDev& pq, const float* q, int nq,
                               const int32_t* entries, int topk, int L, int32_t* nns, float* dists,
                               int32_t* found, int32_t* n_exp, int32_t* n_adc, hipStream_t stream) {
  const size_t smem = SearchSmem::bytes(pq.M, ix.dim, L, topk);
  return with_nb(ix.R, [&](auto nb) {
    return with_mw(pq.M, [&](auto mw) {
      return with_w(pq.chunk_w, [&](auto w) {
        hipLaunchKernelGGL((search_kernel<T, decltype(mw)::value, decltype(w)::value, decltype(nb)::value>),
                           dim3(nq), dim3(64), smem, stream, ix, pq, q, nq, entries, topk, L, nns, dists, found,
                           n_exp, n_adc);
        return hipGetLastError();
      });
    });
  });
}

template <typename T>
hipError_t launch_round_t(const IndexDev& ix, const PQDev& pq, const float* q, int nq, const float* luts,
                          int topk, int L, uint64_t* lists, StepState* st, int32_t* nns, float* dists,
                          int32_t* active, const uint8_t* slots, hipStream_t stream) {
  const size_t smem = (size_t)((ix.dim + 1) & ~1) * 4 + (size_t)list_capacity(L) * 8 +
                      (size_t)list_scratch_words(L) * 4 + (size_t)topk * 8;
  return with_nb(ix.R, [&](auto nb) {
    return with_mw(pq.M, [&](auto mw) {
      hipLaunchKernelGGL((step_round_kernel<T, decltype(mw)::value, decltype(nb)::value>), dim3(nq), dim3(64),
                         smem, stream, ix, pq, q, nq, luts, topk, L, lists, st, nns, dists, active, slots);
      return hipGetLastError();
    });
  });
}

}  // namespace gann

namespace gann {

// One instantiation of each launcher per coordinate type, each in its own
// translation unit (gann_search_{cb,beam}_{u8,f32}.hip, gann_search_lut.hip).
#define GANN_CB_ARGS                                                                                \
  const IndexDev &ix, const PQDev &pq, const float *q, int nq, const int32_t *entries, int topk,     \
      int L, int32_t *nns, float *dists, int32_t *found, int32_t *n_exp, int32_t *n_adc,             \
      int32_t *queue, const int32_t *order, const float *qs_all, int waves, int blocks, bool global_pivots, int lds_groups, \
      size_t smem, hipStream_t stream
#define GANN_BEAM_ARGS                                                                              \
  const IndexDev &ix, const PQDev &pq, const float *q, int nq, const int32_t *entries, int topk,     \
      int L, int bw, int32_t *nns, float *dists, int32_t *found, int32_t *n_exp, int32_t *n_adc,     \
      int32_t *queue, const int32_t *order, const float *qs_all, int waves, int blocks, bool global_pivots, size_t smem,   \
      hipStream_t stream
#define GANN_LUT_ARGS                                                                               \
  const IndexDev &ix, const PQDev &pq, const float *q, int nq, const int32_t *entries, int topk,     \
      int L, int32_t *nns, float *dists, int32_t *found, int32_t *n_exp, int32_t *n_adc,             \
      hipStream_t stream
#define GANN_ROUND_ARGS                                                                             \
  const IndexDev &ix, const PQDev &pq, const float *q, int nq, const float *luts, int topk, int L,   \
      uint64_t *lists, StepState *st, int32_t *nns, float *dists, int32_t *active,                   \
      const uint8_t *slots, hipStream_t stream

hipError_t launch_search_cb_u8(GANN_CB_ARGS);
hipError_t launch_search_cb_f32(GANN_CB_ARGS);
hipError_t launch_search_beam_u8(GANN_BEAM_ARGS);
hipError_t launch_search_beam_f32(GANN_BEAM_ARGS);
hipError_t launch_search_lut_u8(GANN_LUT_ARGS);
hipError_t launch_search_lut_f32(GANN_LUT_ARGS);
hipError_t launch_round_u8(GANN_ROUND_ARGS);
hipError_t launch_round_f32(GANN_ROUND_ARGS);

}  // namespace gann

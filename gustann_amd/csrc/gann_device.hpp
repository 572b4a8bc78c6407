// Device-side building blocks shared by the GustANN search kernels (gfx950,
// wave64).  Every routine reproduces the reference's arithmetic order exactly
// (floating-point contraction is disabled for the whole library and every
// fused multiply-add is written out), so results are bit-identical to the
// reference semantics on identical inputs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gann {

constexpr int kWave = 64;
constexpr int kPivots = 256;
constexpr uint32_t kMask31 = 0x7fffffffu;
constexpr uint32_t kVisited = 0x80000000u;

// Static PQ tables resident in HBM.
struct PQDev {
  int32_t dim;
  int32_t M;
  int32_t chunk_w;          // > 0: chunk m spans dims [m*chunk_w, (m+1)*chunk_w); 0: irregular
  int64_t num_pts;
  const float* pivots;      // [256][dim]  (row-major as stored in <pq>_pivots.bin)
  const float* pivots_t;    // [dim][256]  (transposed like src/pq_search.cu:88-93)
  const float* centroid;    // [dim]
  const int32_t* chunk_off; // [M + 1]
  const uint8_t* codes;     // [num_pts][M]
  const uint8_t* piv_cb;    // pivot rows in the shared-codebook layout (cb_row), for reads through the caches
};

// Disk-index pages resident in HBM (or pinned host memory).
struct IndexDev {
  const uint8_t* pages;  // sector 1.. of <prefix>_disk.index
  int64_t nodes_per_page;
  int64_t node_len;
  int64_t data_len;
  int64_t num_pts;
  int64_t medoid;
  int32_t R;
  int32_t dim;
  // node u's page is u / nodes_per_page = umulhi(u, npp_magic) >> npp_shift
  // for u < 2^31 (npp_shift < 0: one node per page); set by set_page_divisor
  uint32_t npp_magic;
  int32_t npp_shift;
};

// The page divisor of IndexDev: for 2 <= d = nodes_per_page <= 4096 and
// l = ceil(log2 d), m = floor(2^(31+l) / d) + 1 < 2^32 gives
// floor(u / d) = floor(u m / 2^(31+l)) for every u < 2^31 (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994,
// Theorem 4.2 with N = 31), so one 32x32 high multiply and a shift replace
// the 64-bit division.
inline void set_page_divisor(IndexDev& ix) {
  const uint32_t d = (uint32_t)ix.nodes_per_page;
  if (d <= 1) {
    ix.npp_magic = 0;
    ix.npp_shift = -1;
    return;
  }
  int l = 0;
  while ((1u << l) < d) ++l;
  ix.npp_magic = (uint32_t)((1ull << (31 + l)) / d + 1);
  ix.npp_shift = l - 1;
}

// Pivot graph resident in HBM.
struct NavDev {
  const uint8_t* data;  // [n][dim] of the coordinate type
  const int32_t* graph; // [n][max_m], -1 padded
  const int32_t* map;   // [n] base ids
  int64_t n;
  int32_t max_m;
  int32_t start;
};

__device__ __forceinline__ float fma_f(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

__device__ __forceinline__ float to_f(uint8_t v) { return (float)v; }
__device__ __forceinline__ float to_f(float v) { return v; }

// 64-bit ordering key of a candidate: the reference orders by (dist, id with
// bit 31 masked) (src/impl/util.cuh:166-178).  PQ and L2 distances are sums
// of squares, hence non-negative, and the IEEE bit pattern of a non-negative
// float is monotonic in its value, so bits(dist) << 32 | (id & 0x7fffffff) << 1
// compares exactly like the reference's two-level compare.  Bit 0 is free
// and carries the visited flag of a list entry: a flagged entry still sorts
// between its own key and the next key, so raw 64-bit compares of entries
// against fresh keys keep the order and put an entry with the same id at the
// fresh key's lower bound.
constexpr uint64_t kListVisited = 1;
__device__ __forceinline__ uint64_t make_key(float d, uint32_t id) {
  return ((uint64_t)__float_as_uint(d) << 32) | ((uint64_t)(id & kMask31) << 1);
}
__device__ __forceinline__ uint64_t entry_key(uint64_t e) { return e & ~kListVisited; }
__device__ __forceinline__ uint32_t entry_id(uint64_t e) { return (uint32_t)e >> 1; }
__device__ __forceinline__ bool entry_visited(uint64_t e) { return (e & kListVisited) != 0; }
__device__ __forceinline__ float entry_dist(uint64_t e) { return __uint_as_float((uint32_t)(e >> 32)); }

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

// Orders LDS accesses among the lanes of one wavefront (a workgroup barrier
// would also wait for the other waves of a multi-wave workgroup, which run
// unrelated queries).  DS instructions of one wave complete in issue order;
// the fence keeps the compiler from moving accesses across this point.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// s_waitcnt operand: vmcnt(0), expcnt and lgkmcnt not waited for (gfx9
// encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int kVmcntZero = 0x0F70;

__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }

// Inclusive prefix sum over the 64 lanes: DPP row_shr 1/2/4/8 inside each
// row of 16 lanes (out-of-row sources read 0), then the row totals added
// through readlane.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);  // row_shr:8
  const int t0 = __builtin_amdgcn_readlane(v, 15);
  const int t1 = __builtin_amdgcn_readlane(v, 31);
  const int t2 = __builtin_amdgcn_readlane(v, 47);
  const int row = lane_id() >> 4;
  return v + (row == 0 ? 0 : row == 1 ? t0 : row == 2 ? t0 + t1 : t0 + t1 + t2);
}

// Number of set bits of `mask` below this lane.
__device__ __forceinline__ int rank_below(uint64_t mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Per-lane select by a wave-uniform 64-bit lane mask: lane l gets b if bit l
// of m is set, else a (one v_cndmask with the mask in scalar registers).
__device__ __forceinline__ uint32_t lane_select(uint64_t m, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(m));
  return r;
}

// Lanes l with (l & bit) != 0.
__host__ __device__ constexpr uint64_t lanes_with_bit(int bit) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l)
    if (l & bit) m |= 1ull << l;
  return m;
}

// Value of v in lane (this lane ^ M) for a compile-time M, on VALU
// cross-lane paths only (no LDS round trip): DPP quad_perm for 1 and 2, DPP
// row_shl/row_shr:4 for 4, DPP row_ror:8 for 8 (a rotation by 8 within a
// 16-lane row is the xor), v_permlane16_swap for 16, v_permlane32_swap for
// 32.  A swap of v with itself returns {even rows of v duplicated, odd rows
// of v duplicated}, so the partner row is the other element of the pair.
template <int M>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "lane xor");
  const int x = (int)v;
  if constexpr (M == 1) {
    return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0xB1, 0xf, 0xf, true);  // quad_perm [1,0,3,2]
  } else if constexpr (M == 2) {
    return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x4E, 0xf, 0xf, true);  // quad_perm [2,3,0,1]
  } else if constexpr (M == 4) {
    const uint32_t up = (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x104, 0xf, 0xf, true);  // lane + 4
    const uint32_t dn = (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x114, 0xf, 0xf, true);  // lane - 4
    return lane_select(lanes_with_bit(4), up, dn);
  } else if constexpr (M == 8) {
    return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x128, 0xf, 0xf, true);  // row_ror:8
  } else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return lane_select(lanes_with_bit(16), r[1], r[0]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return lane_select(lanes_with_bit(32), r[1], r[0]);
  }
}

template <int M>
__device__ __forceinline__ float xor_lane_f(float v) {
  return __uint_as_float(xor_lane<M>(__float_as_uint(v)));
}

// Value of v in lane - 1 (lane 0 keeps its own): DPP wave_shr:1.
__device__ __forceinline__ uint32_t lane_shr1(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x138, 0xf, 0xf, false);
}

// Lanes that keep the larger key in the compare-exchange of merge size K,
// distance J of the bitonic network.
__host__ __device__ constexpr uint64_t bitonic_max_lanes(int K, int J) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l)
    if (((l & K) == 0) != ((l & J) == 0)) m |= 1ull << l;
  return m;
}

// One compare-exchange stage on a (64-bit key, 32-bit value) pair per lane.
// A lane takes its partner's pair when (partner < own) differs from "this
// lane keeps the larger key"; equal keys (only the ~0 padding) may then
// duplicate a padding value, which no caller reads.
template <int K, int J>
__device__ __forceinline__ void bitonic_step(uint64_t& key, uint32_t& val) {
  const uint32_t klo = (uint32_t)key, khi = (uint32_t)(key >> 32);
  const uint32_t olo = xor_lane<J>(klo);
  const uint32_t ohi = xor_lane<J>(khi);
  const uint32_t ov = xor_lane<J>(val);
  const uint64_t other = ((uint64_t)ohi << 32) | olo;
  const uint64_t sw = ballot64(other < key) ^ bitonic_max_lanes(K, J);
  key = ((uint64_t)lane_select(sw, khi, ohi) << 32) | lane_select(sw, klo, olo);
  val = lane_select(sw, val, ov);
}

template <int K, int J>
__device__ __forceinline__ void bitonic_merge(uint64_t& key, uint32_t& val) {
  bitonic_step<K, J>(key, val);
  if constexpr (J > 1) bitonic_merge<K, J / 2>(key, val);
}

// Bitonic sort of one (key, value) pair per lane, ascending by key across
// the 64 lanes.  Keys other than ~0 must be distinct.
__device__ __forceinline__ void wave_sort64_kv(uint64_t& key, uint32_t& val) {
  bitonic_merge<2, 1>(key, val);
  bitonic_merge<4, 2>(key, val);
  bitonic_merge<8, 4>(key, val);
  bitonic_merge<16, 8>(key, val);
  bitonic_merge<32, 16>(key, val);
  bitonic_merge<64, 32>(key, val);
}

// The same ordering for few keys: `live` (uniform) marks the lanes whose key
// is not ~0.  Each live lane counts the live keys below its own (one
// readlane pair and one compare per live lane; equal keys, which the callers
// never have, are ordered by lane so the positions stay a permutation), the
// other lanes take the positions after them in lane order, and one forward
// permute per 32-bit word moves every pair to its position.  About 5 VALU
// per live lane against ~170 for the bitonic network, so the cheaper form
// up to kFewSort live keys.  Every lane must be active.
constexpr int kFewSort = 16;
__device__ __forceinline__ void wave_sort_few_kv(uint64_t& key, uint32_t& val, uint64_t live) {
  int pos = 0;
  for (uint64_t m = live; m != 0; m &= m - 1) {
    const int l = (int)__builtin_ctzll(m);
    const uint64_t kl = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(key >> 32), l) << 32) |
                        (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, l);
    pos += (kl < key || (kl == key && l < lane_id())) ? 1 : 0;
  }
  if (!((live >> lane_id()) & 1)) pos = __popcll(live) + rank_below(~live);
  const int a = pos << 2;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_permute(a, (int)(uint32_t)key);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_permute(a, (int)(uint32_t)(key >> 32));
  val = (uint32_t)__builtin_amdgcn_ds_permute(a, (int)val);
  key = ((uint64_t)hi << 32) | lo;
}

// The shfl_down tree 16/8/4/2/1 of square_sum_32 (src/impl/util.cuh:36-45)
// over the partials of lanes 0..31, read at lane 0 and returned to every
// lane.  The xor butterfly adds the same operand pairs as shfl_down for the
// lanes that feed lane 0 (l ^ off == l + off for l < off).
__device__ __forceinline__ float square_sum_tree(float v) {
  v = v + xor_lane_f<16>(v);
  v = v + xor_lane_f<8>(v);
  v = v + xor_lane_f<4>(v);
  v = v + xor_lane_f<2>(v);
  v = v + xor_lane_f<1>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
}

// Exact squared L2 in the order of square_sum_32 (src/impl/util.cuh:26-46):
// 32 lane partials over dims l, l+32, ... (fma chains), then the shfl_down
// tree 16/8/4/2/1 read at lane 0.  Lanes 0..31 of the wave take the 32 lane
// roles; the xor butterfly adds the same operand pairs as shfl_down for the
// lanes that feed lane 0 (l ^ off == l + off for l < off).  Returns the value
// to every lane.
template <typename T>
__device__ __forceinline__ float l2_square_sum_32(const float* q, const T* x, int dim) {
  const int lane = lane_id() & 31;
  float v = 0.0f;
  for (int i = lane; i < dim; i += 32) {
    float d = q[i] - to_f(x[i]);
    v = fma_f(d, d, v);
  }
  return square_sum_tree(v);
}

// The same value computed entirely inside one lane (used where every lane
// scores a different vector): 32 partials kept in registers, then the tree.
template <typename T>
__device__ __forceinline__ float l2_square_sum_32_inlane(const float* q, const T* x, int dim) {
  float v[32];
#pragma unroll
  for (int l = 0; l < 32; ++l) v[l] = 0.0f;
  for (int base = 0; base < dim; base += 32) {
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      if (base + l < dim) {
        float d = q[base + l] - to_f(x[base + l]);
        v[l] = fma_f(d, d, v[l]);
      }
    }
  }
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) {
#pragma unroll
    for (int l = 0; l < off; ++l) v[l] = v[l] + v[l + off];
  }
  return v[0];
}

// Builds the LUT of one query into `lut` ([M][256], LDS or global) with the
// reference's arithmetic (src/impl/pq.cuh:8-59): row m accumulates
// (q_i - mu_i - P[k][i])^2 over its dims in ascending order from 0.
// qs must already hold q - centroid.
//
// Thread layout: lane (tid & 63) owns the pivot quad 4*lane .. 4*lane+3 and
// reads it as one float4 of pivots_t[i][*]; the (nthreads / 64) wave groups
// split the chunks.  W > 0: every chunk spans W consecutive dims (the
// compile-time common case, fully unrolled so all pivot loads of a chunk
// group are in flight together); W == 0: chunk bounds from chunk_off.
template <int W>
__device__ __forceinline__ void lut_build(const PQDev& pq, const float* qs, float* lut, int tid,
                                          int nthreads) {
  const int quad = tid & 63;
  const int group = tid >> 6, ngroups = nthreads >> 6;
  const float4* pt = reinterpret_cast<const float4*>(pq.pivots_t);
  float4* lut4 = reinterpret_cast<float4*>(lut);
  if constexpr (W > 0) {
    constexpr int kU = W >= 4 ? 2 : (W == 1 ? 8 : 4);  // chunks per batch
    int m = group;
    for (; m + (kU - 1) * ngroups < pq.M; m += kU * ngroups) {
      float4 p[kU][W];
#pragma unroll
      for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int w = 0; w < W; ++w) p[u][w] = pt[(int64_t)((m + u * ngroups) * W + w) * 64 + quad];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w = 0; w < W; ++w) {
          const float q = qs[(m + u * ngroups) * W + w];
          float d;
          d = q - p[u][w].x; acc.x = fma_f(d, d, acc.x);
          d = q - p[u][w].y; acc.y = fma_f(d, d, acc.y);
          d = q - p[u][w].z; acc.z = fma_f(d, d, acc.z);
          d = q - p[u][w].w; acc.w = fma_f(d, d, acc.w);
        }
        lut4[(m + u * ngroups) * 64 + quad] = acc;
      }
    }
    for (; m < pq.M; m += ngroups) {
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float4 pv = pt[(int64_t)(m * W + w) * 64 + quad];
        const float q = qs[m * W + w];
        float d;
        d = q - pv.x; acc.x = fma_f(d, d, acc.x);
        d = q - pv.y; acc.y = fma_f(d, d, acc.y);
        d = q - pv.z; acc.z = fma_f(d, d, acc.z);
        d = q - pv.w; acc.w = fma_f(d, d, acc.w);
      }
      lut4[m * 64 + quad] = acc;
    }
  } else {
    for (int m = group; m < pq.M; m += ngroups) {
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      const int lo = pq.chunk_off[m], hi = pq.chunk_off[m + 1];
      for (int i = lo; i < hi; ++i) {
        const float4 pv = pt[(int64_t)i * 64 + quad];
        const float q = qs[i];
        float d;
        d = q - pv.x; acc.x = fma_f(d, d, acc.x);
        d = q - pv.y; acc.y = fma_f(d, d, acc.y);
        d = q - pv.z; acc.z = fma_f(d, d, acc.z);
        d = q - pv.w; acc.w = fma_f(d, d, acc.w);
      }
      lut4[m * 64 + quad] = acc;
    }
  }
}

// Sequential ADC sum of one code row (src/impl/pure_mem.cuh:302-308).
// MW > 0: M == 16*MW and the row is read as MW 16-byte words (rows are then
// 16-byte aligned); MW == 0: byte reads for any M.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int MW>
struct CodeRow {
  u32x4 w[MW > 0 ? MW : 1];
  // all codes 0 (lanes without a neighbour: their lookups stay in bounds)
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int k = 0; k < (MW > 0 ? MW : 1); ++k) w[k] = u32x4{0u, 0u, 0u, 0u};
  }
  __device__ __forceinline__ void load(const uint8_t* row, int M) {
    if constexpr (MW > 0) {
      const u32x4* p = reinterpret_cast<const u32x4*>(row);
#pragma unroll
      for (int k = 0; k < MW; ++k) w[k] = p[k];
    } else {
      (void)row;
      (void)M;
    }
  }
  __device__ __forceinline__ float adc(const float* lut, const uint8_t* row, int M) const {
    float dist = 0.0f;
    if constexpr (MW > 0) {
#pragma unroll
      for (int k = 0; k < MW; ++k) {
        const uint32_t ws[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
#pragma unroll
        for (int b = 0; b < 16; ++b) {
          const uint32_t c = (ws[b >> 2] >> (8 * (b & 3))) & 0xffu;
          dist = dist + lut[(k * 16 + b) * kPivots + c];
        }
      }
    } else {
      for (int j = 0; j < M; ++j) dist = dist + lut[j * kPivots + row[j]];
    }
    return dist;
  }
};

}  // namespace gann

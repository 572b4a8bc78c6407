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
};

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
// float is monotonic in its value, so (bits(dist) << 32 | id & 0x7fffffff)
// compares exactly like the reference's two-level compare.
__device__ __forceinline__ uint64_t make_key(float d, uint32_t id) {
  return ((uint64_t)__float_as_uint(d) << 32) | (uint64_t)(id & kMask31);
}
// A list entry keeps the visited bit in bit 31 of its low word.
__device__ __forceinline__ uint64_t entry_key(uint64_t e) { return e & ~(uint64_t)kVisited; }
__device__ __forceinline__ uint32_t entry_id(uint64_t e) { return (uint32_t)e; }
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

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = (uint32_t)__shfl_xor((int)lo, m, kWave);
  hi = (uint32_t)__shfl_xor((int)hi, m, kWave);
  return ((uint64_t)hi << 32) | lo;
}

// Bitonic sort of one 64-bit key per lane, ascending by lane.
__device__ __forceinline__ uint64_t wave_sort64(uint64_t key) {
  const int lane = lane_id();
#pragma unroll
  for (int k = 2; k <= kWave; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      uint64_t other = shfl_xor_u64(key, j);
      bool up = (lane & k) == 0;
      bool lower = (lane & j) == 0;
      bool take_min = (lower == up);
      uint64_t mn = other < key ? other : key;
      uint64_t mx = other < key ? key : other;
      key = take_min ? mn : mx;
    }
  }
  return key;
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
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) v = v + __shfl_xor(v, off, 32);
  return __shfl(v, 0, kWave);
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

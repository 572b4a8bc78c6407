// Exact k-nearest-neighbour search by squared L2 (ties broken by the smaller
// id): the ground truth that recall is measured against.  The reference
// takes its ground truth from external tools; this is the GPU counterpart of
// the repository's CPU brute force (index_builder.cpp gib_brute_force).
//
// One wavefront owns 32 queries and a slice of the base set and scans it in
// tiles of 32 points.
//  * uint8: the 32x32 tile of dot products comes from v_mfma_i32_32x32x32_i8
//    on x - 128 and q - 128 (int8), so ||q - x||^2 = |q'|^2 + |x'|^2 - 2 q'.x'
//    is exact in int32 (at most 256 * 255^2 < 2^24, exact again as float).
//  * float: every lane forms 16 distances directly, sum over the dims in
//    ascending order of fma(t, t, s), t = q - x.
// A distance below the query's current k-th best is appended to the query's
// LDS buffer; a buffer that could overflow with the next tile is cut back to
// its k best by rank.  Points are scanned in increasing id order, so a tie
// with the k-th best loses to it.  Each wavefront writes its sorted k best
// per query; a tree of pairwise merges on the device folds the slices.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "gann_device.hpp"
#include "gann_knn.hpp"

namespace gann {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kQB = 32;  // queries per wavefront (MFMA rows)
constexpr int kTP = 32;  // points per tile (MFMA columns)
constexpr int kPF = 4;   // uint8 tiles in flight per wavefront
constexpr int kMaxK = 128;

// Row of accumulator register i of this lane in a 32x32 MFMA result (the
// column is lane % 32).
__device__ __forceinline__ int acc_row(int i, int lane) {
  return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
}

// Candidate key: bits(dist) << 32 | id.  Distances are non-negative and ids
// non-negative, so one unsigned compare orders (dist, id) lexicographically.
__device__ __forceinline__ uint64_t cand_key(float d, int32_t id) {
  return ((uint64_t)__float_as_uint(d) << 32) | (uint32_t)id;
}

// Per-wavefront candidate buffers: query m keeps keys [0, cnt[m]) of
// bk[m * cap ...]; thr[m] is the k-th smallest kept distance once k are kept
// (+inf before).  cap = k + 64 >= k + one tile.
struct KnnBuf {
  uint64_t* bk;
  int32_t* cnt;
  float* thr;
  int cap, k;

  __device__ void init() {
    const int lane = lane_id();
    if (lane < kQB) {
      cnt[lane] = 0;
      thr[lane] = INFINITY;
    }
    wave_sync();
  }

  __device__ __forceinline__ void append(int m, float d, int32_t id) {
    const int slot = atomicAdd(&cnt[m], 1);
    bk[(size_t)m * cap + slot] = cand_key(d, id);
  }

  // Keeps the k smallest keys of query m, sorted (each key's rank is the
  // number of smaller keys).
  __device__ void compact(int m) {
    const int lane = lane_id();
    const int n = cnt[m];
    uint64_t* k_m = bk + (size_t)m * cap;
    uint64_t v[3];
    int rk[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int e = lane + kWave * j;
      v[j] = e < n ? k_m[e] : ~(uint64_t)0;
      rk[j] = 0;
    }
#pragma unroll 8
    for (int e2 = 0; e2 < n; ++e2) {
      const uint64_t w = k_m[e2];
#pragma unroll
      for (int j = 0; j < 3; ++j) rk[j] += w < v[j] ? 1 : 0;
    }
    wave_sync();
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int e = lane + kWave * j;
      if (e < n && rk[j] < k) k_m[rk[j]] = v[j];
    }
    wave_sync();
    if (lane == 0) {
      cnt[m] = min(n, k);
      thr[m] = n >= k ? __uint_as_float((uint32_t)(k_m[k - 1] >> 32)) : INFINITY;
    }
    wave_sync();
  }

  // Cuts back every buffer that could overflow with one more tile; returns
  // whether any was cut.
  __device__ bool maybe_compact() {
    const int lane = lane_id();
    uint64_t need = ballot64(lane < kQB && cnt[lane] > cap - kTP);
    const bool any = need != 0;
    while (need) {
      const int m = (int)__builtin_ctzll(need);
      need &= need - 1;
      compact(m);
    }
    return any;
  }

  __device__ void finish(int q0, int nq, int64_t slice, float* part_d, int32_t* part_i) {
    const int lane = lane_id();
    for (int m = 0; m < kQB && q0 + m < nq; ++m) {
      compact(m);
      const int n = cnt[m];
      const int64_t o = (slice * nq + q0 + m) * (int64_t)k;
      for (int j = lane; j < k; j += kWave) {
        const uint64_t key = j < n ? bk[(size_t)m * cap + j] : 0;
        part_d[o + j] = j < n ? __uint_as_float((uint32_t)(key >> 32)) : INFINITY;
        part_i[o + j] = j < n ? (int32_t)(uint32_t)key : -1;
      }
    }
  }
};

__device__ __forceinline__ KnnBuf knn_buf(uint8_t* smem, int k) {
  KnnBuf B;
  B.k = k;
  B.cap = k + 64;
  B.bk = reinterpret_cast<uint64_t*>(smem);
  B.cnt = reinterpret_cast<int32_t*>(B.bk + (size_t)kQB * B.cap);
  B.thr = reinterpret_cast<float*>(B.cnt + kQB);
  return B;
}

// x - 128 as int8, rows padded with zeros to dp bytes, and |x - 128|^2.
__global__ void knn_prep_u8_kernel(const uint8_t* __restrict__ x, int64_t n, int dim, int dp,
                                   int8_t* __restrict__ xs, int32_t* __restrict__ xn) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int32_t s = 0;
  for (int d = 0; d < dp; ++d) {
    const int v = d < dim ? (int)x[i * dim + d] - 128 : 0;
    xs[i * dp + d] = (int8_t)v;
    s += v * v;
  }
  xn[i] = s;
}

// The same for dim == dp (a multiple of 32): one thread per 16 bytes, the
// norm accumulated with an atomic add per chunk (xn zeroed first).
__global__ void knn_prep_u8_wide_kernel(const uint4* __restrict__ x, int64_t chunks, int cpr,
                                        uint4* __restrict__ xs, int32_t* __restrict__ xn) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= chunks) return;
  const uint4 v = x[c];
  const uint32_t w[4] = {v.x ^ 0x80808080u, v.y ^ 0x80808080u, v.z ^ 0x80808080u,
                         v.w ^ 0x80808080u};
  int32_t s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int t = (int)(int8_t)(uint8_t)(w[j] >> (8 * b));
      s += t * t;
    }
  xs[c] = make_uint4(w[0], w[1], w[2], w[3]);
  atomicAdd(&xn[c / cpr], s);
}

// One 32-point tile of B operands (lane: point t0 + lane % 32, bytes
// 16 * (lane / 32) + 32 s) and the point's |x'|^2; points at or past `end`
// (any distance past it) read row `start` and are marked invalid.
template <int STEPS>
struct KnnTile {
  v4i b[STEPS];
  int32_t xn;
  bool valid;
  __device__ __forceinline__ void load(const int8_t* xs, const int32_t* xnorm, int64_t t0,
                                       int64_t start, int64_t end, int lane) {
    constexpr int dp = 32 * STEPS;
    const int64_t p = t0 + (lane & 31);
    const int64_t r = p < end ? p : start;
    const int8_t* xrow = xs + r * dp + 16 * (lane >> 5);
#pragma unroll
    for (int s = 0; s < STEPS; ++s) b[s] = *reinterpret_cast<const v4i*>(xrow + 32 * s);
    xn = xnorm[r];
    valid = p < end;
  }
};

template <int STEPS>
__global__ __launch_bounds__(64) void knn_u8_kernel(const int8_t* __restrict__ xs,
                                                    const int32_t* __restrict__ xn, int64_t n,
                                                    const int8_t* __restrict__ qs,
                                                    const int32_t* __restrict__ qn, int nq, int k,
                                                    int64_t slice_len, int64_t id_base,
                                                    float* __restrict__ part_d,
                                                    int32_t* __restrict__ part_i) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  constexpr int dp = 32 * STEPS;
  const int lane = lane_id();
  const int q0 = blockIdx.x * kQB;
  const int64_t slice = blockIdx.y;
  const int64_t start = slice * slice_len, end = min(n, start + slice_len);
  KnnBuf B = knn_buf(smem_raw, k);
  B.init();
  // A: query q0 + lane % 32, bytes 16 * (lane / 32) + 32 s (query rows are
  // padded to a multiple of 32 on the host)
  v4i a[STEPS];
  const int8_t* qrow = qs + (size_t)(q0 + (lane & 31)) * dp + 16 * (lane >> 5);
#pragma unroll
  for (int s = 0; s < STEPS; ++s) a[s] = *reinterpret_cast<const v4i*>(qrow + 32 * s);
  // distances are exact integers: thresholds in int32 (rows past nq take
  // nothing)
  int32_t qn_r[16], thr_r[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int m = acc_row(i, lane);
    qn_r[i] = qn[q0 + m];
    thr_r[i] = q0 + m < nq ? INT32_MAX : INT32_MIN;
  }
  // the query rows and norms are waited for here, before the loop: loads
  // left pending into it would make their first uses there wait on the tile
  // loads too, on every tile
#pragma unroll
  for (int s = 0; s < STEPS; ++s) asm volatile("" ::"v"(a[s]));
#pragma unroll
  for (int i = 0; i < 16; ++i) asm volatile("" ::"v"(qn_r[i]));
  // kPF tiles in flight: tile t0 is used kPF tiles after its loads were
  // issued.  The loads are unconditional (tiles past the slice read row
  // `start`, marked invalid), so every path through the loop has the same
  // loads outstanding and the wait before a tile's products covers only
  // that tile.
  // (the first kPF are requested in tile order, as the loop requests them,
  // so the wait at the loop head is the same from either side)
  KnnTile<STEPS> tl[kPF];
#pragma unroll
  for (int u = 0; u < kPF; ++u) {
    tl[u].load(xs, xn, start + u * kTP, start, end, lane);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int64_t g = start; g < end; g += kPF * kTP) {
#pragma unroll
    for (int u = 0; u < kPF; ++u) {
      const int64_t t0 = g + u * kTP;
      v16i acc = {};
#pragma unroll
      for (int s = 0; s < STEPS; ++s)
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s], tl[u].b[s], acc, 0, 0, 0);
      const bool valid = tl[u].valid;
      int32_t dist[16];
      uint64_t any = 0;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        dist[i] = qn_r[i] + tl[u].xn - 2 * acc[i];
        any |= ballot64(valid && dist[i] < thr_r[i]);
      }
      tl[u].load(xs, xn, t0 + kPF * kTP, start, end, lane);
      if (any) {
        const int32_t id = (int32_t)(t0 + (lane & 31) + id_base);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (valid && dist[i] < thr_r[i]) B.append(acc_row(i, lane), (float)dist[i], id);
        }
        wave_sync();
        if (B.maybe_compact()) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int m = acc_row(i, lane);
            const float t = B.thr[m];
            if (q0 + m < nq) thr_r[i] = t == INFINITY ? INT32_MAX : (int32_t)t;
          }
        }
      }
    }
  }
  B.finish(q0, nq, slice, part_d, part_i);
}

// Float: the 32 queries of the wavefront in LDS after the buffers.
__global__ __launch_bounds__(64) void knn_f32_kernel(const float* __restrict__ x, int64_t n,
                                                     int dim, const float* __restrict__ q, int nq,
                                                     int k, int64_t slice_len, int64_t id_base,
                                                     float* __restrict__ part_d,
                                                     int32_t* __restrict__ part_i) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  const int lane = lane_id();
  const int q0 = blockIdx.x * kQB;
  const int64_t slice = blockIdx.y;
  const int64_t start = slice * slice_len, end = min(n, start + slice_len);
  KnnBuf B = knn_buf(smem_raw, k);
  float* qt = reinterpret_cast<float*>(B.thr + kQB);
  for (int e = lane; e < kQB * dim; e += kWave) {
    const int m = e / dim;
    qt[e] = q0 + m < nq ? q[(size_t)(q0 + m) * dim + (e - m * dim)] : 0.0f;
  }
  B.init();
  float thr_r[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) thr_r[i] = INFINITY;
  for (int64_t t0 = start; t0 < end; t0 += kTP) {
    const int64_t p = t0 + (lane & 31);
    const bool valid = p < end;
    const float* xr = x + (size_t)(valid ? p : start) * dim;
    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    for (int d = 0; d < dim; ++d) {
      const float xv = xr[d];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float t = qt[acc_row(i, lane) * dim + d] - xv;
        acc[i] = fma_f(t, t, acc[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = acc_row(i, lane);
      if (valid && q0 + m < nq && acc[i] < thr_r[i]) B.append(m, acc[i], (int32_t)(p + id_base));
    }
    wave_sync();
    if (B.maybe_compact()) {
#pragma unroll
      for (int i = 0; i < 16; ++i) thr_r[i] = B.thr[acc_row(i, lane)];
    }
  }
  B.finish(q0, nq, slice, part_d, part_i);
}

// One level of the slice merge: for query blockIdx.x, the sorted k-lists of
// slots a and b = a + stride (a = 2 * stride * blockIdx.y) become the first k
// of their union in (dist, id) order, written to slot a.  Entry j of list A
// goes to j + #{B < A[j]}, entry j of B to j + #{A <= B[j]}: a stable merge,
// so the padding entries (+inf, -1), all equal, still take distinct places
// and order after every real entry.  Both lists are read into LDS before any
// write, and each block owns its two slots.
__global__ __launch_bounds__(64) void knn_merge_kernel(float* __restrict__ part_d,
                                                       int32_t* __restrict__ part_i, int nq, int k,
                                                       int64_t slots, int64_t stride) {
  __shared__ uint64_t ka[kMaxK], kb[kMaxK];
  const int q = blockIdx.x;
  const int64_t a = (int64_t)blockIdx.y * 2 * stride, b = a + stride;
  if (b >= slots) return;
  const int lane = threadIdx.x;
  const size_t oa = ((size_t)a * nq + q) * k, ob = ((size_t)b * nq + q) * k;
  for (int j = lane; j < k; j += kWave) {
    ka[j] = cand_key(part_d[oa + j], part_i[oa + j]);
    kb[j] = cand_key(part_d[ob + j], part_i[ob + j]);
  }
  __syncthreads();
  for (int j = lane; j < k; j += kWave) {
    const uint64_t x = ka[j], y = kb[j];
    int lo = 0, hi = k;
    while (lo < hi) {
      const int m = (lo + hi) >> 1;
      if (kb[m] < x) lo = m + 1; else hi = m;
    }
    const int ra = j + lo;
    lo = 0, hi = k;
    while (lo < hi) {
      const int m = (lo + hi) >> 1;
      if (ka[m] <= y) lo = m + 1; else hi = m;
    }
    const int rb = j + lo;
    if (ra < k) {
      part_d[oa + ra] = __uint_as_float((uint32_t)(x >> 32));
      part_i[oa + ra] = (int32_t)(uint32_t)x;
    }
    if (rb < k) {
      part_d[oa + rb] = __uint_as_float((uint32_t)(y >> 32));
      part_i[oa + rb] = (int32_t)(uint32_t)y;
    }
  }
}

size_t knn_buf_bytes(int k) { return (size_t)kQB * (k + 64) * 8 + (size_t)kQB * 8; }

}  // namespace

hipError_t launch_knn_merge(float* part_d, int32_t* part_i, int nq, int k, int64_t slots,
                            hipStream_t stream) {
  if (k < 1 || k > kMaxK || nq < 0) return hipErrorInvalidValue;
  if (nq == 0) return hipSuccess;
  for (int64_t stride = 1; stride < slots; stride *= 2) {
    const dim3 grid((unsigned)nq, (unsigned)((slots + 2 * stride - 1) / (2 * stride)));
    hipLaunchKernelGGL(knn_merge_kernel, grid, dim3(kWave), 0, stream, part_d, part_i, nq, k, slots,
                       stride);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

int knn_queries_per_block() { return kQB; }

size_t knn_smem_bytes(int dtype, int dim, int k) {
  return knn_buf_bytes(k) + (dtype == 0 ? 0 : (size_t)kQB * dim * 4);
}

hipError_t launch_knn_prep_u8(const uint8_t* x, int64_t n, int dim, int dp, int8_t* xs, int32_t* xn,
                              hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  if (dim == dp) {
    hipError_t e = hipMemsetAsync(xn, 0, (size_t)n * 4, stream);
    if (e != hipSuccess) return e;
    const int cpr = dp / 16;
    const int64_t chunks = n * cpr;
    hipLaunchKernelGGL(knn_prep_u8_wide_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                       stream, reinterpret_cast<const uint4*>(x), chunks, cpr,
                       reinterpret_cast<uint4*>(xs), xn);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(knn_prep_u8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, x,
                     n, dim, dp, xs, xn);
  return hipGetLastError();
}

hipError_t launch_knn_u8(const int8_t* xs, const int32_t* xn, int64_t n, int dp, const int8_t* qs,
                         const int32_t* qn, int nq, int k, int64_t slices, int64_t slice_len,
                         int64_t id_base, float* part_d, int32_t* part_i, hipStream_t stream) {
  const dim3 grid((unsigned)((nq + kQB - 1) / kQB), (unsigned)slices);
  const size_t smem = knn_smem_bytes(0, dp, k);
  switch (dp / 32) {
#define GANN_KNN_CASE(S)                                                                      \
  case S:                                                                                     \
    hipLaunchKernelGGL(knn_u8_kernel<S>, grid, dim3(64), smem, stream, xs, xn, n, qs, qn, nq, \
                       k, slice_len, id_base, part_d, part_i);                                \
    break;
    GANN_KNN_CASE(1)
    GANN_KNN_CASE(2)
    GANN_KNN_CASE(3)
    GANN_KNN_CASE(4)
    GANN_KNN_CASE(5)
    GANN_KNN_CASE(6)
    GANN_KNN_CASE(7)
    GANN_KNN_CASE(8)
#undef GANN_KNN_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_knn_f32(const float* x, int64_t n, int dim, const float* q, int nq, int k,
                          int64_t slices, int64_t slice_len, int64_t id_base, float* part_d,
                          int32_t* part_i, hipStream_t stream) {
  const dim3 grid((unsigned)((nq + kQB - 1) / kQB), (unsigned)slices);
  hipLaunchKernelGGL(knn_f32_kernel, grid, dim3(64), knn_smem_bytes(1, dim, k), stream, x, n, dim,
                     q, nq, k, slice_len, id_base, part_d, part_i);
  return hipGetLastError();
}

}  // namespace gann

// Exact k-nearest-neighbour search by squared L2 (ties broken by the smaller
// id): the ground truth that recall is measured against.  The reference
// takes its ground truth from external tools; this is the GPU counterpart of
// the repository's CPU brute force (index_builder.cpp gib_brute_force).
//
// One wavefront owns a block of queries and a slice of the base set and
// scans it in tiles of 32 points.
//  * uint8: the dot products come from int8 MFMA on x - 128 and q - 128, so
//    ||q - x||^2 = |q'|^2 + |x'|^2 - 2 q'.x' is exact in int32 (at most
//    256 * 255^2 < 2^24, exact again as float).  Two forms (U8Form): 32
//    queries with one 32x32 block of v_mfma_i32_32x32x32_i8 per tile, or 16
//    queries with two 16x16 blocks of v_mfma_i32_16x16x64_i8, whose halved
//    candidate buffers let more wavefronts fit a CU's LDS when k is large.
//  * float: 32 queries; every lane forms 16 distances directly, sum over the
//    dims in ascending order of fma(t, t, s), t = q - x.
// A distance below the query's current k-th best is appended to the query's
// LDS buffer; a buffer that could overflow with the next tile is cut back to
// its k best (a merge of the new keys into the sorted kept ones).  Points are
// scanned in increasing id order, so a tie with the k-th best loses to it.
// Each wavefront writes its sorted k best per query; a tree of pairwise
// merges on the device folds the slices.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "gann_device.hpp"
#include "gann_knn.hpp"

namespace gann {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kQB = 32;   // float: queries per wavefront
constexpr int kTP = 32;   // points per tile
constexpr int kPF = 4;    // uint8 tiles in flight per wavefront
constexpr int kMaxK = 128;

// The query of distance i of this lane in a 32x32 block (the point is
// lane % 32): the layout of a 32x32 MFMA result, used by the float kernel too.
__device__ __forceinline__ int acc_row(int i, int lane) {
  return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
}


// Candidate key: bits(dist) << 32 | id.  Distances are non-negative and ids
// non-negative, so one unsigned compare orders (dist, id) lexicographically.
__device__ __forceinline__ uint64_t cand_key(float d, int32_t id) {
  return ((uint64_t)__float_as_uint(d) << 32) | (uint32_t)id;
}

// Per-wavefront candidate buffers of QB queries: query m keeps keys
// [0, cnt[m]) of bk[m * cap ...], of which the first srt[m] (those kept by
// the last cut) are sorted; thr[m] is the k-th smallest kept distance once k
// are kept (+inf before).  cap = k + 64 >= k + one tile.
template <int QB>
struct KnnBuf {
  uint64_t* bk;
  int32_t* cnt;
  float* thr;
  int32_t* srt;
  int cap, k;

  __device__ void init() {
    const int lane = lane_id();
    if (lane < QB) {
      cnt[lane] = 0;
      thr[lane] = INFINITY;
      srt[lane] = 0;
    }
    wave_sync();
  }

  __device__ __forceinline__ void append(int m, float d, int32_t id) {
    const int slot = atomicAdd(&cnt[m], 1);
    bk[(size_t)m * cap + slot] = cand_key(d, id);
  }

  // Keeps the k smallest keys of query m, sorted.  The keys are distinct
  // (one per point).  With a sorted prefix of h and at most 64 keys after it
  // (every cut but a query's first), a merge: new key x goes to
  // #{new < x} + #{old < x}, old key i to i + #{new < old i}; the counts over
  // the new keys come from one pass over them, #{old < x} from a binary
  // search of the prefix.  Otherwise each key goes to its rank among all.
  __device__ void compact(int m) {
    const int lane = lane_id();
    const int n = cnt[m], h = srt[m], nn = n - h;
    uint64_t* k_m = bk + (size_t)m * cap;
    if (h > 0 && nn <= kWave) {
      const uint64_t x = lane < nn ? k_m[h + lane] : ~(uint64_t)0;
      const uint64_t o0 = lane < h ? k_m[lane] : ~(uint64_t)0;
      const uint64_t o1 = lane + kWave < h ? k_m[lane + kWave] : ~(uint64_t)0;
      int rn = 0, c0 = 0, c1 = 0;
#pragma unroll 8
      for (int j = 0; j < nn; ++j) {
        const uint64_t w = k_m[h + j];
        rn += w < x ? 1 : 0;
        c0 += w < o0 ? 1 : 0;
        c1 += w < o1 ? 1 : 0;
      }
      int lo = 0, hi = h;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (k_m[mid] < x) lo = mid + 1; else hi = mid;
      }
      wave_sync();
      if (lane < nn && rn + lo < k) k_m[rn + lo] = x;
      if (lane < h && lane + c0 < k) k_m[lane + c0] = o0;
      if (lane + kWave < h && lane + kWave + c1 < k) k_m[lane + kWave + c1] = o1;
      wave_sync();
      if (lane == 0) {
        cnt[m] = srt[m] = min(n, k);
        thr[m] = n >= k ? __uint_as_float((uint32_t)(k_m[k - 1] >> 32)) : INFINITY;
      }
      wave_sync();
      return;
    }
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
      cnt[m] = srt[m] = min(n, k);
      thr[m] = n >= k ? __uint_as_float((uint32_t)(k_m[k - 1] >> 32)) : INFINITY;
    }
    wave_sync();
  }

  // Cuts back every buffer that could overflow with one more tile; returns
  // whether any was cut.
  __device__ bool maybe_compact() {
    const int lane = lane_id();
    uint64_t need = ballot64(lane < QB && cnt[lane] > cap - kTP);
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
    for (int m = 0; m < QB && q0 + m < nq; ++m) {
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

template <int QB>
__device__ __forceinline__ KnnBuf<QB> knn_buf(uint8_t* smem, int k) {
  KnnBuf<QB> B;
  B.k = k;
  B.cap = k + 64;
  B.bk = reinterpret_cast<uint64_t*>(smem);
  B.cnt = reinterpret_cast<int32_t*>(B.bk + (size_t)QB * B.cap);
  B.thr = reinterpret_cast<float*>(B.cnt + QB);
  B.srt = B.cnt + 2 * QB;
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

// The two uint8 forms.  A form fixes the queries per wavefront QB, the K
// bytes of one product step (kK = 1024 / QB: 64 lanes x 16 bytes cover QB
// rows), and where each of a lane's kND distances of a 32-point tile sits:
// its query (one of the lane's kNR query slots) and its column block h
// (points t0 + QB h + lane % QB).  Lane l holds bytes 16 (l / QB) + kK s of
// query row l % QB and of the points of its column, the same K bytes on
// both sides, so every product is a whole dot product.
template <int QB, int STEPS>
struct U8Form;

// 32 queries: one 32x32 block per tile from v_mfma_i32_32x32x32_i8;
// distance i is query 8 (i / 4) + 4 (lane / 32) + i % 4.  Reads each point
// once per 32 queries.
template <int STEPS>
struct U8Form<32, STEPS> {
  static constexpr int kK = 32, kH = 1, kND = 16, kNR = 16;
  static __device__ __forceinline__ int slot(int i) { return i; }
  static __device__ __forceinline__ int block(int) { return 0; }
  static __device__ __forceinline__ int row(int r, int lane) { return acc_row(r, lane); }
  static __device__ __forceinline__ void products(const v4i* a, const v4i (*b)[STEPS], int32_t* dot) {
    typedef int v16i __attribute__((ext_vector_type(16)));
    v16i acc = {};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s], b[0][s], acc, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < kND; ++i) dot[i] = acc[i];
  }
};

// 16 queries: two 16x16 blocks per tile from v_mfma_i32_16x16x64_i8;
// distance i is query 4 (lane / 16) + i % 4 of block i / 4.  Half the
// candidate buffers of the 32-query form, so more wavefronts fit a CU's LDS
// when k is large, for twice the point reads.
template <int STEPS>
struct U8Form<16, STEPS> {
  static constexpr int kK = 64, kH = 2, kND = 8, kNR = 4;
  static __device__ __forceinline__ int slot(int i) { return i & 3; }
  static __device__ __forceinline__ int block(int i) { return i >> 2; }
  static __device__ __forceinline__ int row(int r, int lane) { return 4 * (lane >> 4) + r; }
  static __device__ __forceinline__ void products(const v4i* a, const v4i (*b)[STEPS], int32_t* dot) {
    v4i acc[2] = {};
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int s = 0; s < STEPS; ++s)
        acc[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[s], b[h][s], acc[h], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < kND; ++i) dot[i] = acc[i >> 2][i & 3];
  }
};

// One 32-point tile of B operands (column block h: points t0 + QB h + lane %
// QB, bytes 16 (lane / QB) + kK s of each) and the points' |x'|^2; points at
// or past `end` (any distance past it) read row `start` and are marked
// invalid.
template <int QB, int STEPS>
struct KnnTile {
  using F = U8Form<QB, STEPS>;
  v4i b[F::kH][STEPS];
  int32_t xn[F::kH];
  bool valid[F::kH];
  __device__ __forceinline__ void load(const int8_t* xs, const int32_t* xnorm, int64_t t0,
                                       int64_t start, int64_t end, int lane) {
    constexpr int dp = F::kK * STEPS;
#pragma unroll
    for (int h = 0; h < F::kH; ++h) {
      const int64_t p = t0 + QB * h + lane % QB;
      const int64_t r = p < end ? p : start;
      const int8_t* xrow = xs + r * dp + 16 * (lane / QB);
#pragma unroll
      for (int s = 0; s < STEPS; ++s) b[h][s] = *reinterpret_cast<const v4i*>(xrow + F::kK * s);
      xn[h] = xnorm[r];
      valid[h] = p < end;
    }
  }
};

template <int QB, int STEPS>
__global__ __launch_bounds__(64) void knn_u8_kernel(const int8_t* __restrict__ xs,
                                                    const int32_t* __restrict__ xn, int64_t n,
                                                    const int8_t* __restrict__ qs,
                                                    const int32_t* __restrict__ qn, int nq, int k,
                                                    int64_t slice_len, int64_t id_base,
                                                    float* __restrict__ part_d,
                                                    int32_t* __restrict__ part_i) {
  using F = U8Form<QB, STEPS>;
  extern __shared__ __align__(16) uint8_t smem_raw[];
  constexpr int dp = F::kK * STEPS;
  const int lane = lane_id();
  const int q0 = blockIdx.x * QB;
  const int64_t slice = blockIdx.y;
  const int64_t start = slice * slice_len, end = min(n, start + slice_len);
  KnnBuf<QB> B = knn_buf<QB>(smem_raw, k);
  B.init();
  // A: query q0 + lane % QB, bytes 16 * (lane / QB) + kK s (query rows are
  // padded to a multiple of QB on the host)
  v4i a[STEPS];
  const int8_t* qrow = qs + (size_t)(q0 + lane % QB) * dp + 16 * (lane / QB);
#pragma unroll
  for (int s = 0; s < STEPS; ++s) a[s] = *reinterpret_cast<const v4i*>(qrow + F::kK * s);
  // distances are exact integers: thresholds in int32 (rows past nq take
  // nothing)
  int32_t qn_r[F::kNR], thr_r[F::kNR];
#pragma unroll
  for (int r = 0; r < F::kNR; ++r) {
    const int m = F::row(r, lane);
    qn_r[r] = qn[q0 + m];
    thr_r[r] = q0 + m < nq ? INT32_MAX : INT32_MIN;
  }
  // the query rows and norms are waited for here, before the loop: loads
  // left pending into it would make their first uses there wait on the tile
  // loads too, on every tile
#pragma unroll
  for (int s = 0; s < STEPS; ++s) asm volatile("" ::"v"(a[s]));
#pragma unroll
  for (int r = 0; r < F::kNR; ++r) asm volatile("" ::"v"(qn_r[r]));
  // kPF tiles in flight: tile t0 is used kPF tiles after its loads were
  // issued.  The loads are unconditional (tiles past the slice read row
  // `start`, marked invalid), so every path through the loop has the same
  // loads outstanding and the wait before a tile's products covers only
  // that tile (the first kPF are requested in tile order, as the loop
  // requests them, so the wait at the loop head is the same from either
  // side).
  KnnTile<QB, STEPS> tl[kPF];
#pragma unroll
  for (int u = 0; u < kPF; ++u) {
    tl[u].load(xs, xn, start + u * kTP, start, end, lane);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int64_t g = start; g < end; g += kPF * kTP) {
#pragma unroll
    for (int u = 0; u < kPF; ++u) {
      const int64_t t0 = g + u * kTP;
      int32_t dist[F::kND];
      F::products(a, tl[u].b, dist);
      bool valid[F::kH];
#pragma unroll
      for (int h = 0; h < F::kH; ++h) valid[h] = tl[u].valid[h];
      uint64_t any = 0;
#pragma unroll
      for (int i = 0; i < F::kND; ++i) {
        dist[i] = qn_r[F::slot(i)] + tl[u].xn[F::block(i)] - 2 * dist[i];
        any |= ballot64(valid[F::block(i)] && dist[i] < thr_r[F::slot(i)]);
      }
      tl[u].load(xs, xn, t0 + kPF * kTP, start, end, lane);
      if (any) {
        const int32_t id = (int32_t)(t0 + lane % QB + id_base);
#pragma unroll
        for (int i = 0; i < F::kND; ++i) {
          if (valid[F::block(i)] && dist[i] < thr_r[F::slot(i)])
            B.append(F::row(F::slot(i), lane), (float)dist[i], id + QB * F::block(i));
        }
        wave_sync();
        if (B.maybe_compact()) {
#pragma unroll
          for (int r = 0; r < F::kNR; ++r) {
            const int m = F::row(r, lane);
            const float t = B.thr[m];
            if (q0 + m < nq) thr_r[r] = t == INFINITY ? INT32_MAX : (int32_t)t;
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
  KnnBuf<kQB> B = knn_buf<kQB>(smem_raw, k);
  float* qt = reinterpret_cast<float*>(B.srt + kQB);
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

size_t knn_buf_bytes(int qb, int k) { return (size_t)qb * (k + 64) * 8 + (size_t)qb * 12; }

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

size_t knn_smem_bytes(int dtype, int qb, int dim, int k) {
  return dtype == 0 ? knn_buf_bytes(qb, k) : knn_buf_bytes(kQB, k) + (size_t)kQB * dim * 4;
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

namespace {

// Calls f with the uint8 kernel of QB queries for rows of dp bytes (a
// multiple of 1024 / QB, at most 256).
template <int QB, typename F>
hipError_t with_knn_u8_kernel(int dp, F f) {
  constexpr int kK = U8Form<QB, 1>::kK;
  if (dp % kK != 0) return hipErrorInvalidValue;
  switch (dp / kK) {
    case 1: return f(knn_u8_kernel<QB, 1>);
    case 2: return f(knn_u8_kernel<QB, 2>);
    case 3: return f(knn_u8_kernel<QB, 3>);
    case 4: return f(knn_u8_kernel<QB, 4>);
    default: break;
  }
  if constexpr (QB == 32) {
    switch (dp / kK) {
      case 5: return f(knn_u8_kernel<QB, 5>);
      case 6: return f(knn_u8_kernel<QB, 6>);
      case 7: return f(knn_u8_kernel<QB, 7>);
      case 8: return f(knn_u8_kernel<QB, 8>);
      default: break;
    }
  }
  return hipErrorInvalidValue;
}

template <int QB>
int u8_blocks_per_cu(int dp, int k) {
  int nb = 0;
  const size_t smem = knn_smem_bytes(0, QB, dp, k);
  const hipError_t e = with_knn_u8_kernel<QB>(dp, [&](auto kern) {
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, kWave, smem);
  });
  return e == hipSuccess ? nb : 0;
}

}  // namespace

KnnU8Form knn_u8_form(int dim, int k) {
  KnnU8Form q32{32, (dim + 31) / 32 * 32, 0}, q16{16, (dim + 63) / 64 * 64, 0};
  q32.blocks_per_cu = u8_blocks_per_cu<32>(q32.dp, k);
  q16.blocks_per_cu = u8_blocks_per_cu<16>(q16.dp, k);
  return 16 * q16.blocks_per_cu > 32 * q32.blocks_per_cu ? q16 : q32;
}

int knn_f32_blocks_per_cu(int dim, int k) {
  int nb = 0;
  const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, knn_f32_kernel, kWave,
                                                                   knn_smem_bytes(1, kQB, dim, k));
  return e == hipSuccess ? nb : 0;
}

hipError_t launch_knn_u8(const KnnU8Form& form, const int8_t* xs, const int32_t* xn, int64_t n,
                         const int8_t* qs, const int32_t* qn, int nq, int k, int64_t slices,
                         int64_t slice_len, int64_t id_base, float* part_d, int32_t* part_i,
                         hipStream_t stream) {
  const dim3 grid((unsigned)((nq + form.qb - 1) / form.qb), (unsigned)slices);
  const size_t smem = knn_smem_bytes(0, form.qb, form.dp, k);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(kWave), smem, stream, xs, xn, n, qs, qn, nq, k, slice_len,
                       id_base, part_d, part_i);
    return hipGetLastError();
  };
  if (form.qb == 32) return with_knn_u8_kernel<32>(form.dp, go);
  if (form.qb == 16) return with_knn_u8_kernel<16>(form.dp, go);
  return hipErrorInvalidValue;
}

hipError_t launch_knn_f32(const float* x, int64_t n, int dim, const float* q, int nq, int k,
                          int64_t slices, int64_t slice_len, int64_t id_base, float* part_d,
                          int32_t* part_i, hipStream_t stream) {
  const dim3 grid((unsigned)((nq + kQB - 1) / kQB), (unsigned)slices);
  hipLaunchKernelGGL(knn_f32_kernel, grid, dim3(64), knn_smem_bytes(1, kQB, dim, k), stream, x, n, dim,
                     q, nq, k, slice_len, id_base, part_d, part_i);
  return hipGetLastError();
}

}  // namespace gann

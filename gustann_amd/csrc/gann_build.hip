// GPU Vamana graph builder for uint8 points (gfx950, wave64).
//
// The reference builds its graphs with DiskANN's CPU tools
// (scripts/build_diskann_index.sh:7, scripts/gen_pivot_graph.sh:13), which
// are absent here; index_builder.cpp restates Vamana on the CPU: a random
// initial graph, then for every point in a seeded random order a greedy
// search from the medoid, RobustPrune with alpha over the expanded nodes and
// the current neighbours, and reverse edges, in a pass with alpha = 1 and a
// pass with the given alpha.  This file runs the same steps on the device,
// for batches of points at a time:
//   1. build_search_kernel: one wavefront per point, greedy search over the
//      current graph with exact distances and the list update of the search
//      kernels (gann_list.hpp); the best expanded nodes are the candidates.
//   2. build_prune_fwd_kernel: RobustPrune of candidates + current
//      neighbours into the point's list; its edges become reverse-edge
//      requests (target << 32 | source).
//   3. the requests are sorted by target and each target's run is handled by
//      one wavefront (build_reverse_kernel): appended while the list has
//      room (up to C = ceil(1.3 R), DiskANN's slack), else the list and the
//      new sources are pruned back to R.
//   4. after the passes, lists longer than R are pruned back to R.
// Points of one batch see the graph as it was when the batch started; the
// searches follow the first R entries of each list.
// Distances are exact: |a|^2 + |b|^2 - 2 a.b with v_dot4_u32_u8, below 2^24
// for dim <= 256, so they are exact floats equal to the host builder's.
#include "gann_build.hpp"

#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <climits>
#include <cmath>
#include <type_traits>

#include "gann_device.hpp"
#include "gann_list.hpp"

namespace gann {
namespace {

typedef const __attribute__((address_space(4))) uint32_t* ConstU32;

// Row `id` for the whole wavefront, read with scalar loads (the rows are
// not written while the builder runs): w[i] = 32-bit word i.
template <int NC>
__device__ __forceinline__ void uniform_row(const uint8_t* x, int dp, uint32_t id,
                                            uint32_t (&w)[4 * NC]) {
  uint64_t a = (uint64_t)(x + (int64_t)id * dp);
  asm volatile("" : "+s"(a));
  ConstU32 p = (ConstU32)a;
#pragma unroll
  for (int i = 0; i < 4 * NC; ++i) w[i] = p[i];
}

__device__ __forceinline__ uint32_t dot16(const u32x4& a, const u32x4& b, uint32_t acc) {
  acc = __builtin_amdgcn_udot4(a.x, b.x, acc, false);
  acc = __builtin_amdgcn_udot4(a.y, b.y, acc, false);
  acc = __builtin_amdgcn_udot4(a.z, b.z, acc, false);
  return __builtin_amdgcn_udot4(a.w, b.w, acc, false);
}

// Dot product of a wave-uniform row with this lane's row (global memory).
template <int NC>
__device__ __forceinline__ uint32_t row_dot(const uint32_t (&w)[4 * NC], const uint8_t* row) {
  const u32x4* r = reinterpret_cast<const u32x4*>(row);
  u32x4 v[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) v[c] = r[c];
  uint32_t acc = 0;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const u32x4 q = {w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]};
    acc = dot16(q, v[c], acc);
  }
  return acc;
}

__device__ __forceinline__ float sq_dist(int32_t na, int32_t nb, uint32_t dot) {
  return (float)(na + nb - 2 * (int32_t)dot);
}

// ------------------------------------------------------------------ preparation

__global__ __launch_bounds__(256) void norms_kernel(const uint8_t* __restrict__ x, int64_t n, int dp,
                                                    int32_t* __restrict__ xn) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const u32x4* r = reinterpret_cast<const u32x4*>(x + i * dp);
  uint32_t acc = 0;
  for (int c = 0; c < dp / 16; ++c) {
    const u32x4 v = r[c];
    acc = dot16(v, v, acc);
  }
  xn[i] = (int32_t)acc;
}

__global__ __launch_bounds__(256) void col_sums_kernel(const uint8_t* __restrict__ x, int64_t n, int dp,
                                                       unsigned long long* __restrict__ sums) {
  __shared__ unsigned long long acc[256];
  acc[threadIdx.x] = 0;
  __syncthreads();
  const int gpr = dp / 4;      // words per row
  const int rpb = 256 / gpr;   // rows per block step; threads past rpb * gpr idle
  const int w = (int)threadIdx.x % gpr;
  uint32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  for (int64_t r = (int)threadIdx.x < rpb * gpr ? (int64_t)blockIdx.x * rpb + (int)threadIdx.x / gpr : n;
       r < n; r += (int64_t)gridDim.x * rpb) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(x + r * dp + 4 * w);
    s0 += v & 0xffu;
    s1 += (v >> 8) & 0xffu;
    s2 += (v >> 16) & 0xffu;
    s3 += v >> 24;
  }
  atomicAdd(&acc[4 * w + 0], (unsigned long long)s0);
  atomicAdd(&acc[4 * w + 1], (unsigned long long)s1);
  atomicAdd(&acc[4 * w + 2], (unsigned long long)s2);
  atomicAdd(&acc[4 * w + 3], (unsigned long long)s3);
  __syncthreads();
  if ((int)threadIdx.x < dp) atomicAdd(&sums[threadIdx.x], acc[threadIdx.x]);
}

// Squared distance to the mean summed over dims in order with a fused
// multiply-add per dim, as the host builder's medoid search evaluates it.
__global__ __launch_bounds__(256) void medoid_kernel(const uint8_t* __restrict__ x, int64_t n, int dim,
                                                     int dp, const float* __restrict__ mean,
                                                     unsigned long long* __restrict__ best) {
  __shared__ float m[256];
  for (int i = threadIdx.x; i < 256; i += blockDim.x) m[i] = i < dim ? mean[i] : 0.0f;
  __syncthreads();
  unsigned long long b = ~0ull;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n;
       r += (int64_t)gridDim.x * blockDim.x) {
    const u32x4* row = reinterpret_cast<const u32x4*>(x + r * dp);
    float s = 0.0f;
    for (int c = 0; c < dp / 16; ++c) {
      const u32x4 v = row[c];
      const uint32_t ws[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int i = 16 * c + t;
        if (i < dim) {
          const float d = m[i] - (float)((ws[t >> 2] >> (8 * (t & 3))) & 0xffu);
          s = fma_f(d, d, s);
        }
      }
    }
    const unsigned long long k = ((unsigned long long)__float_as_uint(s) << 32) | (unsigned long long)r;
    b = k < b ? k : b;
  }
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(b, off, kWave);
    b = o < b ? o : b;
  }
  if (lane_id() == 0) atomicMin(best, b);
}

// splitmix64-seeded xoshiro256** stream per node (the host builder's Rng).
struct DevRng {
  uint64_t s[4];
  __device__ static uint64_t splitmix(uint64_t& x) {
    uint64_t z = (x += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  }
  __device__ DevRng(uint64_t seed, uint64_t stream) {
    uint64_t x = seed * 0x9e3779b97f4a7c15ull ^ (stream + 0x632be59bd9b4e019ull);
    for (int i = 0; i < 4; ++i) s[i] = splitmix(x);
  }
  __device__ static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
  __device__ uint64_t next() {
    const uint64_t r = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return r;
  }
  __device__ uint64_t below(uint64_t n) {
    const double u = (double)(next() >> 11) * (1.0 / 9007199254740992.0);
    return (uint64_t)(u * (double)n) % n;
  }
};

constexpr int kMaxDraws = 1 << 20;  // bound on the rejection loop of one node

__global__ __launch_bounds__(256) void random_graph_kernel(BuildDev g, int init_deg, uint64_t seed) {
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= g.n) return;
  DevRng r(seed, (uint64_t)u + 1);
  uint32_t* out = g.nbr + u * g.C;
  int k = 0;
  for (int draws = 0; k < init_deg && draws < kMaxDraws; ++draws) {
    const uint32_t v = (uint32_t)r.below((uint64_t)g.n);
    if (v == (uint32_t)u) continue;
    bool dup = false;
    for (int j = 0; j < k; ++j) dup |= out[j] == v;
    if (!dup) out[k++] = v;
  }
  g.deg[u] = (uint32_t)k;
}

// ------------------------------------------------------------------ build search

__host__ __device__ inline size_t search_wave_bytes(int L) {
  const size_t b = (size_t)list_capacity(L) * 8 + (size_t)list_scratch_words(L) * 4 + (size_t)kBuildPoolMax * 8;
  return (b + 15) & ~(size_t)15;
}

template <int NC>
__global__ __launch_bounds__(256) void build_search_kernel(BuildDev g, const uint32_t* __restrict__ pts,
                                                           int npts, uint32_t start, int L,
                                                           uint32_t* __restrict__ pool_id,
                                                           float* __restrict__ pool_d,
                                                           int32_t* __restrict__ pool_n,
                                                           int32_t* __restrict__ queue) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  const int lane = lane_id();
  uint8_t* wbase = smem_raw + (size_t)(threadIdx.x >> 6) * search_wave_bytes(L);
  uint64_t* A = reinterpret_cast<uint64_t*>(wbase);
  uint32_t* BM = reinterpret_cast<uint32_t*>(A + list_capacity(L));
  float* td = reinterpret_cast<float*>(BM + list_scratch_words(L));
  int32_t* ti = reinterpret_cast<int32_t*>(td + kBuildPoolMax);
  const int64_t cap = g.n + 2;
  for (;;) {
    int qi = 0;
    if (lane == 0) qi = atomicAdd(queue, 1);
    qi = __builtin_amdgcn_readfirstlane(__shfl(qi, 0, kWave));
    if (qi >= npts) break;
    const uint32_t p = (uint32_t)__builtin_amdgcn_readfirstlane((int)pts[qi]);
    uint32_t w[4 * NC];
    uniform_row<NC>(g.x, g.dp, p, w);
    const int32_t np = __builtin_amdgcn_readfirstlane(g.xn[p]);
    uint32_t u = start;
    float du = sq_dist(np, g.xn[u], row_dot<NC>(w, g.x + (int64_t)u * g.dp));
    int sz = 0, fu = 0;
    TopK top(td, ti, kBuildPoolMax);
    for (int64_t exps = 1;; ++exps) {
      // up to C neighbours (a list in its slack), 64 per list update
      const int deg = __builtin_amdgcn_readfirstlane((int)min(g.deg[u], (uint32_t)g.C));
      int part = 0;
      for (; part + kWave < deg; part += kWave) {
        uint64_t key = ~(uint64_t)0;
        const uint32_t v = g.nbr[(int64_t)u * g.C + part + lane];
        if ((int64_t)v < g.n)
          key = make_key(sq_dist(np, g.xn[v], row_dot<NC>(w, g.x + (int64_t)v * g.dp)), v);
        const ListPlan Pi = list_plan(A, L, key, kWave, sz, fu);
        int lb = list_apply<false>(A, BM, Pi);
        sz = Pi.nsz;
        // the exact first unvisited entry for the next update
        for (fu = sz; lb < sz; lb += kWave) {
          const uint64_t m = ballot64(lb + lane < sz && !entry_visited(A[lb + lane]));
          if (m) {
            fu = lb + (int)__builtin_ctzll(m);
            break;
          }
        }
      }
      const int dl = deg - part;
      uint64_t key = ~(uint64_t)0;  // padding and out-of-range ids sort last and are dropped
      if (lane < dl) {
        const uint32_t v = g.nbr[(int64_t)u * g.C + part + lane];
        if ((int64_t)v < g.n)
          key = make_key(sq_dist(np, g.xn[v], row_dot<NC>(w, g.x + (int64_t)v * g.dp)), v);
      }
      const ListPlan P = list_plan(A, L, key, dl, sz, fu);
      fu = list_apply(A, BM, P);
      sz = P.nsz;
      top.push(du, (int32_t)u);
      if (P.cand < 0 || exps >= cap) break;
      u = entry_id(P.sel);
      du = entry_dist(P.sel);
    }
    top.store(reinterpret_cast<int32_t*>(pool_id), pool_d, qi);
    if (lane == 0) pool_n[qi] = top.found;
    wave_sync();
  }
}

// ------------------------------------------------------------------ RobustPrune

// Per-wave LDS: keys | sorted keys | occlusion | norms | ids (kBuildCandMax
// each) | kept or current list (kOutWords) | candidate rows (stride dp + 16:
// the 16-byte reads of 16 consecutive lanes fall on distinct banks).
constexpr int kOutWords = 128;
static_assert(kOutWords >= kBuildSlackMax && kOutWords >= kWave, "list buffer");
struct PruneSmem {
  static __host__ __device__ size_t row_stride(int dp) { return (size_t)dp + 16; }
  static __host__ __device__ size_t bytes(int dp) {
    const size_t b = (size_t)kBuildCandMax * (8 + 8 + 4 + 4 + 4) + kOutWords * 4 +
                     row_stride(dp) * kBuildCandMax;
    return (b + 15) & ~(size_t)15;
  }
  uint64_t* keys;
  uint64_t* srt;
  float* occl;
  int32_t* cn;
  uint32_t* cid;
  uint32_t* outl;
  uint8_t* rows;
  __device__ explicit PruneSmem(uint8_t* ws) {
    keys = reinterpret_cast<uint64_t*>(ws);
    srt = keys + kBuildCandMax;
    occl = reinterpret_cast<float*>(srt + kBuildCandMax);
    cn = reinterpret_cast<int32_t*>(occl + kBuildCandMax);
    cid = reinterpret_cast<uint32_t*>(cn + kBuildCandMax);
    outl = cid + kBuildCandMax;
    rows = reinterpret_cast<uint8_t*>(outl + kOutWords);
  }
};

// RobustPrune (index_builder.cpp robust_prune, DiskANN's occlusion rule) of
// point p over the nc candidate keys in S.keys (make_key of the exact
// distance to p): sorted by (distance, id), repeated ids and p dropped; the
// closest remaining candidate is kept and every later candidate j gets
// occlusion max(occl_j, d(p, j) / d(kept, j)) (infinity for d = 0); a
// candidate with occlusion above alpha is skipped; at most R are kept.
// Writes the kept list to S.outl and to p's row of the graph; returns its
// length.
template <int NC>
__device__ int prune_wave(const BuildDev& g, uint32_t p, int nc, float alpha, const PruneSmem& S) {
  constexpr int KPL = (kBuildCandMax + kWave - 1) / kWave;
  const int lane = lane_id();
  const int rs = (int)PruneSmem::row_stride(g.dp);
  wave_sync();  // keys written
  // stable rank sort: position = keys below + equal keys at smaller index
  uint64_t mk[KPL];
  int rk[KPL];
#pragma unroll
  for (int t = 0; t < KPL; ++t) {
    const int i = lane + kWave * t;
    mk[t] = i < nc ? S.keys[i] : ~(uint64_t)0;
    rk[t] = 0;
  }
  for (int j = 0; j < nc; ++j) {
    const uint64_t kj = S.keys[j];
#pragma unroll
    for (int t = 0; t < KPL; ++t) {
      const int i = lane + kWave * t;
      rk[t] += (kj < mk[t] || (kj == mk[t] && j < i)) ? 1 : 0;
    }
  }
#pragma unroll
  for (int t = 0; t < KPL; ++t)
    if (lane + kWave * t < nc) S.srt[rk[t]] = mk[t];
  wave_sync();
  // distinct ids other than p, in order (equal ids have equal keys)
  int m = 0;
  for (int b = 0; b < nc; b += kWave) {
    const int i = b + lane;
    const uint64_t e = i < nc ? S.srt[i] : ~(uint64_t)0;
    const bool keep = i < nc && entry_id(e) != p && (i == 0 || S.srt[i - 1] != e);
    const uint64_t mask = ballot64(keep);
    if (keep) S.keys[m + rank_below(mask)] = e;
    m += __popcll(mask);
  }
  wave_sync();
  for (int c = lane; c < m; c += kWave) {
    const uint32_t id = entry_id(S.keys[c]);
    S.cid[c] = id;
    S.cn[c] = g.xn[id];
    S.occl[c] = 0.0f;
  }
  wave_sync();
  for (int t = lane; t < m * NC; t += kWave) {
    const int c = t / NC, ch = t - c * NC;
    *reinterpret_cast<u32x4*>(S.rows + c * rs + ch * 16) =
        *reinterpret_cast<const u32x4*>(g.x + (int64_t)S.cid[c] * g.dp + ch * 16);
  }
  wave_sync();
  int kept = 0;
  for (int i = 0; i < m && kept < g.R; ++i) {
    if (S.occl[i] > alpha) continue;
    if (lane == 0) S.outl[kept] = S.cid[i];
    ++kept;
    u32x4 ri[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) ri[c] = *reinterpret_cast<const u32x4*>(S.rows + i * rs + c * 16);
    const int32_t ni = S.cn[i];
    for (int jb = ((i + 1) / kWave) * kWave; jb < m; jb += kWave) {
      const int j = jb + lane;
      if (j > i && j < m) {
        const float oj = S.occl[j];
        if (!(oj > alpha)) {
          const u32x4* rj = reinterpret_cast<const u32x4*>(S.rows + j * rs);
          uint32_t acc = 0;
#pragma unroll
          for (int c = 0; c < NC; ++c) acc = dot16(ri[c], rj[c], acc);
          const float djk = sq_dist(ni, S.cn[j], acc);
          const float f = djk == 0.0f ? INFINITY : entry_dist(S.keys[j]) / djk;
          if (f > oj) S.occl[j] = f;
        }
      }
    }
    wave_sync();
  }
  wave_sync();
  if (lane < kept) g.nbr[(int64_t)p * g.C + lane] = S.outl[lane];
  if (lane == 0) g.deg[p] = (uint32_t)kept;
  return kept;
}

template <int NC>
__global__ __launch_bounds__(256) void build_prune_fwd_kernel(BuildDev g, const uint32_t* __restrict__ pts,
                                                              int npts, const uint32_t* __restrict__ pool_id,
                                                              const float* __restrict__ pool_d,
                                                              const int32_t* __restrict__ pool_n, float alpha,
                                                              unsigned long long* __restrict__ pairs,
                                                              int32_t* __restrict__ queue) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  const int lane = lane_id();
  const PruneSmem S(smem_raw + (size_t)(threadIdx.x >> 6) * PruneSmem::bytes(g.dp));
  const int R = g.R;
  for (;;) {
    int qi = 0;
    if (lane == 0) qi = atomicAdd(queue, 1);
    qi = __builtin_amdgcn_readfirstlane(__shfl(qi, 0, kWave));
    if (qi >= npts) break;
    const uint32_t p = (uint32_t)__builtin_amdgcn_readfirstlane((int)pts[qi]);
    const int dg = __builtin_amdgcn_readfirstlane((int)min(g.deg[p], (uint32_t)g.C));
    // the pool (sorted by distance) keeps its closest entries when it and
    // the current list exceed the candidate buffer
    const int npool =
        __builtin_amdgcn_readfirstlane(min(min(max(pool_n[qi], 0), kBuildPoolMax), kBuildCandMax - dg));
    for (int j = lane; j < npool; j += kWave)
      S.keys[j] = make_key(pool_d[(int64_t)qi * kBuildPoolMax + j], pool_id[(int64_t)qi * kBuildPoolMax + j]);
    if (dg > 0) {
      uint32_t w[4 * NC];
      uniform_row<NC>(g.x, g.dp, p, w);
      const int32_t np = __builtin_amdgcn_readfirstlane(g.xn[p]);
      for (int j = lane; j < dg; j += kWave) {
        const uint32_t v = g.nbr[(int64_t)p * g.C + j];
        S.keys[npool + j] = make_key(sq_dist(np, g.xn[v], row_dot<NC>(w, g.x + (int64_t)v * g.dp)), v);
      }
    }
    const int kept = prune_wave<NC>(g, p, npool + dg, alpha, S);
    if (lane < R)
      pairs[(int64_t)qi * R + lane] =
          lane < kept ? (((unsigned long long)S.outl[lane] << 32) | p) : ~0ull;
    wave_sync();
  }
}

// ------------------------------------------------------------------ reverse edges

__global__ __launch_bounds__(256) void seg_flags_kernel(const unsigned long long* __restrict__ k, int64_t n,
                                                        uint8_t* __restrict__ flags) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) flags[i] = (i == 0 || (k[i] >> 32) != (k[i - 1] >> 32)) ? 1 : 0;
}

template <int NC>
__global__ __launch_bounds__(256) void build_reverse_kernel(BuildDev g, const unsigned long long* __restrict__ pairs,
                                                            int64_t npairs, const int32_t* __restrict__ seg_start,
                                                            const int32_t* __restrict__ n_seg, float alpha,
                                                            int32_t* __restrict__ queue) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  constexpr int kGrab = 8;  // runs taken per queue access
  const int lane = lane_id();
  const PruneSmem S(smem_raw + (size_t)(threadIdx.x >> 6) * PruneSmem::bytes(g.dp));
  const int ns = __builtin_amdgcn_readfirstlane(*n_seg);
  for (;;) {
    int s0 = 0;
    if (lane == 0) s0 = atomicAdd(queue, kGrab);
    s0 = __builtin_amdgcn_readfirstlane(__shfl(s0, 0, kWave));
    if (s0 >= ns) break;
    for (int s = s0; s < min(s0 + kGrab, ns); ++s) {
      const int64_t a = seg_start[s];
      const int64_t b = s + 1 < ns ? (int64_t)seg_start[s + 1] : npairs;
      const uint32_t v = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(pairs[a] >> 32));
      if ((int64_t)v >= g.n) continue;  // the run of unused slots
      const int dv = __builtin_amdgcn_readfirstlane((int)min(g.deg[v], (uint32_t)g.C));
      // the current list, one entry per lane and register (C <= 2 * 64)
      const uint32_t l0 = lane < dv ? g.nbr[(int64_t)v * g.C + lane] : 0xffffffffu;
      const uint32_t l1 = lane + kWave < dv ? g.nbr[(int64_t)v * g.C + kWave + lane] : 0xffffffffu;
      // new sources: not listed yet, at most kBuildCandMax - dv of them
      const int room = kBuildCandMax - dv;
      int m_new = 0;
      for (int64_t t = a; t < b && m_new < room; t += kWave) {
        const int64_t i = t + lane;
        const uint32_t src = i < b ? (uint32_t)pairs[i] : 0xffffffffu;
        uint64_t cand = ballot64(i < b && src != v && (int64_t)src < g.n);
        uint64_t keep = 0;
        while (cand) {
          const int j = (int)__builtin_ctzll(cand);
          cand &= cand - 1;
          const uint32_t sj = (uint32_t)__builtin_amdgcn_readlane((int)src, j);
          if (!ballot64(l0 == sj || l1 == sj)) keep |= 1ull << j;
        }
        const bool ok = (keep >> lane) & 1;
        const int pos = m_new + rank_below(keep);
        if (ok && pos < room) S.cid[pos] = src;
        m_new = min(m_new + (int)__popcll(keep), room);
      }
      wave_sync();
      if (dv + m_new <= g.C) {
        for (int e = lane; e < m_new; e += kWave) g.nbr[(int64_t)v * g.C + dv + e] = S.cid[e];
        if (lane == 0) g.deg[v] = (uint32_t)(dv + m_new);
      } else {
        uint32_t w[4 * NC];
        uniform_row<NC>(g.x, g.dp, v, w);
        const int32_t nv = __builtin_amdgcn_readfirstlane(g.xn[v]);
        if (lane < dv) S.outl[lane] = l0;
        if (lane + kWave < dv) S.outl[kWave + lane] = l1;
        wave_sync();
        for (int c = lane; c < dv + m_new; c += kWave) {
          const uint32_t id = c < dv ? S.outl[c] : S.cid[c - dv];
          S.keys[c] = make_key(sq_dist(nv, g.xn[id], row_dot<NC>(w, g.x + (int64_t)id * g.dp)), id);
        }
        prune_wave<NC>(g, v, dv + m_new, alpha, S);
      }
      wave_sync();
    }
  }
}

// Lists longer than R pruned back to R, one wavefront per node.
template <int NC>
__global__ __launch_bounds__(256) void build_final_prune_kernel(BuildDev g, float alpha, int32_t* __restrict__ queue) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  const int lane = lane_id();
  const PruneSmem S(smem_raw + (size_t)(threadIdx.x >> 6) * PruneSmem::bytes(g.dp));
  for (;;) {
    int base = 0;
    if (lane == 0) base = atomicAdd(queue, kWave);
    base = __builtin_amdgcn_readfirstlane(__shfl(base, 0, kWave));
    if ((int64_t)base >= g.n) break;
    // the lanes' nodes, then the long lists among them one at a time
    const int64_t mine = (int64_t)base + lane;
    const bool longer = mine < g.n && (int)g.deg[mine] > g.R;
    uint64_t todo = ballot64(longer);
    while (todo) {
      const int l = (int)__builtin_ctzll(todo);
      todo &= todo - 1;
      const uint32_t v = (uint32_t)(base + l);
      const int dv = __builtin_amdgcn_readfirstlane((int)min(g.deg[v], (uint32_t)g.C));
      uint32_t w[4 * NC];
      uniform_row<NC>(g.x, g.dp, v, w);
      const int32_t nv = __builtin_amdgcn_readfirstlane(g.xn[v]);
      for (int c = lane; c < dv; c += kWave) {
        const uint32_t id = g.nbr[(int64_t)v * g.C + c];
        S.keys[c] = make_key(sq_dist(nv, g.xn[id], row_dot<NC>(w, g.x + (int64_t)id * g.dp)), id);
      }
      prune_wave<NC>(g, v, dv, alpha, S);
      wave_sync();
    }
  }
}

// The lists in rows of R entries (out [n][R]) for one contiguous download.
__global__ __launch_bounds__(256) void compact_rows_kernel(const uint32_t* __restrict__ nbr, int64_t n, int C, int R,
                                                           uint32_t* __restrict__ out) {
  const int64_t total = n * R;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x)
    out[i] = nbr[(i / R) * C + i % R];
}

// One RobustPrune of p over explicit candidates (diagnostic entry).
template <int NC>
__global__ __launch_bounds__(64) void prune_one_kernel(BuildDev g, uint32_t p, const uint32_t* __restrict__ cand,
                                                       int ncand, float alpha, uint32_t* __restrict__ out,
                                                       int32_t* __restrict__ nout) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  const int lane = lane_id();
  const PruneSmem S(smem_raw);
  uint32_t w[4 * NC];
  uniform_row<NC>(g.x, g.dp, p, w);
  const int32_t np = __builtin_amdgcn_readfirstlane(g.xn[p]);
  for (int c = lane; c < ncand; c += kWave) {
    const uint32_t id = cand[c];
    S.keys[c] = make_key(sq_dist(np, g.xn[id], row_dot<NC>(w, g.x + (int64_t)id * g.dp)), id);
  }
  const int kept = prune_wave<NC>(g, p, ncand, alpha, S);
  if (lane < kept) out[lane] = S.outl[lane];
  if (lane == 0) *nout = kept;
}

// ------------------------------------------------------------------ PQ encoding

// One thread per point: for every chunk, the first of the 256 pivots with
// the smallest distance, accumulated as fma(t, t, d) over the chunk's dims
// in order with t = (x - centroid) - pivot (index_builder.cpp pq_encode).
// Pivot reads are wave-uniform.
template <typename T>
__global__ __launch_bounds__(256) void pq_encode_kernel(const T* __restrict__ x, int64_t n, int dim,
                                                        const float* __restrict__ pivots,
                                                        const float* __restrict__ centroid,
                                                        const int32_t* __restrict__ off, int M,
                                                        uint8_t* __restrict__ codes) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool ok = i < n;
  const T* row = x + (ok ? i : 0) * dim;
  for (int m = 0; m < M; ++m) {
    const int lo = off[m], w = off[m + 1] - lo;
    float xv[kPqEncodeMaxW];
#pragma unroll
    for (int j = 0; j < kPqEncodeMaxW; ++j) xv[j] = j < w ? (float)row[lo + j] - centroid[lo + j] : 0.0f;
    float bd = INFINITY;
    int bk = 0;
    for (int k = 0; k < kPivots; ++k) {
      const float* pk = pivots + (int64_t)k * dim + lo;
      float d = 0.0f;
#pragma unroll
      for (int j = 0; j < kPqEncodeMaxW; ++j)
        if (j < w) {
          const float t = xv[j] - pk[j];
          d = fma_f(t, t, d);
        }
      if (d < bd) {
        bd = d;
        bk = k;
      }
    }
    if (ok) codes[i * M + m] = (uint8_t)bk;
  }
}

template <class F>
hipError_t with_nc(int dp, F&& f) {
  switch (dp) {
    case 32: return f(std::integral_constant<int, 2>{});
    case 64: return f(std::integral_constant<int, 4>{});
    case 96: return f(std::integral_constant<int, 6>{});
    case 128: return f(std::integral_constant<int, 8>{});
    case 192: return f(std::integral_constant<int, 12>{});
    case 256: return f(std::integral_constant<int, 16>{});
    default: return hipErrorInvalidValue;
  }
}

unsigned grid_for(int64_t n, int block) { return (unsigned)std::max<int64_t>(1, (n + block - 1) / block); }

}  // namespace

int build_row_bytes(int dim) {
  if (dim < 1) return 0;
  if (dim <= 32) return 32;
  if (dim <= 64) return 64;
  if (dim <= 96) return 96;
  if (dim <= 128) return 128;
  if (dim <= 192) return 192;
  if (dim <= 256) return 256;
  return 0;
}

hipError_t launch_build_norms(const uint8_t* x, int64_t n, int dp, int32_t* xn, hipStream_t stream) {
  hipLaunchKernelGGL(norms_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, x, n, dp, xn);
  return hipGetLastError();
}

hipError_t launch_build_col_sums(const uint8_t* x, int64_t n, int dp, unsigned long long* sums,
                                 hipStream_t stream) {
  if (dp % 4 != 0 || dp > 256) return hipErrorInvalidValue;
  const int rpb = 256 / (dp / 4);
  const unsigned grid = (unsigned)std::min<int64_t>(4096, std::max<int64_t>(1, (n + rpb - 1) / rpb));
  hipLaunchKernelGGL(col_sums_kernel, dim3(grid), dim3(256), 0, stream, x, n, dp, sums);
  return hipGetLastError();
}

hipError_t launch_build_medoid(const uint8_t* x, int64_t n, int dim, int dp, const float* mean,
                               unsigned long long* best, hipStream_t stream) {
  if (dim > 256 || dp > 256) return hipErrorInvalidValue;
  const unsigned grid = (unsigned)std::min<int64_t>(8192, grid_for(n, 256));
  hipLaunchKernelGGL(medoid_kernel, dim3(grid), dim3(256), 0, stream, x, n, dim, dp, mean, best);
  return hipGetLastError();
}

hipError_t launch_build_random_graph(BuildDev g, int init_deg, uint64_t seed, hipStream_t stream) {
  if (init_deg > g.R || g.C < g.R) return hipErrorInvalidValue;
  hipLaunchKernelGGL(random_graph_kernel, dim3(grid_for(g.n, 256)), dim3(256), 0, stream, g, init_deg, seed);
  return hipGetLastError();
}

size_t build_search_smem_bytes(int L, int waves) { return search_wave_bytes(L) * (size_t)waves; }

hipError_t launch_build_search(BuildDev g, const uint32_t* pts, int npts, uint32_t start, int L,
                               uint32_t* pool_id, float* pool_d, int32_t* pool_n, int32_t* queue, int cus,
                               hipStream_t stream) {
  if (g.R < 1 || g.R > kWave || g.C < g.R || g.C > kBuildSlackMax || L < 1) return hipErrorInvalidValue;
  const size_t smem = build_search_smem_bytes(L, 4);
  const unsigned grid = (unsigned)std::max(1, std::min(8 * cus, (npts + 3) / 4));
  return with_nc(g.dp, [&](auto nc) {
    hipLaunchKernelGGL(build_search_kernel<decltype(nc)::value>, dim3(grid), dim3(256), smem, stream, g, pts,
                       npts, start, L, pool_id, pool_d, pool_n, queue);
    return hipGetLastError();
  });
}

int build_prune_waves(int dp, size_t lds_limit) {
  const size_t b = PruneSmem::bytes(dp);
  return (int)std::min<size_t>(4, lds_limit / b);
}

hipError_t launch_build_prune_fwd(BuildDev g, const uint32_t* pts, int npts, const uint32_t* pool_id,
                                  const float* pool_d, const int32_t* pool_n, float alpha,
                                  unsigned long long* pairs, int32_t* queue, int cus, size_t lds_limit,
                                  hipStream_t stream) {
  if (g.R < 1 || g.R > kWave || g.C < g.R || g.C > kBuildSlackMax) return hipErrorInvalidValue;
  const int waves = build_prune_waves(g.dp, lds_limit);
  if (waves < 1) return hipErrorInvalidValue;
  const size_t smem = PruneSmem::bytes(g.dp) * (size_t)waves;
  const unsigned grid = (unsigned)std::max(1, std::min(2 * cus, (npts + waves - 1) / waves));
  return with_nc(g.dp, [&](auto nc) {
    hipLaunchKernelGGL(build_prune_fwd_kernel<decltype(nc)::value>, dim3(grid), dim3(64 * waves), smem, stream,
                       g, pts, npts, pool_id, pool_d, pool_n, alpha, pairs, queue);
    return hipGetLastError();
  });
}

hipError_t build_segments_temp_bytes(int64_t npairs, size_t* bytes) {
  if (npairs < 1 || npairs > INT32_MAX) return hipErrorInvalidValue;
  size_t a = 0, b = 0;
  hipError_t e = hipcub::DeviceRadixSort::SortKeys(nullptr, a, (const unsigned long long*)nullptr,
                                                   (unsigned long long*)nullptr, (int)npairs, 0, 64);
  if (e != hipSuccess) return e;
  e = hipcub::DeviceSelect::Flagged(nullptr, b, hipcub::CountingInputIterator<int32_t>(0), (const uint8_t*)nullptr,
                                    (int32_t*)nullptr, (int32_t*)nullptr, (int)npairs);
  *bytes = std::max(a, b);
  return e;
}

hipError_t launch_build_segments(void* temp, size_t temp_bytes, const unsigned long long* pairs_in,
                                 unsigned long long* pairs_out, int64_t npairs, uint8_t* flags,
                                 int32_t* seg_start, int32_t* n_seg, hipStream_t stream) {
  if (npairs < 1 || npairs > INT32_MAX) return hipErrorInvalidValue;
  size_t tb = temp_bytes;
  hipError_t e = hipcub::DeviceRadixSort::SortKeys(temp, tb, pairs_in, pairs_out, (int)npairs, 0, 64, stream);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(seg_flags_kernel, dim3(grid_for(npairs, 256)), dim3(256), 0, stream, pairs_out, npairs, flags);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  tb = temp_bytes;
  return hipcub::DeviceSelect::Flagged(temp, tb, hipcub::CountingInputIterator<int32_t>(0), flags, seg_start,
                                       n_seg, (int)npairs, stream);
}

hipError_t launch_build_reverse(BuildDev g, const unsigned long long* pairs, int64_t npairs,
                                const int32_t* seg_start, const int32_t* n_seg, float alpha, int32_t* queue,
                                int cus, size_t lds_limit, hipStream_t stream) {
  if (g.R < 1 || g.R > kWave || g.C < g.R || g.C > kBuildSlackMax) return hipErrorInvalidValue;
  const int waves = build_prune_waves(g.dp, lds_limit);
  if (waves < 1) return hipErrorInvalidValue;
  const size_t smem = PruneSmem::bytes(g.dp) * (size_t)waves;
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(2 * cus, (npairs + waves - 1) / waves));
  return with_nc(g.dp, [&](auto nc) {
    hipLaunchKernelGGL(build_reverse_kernel<decltype(nc)::value>, dim3(grid), dim3(64 * waves), smem, stream, g,
                       pairs, npairs, seg_start, n_seg, alpha, queue);
    return hipGetLastError();
  });
}

hipError_t launch_pq_encode(const void* x, int dtype, int64_t n, int dim, const float* pivots,
                            const float* centroid, const int32_t* chunk_off, int M, uint8_t* codes,
                            hipStream_t stream) {
  if (n < 1) return hipSuccess;
  const dim3 grid(grid_for(n, 256));
  if (dtype == 0)
    hipLaunchKernelGGL(pq_encode_kernel<uint8_t>, grid, dim3(256), 0, stream, (const uint8_t*)x, n, dim, pivots,
                       centroid, chunk_off, M, codes);
  else
    hipLaunchKernelGGL(pq_encode_kernel<float>, grid, dim3(256), 0, stream, (const float*)x, n, dim, pivots,
                       centroid, chunk_off, M, codes);
  return hipGetLastError();
}

hipError_t launch_build_final_prune(BuildDev g, float alpha, int32_t* queue, int cus, size_t lds_limit,
                                    hipStream_t stream) {
  if (g.R < 1 || g.R > kWave || g.C < g.R || g.C > kBuildSlackMax) return hipErrorInvalidValue;
  const int waves = build_prune_waves(g.dp, lds_limit);
  if (waves < 1) return hipErrorInvalidValue;
  const size_t smem = PruneSmem::bytes(g.dp) * (size_t)waves;
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(2 * cus, (g.n + 63) / 64));
  return with_nc(g.dp, [&](auto nc) {
    hipLaunchKernelGGL(build_final_prune_kernel<decltype(nc)::value>, dim3(grid), dim3(64 * waves), smem, stream,
                       g, alpha, queue);
    return hipGetLastError();
  });
}

hipError_t launch_build_compact(BuildDev g, uint32_t* out, hipStream_t stream) {
  const unsigned grid = (unsigned)std::min<int64_t>(16384, grid_for(g.n * g.R, 256));
  hipLaunchKernelGGL(compact_rows_kernel, dim3(grid), dim3(256), 0, stream, g.nbr, g.n, g.C, g.R, out);
  return hipGetLastError();
}

hipError_t launch_build_prune_one(BuildDev g, uint32_t p, const uint32_t* cand, int ncand, float alpha,
                                  uint32_t* out, int32_t* nout, size_t lds_limit, hipStream_t stream) {
  if (ncand < 0 || ncand > kBuildCandMax || g.R < 1 || g.R > kWave || g.C < g.R) return hipErrorInvalidValue;
  if (PruneSmem::bytes(g.dp) > lds_limit) return hipErrorInvalidValue;
  return with_nc(g.dp, [&](auto nc) {
    hipLaunchKernelGGL(prune_one_kernel<decltype(nc)::value>, dim3(1), dim3(64), PruneSmem::bytes(g.dp), stream, g,
                       p, cand, ncand, alpha, out, nout);
    return hipGetLastError();
  });
}

}  // namespace gann

// Index builder and synthetic-data generator (host C++17 + OpenMP).
//
// The reference builds its indexes with the external DiskANN tools
// (scripts/build_diskann_index.sh:7, scripts/gen_pivot_graph.sh:12-14), which
// are absent here.  This library produces the same file formats from its own
// implementation:
//   * seeded Gaussian-mixture data (uint8 clipped, or float L2-normalised),
//   * a Vamana graph (greedy search + RobustPrune with alpha, two passes),
//   * a product quantizer (mean-centred, contiguous chunks, 256-way k-means),
//   * the pivot ("nav") graph: a sampled subset (bin/gen_small_file.cpp:18-25:
//     mt19937(114514), shuffle, keep n, sort) with its own small Vamana graph,
//   * exact brute-force ground truth (ties broken by the smaller id).
// Everything is exported with a C ABI (prefix gib_) for the Python package.
#include <omp.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <numeric>
#include <random>
#include <string>
#include <vector>

#include "formats.hpp"

namespace {

thread_local std::string g_err;
// Progress lines on stderr during long graph builds (gib_set_verbose).
std::atomic<int> g_verbose{0};

// ------------------------------------------------------------------ RNG
// splitmix64 seeding + xoshiro256**; Box-Muller normals.  Streams are
// derived per item so results do not depend on the thread count.
struct Rng {
  uint64_t s[4];
  static uint64_t splitmix(uint64_t& x) {
    uint64_t z = (x += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  }
  Rng(uint64_t seed, uint64_t stream) {
    uint64_t x = seed * 0x9e3779b97f4a7c15ull ^ (stream + 0x632be59bd9b4e019ull);
    for (auto& v : s) v = splitmix(x);
  }
  static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
  uint64_t next() {
    uint64_t r = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return r;
  }
  double uniform() { return (next() >> 11) * (1.0 / 9007199254740992.0); }  // [0,1)
  uint64_t below(uint64_t n) { return (uint64_t)(uniform() * (double)n) % n; }
  double normal() {
    double u1 = uniform(), u2 = uniform();
    if (u1 < 1e-300) u1 = 1e-300;
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
  }
};

// ------------------------------------------------------------------ distances
inline float l2_u8(const uint8_t* a, const uint8_t* b, int64_t d) {
  int32_t s = 0;
  for (int64_t i = 0; i < d; ++i) {
    int32_t t = (int32_t)a[i] - (int32_t)b[i];
    s += t * t;
  }
  return (float)s;
}
inline float l2_f32(const float* a, const float* b, int64_t d) {
  float s = 0.f;
  for (int64_t i = 0; i < d; ++i) {
    float t = a[i] - b[i];
    s += t * t;
  }
  return s;
}

struct Points {
  const void* data;
  int64_t n, dim;
  int dtype;  // 0 u8, 1 f32
  float dist(int64_t a, int64_t b) const {
    if (dtype == 0) {
      const uint8_t* p = (const uint8_t*)data;
      return l2_u8(p + a * dim, p + b * dim, dim);
    }
    const float* p = (const float*)data;
    return l2_f32(p + a * dim, p + b * dim, dim);
  }
  float dist_to(const float* q, int64_t b) const {
    float s = 0.f;
    if (dtype == 0) {
      const uint8_t* p = (const uint8_t*)data + b * dim;
      for (int64_t i = 0; i < dim; ++i) {
        float t = q[i] - (float)p[i];
        s += t * t;
      }
    } else {
      const float* p = (const float*)data + b * dim;
      for (int64_t i = 0; i < dim; ++i) {
        float t = q[i] - p[i];
        s += t * t;
      }
    }
    return s;
  }
};

// ------------------------------------------------------------------ Vamana
struct Cand {
  float d;
  uint32_t id;
  bool operator<(const Cand& o) const { return d < o.d || (d == o.d && id < o.id); }
};

// Adjacency with slack: a list may grow to C = ceil(1.3 R) entries through
// reverse edges before it is pruned back to R (DiskANN's graph slack), so
// that most reverse insertions do not trigger a prune.
struct Graph {
  int64_t n, R, C;
  std::vector<uint32_t> nbr;  // [n][C]
  std::vector<uint32_t> deg;  // [n]
  std::vector<std::mutex> locks;
  Graph(int64_t n_, int64_t R_)
      : n(n_), R(R_), C((R_ * 13 + 9) / 10), nbr((size_t)(n_ * ((R_ * 13 + 9) / 10))),
        deg((size_t)n_, 0), locks((size_t)n_) {}
  uint32_t* row(int64_t u) { return nbr.data() + u * C; }
  const uint32_t* row(int64_t u) const { return nbr.data() + u * C; }
};

// Greedy best-first search with a sorted list of size L; `pool` receives the
// expanded nodes (DiskANN's visited set used as pruning candidates).
struct Searcher {
  std::vector<uint32_t> tag;
  uint32_t epoch = 0;
  std::vector<Cand> list, pool;
  std::vector<uint32_t> snapshot;
  explicit Searcher(int64_t n) : tag((size_t)n, 0) {}

  void search(const Points& P, const Graph& G, int64_t q, uint32_t start, int64_t L) {
    if (++epoch == 0) {
      std::fill(tag.begin(), tag.end(), 0);
      epoch = 1;
    }
    list.clear();
    pool.clear();
    std::vector<uint8_t> expanded;
    auto push = [&](uint32_t v) {
      if (tag[v] == epoch) return;
      tag[v] = epoch;
      Cand c{P.dist(q, v), v};
      if ((int64_t)list.size() == L && !(c < list.back())) return;
      auto it = std::lower_bound(list.begin(), list.end(), c);
      size_t pos = (size_t)(it - list.begin());
      list.insert(it, c);
      expanded.insert(expanded.begin() + (long)pos, 0);
      if ((int64_t)list.size() > L) {
        list.pop_back();
        expanded.pop_back();
      }
    };
    push(start);
    size_t i = 0;
    while (i < list.size()) {
      if (expanded[i]) {
        ++i;
        continue;
      }
      expanded[i] = 1;
      uint32_t u = list[i].id;
      pool.push_back(list[i]);
      {
        std::lock_guard<std::mutex> g(const_cast<Graph&>(G).locks[u]);
        snapshot.assign(G.row(u), G.row(u) + G.deg[u]);
      }
      size_t before = i;
      for (uint32_t v : snapshot) push(v);
      // restart from the first unexpanded entry (insertions may land before i)
      i = 0;
      while (i < list.size() && expanded[i]) ++i;
      (void)before;
    }
  }
};

// RobustPrune (DiskANN): keep the closest candidate, drop every candidate it
// alpha-dominates, repeat until R are kept.
void robust_prune(const Points& P, int64_t p, std::vector<Cand>& cand, float alpha, int64_t R,
                  std::vector<uint32_t>& out) {
  constexpr size_t kMaxCand = 750;  // DiskANN's maxc
  std::sort(cand.begin(), cand.end());
  cand.erase(std::unique(cand.begin(), cand.end(),
                         [](const Cand& a, const Cand& b) { return a.id == b.id; }),
             cand.end());
  if (cand.size() > kMaxCand) cand.resize(kMaxCand);
  out.clear();
  std::vector<float> occl(cand.size(), 0.f);
  for (size_t i = 0; i < cand.size() && (int64_t)out.size() < R; ++i) {
    if (cand[i].id == (uint32_t)p || occl[i] > alpha) continue;
    out.push_back(cand[i].id);
    for (size_t j = i + 1; j < cand.size(); ++j) {
      if (occl[j] > alpha) continue;
      float djk = P.dist(cand[i].id, cand[j].id);
      float f = djk == 0.f ? INFINITY : cand[j].d / djk;
      if (f > occl[j]) occl[j] = f;
    }
  }
}

int64_t find_medoid(const Points& P, int nthreads) {
  std::vector<double> mean((size_t)P.dim, 0.0);
  for (int64_t i = 0; i < P.n; ++i)
    for (int64_t j = 0; j < P.dim; ++j)
      mean[(size_t)j] += P.dtype == 0 ? ((const uint8_t*)P.data)[i * P.dim + j]
                                      : ((const float*)P.data)[i * P.dim + j];
  std::vector<float> m((size_t)P.dim);
  for (int64_t j = 0; j < P.dim; ++j) m[(size_t)j] = (float)(mean[(size_t)j] / (double)P.n);
  int64_t best = 0;
  float bd = INFINITY;
#pragma omp parallel num_threads(nthreads)
  {
    int64_t lb = 0;
    float ld = INFINITY;
#pragma omp for schedule(static)
    for (int64_t i = 0; i < P.n; ++i) {
      float d = P.dist_to(m.data(), i);
      if (d < ld || (d == ld && i < lb)) {
        ld = d;
        lb = i;
      }
    }
#pragma omp critical
    if (ld < bd || (ld == bd && lb < best)) {
      bd = ld;
      best = lb;
    }
  }
  return best;
}

void vamana(const Points& P, int64_t R, int64_t L, float alpha, uint64_t seed, int nthreads,
            Graph& G, int64_t medoid) {
  const int64_t n = P.n;
  // random initial graph with R/2 out-edges per node (no self loops, no duplicates)
  int64_t init_deg = std::min<int64_t>(R / 2 > 0 ? R / 2 : 1, n - 1);
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int64_t u = 0; u < n; ++u) {
    Rng r(seed, (uint64_t)u + 1);
    uint32_t* out = G.row(u);
    int64_t k = 0;
    while (k < init_deg) {
      uint32_t v = (uint32_t)r.below((uint64_t)n);
      if (v == (uint32_t)u) continue;
      bool dup = false;
      for (int64_t j = 0; j < k; ++j) dup |= out[j] == v;
      if (!dup) out[k++] = v;
    }
    G.deg[(size_t)u] = (uint32_t)k;
  }
  std::vector<uint32_t> order((size_t)n);
  std::iota(order.begin(), order.end(), 0u);
  {
    std::mt19937_64 g(seed ^ 0x5eedull);
    std::shuffle(order.begin(), order.end(), g);
  }
  auto prune_row = [&](int64_t v, float a, std::vector<uint32_t>& vp) {
    std::vector<Cand> vc;
    {
      std::lock_guard<std::mutex> g(G.locks[(size_t)v]);
      const uint32_t* vn = G.row(v);
      for (uint32_t j = 0; j < G.deg[(size_t)v]; ++j) vc.push_back(Cand{P.dist(v, vn[j]), vn[j]});
    }
    robust_prune(P, v, vc, a, R, vp);
    std::lock_guard<std::mutex> g(G.locks[(size_t)v]);
    std::copy(vp.begin(), vp.end(), G.row(v));
    G.deg[(size_t)v] = (uint32_t)vp.size();
  };
  const float alphas[2] = {1.0f, alpha};
  for (float a : alphas) {
#pragma omp parallel num_threads(nthreads)
    {
      Searcher S(n);
      std::vector<Cand> cand;
      std::vector<uint32_t> pruned, vp;
#pragma omp for schedule(dynamic, 64)
      for (int64_t oi = 0; oi < n; ++oi) {
        if (g_verbose.load(std::memory_order_relaxed) && n >= 1000000 && oi % (n / 20) == 0)
          std::fprintf(stderr, "[vamana] alpha %.2f: %lld / %lld\n", (double)a, (long long)oi,
                       (long long)n);
        int64_t p = order[(size_t)oi];
        S.search(P, G, p, (uint32_t)medoid, L);
        cand = S.pool;
        {
          std::lock_guard<std::mutex> g(G.locks[(size_t)p]);
          const uint32_t* pn = G.row(p);
          for (uint32_t j = 0; j < G.deg[(size_t)p]; ++j) cand.push_back(Cand{P.dist(p, pn[j]), pn[j]});
        }
        robust_prune(P, p, cand, a, R, pruned);
        {
          std::lock_guard<std::mutex> g(G.locks[(size_t)p]);
          std::copy(pruned.begin(), pruned.end(), G.row(p));
          G.deg[(size_t)p] = (uint32_t)pruned.size();
        }
        // reverse edges; a list that overflows its slack is pruned back to R
        for (uint32_t v : pruned) {
          bool need_prune = false;
          {
            std::lock_guard<std::mutex> g(G.locks[v]);
            uint32_t* vn = G.row(v);
            uint32_t dv = G.deg[v];
            bool present = false;
            for (uint32_t j = 0; j < dv; ++j) present |= vn[j] == (uint32_t)p;
            if (!present) {
              if ((int64_t)dv < G.C) {
                vn[dv] = (uint32_t)p;
                G.deg[v] = ++dv;
              }
              need_prune = (int64_t)dv >= G.C;
            }
          }
          if (need_prune) prune_row(v, a, vp);
        }
      }
    }
  }
  // final pass: every list back to at most R
#pragma omp parallel num_threads(nthreads)
  {
    std::vector<uint32_t> vp;
#pragma omp for schedule(dynamic, 256)
    for (int64_t v = 0; v < n; ++v)
      if ((int64_t)G.deg[(size_t)v] > R) prune_row(v, alpha, vp);
  }
}

// ------------------------------------------------------------------ PQ
void pq_train(const Points& P, int M, int64_t sample, int iters, uint64_t seed, int nthreads,
              gann::PQHost& pq) {
  const int64_t D = P.dim;
  pq.dim = (int)D;
  pq.num_chunks = M;
  pq.chunk_offsets.resize((size_t)M + 1);
  // contiguous chunks, sizes differ by at most one (earlier chunks larger)
  for (int m = 0; m <= M; ++m) pq.chunk_offsets[(size_t)m] = (int32_t)((D * m) / M);
  auto val = [&](int64_t i, int64_t j) -> float {
    return P.dtype == 0 ? (float)((const uint8_t*)P.data)[i * D + j] : ((const float*)P.data)[i * D + j];
  };
  // centroid = mean of all points (uint8: exact integer sums, so the
  // threads' partial sums give the same double as a sequential pass)
  pq.centroid.assign((size_t)D, 0.f);
  {
    std::vector<double> acc((size_t)D, 0.0);
    if (P.dtype == 0) {
      std::vector<int64_t> tot((size_t)D, 0);
#pragma omp parallel num_threads(nthreads)
      {
        std::vector<int64_t> part((size_t)D, 0);
        const uint8_t* x = (const uint8_t*)P.data;
#pragma omp for schedule(static)
        for (int64_t i = 0; i < P.n; ++i)
          for (int64_t j = 0; j < D; ++j) part[(size_t)j] += x[i * D + j];
#pragma omp critical
        for (int64_t j = 0; j < D; ++j) tot[(size_t)j] += part[(size_t)j];
      }
      for (int64_t j = 0; j < D; ++j) acc[(size_t)j] = (double)tot[(size_t)j];
    } else {
      for (int64_t i = 0; i < P.n; ++i)
        for (int64_t j = 0; j < D; ++j) acc[(size_t)j] += val(i, j);
    }
    for (int64_t j = 0; j < D; ++j) pq.centroid[(size_t)j] = (float)(acc[(size_t)j] / (double)P.n);
  }
  // training sample
  int64_t ns = std::min<int64_t>(sample, P.n);
  std::vector<int64_t> ids((size_t)P.n);
  std::iota(ids.begin(), ids.end(), 0);
  {
    std::mt19937_64 g(seed);
    for (int64_t i = 0; i < ns; ++i) {
      int64_t j = i + (int64_t)(g() % (uint64_t)(P.n - i));
      std::swap(ids[(size_t)i], ids[(size_t)j]);
    }
  }
  pq.pivots.assign((size_t)(256 * D), 0.f);
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
  for (int m = 0; m < M; ++m) {
    int64_t lo = pq.chunk_offsets[(size_t)m], hi = pq.chunk_offsets[(size_t)m + 1], w = hi - lo;
    if (w == 0) continue;
    std::vector<float> X((size_t)(ns * w));
    for (int64_t i = 0; i < ns; ++i)
      for (int64_t j = 0; j < w; ++j)
        X[(size_t)(i * w + j)] = val(ids[(size_t)i], lo + j) - pq.centroid[(size_t)(lo + j)];
    std::vector<float> C((size_t)(256 * w));
    Rng r(seed, 1000 + (uint64_t)m);
    for (int k = 0; k < 256; ++k) {
      int64_t s = (int64_t)r.below((uint64_t)ns);
      for (int64_t j = 0; j < w; ++j) C[(size_t)(k * w + j)] = X[(size_t)(s * w + j)];
    }
    std::vector<int> asg((size_t)ns);
    std::vector<double> sum((size_t)(256 * w));
    std::vector<int64_t> cnt(256);
    for (int it = 0; it < iters; ++it) {
      for (int64_t i = 0; i < ns; ++i) {
        float bd = INFINITY;
        int bk = 0;
        for (int k = 0; k < 256; ++k) {
          float d = 0.f;
          for (int64_t j = 0; j < w; ++j) {
            float t = X[(size_t)(i * w + j)] - C[(size_t)(k * w + j)];
            d += t * t;
          }
          if (d < bd) {
            bd = d;
            bk = k;
          }
        }
        asg[(size_t)i] = bk;
      }
      std::fill(sum.begin(), sum.end(), 0.0);
      std::fill(cnt.begin(), cnt.end(), 0);
      for (int64_t i = 0; i < ns; ++i) {
        int k = asg[(size_t)i];
        ++cnt[(size_t)k];
        for (int64_t j = 0; j < w; ++j) sum[(size_t)(k * w + j)] += X[(size_t)(i * w + j)];
      }
      for (int k = 0; k < 256; ++k) {
        if (cnt[(size_t)k] == 0) {  // re-seed an empty cluster
          int64_t s = (int64_t)r.below((uint64_t)ns);
          for (int64_t j = 0; j < w; ++j) C[(size_t)(k * w + j)] = X[(size_t)(s * w + j)];
          continue;
        }
        for (int64_t j = 0; j < w; ++j)
          C[(size_t)(k * w + j)] = (float)(sum[(size_t)(k * w + j)] / (double)cnt[(size_t)k]);
      }
    }
    for (int k = 0; k < 256; ++k)
      for (int64_t j = 0; j < w; ++j) pq.pivots[(size_t)(k * D + lo + j)] = C[(size_t)(k * w + j)];
  }
}

// Code of each chunk: the first pivot with the smallest distance, the
// distance accumulated as fma(t, t, d) over the chunk's dims in order with
// t = (x - centroid) - pivot, the operations of the search's LUT entry.
void pq_encode(const Points& P, int nthreads, gann::PQHost& pq) {
  const int64_t D = P.dim;
  const int M = pq.num_chunks;
  pq.num_pts = P.n;
  pq.codes.assign((size_t)(P.n * M), 0);
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int64_t i = 0; i < P.n; ++i) {
    for (int m = 0; m < M; ++m) {
      int64_t lo = pq.chunk_offsets[(size_t)m], hi = pq.chunk_offsets[(size_t)m + 1];
      float bd = INFINITY;
      int bk = 0;
      for (int k = 0; k < 256; ++k) {
        float d = 0.f;
        for (int64_t j = lo; j < hi; ++j) {
          float x = (P.dtype == 0 ? (float)((const uint8_t*)P.data)[i * D + j]
                                  : ((const float*)P.data)[i * D + j]) -
                    pq.centroid[(size_t)j];
          float t = x - pq.pivots[(size_t)(k * D + j)];
          d = std::fma(t, t, d);
        }
        if (d < bd) {
          bd = d;
          bk = k;
        }
      }
      pq.codes[(size_t)(i * M + m)] = (uint8_t)bk;
    }
  }
}

}  // namespace

extern "C" {

const char* gib_last_error(void) { return g_err.c_str(); }

void gib_set_verbose(int on) { g_verbose.store(on ? 1 : 0); }

// Gaussian mixture, uint8: centres ~ U[lo, hi]^dim (from centre_seed),
// point = round(centre + N(0, sigma^2)) clipped to [0, 255] (from
// point_seed; base points and queries share centres, not noise).
// cluster_of (nullable, [n]) selects each point's cluster; NULL draws it
// uniformly.  Point i uses stream i, so the output is independent of the
// thread count.
int gib_gen_mixture_u8(int64_t n, int64_t dim, int64_t nclusters, uint64_t centre_seed,
                       uint64_t point_seed, double lo, double hi, double sigma,
                       const int32_t* cluster_of, uint8_t* out, int32_t* cluster_out,
                       int nthreads) {
  std::vector<float> centres((size_t)(nclusters * dim));
  {
    Rng r(centre_seed, 0);
    for (auto& c : centres) c = (float)(lo + (hi - lo) * r.uniform());
  }
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    Rng r(point_seed ^ 0xa5a5a5a5a5a5a5a5ull, (uint64_t)i + 1);
    int64_t c = cluster_of ? cluster_of[i] : (int64_t)r.below((uint64_t)nclusters);
    if (cluster_out) cluster_out[i] = (int32_t)c;
    for (int64_t j = 0; j < dim; ++j) {
      double v = std::nearbyint((double)centres[(size_t)(c * dim + j)] + sigma * r.normal());
      out[i * dim + j] = (uint8_t)std::min(255.0, std::max(0.0, v));
    }
  }
  return 0;
}

// Gaussian mixture, float, L2-normalised: centres ~ N(0,1)^dim normalised
// (from centre_seed), point = normalise(centre + N(0, sigma^2)) (from point_seed).
int gib_gen_mixture_f32(int64_t n, int64_t dim, int64_t nclusters, uint64_t centre_seed,
                        uint64_t point_seed, double sigma, const int32_t* cluster_of, float* out,
                        int32_t* cluster_out, int nthreads) {
  std::vector<double> centres((size_t)(nclusters * dim));
  {
    Rng r(centre_seed, 0);
    for (int64_t c = 0; c < nclusters; ++c) {
      double s = 0;
      for (int64_t j = 0; j < dim; ++j) {
        double v = r.normal();
        centres[(size_t)(c * dim + j)] = v;
        s += v * v;
      }
      s = std::sqrt(s);
      for (int64_t j = 0; j < dim; ++j) centres[(size_t)(c * dim + j)] /= s;
    }
  }
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    Rng r(point_seed ^ 0xa5a5a5a5a5a5a5a5ull, (uint64_t)i + 1);
    int64_t c = cluster_of ? cluster_of[i] : (int64_t)r.below((uint64_t)nclusters);
    if (cluster_out) cluster_out[i] = (int32_t)c;
    std::vector<double> v((size_t)dim);
    double s = 0;
    for (int64_t j = 0; j < dim; ++j) {
      v[(size_t)j] = centres[(size_t)(c * dim + j)] + sigma * r.normal();
      s += v[(size_t)j] * v[(size_t)j];
    }
    s = std::sqrt(s);
    for (int64_t j = 0; j < dim; ++j) out[i * dim + j] = (float)(v[(size_t)j] / s);
  }
  return 0;
}

// Zipf(s) cluster ids in [0, nclusters) by rejection-inversion (Hoermann and
// Derflinger, ACM TOMACS 6.3, 1996), the method of bin/zipf.hpp; rank 1 maps
// to cluster 0.
int gib_zipf_clusters(int64_t n, int64_t nclusters, double s, uint64_t seed, int32_t* out) {
  if (s <= 0 || nclusters < 1) {
    g_err = "zipf: need s > 0 and nclusters >= 1";
    return 1;
  }
  auto H = [s](double x) { return std::fabs(1.0 - s) < 1e-8 ? std::log(x) : (std::pow(x, 1.0 - s) - 1.0) / (1.0 - s); };
  auto Hinv = [s](double x) { return std::fabs(1.0 - s) < 1e-8 ? std::exp(x) : std::pow(1.0 + x * (1.0 - s), 1.0 / (1.0 - s)); };
  auto h = [s](double x) { return std::pow(x, -s); };
  const double Hx1 = H(1.5) - h(1.0), Hn = H((double)nclusters + 0.5);
  const double cut = 1.0 - Hinv(H(1.5) - h(1.0));
  Rng r(seed, 7);
  for (int64_t i = 0; i < n; ++i) {
    for (;;) {
      double u = Hx1 + (Hn - Hx1) * r.uniform();
      double x = Hinv(u);
      double k = std::nearbyint(x);
      if (k < 1) k = 1;
      if (k > (double)nclusters) k = (double)nclusters;
      if (k - x <= cut || u >= H(k + 0.5) - h(k)) {
        out[i] = (int32_t)k - 1;
        break;
      }
    }
  }
  return 0;
}

// Vamana graph; out_nbr [n][R] (first out_deg[i] valid), *out_medoid.
int gib_vamana(const void* data, int64_t n, int64_t dim, int dtype, int64_t R, int64_t L,
               float alpha, uint64_t seed, int nthreads, uint32_t* out_nbr, uint32_t* out_deg,
               int64_t* out_medoid) {
  if (n < 2 || R < 1 || L < 1) {
    g_err = "vamana: need n >= 2, R >= 1, L >= 1";
    return 1;
  }
  Points P{data, n, dim, dtype};
  int64_t med = find_medoid(P, nthreads);
  Graph G(n, R);
  vamana(P, R, L, alpha, seed, nthreads, G, med);
  for (int64_t u = 0; u < n; ++u) {
    std::memcpy(out_nbr + u * R, G.row(u), sizeof(uint32_t) * (size_t)G.deg[(size_t)u]);
    out_deg[u] = G.deg[(size_t)u];
  }
  *out_medoid = med;
  return 0;
}

// Product quantizer training + encoding.  pivots [256][dim], centroid [dim],
// chunk_offsets [M+1], codes [n][M].
// Product quantizer training only (pivots, centroid, chunk offsets).
int gib_pq_train(const void* data, int64_t n, int64_t dim, int dtype, int M, int64_t sample, int iters,
                 uint64_t seed, int nthreads, float* pivots, float* centroid, int32_t* chunk_offsets) {
  if (M < 1 || M > dim) {
    g_err = "pq: need 1 <= M <= dim";
    return 1;
  }
  Points P{data, n, dim, dtype};
  gann::PQHost pq;
  pq_train(P, M, sample, iters, seed, nthreads, pq);
  std::memcpy(pivots, pq.pivots.data(), sizeof(float) * pq.pivots.size());
  std::memcpy(centroid, pq.centroid.data(), sizeof(float) * pq.centroid.size());
  std::memcpy(chunk_offsets, pq.chunk_offsets.data(), sizeof(int32_t) * pq.chunk_offsets.size());
  return 0;
}

int gib_pq(const void* data, int64_t n, int64_t dim, int dtype, int M, int64_t sample, int iters,
           uint64_t seed, int nthreads, float* pivots, float* centroid, int32_t* chunk_offsets,
           uint8_t* codes) {
  if (M < 1 || M > dim) {
    g_err = "pq: need 1 <= M <= dim";
    return 1;
  }
  Points P{data, n, dim, dtype};
  gann::PQHost pq;
  pq_train(P, M, sample, iters, seed, nthreads, pq);
  pq_encode(P, nthreads, pq);
  std::memcpy(pivots, pq.pivots.data(), sizeof(float) * pq.pivots.size());
  std::memcpy(centroid, pq.centroid.data(), sizeof(float) * pq.centroid.size());
  std::memcpy(chunk_offsets, pq.chunk_offsets.data(), sizeof(int32_t) * pq.chunk_offsets.size());
  std::memcpy(codes, pq.codes.data(), pq.codes.size());
  return 0;
}

// bin/gen_small_file.cpp:18-25: ids 0..num_data-1, std::shuffle with
// std::mt19937(114514), keep the first num_samp, sort ascending.
int gib_sample_ids(int64_t num_data, int64_t num_samp, int32_t* out) {
  if (num_samp > num_data || num_samp < 1) {
    g_err = "sample: need 1 <= num_samp <= num_data";
    return 1;
  }
  std::mt19937 gen(114514);
  std::vector<int> vec;
  vec.reserve((size_t)num_data);
  for (int i = 0; i < (int)num_data; i++) vec.push_back(i);
  std::shuffle(vec.begin(), vec.end(), gen);
  vec.resize((size_t)num_samp);
  std::sort(vec.begin(), vec.end());
  std::copy(vec.begin(), vec.end(), out);
  return 0;
}

// Exact k nearest base points per query (squared L2, ties by smaller id).
int gib_brute_force(const void* base, int64_t n, const float* queries, int64_t nq, int64_t dim,
                    int dtype, int64_t k, int32_t* out_ids, float* out_dists, int nthreads) {
  Points P{base, n, dim, dtype};
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
  for (int64_t qi = 0; qi < nq; ++qi) {
    const float* q = queries + qi * dim;
    std::vector<Cand> best;
    best.reserve((size_t)k + 1);
    for (int64_t i = 0; i < n; ++i) {
      Cand c{P.dist_to(q, i), (uint32_t)i};
      if ((int64_t)best.size() == k && !(c < best.back())) continue;
      best.insert(std::upper_bound(best.begin(), best.end(), c), c);
      if ((int64_t)best.size() > k) best.pop_back();
    }
    for (int64_t j = 0; j < k; ++j) {
      out_ids[qi * k + j] = j < (int64_t)best.size() ? (int32_t)best[(size_t)j].id : -1;
      if (out_dists) out_dists[qi * k + j] = j < (int64_t)best.size() ? best[(size_t)j].d : INFINITY;
    }
  }
  return 0;
}

// Writes <prefix>_disk.index from coords and a fixed-stride adjacency.
int gib_write_disk_index(const char* path, const void* coords, int64_t n, int64_t dim,
                         int64_t elem_size, int64_t R, int64_t medoid, const uint32_t* nbr,
                         const uint32_t* deg) {
  std::vector<int64_t> off((size_t)n + 1, 0);
  std::vector<uint32_t> ids;
  ids.reserve((size_t)(n * R));
  for (int64_t i = 0; i < n; ++i) {
    for (uint32_t j = 0; j < deg[i]; ++j) ids.push_back(nbr[i * R + j]);
    off[(size_t)i + 1] = (int64_t)ids.size();
  }
  if (!gann::write_disk_index(path, n, dim, elem_size, R, medoid, coords, off.data(), ids.data(), &g_err))
    return 1;
  return 0;
}

int gib_write_pq(const char* prefix, const float* pivots, const float* centroid,
                 const int32_t* chunk_offsets, int32_t dim, int32_t M, const uint8_t* codes,
                 int64_t n) {
  gann::PQHost pq;
  pq.dim = dim;
  pq.num_chunks = M;
  pq.num_pts = n;
  pq.pivots.assign(pivots, pivots + 256 * (int64_t)dim);
  pq.centroid.assign(centroid, centroid + dim);
  pq.chunk_offsets.assign(chunk_offsets, chunk_offsets + M + 1);
  pq.codes.assign(codes, codes + n * M);
  std::string p(prefix);
  if (!gann::write_pq(p + "_pivots.bin", p + "_compressed.bin", pq, &g_err)) return 1;
  return 0;
}

// Writes nav/{nav_index, nav_index.data, map.txt} under dir.
int gib_write_nav(const char* dir, const void* data, int64_t n, int64_t dim, int64_t elem_size,
                  const uint32_t* nbr, const uint32_t* deg, int64_t R, int32_t start,
                  const int32_t* mapping) {
  gann::NavHost nav;
  nav.num_node = n;
  nav.dim = (int)dim;
  nav.start = start;
  nav.data.assign((const uint8_t*)data, (const uint8_t*)data + n * dim * elem_size);
  nav.mapping.assign(mapping, mapping + n);
  std::vector<int64_t> off((size_t)n + 1, 0);
  std::vector<uint32_t> ids;
  for (int64_t i = 0; i < n; ++i) {
    for (uint32_t j = 0; j < deg[i]; ++j) ids.push_back(nbr[i * R + j]);
    off[(size_t)i + 1] = (int64_t)ids.size();
  }
  if (!gann::write_nav(dir, nav, elem_size, off, ids, &g_err)) return 1;
  return 0;
}

// Parses an index with the same readers libgustann_hip.so uses (formats.hpp),
// without a device: out[0..11] = num_pts, dim, medoid, node_len,
// nodes_per_page, max_m, num_pages, pq_dim, pq_num_chunks, pq_num_pts,
// nav_num_node, nav_max_m.  nav_prefix may be NULL or "".
int gib_inspect(const char* index_file, const char* pq_prefix, const char* nav_prefix,
                int64_t elem_size, int64_t* out) {
  gann::DiskLayout L;
  if (!gann::parse_disk_meta(index_file, elem_size, &L, &g_err)) return 1;
  gann::PQHost pq;
  std::string pp(pq_prefix);
  if (!gann::read_pq(pp + "_pivots.bin", pp + "_compressed.bin", &pq, true, &g_err)) return 1;
  gann::NavHost nav;
  if (nav_prefix && *nav_prefix && !gann::read_nav(nav_prefix, elem_size, &nav, &g_err)) return 1;
  int64_t v[12] = {L.num_pts, L.dim, L.medoid, L.node_len, L.nodes_per_page, L.max_m, L.num_pages,
                   pq.dim, pq.num_chunks, pq.num_pts, nav.num_node, nav.max_m};
  std::memcpy(out, v, sizeof(v));
  return 0;
}

int gib_write_vecs(const char* path, int64_t elem, int64_t n, int64_t d, const void* data) {
  if (!gann::write_vecs(path, (size_t)elem, n, d, data, &g_err)) return 1;
  return 0;
}

}  // extern "C"

/* CPU oracle for GustANN's in-memory search path: TEST INFRASTRUCTURE ONLY.
 * See gann_oracle.h for the contract.  Every function follows the reference
 * file:line given in its comment; the comments name the reference's own
 * variables so the two can be read side by side.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -mfma, pthreads).
 */
#define _GNU_SOURCE
#include "gann_oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>

#define MASK31 0x7fffffffu
#define VISITED 0x80000000u

/* ------------------------------------------------------------------ threads */

static int g_pin_threads = 0;

void orc_set_pin_threads(int32_t on) { g_pin_threads = on != 0; }

/* Worker t of a pool runs on the (t mod n)-th of the n CPUs the process may
 * use, so a pool of n workers puts one on each core. */
static void pin_worker(int32_t t) {
  if (!g_pin_threads) return;
  cpu_set_t allowed, one;
  if (sched_getaffinity(0, sizeof allowed, &allowed) != 0) return;
  const int n = CPU_COUNT(&allowed);
  if (n <= 0) return;
  int want = t % n, seen = 0;
  for (int c = 0; c < CPU_SETSIZE; ++c) {
    if (!CPU_ISSET(c, &allowed)) continue;
    if (seen++ == want) {
      CPU_ZERO(&one);
      CPU_SET(c, &one);
      pthread_setaffinity_np(pthread_self(), sizeof one, &one);
      return;
    }
  }
}

/* ------------------------------------------------------------------ PQ */

/* src/impl/pq.cuh:8-59 (PQSearchData::init_query).  The reference zeroes the
 * LUT (:12-14), subtracts the centroid from q in place (:22-24), then for
 * each dim i in ascending order adds (q'[i] - pivots_t[i][j])^2 into row
 * chunk_id[i] for every pivot j (:35-43).  Row m therefore accumulates its
 * dims in ascending order, starting from 0. */
void orc_lut_build(const float* pivots, const float* centroid, const int32_t* chunk_offsets,
                   int32_t dim, int32_t num_chunks, const float* q, float* lut) {
  for (int32_t i = 0; i < num_chunks * ORC_NUM_PIVOTS; ++i) lut[i] = 0.0f;
  for (int32_t m = 0; m < num_chunks; ++m) {
    float* row = lut + (int64_t)m * ORC_NUM_PIVOTS;
    for (int32_t i = chunk_offsets[m]; i < chunk_offsets[m + 1]; ++i) {
      float qs = q[i] - centroid[i];
      for (int32_t j = 0; j < ORC_NUM_PIVOTS; ++j) {
        float d = qs - pivots[(int64_t)j * dim + i];
        row[j] = fmaf(d, d, row[j]);
      }
    }
  }
}

/* src/impl/pq.cuh:22-24 then :54-56: q[i] -= centroid[i]; ...; q[i] += centroid[i]. */
void orc_query_restore(const float* centroid, int32_t dim, const float* q, float* q_out) {
  for (int32_t i = 0; i < dim; ++i) {
    volatile float qs = q[i] - centroid[i]; /* keep the two roundings */
    q_out[i] = qs + centroid[i];
  }
}

/* src/impl/pure_mem.cuh:302-308: dist = 0; dist += dist_vec[j*256 + cdata[j]]. */
float orc_adc(const float* lut, int32_t num_chunks, const uint8_t* code) {
  float dist = 0.0f;
  for (int32_t j = 0; j < num_chunks; ++j) dist += lut[(int64_t)j * ORC_NUM_PIVOTS + code[j]];
  return dist;
}

typedef struct {
  const float *pivots, *centroid;
  const int32_t* chunk_offsets;
  int32_t dim, num_chunks;
  const uint8_t* codes;
  int64_t num_pts;
  const float* q;
  int32_t nq;
  const int32_t* ids;
  int32_t ids_per_q;
  float* out;
  int32_t t, nthreads;
} adc_job;

static void* adc_worker(void* arg) {
  adc_job* J = (adc_job*)arg;
  pin_worker(J->t);
  float* lut = (float*)malloc(sizeof(float) * (size_t)J->num_chunks * ORC_NUM_PIVOTS);
  for (int32_t qi = J->t; qi < J->nq; qi += J->nthreads) {
    orc_lut_build(J->pivots, J->centroid, J->chunk_offsets, J->dim, J->num_chunks,
                  J->q + (int64_t)qi * J->dim, lut);
    const int32_t* ids = J->ids + (int64_t)qi * J->ids_per_q;
    float* out = J->out + (int64_t)qi * J->ids_per_q;
    for (int32_t s = 0; s < J->ids_per_q; ++s) {
      int64_t id = ids[s];
      out[s] = (id >= 0 && id < J->num_pts)
                   ? orc_adc(lut, J->num_chunks, J->codes + id * J->num_chunks)
                   : NAN;
    }
  }
  free(lut);
  return NULL;
}

void orc_adc_scan(const float* pivots, const float* centroid, const int32_t* chunk_offsets,
                  int32_t dim, int32_t num_chunks, const uint8_t* codes, int64_t num_pts,
                  const float* q, int32_t nq, const int32_t* ids, int32_t ids_per_q, float* out,
                  int32_t nthreads) {
  if (nthreads < 1) nthreads = 1;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
  adc_job* jobs = (adc_job*)malloc(sizeof(adc_job) * (size_t)nthreads);
  for (int32_t t = 0; t < nthreads; ++t) {
    adc_job j = {pivots, centroid, chunk_offsets, dim, num_chunks, codes, num_pts, q, nq,
                 ids, ids_per_q, out, t, nthreads};
    jobs[t] = j;
    pthread_create(&th[t], NULL, adc_worker, &jobs[t]);
  }
  for (int32_t t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
  free(jobs);
  free(th);
}

/* ------------------------------------------------------------------ exact L2 */

/* src/impl/util.cuh:26-46 (square_sum_32): lane l sums dims l, l+32, ...
 * as val += _val*_val (contracted to fma), then val += shfl_down(val, off)
 * for off = 16, 8, 4, 2, 1; the caller reads lane 0's value (the final
 * __shfl_sync broadcasts it).  For lane 0 only lanes < off matter at each
 * step, so v[l] = v[l] + v[l + off] for l < off reproduces it exactly. */
float orc_l2(const float* q, const void* x, int32_t dtype, int32_t dim) {
  float v[32];
  for (int l = 0; l < 32; ++l) {
    float acc = 0.0f;
    for (int32_t i = l; i < dim; i += 32) {
      float xi = dtype == 0 ? (float)((const uint8_t*)x)[i] : ((const float*)x)[i];
      float d = q[i] - xi;
      acc = fmaf(d, d, acc);
    }
    v[l] = acc;
  }
  for (int off = 16; off > 0; off >>= 1)
    for (int l = 0; l < off; ++l) v[l] = v[l] + v[l + off];
  return v[0];
}

static inline const void* nav_vec(const orc_index* ix, int64_t i) {
  size_t es = ix->dtype == 0 ? 1 : 4;
  return (const uint8_t*)ix->nav_data + (size_t)i * (size_t)ix->dim * es;
}

/* ------------------------------------------------------------------ nav entry */

/* src/impl/nav.cuh:13-135 (get_entry_kernel_inner), one 32-lane warp per
 * query.  The pool is 32 (id, dist) slots: 0..3 are kept (L = 4), 4..31 take
 * the expanded node's first <= 28 neighbours (R = 28); slots beyond the
 * current neighbour count keep stale entries from earlier iterations.
 *
 * Quirks reproduced:
 *  - neighbour reads walk the flat -1-padded graph array from u*max_m for
 *    28 slots, stopping at -1 (:69-72); an index past the end of the array
 *    stops too (the reference would read out of bounds there);
 *  - selection step i (0..3): lanes t < i are excluded with +inf; a lane
 *    t >= i whose id equals slot i-1 (masked) is folded: its dist becomes +inf
 *    in memory and its bits are ORed into slot i-1 (:85-92).  Several folding
 *    lanes store to slot i-1 at once in the reference; the oracle and the HIP
 *    kernel take the union of their bits;
 *  - argmin is a shfl_down tree with strict '<' (:94-102): on ties the lane
 *    kept is fixed by the tree, not by the smallest index;
 *  - the swap of slot i with the winner happens only if their stored dists
 *    differ (:105-116), including the all-+inf case where the winner is lane 0;
 *  - the next slot is the lowest unvisited of all 32 if it is < 4 (:120-129).
 * The loop is bounded by 4*n + 64 expansions (the reference has no bound). */
int32_t orc_nav_entry_local(const orc_index* ix, const float* q, int32_t* iters) {
  uint32_t pid[32];
  float pd[32];
  const int L = ORC_NAV_KEEP, R = ORC_NAV_EXPAND;
  const int64_t total = ix->nav_num_node * (int64_t)ix->nav_max_m;
  pid[0] = (uint32_t)ix->nav_start;
  pd[0] = orc_l2(q, nav_vec(ix, ix->nav_start), ix->dtype, (int32_t)ix->dim);
  for (int t = 1; t < 32; ++t) {
    pid[t] = 0xffffffffu;
    pd[t] = INFINITY;
  }
  int idx = 0;
  int64_t it = 0, cap = 4 * ix->nav_num_node + 64;
  while (idx != -1 && it < cap) {
    ++it;
    uint32_t u = pid[idx];
    pid[idx] |= VISITED;
    for (int i = 0; i < R; ++i) {
      int64_t flat = (int64_t)(u & MASK31) * ix->nav_max_m + i;
      int32_t v = flat < total ? ix->nav_graph[flat] : -1;
      if (v == -1) break;
      pid[i + L] = (uint32_t)v;
      pd[i + L] = orc_l2(q, nav_vec(ix, v), ix->dtype, (int32_t)ix->dim);
    }
    for (int i = 0; i < L; ++i) {
      float rd[32];
      int rp[32];
      uint32_t folded = 0;
      for (int t = 0; t < 32; ++t) {
        rd[t] = pd[t];
        rp[t] = t;
        if (t < i) {
          rd[t] = INFINITY;
        } else if (i != 0 && ((pid[t] ^ pid[i - 1]) & MASK31) == 0) {
          folded |= pid[t];
          pd[t] = INFINITY;
          rd[t] = INFINITY;
        }
      }
      if (i != 0) pid[i - 1] |= folded;
      for (int off = 16; off > 0; off >>= 1)
        for (int l = 0; l < off; ++l)
          if (rd[l + off] < rd[l]) {
            rd[l] = rd[l + off];
            rp[l] = rp[l + off];
          }
      int pos = rp[0];
      if (i != pos) {
        float tv = pd[i], yv = pd[pos];
        if (tv != yv) {
          pd[i] = yv;
          pd[pos] = tv;
          uint32_t m = pid[i];
          pid[i] = pid[pos];
          pid[pos] = m;
        }
      }
    }
    int x = 32;
    for (int t = 0; t < 32; ++t)
      if (!(pid[t] & VISITED)) {
        x = t;
        break;
      }
    idx = x < L ? x : -1;
  }
  if (iters) *iters = (int32_t)it;
  return (int32_t)(pid[0] & MASK31);
}

int32_t orc_entry(const orc_index* ix, const float* q, int32_t* fallback) {
  if (fallback) *fallback = 0;
  if (ix->nav_num_node <= 0) return (int32_t)ix->medoid;
  int32_t local = orc_nav_entry_local(ix, q, NULL);
  if (local < 0 || local >= ix->nav_num_node) {
    if (fallback) *fallback = 1;
    return (int32_t)ix->medoid;
  }
  int32_t base = ix->nav_map[local];
  if (base < 0 || base >= ix->num_pts) {
    if (fallback) *fallback = 1;
    return (int32_t)ix->medoid;
  }
  return base;
}

/* ------------------------------------------------------------------ search */

/* src/impl/util.cuh:166-178: first index in [l, r) whose key is not below
 * (d, x & 0x7fffffff); keys compare dist first, then the masked id. */
static int lower_bound_key(const float* dist, const uint32_t* id, int l, int r, float d,
                           uint32_t x) {
  x &= MASK31;
  while (l < r) {
    int mid = (l + r) / 2;
    if (dist[mid] < d || (dist[mid] == d && (id[mid] & MASK31) < x))
      l = mid + 1;
    else
      r = mid;
  }
  return l;
}

/* src/impl/util.cuh:116-163 (retset_push_32): elements greater than value
 * move one slot right (dropping past max_size); value lands after every
 * element <= value; size grows up to max_size. */
static void topk_push(float* dist, int32_t* ids, int32_t* size, int32_t max_size, float value,
                      int32_t value_id) {
  int p = *size;
  while (p > 0 && dist[p - 1] > value) {
    if (p < max_size) {
      dist[p] = dist[p - 1];
      ids[p] = ids[p - 1];
    }
    --p;
  }
  if (p < max_size) {
    dist[p] = value;
    ids[p] = value_id;
  }
  if (*size + 1 <= max_size) ++*size;
}

static int key_lt(float da, uint32_t ia, float db, uint32_t ib) {
  return da < db || (da == db && (ia & MASK31) < (ib & MASK31));
}

/* One query of search_graph_kernel_gpumem (src/impl/pure_mem.cuh:243-432).
 * Arrays tmp_* / mv_* / mv_pos are the reference's LDS arrays, each L + R
 * long (:267-272).  Returns the number of invariant violations (check). */
static int64_t search_one(const orc_index* ix, const float* q, int32_t entry, int32_t topk,
                          int32_t L, int32_t* nns, float* dists, int32_t* found, int32_t* n_exp,
                          float* lut, float* qr, uint32_t* tmp_id, float* tmp_dist,
                          uint32_t* mv_id, float* mv_dist, int32_t* mv_pos, int check) {
  const int64_t R = ix->max_m, M = ix->num_chunks;
  const int64_t data_len = ix->dim * (ix->dtype == 0 ? 1 : 4);
  int64_t violations = 0;
  orc_lut_build(ix->pivots, ix->centroid, ix->chunk_offsets, (int32_t)ix->dim,
                (int32_t)M, q, lut);                                             /* :284 */
  orc_query_restore(ix->centroid, (int32_t)ix->dim, q, qr);
  for (int32_t j = 0; j < topk; ++j) {
    nns[j] = 0;
    dists[j] = 0.0f;
  }
  *found = 0;
  int32_t sz = 0; /* ctx_size (:279-282) */
  int64_t u = entry;
  int32_t exps = 0;
  const int64_t cap = ix->num_pts + 2; /* unreachable for a valid index */
  while (u != -1 && exps < cap) {
    ++exps;
    const uint8_t* rec = ix->pages + (u / ix->nodes_per_page) * 4096 +
                         (u % ix->nodes_per_page) * ix->node_len;          /* :261-265 */
    int32_t deg;
    memcpy(&deg, rec + data_len, 4);                                       /* :290-292 */
    if (deg > R) deg = (int32_t)R; /* loaders reject such records */
    if (deg < 0) deg = 0;
    const uint8_t* edge = rec + data_len + 4;
    /* ADC of every neighbour; padding lanes get (0xffffffff - t, +inf) (:295-310) */
    for (int64_t t = 0; t < R; ++t) {
      if (t >= deg) {
        tmp_id[sz + t] = 0xffffffffu - (uint32_t)t;
        tmp_dist[sz + t] = INFINITY;
      } else {
        uint32_t v;
        memcpy(&v, edge + 4 * t, 4);
        tmp_id[sz + t] = v;
        tmp_dist[sz + t] = orc_adc(lut, (int32_t)M, ix->codes + (int64_t)v * M);
      }
    }
    /* bottom-up merge sort of the deg new pairs by merge-path ranks (:314-348) */
    for (int len = 2; len < 2 * deg; len *= 2) {
      for (int t = 0; t < deg; ++t) {
        int start = (t / len) * len;
        int mid = start + len / 2 < deg ? start + len / 2 : deg;
        int end = start + len < deg ? start + len : deg;
        if (t >= start && t < mid)
          mv_pos[t] = lower_bound_key(tmp_dist + sz + mid, tmp_id + sz + mid, 0, end - mid,
                                      tmp_dist[sz + t], tmp_id[sz + t]) + t;
        if (t >= mid && t < end)
          mv_pos[t] = lower_bound_key(tmp_dist + sz, tmp_id + sz, start, mid, tmp_dist[sz + t],
                                      tmp_id[sz + t]) + t - mid;
      }
      for (int t = 0; t < deg; ++t) {
        mv_id[mv_pos[t]] = tmp_id[sz + t];
        mv_dist[mv_pos[t]] = tmp_dist[sz + t];
      }
      for (int t = 0; t < deg; ++t) {
        tmp_id[sz + t] = mv_id[t];
        tmp_dist[sz + t] = mv_dist[t];
      }
    }
    /* external merge: a new item equal to an old one goes right after it
     * (:350-376), then the size is capped at 2L (:377) */
    for (int t = 0; t < deg; ++t) {
      int id = lower_bound_key(tmp_dist, tmp_id, 0, sz, tmp_dist[sz + t], tmp_id[sz + t]);
      if (id != sz && ((tmp_id[id] ^ tmp_id[sz + t]) & MASK31) == 0) ++id;
      mv_pos[sz + t] = id + t;
    }
    for (int i = 0; i < sz; ++i)
      mv_pos[i] = lower_bound_key(tmp_dist + sz, tmp_id + sz, 0, deg, tmp_dist[i], tmp_id[i]) + i;
    for (int i = 0; i < sz + deg; ++i) {
      mv_id[mv_pos[i]] = tmp_id[i];
      mv_dist[mv_pos[i]] = tmp_dist[i];
    }
    int32_t sz2 = sz + deg < 2 * L ? sz + deg : 2 * L;
    /* dedup of adjacent equal ids + first unvisited (:380-419).  Positions
     * past sz2 are not candidates: the reference reads stale LDS there and
     * its "no candidate" value sz2 + 1 can also be < L; both are undefined
     * and are taken as "stop". */
    int32_t count = 0, sel = -1;
    for (int i = 0; i < sz2; ++i) {
      int flag = i != 0 && ((mv_id[i] ^ mv_id[i - 1]) & MASK31) == 0;
      if (flag) {
        ++count;
        continue;
      }
      int mvp = i - count;
      tmp_id[mvp] = mv_id[i];
      tmp_dist[mvp] = mv_dist[i];
      if (sel < 0 && !(mv_id[i] & VISITED)) sel = mvp;
    }
    /* exact rerank of the node just expanded + top-k insertion (:420-423) */
    {
      float d = orc_l2(qr, rec, ix->dtype, (int32_t)ix->dim);
      topk_push(dists, nns, found, topk, d, (int32_t)u);
    }
    if (sel < 0 || sel >= L) {
      u = -1;
    } else {
      u = tmp_id[sel];
      sz = sz2 - count < L ? sz2 - count : L;
      tmp_id[sel] |= VISITED;
    }
    if (check) {
      int32_t n = (u == -1) ? (sz2 - count < L ? sz2 - count : L) : sz;
      if (n > L) ++violations;
      for (int i = 1; i < n; ++i) {
        if (!key_lt(tmp_dist[i - 1], tmp_id[i - 1], tmp_dist[i], tmp_id[i])) ++violations;
        if (((tmp_id[i] ^ tmp_id[i - 1]) & MASK31) == 0) ++violations;
      }
    }
  }
  if (n_exp) *n_exp = exps;
  return violations;
}

typedef struct {
  const orc_index* ix;
  const float* q;
  int32_t nq;
  const int32_t* entries;
  int32_t topk, L;
  int32_t *nns, *found, *n_exp;
  float* dists;
  int32_t t, nthreads, check;
  int64_t violations;
} search_job;

static void* search_worker(void* arg) {
  search_job* J = (search_job*)arg;
  pin_worker(J->t);
  const orc_index* ix = J->ix;
  int64_t cap = J->L + ix->max_m;
  float* lut = (float*)malloc(sizeof(float) * (size_t)ix->num_chunks * ORC_NUM_PIVOTS);
  float* qr = (float*)malloc(sizeof(float) * (size_t)ix->dim);
  uint32_t* tmp_id = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)cap);
  uint32_t* mv_id = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)cap);
  float* tmp_dist = (float*)malloc(sizeof(float) * (size_t)cap);
  float* mv_dist = (float*)malloc(sizeof(float) * (size_t)cap);
  int32_t* mv_pos = (int32_t*)malloc(sizeof(int32_t) * (size_t)cap);
  for (int32_t qi = J->t; qi < J->nq; qi += J->nthreads) {
    const float* q = J->q + (int64_t)qi * ix->dim;
    int32_t entry = J->entries ? J->entries[qi] : orc_entry(ix, q, NULL);
    int32_t ne = 0;
    J->violations += search_one(ix, q, entry, J->topk, J->L, J->nns + (int64_t)qi * J->topk,
                                J->dists + (int64_t)qi * J->topk, J->found + qi, &ne, lut, qr,
                                tmp_id, tmp_dist, mv_id, mv_dist, mv_pos, J->check);
    if (J->n_exp) J->n_exp[qi] = ne;
  }
  free(lut);
  free(qr);
  free(tmp_id);
  free(mv_id);
  free(tmp_dist);
  free(mv_dist);
  free(mv_pos);
  return NULL;
}

int64_t orc_search(const orc_index* ix, const float* q, int32_t nq, const int32_t* entries,
                   int32_t topk, int32_t L, int32_t* nns, float* dists, int32_t* found,
                   int32_t* n_expansions, int32_t nthreads, int32_t check) {
  if (nthreads < 1) nthreads = 1;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
  search_job* jobs = (search_job*)calloc((size_t)nthreads, sizeof(search_job));
  for (int32_t t = 0; t < nthreads; ++t) {
    search_job j = {ix, q, nq, entries, topk, L, nns, found, n_expansions, dists,
                    t, nthreads, check, 0};
    jobs[t] = j;
    pthread_create(&th[t], NULL, search_worker, &jobs[t]);
  }
  int64_t v = 0;
  for (int32_t t = 0; t < nthreads; ++t) {
    pthread_join(th[t], NULL);
    v += jobs[t].violations;
  }
  free(jobs);
  free(th);
  return v;
}

/* ------------------------------------------------------------------ beam */

/* orc_search_beam (gann_oracle.h): a sorted array of at most L entries. */
typedef struct {
  float* dist;
  uint32_t* id;
  uint8_t* visited;
  int32_t size;
} beam_list;

static void beam_insert(beam_list* B, int32_t L, float d, uint32_t v) {
  int pos = lower_bound_key(B->dist, B->id, 0, B->size, d, v);
  for (int i = 0; i < B->size; ++i)
    if (B->id[i] == v) return; /* listed already */
  if (pos >= L) return;
  int last = B->size < L ? B->size : L - 1; /* the entry at L - 1 falls off a full list */
  for (int i = last; i > pos; --i) {
    B->dist[i] = B->dist[i - 1];
    B->id[i] = B->id[i - 1];
    B->visited[i] = B->visited[i - 1];
  }
  B->dist[pos] = d;
  B->id[pos] = v;
  B->visited[pos] = 0;
  if (B->size < L) ++B->size;
}

static void search_beam_one(const orc_index* ix, const float* q, int32_t entry, int32_t topk,
                            int32_t L, int32_t bw, int32_t* nns, float* dists, int32_t* found,
                            int32_t* n_exp, float* lut, float* qr, beam_list* B, int64_t* sel) {
  const int64_t R = ix->max_m, M = ix->num_chunks;
  const int64_t data_len = ix->dim * (ix->dtype == 0 ? 1 : 4);
  orc_lut_build(ix->pivots, ix->centroid, ix->chunk_offsets, (int32_t)ix->dim, (int32_t)M, q,
                lut);
  orc_query_restore(ix->centroid, (int32_t)ix->dim, q, qr);
  for (int32_t j = 0; j < topk; ++j) {
    nns[j] = 0;
    dists[j] = 0.0f;
  }
  *found = 0;
  B->size = 0;
  int32_t exps = 0;
  const int64_t cap = ix->num_pts + 2;
  int32_t nsel = 0;
  if (entry >= 0) sel[nsel++] = entry;
  while (nsel > 0) {
    for (int32_t b = 0; b < nsel && exps < cap; ++b) {
      const int64_t u = sel[b];
      ++exps;
      const uint8_t* rec = ix->pages + (u / ix->nodes_per_page) * 4096 +
                           (u % ix->nodes_per_page) * ix->node_len;
      int32_t deg;
      memcpy(&deg, rec + data_len, 4);
      if (deg > R) deg = (int32_t)R;
      if (deg < 0) deg = 0;
      const uint8_t* edge = rec + data_len + 4;
      for (int32_t t = 0; t < deg; ++t) {
        uint32_t v;
        memcpy(&v, edge + 4 * t, 4);
        beam_insert(B, L, orc_adc(lut, (int32_t)M, ix->codes + (int64_t)v * M), v);
      }
      topk_push(dists, nns, found, topk, orc_l2(qr, rec, ix->dtype, (int32_t)ix->dim), (int32_t)u);
    }
    nsel = 0;
    if (exps >= cap) break;
    for (int32_t i = 0; i < B->size && nsel < bw; ++i) {
      if (B->visited[i]) continue;
      B->visited[i] = 1;
      sel[nsel++] = B->id[i];
    }
  }
  if (n_exp) *n_exp = exps;
}

typedef struct {
  const orc_index* ix;
  const float* q;
  int32_t nq;
  const int32_t* entries;
  int32_t topk, L, bw;
  int32_t *nns, *found, *n_exp;
  float* dists;
  int32_t t, nthreads;
} beam_job;

static void* beam_worker(void* arg) {
  beam_job* J = (beam_job*)arg;
  pin_worker(J->t);
  const orc_index* ix = J->ix;
  float* lut = (float*)malloc(sizeof(float) * (size_t)ix->num_chunks * ORC_NUM_PIVOTS);
  float* qr = (float*)malloc(sizeof(float) * (size_t)ix->dim);
  beam_list B;
  B.dist = (float*)malloc(sizeof(float) * (size_t)J->L);
  B.id = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)J->L);
  B.visited = (uint8_t*)malloc((size_t)J->L);
  int64_t* sel = (int64_t*)malloc(sizeof(int64_t) * (size_t)(J->bw > 1 ? J->bw : 1));
  for (int32_t qi = J->t; qi < J->nq; qi += J->nthreads) {
    const float* q = J->q + (int64_t)qi * ix->dim;
    int32_t entry = J->entries ? J->entries[qi] : orc_entry(ix, q, NULL);
    int32_t ne = 0;
    search_beam_one(ix, q, entry, J->topk, J->L, J->bw, J->nns + (int64_t)qi * J->topk,
                    J->dists + (int64_t)qi * J->topk, J->found + qi, &ne, lut, qr, &B, sel);
    if (J->n_exp) J->n_exp[qi] = ne;
  }
  free(lut);
  free(qr);
  free(B.dist);
  free(B.id);
  free(B.visited);
  free(sel);
  return NULL;
}

int64_t orc_search_beam(const orc_index* ix, const float* q, int32_t nq, const int32_t* entries,
                        int32_t topk, int32_t L, int32_t bw, int32_t* nns, float* dists,
                        int32_t* found, int32_t* n_expansions, int32_t nthreads) {
  if (nthreads < 1) nthreads = 1;
  if (bw < 1) bw = 1;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
  beam_job* jobs = (beam_job*)calloc((size_t)nthreads, sizeof(beam_job));
  for (int32_t t = 0; t < nthreads; ++t) {
    beam_job j = {ix, q, nq, entries, topk, L, bw, nns, found, n_expansions, dists, t, nthreads};
    jobs[t] = j;
    pthread_create(&th[t], NULL, beam_worker, &jobs[t]);
  }
  for (int32_t t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
  free(jobs);
  free(th);
  return 0;
}

/* ------------------------------------------------------------------ recall */

static int cmp_i32(const void* a, const void* b) {
  int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
  return (x > y) - (x < y);
}

/* bin/utils.hpp:104-116: std::set of the first k gt ids; each result slot
 * that is in the set counts once (duplicates count per occurrence). */
double orc_recall(const int32_t* res, const int32_t* gt, int32_t num, int32_t gt_dim, int32_t k) {
  int64_t cnt = 0;
  int32_t* s = (int32_t*)malloc(sizeof(int32_t) * (size_t)(k > 0 ? k : 1));
  for (int32_t i = 0; i < num; ++i) {
    memcpy(s, gt + (int64_t)i * gt_dim, sizeof(int32_t) * (size_t)k);
    qsort(s, (size_t)k, sizeof(int32_t), cmp_i32);
    for (int32_t j = 0; j < k; ++j) {
      int32_t key = res[(int64_t)i * k + j];
      if (bsearch(&key, s, (size_t)k, sizeof(int32_t), cmp_i32)) ++cnt;
    }
  }
  free(s);
  return (double)cnt / ((double)num * k);
}

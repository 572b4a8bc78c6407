// Candidate-list update and top-k insertion shared by the search kernels
// (gann_kernels.hip) and the graph builder (gann_build.hip): one wavefront
// per query, list and scratch in LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <climits>
#include <type_traits>

#include "gann_device.hpp"

namespace gann {

// Per-expansion list update shared by the fused and the step-wise kernels.
//
// The reference (src/impl/pure_mem.cuh:350-419) merges the sorted new run
// into the list by merge-path ranks, caps the result at 2L, removes every
// entry whose id equals its predecessor's (a new copy always lands right
// after its old copy, :358-360), caps at L and takes the first unvisited
// entry below L.  The same list results from inserting only the new entries
// that are not already present:
//  * the 2L cap never changes the first L distinct entries (each id occurs
//    at most twice among the first 2L merged entries), so it is dropped;
//  * a new entry is a duplicate iff the old entry at its lower bound has the
//    same id; the others move in at rank + (earlier inserted count);
//  * an old entry i moves right by the number of inserted entries ranked at
//    or before i;
//  * every entry before the first unvisited one is visited, so the next
//    node is min(new position of the old first-unvisited entry, position of
//    the first inserted entry), tracked incrementally in fu.
// The update runs in two phases so the caller can start fetching the next
// node's record between them: plan() ranks the new run and picks the next
// node without writing; apply() shifts the list in place (top chunk first,
// skipping everything below the first insertion) and marks the node visited.
// A: the list (sorted by key, distinct ids, visited flag in bit 0), of
// list_capacity(L) entries; BM: list_scratch_words(L) words of scratch.

// Scratch words per wave for the list update: a bitmap of the positions the
// inserted entries take, two words per 64-entry chunk.
__host__ __device__ constexpr int list_scratch_words(int L) { return 2 * ((L + kWave - 1) / kWave); }

// Entries allocated for a list of at most L: L rounded up to whole 64-entry
// chunks, so that every lane of a chunk the update touches is inside the
// wave's own list.
__host__ __device__ constexpr int list_capacity(int L) { return (L + kWave - 1) / kWave * kWave; }

// Rank of `key` in the sorted list A[0..sz): the number of entries ordered
// below it.  A first level shared by all lanes splits the list into 9
// segments of s entries and reads the last entry of the first 8 (uniform
// addresses); the entries below key are a prefix of those probes, so their
// count fixes the lane's segment.  Uniform steps finish it: one binary step
// when the largest power of two q within the span is an odd power, then
// 4-ary levels q, q/4, ..., 4 of 3 probes each, issued together (reads
// clamped into the segment, probes at or past its end count as not below),
// then the level q = 1, which reads the four entries from its lower bound
// so that the entry at the result arrives with it (at_r: the entry at
// min(result, sz - 1), for the duplicate test).  A 263-entry segment takes 5
// dependent LDS reads instead of 9 plus the duplicate test's.  Every lane
// runs the search, whether its key is live or not (`active`: the result is
// 0 where it is not), so that the first level's reads, at addresses the same
// in every lane, are issued together rather than one after another under
// the live lanes' mask.
__device__ __forceinline__ int list_rank(const uint64_t* A, int sz, uint64_t key, bool active, uint64_t& at_r) {
  at_r = 0;
  int lo = 0, end = sz, span = sz;  // answer in [lo, end]; span bounds end - lo
  if (sz > 8) {
    const int s = (sz + 8) / 9;
    int cnt = 0;
#pragma unroll
    for (int m = 0; m < 8; ++m) cnt += A[min(s * (m + 1) - 1, sz - 1)] < key ? 1 : 0;
    lo = min(s * cnt, sz);
    end = cnt == 8 ? sz : min(s * (cnt + 1) - 1, sz - 1);
    span = s;
  }
  if (span <= 0) return 0;  // sz == 0
  const int last = max(end - 1, 0), top = sz - 1;
  int lq = 31 - __builtin_clz((unsigned)span);  // q = 1 << lq, uniform
  if (lq & 1) {
    const int p = lo + (1 << lq) - 1;
    const uint64_t a = A[min(p, last)];
    if (p < end && a < key) lo += 1 << lq;
    --lq;
  }
  for (; lq >= 2; lq -= 2) {
    const int q = 1 << lq;
    const int p1 = lo + q - 1, p2 = p1 + q, p3 = p2 + q;
    const uint64_t a1 = A[min(p1, last)], a2 = A[min(p2, last)], a3 = A[min(p3, last)];
    const int c = (p1 < end && a1 < key ? 1 : 0) + (p2 < end && a2 < key ? 1 : 0) + (p3 < end && a3 < key ? 1 : 0);
    lo += c * q;
  }
  // q = 1: positions lo .. lo + 2 decide, lo + 3 is read for at_r only;
  // clamping to sz - 1 instead of the segment's end reads the same entries
  // wherever a probe counts (below end <= sz)
  const uint64_t a0 = A[min(lo, top)], a1 = A[min(lo + 1, top)], a2 = A[min(lo + 2, top)],
                 a3 = A[min(lo + 3, top)];
  const int c = (lo < end && a0 < key ? 1 : 0) + (lo + 1 < end && a1 < key ? 1 : 0) +
                (lo + 2 < end && a2 < key ? 1 : 0);
  at_r = c == 0 ? a0 : c == 1 ? a1 : c == 2 ? a2 : a3;
  return active ? lo + c : 0;
}

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}

struct ListPlan {
  uint64_t nkey;  // lanes 0..n_nd-1: the inserted entries, ascending; other lanes ~0
  int p;          // lanes 0..n_nd-1: position of the lane's entry in the new list
  int n_nd;       // inserted count (uniform)
  int p0;         // position of the first inserted entry (uniform, INT_MAX if none)
  int cand;       // position of the next node in the new list (uniform, -1: stop)
  uint64_t sel;   // the selected entry (uniform)
  int nsz;        // new list size (uniform)
  int lb;         // every entry before lb is visited in the new list (uniform, <= nsz)
};

// Ranks each lane's candidate (lanes < deg) in the list, drops those whose id
// is listed already, sorts the rest with their ranks into lanes 0..n_nd-1
// (an inserted entry's position is then rank + lane) and picks the next node.
//
// A candidate ranked at L (the list is full and every entry orders below it)
// is dropped with the duplicates before the sort: it could only land at a
// position >= L, and it orders after every inserted entry, so the others'
// positions are unchanged.  Most expansions of a converged search have no
// candidate left (about four in five at L = 448 on a 128-d uint8 mixture)
// and skip the sort.
__device__ __forceinline__ ListPlan list_plan(const uint64_t* A, int L, uint64_t key, int deg,
                                              int sz, int fu) {
  const int lane = lane_id();
  const uint64_t fu_entry = fu < sz ? A[fu] : 0;
  const bool active = lane < deg;
  uint64_t at_r;
  uint32_t r = (uint32_t)list_rank(A, sz, key, active, at_r);
  // a candidate whose id is listed already sits at its lower bound
  const bool dup = active && (int)r < sz && entry_id(at_r) == entry_id(key);
  if (!active || dup || (int)r >= L) key = ~(uint64_t)0;  // never a real key: ids are < 2^31 - 1
  const uint64_t live = ballot64(key != ~(uint64_t)0);
  // uniform branches; the sort keeps the count
  if (live != 0) {
    if (__popcll(live) <= kFewSort)
      wave_sort_few_kv(key, r, live);
    else
      wave_sort64_kv(key, r);
  }
  ListPlan P;
  P.nkey = key;
  P.n_nd = __popcll(live);
  P.p = (int)r + lane;
  P.p0 = P.n_nd ? __builtin_amdgcn_readlane((int)r, 0) : INT_MAX;
  P.nsz = min(sz + P.n_nd, L);
  int fu_new = INT_MAX;
  if (fu < sz) fu_new = fu + __popcll(ballot64(lane < P.n_nd && (int)r <= fu));
  const int cand = min(fu_new, P.p0);
  P.lb = min(cand, P.nsz);
  if (cand >= P.nsz) {
    P.cand = -1;
    P.sel = 0;
  } else {
    P.cand = cand;
    P.sel = cand == fu_new ? fu_entry : readlane64(key, 0);
  }
  return P;
}

// Applies the plan in place and returns the new first-unvisited index.  The
// positions the inserted entries take are marked in the bitmap BM; output
// position j then holds inserted entry nb(j) (nb = inserted entries placed
// before j) if marked, else old entry j - nb(j).  The old entries are
// gathered into the unmarked positions in windows of 16 chunks, top window
// first (near the start of the list the last ones may be of 8, 4, 2 or 1):
// a batch reads only positions below its highest output and at or above its
// lowest output minus 64, and writes after all its reads, so no source is
// overwritten before it is read; chunks below the first insertion that a
// batch covers have no marks and copy onto themselves.  Then each inserted
// entry is stored at its marked position by the lane that holds it.
// kSelect = false (beam search) only applies the insertions and returns P.lb.
template <bool kSelect = true>
__device__ __forceinline__ int list_apply(uint64_t* A, uint32_t* BM, const ListPlan& P) {
  constexpr int kBatch = 16;
  const int lane = lane_id();
  wave_sync();  // all reads of plan() done
  const int start = min(P.p0, P.nsz);
  if (start < P.nsz) {
    const int cb = start / kWave, ct = (P.nsz - 1) / kWave;  // first and top chunk that change
    // the last full window may sweep up to kBatch - 1 chunks below cb: their
    // marks are cleared as well, so they copy onto themselves
    const int c0 = max(0, cb - (kBatch - 1));
    for (int w = lane; w < 2 * (ct - c0 + 1); w += kWave) BM[2 * c0 + w] = 0u;
    wave_sync();
    const bool placed = lane < P.n_nd && P.p < P.nsz;
    if (placed) atomicOr(&BM[P.p >> 5], 1u << (P.p & 31));
    // positions from nsz to the end of the top chunk are marked as well, so
    // that they keep their entries like the inserted positions do
    const int jt = kWave * ct + lane;
    if (jt >= P.nsz) atomicOr(&BM[jt >> 5], 1u << (jt & 31));
    const int n_tail = kWave * (ct + 1) - P.nsz;
    // inserted entries placed below the chunk being gathered, counted down
    // from the top; it starts with the top chunk's n_tail extra marks, so
    // that every chunk subtracts its whole mask
    int below = __popcll(ballot64(placed)) + n_tail;
    wave_sync();
    // One chunk of a batch: output j = 64 c + lane takes old entry j - nb
    // (nb = below + marked positions of the chunk below this lane, the count
    // folded into mbcnt's addend), or keeps its own entry where it is marked
    // (selected by the mask itself, one v_cndmask).
    auto gather = [&](uint64_t mo, int j, uint64_t& val) {
      const int nb = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mo >> 32),
                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)mo, (uint32_t)below));
      val = A[(int)lane_select(mo, (uint32_t)(j - nb), (uint32_t)j)];
    };
    // Straight-line batches: every lane reads one entry per chunk and writes
    // it back, with no branch between the reads and the writes, all reads of
    // a batch before its writes.  Full windows of kBatch chunks [b_hi - 16,
    // b_hi) from the top: the chunk of each slot, its mask word in the batch's
    // read and its LDS offset are fixed at compile time.
    // One full window of kB chunks [b_hi - kB, b_hi) (b_hi >= kB).
    int b_hi = ct + 1;
    auto window = [&](auto kb) {
      constexpr int kB = decltype(kb)::value;
      const int b_lo = b_hi - kB;
      const uint32_t wv = lane < 2 * kB ? BM[2 * b_lo + lane] : 0u;
      const int jtop = kWave * (b_hi - 1) + lane;
      uint64_t val[kB];
#pragma unroll
      for (int t = 0; t < kB; ++t) {
        constexpr int kTop = 2 * (kB - 1);
        const uint64_t mo = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)wv, kTop - 2 * t + 1) << 32) |
                            (uint32_t)__builtin_amdgcn_readlane((int)wv, kTop - 2 * t);
        below -= __popcll(mo);
        gather(mo, jtop - kWave * t, val[t]);
      }
      wave_sync();
#pragma unroll
      for (int t = 0; t < kB; ++t) A[jtop - kWave * t] = val[t];
      wave_sync();
      b_hi = b_lo;
    };
    while (b_hi > cb && b_hi >= kBatch) window(std::integral_constant<int, kBatch>{});
    // What is left lies in the first kBatch - 1 chunks of the list (so c0 is
    // chunk 0 and every chunk below cb copies onto itself): windows of 8, 4,
    // 2 and 1 chunks down from b_hi, each taken while chunks above cb remain
    // and it fits above chunk 0 -- usually one, at most four.
    if (b_hi > cb && b_hi >= 8) window(std::integral_constant<int, 8>{});
    if (b_hi > cb && b_hi >= 4) window(std::integral_constant<int, 4>{});
    if (b_hi > cb && b_hi >= 2) window(std::integral_constant<int, 2>{});
    if (b_hi > cb && b_hi >= 1) window(std::integral_constant<int, 1>{});
    // the inserted entries into their marked positions, after every old
    // entry has moved out of the way
    if (placed) A[P.p] = P.nkey;
    wave_sync();
  }
  if (!kSelect) return P.lb;
  if (P.cand < 0) return P.nsz;
  if (lane == 0) A[P.cand] = P.sel | kListVisited;
  wave_sync();
  int nfu = P.nsz;
  for (int base = P.cand + 1; base < P.nsz; base += kWave) {
    const int i = base + lane;
    const uint64_t m = ballot64(i < P.nsz && !entry_visited(A[i]));
    if (m) {
      nfu = base + (int)__builtin_ctzll(m);
      break;
    }
  }
  return nfu;
}

// The plan of one expansion whose neighbours come in NB blocks of 64 (block
// b holds neighbours 64b .. 64b+63 in key[b], ~0 past deg; graph degree up
// to 64 NB).  Every block but the last non-empty one is inserted without a
// selection (list_apply<false>), then the last block is planned as usual.
// This is the list the reference's single merge of all deg neighbours gives
// (src/impl/pure_mem.cuh:314-419): the list is always the first L of the
// sorted union of everything listed so far (an id once, with the listed
// copy's visited flag), and the first L of (the first L of A ∪ B) ∪ C is the
// first L of A ∪ B ∪ C; a neighbour list holds no id twice, so no block
// duplicates another's entry, and the first unvisited entry is carried from
// block to block (list_apply<false> returns it).  sz and fu are updated for
// the blocks applied here; the caller applies the returned plan.
template <int NB>
__device__ __forceinline__ ListPlan list_plan_nb(uint64_t* A, uint32_t* BM, int L,
                                                 const uint64_t (&key)[NB], int deg, int& sz,
                                                 int& fu) {
  static_assert(NB == 1 || NB == 2, "one or two neighbour blocks");
  if constexpr (NB == 2) {
    if (deg > kWave) {
      const ListPlan P0 = list_plan(A, L, key[0], kWave, sz, fu);
      fu = list_apply<false>(A, BM, P0);
      sz = P0.nsz;
      return list_plan(A, L, key[1], deg - kWave, sz, fu);
    }
  }
  return list_plan(A, L, key[0], min(deg, kWave), sz, fu);
}

// Top-k insertion of (d, id) into the sorted LDS list (src/impl/util.cuh:116-163):
// the value lands after the last element that is not greater than it,
// greater elements shift right, the list keeps at most k.
__device__ __forceinline__ void topk_push(float* td, int32_t* ti, int* found, int k, float d,
                                          int32_t id) {
  const int lane = lane_id();
  const int n = *found;
  // position = 1 + index of the last element with !(elem > d)
  int pos = 0;
  for (int base = 0; base < n; base += kWave) {
    const int j = base + lane;
    const uint64_t ng = ballot64(j < n && !(td[j] > d));
    if (ng) pos = base + 64 - (int)__builtin_clzll(ng);
  }
  // shift [pos, last) right by one, last chunk first; the element at index
  // k-1 of a full list falls off
  const int last = min(n, k - 1);
  if (last > pos) {
    for (int base = ((last - 1) / kWave) * kWave; base >= (pos / kWave) * kWave; base -= kWave) {
      const int j = base + lane;
      const bool mv = j >= pos && j < last;
      float vd = 0.f;
      int32_t vi = 0;
      if (mv) {
        vd = td[j];
        vi = ti[j];
      }
      wave_sync();
      if (mv) {
        td[j + 1] = vd;
        ti[j + 1] = vi;
      }
      wave_sync();
    }
  }
  if (lane == 0 && pos < k) {
    td[pos] = d;
    ti[pos] = id;
  }
  if (n + 1 <= k) *found = n + 1;
  wave_sync();
}

// The same insertion with the list in registers (k <= 64): lane j holds
// element j and the shift is one DPP lane shift.
__device__ __forceinline__ void topk_push_regs(float& td, int32_t& ti, int& found, int k, float d,
                                               int32_t id) {
  const int lane = lane_id();
  const int n = found;
  const uint64_t ng = ballot64(lane < n && !(td > d));
  const int pos = ng ? 64 - (int)__builtin_clzll(ng) : 0;
  const int last = min(n, k - 1);
  const float sd = __uint_as_float(lane_shr1(__float_as_uint(td)));
  const int32_t si = (int32_t)lane_shr1((uint32_t)ti);
  if (lane > pos && lane <= last) {
    td = sd;
    ti = si;
  }
  if (lane == pos && pos < k) {
    td = d;
    ti = id;
  }
  if (n + 1 <= k) found = n + 1;
}

// Top-k state of one query: registers for k <= 64, else the LDS arrays td/ti.
struct TopK {
  float* td;
  int32_t* ti;
  int k, found;
  float rd;
  int32_t ri;
  __device__ __forceinline__ TopK(float* td_, int32_t* ti_, int k_)
      : td(td_), ti(ti_), k(k_), found(0), rd(0.0f), ri(0) {}
  __device__ __forceinline__ void push(float d, int32_t id) {
    if (k <= kWave)
      topk_push_regs(rd, ri, found, k, d, id);
    else
      topk_push(td, ti, &found, k, d, id);
  }
  // slots past found are 0, as in the reference's zero-initialised vectors
  __device__ __forceinline__ void store(int32_t* nns, float* dists, int64_t qi) const {
    const int lane = lane_id();
    if (k <= kWave) {
      if (lane < k) {
        const bool ok = lane < found;
        nns[qi * k + lane] = ok ? ri : 0;
        dists[qi * k + lane] = ok ? rd : 0.0f;
      }
    } else {
      for (int j = lane; j < k; j += kWave) {
        const bool ok = j < found;
        nns[qi * k + j] = ok ? ti[j] : 0;
        dists[qi * k + j] = ok ? td[j] : 0.0f;
      }
    }
  }
};

}  // namespace gann

// Exact tie order of the reference's selections, for the rare tokens where
// equal scores straddle a cut.
//
// The reference selects the top-4 groups and the top-8 experts with
// torch.topk(sorted=False) (reference moe/ref_moe.py:111, :119). On the CPU,
// torch fills (value, index) pairs in index order and runs
// std::nth_element(first, first + k - 1, last, greater) on them
// (ATen/native/TopKImpl.h:44-80 in torch 2.10.0), so WHICH of several equal
// values lands among the first k is decided by libstdc++'s introselect (GCC 11,
// the compiler torch 2.10.0 was built with: bits/stl_algo.h __introselect and
// its helpers, bits/stl_heap.h for the heap-select fallback). When no tie
// straddles the cut the selected set is unique and this code never runs.
//
// wave_nth_element runs that introselect on up to 256 (key, id) entries held in
// a per-wave LDS scratch, with the 64 lanes of one wave:
//  * the median-of-3 pivot choice and the final insertion sort of <= 3 entries
//    are uniform scalar decisions (lane 0 moves the entries);
//  * each Hoare partition (__unguarded_partition) is done at once: the scan from
//    the left stops at entries not greater than the pivot, the scan from the
//    right at entries not less than it; the k-th left stop (ascending) swaps with
//    the k-th right stop (descending) for every k with left < right, a prefix of
//    the k's; the returned cut is min(next left stop, last right stop swapped).
//    The stops are ranked with ballots and prefix popcounts, positions scattered
//    to LDS by rank, partners gathered from there;
//  * the heap-select fallback at depth 0 (reachable only with adversarial
//    inputs) runs sequentially on lane 0.
// Keys are order-preserving integer images of the fp32 values (equal keys are
// equal values; the inputs here are finite).
#pragma once

#include "moe_common.h"

namespace moe {

struct TieScratch {
  uint32_t key[E_GLOBAL];
  uint32_t id[E_GLOBAL];
  uint16_t lpos[E_GLOBAL];  // position of the k-th left stop of a partition
  uint16_t rpos[E_GLOBAL];  // position of the k-th right stop
};
static_assert(sizeof(TieScratch) == 3072, "3 KB per wave");

// The scratch is addressed in the LDS address space explicitly, so every access
// is a ds_* instruction (a generic pointer to volatile data compiles to flat ones).
typedef volatile __attribute__((address_space(3))) TieScratch VTie;

__device__ __forceinline__ VTie& lds_tie(TieScratch* p) { return *(VTie*)p; }

__device__ __forceinline__ void tie_move(VTie& s, int dst, int src) {
  s.key[dst] = s.key[src];
  s.id[dst] = s.id[src];
}

__device__ __forceinline__ void tie_swap(VTie& s, int a, int b) {
  const uint32_t ka = s.key[a], kb = s.key[b], ia = s.id[a], ib = s.id[b];
  s.key[a] = kb;
  s.key[b] = ka;
  s.id[a] = ib;
  s.id[b] = ia;
}

// bits/stl_heap.h __push_heap / __adjust_heap with comp = greater, one lane.
__device__ __forceinline__ void tie_adjust_heap(VTie& s, int first, int hole, int len, uint32_t vk, uint32_t vi) {
  const int top = hole;
  int child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (s.key[first + child] > s.key[first + child - 1]) child--;
    tie_move(s, first + hole, first + child);
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    tie_move(s, first + hole, first + child - 1);
    hole = child - 1;
  }
  int parent = (hole - 1) / 2;
  while (hole > top && s.key[first + parent] > vk) {
    tie_move(s, first + hole, first + parent);
    hole = parent;
    parent = (hole - 1) / 2;
  }
  s.key[first + hole] = vk;
  s.id[first + hole] = vi;
}

// bits/stl_algo.h __heap_select(first, middle, last) then iter_swap(first, nth).
__device__ __forceinline__ void tie_heap_select(VTie& s, int first, int middle, int last, int nth) {
  const int len = middle - first;
  if (len >= 2) {
    for (int parent = (len - 2) / 2;; --parent) {
      tie_adjust_heap(s, first, parent, len, s.key[first + parent], s.id[first + parent]);
      if (parent == 0) break;
    }
  }
  for (int i = middle; i < last; ++i) {
    if (s.key[i] > s.key[first]) {
      const uint32_t vk = s.key[i], vi = s.id[i];
      tie_move(s, i, first);
      tie_adjust_heap(s, first, 0, len, vk, vi);
    }
  }
  tie_swap(s, first, nth);
}

// bits/stl_algo.h __insertion_sort(first, last) with comp = greater, one lane.
__device__ __forceinline__ void tie_insertion_sort(VTie& s, int first, int last) {
  for (int i = first + 1; i < last; ++i) {
    const uint32_t vk = s.key[i], vi = s.id[i];
    int hole = i;
    if (vk > s.key[first]) {
      for (; hole > first; --hole) tie_move(s, hole, hole - 1);
    } else {
      while (vk > s.key[hole - 1]) {
        tie_move(s, hole, hole - 1);
        --hole;
      }
    }
    s.key[hole] = vk;
    s.id[hole] = vi;
  }
}

// std::nth_element(e, e + nth, e + n, greater) on entries [0, n) of s, n <= 256,
// by the whole wave (every lane calls it with the same n, nth). LDS operations of
// one wave complete in issue order and every access is volatile, so a lane's
// read after another lane's write (in program order) sees the write.
__device__ __forceinline__ void wave_nth_element(VTie& s, int n, int nth) {
  const int lane = threadIdx.x & 63;
  const unsigned long long below = (1ull << lane) - 1ull;
  const unsigned long long above = ~below & ~(1ull << lane);
  int first = 0, last = n;
  int depth = 2 * (31 - __builtin_clz((unsigned)n));
  while (last - first > 3) {
    if (depth == 0) {
      if (lane == 0) tie_heap_select(s, first, nth + 1, last, nth);
      return;
    }
    --depth;
    // __move_median_to_first(first, first + 1, mid, last - 1)
    const int mid = first + (last - first) / 2;
    const uint32_t ka = s.key[first + 1], kb = s.key[mid], kc = s.key[last - 1];
    int m;
    if (ka > kb) m = kb > kc ? mid : (ka > kc ? last - 1 : first + 1);
    else m = ka > kc ? first + 1 : (kb > kc ? last - 1 : mid);
    if (lane == 0) tie_swap(s, first, m);
    const uint32_t p = s.key[first];
    // stops of the two scans over [first + 1, last); position q = lane + 64 j
    bool ls[4], rs[4];
    unsigned long long L[4], R[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = lane + 64 * j;
      const bool in = q > first && q < last;
      const uint32_t k = in ? s.key[q] : 0u;
      ls[j] = in && !(k > p);
      rs[j] = in && !(p > k);
      L[j] = __ballot(ls[j]);
      R[j] = __ballot(rs[j]);
    }
    int rl[4], rr[4], nl = 0, nr = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // left stops ranked ascending
      rl[j] = nl + __popcll(L[j] & below);
      nl += __popcll(L[j]);
    }
#pragma unroll
    for (int j = 3; j >= 0; --j) {  // right stops ranked descending
      rr[j] = nr + __popcll(R[j] & above);
      nr += __popcll(R[j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = lane + 64 * j;
      if (ls[j]) s.lpos[rl[j]] = (uint16_t)q;
      if (rs[j]) s.rpos[rr[j]] = (uint16_t)q;
    }
    // swaps: left stop k with right stop k while left < right (a prefix of the k)
    int nswap = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = lane + 64 * j;
      const bool sw = ls[j] && rl[j] < nr && (int)s.rpos[rl[j]] > q;
      nswap += __popcll(__ballot(sw));
    }
    int cut = nswap < nl ? (int)s.lpos[nswap] : last;
    if (nswap > 0) cut = min(cut, (int)s.rpos[nswap - 1]);
    uint32_t nk[4], ni[4];
    bool wr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int partner = -1;
      if (ls[j] && rl[j] < nswap) partner = (int)s.rpos[rl[j]];
      else if (rs[j] && rr[j] < nswap) partner = (int)s.lpos[rr[j]];
      wr[j] = partner >= 0;
      nk[j] = wr[j] ? s.key[partner] : 0u;
      ni[j] = wr[j] ? s.id[partner] : 0u;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = lane + 64 * j;
      if (wr[j]) {
        s.key[q] = nk[j];
        s.id[q] = ni[j];
      }
    }
    if (cut <= nth) first = cut;
    else last = cut;
  }
  if (lane == 0) tie_insertion_sort(s, first, last);
}

}  // namespace moe

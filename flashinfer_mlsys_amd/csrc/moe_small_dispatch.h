// Dispatch of up to 64 tokens inside one workgroup's LDS (reference
// moe/ref_moe.py:131-145): per local expert, the ascending list of tokens that
// selected it, the pair weights and each (token, slot)'s pair index.
//
// With T <= 64 one token fits one lane, so a 32-bit local-expert mask per token
// turns every expert's token list into one wave ballot: its popcount is the
// expert's count and the popcount below a lane is that token's rank. Used by the
// decode GEMM1 kernel (each workgroup derives the dispatch itself, so no header
// has to be read back from memory before the weight stream starts) and by the
// dispatch tap kernel.
#pragma once

#include "moe_common.h"

namespace moe {

constexpr int SMALL_T = 64;
constexpr int SMALL_P = SMALL_T * TOP_K;

struct SmallDispatch {
  int cnt[E_LOCAL];
  int seg[E_LOCAL + 1];
  int nact;
  int active[E_LOCAL];
  int ids[SMALL_P];    // routed global ids, [T, 8] ascending per token
  float wts[SMALL_P];  // their routing weights
  int tok[SMALL_P];    // pair -> token
  float pw[SMALL_P];   // pair -> routing weight
  int pair[SMALL_P];   // (token, slot) -> pair, -1 if the slot's expert is not local
  uint32_t mask[SMALL_T];
};

// The phases below are called by every thread of the workgroup (blockDim.x a
// multiple of 64 and at least SMALL_P; T <= SMALL_T) and synchronise through LDS
// only (lds_barrier), so loads in flight, such as prefetched weights, are not
// waited for.
//
// Phase 1a, from the routed ids and weights already in d.ids / d.wts and visible
// to every thread: one local-expert mask per token (bit e: local expert e).
__device__ __forceinline__ void dispatch_small_masks(int T, int offset, SmallDispatch& d) {
  const int tid = threadIdx.x;
  if (tid < SMALL_T) d.mask[tid] = 0u;
  lds_barrier();
  if (tid < T * TOP_K) {
    const unsigned le = (unsigned)(d.ids[tid] - offset);
    if (le < (unsigned)E_LOCAL) atomicOr(&d.mask[tid >> 3], 1u << le);
    d.pair[tid] = -1;
  }
  lds_barrier();
}

// The active local experts as a bit set, from the token masks (any wave, after
// dispatch_small_masks; wave-uniform result).
__device__ __forceinline__ uint32_t small_active_set(int T, const SmallDispatch& d) {
  const int lane = threadIdx.x & 63;
  uint32_t m = lane < T ? d.mask[lane] : 0u;
  m |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xF, 0xF, false);   // lane ^ 1
  m |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xF, 0xF, false);   // lane ^ 2
  m |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x141, 0xF, 0xF, false);  // half-row mirror
  m |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x140, 0xF, 0xF, false);  // row mirror
  return (uint32_t)__builtin_amdgcn_readlane((int)m, 0) | (uint32_t)__builtin_amdgcn_readlane((int)m, 16) |
         (uint32_t)__builtin_amdgcn_readlane((int)m, 32) | (uint32_t)__builtin_amdgcn_readlane((int)m, 48);
}

// Position of the n-th (from 0) set bit of a wave-uniform bit set.
__device__ __forceinline__ int nth_set_bit(uint32_t set, int n) {
  for (int j = 0; j < n; ++j) set &= set - 1u;
  return __builtin_ctz(set);
}

// Phase 1b: per-expert counts, segment starts and the active list.
__device__ __forceinline__ void dispatch_small_counts_from_masks(int T, SmallDispatch& d) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  for (int le = wave; le < E_LOCAL; le += nw) {
    const unsigned long long m = __ballot(lane < T && ((d.mask[lane] >> le) & 1u));
    if (lane == 0) d.cnt[le] = __popcll(m);
  }
  lds_barrier();
  if (wave == 0) {  // segment starts and the active list by one wave: lane e holds expert e
    const int c = lane < E_LOCAL ? d.cnt[lane] : 0;
    int incl = c;  // inclusive prefix sum over lanes
#pragma unroll
    for (int k = 1; k < E_LOCAL; k <<= 1) {
      const int y = __shfl_up(incl, k);
      if (lane >= k) incl += y;
    }
    const unsigned long long act = __ballot(lane < E_LOCAL && c > 0);
    const int nact = __popcll(act);
    if (lane < E_LOCAL) {
      d.seg[lane] = incl - c;
      if (c > 0) d.active[__popcll(act & ((1ull << lane) - 1ull))] = lane;  // ascending ids
      if (lane >= nact) d.active[lane] = -1;
    }
    if (lane == E_LOCAL - 1) {
      d.seg[E_LOCAL] = incl;
      d.nact = nact;
    }
  }
  lds_barrier();
}

// Phase 1 (1a + 1b): masks, counts, segment starts and the active list. Enough
// to know which weights the workgroup will stream.
__device__ __forceinline__ void dispatch_small_counts_lds(int T, int offset, SmallDispatch& d) {
  dispatch_small_masks(T, offset, d);
  dispatch_small_counts_from_masks(T, d);
}

// Phase 1 from routed ids and weights in memory.
__device__ __forceinline__ void dispatch_small_ids(const int32_t* __restrict__ ids, const float* __restrict__ wts,
                                                   int T, SmallDispatch& d) {
  const int tid = threadIdx.x;
  if (tid < T * TOP_K) {
    d.ids[tid] = ids[tid];
    d.wts[tid] = wts[tid];
  }
}
__device__ __forceinline__ void dispatch_small_counts(const int32_t* __restrict__ ids, const float* __restrict__ wts,
                                                      int T, int offset, SmallDispatch& d) {
  dispatch_small_ids(ids, wts, T, d);
  dispatch_small_counts_lds(T, offset, d);
}

// Phase 2: every expert's ascending token list, the pair weights and each
// (token, slot)'s pair index.
__device__ __forceinline__ void dispatch_small_lists(int T, int offset, SmallDispatch& d) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int le = wave; le < E_LOCAL; le += nw) {
    const bool has = lane < T && ((d.mask[lane] >> le) & 1u);
    const unsigned long long m = __ballot(has);
    if (has) {
      const int pos = d.seg[le] + __popcll(m & lt);
      int slot = 0;
#pragma unroll
      for (int j = 0; j < TOP_K; ++j) slot = d.ids[lane * TOP_K + j] == offset + le ? j : slot;
      d.tok[pos] = lane;
      d.pw[pos] = d.wts[lane * TOP_K + slot];
      d.pair[lane * TOP_K + slot] = pos;
    }
  }
  lds_barrier();
}

__device__ __forceinline__ void dispatch_small(const int32_t* __restrict__ ids, const float* __restrict__ wts, int T,
                                               int offset, SmallDispatch& d) {
  dispatch_small_counts(ids, wts, T, offset, d);
  dispatch_small_lists(T, offset, d);
}

// Writes the dispatch to memory in the layout of the dispatch kernels (header,
// perm_tok, perm_w, tok_pair). Called by every thread of one workgroup.
__device__ __forceinline__ void store_small_dispatch(const SmallDispatch& d, int T, DispatchHeader* __restrict__ hdr,
                                                     int32_t* __restrict__ perm_tok, float* __restrict__ perm_w,
                                                     int32_t* __restrict__ tok_pair) {
  const int tid = threadIdx.x;
  if (tid < E_LOCAL) {
    hdr->counts[tid] = d.cnt[tid];
    hdr->seg_start[tid] = d.seg[tid];
    hdr->active[tid] = d.active[tid];
  }
  if (tid == 0) {
    hdr->seg_start[E_LOCAL] = d.seg[E_LOCAL];
    hdr->n_active = d.nact;
  }
  const int P = d.seg[E_LOCAL];
  for (int p = tid; p < P; p += blockDim.x) {
    perm_tok[p] = d.tok[p];
    perm_w[p] = d.pw[p];
  }
  for (int i = tid; i < T * TOP_K; i += blockDim.x) tok_pair[i] = d.pair[i];
}

}  // namespace moe

// Dispatch of up to 128 tokens inside one workgroup's LDS (reference
// moe/ref_moe.py:131-145): per local expert, the ascending list of tokens that
// selected it, the pair weights and each (token, slot)'s pair index.
//
// Tokens sit in lanes as two halves (token lane + 64 h), so a 32-bit
// local-expert mask per token turns every expert's token list into two wave
// ballots: their popcounts are the expert's count and the popcounts below a
// lane (the first half's whole count before the second half) are that token's
// rank. With T <= 64 the second half is empty and skipped. Used by the
// decode GEMM1 kernel (each workgroup derives the dispatch itself, so no header
// has to be read back from memory before the weight stream starts) and by the
// dispatch tap kernel.
#pragma once

#include "moe_common.h"

namespace moe {

constexpr int SMALL_T = 128;  // the largest token capacity (TM below: 64 or 128)

// The LDS dispatch of at most TM tokens (TM / 64 halves of 64 tokens). The
// kernels that use it are built for TM = 64 and TM = 128 and launched with the
// smaller one that holds T, so that calls of at most 64 tokens run the
// one-half code.
template <int TM>
struct SmallDispatch {
  static_assert(TM % 64 == 0 && TM <= SMALL_T, "whole halves of 64 tokens");
  static constexpr int HALVES = TM / 64;  // token t = lane + 64 h
  static constexpr int P = TM * TOP_K;
  int cnt[E_LOCAL];
  int seg[E_LOCAL + 1];
  int nact;
  int active[E_LOCAL];
  int ids[P];    // routed global ids, [T, 8] ascending per token
  float wts[P];  // their routing weights
  int tok[P];    // pair -> token
  float pw[P];   // pair -> routing weight
  int pair[P];   // (token, slot) -> pair, -1 if the slot's expert is not local
  uint32_t mask[TM];
};

// The phases below are called by every thread of the workgroup (blockDim.x a
// multiple of 64 and at least TM; T <= TM) and synchronise through LDS
// only (lds_barrier), so loads in flight, such as prefetched weights, are not
// waited for.
//
// Phase 1a, from the routed ids and weights already in d.ids / d.wts and visible
// to every thread: one local-expert mask per token (bit e: local expert e).
template <int TM>
__device__ __forceinline__ void dispatch_small_masks(int T, int offset, SmallDispatch<TM>& d) {
  const int tid = threadIdx.x;
  if (tid < TM) d.mask[tid] = 0u;
  lds_barrier();
  for (int i = tid; i < T * TOP_K; i += blockDim.x) {
    const unsigned le = (unsigned)(d.ids[i] - offset);
    if (le < (unsigned)E_LOCAL) atomicOr(&d.mask[i >> 3], 1u << le);
    d.pair[i] = -1;
  }
  lds_barrier();
}

// The active local experts as a bit set, from the token masks (any wave, after
// dispatch_small_masks; wave-uniform result).
template <int TM>
__device__ __forceinline__ uint32_t small_active_set(int T, const SmallDispatch<TM>& d) {
  const int lane = threadIdx.x & 63;
  uint32_t m = 0u;
#pragma unroll
  for (int h = 0; h < SmallDispatch<TM>::HALVES; ++h) m |= lane + 64 * h < T ? d.mask[lane + 64 * h] : 0u;
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
template <int TM>
__device__ __forceinline__ void dispatch_small_counts_from_masks(int T, SmallDispatch<TM>& d) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  for (int le = wave; le < E_LOCAL; le += nw) {
    int c = 0;
#pragma unroll
    for (int h = 0; h < SmallDispatch<TM>::HALVES; ++h) {
      const int t = lane + 64 * h;
      c += __popcll(__ballot(t < T && ((d.mask[t] >> le) & 1u)));
    }
    if (lane == 0) d.cnt[le] = c;
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
template <int TM>
__device__ __forceinline__ void dispatch_small_counts_lds(int T, int offset, SmallDispatch<TM>& d) {
  dispatch_small_masks(T, offset, d);
  dispatch_small_counts_from_masks(T, d);
}

// Phase 1 from routed ids and weights in memory.
template <int TM>
__device__ __forceinline__ void dispatch_small_ids(const int32_t* __restrict__ ids, const float* __restrict__ wts,
                                                   int T, SmallDispatch<TM>& d) {
  for (int i = threadIdx.x; i < T * TOP_K; i += blockDim.x) {
    d.ids[i] = ids[i];
    d.wts[i] = wts[i];
  }
}
template <int TM>
__device__ __forceinline__ void dispatch_small_counts(const int32_t* __restrict__ ids, const float* __restrict__ wts,
                                                      int T, int offset, SmallDispatch<TM>& d) {
  dispatch_small_ids(ids, wts, T, d);
  dispatch_small_counts_lds(T, offset, d);
}

// Phase 2: every expert's ascending token list, the pair weights and each
// (token, slot)'s pair index.
template <int TM>
__device__ __forceinline__ void dispatch_small_lists(int T, int offset, SmallDispatch<TM>& d) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int le = wave; le < E_LOCAL; le += nw) {
    int base = d.seg[le];
    for (int h = 0; h < SmallDispatch<TM>::HALVES && 64 * h < T; ++h) {  // uniform
      const int t = lane + 64 * h;
      const bool has = t < T && ((d.mask[t] >> le) & 1u);
      const unsigned long long m = __ballot(has);
      if (has) {
        const int pos = base + __popcll(m & lt);
        int slot = 0;
#pragma unroll
        for (int j = 0; j < TOP_K; ++j) slot = d.ids[t * TOP_K + j] == offset + le ? j : slot;
        d.tok[pos] = t;
        d.pw[pos] = d.wts[t * TOP_K + slot];
        d.pair[t * TOP_K + slot] = pos;
      }
      base += __popcll(m);
    }
  }
  lds_barrier();
}

template <int TM>
__device__ __forceinline__ void dispatch_small(const int32_t* __restrict__ ids, const float* __restrict__ wts, int T,
                                               int offset, SmallDispatch<TM>& d) {
  dispatch_small_counts(ids, wts, T, offset, d);
  dispatch_small_lists(T, offset, d);
}

// Writes the dispatch to memory in the layout of the dispatch kernels (header,
// perm_tok, perm_w, tok_pair). Called by every thread of one workgroup.
template <int TM>
__device__ __forceinline__ void store_small_dispatch(const SmallDispatch<TM>& d, int T, DispatchHeader* __restrict__ hdr,
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

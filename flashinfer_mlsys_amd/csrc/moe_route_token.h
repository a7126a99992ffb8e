// One token's noaux_tc routing by one wave64 (reference moe/ref_moe.py:94-126),
// shared by the routing kernel and the decode GEMM1 kernel (which routes up to
// 8 tokens itself, one per wave, so a small decode call needs no routing launch).
#pragma once

#include "moe_common.h"

namespace moe {

// Float -> unsigned key with the same order (larger float, larger key).
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ int popc_ballot(bool p) { return __popcll(__ballot(p)); }

// Routes token t with the calling wave (ref_moe.py:94-126). Lane l holds experts
// 4l..4l+3, so the 8 lanes 8g..8g+7 hold routing group g.
//  * scores: s = 1/(1+exp(-x)) with exp(-x) evaluated in fp64 and rounded once
//    to fp32 (the correctly rounded value), IEEE fp32 division; sb = s + bias.
//  * group score = sum of the two largest sb of the group (multiset top-2 merged
//    over the group's 8 lanes); a group is kept when fewer than 4 groups beat it
//    (larger score, or equal score and lower index).
//  * the 8 experts are the 8 largest sb among the kept groups (others masked to
//    the most negative finite float): the 8th largest key is found by a 32-step
//    bitwise search on order-preserving keys with wave ballots + popcounts, then
//    every key above it is taken plus the lowest-id keys equal to it.
//  * weights = s / (sum of the 8 selected s + 1e-20) * rsf (unbiased s).
// Writes, through generic pointers (global or LDS), the ascending selected ids
// and their weights at ids[t*8 + pos], w[t*8 + pos]; tok_pair slots get -1.
__device__ __forceinline__ void route_token(const float* __restrict__ logits, const uint16_t* __restrict__ bias,
                                            int t, float rsf, int32_t* ids, float* wts, int32_t* tok_pair) {
  const int lane = threadIdx.x & 63;
  const float4 x4 = *reinterpret_cast<const float4*>(logits + (size_t)t * E_GLOBAL + 4 * lane);
  const uint2 b2 = *reinterpret_cast<const uint2*>(bias + 4 * lane);
  const float x[4] = {x4.x, x4.y, x4.z, x4.w};
  const float b[4] = {__uint_as_float(b2.x << 16), __uint_as_float(b2.x & 0xffff0000u),
                      __uint_as_float(b2.y << 16), __uint_as_float(b2.y & 0xffff0000u)};
  float s[4], sb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float e = (float)exp(-(double)x[i]);
    s[i] = 1.0f / (1.0f + e);
    sb[i] = s[i] + b[i];
  }

  float m1 = fmaxf(fmaxf(sb[0], sb[1]), fmaxf(sb[2], sb[3]));
  float m2 = fmaxf(fminf(fmaxf(sb[0], sb[1]), fmaxf(sb[2], sb[3])),
                   fmaxf(fminf(sb[0], sb[1]), fminf(sb[2], sb[3])));
#pragma unroll
  for (int k = 1; k < 8; k <<= 1) {
    const float o1 = __shfl_xor(m1, k);
    const float o2 = __shfl_xor(m2, k);
    const float n2 = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
    m1 = fmaxf(m1, o1);
    m2 = n2;
  }
  const float gscore = m1 + m2;
  const int g = lane >> 3;
  int beaten = 0;
#pragma unroll
  for (int j = 0; j < N_GROUP; ++j) {
    const float oj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gscore), j * 8));
    beaten += (oj > gscore || (oj == gscore && j < g)) ? 1 : 0;
  }
  const bool keep = beaten < TOPK_GROUP;

  uint32_t key[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) key[i] = order_key(keep ? sb[i] : -3.402823466e+38f);
  uint32_t th = 0;
#pragma unroll 4
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t trial = th | (1u << bit);
    const int c = popc_ballot(key[0] >= trial) + popc_ballot(key[1] >= trial) + popc_ballot(key[2] >= trial) +
                  popc_ballot(key[3] >= trial);
    th = c >= TOP_K ? trial : th;
  }
  const unsigned long long lt = (1ull << lane) - 1ull;
  bool sel[4], eq[4];
  int n_gt = 0, eq_below = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sel[i] = key[i] > th;
    eq[i] = key[i] == th;
    n_gt += popc_ballot(sel[i]);
    eq_below += __popcll(__ballot(eq[i]) & lt);
  }
  const int need = TOP_K - n_gt;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (eq[i]) {
      sel[i] = eq_below < need;
      ++eq_below;
    }
  }
  int pos = 0;
  float ssum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    pos += __popcll(__ballot(sel[i]) & lt);
    ssum += sel[i] ? s[i] : 0.f;
  }
#pragma unroll
  for (int k = 1; k < 64; k <<= 1) ssum += __shfl_xor(ssum, k);
  const float denom = ssum + 1e-20f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (sel[i]) {
      ids[(size_t)t * TOP_K + pos] = 4 * lane + i;
      wts[(size_t)t * TOP_K + pos] = (s[i] / denom) * rsf;
      ++pos;
    }
  }
  if (tok_pair && lane < TOP_K) tok_pair[(size_t)t * TOP_K + lane] = -1;
}

}  // namespace moe

// One token's noaux_tc routing by one wave64 (reference moe/ref_moe.py:94-126),
// shared by the routing kernel and the decode GEMM1 kernel (which routes up to
// 8 tokens itself, one per wave, so a small decode call needs no routing launch).
#pragma once

#include "moe_common.h"
#include "moe_route_ties.h"

namespace moe {

// Float -> unsigned key with the same order (larger float, larger key).
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ int popc_ballot(bool p) { return __popcll(__ballot(p)); }

// DPP lane moves within rows of 16 (gfx9 encodings): quad_perm [1,0,3,2] and
// [2,3,0,1] are lane ^ 1 and lane ^ 2; half-row mirror maps lane i of each 8-lane
// half to 7 - i; row mirror maps lane i of each row to 15 - i.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// Compare-exchange of (key, slot) pairs into (larger key, or equal key and lower slot) first.
__device__ __forceinline__ void cx(uint32_t& ka, int& ia, uint32_t& kb, int& ib) {
  const bool sw = kb > ka || (kb == ka && ib < ia);
  const uint32_t k = sw ? kb : ka, l = sw ? ka : kb;
  const int i = sw ? ib : ia, j = sw ? ia : ib;
  ka = k; kb = l; ia = i; ib = j;
}

// Routes token t with the calling wave (ref_moe.py:94-126). Lane l holds experts
// 4l..4l+3, so the 8 lanes 8g..8g+7 hold routing group g.
//  * scores: s = 1/(1+exp(-x)) with exp(-x) evaluated in fp64 and rounded once
//    to fp32 (the correctly rounded value), IEEE fp32 division; sb = s + bias.
//  * group score = sum of the two largest sb of the group (multiset top-2 merged
//    over the group's 8 lanes); the 4 groups with the largest scores are kept.
//  * the 8 experts are the 8 largest sb among the kept groups (others masked to
//    the most negative finite float): each lane sorts its 4 order-preserving keys
//    (larger first); 8 rounds then take the wave maximum of the lanes' first keys,
//    and a lane holding it selects that expert and drops it from its list.
//  * when equal scores straddle a cut (the 4th and 5th group scores, or the 8th
//    and 9th expert keys, are equal) the kept set is not fixed by the values
//    alone; the reference's torch.topk(sorted=False) then keeps the entries
//    std::nth_element leaves in front, and the wave reproduces that order
//    (wave_nth_element) in `tie`, a 3 KB LDS scratch of its own.
//  * weights = s / (sum of the 8 selected s + 1e-20) * rsf (unbiased s).
// Writes, through generic pointers (global or LDS), the ascending selected ids
// and their weights at ids[t*8 + pos], w[t*8 + pos]; tok_pair slots get -1.
__device__ __forceinline__ void route_token(const float* __restrict__ logits, const uint16_t* __restrict__ bias,
                                            int t, float rsf, int32_t* ids, float* wts, int32_t* tok_pair,
                                            TieScratch* tie) {
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
  // merge (largest, second largest) with lane ^ 1, lane ^ 2, then the mirrored
  // half-row partner: every lane of the 8-lane group ends with the group's top 2
  // (max and min only, so the result does not depend on the merge order).
  auto merge = [&](float o1, float o2) {
    const float n2 = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
    m1 = fmaxf(m1, o1);
    m2 = n2;
  };
  merge(dpp_f<DPP_XOR1>(m1), dpp_f<DPP_XOR1>(m2));
  merge(dpp_f<DPP_XOR2>(m1), dpp_f<DPP_XOR2>(m2));
  merge(dpp_f<DPP_HALF_MIRROR>(m1), dpp_f<DPP_HALF_MIRROR>(m2));
  const float gscore = m1 + m2;
  const int g = lane >> 3;
  int above = 0, equal = 0;  // groups with a larger / the same score (this one included)
#pragma unroll
  for (int j = 0; j < N_GROUP; ++j) {
    const float oj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gscore), j * 8));
    above += oj > gscore ? 1 : 0;
    equal += oj == gscore ? 1 : 0;
  }
  bool keep = above < TOPK_GROUP;
  if (__ballot(above < TOPK_GROUP && above + equal > TOPK_GROUP)) {  // equal scores straddle the cut
    VTie& s = lds_tie(tie);
    if ((lane & 7) == 0) {
      s.key[g] = order_key(gscore);
      s.id[g] = (uint32_t)g;
    }
    wave_nth_element(s, N_GROUP, TOPK_GROUP - 1);
    keep = false;
#pragma unroll
    for (int j = 0; j < TOPK_GROUP; ++j) keep |= (int)s.id[j] == g;
  }

  // keys of finite floats are >= 0x00800000, so 0 marks an emptied list entry
  uint32_t key[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) key[i] = order_key(keep ? sb[i] : -3.402823466e+38f);
  uint32_t k0 = key[0], k1 = key[1], k2 = key[2], k3 = key[3];
  int i0 = 0, i1 = 1, i2 = 2, i3 = 3;
  cx(k0, i0, k1, i1);
  cx(k2, i2, k3, i3);
  cx(k0, i0, k2, i2);
  cx(k1, i1, k3, i3);
  cx(k1, i1, k2, i2);
  // wave maximum of the lists' first keys: within rows of 16, then the 4 rows
  auto wave_max = [&](uint32_t m) {
    m = max(m, dpp_u<DPP_XOR1>(m));
    m = max(m, dpp_u<DPP_XOR2>(m));
    m = max(m, dpp_u<DPP_HALF_MIRROR>(m));
    m = max(m, dpp_u<DPP_MIRROR>(m));
    return max(max((uint32_t)__builtin_amdgcn_readlane((int)m, 0), (uint32_t)__builtin_amdgcn_readlane((int)m, 16)),
               max((uint32_t)__builtin_amdgcn_readlane((int)m, 32), (uint32_t)__builtin_amdgcn_readlane((int)m, 48)));
  };
  uint32_t selmask = 0;  // bit i: this lane's expert 4 lane + i is selected
  uint32_t mx = 0;
#pragma unroll
  for (int r = 0; r < TOP_K; ++r) {
    mx = wave_max(k0);
    const int win = __builtin_ctzll(__ballot(k0 == mx));  // one lane holding the maximum
    if (lane == win) {
      selmask |= 1u << i0;
      k0 = k1; i0 = i1;
      k1 = k2; i1 = i2;
      k2 = k3; i2 = i3;
      k3 = 0u;
    }
  }
  if (wave_max(k0) == mx) {  // the 9th largest key equals the 8th: a tie straddles the cut
    VTie& s = lds_tie(tie);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s.key[4 * lane + i] = key[i];
      s.id[4 * lane + i] = (uint32_t)(4 * lane + i);
    }
    wave_nth_element(s, E_GLOBAL, TOP_K - 1);
    selmask = 0;
#pragma unroll
    for (int j = 0; j < TOP_K; ++j) {
      const uint32_t e = s.id[j];
      if ((int)(e >> 2) == lane) selmask |= 1u << (e & 3u);
    }
  }
  bool sel[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sel[i] = (selmask >> i) & 1u;
  const unsigned long long lt = (1ull << lane) - 1ull;
  int pos = 0;
  float ssum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    pos += __popcll(__ballot(sel[i]) & lt);
    ssum += sel[i] ? s[i] : 0.f;
  }
  // sum over the wave: within each row of 16 (every lane of the row ends with the
  // same value), then the four row sums in row order
  ssum += dpp_f<DPP_XOR1>(ssum);
  ssum += dpp_f<DPP_XOR2>(ssum);
  ssum += dpp_f<DPP_HALF_MIRROR>(ssum);
  ssum += dpp_f<DPP_MIRROR>(ssum);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ssum), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ssum), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ssum), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ssum), 48));
  const float denom = ((r0 + r1) + (r2 + r3)) + 1e-20f;
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

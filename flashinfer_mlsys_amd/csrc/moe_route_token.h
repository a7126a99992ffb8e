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

// The routing score s = 1/(1+exp(-x)): exact_sigmoid takes exp(-x) in fp64
// rounded once to fp32 (the correctly rounded value) and an IEEE fp32 division;
// fast_sigmoid uses the hardware's v_exp_f32 and v_rcp_f32, within 1.5 * 2^-23
// of exact_sigmoid over every fp32 input on gfx950 (an exhaustive check).
__device__ __forceinline__ float exact_sigmoid(float x) { return 1.0f / (1.0f + (float)exp(-(double)x)); }

__device__ __forceinline__ float fast_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}

// Compare-exchange of (key, slot) pairs into (larger key, or equal key and lower slot) first.
__device__ __forceinline__ void cx(uint32_t& ka, int& ia, uint32_t& kb, int& ib) {
  const bool sw = kb > ka || (kb == ka && ib < ia);
  const uint32_t k = sw ? kb : ka, l = sw ? ka : kb;
  const int i = sw ? ib : ia, j = sw ? ia : ib;
  ka = k; kb = l; ia = i; ib = j;
}

// Exact routing of token t by the calling wave (ref_moe.py:94-126). Lane l holds
// experts 4l..4l+3, so the 8 lanes 8g..8g+7 hold routing group g.
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
__device__ __forceinline__ void route_token_exact(const float* __restrict__ logits, const uint16_t* __restrict__ bias,
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
    s[i] = exact_sigmoid(x[i]);
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
  int pos0 = 0;  // selected experts of the lanes below: this lane's first position
#pragma unroll
  for (int i = 0; i < 4; ++i) pos0 += __popcll(__ballot(sel[i]) & lt);
  // the denominator: the 8 selected s gathered in ascending id order (through the
  // scratch), summed by the tree ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7))
  // in every 8-lane slice, the same sum as the fast path's, so a token's weights
  // do not depend on which path routed it
  VTie& sc = lds_tie(tie);
  {
    int pos = pos0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (sel[i]) {
        sc.key[pos] = __float_as_uint(s[i]);
        ++pos;
      }
    }
  }
  float ssum = __uint_as_float(sc.key[lane & (TOP_K - 1)]);
  ssum += dpp_f<DPP_XOR1>(ssum);
  ssum += dpp_f<DPP_XOR2>(ssum);
  ssum += dpp_f<DPP_HALF_MIRROR>(ssum);
  const float denom = ssum + 1e-20f;
  int pos = pos0;
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

// Wave-wide maximum / minimum of an unsigned value: within rows of 16 lanes, then
// row_bcast:15 (rows 1 and 3 take lane 15 of the row before) and row_bcast:31
// (rows 2 and 3 take lane 31) carry the row results up to lane 63. The rows a
// broadcast does not write keep their value (the destination is the source).
#define MOE_BCAST_STEP(op, m, ctrl, rows) \
  asm("s_nop 1\n\t" op " %0, %0, %0 " ctrl " row_mask:" rows " bank_mask:0xf" : "+v"(m))

__device__ __forceinline__ uint32_t wave_umax(uint32_t m) {
  m = max(m, dpp_u<DPP_XOR1>(m));
  m = max(m, dpp_u<DPP_XOR2>(m));
  m = max(m, dpp_u<DPP_HALF_MIRROR>(m));
  m = max(m, dpp_u<DPP_MIRROR>(m));
  MOE_BCAST_STEP("v_max_u32_dpp", m, "row_bcast:15", "0xa");
  MOE_BCAST_STEP("v_max_u32_dpp", m, "row_bcast:31", "0xc");
  return (uint32_t)__builtin_amdgcn_readlane((int)m, 63);
}

__device__ __forceinline__ uint32_t wave_umin(uint32_t m) {
  m = min(m, dpp_u<DPP_XOR1>(m));
  m = min(m, dpp_u<DPP_XOR2>(m));
  m = min(m, dpp_u<DPP_HALF_MIRROR>(m));
  m = min(m, dpp_u<DPP_MIRROR>(m));
  MOE_BCAST_STEP("v_min_u32_dpp", m, "row_bcast:15", "0xa");
  MOE_BCAST_STEP("v_min_u32_dpp", m, "row_bcast:31", "0xc");
  return (uint32_t)__builtin_amdgcn_readlane((int)m, 63);
}

// Inverse of order_key.
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Descending compare-exchange of two keys.
__device__ __forceinline__ void cx_desc(uint32_t& a, uint32_t& b) {
  const uint32_t hi = max(a, b), lo = min(a, b);
  a = hi;
  b = lo;
}

// Routing of token t with a fast sigmoid, for the tokens whose selection the
// fast scores provably share with the exact ones (ref_moe.py:94-126; the exact
// rule is route_token_exact's). Returns false, having written nothing, for the
// others.
//  * s' = fast_sigmoid(x), within 1.5 * 2^-23 of the exact s for every fp32 x;
//    the bound used below is 2^-20. With M = max |s' + bias| over the
//    token, every sb' = s' + bias lies within D = 2^-19 + 2^-22 M of its exact sb
//    (both sums round once), and a group score (the top-2 sum, which moves by at
//    most the two top entries' D, plus its rounding) within 2^-18 + 2^-20 M.
//  * the group cut and the expert cut are taken on the fast scores; when the 4th
//    and 5th group scores differ by more than twice the group bound and the 8th
//    and 9th expert scores by more than twice D, the exact scores keep the same
//    groups and the same 8 experts. Otherwise (near or exact ties, non-finite
//    scores) the token goes to the exact path.
//  * group cut: the 8 group keys are sorted on the scalar unit (19 exchanges).
//  * expert cut: the 8 top-2 entries of the kept groups are 8 distinct experts,
//    so the 8th largest score is at least theta, the smallest of them. The C keys
//    >= theta are the candidates; the C - 8 smallest are dropped one per round
//    (wave minimum of each lane's smallest candidate), so the 8th key is the
//    smallest remaining and the 9th the last one dropped (or, when C = 8, the
//    largest key below theta). More than 20 extra candidates: exact path.
//  * weights: the 8 selected logits are gathered into lanes 0-7 in ascending id
//    order (LDS), whose exact s (the exact path's rule) and sum give the weights.
__device__ __forceinline__ bool route_token_fast(const float* __restrict__ logits, const uint16_t* __restrict__ bias,
                                                 int t, float rsf, int32_t* ids, float* wts, int32_t* tok_pair,
                                                 TieScratch* tie) {
  const int lane = threadIdx.x & 63;
  const float4 x4 = *reinterpret_cast<const float4*>(logits + (size_t)t * E_GLOBAL + 4 * lane);
  const uint2 b2 = *reinterpret_cast<const uint2*>(bias + 4 * lane);
  const float x[4] = {x4.x, x4.y, x4.z, x4.w};
  const float b[4] = {__uint_as_float(b2.x << 16), __uint_as_float(b2.x & 0xffff0000u),
                      __uint_as_float(b2.y << 16), __uint_as_float(b2.y & 0xffff0000u)};
  float sb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sb[i] = fast_sigmoid(x[i]) + b[i];
  }
  bool finite = true;  // (a NaN fails the compare)
#pragma unroll
  for (int i = 0; i < 4; ++i) finite &= fabsf(sb[i]) <= 3.0e38f;
  if (__ballot(!finite)) return false;
  const float amax = fmaxf(fmaxf(fabsf(sb[0]), fabsf(sb[1])), fmaxf(fabsf(sb[2]), fabsf(sb[3])));
  const float M = __uint_as_float(wave_umax(__float_as_uint(amax)));  // finite, >= 0: bits order as values

  // group top-2 (multiset), merged over the group's 8 lanes
  float m1 = fmaxf(fmaxf(sb[0], sb[1]), fmaxf(sb[2], sb[3]));
  float m2 = fmaxf(fminf(fmaxf(sb[0], sb[1]), fmaxf(sb[2], sb[3])),
                   fmaxf(fminf(sb[0], sb[1]), fminf(sb[2], sb[3])));
  auto merge = [&](float o1, float o2) {
    const float n2 = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
    m1 = fmaxf(m1, o1);
    m2 = n2;
  };
  merge(dpp_f<DPP_XOR1>(m1), dpp_f<DPP_XOR1>(m2));
  merge(dpp_f<DPP_XOR2>(m1), dpp_f<DPP_XOR2>(m2));
  merge(dpp_f<DPP_HALF_MIRROR>(m1), dpp_f<DPP_HALF_MIRROR>(m2));
  const uint32_t gk = order_key(m1 + m2);
  uint32_t k[N_GROUP];
#pragma unroll
  for (int j = 0; j < N_GROUP; ++j) k[j] = (uint32_t)__builtin_amdgcn_readlane((int)gk, 8 * j);
  // descending sorting network on the scalar unit
  cx_desc(k[0], k[2]); cx_desc(k[1], k[3]); cx_desc(k[4], k[6]); cx_desc(k[5], k[7]);
  cx_desc(k[0], k[4]); cx_desc(k[1], k[5]); cx_desc(k[2], k[6]); cx_desc(k[3], k[7]);
  cx_desc(k[0], k[1]); cx_desc(k[2], k[3]); cx_desc(k[4], k[5]); cx_desc(k[6], k[7]);
  cx_desc(k[2], k[4]); cx_desc(k[3], k[5]);
  cx_desc(k[1], k[4]); cx_desc(k[3], k[6]);
  cx_desc(k[1], k[2]); cx_desc(k[3], k[4]); cx_desc(k[5], k[6]);
  const uint32_t k4 = k[TOPK_GROUP - 1], k5 = k[TOPK_GROUP];
  if (!(key_value(k4) - key_value(k5) > 0x1p-17f + 0x1p-18f * M)) return false;
  const bool keep = gk >= k4;  // exactly the 4 groups above the cut

  uint32_t key[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) key[i] = keep ? order_key(sb[i]) : 0x00800000u;  // order_key(-FLT_MAX)
  uint32_t k0 = key[0], k1 = key[1], k2 = key[2], k3 = key[3];
  cx_desc(k0, k1);
  cx_desc(k2, k3);
  cx_desc(k0, k2);
  cx_desc(k1, k3);
  cx_desc(k1, k2);
  const uint32_t theta = wave_umin(keep ? order_key(m2) : 0xffffffffu);
  const bool c0 = k0 >= theta, c1 = k1 >= theta, c2 = k2 >= theta, c3 = k3 >= theta;
  const int C = popc_ballot(c0) + popc_ballot(c1) + popc_ballot(c2) + popc_ballot(c3);
  int cl = (int)c0 + (int)c1 + (int)c2 + (int)c3;  // this lane's candidates: k0..k(cl-1)
  // all-ones where entry i is a candidate (i < cl); selects without branches
  auto cmask = [&](int i) { return (uint32_t)((i - cl) >> 31); };
  auto smallest = [&]() {  // the lane's smallest candidate (all-ones without one)
    return min(min(k0 | ~cmask(0), k1 | ~cmask(1)), min(k2 | ~cmask(2), k3 | ~cmask(3)));
  };
  uint32_t k8, k9;
  if (C == TOP_K) {
    k8 = theta;
    k9 = wave_umax(max(max(k0 & ~cmask(0), k1 & ~cmask(1)), max(k2 & ~cmask(2), k3 & ~cmask(3))));
  } else {
    if (C > TOP_K + 20) return false;
    uint32_t mn = 0;
    for (int r = TOP_K; r < C; ++r) {  // uniform trip count
      const uint32_t sm = smallest();
      mn = wave_umin(sm);
      const int win = __builtin_ctzll(__ballot(sm == mn));
      cl -= lane == win ? 1 : 0;
    }
    k9 = mn;
    k8 = wave_umin(smallest());
  }
  const float a8 = key_value(k8), a9 = key_value(k9);
  if (!(a8 - a9 > 0x1p-18f + 0x1p-21f * M)) return false;

  // the 8 selected (keys >= k8), gathered in ascending id order into lanes 0-7
  bool sel[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) sel[i] = key[i] >= k8;
  int pos = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) pos += __popcll(__ballot(sel[i]) & ((1ull << lane) - 1ull));
  VTie& sc = lds_tie(tie);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (sel[i]) {
      sc.key[pos] = __float_as_uint(x[i]);
      sc.id[pos] = (uint32_t)(4 * lane + i);
      ++pos;
    }
  }
  const int j = lane & (TOP_K - 1);
  const float xj = __uint_as_float(sc.key[j]);
  const int idj = (int)sc.id[j];
  const float sj = exact_sigmoid(xj);
  // the 8-lane tree ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7)) (each 8-lane
  // slice holds the same 8 values), as the exact path sums them
  float ssum = sj;
  ssum += dpp_f<DPP_XOR1>(ssum);
  ssum += dpp_f<DPP_XOR2>(ssum);
  ssum += dpp_f<DPP_HALF_MIRROR>(ssum);
  if (lane < TOP_K) {
    ids[(size_t)t * TOP_K + lane] = idj;
    wts[(size_t)t * TOP_K + lane] = (sj / (ssum + 1e-20f)) * rsf;
    if (tok_pair) tok_pair[(size_t)t * TOP_K + lane] = -1;
  }
  return true;
}

// Routes token t with the calling wave (ref_moe.py:94-126). FAST: the fast path
// where it provably selects what the exact rule selects, the exact path
// otherwise; it issues about half the exact path's instructions but its chain of
// dependent steps is longer, so it pays where many tokens share each SIMD (large
// T) and the exact path alone is quicker for a few tokens.
template <bool FAST>
__device__ __forceinline__ void route_token(const float* __restrict__ logits, const uint16_t* __restrict__ bias,
                                            int t, float rsf, int32_t* ids, float* wts, int32_t* tok_pair,
                                            TieScratch* tie) {
  if (!FAST || !route_token_fast(logits, bias, t, rsf, ids, wts, tok_pair, tie))
    route_token_exact(logits, bias, t, rsf, ids, wts, tok_pair, tie);
}

}  // namespace moe

// noaux_tc routing and per-expert dispatch for the FP8 DeepSeek-V3 MoE operator.
//
// route_kernel     -- reference moe/ref_moe.py:94-126 (sigmoid + bias, top-2-sum
//                     group scores, top-4 of 8 groups, top-8 experts inside them,
//                     weights from the unbiased sigmoid normalised over the 8 and
//                     scaled). One wave64 per token, 4 experts per lane; the
//                     top-8 is a ballot/popcount threshold search (no serial
//                     arg-max rounds).
// dispatch_kernel  -- reference moe/ref_moe.py:131-145 (for each local expert the
//                     ascending list of tokens that selected it). One workgroup
//                     per local expert: a histogram of all local ids gives every
//                     segment's start, then a ballot/popcount scan writes the
//                     expert's tokens in ascending order. No atomics on global
//                     memory, no host synchronisation.
// dispatch_small_kernel -- the decode-size dispatch (T <= 64) in one workgroup.
#include "moe_common.h"
#include "moe_small_dispatch.h"

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

__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits,
                                                    const uint16_t* __restrict__ bias, int T, float rsf,
                                                    int32_t* __restrict__ topk_ids, float* __restrict__ topk_w,
                                                    int32_t* __restrict__ tok_pair) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  route_token(logits, bias, t, rsf, topk_ids, topk_w, tok_pair);
}

// One workgroup per local expert (grid = 32). See the file comment.
__global__ __launch_bounds__(256) void dispatch_kernel(const int32_t* __restrict__ topk_ids,
                                                       const float* __restrict__ topk_w, int T, int offset,
                                                       DispatchHeader* __restrict__ hdr,
                                                       int32_t* __restrict__ perm_tok, float* __restrict__ perm_w,
                                                       int32_t* __restrict__ tok_pair) {
  __shared__ int hist[E_LOCAL];
  __shared__ int wave_cnt[4];
  __shared__ int seg_base;
  const int le = blockIdx.x;
  const int ge = offset + le;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid < E_LOCAL) hist[tid] = 0;
  __syncthreads();
  for (int t = tid; t < T; t += 256) {
    const int4* row = reinterpret_cast<const int4*>(topk_ids + (size_t)t * TOP_K);
    const int4 a = row[0], b = row[1];
    const int v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < TOP_K; ++j) {
      const unsigned l = (unsigned)(v[j] - offset);
      if (l < (unsigned)E_LOCAL) atomicAdd(&hist[l], 1);
    }
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0, nact = 0;
    for (int e = 0; e < E_LOCAL; ++e) {
      if (e == le) seg_base = acc;
      if (le == 0) {
        hdr->counts[e] = hist[e];
        hdr->seg_start[e] = acc;
        if (hist[e] > 0) hdr->active[nact++] = e;
      }
      acc += hist[e];
    }
    if (le == 0) {
      hdr->seg_start[E_LOCAL] = acc;
      hdr->n_active = nact;
      for (int e = nact; e < E_LOCAL; ++e) hdr->active[e] = -1;
    }
  }
  __syncthreads();
  int base = seg_base;
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  for (int t0 = 0; t0 < T; t0 += 256) {
    const int t = t0 + tid;
    int slot = -1;
    if (t < T) {
      const int4* row = reinterpret_cast<const int4*>(topk_ids + (size_t)t * TOP_K);
      const int4 a = row[0], b = row[1];
      const int v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < TOP_K; ++j) slot = v[j] == ge ? j : slot;
    }
    const unsigned long long m = __ballot(slot >= 0);
    if (lane == 0) wave_cnt[wave] = __popcll(m);
    __syncthreads();
    int wbase = 0, total = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      wbase += w < wave ? wave_cnt[w] : 0;
      total += wave_cnt[w];
    }
    if (slot >= 0) {
      const int pos = base + wbase + __popcll(m & lt_mask);
      perm_tok[pos] = t;
      perm_w[pos] = topk_w[(size_t)t * TOP_K + slot];
      tok_pair[(size_t)t * TOP_K + slot] = pos;
    }
    base += total;
    __syncthreads();
  }
}


// Dispatch of up to 64 tokens in one workgroup with the same device code the
// decode GEMM1 kernel runs in each of its workgroups (dispatch tap).
__global__ __launch_bounds__(SMALL_P) void dispatch_small_kernel(const int32_t* __restrict__ topk_ids,
                                                                 const float* __restrict__ topk_w, int T, int offset,
                                                                 DispatchHeader* __restrict__ hdr,
                                                                 int32_t* __restrict__ perm_tok,
                                                                 float* __restrict__ perm_w,
                                                                 int32_t* __restrict__ tok_pair) {
  __shared__ SmallDispatch d;
  dispatch_small(topk_ids, topk_w, T, offset, d);
  store_small_dispatch(d, T, hdr, perm_tok, perm_w, tok_pair);
}

}  // namespace moe

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
namespace moe {

hipError_t launch_route(const float* logits, const uint16_t* bias, int T, float rsf, int32_t* topk_ids,
                        float* topk_w, int32_t* tok_pair, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(route_kernel, dim3((T + 3) / 4), dim3(256), 0, stream, logits, bias, T, rsf, topk_ids,
                     topk_w, tok_pair);
  return hipGetLastError();
}

hipError_t launch_dispatch_small(const int32_t* topk_ids, const float* topk_w, int T, int offset,
                                 DispatchHeader* hdr, int32_t* perm_tok, float* perm_w, int32_t* tok_pair,
                                 hipStream_t stream) {
  if (T <= 0 || T > SMALL_T) return hipErrorInvalidValue;
  hipLaunchKernelGGL(dispatch_small_kernel, dim3(1), dim3(SMALL_P), 0, stream, topk_ids, topk_w, T, offset, hdr,
                     perm_tok, perm_w, tok_pair);
  return hipGetLastError();
}

hipError_t launch_dispatch(const int32_t* topk_ids, const float* topk_w, int T, int offset, DispatchHeader* hdr,
                           int32_t* perm_tok, float* perm_w, int32_t* tok_pair, hipStream_t stream) {
  hipLaunchKernelGGL(dispatch_kernel, dim3(E_LOCAL), dim3(256), 0, stream, topk_ids, topk_w, T, offset, hdr,
                     perm_tok, perm_w, tok_pair);
  return hipGetLastError();
}

}  // namespace moe

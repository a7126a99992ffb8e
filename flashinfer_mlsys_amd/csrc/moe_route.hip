// noaux_tc routing and per-expert dispatch for the FP8 DeepSeek-V3 MoE operator.
//
// route_kernel     -- reference moe/ref_moe.py:94-126 (sigmoid + bias, top-2-sum
//                     group scores, top-4 of 8 groups, top-8 experts inside them,
//                     weights from the unbiased sigmoid normalised over the 8 and
//                     scaled). One wave64 per token, 4 experts per lane, 8 lanes
//                     per 32-expert group; the choices are made with cross-lane
//                     shuffles, no LDS.
// dispatch_kernel  -- reference moe/ref_moe.py:131-145 (for each local expert the
//                     ascending list of tokens that selected it). One workgroup
//                     per local expert: a histogram of all local ids gives every
//                     segment's start, then a ballot/popcount scan writes the
//                     expert's tokens in ascending order. No atomics on global
//                     memory, no host synchronisation.
#include "moe_common.h"

namespace moe {

// Selection key order: larger value first, lower expert id on equal values.
__device__ __forceinline__ bool beats(float v, int i, float ov, int oi) {
  return ov > v || (ov == v && oi < i);
}

__device__ __forceinline__ float pick4(const float (&a)[4], int k) {
  float r = a[0];
  r = k == 1 ? a[1] : r;
  r = k == 2 ? a[2] : r;
  r = k == 3 ? a[3] : r;
  return r;
}

// Routes token t with the calling wave. Lanes 0..7 store slot `lane` of the
// ascending selection: expert id, routing weight, and -1 into tok_pair (the
// dispatch kernel overwrites the slots of local experts).
__device__ __forceinline__ void route_token(const float* __restrict__ logits, const uint16_t* __restrict__ bias,
                                            int t, float rsf, int32_t* __restrict__ topk_ids,
                                            float* __restrict__ topk_w, int32_t* __restrict__ tok_pair) {
  const int lane = threadIdx.x & 63;
  const float4 x4 = *reinterpret_cast<const float4*>(logits + (size_t)t * E_GLOBAL + 4 * lane);
  const uint2 b2 = *reinterpret_cast<const uint2*>(bias + 4 * lane);
  const float x[4] = {x4.x, x4.y, x4.z, x4.w};
  const float b[4] = {__uint_as_float(b2.x << 16), __uint_as_float(b2.x & 0xffff0000u),
                      __uint_as_float(b2.y << 16), __uint_as_float(b2.y & 0xffff0000u)};
  float s[4], sb[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // exp(-x) rounded once to fp32 (evaluated in fp64), then 1/(1+e) in fp32
    // with IEEE division: the correctly rounded form of ref_moe.py:99.
    const float e = (float)exp(-(double)x[i]);
    s[i] = 1.0f / (1.0f + e);
    sb[i] = s[i] + b[i];
  }

  // Group score = sum of the two largest biased scores of the 32-expert group
  // (ref_moe.py:106-108). Multiset top-2 merged across the group's 8 lanes.
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

  // Top-4 of the 8 group scores (ref_moe.py:110-114): keep a group when fewer
  // than 4 groups beat it.
  const int g = lane >> 3;
  int rank = 0;
#pragma unroll
  for (int j = 0; j < N_GROUP; ++j) {
    const float oj = __shfl(gscore, j * 8);
    rank += beats(gscore, g, oj, j) ? 1 : 0;
  }
  const bool keep = rank < TOPK_GROUP;

  // Top-8 of the biased scores inside the kept groups, others masked to the
  // most negative finite float (ref_moe.py:116-119). Eight rounds of a
  // wave-wide arg-max; the winner's lane retires that candidate.
  float cand[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) cand[i] = keep ? sb[i] : -3.402823466e+38f;
  unsigned taken = 0;
  int sel_id[TOP_K];
  float sel_s[TOP_K];
#pragma unroll
  for (int r = 0; r < TOP_K; ++r) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (!(taken & (1u << i)) && beats(bv, bi, cand[i], 4 * lane + i)) {
        bv = cand[i];
        bi = 4 * lane + i;
      }
    }
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) {
      const float ov = __shfl_xor(bv, k);
      const int oi = __shfl_xor(bi, k);
      if (beats(bv, bi, ov, oi)) {
        bv = ov;
        bi = oi;
      }
    }
    if ((bi >> 2) == lane) taken |= 1u << (bi & 3);
    sel_id[r] = bi;
    sel_s[r] = __shfl(pick4(s, bi & 3), bi >> 2);
  }

  // Ascending expert ids (the canonical order of a selected set).
#pragma unroll
  for (int a = 1; a < TOP_K; ++a) {
#pragma unroll
    for (int c = a; c > 0; --c) {
      if (sel_id[c] < sel_id[c - 1]) {
        const int ti = sel_id[c]; sel_id[c] = sel_id[c - 1]; sel_id[c - 1] = ti;
        const float ts = sel_s[c]; sel_s[c] = sel_s[c - 1]; sel_s[c - 1] = ts;
      }
    }
  }
  // Weights from the unbiased scores over all 8 selected experts (ref_moe.py:121-126).
  float sum = 0.f;
#pragma unroll
  for (int r = 0; r < TOP_K; ++r) sum += sel_s[r];
  const float denom = sum + 1e-20f;

  if (lane < TOP_K) {
    int my_id = sel_id[0];
    float my_s = sel_s[0];
#pragma unroll
    for (int r = 1; r < TOP_K; ++r) {
      my_id = lane == r ? sel_id[r] : my_id;
      my_s = lane == r ? sel_s[r] : my_s;
    }
    topk_ids[(size_t)t * TOP_K + lane] = my_id;
    topk_w[(size_t)t * TOP_K + lane] = (my_s / denom) * rsf;
    if (tok_pair) tok_pair[(size_t)t * TOP_K + lane] = -1;
  }
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

hipError_t launch_dispatch(const int32_t* topk_ids, const float* topk_w, int T, int offset, DispatchHeader* hdr,
                           int32_t* perm_tok, float* perm_w, int32_t* tok_pair, hipStream_t stream) {
  hipLaunchKernelGGL(dispatch_kernel, dim3(E_LOCAL), dim3(256), 0, stream, topk_ids, topk_w, T, offset, hdr,
                     perm_tok, perm_w, tok_pair);
  return hipGetLastError();
}

}  // namespace moe

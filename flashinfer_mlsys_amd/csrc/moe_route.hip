// noaux_tc routing and per-expert dispatch for the FP8 DeepSeek-V3 MoE operator.
//
// route_kernel     -- reference moe/ref_moe.py:94-126 (sigmoid + bias, top-2-sum
//                     group scores, top-4 of 8 groups, top-8 experts inside them,
//                     weights from the unbiased sigmoid normalised over the 8 and
//                     scaled). One wave64 per token, 4 experts per lane; the
//                     top-8 by 8 rounds of wave arg-max, and the reference's
//                     nth_element order where equal keys straddle a cut
//                     (moe_route_token.h, moe_route_ties.h).
// dispatch_kernel  -- reference moe/ref_moe.py:131-145 (for each local expert the
//                     ascending list of tokens that selected it). One workgroup
//                     per local expert: a histogram of all local ids gives every
//                     segment's start, then a ballot/popcount scan writes the
//                     expert's tokens in ascending order. No atomics on global
//                     memory, no host synchronisation.
// dispatch_small_kernel -- the decode-size dispatch (T <= 64) in one workgroup.
#include "moe_common.h"
#include "moe_route_token.h"
#include "moe_small_dispatch.h"

namespace moe {

__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits,
                                                    const uint16_t* __restrict__ bias, int T, float rsf,
                                                    int32_t* __restrict__ topk_ids, float* __restrict__ topk_w,
                                                    int32_t* __restrict__ tok_pair) {
  __shared__ TieScratch tie[4];
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  route_token(logits, bias, t, rsf, topk_ids, topk_w, tok_pair, &tie[threadIdx.x >> 6]);
}

// One workgroup per local expert (grid = 32): each walks all T tokens in
// 256-token steps (two barriers per step), so its time grows with T; used
// above DISPATCH_CHUNKED_MAX_T tokens, where dispatch_chunked_kernel's total
// work (which grows with T^2) would be larger.
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

// One workgroup per 512-token chunk (grid = ceil(T / 512)), all chunks in
// parallel and with no scratch memory: every workgroup histograms the local
// ids of all T tokens (totals -> segment starts) and of the tokens before its
// chunk (its offset inside each segment), then ranks its own tokens per expert
// with one wave ballot per expert and a prefix over its 8 waves. Within each
// expert the tokens stay in ascending order (reference ref_moe.py:131-145).
// Workgroup 0 writes the header.
constexpr int DISPATCH_CHUNK = 512;
constexpr int DISPATCH_CHUNKED_MAX_T = 131072;

__global__ __launch_bounds__(DISPATCH_CHUNK) void dispatch_chunked_kernel(
    const int32_t* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int offset,
    DispatchHeader* __restrict__ hdr, int32_t* __restrict__ perm_tok, float* __restrict__ perm_w,
    int32_t* __restrict__ tok_pair) {
  constexpr int NW = DISPATCH_CHUNK / 64;
  __shared__ int hist_all[E_LOCAL], hist_pre[E_LOCAL], seg[E_LOCAL];
  __shared__ unsigned long long wmask[NW][E_LOCAL];  // per wave and expert: lanes whose token selected it
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t0 = blockIdx.x * DISPATCH_CHUNK;
  if (tid < E_LOCAL) {
    hist_all[tid] = 0;
    hist_pre[tid] = 0;
  }
  __syncthreads();
  for (int t = tid; t < T; t += DISPATCH_CHUNK) {
    const int4* row = reinterpret_cast<const int4*>(topk_ids + (size_t)t * TOP_K);
    const int4 a = row[0], b = row[1];
    const int v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < TOP_K; ++j) {
      const unsigned l = (unsigned)(v[j] - offset);
      if (l < (unsigned)E_LOCAL) {
        atomicAdd(&hist_all[l], 1);
        if (t < t0) atomicAdd(&hist_pre[l], 1);
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0, nact = 0;
    for (int e = 0; e < E_LOCAL; ++e) {
      seg[e] = acc;
      if (blockIdx.x == 0) {
        hdr->counts[e] = hist_all[e];
        hdr->seg_start[e] = acc;
        if (hist_all[e] > 0) hdr->active[nact++] = e;
      }
      acc += hist_all[e];
    }
    if (blockIdx.x == 0) {
      hdr->seg_start[E_LOCAL] = acc;
      hdr->n_active = nact;
      for (int e = nact; e < E_LOCAL; ++e) hdr->active[e] = -1;
    }
  }
  // this chunk's tokens: which local experts each selected, and in which slot
  const int t = t0 + tid;
  uint32_t mask = 0u;
  int slot_of[TOP_K];
  if (t < T) {
    const int4* row = reinterpret_cast<const int4*>(topk_ids + (size_t)t * TOP_K);
    const int4 a = row[0], b = row[1];
    const int v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < TOP_K; ++j) {
      slot_of[j] = v[j] - offset;
      if ((unsigned)slot_of[j] < (unsigned)E_LOCAL) mask |= 1u << slot_of[j];
    }
  }
  for (int e = 0; e < E_LOCAL; ++e) {  // uniform over the wave
    const unsigned long long m = __ballot((mask >> e) & 1u);
    if (lane == 0) wmask[wave][e] = m;
  }
  __syncthreads();
  if (mask) {
    const unsigned long long lt = (1ull << lane) - 1ull;
#pragma unroll
    for (int j = 0; j < TOP_K; ++j) {
      const int e = slot_of[j];
      if ((unsigned)e >= (unsigned)E_LOCAL) continue;
      int before = 0;  // earlier waves' tokens of this chunk that selected e
      for (int w = 0; w < wave; ++w) before += __popcll(wmask[w][e]);
      const int pos = seg[e] + hist_pre[e] + before + __popcll(wmask[wave][e] & lt);
      perm_tok[pos] = t;
      perm_w[pos] = topk_w[(size_t)t * TOP_K + j];
      tok_pair[(size_t)t * TOP_K + j] = pos;
    }
  }
}

hipError_t launch_dispatch(const int32_t* topk_ids, const float* topk_w, int T, int offset, DispatchHeader* hdr,
                           int32_t* perm_tok, float* perm_w, int32_t* tok_pair, hipStream_t stream) {
  if (T <= DISPATCH_CHUNKED_MAX_T) {
    const int chunks = T > 0 ? (T + DISPATCH_CHUNK - 1) / DISPATCH_CHUNK : 1;
    hipLaunchKernelGGL(dispatch_chunked_kernel, dim3(chunks), dim3(DISPATCH_CHUNK), 0, stream, topk_ids, topk_w, T,
                       offset, hdr, perm_tok, perm_w, tok_pair);
  } else {
    hipLaunchKernelGGL(dispatch_kernel, dim3(E_LOCAL), dim3(256), 0, stream, topk_ids, topk_w, T, offset, hdr,
                       perm_tok, perm_w, tok_pair);
  }
  return hipGetLastError();
}

}  // namespace moe

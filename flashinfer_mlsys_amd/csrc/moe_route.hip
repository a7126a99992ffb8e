// noaux_tc routing and per-expert dispatch for the FP8 DeepSeek-V3 MoE operator.
//
// route_kernel     -- reference moe/ref_moe.py:94-126 (sigmoid + bias, top-2-sum
//                     group scores, top-4 of 8 groups, top-8 experts inside them,
//                     weights from the unbiased sigmoid normalised over the 8 and
//                     scaled). One wave64 per token, 4 experts per lane; the
//                     top-8 by 8 rounds of wave arg-max, and the reference's
//                     nth_element order where equal keys straddle a cut
//                     (moe_route_token.h, moe_route_ties.h). From 6,144 tokens
//                     on, tokens first take the fast path (hardware exp/rcp
//                     scores, cuts certified against their error bound).
// dispatch_count_kernel, dispatch_scatter_kernel -- reference
//                     moe/ref_moe.py:131-145 (for each local expert the ascending
//                     list of tokens that selected it): per-chunk counts, then
//                     segment starts and ballot/popcount ranks. No atomics, no
//                     host synchronisation.
// dispatch_small_kernel -- the decode-size dispatch (T <= 64) in one workgroup.
#include "moe_common.h"
#include "moe_route_token.h"
#include "moe_small_dispatch.h"

namespace moe {

template <bool FAST>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits,
                                                    const uint16_t* __restrict__ bias, int T, float rsf,
                                                    int32_t* __restrict__ topk_ids, float* __restrict__ topk_w,
                                                    int32_t* __restrict__ tok_pair) {
  __shared__ TieScratch tie[4];
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  route_token<FAST>(logits, bias, t, rsf, topk_ids, topk_w, tok_pair, &tie[threadIdx.x >> 6]);
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

constexpr int kRouteFastMinTokens = 6144;  // 6 tokens per SIMD

hipError_t launch_route(const float* logits, const uint16_t* bias, int T, float rsf, int32_t* topk_ids,
                        float* topk_w, int32_t* tok_pair, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  if (T >= kRouteFastMinTokens)
    hipLaunchKernelGGL(route_kernel<true>, dim3((T + 3) / 4), dim3(256), 0, stream, logits, bias, T, rsf, topk_ids,
                       topk_w, tok_pair);
  else
    hipLaunchKernelGGL(route_kernel<false>, dim3((T + 3) / 4), dim3(256), 0, stream, logits, bias, T, rsf, topk_ids,
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

// Dispatch in two kernels over chunks of DISPATCH_CHUNK tokens, with the
// per-chunk counts in between (no atomics, no host synchronisation):
//  * dispatch_count_kernel: workgroup c counts, per local expert, the tokens of
//    chunk c that selected it (one ballot per expert and wave) into
//    chunk_counts[c][32];
//  * dispatch_scatter_kernel: workgroup c sums the chunk counts of all chunks
//    (totals -> segment starts) and of the chunks before it (its offset inside
//    each segment), then ranks its own tokens per expert with one ballot per
//    expert and wave and a prefix over its waves. Within each expert the tokens
//    stay in ascending order (reference ref_moe.py:131-145). Workgroup 0 writes
//    the header.
// Each workgroup reads its chunk's ids and 32 ints per chunk, so the work grows
// linearly with T (a single kernel in which every workgroup re-counts all T
// tokens grows with T^2).
constexpr int DISPATCH_WAVES = DISPATCH_CHUNK / 64;

__device__ __forceinline__ uint32_t local_mask(const int32_t* __restrict__ topk_ids, int t, int T, int offset,
                                               int (&slot_of)[TOP_K]) {
  uint32_t mask = 0u;
#pragma unroll
  for (int j = 0; j < TOP_K; ++j) slot_of[j] = -1;
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
  return mask;
}

__global__ __launch_bounds__(DISPATCH_CHUNK) void dispatch_count_kernel(const int32_t* __restrict__ topk_ids, int T,
                                                                        int offset,
                                                                        int32_t* __restrict__ chunk_counts) {
  __shared__ int wcnt[DISPATCH_WAVES][E_LOCAL];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int slot_of[TOP_K];
  const uint32_t mask = local_mask(topk_ids, blockIdx.x * DISPATCH_CHUNK + tid, T, offset, slot_of);
  int mine = 0;  // lane e < 32: this wave's tokens that selected expert e
#pragma unroll
  for (int e = 0; e < E_LOCAL; ++e) {
    const int c = __popcll(__ballot((mask >> e) & 1u));
    mine = lane == e ? c : mine;
  }
  if (lane < E_LOCAL) wcnt[wave][lane] = mine;
  __syncthreads();
  if (tid < E_LOCAL) {
    int s = 0;
#pragma unroll
    for (int w = 0; w < DISPATCH_WAVES; ++w) s += wcnt[w][tid];
    chunk_counts[(size_t)blockIdx.x * E_LOCAL + tid] = s;
  }
}

__global__ __launch_bounds__(DISPATCH_CHUNK) void dispatch_scatter_kernel(
    const int32_t* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int offset,
    const int32_t* __restrict__ chunk_counts, DispatchHeader* __restrict__ hdr, int32_t* __restrict__ perm_tok,
    float* __restrict__ perm_w, int32_t* __restrict__ tok_pair) {
  constexpr int PARTS = DISPATCH_CHUNK / E_LOCAL;  // threads per expert summing the chunk counts
  __shared__ int part_all[PARTS][E_LOCAL], part_pre[PARTS][E_LOCAL];
  __shared__ int seg[E_LOCAL], pre[E_LOCAL];
  __shared__ unsigned long long wmask[DISPATCH_WAVES][E_LOCAL];  // per wave and expert: lanes whose token selected it
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nchunks = gridDim.x, chunk = blockIdx.x;
  // this chunk's tokens (which local experts each selected, in which slot) and
  // their weights are requested first, so that their latency overlaps the chunk
  // counts' below
  const int t = chunk * DISPATCH_CHUNK + tid;
  int slot_of[TOP_K];
  const uint32_t mask = local_mask(topk_ids, t, T, offset, slot_of);
  float4 w8[2] = {float4{0.f, 0.f, 0.f, 0.f}, float4{0.f, 0.f, 0.f, 0.f}};
  if (t < T) {
    w8[0] = reinterpret_cast<const float4*>(topk_w + (size_t)t * TOP_K)[0];
    w8[1] = reinterpret_cast<const float4*>(topk_w + (size_t)t * TOP_K)[1];
  }
  {
    const int e = tid & (E_LOCAL - 1), part = tid / E_LOCAL;
    int all = 0, before = 0;
    for (int c = part; c < nchunks; c += PARTS) {
      const int v = chunk_counts[(size_t)c * E_LOCAL + e];
      all += v;
      before += c < chunk ? v : 0;
    }
    part_all[part][e] = all;
    part_pre[part][e] = before;
  }
  for (int e = 0; e < E_LOCAL; ++e) {  // uniform over the wave
    const unsigned long long m = __ballot((mask >> e) & 1u);
    if (lane == 0) wmask[wave][e] = m;
  }
  __syncthreads();
  if (tid < E_LOCAL) {  // lanes 0-31 of wave 0: one expert each
    int total = 0, b = 0;
#pragma unroll
    for (int p = 0; p < PARTS; ++p) {
      total += part_all[p][tid];
      b += part_pre[p][tid];
    }
    int incl = total;  // inclusive scan over the experts
#pragma unroll
    for (int d = 1; d < E_LOCAL; d <<= 1) {
      const int o = __shfl_up(incl, d);
      if (tid >= d) incl += o;
    }
    seg[tid] = incl - total;
    pre[tid] = b;
    if (chunk == 0) {
      const unsigned long long act = __ballot(total > 0);
      hdr->counts[tid] = total;
      hdr->seg_start[tid] = incl - total;
      if (tid == E_LOCAL - 1) hdr->seg_start[E_LOCAL] = incl;
      const int nact = __popcll(act);
      if (tid == 0) hdr->n_active = nact;
      if (total > 0) hdr->active[__popcll(act & ((1ull << tid) - 1ull))] = tid;
      if (tid >= nact) hdr->active[tid] = -1;
    }
  }
  __syncthreads();
  if (mask) {
    const unsigned long long lt = (1ull << lane) - 1ull;
    const float wv[TOP_K] = {w8[0].x, w8[0].y, w8[0].z, w8[0].w, w8[1].x, w8[1].y, w8[1].z, w8[1].w};
#pragma unroll
    for (int j = 0; j < TOP_K; ++j) {
      const int e = slot_of[j];
      if ((unsigned)e >= (unsigned)E_LOCAL) continue;
      int before = 0;  // earlier waves' tokens of this chunk that selected e
      for (int w = 0; w < wave; ++w) before += __popcll(wmask[w][e]);
      const int pos = seg[e] + pre[e] + before + __popcll(wmask[wave][e] & lt);
      perm_tok[pos] = t;
      perm_w[pos] = wv[j];
      tok_pair[(size_t)t * TOP_K + j] = pos;
    }
  }
}

hipError_t launch_dispatch(const int32_t* topk_ids, const float* topk_w, int T, int offset, DispatchHeader* hdr,
                           int32_t* perm_tok, float* perm_w, int32_t* tok_pair, int32_t* chunk_counts,
                           hipStream_t stream) {
  const int chunks = T > 0 ? dispatch_chunks(T) : 1;
  hipLaunchKernelGGL(dispatch_count_kernel, dim3(chunks), dim3(DISPATCH_CHUNK), 0, stream, topk_ids, T, offset,
                     chunk_counts);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(chunks), dim3(DISPATCH_CHUNK), 0, stream, topk_ids, topk_w, T,
                     offset, chunk_counts, hdr, perm_tok, perm_w, tok_pair);
  return hipGetLastError();
}

}  // namespace moe

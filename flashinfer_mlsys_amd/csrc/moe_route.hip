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
// route_count_kernel -- route_kernel for 16 tokens per workgroup (one per wave)
//                     that also counts, per local expert, the group's tokens that
//                     selected it (a row of 32 counts): the first half of the
//                     prefill dispatch, without a launch of its own.
// dispatch_count_kernel, dispatch_scatter_kernel -- reference
//                     moe/ref_moe.py:131-145 (for each local expert the ascending
//                     list of tokens that selected it): count rows (from given ids,
//                     for the dispatch tap), then segment starts and ballot/popcount
//                     ranks. No atomics, no host synchronisation.
// dispatch_small_kernel -- the decode-size dispatch (T <= SMALL_T) in one workgroup.
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

// Routing of COUNT_ROW_TOKENS tokens (wave w: token 16 b + w) into LDS, then
// copied out, and the group's row of per-expert counts: lanes 0-7 of each wave
// take one selected id each, and their local bits are ORed into the token's mask.
template <bool FAST>
__global__ __launch_bounds__(64 * COUNT_ROW_TOKENS) void route_count_kernel(
    const float* __restrict__ logits, const uint16_t* __restrict__ bias, int T, float rsf, int offset,
    int32_t* __restrict__ topk_ids, float* __restrict__ topk_w, int32_t* __restrict__ tok_pair,
    int32_t* __restrict__ count_rows_out) {
  __shared__ TieScratch tie[COUNT_ROW_TOKENS];
  __shared__ int32_t sid[COUNT_ROW_TOKENS * TOP_K];
  __shared__ float swt[COUNT_ROW_TOKENS * TOP_K];
  __shared__ uint32_t tmask[COUNT_ROW_TOKENS];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t0 = blockIdx.x * COUNT_ROW_TOKENS, t = t0 + wave;
  uint32_t mask = 0u;
  if (t < T) {
    route_token<FAST>(logits + (size_t)t0 * E_GLOBAL, bias, wave, rsf, sid, swt, tok_pair + (size_t)t0 * TOP_K,
                      &tie[wave]);
    // the wave's own LDS writes are visible to its own reads, in order
    const int le = lane < TOP_K ? sid[wave * TOP_K + lane] - offset : -1;
    mask = (unsigned)le < (unsigned)E_LOCAL ? 1u << le : 0u;
    mask |= __shfl_xor(mask, 1);
    mask |= __shfl_xor(mask, 2);
    mask |= __shfl_xor(mask, 4);
  }
  if (lane == 0) tmask[wave] = mask;
  __syncthreads();
  const int tid = threadIdx.x;
  const int nvalid = min(COUNT_ROW_TOKENS, T - t0);
  if (tid < nvalid * TOP_K) {
    topk_ids[(size_t)t0 * TOP_K + tid] = sid[tid];
    topk_w[(size_t)t0 * TOP_K + tid] = swt[tid];
  }
  if (tid < E_LOCAL) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < COUNT_ROW_TOKENS; ++w) c += (tmask[w] >> tid) & 1u;
    count_rows_out[(size_t)blockIdx.x * E_LOCAL + tid] = c;
  }
}

// Dispatch of up to SMALL_T tokens in one workgroup with the same device code
// the decode GEMM1 kernel runs in each of its workgroups (dispatch tap).
constexpr int DISPATCH_SMALL_THREADS = 512;
static_assert(DISPATCH_SMALL_THREADS >= SMALL_T, "a thread per token mask");
template <int TM>
__global__ __launch_bounds__(DISPATCH_SMALL_THREADS) void dispatch_small_kernel(const int32_t* __restrict__ topk_ids,
                                                                 const float* __restrict__ topk_w, int T, int offset,
                                                                 DispatchHeader* __restrict__ hdr,
                                                                 int32_t* __restrict__ perm_tok,
                                                                 float* __restrict__ perm_w,
                                                                 int32_t* __restrict__ tok_pair) {
  __shared__ SmallDispatch<TM> d;
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

hipError_t launch_route_count(const float* logits, const uint16_t* bias, int T, float rsf, int offset,
                              int32_t* topk_ids, float* topk_w, int32_t* tok_pair, int32_t* count_rows_out,
                              hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  const dim3 grid(count_rows(T)), block(64 * COUNT_ROW_TOKENS);
  if (T >= kRouteFastMinTokens)
    hipLaunchKernelGGL(route_count_kernel<true>, grid, block, 0, stream, logits, bias, T, rsf, offset, topk_ids,
                       topk_w, tok_pair, count_rows_out);
  else
    hipLaunchKernelGGL(route_count_kernel<false>, grid, block, 0, stream, logits, bias, T, rsf, offset, topk_ids,
                       topk_w, tok_pair, count_rows_out);
  return hipGetLastError();
}

hipError_t launch_dispatch_small(const int32_t* topk_ids, const float* topk_w, int T, int offset,
                                 DispatchHeader* hdr, int32_t* perm_tok, float* perm_w, int32_t* tok_pair,
                                 hipStream_t stream) {
  if (T <= 0 || T > SMALL_T) return hipErrorInvalidValue;
  if (T <= 64)
    hipLaunchKernelGGL(dispatch_small_kernel<64>, dim3(1), dim3(DISPATCH_SMALL_THREADS), 0, stream, topk_ids, topk_w,
                       T, offset, hdr, perm_tok, perm_w, tok_pair);
  else
    hipLaunchKernelGGL(dispatch_small_kernel<SMALL_T>, dim3(1), dim3(DISPATCH_SMALL_THREADS), 0, stream, topk_ids,
                       topk_w, T, offset, hdr, perm_tok, perm_w, tok_pair);
  return hipGetLastError();
}

// Dispatch over chunks of DISPATCH_CHUNK tokens with count rows in between (no
// atomics, no host synchronisation):
//  * the count rows: row g holds, per local expert, the number of tokens
//    16 g .. 16 g + 15 that selected it (route_count_kernel writes them while
//    routing; dispatch_count_kernel from given ids, for the dispatch tap);
//  * dispatch_scatter_kernel: workgroup c sums the rows of all groups (totals ->
//    segment starts) and of the groups before its chunk (its offset inside each
//    segment), then ranks its own tokens per expert with one ballot per expert
//    and wave and a prefix over its waves. Within each expert the tokens stay in
//    ascending order (reference ref_moe.py:131-145). Workgroup 0 writes the header.
// Each scatter workgroup reads its chunk's ids and the count rows, 2 words per
// token (the rows are small next to the GEMMs' operands at every T the forward
// runs on: one chunk of at most MOE_FP8_CHUNK_TOKENS tokens).
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

// Count rows from given ids: wave w of workgroup b covers rows RPW (4 b + w) ..
// + RPW - 1 (its 64 tokens); lane e < 32 writes expert e's count of each of them.
constexpr int RPW = 64 / COUNT_ROW_TOKENS;  // count rows per wave
__global__ __launch_bounds__(DISPATCH_CHUNK) void dispatch_count_kernel(const int32_t* __restrict__ topk_ids, int T,
                                                                        int offset,
                                                                        int32_t* __restrict__ count_rows_out) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int slot_of[TOP_K];
  const uint32_t mask = local_mask(topk_ids, blockIdx.x * DISPATCH_CHUNK + tid, T, offset, slot_of);
  int mine[RPW];  // lane e < 32: expert e's count in each row's slice of lanes
#pragma unroll
  for (int q = 0; q < RPW; ++q) mine[q] = 0;
  constexpr unsigned long long SLICE = (1ull << COUNT_ROW_TOKENS) - 1ull;
#pragma unroll
  for (int e = 0; e < E_LOCAL; ++e) {
    const unsigned long long b = __ballot((mask >> e) & 1u);
    if (lane == e) {
#pragma unroll
      for (int q = 0; q < RPW; ++q) mine[q] = __popcll((b >> (COUNT_ROW_TOKENS * q)) & SLICE);
    }
  }
  const int row0 = (blockIdx.x * DISPATCH_WAVES + wave) * RPW, rows = count_rows(T);
  if (lane < E_LOCAL) {
#pragma unroll
    for (int q = 0; q < RPW; ++q)
      if (row0 + q < rows) count_rows_out[(size_t)(row0 + q) * E_LOCAL + lane] = mine[q];
  }
}

__global__ __launch_bounds__(DISPATCH_CHUNK) void dispatch_scatter_kernel(
    const int32_t* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int offset,
    const int32_t* __restrict__ crow, DispatchHeader* __restrict__ hdr, int32_t* __restrict__ perm_tok,
    float* __restrict__ perm_w, int32_t* __restrict__ tok_pair) {
  constexpr int PARTS = DISPATCH_CHUNK / (E_LOCAL / 4);  // threads per group of 4 experts summing the count rows
  __shared__ int part_all[PARTS][E_LOCAL], part_pre[PARTS][E_LOCAL];
  __shared__ int seg[E_LOCAL], pre[E_LOCAL];
  __shared__ unsigned long long wmask[DISPATCH_WAVES][E_LOCAL];  // per wave and expert: lanes whose token selected it
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int chunk = blockIdx.x;
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
    // thread: experts 4 q .. 4 q + 3 (one 16 B load per row), rows part, part + PARTS, ...
    const int q = tid & (E_LOCAL / 4 - 1), part = tid / (E_LOCAL / 4);
    const int nrows = count_rows(T), first = chunk * (DISPATCH_CHUNK / COUNT_ROW_TOKENS);
    int4 all = {0, 0, 0, 0}, before = {0, 0, 0, 0};
#pragma unroll 8
    for (int r = part; r < nrows; r += PARTS) {
      const int4 v = reinterpret_cast<const int4*>(crow + (size_t)r * E_LOCAL)[q];
      all.x += v.x; all.y += v.y; all.z += v.z; all.w += v.w;
      if (r < first) {
        before.x += v.x; before.y += v.y; before.z += v.z; before.w += v.w;
      }
    }
    part_all[part][4 * q] = all.x; part_all[part][4 * q + 1] = all.y;
    part_all[part][4 * q + 2] = all.z; part_all[part][4 * q + 3] = all.w;
    part_pre[part][4 * q] = before.x; part_pre[part][4 * q + 1] = before.y;
    part_pre[part][4 * q + 2] = before.z; part_pre[part][4 * q + 3] = before.w;
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

hipError_t launch_dispatch_scatter(const int32_t* topk_ids, const float* topk_w, int T, int offset,
                                   DispatchHeader* hdr, int32_t* perm_tok, float* perm_w, int32_t* tok_pair,
                                   const int32_t* count_rows_in, hipStream_t stream) {
  const int chunks = T > 0 ? dispatch_chunks(T) : 1;
  hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(chunks), dim3(DISPATCH_CHUNK), 0, stream, topk_ids, topk_w, T,
                     offset, count_rows_in, hdr, perm_tok, perm_w, tok_pair);
  return hipGetLastError();
}

hipError_t launch_dispatch(const int32_t* topk_ids, const float* topk_w, int T, int offset, DispatchHeader* hdr,
                           int32_t* perm_tok, float* perm_w, int32_t* tok_pair, int32_t* count_rows_buf,
                           hipStream_t stream) {
  if (T > 0) {
    hipLaunchKernelGGL(dispatch_count_kernel, dim3(dispatch_chunks(T)), dim3(DISPATCH_CHUNK), 0, stream, topk_ids, T,
                       offset, count_rows_buf);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return launch_dispatch_scatter(topk_ids, topk_w, T, offset, hdr, perm_tok, perm_w, tok_pair, count_rows_buf,
                                 stream);
}

}  // namespace moe

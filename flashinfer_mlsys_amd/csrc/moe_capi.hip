// extern "C" boundary of libmoe_mi355x.so (declarations and contract in
// include/moe_fp8.h). Validates arguments, carves the workspace and enqueues
// the kernels on the caller's stream: route -> dispatch -> GEMM1+SwiGLU ->
// GEMM2 x weight -> ordered combine (inside GEMM2 in the decode shape). No host
// synchronisation, no allocation.
#include "moe_common.h"
#include "moe_host.h"
#include "moe_small_dispatch.h"
#include "../../include/moe_fp8.h"

#include <algorithm>
#include <atomic>

namespace moe {
hipError_t launch_route(const float*, const uint16_t*, int, float, int32_t*, float*, int32_t*, hipStream_t);
hipError_t launch_route_count(const float*, const uint16_t*, int, float, int, int32_t*, float*, int32_t*, int32_t*,
                              hipStream_t);
hipError_t launch_dispatch(const int32_t*, const float*, int, int, DispatchHeader*, int32_t*, float*, int32_t*,
                           int32_t*, hipStream_t);
hipError_t launch_dispatch_scatter(const int32_t*, const float*, int, int, DispatchHeader*, int32_t*, float*,
                                   int32_t*, const int32_t*, hipStream_t);
hipError_t launch_dispatch_small(const int32_t*, const float*, int, int, DispatchHeader*, int32_t*, float*, int32_t*,
                                 hipStream_t);
hipError_t launch_gemm1_decode(const float*, const uint16_t*, float, bool, const uint8_t*, const float*, int, int,
                               const uint8_t*, const float*, int32_t*, float*, DispatchHeader*, int32_t*, float*,
                               int32_t*, uint16_t*, int, hipStream_t);
hipError_t launch_quantize_1x128(const uint16_t*, int, uint8_t*, float*, hipStream_t);
hipError_t launch_router_logits(const uint16_t*, const uint16_t*, int, float*, int, hipStream_t);
hipError_t launch_router_quantize(const uint16_t*, const uint16_t*, int, float*, uint8_t*, float*, int, hipStream_t);
hipError_t launch_gemm2_decode(const uint16_t*, const uint8_t*, const float*, const DispatchHeader*, const int32_t*,
                               const float*, int, uint16_t*, hipStream_t);
int gemm1_decode_blocks_per_cu(int T);
hipError_t launch_gemm1_prefill(const uint8_t*, const float*, int, const uint8_t*, const float*,
                               const DispatchHeader*, const int32_t*, uint16_t*, int, hipStream_t);
hipError_t launch_gemm2_loader(const uint16_t*, const uint8_t*, const float*, const DispatchHeader*, const float*,
                               uint16_t*, int, hipStream_t);
hipError_t launch_combine(const uint16_t*, const int32_t*, int, uint16_t*, hipStream_t);
}  // namespace moe

namespace {

constexpr int kMaxDevices = 64;
constexpr int kDecodeMaxTokens = MOE_FP8_DECODE_MAX_TOKENS;  // decode shape (LDS dispatch, streaming GEMMs)
static_assert(kDecodeMaxTokens <= moe::SMALL_T, "the decode kernels' LDS dispatch holds SMALL_T tokens");
constexpr int kRouteInGemm1MaxTokens = 8;   // and routing inside GEMM1 (one token per wave) up to this many
std::atomic<int> g_cu_count[kMaxDevices];
thread_local const char* t_last_hip_error = "no error";

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int hip_fail(hipError_t e) {
  t_last_hip_error = hipGetErrorString(e);
  return MOE_ERR_HIP;
}

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int n = g_cu_count[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  g_cu_count[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Offsets outside [-256, 256] select no local expert; clamp so int arithmetic stays small.
int clamp_offset(int64_t off) { return off < -256 ? -256 : (off > 256 ? 256 : (int)off); }

}  // namespace

extern "C" {

size_t moe_fp8_workspace_size(int64_t T) {
  if (T < 0 || T > MOE_FP8_MAX_TOKENS) return 0;
  return moe::WorkspaceLayout::make(T < MOE_FP8_CHUNK_TOKENS ? T : MOE_FP8_CHUNK_TOKENS).total;
}

}  // extern "C"

namespace {

struct Call {
  const float* logits;
  const uint16_t* bias;
  const uint8_t* hidden;
  const float* hscale;
  const uint8_t* w13;
  const float* s13;
  const uint8_t* w2;
  const float* s2;
  int T;
  int hs_stride;  // row stride of hidden_states_scale [56, T_call]: T, or the whole call's T for a chunk
  int offset;
  float rsf;
  uint16_t* out;
  bool decode;  // T <= kDecodeMaxTokens and the shape is not forced to the prefill kernels
  hipStream_t stream;
  moe::DispatchHeader* hdr;
  int32_t *topk_ids, *tok_pair, *perm_tok, *chunk_counts;
  float *topk_w, *perm_w;
  uint16_t *c_act, *partial;  // fp16: C * 2^-8 and the pair rows w * O * 2^-8
};

int check_call(const float* routing_logits, const uint16_t* routing_bias, const uint8_t* hidden_states,
               const float* hidden_states_scale, const uint8_t* gemm1_weights, const float* gemm1_weights_scale,
               const uint8_t* gemm2_weights, const float* gemm2_weights_scale, int64_t T, int64_t local_expert_offset,
               double routed_scaling_factor, uint16_t* output, void* workspace, size_t workspace_bytes, void* stream,
               int shape, Call& c) {
  using namespace moe;
  if (shape != MOE_SHAPE_AUTO && shape != MOE_SHAPE_PREFILL) return MOE_ERR_ARG;
  if (T < 0 || T > MOE_FP8_MAX_TOKENS) return MOE_ERR_SIZE;
  if (T == 0) return MOE_OK;
  if (!routing_logits || !routing_bias || !hidden_states || !hidden_states_scale || !gemm1_weights ||
      !gemm1_weights_scale || !gemm2_weights || !gemm2_weights_scale || !output || !workspace)
    return MOE_ERR_NULL;
  if (!aligned16(routing_logits) || !aligned16(routing_bias) || !aligned16(hidden_states) ||
      !aligned16(hidden_states_scale) || !aligned16(gemm1_weights) || !aligned16(gemm1_weights_scale) ||
      !aligned16(gemm2_weights) || !aligned16(gemm2_weights_scale) || !aligned16(output) || !aligned16(workspace))
    return MOE_ERR_ALIGN;
  const bool decode = shape == MOE_SHAPE_AUTO && T <= kDecodeMaxTokens;
  // calls above MOE_FP8_CHUNK_TOKENS run chunk by chunk in one chunk's workspace
  const int64_t Tw = T < MOE_FP8_CHUNK_TOKENS ? T : MOE_FP8_CHUNK_TOKENS;
  const WorkspaceLayout L = WorkspaceLayout::make(Tw, !decode);  // the decode kernels use no partial rows
  if (workspace_bytes < L.total) return MOE_ERR_WORKSPACE;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  c.logits = routing_logits;
  c.bias = routing_bias;
  c.hidden = hidden_states;
  c.hscale = hidden_states_scale;
  c.w13 = gemm1_weights;
  c.s13 = gemm1_weights_scale;
  c.w2 = gemm2_weights;
  c.s2 = gemm2_weights_scale;
  c.T = (int)T;
  c.hs_stride = (int)T;
  c.offset = clamp_offset(local_expert_offset);
  c.rsf = (float)routed_scaling_factor;
  c.out = output;
  c.decode = decode;
  c.stream = reinterpret_cast<hipStream_t>(stream);
  c.hdr = reinterpret_cast<DispatchHeader*>(ws + L.hdr);
  c.topk_ids = reinterpret_cast<int32_t*>(ws + L.topk_ids);
  c.topk_w = reinterpret_cast<float*>(ws + L.topk_w);
  c.tok_pair = reinterpret_cast<int32_t*>(ws + L.tok_pair);
  c.perm_tok = reinterpret_cast<int32_t*>(ws + L.perm_tok);
  c.perm_w = reinterpret_cast<float*>(ws + L.perm_w);
  c.c_act = reinterpret_cast<uint16_t*>(ws + L.c_act);
  c.partial = reinterpret_cast<uint16_t*>(ws + L.partial);
  c.chunk_counts = reinterpret_cast<int32_t*>(ws + L.chunk_counts);
  return 1;  // valid, work to do
}

// Stage 0: routing (+ dispatch in the prefill shape; nothing for a decode call
// of at most 8 tokens, routed inside GEMM1); 1: GEMM1 + SwiGLU (+ the
// in-workgroup dispatch in the decode shape); 2: GEMM2 x weight (prefill: into
// one fp16 row per pair; decode: with the ordered per-token sum, straight to the
// bf16 output); 3: the ordered combine of the prefill rows to bf16 (nothing in
// the decode shape).
hipError_t run_stage(int stage, const Call& c) {
  using namespace moe;
  const int max_active = c.T * TOP_K < E_LOCAL ? c.T * TOP_K : E_LOCAL;
  switch (stage) {
    case 0:
      if (c.decode && c.T <= kRouteInGemm1MaxTokens) return hipSuccess;  // routed inside GEMM1
      if (c.decode) return launch_route(c.logits, c.bias, c.T, c.rsf, c.topk_ids, c.topk_w, nullptr, c.stream);
      {
        // routing + the count rows in one launch, then the scatter
        hipError_t e = launch_route_count(c.logits, c.bias, c.T, c.rsf, c.offset, c.topk_ids, c.topk_w, c.tok_pair,
                                          c.chunk_counts, c.stream);
        if (e != hipSuccess) return e;
        return launch_dispatch_scatter(c.topk_ids, c.topk_w, c.T, c.offset, c.hdr, c.perm_tok, c.perm_w, c.tok_pair,
                                       c.chunk_counts, c.stream);
      }
    case 1:
      if (c.decode) {
        const int grid = std::min(max_active * (I / 8), cu_count() * gemm1_decode_blocks_per_cu(c.T));
        return launch_gemm1_decode(c.logits, c.bias, c.rsf, c.T <= kRouteInGemm1MaxTokens, c.hidden, c.hscale, c.T,
                                   c.offset, c.w13, c.s13, c.topk_ids, c.topk_w, c.hdr, c.perm_tok, c.perm_w,
                                   c.tok_pair, c.c_act, grid, c.stream);
      }
      return launch_gemm1_prefill(c.hidden, c.hscale, c.hs_stride, c.w13, c.s13, c.hdr, c.perm_tok, c.c_act,
                                 (cu_count() + 7) / 8 * 8, c.stream);
    case 2:
      if (c.decode) return launch_gemm2_decode(c.c_act, c.w2, c.s2, c.hdr, c.perm_tok, c.perm_w, c.T, c.out, c.stream);
      return launch_gemm2_loader(c.c_act, c.w2, c.s2, c.hdr, c.perm_w, c.partial, (cu_count() + 7) / 8 * 8,
                                 c.stream);
    case 3:
      if (c.decode) return hipSuccess;  // summed inside GEMM2
      return launch_combine(c.partial, c.tok_pair, c.T, c.out, c.stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

extern "C" {

static int forward(int shape, const float* routing_logits, const uint16_t* routing_bias,
                   const uint8_t* hidden_states, const float* hidden_states_scale, const uint8_t* gemm1_weights,
                   const float* gemm1_weights_scale, const uint8_t* gemm2_weights, const float* gemm2_weights_scale,
                   int64_t T, int64_t local_expert_offset, double routed_scaling_factor, uint16_t* output,
                   void* workspace, size_t workspace_bytes, void* stream) {
  Call c;
  const int v = check_call(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                           gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, T, local_expert_offset,
                           routed_scaling_factor, output, workspace, workspace_bytes, stream, shape, c);
  if (v <= 0) return v;
  // Tokens are independent (routing, experts and the sum over a token's experts
  // are all per token), so a call above MOE_FP8_CHUNK_TOKENS runs as consecutive
  // calls over token chunks, each with the chunk's rows of every per-token input
  // and output; only hidden_states_scale [56, T] keeps the whole call's row
  // stride. Every chunk's result is bit for bit the one a separate call gives.
  const int T_all = c.T;
  for (int t0 = 0; t0 < T_all; t0 += MOE_FP8_CHUNK_TOKENS) {
    Call k = c;
    k.T = T_all - t0 < MOE_FP8_CHUNK_TOKENS ? T_all - t0 : MOE_FP8_CHUNK_TOKENS;
    k.logits = c.logits + (size_t)t0 * moe::E_GLOBAL;
    k.hidden = c.hidden + (size_t)t0 * moe::H;
    k.hscale = c.hscale + t0;
    k.out = c.out + (size_t)t0 * moe::H;
    for (int stage = 0; stage < 4; ++stage) {
      const hipError_t e = run_stage(stage, k);
      if (e != hipSuccess) return hip_fail(e);
    }
  }
  return MOE_OK;
}

int moe_fp8_forward(const float* routing_logits, const uint16_t* routing_bias, const uint8_t* hidden_states,
                    const float* hidden_states_scale, const uint8_t* gemm1_weights,
                    const float* gemm1_weights_scale, const uint8_t* gemm2_weights,
                    const float* gemm2_weights_scale, int64_t T, int64_t local_expert_offset,
                    double routed_scaling_factor, uint16_t* output, void* workspace, size_t workspace_bytes,
                    void* stream) {
  return forward(MOE_SHAPE_AUTO, routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                 gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, T, local_expert_offset,
                 routed_scaling_factor, output, workspace, workspace_bytes, stream);
}

int moe_fp8_forward_shape(int shape, const float* routing_logits, const uint16_t* routing_bias,
                          const uint8_t* hidden_states, const float* hidden_states_scale,
                          const uint8_t* gemm1_weights, const float* gemm1_weights_scale,
                          const uint8_t* gemm2_weights, const float* gemm2_weights_scale, int64_t T,
                          int64_t local_expert_offset, double routed_scaling_factor, uint16_t* output,
                          void* workspace, size_t workspace_bytes, void* stream) {
  return forward(shape, routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                 gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, T, local_expert_offset,
                 routed_scaling_factor, output, workspace, workspace_bytes, stream);
}

int moe_fp8_run_stage(int stage, int shape, const float* routing_logits, const uint16_t* routing_bias,
                      const uint8_t* hidden_states, const float* hidden_states_scale, const uint8_t* gemm1_weights,
                      const float* gemm1_weights_scale, const uint8_t* gemm2_weights,
                      const float* gemm2_weights_scale, int64_t T, int64_t local_expert_offset,
                      double routed_scaling_factor, uint16_t* output, void* workspace, size_t workspace_bytes,
                      void* stream) {
  if (stage < 0 || stage > 3) return MOE_ERR_ARG;
  if (T > MOE_FP8_CHUNK_TOKENS) return MOE_ERR_SIZE;  // a stage spans the whole call, which is one chunk at most
  Call c;
  const int v = check_call(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                           gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, T, local_expert_offset,
                           routed_scaling_factor, output, workspace, workspace_bytes, stream, shape, c);
  if (v <= 0) return v;
  const hipError_t e = run_stage(stage, c);
  return e == hipSuccess ? MOE_OK : hip_fail(e);
}

int moe_fp8_route(const float* routing_logits, const uint16_t* routing_bias, int64_t T,
                  double routed_scaling_factor, int32_t* topk_ids, float* topk_w, int32_t* tok_pair,
                  void* stream) {
  if (T < 0 || T > MOE_FP8_MAX_TAP_TOKENS) return MOE_ERR_SIZE;
  if (T == 0) return MOE_OK;
  if (!routing_logits || !routing_bias || !topk_ids || !topk_w) return MOE_ERR_NULL;
  if (!aligned16(routing_logits) || !aligned16(routing_bias) || !aligned16(topk_ids) || !aligned16(topk_w) ||
      (tok_pair && !aligned16(tok_pair)))
    return MOE_ERR_ALIGN;
  hipError_t e = moe::launch_route(routing_logits, routing_bias, (int)T, (float)routed_scaling_factor, topk_ids,
                                   topk_w, tok_pair, reinterpret_cast<hipStream_t>(stream));
  return e == hipSuccess ? MOE_OK : hip_fail(e);
}

int moe_fp8_dispatch(const int32_t* topk_ids, const float* topk_w, int64_t T, int64_t local_expert_offset,
                     int32_t* header, size_t header_words, int32_t* perm_tok, float* perm_w, int32_t* tok_pair,
                     void* stream) {
  if (T < 0 || T > MOE_FP8_MAX_TAP_TOKENS) return MOE_ERR_SIZE;
  if (header && header_words < (size_t)MOE_FP8_DISPATCH_HEADER_WORDS(T)) return MOE_ERR_WORKSPACE;
  if (!header || !perm_tok || !perm_w || !tok_pair || (T > 0 && (!topk_ids || !topk_w))) return MOE_ERR_NULL;
  if (!aligned16(header) || !aligned16(perm_tok) || !aligned16(perm_w) || !aligned16(tok_pair) ||
      (T > 0 && (!aligned16(topk_ids) || !aligned16(topk_w))))
    return MOE_ERR_ALIGN;
  hipError_t e = moe::launch_dispatch(topk_ids, topk_w, (int)T, clamp_offset(local_expert_offset),
                                      reinterpret_cast<moe::DispatchHeader*>(header), perm_tok, perm_w, tok_pair,
                                      header + MOE_FP8_HEADER_WORDS, reinterpret_cast<hipStream_t>(stream));
  return e == hipSuccess ? MOE_OK : hip_fail(e);
}

int moe_fp8_route_dispatch(int shape, const float* routing_logits, const uint16_t* routing_bias, int64_t T,
                           int64_t local_expert_offset, double routed_scaling_factor, int32_t* topk_ids,
                           float* topk_w, int32_t* header, size_t header_words, int32_t* perm_tok, float* perm_w,
                           int32_t* tok_pair, void* stream) {
  using namespace moe;
  if (shape != MOE_SHAPE_AUTO && shape != MOE_SHAPE_PREFILL) return MOE_ERR_ARG;
  if (T < 0 || T > MOE_FP8_MAX_TAP_TOKENS) return MOE_ERR_SIZE;
  if (header && header_words < (size_t)MOE_FP8_DISPATCH_HEADER_WORDS(T)) return MOE_ERR_WORKSPACE;
  if (T == 0) return MOE_OK;
  if (!routing_logits || !routing_bias || !topk_ids || !topk_w || !header || !perm_tok || !perm_w || !tok_pair)
    return MOE_ERR_NULL;
  if (!aligned16(routing_logits) || !aligned16(routing_bias) || !aligned16(topk_ids) || !aligned16(topk_w) ||
      !aligned16(header) || !aligned16(perm_tok) || !aligned16(perm_w) || !aligned16(tok_pair))
    return MOE_ERR_ALIGN;
  const int t = (int)T, off = clamp_offset(local_expert_offset);
  const float rsf = (float)routed_scaling_factor;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  auto* hdr = reinterpret_cast<DispatchHeader*>(header);
  hipError_t e;
  const bool decode = shape == MOE_SHAPE_AUTO && t <= kDecodeMaxTokens;
  if (decode) {
    e = launch_route(routing_logits, routing_bias, t, rsf, topk_ids, topk_w, nullptr, s);
    if (e == hipSuccess) e = launch_dispatch_small(topk_ids, topk_w, t, off, hdr, perm_tok, perm_w, tok_pair, s);
  } else {
    e = launch_route_count(routing_logits, routing_bias, t, rsf, off, topk_ids, topk_w, tok_pair,
                           header + MOE_FP8_HEADER_WORDS, s);
    if (e == hipSuccess)
      e = launch_dispatch_scatter(topk_ids, topk_w, t, off, hdr, perm_tok, perm_w, tok_pair,
                                  header + MOE_FP8_HEADER_WORDS, s);
  }
  return e == hipSuccess ? MOE_OK : hip_fail(e);
}

int moe_fp8_quantize_activations(const uint16_t* hidden_bf16, int64_t T, uint8_t* hidden_states,
                                 float* hidden_states_scale, void* stream) {
  if (T < 0 || T > MOE_FP8_MAX_TAP_TOKENS) return MOE_ERR_SIZE;
  if (T == 0) return MOE_OK;
  if (!hidden_bf16 || !hidden_states || !hidden_states_scale) return MOE_ERR_NULL;
  if (!aligned16(hidden_bf16) || !aligned16(hidden_states) || !aligned16(hidden_states_scale)) return MOE_ERR_ALIGN;
  hipError_t e = moe::launch_quantize_1x128(hidden_bf16, (int)T, hidden_states, hidden_states_scale,
                                            reinterpret_cast<hipStream_t>(stream));
  return e == hipSuccess ? MOE_OK : hip_fail(e);
}

int moe_fp8_router_logits(const uint16_t* hidden_bf16, const uint16_t* gate_weight, int64_t T,
                          float* routing_logits, void* stream) {
  if (T < 0 || T > MOE_FP8_MAX_TAP_TOKENS) return MOE_ERR_SIZE;
  if (T == 0) return MOE_OK;
  if (!hidden_bf16 || !gate_weight || !routing_logits) return MOE_ERR_NULL;
  if (!aligned16(hidden_bf16) || !aligned16(gate_weight) || !aligned16(routing_logits)) return MOE_ERR_ALIGN;
  hipError_t e = moe::launch_router_logits(hidden_bf16, gate_weight, (int)T, routing_logits, cu_count(),
                                           reinterpret_cast<hipStream_t>(stream));
  return e == hipSuccess ? MOE_OK : hip_fail(e);
}

int moe_fp8_router_quantize(const uint16_t* hidden_bf16, const uint16_t* gate_weight, int64_t T,
                            float* routing_logits, uint8_t* hidden_states, float* hidden_states_scale, void* stream) {
  if (T < 0 || T > MOE_FP8_MAX_TAP_TOKENS) return MOE_ERR_SIZE;
  if (T == 0) return MOE_OK;
  if (!hidden_bf16 || !gate_weight || !routing_logits || !hidden_states || !hidden_states_scale) return MOE_ERR_NULL;
  if (!aligned16(hidden_bf16) || !aligned16(gate_weight) || !aligned16(routing_logits) || !aligned16(hidden_states) ||
      !aligned16(hidden_states_scale))
    return MOE_ERR_ALIGN;
  hipError_t e = moe::launch_router_quantize(hidden_bf16, gate_weight, (int)T, routing_logits, hidden_states,
                                             hidden_states_scale, cu_count(), reinterpret_cast<hipStream_t>(stream));
  return e == hipSuccess ? MOE_OK : hip_fail(e);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free forward for decode sizes: the workspace is a file-scope
// device array (each device holds its own copy, for the life of the process),
// addressed through the pointer hipGetSymbolAddress returns on that device.
// ---------------------------------------------------------------------------
namespace {

constexpr size_t kNoAllocScratchBytes = moe::WorkspaceLayout::make(MOE_FP8_NOALLOC_MAX_TOKENS, false).total;
static_assert(kNoAllocScratchBytes < (4u << 20), "a modest scratch: header, ids, permutation and fp16 C rows");

__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

struct ScratchAddress {
  hipError_t err = hipErrorInvalidDevice;
  void* ptr = nullptr;
};
moe::PerDeviceOnce<ScratchAddress> g_scratch;

// The current device's copy of `scratch`, looked up once per device.
int scratch_address(void** out) {
  ScratchAddress a;
  if (!g_scratch.get([] {
        ScratchAddress r;
        r.err = hipGetSymbolAddress(&r.ptr, HIP_SYMBOL(scratch));
        return r;
      }, a))
    return hip_fail(hipErrorInvalidDevice);
  if (a.err != hipSuccess) return hip_fail(a.err);
  if (a.ptr == nullptr) return hip_fail(hipErrorInvalidSymbol);
  *out = a.ptr;
  return MOE_OK;
}

}  // namespace

extern "C" {

int moe_fp8_forward_noalloc(const float* routing_logits, const uint16_t* routing_bias, const uint8_t* hidden_states,
                            const float* hidden_states_scale, const uint8_t* gemm1_weights,
                            const float* gemm1_weights_scale, const uint8_t* gemm2_weights,
                            const float* gemm2_weights_scale, int64_t T, int64_t local_expert_offset,
                            double routed_scaling_factor, uint16_t* output, void* stream) {
  if (T < 0) return MOE_ERR_SIZE;
  if (T > MOE_FP8_NOALLOC_MAX_TOKENS) return MOE_ERR_NOALLOC_SIZE;
  if (T == 0) return MOE_OK;
  void* ws = nullptr;
  const int r = scratch_address(&ws);
  if (r != MOE_OK) return r;
  return forward(MOE_SHAPE_AUTO, routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                 gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, T, local_expert_offset,
                 routed_scaling_factor, output, ws, kNoAllocScratchBytes, stream);
}

const char* moe_fp8_strerror(int code) {
  switch (code) {
    case MOE_OK: return "ok";
    case MOE_ERR_NULL: return "a required pointer is NULL";
    case MOE_ERR_SIZE: return "token count out of range";
    case MOE_ERR_ALIGN: return "a pointer is not 16-byte aligned";
    case MOE_ERR_WORKSPACE: return "workspace smaller than moe_fp8_workspace_size(T)";
    case MOE_ERR_HIP: return "HIP launch failed";
    case MOE_ERR_ARG: return "an enumerated argument (stage, shape) is out of range";
    case MOE_ERR_NOALLOC_SIZE:
      return "token count beyond MOE_FP8_NOALLOC_MAX_TOKENS (64) for moe_fp8_forward_noalloc; use moe_fp8_forward";
    default: return "unknown error";
  }
}

const char* moe_fp8_last_hip_error(void) { return t_last_hip_error; }

int moe_fp8_abi_version(void) { return 3; }

}  // extern "C"

// extern "C" boundary of libmoe_mi355x.so (declarations and contract in
// include/moe_fp8.h). Validates arguments, carves the workspace and enqueues
// the kernels on the caller's stream: route -> dispatch -> GEMM1+SwiGLU ->
// GEMM2 x weight -> ordered combine. No host synchronisation, no allocation.
#include "moe_common.h"
#include "../../include/moe_fp8.h"

#include <atomic>

namespace moe {
hipError_t launch_route(const float*, const uint16_t*, int, float, int32_t*, float*, int32_t*, hipStream_t);
hipError_t launch_dispatch(const int32_t*, const float*, int, int, DispatchHeader*, int32_t*, float*, int32_t*,
                           hipStream_t);
hipError_t launch_gemm1_stream(const uint8_t*, const float*, int, const uint8_t*, const float*,
                               const DispatchHeader*, const int32_t*, uint16_t*, int, hipStream_t);
hipError_t launch_gemm2_stream(const uint16_t*, const uint8_t*, const float*, const DispatchHeader*, const float*,
                               float*, int, hipStream_t);
hipError_t launch_gemm1_tiled(const uint8_t*, const float*, int, const uint8_t*, const float*,
                              const DispatchHeader*, const int32_t*, uint16_t*, int, hipStream_t);
hipError_t launch_gemm2_tiled(const uint16_t*, const uint8_t*, const float*, const DispatchHeader*, const float*,
                              float*, int, hipStream_t);
hipError_t launch_combine(const float*, const int32_t*, int, uint16_t*, hipStream_t);
}  // namespace moe

namespace {

constexpr int kMaxDevices = 64;
constexpr int kStreamMaxTokens = 64;  // decode shape up to this many tokens
std::atomic<int> g_cu_count[kMaxDevices];
std::atomic<int> g_path{0};
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
  return moe::WorkspaceLayout::make(T).total;
}

}  // extern "C"

namespace {

// Records events[i] (when given) before stage i and events[5] after the last:
// route, dispatch, GEMM1+SwiGLU, GEMM2 x weight, combine.
int forward_impl(const float* routing_logits, const uint16_t* routing_bias, const uint8_t* hidden_states,
                 const float* hidden_states_scale, const uint8_t* gemm1_weights, const float* gemm1_weights_scale,
                 const uint8_t* gemm2_weights, const float* gemm2_weights_scale, int64_t T,
                 int64_t local_expert_offset, double routed_scaling_factor, uint16_t* output, void* workspace,
                 size_t workspace_bytes, void* stream, void* const* events) {
  using namespace moe;
  if (T < 0 || T > MOE_FP8_MAX_TOKENS) return MOE_ERR_SIZE;
  if (T == 0) return MOE_OK;
  if (!routing_logits || !routing_bias || !hidden_states || !hidden_states_scale || !gemm1_weights ||
      !gemm1_weights_scale || !gemm2_weights || !gemm2_weights_scale || !output || !workspace)
    return MOE_ERR_NULL;
  if (!aligned16(routing_logits) || !aligned16(routing_bias) || !aligned16(hidden_states) ||
      !aligned16(hidden_states_scale) || !aligned16(gemm1_weights) || !aligned16(gemm1_weights_scale) ||
      !aligned16(gemm2_weights) || !aligned16(gemm2_weights_scale) || !aligned16(output) || !aligned16(workspace))
    return MOE_ERR_ALIGN;
  const WorkspaceLayout L = WorkspaceLayout::make(T);
  if (workspace_bytes < L.total) return MOE_ERR_WORKSPACE;

  const int t = (int)T;
  const int off = clamp_offset(local_expert_offset);
  const float rsf = (float)routed_scaling_factor;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  auto* hdr = reinterpret_cast<DispatchHeader*>(ws + L.hdr);
  auto* topk_ids = reinterpret_cast<int32_t*>(ws + L.topk_ids);
  auto* topk_w = reinterpret_cast<float*>(ws + L.topk_w);
  auto* tok_pair = reinterpret_cast<int32_t*>(ws + L.tok_pair);
  auto* perm_tok = reinterpret_cast<int32_t*>(ws + L.perm_tok);
  auto* perm_w = reinterpret_cast<float*>(ws + L.perm_w);
  auto* c_act = reinterpret_cast<uint16_t*>(ws + L.c_act);
  auto* partial = reinterpret_cast<float*>(ws + L.partial);

  hipError_t e;
  auto mark = [&](int i) -> hipError_t {
    return events ? hipEventRecord(reinterpret_cast<hipEvent_t>(events[i]), s) : hipSuccess;
  };
  if ((e = mark(0)) != hipSuccess) return hip_fail(e);
  if ((e = launch_route(routing_logits, routing_bias, t, rsf, topk_ids, topk_w, tok_pair, s)) != hipSuccess)
    return hip_fail(e);
  if ((e = mark(1)) != hipSuccess) return hip_fail(e);
  if ((e = launch_dispatch(topk_ids, topk_w, t, off, hdr, perm_tok, perm_w, tok_pair, s)) != hipSuccess)
    return hip_fail(e);
  if ((e = mark(2)) != hipSuccess) return hip_fail(e);

  const int path = g_path.load(std::memory_order_relaxed);
  const bool stream_shape = path == 1 || (path == 0 && t <= kStreamMaxTokens);
  if (stream_shape) {
    const int max_active = t * TOP_K < E_LOCAL ? t * TOP_K : E_LOCAL;
    if ((e = launch_gemm1_stream(hidden_states, hidden_states_scale, t, gemm1_weights, gemm1_weights_scale, hdr,
                                 perm_tok, c_act, max_active, s)) != hipSuccess)
      return hip_fail(e);
    if ((e = mark(3)) != hipSuccess) return hip_fail(e);
    if ((e = launch_gemm2_stream(c_act, gemm2_weights, gemm2_weights_scale, hdr, perm_w, partial, max_active, s)) !=
        hipSuccess)
      return hip_fail(e);
  } else {
    const int grid = (cu_count() * 2 + 7) / 8 * 8;
    if ((e = launch_gemm1_tiled(hidden_states, hidden_states_scale, t, gemm1_weights, gemm1_weights_scale, hdr,
                                perm_tok, c_act, grid, s)) != hipSuccess)
      return hip_fail(e);
    if ((e = mark(3)) != hipSuccess) return hip_fail(e);
    if ((e = launch_gemm2_tiled(c_act, gemm2_weights, gemm2_weights_scale, hdr, perm_w, partial, grid, s)) !=
        hipSuccess)
      return hip_fail(e);
  }
  if ((e = mark(4)) != hipSuccess) return hip_fail(e);
  if ((e = launch_combine(partial, tok_pair, t, output, s)) != hipSuccess) return hip_fail(e);
  if ((e = mark(5)) != hipSuccess) return hip_fail(e);
  return MOE_OK;
}

}  // namespace

extern "C" {

int moe_fp8_forward(const float* routing_logits, const uint16_t* routing_bias, const uint8_t* hidden_states,
                    const float* hidden_states_scale, const uint8_t* gemm1_weights,
                    const float* gemm1_weights_scale, const uint8_t* gemm2_weights,
                    const float* gemm2_weights_scale, int64_t T, int64_t local_expert_offset,
                    double routed_scaling_factor, uint16_t* output, void* workspace, size_t workspace_bytes,
                    void* stream) {
  return forward_impl(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                      gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, T, local_expert_offset,
                      routed_scaling_factor, output, workspace, workspace_bytes, stream, nullptr);
}

int moe_fp8_forward_timed(const float* routing_logits, const uint16_t* routing_bias, const uint8_t* hidden_states,
                          const float* hidden_states_scale, const uint8_t* gemm1_weights,
                          const float* gemm1_weights_scale, const uint8_t* gemm2_weights,
                          const float* gemm2_weights_scale, int64_t T, int64_t local_expert_offset,
                          double routed_scaling_factor, uint16_t* output, void* workspace, size_t workspace_bytes,
                          void* stream, void* const* events) {
  if (!events) return MOE_ERR_NULL;
  for (int i = 0; i < 6; ++i)
    if (!events[i]) return MOE_ERR_NULL;
  return forward_impl(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                      gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, T, local_expert_offset,
                      routed_scaling_factor, output, workspace, workspace_bytes, stream, events);
}

int moe_fp8_route(const float* routing_logits, const uint16_t* routing_bias, int64_t T,
                  double routed_scaling_factor, int32_t* topk_ids, float* topk_w, int32_t* tok_pair,
                  void* stream) {
  if (T < 0 || T > MOE_FP8_MAX_TOKENS) return MOE_ERR_SIZE;
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
                     int32_t* header, int32_t* perm_tok, float* perm_w, int32_t* tok_pair, void* stream) {
  if (T < 0 || T > MOE_FP8_MAX_TOKENS) return MOE_ERR_SIZE;
  if (!header || !perm_tok || !perm_w || !tok_pair || (T > 0 && (!topk_ids || !topk_w))) return MOE_ERR_NULL;
  if (!aligned16(header) || !aligned16(perm_tok) || !aligned16(perm_w) || !aligned16(tok_pair) ||
      (T > 0 && (!aligned16(topk_ids) || !aligned16(topk_w))))
    return MOE_ERR_ALIGN;
  hipError_t e = moe::launch_dispatch(topk_ids, topk_w, (int)T, clamp_offset(local_expert_offset),
                                      reinterpret_cast<moe::DispatchHeader*>(header), perm_tok, perm_w, tok_pair,
                                      reinterpret_cast<hipStream_t>(stream));
  return e == hipSuccess ? MOE_OK : hip_fail(e);
}

int moe_fp8_set_path(int path) {
  if (path < 0 || path > 2) return -1;
  return g_path.exchange(path);
}

const char* moe_fp8_strerror(int code) {
  switch (code) {
    case MOE_OK: return "ok";
    case MOE_ERR_NULL: return "a required pointer is NULL";
    case MOE_ERR_SIZE: return "token count out of range";
    case MOE_ERR_ALIGN: return "a pointer is not 16-byte aligned";
    case MOE_ERR_WORKSPACE: return "workspace smaller than moe_fp8_workspace_size(T)";
    case MOE_ERR_HIP: return "HIP launch failed";
    default: return "unknown error";
  }
}

const char* moe_fp8_last_hip_error(void) { return t_last_hip_error; }

int moe_fp8_abi_version(void) { return 1; }

}  // extern "C"

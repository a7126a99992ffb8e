/*
 * C ABI of libmoe_mi355x.so: the FP8 block-scale DeepSeek-V3 MoE operator
 * "moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048" for one GPU's
 * 32-local-expert share, built for MI355X (gfx950).
 *
 * All tensor arguments are device pointers to row-major contiguous buffers,
 * 16-byte aligned. Nothing here allocates, synchronises the host or throws:
 * work is enqueued on `stream` (a hipStream_t, NULL = default stream) and
 * errors come back as negative return codes (see moe_fp8_strerror).
 * Calls on different streams are independent when each passes its own
 * workspace; the only process-global state is per-device set-up done once
 * (the compute-unit count, kernel attributes), safe under concurrent callers.
 *
 * Routing ties: when equal scores straddle the top-4-group or the top-8-expert
 * cut, the experts kept are the ones the reference keeps when it runs on the
 * CPU (torch.topk(sorted=False) there is libstdc++'s std::nth_element, which
 * the kernels replay). The reference run on a CUDA device breaks such ties by
 * its own selection algorithm, which no fixture here pins: on exact ties,
 * agreement with a CUDA-run reference is not established.
 */
#ifndef MOE_FP8_H
#define MOE_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MOE_OK = 0,
  MOE_ERR_NULL = -1,      /* a required pointer is NULL */
  MOE_ERR_SIZE = -2,      /* T < 0 or T beyond MOE_FP8_MAX_TOKENS (MOE_FP8_MAX_TAP_TOKENS for the
                             entry points other than the forward) */
  MOE_ERR_ALIGN = -3,     /* a pointer is not 16-byte aligned */
  MOE_ERR_WORKSPACE = -4, /* workspace_bytes < moe_fp8_workspace_size(T), or a dispatch
                             header shorter than MOE_FP8_DISPATCH_HEADER_WORDS(T) */
  MOE_ERR_HIP = -5,       /* a HIP launch failed; see moe_fp8_last_hip_error() */
  MOE_ERR_ARG = -6,       /* an enumerated argument (stage, shape) is out of range */
  MOE_ERR_NOALLOC_SIZE = -7 /* T beyond MOE_FP8_NOALLOC_MAX_TOKENS in moe_fp8_forward_noalloc */
};

/* Kernel shape of the expert GEMMs, for the test and benchmark entry points
 * below (moe_fp8_forward always uses MOE_SHAPE_AUTO): the decode kernels for
 * T <= MOE_FP8_DECODE_MAX_TOKENS and the prefill kernels above (AUTO), or the
 * prefill kernels at any T. */
enum { MOE_SHAPE_AUTO = 0, MOE_SHAPE_PREFILL = 1 };
#define MOE_FP8_DECODE_MAX_TOKENS 96

/* Largest T the forward entry points accept (they run calls above
 * MOE_FP8_CHUNK_TOKENS chunk by chunk), and the largest T of every other entry
 * point (routing, dispatch, the producer-side kernels), whose 32-bit offsets
 * cover T * 7168 * 2 bytes. */
#define MOE_FP8_MAX_TOKENS (1 << 20)
#define MOE_FP8_MAX_TAP_TOKENS (1 << 17)

/* Forward calls above this many tokens run the operator over consecutive token
 * chunks of this size (the last one shorter), in one chunk's workspace: the
 * worst-case workspace (8 local pairs per token, an fp16 row of C and of the
 * weighted GEMM2 output for every pair) is about 144 KB per token, 2.4 GB for
 * one chunk. Tokens are independent, so the output is bit for bit the
 * unchunked one. */
#define MOE_FP8_CHUNK_TOKENS (1 << 14)

/* Words of the `header` buffer moe_fp8_dispatch and moe_fp8_route_dispatch take
 * for T tokens: the dispatch header (MOE_FP8_HEADER_WORDS) followed by 32 counts
 * per group of 16 tokens, which the counting and the scatter kernels exchange.
 * Both entry points take the buffer's size and return MOE_ERR_WORKSPACE when it
 * is shorter than this. */
#define MOE_FP8_HEADER_WORDS 128
#define MOE_FP8_DISPATCH_HEADER_WORDS(T) (MOE_FP8_HEADER_WORDS + 32 * (((T) + 15) / 16))

/* Bytes of device workspace one forward call needs for T tokens (worst case
 * of 8 routed local pairs per token; for T above MOE_FP8_CHUNK_TOKENS the size
 * for one chunk). */
size_t moe_fp8_workspace_size(int64_t T);

/*
 * Whole operator, destination-passing style.
 * Replaces the reference's C++ entry point
 *   void kernel(at::Tensor routing_logits, at::Tensor routing_bias,
 *               at::Tensor hidden_states, at::Tensor hidden_states_scale,
 *               at::Tensor gemm1_weights, at::Tensor gemm1_weights_scale,
 *               at::Tensor gemm2_weights, at::Tensor gemm2_weights_scale,
 *               int64_t local_expert_offset, double routed_scaling_factor,
 *               at::Tensor output)                 (solution/cuda/kernel_v2.cu:146-158)
 * and the Python `kernel(..., output)` of solution/triton/kernel.py:292-305,
 * with the reference semantics of reference moe/ref_moe.py:4-168.
 *
 *   routing_logits       fp32 [T, 256]
 *   routing_bias         bf16 [256] (raw bits)
 *   hidden_states        e4m3 [T, 7168] (raw bytes)
 *   hidden_states_scale  fp32 [56, T]   (one scale per 1x128 block, transposed)
 *   gemm1_weights        e4m3 [32, 4096, 7168]; gemm1_weights_scale fp32 [32, 32, 56]
 *   gemm2_weights        e4m3 [32, 7168, 2048]; gemm2_weights_scale fp32 [32, 56, 16]
 *   output               bf16 [T, 7168] (raw bits), written in full
 * Local experts are global ids [local_expert_offset, local_expert_offset + 32)
 * clipped to [0, 256); tokens with no local expert get zeros.
 */
int moe_fp8_forward(const float* routing_logits, const uint16_t* routing_bias, const uint8_t* hidden_states,
                    const float* hidden_states_scale, const uint8_t* gemm1_weights,
                    const float* gemm1_weights_scale, const uint8_t* gemm2_weights,
                    const float* gemm2_weights_scale, int64_t T, int64_t local_expert_offset,
                    double routed_scaling_factor, uint16_t* output, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * moe_fp8_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid allocation). No counterpart in the reference. The workspace is a
 * library-owned device array of about 2.1 MB that each GPU holds from the first
 * call on it until the process ends; nothing here allocates. Limits:
 *   - T <= MOE_FP8_NOALLOC_MAX_TOKENS (64, the decode kernels); larger T returns
 *     MOE_ERR_NOALLOC_SIZE (use moe_fp8_forward with a workspace);
 *   - every call on one GPU shares that GPU's array: calls that overlap on one
 *     GPU (e.g. on two streams without ordering between them) race and give
 *     wrong results; order them on one stream.
 * Results are bit-identical to moe_fp8_forward's on the same inputs.
 */
#define MOE_FP8_NOALLOC_MAX_TOKENS 64
int moe_fp8_forward_noalloc(const float* routing_logits, const uint16_t* routing_bias, const uint8_t* hidden_states,
                            const float* hidden_states_scale, const uint8_t* gemm1_weights,
                            const float* gemm1_weights_scale, const uint8_t* gemm2_weights,
                            const float* gemm2_weights_scale, int64_t T, int64_t local_expert_offset,
                            double routed_scaling_factor, uint16_t* output, void* stream);

/*
 * moe_fp8_forward with the expert-GEMM kernel shape chosen per call (one of
 * MOE_SHAPE_*). No reference counterpart: tests run both kernel shapes on the
 * same inputs. Everything else as moe_fp8_forward.
 */
int moe_fp8_forward_shape(int shape, const float* routing_logits, const uint16_t* routing_bias,
                          const uint8_t* hidden_states, const float* hidden_states_scale,
                          const uint8_t* gemm1_weights, const float* gemm1_weights_scale,
                          const uint8_t* gemm2_weights, const float* gemm2_weights_scale, int64_t T,
                          int64_t local_expert_offset, double routed_scaling_factor, uint16_t* output,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * Runs one stage of moe_fp8_forward_shape(shape, ...) with the same arguments, reading and
 * writing the workspace as the forward does: 0 = routing (+ dispatch in the
 * prefill shape), 1 = GEMM1 + SwiGLU (+ the in-workgroup dispatch in the decode
 * shape), 2 = GEMM2 x routing weight (+ the ordered combine in the decode
 * shape), 3 = the combine (prefill shape; nothing in the decode shape, i.e.
 * MOE_SHAPE_AUTO with T <= MOE_FP8_DECODE_MAX_TOKENS). A stage's inputs must already be in
 * the workspace (a moe_fp8_forward with the same arguments ran on it); T at most
 * MOE_FP8_CHUNK_TOKENS (MOE_ERR_SIZE above: the forward would run chunks). No
 * reference counterpart (the reference timed its stages with torch.profiler,
 * scripts/ncu_profile.py:89-143): the benchmark times each kernel over many
 * back-to-back launches of its stage.
 */
int moe_fp8_run_stage(int stage, int shape, const float* routing_logits, const uint16_t* routing_bias,
                      const uint8_t* hidden_states, const float* hidden_states_scale, const uint8_t* gemm1_weights,
                      const float* gemm1_weights_scale, const uint8_t* gemm2_weights,
                      const float* gemm2_weights_scale, int64_t T, int64_t local_expert_offset,
                      double routed_scaling_factor, uint16_t* output, void* workspace, size_t workspace_bytes,
                      void* stream);

/*
 * Routing stage alone (reference moe/ref_moe.py:94-126; the sigmoid/bias kernel
 * and top-k chain of solution/cuda/kernel_v2.cu:170-206).
 * Writes, per token, the 8 selected global expert ids in ascending order
 * (int32 [T, 8]) and their routing weights (fp32 [T, 8]). If tok_pair is not
 * NULL every one of its T*8 slots is set to -1. Where equal scores straddle the
 * group or expert cut, the kept set is the one the reference's
 * torch.topk(sorted=False) keeps on the CPU (std::nth_element's order).
 */
int moe_fp8_route(const float* routing_logits, const uint16_t* routing_bias, int64_t T,
                  double routed_scaling_factor, int32_t* topk_ids, float* topk_w, int32_t* tok_pair,
                  void* stream);

/*
 * Dispatch stage alone (reference moe/ref_moe.py:131-145; the nonzero / sort /
 * cumsum dispatch of solution/cuda/kernel_v2.cu:208-244, without its host sync).
 * From the routing stage's ids and weights, writes
 *   header   int32 [MOE_FP8_DISPATCH_HEADER_WORDS(T)]: counts[32], seg_start[33]
 *            (seg_start[32] = P), n_active, active[32] (local ids with tokens,
 *            ascending), padding to 128 words, then the per-chunk counts
 *   perm_tok int32 [8T]: for each local expert in order, its tokens ascending
 *   perm_w   fp32  [8T]: the routing weight of each (token, expert) pair
 *   tok_pair int32 [T, 8]: pair index of slot j of token t; must hold -1 on
 *            entry (moe_fp8_route sets that), local slots are overwritten.
 */
int moe_fp8_dispatch(const int32_t* topk_ids, const float* topk_w, int64_t T, int64_t local_expert_offset,
                     int32_t* header, size_t header_words, int32_t* perm_tok, float* perm_w, int32_t* tok_pair,
                     void* stream);

/*
 * Routing and dispatch as moe_fp8_forward_shape(shape, ...) runs them (in the
 * decode shape the routing kernel plus, in one workgroup, the dispatch code
 * every decode GEMM1 workgroup runs; otherwise the two kernels above), writing
 * topk_ids / topk_w [T, 8], header [MOE_FP8_DISPATCH_HEADER_WORDS(T)], perm_tok / perm_w [8T] and
 * tok_pair [T, 8] (fully written: -1 for non-local slots). Parity tap for
 * reference moe/ref_moe.py:94-145.
 */
int moe_fp8_route_dispatch(int shape, const float* routing_logits, const uint16_t* routing_bias, int64_t T,
                           int64_t local_expert_offset, double routed_scaling_factor, int32_t* topk_ids,
                           float* topk_w, int32_t* header, size_t header_words, int32_t* perm_tok, float* perm_w,
                           int32_t* tok_pair, void* stream);

/*
 * Producer-side FP8 activation quantiser (the step before this operator:
 * reference moe/weight_origins_dataflow.md:19-21, :131-142; its formula as in
 * solution/triton/dsl-temp1.py:479-484). Per 1 x 128 block of the bf16 hidden
 * states [T, 7168]: amax = max |x| clamped below at 1e-12, scale = amax / 448,
 * q = e4m3(x / scale) with round to nearest even. Writes hidden_states e4m3
 * [T, 7168] and hidden_states_scale fp32 [56, T] (transposed), i.e. exactly
 * the operator's hidden_states / hidden_states_scale inputs. Stream-ordered.
 */
int moe_fp8_quantize_activations(const uint16_t* hidden_bf16, int64_t T, uint8_t* hidden_states,
                                 float* hidden_states_scale, void* stream);

/*
 * Router GEMM, the linear layer that produces this operator's routing_logits
 * input (reference moe/weight_origins_dataflow.md:21, :151-154: "x @
 * gate_weight.T (linear layer, no activation)"): routing_logits fp32 [T, 256] =
 * hidden_bf16 [T, 7168] x gate_weight^T, gate_weight bf16 [256, 7168]; the
 * products are exact in fp32 and summed in fp32 in a fixed order (the same
 * logits on every call). All pointers 16-byte aligned. Stream-ordered.
 */
int moe_fp8_router_logits(const uint16_t* hidden_bf16, const uint16_t* gate_weight, int64_t T,
                          float* routing_logits, void* stream);

/*
 * Both producer-side steps (the router GEMM of moe_fp8_router_logits and the
 * quantiser of moe_fp8_quantize_activations, reference
 * moe/weight_origins_dataflow.md:19-21 and :21, :151-154, which read the same
 * x): one pass over the bf16 hidden states below 576 tokens, the two kernels
 * in turn from 576 on; writes the same routing_logits, hidden_states and
 * hidden_states_scale, bit for bit, as the two separate calls. All pointers
 * 16-byte aligned. Stream-ordered.
 */
int moe_fp8_router_quantize(const uint16_t* hidden_bf16, const uint16_t* gate_weight, int64_t T,
                            float* routing_logits, uint8_t* hidden_states, float* hidden_states_scale, void* stream);

const char* moe_fp8_strerror(int code);
const char* moe_fp8_last_hip_error(void);
int moe_fp8_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MOE_FP8_H */

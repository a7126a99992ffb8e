// Shared constants, vector types and device helpers for the FP8 block-scale
// DeepSeek-V3 MoE kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

// Fixed operator geometry (reference moe/ref_moe.py:33-54).
constexpr int H = 7168;            // hidden size
constexpr int I = 2048;            // intermediate size
constexpr int N1 = 2 * I;          // gemm1 output width (first half X1, second half X2)
constexpr int E_GLOBAL = 256;
constexpr int E_LOCAL = 32;
constexpr int TOP_K = 8;
constexpr int N_GROUP = 8;
constexpr int TOPK_GROUP = 4;
constexpr int GROUP_SIZE = E_GLOBAL / N_GROUP;  // 32
constexpr int BLK = 128;           // quantisation block edge
constexpr int NB_H = H / BLK;      // 56
constexpr int NB_I = I / BLK;      // 16
constexpr int NB_N1 = N1 / BLK;    // 32

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// Device-side dispatch header at the start of the workspace.
struct DispatchHeader {
  int32_t counts[E_LOCAL];         // tokens per local expert
  int32_t seg_start[E_LOCAL + 1];  // exclusive scan of counts; seg_start[32] = P
  int32_t n_active;                // experts with count > 0
  int32_t active[E_LOCAL];         // their local ids, ascending
  int32_t pad[256 / 4 * 2 - (E_LOCAL * 3 + 2)];
};
static_assert(sizeof(DispatchHeader) == 512, "header is 512 bytes");

// One MFMA over a full 128-wide K block: D(16x16 fp32) = A(16x128 e4m3) * B(128x16 e4m3).
// Lane l holds row (l % 16) of A / column (l % 16) of B and the 32 K values
// [32*(l/16), 32*(l/16)+32); the result holds rows 4*(l/16)+r, column l % 16.
// E8M0 scale 127 is 2^0: block scales are applied in fp32 by the caller.
__device__ __forceinline__ v4f mfma_fp8_k128(const v8i& a, const v8i& b) {
  v4f z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 127, 0, 127);
}

// D += A(16x32 bf16) * B(32x16 bf16); lane l holds row/column l % 16 and
// K values [8*(l/16), 8*(l/16)+8).
__device__ __forceinline__ v4f mfma_bf16_k32(const v8bf& a, const v8bf& b, const v4f& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// D += A(16x32 fp16) * B(32x16 fp16); the same lane layout as mfma_bf16_k32.
__device__ __forceinline__ v4f mfma_f16_k32(const v8h& a, const v8h& b, const v4f& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Eight e4m3 codes (two dwords) -> eight fp16 in K order, exactly: every e4m3 value
// (at most 448 in magnitude, subnormals down to 2^-9) is an fp16 value.
// v_cvt_scalef32_pk_f16_fp8 with scale 1.0 converts the two codes of one 16-bit half
// (checked on the GPU against the OCP table for all 256 codes in all 4 byte positions).
__device__ __forceinline__ v8h fp8x8_to_f16x8(uint32_t w0, uint32_t w1) {
  const v2h a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false);
  const v2h b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true);
  const v2h c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false);
  const v2h d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true);
  return v8h{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// The SwiGLU output C (the GEMM2 activation operand) is stored as fp16 of C * 2^-8:
// 11 significant bits for |C| in [2^-6, 2^24) and an absolute step of 2^-24 * 2^8
// below (bf16 keeps 8 bits, and its rounding of C moved a few outputs of a skewed
// routing past the 1e-2 / 2e-2 bar through cancellation across experts). Values
// beyond the fp16 range saturate to +-65504 * 2^8; NaN stays NaN. GEMM2 multiplies
// its fp32 accumulators by 2^8 together with the weight block scale.
constexpr float C_STORE_SCALE = 1.0f / 256.0f;
constexpr float C_LOAD_SCALE = 256.0f;
__device__ __forceinline__ uint16_t c_encode(float c) {
  const float x = c * C_STORE_SCALE;  // exact: a power of two
  const float y = x != x ? x : fminf(fmaxf(x, -65504.0f), 65504.0f);
  return __builtin_bit_cast(uint16_t, (_Float16)y);  // round to nearest even
}

// Barrier for LDS traffic only. __syncthreads() also orders global memory, and
// since global stores count in vmcnt like loads, it waits for every load in
// flight (prefetched weights, say) whenever a store precedes it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// fp32 -> bf16 bits, round to nearest even (quiet NaN kept NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__host__ __device__ constexpr size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Dispatch (prefill shape): the routing kernel counts, per group of
// COUNT_ROW_TOKENS tokens (one workgroup), the tokens that selected each local
// expert (a row of 32 counts); the scatter kernel works on chunks of
// DISPATCH_CHUNK tokens and sums the rows of all groups and of those before it.
constexpr int DISPATCH_CHUNK = 256;
constexpr int COUNT_ROW_TOKENS = 16;
__host__ __device__ constexpr int dispatch_chunks(int64_t T) { return (int)((T + DISPATCH_CHUNK - 1) / DISPATCH_CHUNK); }
__host__ __device__ constexpr int count_rows(int64_t T) { return (int)((T + COUNT_ROW_TOKENS - 1) / COUNT_ROW_TOKENS); }

// Workspace layout for T tokens (worst case P = 8T routed pairs). The pair rows
// (fp16 of w * O * 2^-8, one per pair) and the dispatch's count rows come last:
// only the prefill kernels use them, so a decode-shape call needs `total` bytes
// of make(T, false) (the same offsets, without those regions).
struct WorkspaceLayout {
  size_t hdr = 0, topk_ids = 0, topk_w = 0, tok_pair = 0, perm_tok = 0, perm_w = 0, c_act = 0, partial = 0,
         chunk_counts = 0, total = 0;
  __host__ __device__ static constexpr WorkspaceLayout make(int64_t T, bool with_partial = true) {
    WorkspaceLayout L;
    const size_t P = (size_t)T * TOP_K;
    size_t o = 0;
    L.hdr = o;      o += align_up(sizeof(DispatchHeader), 256);
    L.topk_ids = o; o += align_up((size_t)T * TOP_K * 4, 256);
    L.topk_w = o;   o += align_up((size_t)T * TOP_K * 4, 256);
    L.tok_pair = o; o += align_up((size_t)T * TOP_K * 4, 256);
    L.perm_tok = o; o += align_up(P * 4, 256);
    L.perm_w = o;   o += align_up(P * 4, 256);
    L.c_act = o;    o += align_up(P * I * 2, 256);
    L.partial = o;  o += with_partial ? align_up(P * H * 2, 256) : 0;
    L.chunk_counts = o; o += with_partial ? align_up((size_t)count_rows(T) * E_LOCAL * 4, 256) : 0;
    L.total = o;
    return L;
  }
};

}  // namespace moe

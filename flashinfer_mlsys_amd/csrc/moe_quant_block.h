// The arithmetic of one 1 x 128 activation block's FP8 quantisation (reference
// solution/triton/dsl-temp1.py:479-484), shared by the quantiser kernel and the
// router GEMM's fused path so that both write the same bytes:
//   scale = max(amax, 1e-12) / 448
//   code  = e4m3(clamp(x / scale, -448, 448)), IEEE fp32 division, round to
//           nearest even (v_cvt_pk_fp8_f32).
#pragma once

#include "moe_common.h"

namespace moe {

__device__ __forceinline__ float qblock_scale(float amax) { return fmaxf(amax, 1e-12f) / 448.0f; }

// Four values -> four e4m3 codes, first value in the low byte.
__device__ __forceinline__ uint32_t qblock_pack4(float a, float b, float c, float d, float s) {
  const float qa = fminf(fmaxf(a / s, -448.f), 448.f), qb = fminf(fmaxf(b / s, -448.f), 448.f);
  const float qc = fminf(fmaxf(c / s, -448.f), 448.f), qd = fminf(fmaxf(d / s, -448.f), 448.f);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(qa, qb, 0, false) & 0xffffu;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(qc, qd, 0, false) & 0xffffu;
  return lo | (hi << 16);
}

// Eight bf16 (two per 32-bit word, first in the low half) -> fp32.
__device__ __forceinline__ void bf16x8_to_f32(const uint32_t (&w)[4], float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

}  // namespace moe

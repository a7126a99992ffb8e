// Producer-side FP8 activation quantiser: bf16 hidden states [T, 7168] ->
// OCP e4m3 [T, 7168] + fp32 block scales [56, T] (the operator's input layout,
// scales transposed), per 1 x 128 block (reference
// solution/triton/dsl-temp1.py:479-484, the same quantisation the operator's
// inputs carry):
//   amax  = max |x| over the block (fp32), clamped below at 1e-12
//   scale = amax / 448
//   q     = e4m3(x / scale), round to nearest even (IEEE fp32 division first)
// |x / scale| <= 448 up to the division's rounding; the value is clamped to
// +-448 before the conversion, which rounds exactly like torch's cast to
// float8_e4m3fn (checked on every e4m3 value, every midpoint and its fp32
// neighbours).
//
// HBM-bound byte work: one workgroup (4 waves) per 16 tokens x 8 blocks (grid
// ceil(T / 16) x 7, so even a few tokens spread over many CUs); wave w takes
// tokens 4w..4w+3, 16 lanes per (token, block), each lane 8 elements (16 B in,
// 8 B out). The 4 scales a wave writes per block are 4 consecutive floats of
// the transposed scale array.
#include "moe_common.h"

namespace moe {

constexpr int QA_TOK = 16;  // tokens per workgroup
constexpr int QA_KB = 8;    // blocks per workgroup
static_assert(NB_H % QA_KB == 0, "block groups");

__global__ __launch_bounds__(256) void quantize_1x128_kernel(const uint16_t* __restrict__ x, int T,
                                                             uint8_t* __restrict__ q, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane >> 4, r = lane & 15;
  const int t = blockIdx.x * QA_TOK + wave * 4 + sub;
  const bool valid = t < T;
  const uint16_t* xr = x + (size_t)(valid ? t : 0) * H + r * 8;
  uint8_t* qr = q + (size_t)(valid ? t : 0) * H + r * 8;
#pragma unroll
  for (int kb = blockIdx.y * QA_KB; kb < (int)(blockIdx.y + 1) * QA_KB; ++kb) {
    float v[8];
    float m = 0.f;
    if (valid) {
      const uint4 raw = *reinterpret_cast<const uint4*>(xr + kb * BLK);
      const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    }
    // block max over the 16 lanes of this (token, block)
#pragma unroll
    for (int k = 1; k < 16; k <<= 1) m = fmaxf(m, __shfl_xor(m, k));
    const float s = fmaxf(m, 1e-12f) / 448.0f;
    if (valid) {
      uint32_t packed[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float a = fminf(fmaxf(v[4 * i] / s, -448.f), 448.f);
        const float b = fminf(fmaxf(v[4 * i + 1] / s, -448.f), 448.f);
        const float c = fminf(fmaxf(v[4 * i + 2] / s, -448.f), 448.f);
        const float d = fminf(fmaxf(v[4 * i + 3] / s, -448.f), 448.f);
        const uint32_t lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
        const uint32_t hi = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, 0, false) & 0xffffu;
        packed[i] = lo | (hi << 16);
      }
      *reinterpret_cast<uint2*>(qr + kb * BLK) = uint2{packed[0], packed[1]};
      if (r == 0) scale[(size_t)kb * T + t] = s;
    }
  }
}

hipError_t launch_quantize_1x128(const uint16_t* x, int T, uint8_t* q, float* scale, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(quantize_1x128_kernel, dim3((T + QA_TOK - 1) / QA_TOK, NB_H / QA_KB), dim3(256), 0, stream, x, T,
                     q, scale);
  return hipGetLastError();
}

}  // namespace moe

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
#include "moe_quant_block.h"

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
      bf16x8_to_f32(w, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    }
    // block max over the 16 lanes of this (token, block)
#pragma unroll
    for (int k = 1; k < 16; k <<= 1) m = fmaxf(m, __shfl_xor(m, k));
    const float s = qblock_scale(m);
    if (valid) {
      const uint32_t p0 = qblock_pack4(v[0], v[1], v[2], v[3], s), p1 = qblock_pack4(v[4], v[5], v[6], v[7], s);
      *reinterpret_cast<uint2*>(qr + kb * BLK) = uint2{p0, p1};
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

// Tile helpers shared by the LDS-staged kernels: the XCD-aware workgroup
// order, direct global -> LDS loads, the 32-row swizzle, the 32x32 bf16 / fp16 MFMAs.
#pragma once

#include "moe_common.h"

namespace moe {

// Workgroup b of G (G a multiple of 8) -> item index such that the G/8
// workgroups of one XCD (hardware places workgroup b on XCD b % 8) get
// consecutive indices.
__device__ __forceinline__ int xcd_remap(int b, int G) { return (b & 7) * (G >> 3) + (b >> 3); }

// Direct global -> LDS loads: lane l's 16 (or 4) bytes land at lds_dst + 16 l (4 l);
// lds_dst must be uniform over the wave. The compiler does not track these LDS
// writes: readers wait with an explicit s_waitcnt vmcnt.
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ void lds_direct16(const void* gsrc, uint8_t* lds_dst) {
  __builtin_amdgcn_global_load_lds(gsrc, (lds_void_t*)lds_dst, 16, 0, 0);
}
__device__ __forceinline__ void lds_direct4(const void* gsrc, uint8_t* lds_dst) {
  __builtin_amdgcn_global_load_lds(gsrc, (lds_void_t*)lds_dst, 4, 0, 0);
}

typedef float v16f __attribute__((ext_vector_type(16)));

// D += A(32x16 bf16) * B(16x32 bf16); lane l holds row/column l % 32 and K values
// [8 (l / 32), 8 (l / 32) + 8); output element i of lane l is row
// 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32.
__device__ __forceinline__ v16f mfma_bf16_32x32x16(const v8bf& a, const v8bf& b, const v16f& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// The same with fp16 operands.
__device__ __forceinline__ v16f mfma_f16_32x32x16(const v8h& a, const v8h& b, const v16f& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Offset of row r (0..31), 16 B chunk c (0..7) in a 32-row x 128 B region
// written by 4 direct loads (load j: rows 8 j..8 j+7, lane l: row 8 j + l / 8,
// chunk (l % 8) ^ (l / 8) ^ (j % 2), at 1024 j + 16 l).
__device__ __forceinline__ int sw32(int r, int c) {
  const int j = r >> 3, rr = r & 7;
  return j * 1024 + 16 * (8 * rr + (c ^ rr ^ (j & 1)));
}

}  // namespace moe

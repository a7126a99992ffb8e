// Router GEMM: routing_logits [T, 256] fp32 = hidden [T, 7168] bf16 x gate [256, 7168]^T bf16,
// the linear layer that produces the operator's routing_logits input (reference
// moe/weight_origins_dataflow.md:21, :151-154: "x @ gate_weight.T (linear layer,
// no activation)"). bf16 x bf16 products are exact in fp32; sums run in fp32 on the
// bf16 MFMA (v_mfma_f32_16x16x32_bf16).
//
// Small T (< 576 tokens): one launch; a workgroup computes 16 tokens x 16 experts
// over the whole K, its 8 waves taking 7 of the 56 K blocks each with operands
// loaded straight into MFMA fragment registers (all 56 loads in flight at once),
// then the 8 partial tiles are added through LDS in wave order (deterministic, no
// atomics, no workspace).
//
// With QUANT the small-T kernel also writes the operator's FP8 activation inputs
// (e4m3 rows [T, 7168] and 1 x 128 block scales [56, T]) from the hidden states
// it reads anyway, with the quantiser kernel's arithmetic, each (token, K block)
// exactly once: the workgroup of expert tile y quantises the K blocks kb with
// kb % 16 == y from the fragments it holds (one pass over x instead of two:
// 15 us instead of 20 at T=64). From RT2_MIN_T tokens on the two producer steps
// run as the tiled kernel and the quantiser kernel: the same quantisation inside
// the tiled kernel's compute waves (2 per SIMD, next to the loader waves) cost
// more than the separate quantiser (84 against 49 + 40 us at T=8192).
//
// Larger T: LDS-staged tiles of 128 tokens x 64 experts, 8 compute waves of
// 32 x 32 (v_mfma_f32_32x32x16_bf16) and 4 loader waves that stream each 128-wide
// K block (hidden rows and gate rows, whole 128 B lines, 32-row swizzle) into a
// 3-slot LDS ring two blocks ahead, as the prefill GEMM1 does. Between 576 tokens
// and the token count whose 32-token items fill the CUs once (2,048 on 256 CUs),
// router_ksplit_kernel: 32 x 64 tiles, a 5-slot ring, each K block's MFMA steps
// split over the 8 compute waves and the four K quarters added in LDS in a
// fixed order.
#include "moe_common.h"
#include "moe_host.h"
#include "moe_tile.h"
#include "moe_quant_block.h"

namespace moe {

constexpr int RT_M = 16;  // tokens per small-T tile

__device__ __forceinline__ v8bf load_bf16x8(const uint16_t* p) {
  return __builtin_bit_cast(v8bf, *reinterpret_cast<const v4i*>(p));
}

constexpr int RS_WAVES = 8;
constexpr int RS_KPW = NB_H / RS_WAVES;  // 7 K blocks per wave

template <bool QUANT>
__global__ __launch_bounds__(64 * RS_WAVES) void router_small_kernel(const uint16_t* __restrict__ x,
                                                                     const uint16_t* __restrict__ g, int T,
                                                                     float* __restrict__ logits, uint8_t* __restrict__ q,
                                                                     float* __restrict__ qs) {
  __shared__ float red[RS_WAVES][4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int fr = lane & 15, kg = lane >> 4;
  const int t0 = blockIdx.x * RT_M, e0 = blockIdx.y * 16;
  const int k0 = wave * RS_KPW * BLK;
  const uint16_t* xp = x + (size_t)min(t0 + fr, T - 1) * H + k0 + 8 * kg;
  const uint16_t* gp = g + (size_t)(e0 + fr) * H + k0 + 8 * kg;
  v8bf a[RS_KPW][4], b[RS_KPW][4];
#pragma unroll
  for (int kk = 0; kk < RS_KPW; ++kk)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      a[kk][s] = load_bf16x8(xp + kk * BLK + 32 * s);
      b[kk][s] = load_bf16x8(gp + kk * BLK + 32 * s);
    }
  __builtin_amdgcn_sched_barrier(0);  // all 56 loads in flight before the first product waits
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < RS_KPW; ++kk)
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = mfma_bf16_k32(a[kk][s], b[kk][s], acc);
#pragma unroll
  for (int r = 0; r < 4; ++r) red[wave][r][lane] = acc[r];
  if (QUANT) {
    // lane (fr, kg) holds K 32 s + 8 kg + [0, 8) of token row fr for s = 0..3; the
    // row's 4 lanes are fr, fr + 16, fr + 32, fr + 48
    const int t = t0 + fr;
#pragma unroll
    for (int kk = 0; kk < RS_KPW; ++kk) {
      const int kb = wave * RS_KPW + kk;
      if (kb % 16 != (int)blockIdx.y) continue;  // wave-uniform
      float v[4][8];
      float m = 0.f;
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const v4i w = __builtin_bit_cast(v4i, a[kk][s4]);
        const uint32_t wu[4] = {(uint32_t)w[0], (uint32_t)w[1], (uint32_t)w[2], (uint32_t)w[3]};
        bf16x8_to_f32(wu, v[s4]);
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[s4][i]));
      }
      m = fmaxf(m, __shfl_xor(m, 16));
      m = fmaxf(m, __shfl_xor(m, 32));
      const float sc = qblock_scale(m);
      if (t < T) {
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          const uint32_t p0 = qblock_pack4(v[s4][0], v[s4][1], v[s4][2], v[s4][3], sc);
          const uint32_t p1 = qblock_pack4(v[s4][4], v[s4][5], v[s4][6], v[s4][7], sc);
          *reinterpret_cast<uint2*>(q + (size_t)t * H + kb * BLK + 32 * s4 + 8 * kg) = uint2{p0, p1};
        }
        if (kg == 0) qs[(size_t)kb * T + t] = sc;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x < 256) {  // entry (r, lane): token row 4 (lane / 16) + r, expert column lane % 16
    const int r = threadIdx.x >> 6, ln = threadIdx.x & 63;
    float v = red[0][r][ln];
#pragma unroll
    for (int w = 1; w < RS_WAVES; ++w) v += red[w][r][ln];
    const int t = t0 + 4 * (ln >> 4) + r;
    if (t < T) logits[(size_t)t * E_GLOBAL + e0 + (ln & 15)] = v;
  }
}

constexpr int RT2_BM = 128;                                  // tokens per item
constexpr int RT2_BN = 64;                                   // experts per item
constexpr int RT2_NT = E_GLOBAL / RT2_BN;                    // 4 expert tiles
constexpr int RT2_REG = 4096;                                // 32 rows x 128 B
constexpr int RT2_A_BYTES = RT2_BM * BLK * 2;                // 32 KB: 4 row blocks x 2 lines
constexpr int RT2_STAGE = RT2_A_BYTES + RT2_BN * BLK * 2;    // + 16 KB: 2 row blocks x 2 lines
constexpr int RT2_NSTAGE = 3;
constexpr int RT2_CWAVES = 8, RT2_PWAVES = 4;
constexpr int RT2_JOBS = RT2_STAGE / 1024 / RT2_PWAVES;      // 12 load instructions per loader wave per block
constexpr int RT2_MIN_T = 576;
static_assert(RT2_JOBS * RT2_PWAVES * 1024 == RT2_STAGE, "load split");

__global__ __launch_bounds__(64 * (RT2_CWAVES + RT2_PWAVES), 1) void router_tiled_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ g, int T, float* __restrict__ logits) {
  extern __shared__ __attribute__((aligned(16))) uint8_t rt_lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int total = (T + RT2_BM - 1) / RT2_BM * RT2_NT;
  const int first = xcd_remap(blockIdx.x, gridDim.x);
  int n_items = 0;
  for (int item = first; item < total; item += gridDim.x) ++n_items;
  const int G = n_items * NB_H;

  if (wave >= RT2_CWAVES) {
    // loader wave p: jobs 12 p .. 12 p + 11 of the 48 per block (0-31 hidden rows,
    // 32-47 gate rows); a job moves 8 rows x 128 B (one line of a K block)
    const int p = wave - RT2_CWAVES, ld_row = lane >> 3;
    const uint8_t* src[RT2_JOBS];
    int dst[RT2_JOBS];
    int item = first - (int)gridDim.x, kb = NB_H, slot = 0;
    auto next_item = [&]() {
      item += gridDim.x;
      const int mt = item / RT2_NT, nt = item % RT2_NT;
#pragma unroll
      for (int i = 0; i < RT2_JOBS; ++i) {
        const int job = p * RT2_JOBS + i, rg = job & 3, h = (job >> 2) & 1;
        const int chunk = (lane & 7) ^ ld_row ^ (rg & 1);
        if (job < 32) {
          const int ib = job >> 3;
          const int row = min(mt * RT2_BM + ib * 32 + rg * 8 + ld_row, T - 1);
          src[i] = reinterpret_cast<const uint8_t*>(x + (size_t)row * H) + h * 128 + chunk * 16;
          dst[i] = (ib * 2 + h) * RT2_REG + rg * 1024;
        } else {
          const int jb = (job - 32) >> 3;
          const int e = nt * RT2_BN + jb * 32 + rg * 8 + ld_row;
          src[i] = reinterpret_cast<const uint8_t*>(g + (size_t)e * H) + h * 128 + chunk * 16;
          dst[i] = RT2_A_BYTES + (jb * 2 + h) * RT2_REG + rg * 1024;
        }
      }
      kb = 0;
    };
    auto issue = [&]() {
      if (kb == NB_H) next_item();
      uint8_t* st = rt_lds + slot * RT2_STAGE;
#pragma unroll
      for (int i = 0; i < RT2_JOBS; ++i) lds_direct16(src[i] + kb * 2 * BLK, st + dst[i]);  // 256 B per K block
      slot = slot == RT2_NSTAGE - 1 ? 0 : slot + 1;
      ++kb;
    };
    if (G > 0) issue();
    if (G > 1) issue();
#pragma unroll 1
    for (int gi = 0; gi < G; ++gi) {
      if (gi + 1 < G) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");  // 12 loads per block
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (gi + 2 < G) issue();
    }
    return;
  }

  // compute wave: tokens 32 wm .. of the item, experts 32 wn ..; MFMA step t of a
  // block reads, from line t / 4 of the row, 16 B chunk 4 ((t / 2) % 2) + 2 lg + t % 2
  // (the same for both operands, so the K pairing holds)
  const int wm = wave & 3, wn = wave >> 2;
  const int lr = lane & 31, lg = lane >> 5;
  int off[2][2];
#pragma unroll
  for (int ph = 0; ph < 2; ++ph)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) off[ph][tt] = sw32(lr, 4 * ph + 2 * lg + tt);
  int slot = 0;
  for (int item = first; item < total; item += gridDim.x) {
    const int mt = item / RT2_NT, nt = item % RT2_NT;
    v16f acc = v16f{};
#pragma unroll 1
    for (int kb = 0; kb < NB_H; ++kb) {
      __builtin_amdgcn_s_barrier();  // block kb is in its slot; the slot before it is free
      asm volatile("" ::: "memory");
      const uint8_t* st = rt_lds + slot * RT2_STAGE;
      slot = slot == RT2_NSTAGE - 1 ? 0 : slot + 1;
      const uint8_t* sa = st + (wm * 2) * RT2_REG;
      const uint8_t* sb = st + RT2_A_BYTES + (wn * 2) * RT2_REG;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int line = t >> 2, ph = (t >> 1) & 1, tt = t & 1;
        const v8bf a = *reinterpret_cast<const v8bf*>(sa + line * RT2_REG + off[ph][tt]);
        const v8bf b = *reinterpret_cast<const v8bf*>(sb + line * RT2_REG + off[ph][tt]);
        acc = mfma_bf16_32x32x16(a, b, acc);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this block's LDS reads are done
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = mt * RT2_BM + wm * 32 + 8 * (i >> 2) + 4 * lg + (i & 3);
      if (t < T) logits[(size_t)t * E_GLOBAL + nt * RT2_BN + wn * 32 + lr] = acc[i];
    }
  }
}

// Middle T (from RT2_MIN_T tokens while its items fit on the CUs: 2,048 tokens on
// 256 CUs): the tiled kernel has fewer items than CUs there, and each item's 56 K
// blocks pass a 3-slot ring one memory latency per two blocks (33-36 us whatever
// T; 19-21 us here). Here an item is 32 tokens x 64 experts,
// so four times as many workgroups take part, and its stage (24 KB: one 32-row
// block of hidden rows, two of gate rows) fits a 5-slot ring, four blocks ahead.
// The 8 compute waves split each K block: wave (wn, kq) takes MFMA steps 2 kq and
// 2 kq + 1 of expert half wn, so every wave keeps one 32 x 32 accumulator; after
// the last block the four K quarters are added through LDS in kq order (a fixed
// order; no atomics).
constexpr int RT3_BM = 32;
constexpr int RT3_A_BYTES = RT3_BM * BLK * 2;                // 8 KB: 2 lines
constexpr int RT3_STAGE = RT3_A_BYTES + RT2_BN * BLK * 2;    // + 16 KB: 2 row blocks x 2 lines
constexpr int RT3_NSTAGE = 5;
constexpr int RT3_JOBS = RT3_STAGE / 1024 / RT2_PWAVES;      // 6 load instructions per loader wave per block
constexpr int RT3_RED = 8 * 16 * 64 * 4;                     // 8 waves x 16 values x 64 lanes
constexpr int RT3_LDS = RT3_NSTAGE * RT3_STAGE + RT3_RED;
static_assert(RT3_JOBS * RT2_PWAVES * 1024 == RT3_STAGE && RT3_LDS <= 160 * 1024, "stage");

// s_waitcnt vmcnt for n of the loader's blocks still in flight (n <= 3)
__device__ __forceinline__ void rt3_wait_blocks(int n) {
  switch (n) {
    case 3: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
  }
}

__global__ __launch_bounds__(64 * (RT2_CWAVES + RT2_PWAVES), 1) void router_ksplit_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ g, int T, float* __restrict__ logits) {
  extern __shared__ __attribute__((aligned(16))) uint8_t rt_lds[];
  float* red = reinterpret_cast<float*>(rt_lds + RT3_NSTAGE * RT3_STAGE);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int total = (T + RT3_BM - 1) / RT3_BM * RT2_NT;
  const int first = xcd_remap(blockIdx.x, gridDim.x);
  int n_items = 0;
  for (int item = first; item < total; item += gridDim.x) ++n_items;
  const int G = n_items * NB_H;

  if (wave >= RT2_CWAVES) {
    // loader wave p: jobs 6 p .. 6 p + 5 of the 24 per block (0-7 hidden rows,
    // 8-23 gate rows); a job moves 8 rows x 128 B (one line of a K block)
    const int p = wave - RT2_CWAVES, ld_row = lane >> 3;
    const uint8_t* src[RT3_JOBS];
    int dst[RT3_JOBS];
    int item = first - (int)gridDim.x, kb = NB_H, slot = 0;
    auto next_item = [&]() {
      item += gridDim.x;
      const int mt = item / RT2_NT, nt = item % RT2_NT;
#pragma unroll
      for (int i = 0; i < RT3_JOBS; ++i) {
        const int job = p * RT3_JOBS + i;
        const int chunk_row = ld_row;
        if (job < 8) {
          const int rg = job & 3, h = job >> 2;
          const int row = min(mt * RT3_BM + rg * 8 + ld_row, T - 1);
          src[i] = reinterpret_cast<const uint8_t*>(x + (size_t)row * H) + h * 128 +
                   ((lane & 7) ^ chunk_row ^ (rg & 1)) * 16;
          dst[i] = h * RT2_REG + rg * 1024;
        } else {
          const int jj = job - 8, rg = jj & 3, h = (jj >> 2) & 1, jb = jj >> 3;
          const int e = nt * RT2_BN + jb * 32 + rg * 8 + ld_row;
          src[i] = reinterpret_cast<const uint8_t*>(g + (size_t)e * H) + h * 128 +
                   ((lane & 7) ^ chunk_row ^ (rg & 1)) * 16;
          dst[i] = RT3_A_BYTES + (jb * 2 + h) * RT2_REG + rg * 1024;
        }
      }
      kb = 0;
    };
    auto issue = [&]() {
      if (kb == NB_H) next_item();
      uint8_t* st = rt_lds + slot * RT3_STAGE;
#pragma unroll
      for (int i = 0; i < RT3_JOBS; ++i) lds_direct16(src[i] + kb * 2 * BLK, st + dst[i]);  // 256 B per K block
      slot = slot == RT3_NSTAGE - 1 ? 0 : slot + 1;
      ++kb;
    };
    for (int b = 0; b < RT3_NSTAGE - 1 && b < G; ++b) issue();
#pragma unroll 1
    for (int gi = 0; gi < G; ++gi) {
      rt3_wait_blocks(min(RT3_NSTAGE - 2, G - 1 - gi));  // block gi is in
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (gi + RT3_NSTAGE - 1 < G) issue();
      if (gi % NB_H == NB_H - 1) __builtin_amdgcn_s_barrier();  // the compute waves' K-quarter sum
    }
    return;
  }

  // compute wave (wn, kq): experts 32 wn .. of the item, MFMA steps 2 kq, 2 kq + 1
  // of every K block; step t reads, from line t / 4 of the row, 16 B chunk
  // 4 ((t / 2) % 2) + 2 lg + t % 2 (the same for both operands)
  const int wn = wave & 1, kq = wave >> 1;
  const int lr = lane & 31, lg = lane >> 5;
  int off[2];
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) off[tt] = sw32(lr, 4 * (kq & 1) + 2 * lg + tt);
  const int line = kq >> 1;
  int slot = 0;
  for (int item = first; item < total; item += gridDim.x) {
    const int mt = item / RT2_NT, nt = item % RT2_NT;
    v16f acc = v16f{};
#pragma unroll 1
    for (int kb = 0; kb < NB_H; ++kb) {
      __builtin_amdgcn_s_barrier();  // block kb is in its slot; the slot before it is free
      asm volatile("" ::: "memory");
      const uint8_t* st = rt_lds + slot * RT3_STAGE;
      slot = slot == RT3_NSTAGE - 1 ? 0 : slot + 1;
      const uint8_t* sa = st + line * RT2_REG;
      const uint8_t* sb = st + RT3_A_BYTES + (wn * 2 + line) * RT2_REG;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const v8bf a = *reinterpret_cast<const v8bf*>(sa + off[tt]);
        const v8bf b = *reinterpret_cast<const v8bf*>(sb + off[tt]);
        acc = mfma_bf16_32x32x16(a, b, acc);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this block's LDS reads are done
    }
    // the K quarters: wave w's 16 values per lane to LDS, then wave w takes expert
    // half w % 2, values 4 (w / 2) .. + 3, and adds the quarters in kq order
#pragma unroll
    for (int i = 0; i < 16; ++i) red[(wave * 16 + i) * 64 + lane] = acc[i];
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int i = 4 * kq + ii;  // this wave's value index (kq doubles as the value group)
      float v = red[((0 * 2 + wn) * 16 + i) * 64 + lane];
#pragma unroll
      for (int q = 1; q < 4; ++q) v += red[((q * 2 + wn) * 16 + i) * 64 + lane];
      const int t = mt * RT3_BM + 8 * (i >> 2) + 4 * lg + (i & 3);
      if (t < T) logits[(size_t)t * E_GLOBAL + nt * RT2_BN + wn * 32 + lr] = v;
    }
  }
}

hipError_t launch_quantize_1x128(const uint16_t* x, int T, uint8_t* q, float* scale, hipStream_t stream);

static hipError_t launch_router_tiled(const uint16_t* x, const uint16_t* g, int T, float* logits, int cu,
                                      hipStream_t stream) {
  static PerDeviceOnce<hipError_t> once;
  hipError_t e = hipErrorInvalidDevice;
  once.get([] { return hipFuncSetAttribute(reinterpret_cast<const void*>(router_tiled_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, RT2_NSTAGE * RT2_STAGE); },
           e);
  if (e != hipSuccess) return e;
  const int items = (T + RT2_BM - 1) / RT2_BM * RT2_NT;
  const int grid = min((items + 7) / 8 * 8, (cu + 7) / 8 * 8);
  hipLaunchKernelGGL(router_tiled_kernel, dim3(grid), dim3(64 * (RT2_CWAVES + RT2_PWAVES)), RT2_NSTAGE * RT2_STAGE,
                     stream, x, g, T, logits);
  return hipGetLastError();
}

static hipError_t launch_router_ksplit(const uint16_t* x, const uint16_t* g, int T, float* logits, int cu,
                                       hipStream_t stream) {
  static PerDeviceOnce<hipError_t> once;
  hipError_t e = hipErrorInvalidDevice;
  once.get([] { return hipFuncSetAttribute(reinterpret_cast<const void*>(router_ksplit_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, RT3_LDS); },
           e);
  if (e != hipSuccess) return e;
  const int items = (T + RT3_BM - 1) / RT3_BM * RT2_NT;
  const int grid = min((items + 7) / 8 * 8, (cu + 7) / 8 * 8);
  hipLaunchKernelGGL(router_ksplit_kernel, dim3(grid), dim3(64 * (RT2_CWAVES + RT2_PWAVES)), RT3_LDS, stream, x, g,
                     T, logits);
  return hipGetLastError();
}

// the tiled GEMM by token count: 32-token items with the K steps split over the
// waves while they fit on the CUs in one round, 128-token items beyond
static hipError_t launch_router_gemm(const uint16_t* x, const uint16_t* g, int T, float* logits, int cu,
                                     hipStream_t stream) {
  return (T + RT3_BM - 1) / RT3_BM * RT2_NT <= cu ? launch_router_ksplit(x, g, T, logits, cu, stream)
                                                  : launch_router_tiled(x, g, T, logits, cu, stream);
}

hipError_t launch_router_logits(const uint16_t* x, const uint16_t* g, int T, float* logits, int cu,
                                hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  if (T >= RT2_MIN_T) return launch_router_gemm(x, g, T, logits, cu, stream);
  hipLaunchKernelGGL(router_small_kernel<false>, dim3((T + RT_M - 1) / RT_M, E_GLOBAL / 16), dim3(64 * RS_WAVES), 0,
                     stream, x, g, T, logits, nullptr, nullptr);
  return hipGetLastError();
}

hipError_t launch_router_quantize(const uint16_t* x, const uint16_t* g, int T, float* logits, uint8_t* q, float* qs,
                                  int cu, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  if (T >= RT2_MIN_T) {
    const hipError_t e = launch_router_gemm(x, g, T, logits, cu, stream);
    return e != hipSuccess ? e : launch_quantize_1x128(x, T, q, qs, stream);
  }
  hipLaunchKernelGGL(router_small_kernel<true>, dim3((T + RT_M - 1) / RT_M, E_GLOBAL / 16), dim3(64 * RS_WAVES), 0,
                     stream, x, g, T, logits, q, qs);
  return hipGetLastError();
}

}  // namespace moe

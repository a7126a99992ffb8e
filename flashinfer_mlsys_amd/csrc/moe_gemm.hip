// Grouped expert GEMMs and the ordered combine for the FP8 DeepSeek-V3 MoE.
//
// Per local expert e with token segment rows [seg, seg + cnt) (ascending tokens):
//   GEMM1  G1 = A_e . W13_e^T        [cnt, 7168] x [7168, 4096]  (ref_moe.py:147-153)
//   SwiGLU C  = X1 * silu(X2)        X1 = G1[:, :2048], X2 = G1[:, 2048:] (ref_moe.py:155-159)
//   GEMM2  O  = C . W2_e^T           [cnt, 2048] x [2048, 7168]  (ref_moe.py:161-162)
//   weight O * w[token, e]; out[t] = sum over t's local experts in ascending id,
//   then bf16 (ref_moe.py:164-168): in the decode shape inside GEMM2, in the
//   prefill shape through one row per (token, expert) pair and the combine
//
// GEMM1 runs on the e4m3 MFMA (v_mfma_scale_f32_16x16x128_f8f6f4 with unit E8M0
// scales). One MFMA covers exactly one 128-wide K block, so the fp32 block
// scales are applied once per block: acc += P * (s_act[row, kb] * s_w[nb, kb]).
// GEMM2 runs on the fp16 MFMA: e4m3 weights widen to fp16 exactly, and C is
// stored as fp16 of C * 2^-8 (c_encode: 11 significant bits), the 2^8 going back
// in with the weight block scale.
//
// Two shapes of each GEMM:
//   *_decode  -- T <= 96, few rows per expert, weight-streaming bound. The
//                waves split K, so each weight byte is read once, and the next
//                items' weights are in flight while the current one computes;
//                partial sums meet in LDS. GEMM1: persistent workgroups walk
//                (active expert, 8-column) items. GEMM2: workgroup c owns 28
//                output columns of every active expert and sums each token's
//                pairs itself, writing bf16 rows (no combine kernel).
//   prefill   -- many rows per expert. Persistent workgroups walk a device-built
//                list of (expert, row tile, column tile) items, moving operands
//                global -> LDS with direct loads into a ring of stages, in the
//                exact order the MFMA reads them. GEMM1 (gemm1_prefill_kernel):
//                every wave computes and issues direct loads from inline asm.
//                GEMM2 (gemm2_loader_kernel): loader waves issue the direct loads
//                while compute waves run the MFMAs. The workgroups of one XCD take
//                consecutive items, which share operand tiles, so that XCD's L2
//                serves the repeats.
#include "moe_common.h"
#include <type_traits>
#include "moe_host.h"
#include "moe_route_token.h"
#include "moe_small_dispatch.h"
#include "moe_tile.h"
#include "../../include/moe_fp8.h"

namespace moe {

__device__ __forceinline__ v8i load_v8i(const uint8_t* p) {
  const v4i lo = *reinterpret_cast<const v4i*>(p);
  const v4i hi = *reinterpret_cast<const v4i*>(p + 16);
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

__device__ __forceinline__ float silu_mul(float x1, float x2) {
  return (x2 / (1.0f + expf(-x2))) * x1;
}

// Swizzled 16 x 128 B e4m3 fragment (2 KB), written by two direct loads of 8
// whole row lines each: load j, lane l holds row 8 j + l / 8, 16 B chunk
// (l % 8) ^ (l / 8) ^ j, at 1024 j + 16 l. An MFMA lane m (row m % 16, K bytes
// 32 (m / 16) .. +32 = chunks 2 (m / 16) and 2 (m / 16) + 1) reads its two
// chunks at the offsets below; every 16-lane group of either read hits 16
// distinct 16 B bank slots, so the reads are conflict-free, and each load
// instruction fetches 8 complete 128 B lines (half-line loads reach about a
// third of the per-CU load bandwidth).
__device__ __forceinline__ int frag_sw_offset(int r, int c) {
  const int j = r >> 3, rr = r & 7;
  return j * 1024 + 16 * (8 * rr + (c ^ rr ^ j));
}
__device__ __forceinline__ void frag_sw_offsets(int lane, int& lo, int& hi) {
  const int r = lane & 15, q = lane >> 4;
  lo = frag_sw_offset(r, 2 * q);
  hi = frag_sw_offset(r, 2 * q + 1);
}
__device__ __forceinline__ v8i lds_frag_sw(const uint8_t* f, int lo, int hi) {
  const v4i a = *reinterpret_cast<const v4i*>(f + lo);
  const v4i b = *reinterpret_cast<const v4i*>(f + hi);
  v8i r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

__device__ __forceinline__ v8i lds_frag(const uint8_t* f) {
  const int lane = threadIdx.x & 63;
  const v4i lo = *reinterpret_cast<const v4i*>(f + lane * 16);
  const v4i hi = *reinterpret_cast<const v4i*>(f + 1024 + lane * 16);
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

// ---------------------------------------------------------------------------
// GEMM1 + SwiGLU, decode shape (T <= 96; built for up to 128).
//
// Every workgroup derives the dispatch from the routing output in its own LDS
// (dispatch_small_*): the per-expert counts first, then the first two items'
// weights are requested, then the token lists, so the weight stream starts
// before the lists exist and without reading a header back from memory.
// Workgroup 0 also stores the dispatch for GEMM2.
//
// Items are (active expert, 8-column tile): the MFMA's 16 B columns are W13
// rows n..n+7 (X1) in lanes 0-7 and 2048+n..2048+n+7 (X2) in lanes 8-15, so
// one expert spreads over 256 items and column c's X1 and X2 meet in the LDS
// reduction. Each of the 8 waves owns 7 of the 56 K blocks. A workgroup (one
// per CU) takes a contiguous run of items, so consecutive items mostly share
// the expert. Weights stream through a 3-deep register ring: items i+1 and i+2
// are in flight while item i computes. The activation rows of the current
// expert (16 per pass) sit in LDS in MFMA fragment order, each wave holding
// only its own K slice (direct global -> LDS loads), so no barrier guards
// them; the one barrier per pass is the cross-wave reduction, whose buffer
// alternates between passes.
// ---------------------------------------------------------------------------
constexpr int D1_WAVES = 8;
constexpr int D1_KPW = NB_H / D1_WAVES;  // 7 K blocks per wave
constexpr int D1_NT = I / 8;             // items per expert
constexpr int D1_LOADS = 2 * D1_KPW;     // 16 B loads per lane for one item's weights
static_assert(NB_H % D1_WAVES == 0, "K slices");
static_assert(64 * D1_WAVES >= SMALL_T, "dispatch_small: a thread per token mask");
static_assert(D1_LOADS == 14, "the vmcnt immediates below count 14 loads per item");

template <int TM>
struct G1Shared {
  SmallDispatch<TM> d;
  float red[2][D1_WAVES][4][64];
  __attribute__((aligned(16))) uint8_t a[D1_WAVES][D1_KPW][2][1024];  // wave's K slice, 16 rows, fragment halves
  __attribute__((aligned(16))) float sa[D1_WAVES][D1_KPW + 1][16];    // their activation scales (+16 padding)
  int tok0[D1_WAVES][16];  // per wave: the first expert's first 16 tokens (prologue)
};

struct G1State {
  int cur_le = -1;  // sh.a holds rows a_m0 .. a_m0 + 15 of expert cur_le
  int a_m0 = 0;
  int phase = 0;    // reductions done (selects the red buffer)
};

__device__ __forceinline__ void g1_load_w(v8i (&b)[D1_KPW], const uint8_t* __restrict__ w13, int le, int nt, int kb0) {
  const int lane = threadIdx.x & 63, fr = lane & 15, kg = lane >> 4;
  const int wrow = fr < 8 ? nt * 8 + fr : I + nt * 8 + (fr - 8);
  const uint8_t* wp = w13 + ((size_t)le * N1 + wrow) * H + kb0 * BLK + kg * 32;
#pragma unroll
  for (int kk = 0; kk < D1_KPW; ++kk) b[kk] = load_v8i(wp + kk * BLK);
}

// The first expert's activation rows for the prologue: this wave's K slice (7
// K blocks = 896 B per row) of its first min(cnt, 16) rows and their scales,
// staged into LDS (only this wave reads them) in two steps so that the weight
// requests go out in between: the loads into registers, then the LDS writes,
// which wait only for these loads. The rows travel compactly: load i, lane l
// takes bytes 16 (64 i + l) of the rows' slices laid end to end (row r = byte /
// 896, offset o = byte % 896 = 128 kk + 32 kg + 16 h), so NA loads cover
// floor(1024 NA / 896) rows: 1 load for one row, 4 for four, 14 for sixteen,
// instead of 14 loads of 16 rows that repeat the last one (the load path's time
// per instruction is what these loads cost before the first weight request).
// In LDS, lane (fr, kg)'s fragment bytes are row fr, K 32 kg + [0, 32): half h
// holds bytes [16 h, 16 h + 16). Rows at or past cnt hold zeros or whatever the
// LDS held; they reach only their own MFMA output rows, which are never stored.
// Plain loads and ds_writes, no direct-to-LDS loads: the compiler cannot tell
// which LDS bytes a direct load writes, so every later LDS read would wait for
// all loads in flight, the weight prefetches included.
constexpr int D1_ROW = D1_KPW * BLK;  // 896 B: a row's K slice for one wave
template <int NA>
struct G1AStage {
  v4i rows[NA];
  float sc[2];
};

// Buffer loads for the prologue: a wave-uniform resource (base, byte range) in
// SGPRs, a 32-bit offset per lane. With a range of 0 the loads return zeros
// without a memory access, so the prologue's requests are unconditional: with a
// branch around them the compiler could not count the requests in flight past
// the branch and would wait for all of them before the first LDS work after it.
// Word 3 is the gfx9 raw-buffer format (32-bit data format).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ v4i buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// g1_load_w and g1_stage_a_load for the prologue (zeros, no traffic, when !valid).
__device__ __forceinline__ void g1_load_w_pro(v8i (&b)[D1_KPW], const uint8_t* __restrict__ w13, int le, int nt,
                                              int kb0, bool valid) {
  const int lane = threadIdx.x & 63, fr = lane & 15, kg = lane >> 4;
  const int wrow = fr < 8 ? nt * 8 + fr : I + nt * 8 + (fr - 8);
  const __amdgpu_buffer_rsrc_t r = buf_rsrc(w13 + (size_t)le * N1 * H + kb0 * BLK, valid ? (uint32_t)N1 * H : 0u);
  const uint32_t off = (uint32_t)(wrow * H + kg * 32);
#pragma unroll
  for (int kk = 0; kk < D1_KPW; ++kk) {
    const v4i lo = buf_load16(r, off + kk * BLK), hi = buf_load16(r, off + kk * BLK + 16);
    b[kk] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
}
template <int NA>
__device__ __forceinline__ void g1_stage_a_load_pro(G1AStage<NA>& a, const int* tok, int cnt,
                                                    const uint8_t* __restrict__ hidden,
                                                    const float* __restrict__ hscale, int T, int wave, bool valid) {
  const int lane = threadIdx.x & 63;
  const int kb0 = wave * D1_KPW;
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(hscale, valid ? (uint32_t)(NB_H * T * 4) : 0u);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = lane + 64 * j, kk = (i >> 4) % D1_KPW, r = i & 15;
    const uint32_t off = (uint32_t)(((kb0 + kk) * T + tok[max(min(r, cnt - 1), 0)]) * 4);
    a.sc[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
  }
  const __amdgpu_buffer_rsrc_t rr = buf_rsrc(hidden + kb0 * BLK, valid ? (uint32_t)(T * H) : 0u);
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int byte = 1024 * i + 16 * lane, r = byte / D1_ROW, o = byte % D1_ROW;
    // rows at or past the count read past the range: zeros, no memory access
    const uint32_t off = r < cnt ? (uint32_t)(tok[min(r, 15)] * H + o) : 0xFFFFFFF0u;
    a.rows[i] = buf_load16(rr, off);
  }
}

template <int NA, class SH>
__device__ __forceinline__ void g1_stage_a_store(const G1AStage<NA>& a, SH& sh, int wave) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < 2; ++j) (&sh.sa[wave][0][0])[lane + 64 * j] = a.sc[j];  // lanes past 112: padding
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int byte = 1024 * i + 16 * lane, r = byte / D1_ROW, o = byte % D1_ROW;
    const int kk = o >> 7, kg = (o >> 5) & 3, h = (o >> 4) & 1;  // r < 16: byte < 14 * 1024
    *reinterpret_cast<v4i*>(&sh.a[wave][kk][h][(r + 16 * kg) * 16]) = a.rows[i];
  }
}

// The same in one step, for a change of expert or a later 16-row pass inside the
// run: the scales by 4 B direct loads (no registers held while the weight ring is
// full), the rows through registers; the caller waits for the direct loads.
template <class SH>
__device__ __forceinline__ void g1_stage_a(SH& sh, const uint8_t* __restrict__ hidden,
                                           const float* __restrict__ hscale, int T, int le, int m0, int wave) {
  const auto& d = sh.d;
  const int lane = threadIdx.x & 63, fr = lane & 15, kg = lane >> 4;
  const int cnt = d.cnt[le], seg = d.seg[le], kb0 = wave * D1_KPW;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int i = lane + 64 * j;
    if (i < D1_KPW * 16) {
      const int kk = i >> 4, r = i & 15;
      lds_direct4(hscale + (size_t)(kb0 + kk) * T + d.tok[seg + min(m0 + r, cnt - 1)],
                  reinterpret_cast<uint8_t*>(&sh.sa[wave][0][0] + 64 * j));
    }
  }
  const uint8_t* ap = hidden + (size_t)d.tok[seg + min(m0 + fr, cnt - 1)] * H + kb0 * BLK + kg * 32;
#pragma unroll
  for (int kk = 0; kk < D1_KPW; ++kk)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      *reinterpret_cast<v4i*>(&sh.a[wave][kk][h][lane * 16]) = *reinterpret_cast<const v4i*>(ap + kk * BLK + 16 * h);
}

// One 16-row pass of item (le, nt): rows m0 .. m0 + 15 (staged in sh.a) against
// the item's weights b, the cross-wave reduction, SwiGLU and the C rows.
template <class SH>
__device__ __forceinline__ void g1_pass(int m0, int cnt, int seg, int nt, const v8i (&b)[D1_KPW],
                                        const float (&swu)[D1_KPW], const float (&swg)[D1_KPW], G1State& st,
                                        SH& sh, uint16_t* __restrict__ c_act) {
  const int tid = threadIdx.x, lane = tid & 63, fr = lane & 15, kg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < D1_KPW; ++kk) {
    const v8i a = lds_frag(&sh.a[wave][kk][0][0]);
    const v4f p = mfma_fp8_k128(a, b[kk]);
    const float sw = fr < 8 ? swu[kk] : swg[kk];
    const v4f sa = *reinterpret_cast<const v4f*>(&sh.sa[wave][kk][4 * kg]);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] += p[r] * (sa[r] * sw);
  }
  float(&red)[D1_WAVES][4][64] = sh.red[st.phase & 1];
#pragma unroll
  for (int r = 0; r < 4; ++r) red[wave][r][lane] = acc[r];
  lds_barrier();
  if (tid < 256) {
    const int r = tid >> 6, ln = tid & 63;
    if ((ln & 15) < 8) {
      float x1 = 0.f, x2 = 0.f;
#pragma unroll
      for (int w = 0; w < D1_WAVES; ++w) {
        x1 += red[w][r][ln];
        x2 += red[w][r][ln + 8];
      }
      const int row = m0 + 4 * (ln >> 4) + r;
      if (row < cnt) c_act[(size_t)(seg + row) * I + nt * 8 + (ln & 15)] = c_encode(silu_mul(x1, x2));
    }
  }
  ++st.phase;
}

// Item (le, nt) with the weights in b; requests item + 2's weights into b2. One
// pass per 16 rows of the expert. Loads complete in order, so a wait for rows
// requested after item + 2's weights would wait for those weights as well: the
// rows of every pass are staged before that request goes out, which comes just
// before the last pass (for an expert of at most 16 rows, its only pass: after
// the rows on a change of expert), and the waits of the earlier passes cover
// only their rows and item + 1's weights, requested an item ago. The passes run
// forwards and backwards on alternate items of an expert, so each item starts
// with the rows the previous one left in LDS.
template <bool PF, class SH>
__device__ __forceinline__ void g1_item(int item, int end, v8i (&b)[D1_KPW], v8i (&b2)[D1_KPW], G1State& st,
                                        SH& sh, const uint8_t* __restrict__ hidden,
                                        const float* __restrict__ hscale, int T, const uint8_t* __restrict__ w13,
                                        const float* __restrict__ s13, uint16_t* __restrict__ c_act) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kb0 = wave * D1_KPW;
  const auto& d = sh.d;
  const int le = __builtin_amdgcn_readfirstlane(d.active[item / D1_NT]), nt = item % D1_NT;
  const int cnt = __builtin_amdgcn_readfirstlane(d.cnt[le]), seg = __builtin_amdgcn_readfirstlane(d.seg[le]);
  // weight scales: the X1 block row (lanes 0-7) or the X2 block row (lanes 8-15).
  // Both are read at wave-uniform addresses (scalar loads, counted by lgkmcnt):
  // a per-lane vector load would make the MFMAs wait for vmcnt(0), i.e. for the
  // prefetched weights of the next two items as well. Read before the first
  // pass: for a one-pass item after item + 2's request.
  const float* su = s13 + ((size_t)le * NB_N1 + (nt * 8) / BLK) * NB_H + kb0;
  const float* sg = su + (size_t)NB_I * NB_H;
  float swu[D1_KPW], swg[D1_KPW];
  auto load_scales = [&] {
#pragma unroll
    for (int kk = 0; kk < D1_KPW; ++kk) {
      swu[kk] = su[kk];
      swg[kk] = sg[kk];
    }
  };
  const int last = (cnt - 1) & ~15;                              // the last pass's first row
  const bool back = last > 0 && st.cur_le == le && st.a_m0 == last;  // LDS holds the last pass
  int held = st.cur_le == le ? st.a_m0 : -1;                     // rows in LDS (uniform)
  if (__builtin_expect(last > 0, 0)) {  // more than 16 rows: every pass but the final one
    load_scales();
    for (int q = 0; q < last; q += 16) {
      const int m0 = back ? last - q : q;
      if (held != m0) {
        g1_stage_a(sh, hidden, hscale, T, le, m0, wave);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      g1_pass(m0, cnt, seg, nt, b, swu, swg, st, sh, c_act);
      held = m0;
    }
  }
  const int mf = back ? 0 : last;
  const bool stage = held != mf;
  // (the first item's rows are staged before the weight stream starts; a change
  // of expert later in the run waits here for the weights already in flight)
  if (stage) g1_stage_a(sh, hidden, hscale, T, le, mf, wave);
  const int n2 = item + 2;
  const bool pf = PF || n2 < end;
  if (pf) g1_load_w(b2, w13, __builtin_amdgcn_readfirstlane(d.active[n2 / D1_NT]), n2 % D1_NT, kb0);
  if (stage) {  // the scales' direct loads (and everything before them) have landed; b2 may fly
    if (pf) asm volatile("s_waitcnt vmcnt(14)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  if (last == 0) load_scales();
  g1_pass(mf, cnt, seg, nt, b, swu, swg, st, sh, c_act);
  st.cur_le = le;
  st.a_m0 = mf;
}

// With route_here (T <= D1_WAVES) the workgroup first routes the T tokens
// itself, wave t token t, into its LDS (workgroup 0 also stores the ids and
// weights), instead of reading the routing kernel's output: a small decode
// call is then two launches, not three.
template <int TM>
__global__ __launch_bounds__(64 * D1_WAVES, 2) void gemm1_decode_kernel(
    const float* __restrict__ logits, const uint16_t* __restrict__ bias, float rsf, int route_here,
    const uint8_t* __restrict__ hidden, const float* __restrict__ hscale, int T, int offset,
    const uint8_t* __restrict__ w13, const float* __restrict__ s13, int32_t* __restrict__ topk_ids,
    float* __restrict__ topk_w, DispatchHeader* __restrict__ hdr, int32_t* __restrict__ perm_tok,
    float* __restrict__ perm_w, int32_t* __restrict__ tok_pair, uint16_t* __restrict__ c_act) {
  extern __shared__ __attribute__((aligned(16))) uint8_t g1d_lds[];
  G1Shared<TM>& sh = *reinterpret_cast<G1Shared<TM>*>(g1d_lds);
  const int lane = threadIdx.x & 63;
  if (route_here) {
    const int w = threadIdx.x >> 6;
    // tie scratch: the wave's activation stage, first written after the barrier below
    if (w < T)
      route_token<false>(logits, bias, w, rsf, sh.d.ids, sh.d.wts, nullptr,
                         reinterpret_cast<TieScratch*>(&sh.a[w][0][0][0]));
    lds_barrier();
    if (blockIdx.x == 0 && (int)threadIdx.x < T * TOP_K) {
      topk_ids[threadIdx.x] = sh.d.ids[threadIdx.x];
      topk_w[threadIdx.x] = sh.d.wts[threadIdx.x];
    }
  } else {
    dispatch_small_ids(topk_ids, topk_w, T, sh.d);
  }
  dispatch_small_masks(T, offset, sh.d);
  // The workgroup's items follow from the active set alone, and the first item's
  // activation rows from the token masks: the first expert's rows, then item 0's
  // and item 1's weights are requested before the rest of the dispatch (counts,
  // segments, lists, pair indices) is built in LDS, while they fly. The rows are
  // written to LDS once item 0's weight requests are out (the writes wait only for
  // the rows), so the weight stream never drains before item 0.
  const uint32_t act = small_active_set(T, sh.d);
  const int total = __popc(act) * D1_NT;
  const int per = (total + gridDim.x - 1) / gridDim.x;
  // workgroup b runs on XCD b % 8; xcd_remap gives the 32 workgroups of one XCD
  // consecutive runs of items (neighbouring weight rows): sweep 436.4 -> 434.4 us
  // together with the same mapping in the decode GEMM2
  const int wgi = (gridDim.x & 7) == 0 ? xcd_remap(blockIdx.x, gridDim.x) : (int)blockIdx.x;
  const int begin = wgi * per, end = min(total, begin + per);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), kb0 = wave * D1_KPW;
  G1State st;
  const bool has0 = begin < end, ring = end - begin >= 5, has1 = ring || begin + 1 < end;  // uniform
  const int le0 = has0 ? nth_set_bit(act, begin / D1_NT) : 0;
  const int le1 = has1 ? nth_set_bit(act, (begin + 1) / D1_NT) : 0;
  // le0's first 16 tokens, from the two token halves (token lane + 64 h routes to le0)
  int cnt0 = 0;
#pragma unroll
  for (int h = 0; h < SmallDispatch<TM>::HALVES; ++h) {
    const int t = lane + 64 * h;
    const bool in0 = t < T && ((sh.d.mask[t] >> le0) & 1u);
    const unsigned long long m0 = __ballot(in0);
    const int rank = cnt0 + __popcll(m0 & ((1ull << lane) - 1ull));
    if (in0 && rank < 16) sh.tok0[wave][rank] = t;  // this wave's copy, read only by this wave
    cnt0 += __popcll(m0);
  }
  if (lane == 0 && cnt0 == 0) sh.tok0[wave][0] = 0;  // (no item: any valid index)
  v8i b0[D1_KPW], b1[D1_KPW], b2[D1_KPW];
  // the rows, then item 0's weights, the rows to LDS (a wait for the rows only),
  // item 1's weights: one straight-line copy per compact load count, so that the
  // compiler counts the requests in flight exactly on every path (the paths end
  // alike: item 0's weights, then item 1's)
  auto prologue = [&](auto na) {
    G1AStage<decltype(na)::value> a0;
    g1_stage_a_load_pro(a0, &sh.tok0[wave][0], cnt0, hidden, hscale, T, wave, has0);
    __builtin_amdgcn_sched_barrier(0);  // the rows are requested ahead of the weights
    g1_load_w_pro(b0, w13, le0, begin % D1_NT, kb0, has0);
    g1_stage_a_store(a0, sh, wave);  // waits for the rows only (requested before item 0's weights)
    g1_load_w_pro(b1, w13, le1, (begin + 1) % D1_NT, kb0, has1);
    __builtin_amdgcn_sched_barrier(0);
  };
  if (cnt0 <= 1) prologue(std::integral_constant<int, 1>{});  // uniform
  else if (cnt0 <= 4) prologue(std::integral_constant<int, 4>{});
  else prologue(std::integral_constant<int, 14>{});
  st.cur_le = le0;  // rows 0..15 of le0 are in LDS
  st.a_m0 = 0;
  dispatch_small_counts_from_masks(T, sh.d);
  dispatch_small_lists(T, offset, sh.d);
  if (blockIdx.x == 0) store_small_dispatch(sh.d, T, hdr, perm_tok, perm_w, tok_pair);
  int item = begin;
  if (ring) {
    for (; item + 4 < end; item += 3) {  // items item+2..item+4 exist: unconditional requests
      g1_item<true>(item, end, b0, b2, st, sh, hidden, hscale, T, w13, s13, c_act);
      g1_item<true>(item + 1, end, b1, b0, st, sh, hidden, hscale, T, w13, s13, c_act);
      g1_item<true>(item + 2, end, b2, b1, st, sh, hidden, hscale, T, w13, s13, c_act);
    }
  }
  // the last (at most four) items; b0 holds item, b1 item + 1
  if (item < end) g1_item<false>(item, end, b0, b2, st, sh, hidden, hscale, T, w13, s13, c_act);
  if (item + 1 < end) g1_item<false>(item + 1, end, b1, b0, st, sh, hidden, hscale, T, w13, s13, c_act);
  if (item + 2 < end) g1_item<false>(item + 2, end, b2, b1, st, sh, hidden, hscale, T, w13, s13, c_act);
  if (item + 3 < end) g1_item<false>(item + 3, end, b0, b2, st, sh, hidden, hscale, T, w13, s13, c_act);
}

// ---------------------------------------------------------------------------
// GEMM2 x routing weight + the ordered combine, decode shape (T <= 96; built for up to 128).
//
// Workgroup c owns output columns 28 c .. 28 c + 27 (W2 rows; 256 workgroups
// cover H = 7168 exactly, so every workgroup streams the same weight bytes) and
// takes every active expert in ascending id: one item per expert, 28 W2 rows x
// 2048 as two column blocks of the fp16 16x16x32 MFMA (the second block's last
// 4 columns repeat row 27 and are dropped). Each of the 8 waves owns 2 of the 16
// K blocks. Lane (fr, kg) reads 32 contiguous e4m3 bytes of a W2 row per K block
// and the same 32 K values (fp16, 64 B) of its activation row, so step j of a
// block takes K 32 kg + 8 j + [0, 8) in both operands. Weights stream through a
// 3-deep register ring (items i+1 and i+2 in flight while item i computes); the
// activation rows of item i+1 (the next expert's first 16 pairs) are loaded into
// registers during item i, ahead of item i+2's weights.
//
// The cross-wave sum of an item's tile times the pair's routing weight is added
// to its token's fp32 accumulator in LDS; items run in ascending expert id, so a
// token's sum is 0 + v(e1) + v(e2) + ... in ascending expert order (the order of
// ref_moe.py:164-166's accumulation over local experts). At the end the
// workgroup writes its 28 columns of every token as bf16 (round to nearest
// even), zeros for tokens without a local expert.
// ---------------------------------------------------------------------------
constexpr int D2_WAVES = 8;
constexpr int D2_COLS = 28;
constexpr int D2_NT = H / D2_COLS;       // 256 column chunks: the grid
constexpr int D2_KPW = NB_I / D2_WAVES;  // 2 K blocks per wave
constexpr int D2_LD = 2 * 2 * D2_KPW;    // 16 B weight loads per lane per item
static_assert(H % D2_COLS == 0 && D2_NT == 256 && NB_I % D2_WAVES == 0, "tile shape");
static_assert(D2_COLS % 4 == 0 && D2_COLS <= 32 && D2_COLS > 16, "two 16-column MFMA blocks, 4-column stores");

template <int TM>
struct G2Shared {
  int cnt[E_LOCAL];
  int seg[E_LOCAL + 1];
  int active[E_LOCAL];
  int nact;
  float pw[TM * TOP_K];  // pair -> routing weight
  int ptok[TM * TOP_K];  // pair -> token
  float red[2][D2_WAVES][2][4][64];  // lane index rotated by red_rot (bank-conflict-free reads)
  float acc[TM][33];  // token x column accumulators (row stride 33: the rows of two tokens never share banks)
};

// The cross-wave sum reads, per wave, 4 (column block, row) rows of red at the
// same 16 lane indices; rotating each row's lane index by 16 (2 cb + r) puts
// those 4 rows on 4 different groups of 16 banks.
__device__ __forceinline__ int red_rot(int cb, int r, int lane) { return (lane + 16 * ((2 * cb + r) & 3)) & 63; }

// Weights of expert le for this workgroup's columns c0 .. c0 + 27, this wave's 2 K blocks.
__device__ __forceinline__ void g2_load_w(v4i (&b)[D2_LD], const uint8_t* __restrict__ w2, int le, int c0, int kb0) {
  const int lane = threadIdx.x & 63, fr = lane & 15, kg = lane >> 4;
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int r = min(cb * 16 + fr, D2_COLS - 1);
    const uint8_t* wp = w2 + ((size_t)le * H + c0 + r) * I + kb0 * BLK + kg * 32;
#pragma unroll
    for (int kk = 0; kk < D2_KPW; ++kk) {
      b[(cb * D2_KPW + kk) * 2] = *reinterpret_cast<const v4i*>(wp + kk * BLK);
      b[(cb * D2_KPW + kk) * 2 + 1] = *reinterpret_cast<const v4i*>(wp + kk * BLK + 16);
    }
  }
}

// This wave's K slice (2 K blocks of fp16 activations) of pair rows m0 .. m0 + 15
// of an expert's segment (rows past cnt repeat the last one), in MFMA operand order.
struct G2A {
  v4i q[D2_KPW][4];
};
__device__ __forceinline__ void g2_load_a(G2A& a, const uint16_t* __restrict__ c_act, int seg, int cnt, int m0,
                                          int kb0) {
  const int lane = threadIdx.x & 63, fr = lane & 15, kg = lane >> 4;
  const uint16_t* ap = c_act + (size_t)(seg + min(m0 + fr, cnt - 1)) * I + kb0 * BLK + kg * 32;
#pragma unroll
  for (int kk = 0; kk < D2_KPW; ++kk)
#pragma unroll
    for (int q = 0; q < 4; ++q) a.q[kk][q] = *reinterpret_cast<const v4i*>(ap + kk * BLK + 8 * q);
}

// Item k (expert active[k]): a holds its first 16 pair rows on entry and item
// k + 1's on return; b holds its weights; b2 receives item k + 2's weights. An
// expert of more than 16 rows takes a pass per 16 rows, each after the first
// waiting for its rows and so for everything requested before them, item
// k + 2's weights included. (Requesting those weights after the last pass's
// rows instead, as the decode GEMM1 does, left the compiler unable to count the
// requests in flight on the one-pass path, whose first MFMAs then waited for
// most of them: the decode sweep 434 -> 450 us.)
template <bool PF, class SH>
__device__ __forceinline__ void g2_item(int k, int nact, int c0, G2A& a, v4i (&b)[D2_LD], v4i (&b2)[D2_LD],
                                        int& phase, SH& sh, const uint16_t* __restrict__ c_act,
                                        const uint8_t* __restrict__ w2, const float* __restrict__ s2) {
  const int tid = threadIdx.x, lane = tid & 63, fr = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kb0 = wave * D2_KPW;
  const int le = __builtin_amdgcn_readfirstlane(sh.active[k]);
  const int cnt = __builtin_amdgcn_readfirstlane(sh.cnt[le]), seg = __builtin_amdgcn_readfirstlane(sh.seg[le]);
  // block scales: the 28 columns touch the 128-row scale blocks of c0 and c0 + 27
  const int blo = c0 / BLK, bhi = (c0 + D2_COLS - 1) / BLK;
  const float* sp = s2 + (size_t)le * NB_H * NB_I + kb0;  // wave-uniform: scalar loads
  float sw[2][D2_KPW];
#pragma unroll
  for (int kk = 0; kk < D2_KPW; ++kk) {
    const float lo = sp[blo * NB_I + kk] * C_LOAD_SCALE, hi = sp[bhi * NB_I + kk] * C_LOAD_SCALE;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) sw[cb][kk] = (c0 + min(cb * 16 + fr, D2_COLS - 1)) / BLK == blo ? lo : hi;
  }
  G2A cur = a;
  if (k + 1 < nact) {
    const int ln = __builtin_amdgcn_readfirstlane(sh.active[k + 1]);
    g2_load_a(a, c_act, __builtin_amdgcn_readfirstlane(sh.seg[ln]), __builtin_amdgcn_readfirstlane(sh.cnt[ln]), 0,
              kb0);
  }
  if (PF || k + 2 < nact) g2_load_w(b2, w2, __builtin_amdgcn_readfirstlane(sh.active[k + 2]), c0, kb0);
  for (int m0 = 0; m0 < cnt; m0 += 16) {
    if (m0 > 0) g2_load_a(cur, c_act, seg, cnt, m0, kb0);
    v4f acc[2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      acc[cb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < D2_KPW; ++kk) {
        v4f p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const v4i wq = b[(cb * D2_KPW + kk) * 2 + (j >> 1)];
          const v8h wb = fp8x8_to_f16x8((uint32_t)wq[2 * (j & 1)], (uint32_t)wq[2 * (j & 1) + 1]);
          p = mfma_f16_k32(__builtin_bit_cast(v8h, cur.q[kk][j]), wb, p);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[cb][r] += p[r] * sw[cb][kk];
      }
    }
    float(&red)[D2_WAVES][2][4][64] = sh.red[phase & 1];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][cb][r][red_rot(cb, r, lane)] = acc[cb][r];
    lds_barrier();
    {
      // thread (row, col): pair row m0 + row, column col; MFMA lane (kg, fr) holds
      // rows 4 kg + r, column fr of each column block
      const int row = tid >> 5, col = tid & 31, cb = col >> 4, r = row & 3, src = (row >> 2) * 16 + (col & 15);
      if (col < D2_COLS && m0 + row < cnt) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < D2_WAVES; ++w) v += red[w][cb][r][red_rot(cb, r, src)];
        const int pr = seg + m0 + row;
        sh.acc[sh.ptok[pr]][col] += __fmul_rn(v, sh.pw[pr]);  // product rounded, then the sum
      }
    }
    ++phase;
  }
}

template <int TM>
__global__ __launch_bounds__(64 * D2_WAVES, 2) void gemm2_decode_kernel(
    const uint16_t* __restrict__ c_act, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const DispatchHeader* __restrict__ hdr, const int32_t* __restrict__ perm_tok, const float* __restrict__ perm_w,
    int T, uint16_t* __restrict__ out) {
  __shared__ G2Shared<TM> sh;
  const int tid = threadIdx.x;
  const int c0 = xcd_remap(blockIdx.x, D2_NT) * D2_COLS;  // an XCD's 32 workgroups: neighbouring column chunks
  if (tid < E_LOCAL) {
    sh.cnt[tid] = hdr->counts[tid];
    sh.seg[tid] = hdr->seg_start[tid];
    sh.active[tid] = hdr->active[tid];
  }
  if (tid == 0) {
    sh.seg[E_LOCAL] = hdr->seg_start[E_LOCAL];
    sh.nact = hdr->n_active;
  }
  for (int i = tid; i < TM * 33; i += 64 * D2_WAVES) (&sh.acc[0][0])[i] = 0.f;
  __syncthreads();
  const int nact = __builtin_amdgcn_readfirstlane(sh.nact);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), kb0 = wave * D2_KPW;
  v4i b0[D2_LD], b1[D2_LD], b2[D2_LD];
  G2A a;
  int phase = 0;
  const bool ring = nact >= 5;  // uniform: a steady state with unconditional requests
  // The pair tokens and weights and the first expert's activation rows are
  // requested ahead of item 0's weights, then item 1's weights; the pair tables go
  // to LDS once those requests are out.
  const int P = sh.seg[E_LOCAL];
  constexpr int D2_PPT = (TM * TOP_K + 64 * D2_WAVES - 1) / (64 * D2_WAVES);  // pairs per thread
  float pwv[D2_PPT];
  int ptv[D2_PPT];
#pragma unroll
  for (int j = 0; j < D2_PPT; ++j) {
    const int p = tid + 64 * D2_WAVES * j;
    pwv[j] = p < P ? perm_w[p] : 0.f;
    ptv[j] = p < P ? perm_tok[p] : 0;
  }
  if (nact > 0) {
    const int le0 = __builtin_amdgcn_readfirstlane(sh.active[0]);
    g2_load_a(a, c_act, __builtin_amdgcn_readfirstlane(sh.seg[le0]), __builtin_amdgcn_readfirstlane(sh.cnt[le0]), 0,
              kb0);
    g2_load_w(b0, w2, le0, c0, kb0);
  }
  if (nact > 1) g2_load_w(b1, w2, __builtin_amdgcn_readfirstlane(sh.active[1]), c0, kb0);
#pragma unroll
  for (int j = 0; j < D2_PPT; ++j) {
    const int p = tid + 64 * D2_WAVES * j;
    if (p < P) {
      sh.pw[p] = pwv[j];
      sh.ptok[p] = ptv[j];
    }
  }
  __syncthreads();
  int k = 0;
  if (ring) {
    for (; k + 4 < nact; k += 3) {  // items k+2..k+4 exist
      g2_item<true>(k, nact, c0, a, b0, b2, phase, sh, c_act, w2, s2);
      g2_item<true>(k + 1, nact, c0, a, b1, b0, phase, sh, c_act, w2, s2);
      g2_item<true>(k + 2, nact, c0, a, b2, b1, phase, sh, c_act, w2, s2);
    }
  }
  // the last (at most four) items; b0, b1 hold items k, k + 1
  if (k < nact) g2_item<false>(k, nact, c0, a, b0, b2, phase, sh, c_act, w2, s2);
  if (k + 1 < nact) g2_item<false>(k + 1, nact, c0, a, b1, b0, phase, sh, c_act, w2, s2);
  if (k + 2 < nact) g2_item<false>(k + 2, nact, c0, a, b2, b1, phase, sh, c_act, w2, s2);
  if (k + 3 < nact) g2_item<false>(k + 3, nact, c0, a, b0, b2, phase, sh, c_act, w2, s2);
  __syncthreads();
  // every token's 28 columns as bf16, 4 columns (8 B) per thread
  for (int i = tid; i < T * (D2_COLS / 4); i += 64 * D2_WAVES) {
    const int t = i / (D2_COLS / 4), c = (i % (D2_COLS / 4)) * 4;
    const float* v = &sh.acc[t][c];
    uint2 o;
    o.x = (uint32_t)f32_to_bf16_rne(v[0]) | ((uint32_t)f32_to_bf16_rne(v[1]) << 16);
    o.y = (uint32_t)f32_to_bf16_rne(v[2]) | ((uint32_t)f32_to_bf16_rne(v[3]) << 16);
    *reinterpret_cast<uint2*>(out + (size_t)t * H + c0 + c) = o;
  }
}


// ---------------------------------------------------------------------------
// Items of the tiled (prefill) kernels: (row tile, column tile) pairs.
//
// Row tiles are BM rows of one expert's segment (GEMM1: 256, GEMM2: 128),
// numbered expert by expert in descending order of the experts' row counts
// (ties: lower id first), each expert's tiles in row order. All tiles of an
// expert share its weight tiles, which stay in the caches while they run; the
// largest experts (whose tiles are full and cost the most: the waves skip row
// fragments past the valid count) come first, and the one-tile experts with few
// rows, the cheapest items, last, where they even out the workgroups' finishing
// times. The block order: blocks of TBM row tiles x TBN column tiles (GEMM1 4 x 8,
// GEMM2 8 x 4), row-block major.
//
// Both kernels deal the block order statically in rounds (snake_item): each
// 32-item block runs on the 32 workgroups of one XCD in step, sharing its
// activation and weight tiles in that XCD's L2. (Handing the items out at run
// time from per-XCD atomic work queues was measured: slower for GEMM1, whose
// workgroups then drift apart so that the L2 stops serving the repeats, and no
// faster for GEMM2.)
// ---------------------------------------------------------------------------
constexpr int TB_M = 8, TB_N = 4;

struct TileMap {
  int order[E_LOCAL];     // expert of each rank (descending row count)
  int pref[E_LOCAL + 1];  // first row tile of each rank
  int cnt[E_LOCAL];       // by expert id
  int seg[E_LOCAL];
  int total_m;            // row tiles
};

template <int BM>
__device__ __forceinline__ void build_tile_map(const DispatchHeader* hdr, TileMap& m) {
  const int tid = threadIdx.x;
  if (tid < 64) {
    const int lane = tid;
    const int cnt = lane < E_LOCAL ? hdr->counts[lane] : -1;
    const int seg = lane < E_LOCAL ? hdr->seg_start[lane] : 0;
    int rank = 0;  // experts before this one: more rows, or as many and a lower id
    for (int j = 0; j < E_LOCAL; ++j) {
      const int cj = __shfl(cnt, j);
      rank += (cj > cnt || (cj == cnt && j < lane)) ? 1 : 0;
    }
    if (lane < E_LOCAL) {
      m.cnt[lane] = cnt;
      m.seg[lane] = seg;
      m.order[rank] = lane;
    }
    // tiles by rank: this wave wrote order[] and reads it back (its own LDS
    // accesses stay in order)
    const int e = lane < E_LOCAL ? m.order[lane] : 0;
    int inc = lane < E_LOCAL ? (__shfl(cnt, e) + BM - 1) / BM : 0;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(inc, d);
      if (lane >= d) inc += o;
    }
    if (lane < E_LOCAL) m.pref[lane + 1] = inc;
    if (lane == 0) m.pref[0] = 0;
    if (lane == E_LOCAL - 1) m.total_m = inc;
  }
  __syncthreads();
}

// Row tile k -> its expert and first row within the expert's segment.
template <int BM>
__device__ __forceinline__ void tile_row(const TileMap& m, int k, int& e, int& m0) {
  int j = 0;
  while (m.pref[j + 1] <= k) ++j;
  e = m.order[j];
  m0 = (k - m.pref[j]) * BM;
}

// The static deal: item i of the block order (all blocks row-block
// major, the last row block's blocks shorter) -> item id k * nt_count + nt.
__device__ __forceinline__ int block_order_item(int i, int total_m, int nt_count) {
  const int nbk = nt_count / TB_N, nrb = (total_m + TB_M - 1) / TB_M;
  const int full = (nrb - 1) * nbk * TB_M * TB_N;
  int rb, cb, ii, rows;
  if (i < full) {
    const int b = i / (TB_M * TB_N);
    rb = b / nbk;
    cb = b % nbk;
    ii = i % (TB_M * TB_N);
    rows = TB_M;
  } else {
    rows = total_m - TB_M * (nrb - 1);
    rb = nrb - 1;
    cb = (i - full) / (rows * TB_N);
    ii = (i - full) % (rows * TB_N);
  }
  return (TB_M * rb + ii % rows) * nt_count + TB_N * cb + ii / rows;
}
// Round r of the G workgroups takes items r G .. r G + G - 1 of the block
// order: slot p (xcd_remap: the G / 8 slots of an XCD are consecutive, so each
// 32-item block runs on one XCD with its workgroups in step, sharing the
// block's operand tiles in its L2) takes item r G + p in even rounds and
// r G + G - 1 - p in odd ones, so that the slots that took the cheaper items of
// one round take the costlier ones of the next.
__device__ __forceinline__ int snake_item(int r, int slot, int G) { return r * G + ((r & 1) ? G - 1 - slot : slot); }


// ---------------------------------------------------------------------------
// One 16 x 128 e4m3 MFMA fragment in LDS (two 1 KB halves of 8 rows each).
constexpr int FRAG_BYTES = 2048;

// ---------------------------------------------------------------------------
// GEMM1 + SwiGLU, prefill shape: items of 256 rows x 128 column pairs (X1 rows
// n..n+127 and X2 rows 2048+n..), so an expert with up to 256 rows reads each
// weight byte once. 8 waves as 4 (row groups) x 2 (column halves): wave (wm,
// wn) owns the 16-row fragments 4 mt + wm (mt < 4; the groups interleave, so a
// partly filled tile spreads its valid fragments evenly over the waves) against
// 4 X1 and 4 X2 column fragments: 32 MFMAs of 16x16x128 per K block into 128
// fp32 accumulators. Fragments past the valid rows are skipped, and so are the
// direct loads of activation rows past them.
//
// Every wave computes, and every wave moves an eighth of each K block global ->
// LDS with direct loads into a ring of stages. An item with more than 128 valid
// rows uses 2 stages of 66 KB (the loads of block kb+1 fly while kb computes);
// one with at most 128 uses 3 stages of 50 KB (its activation part is half as
// large), so the loads of kb+2 fly while kb computes: such items do little MFMA
// work per block and would otherwise wait for an HBM round trip every block.
// The direct loads are issued from inline asm: the compiler does not track them,
// so it puts no wait for them before the fragment reads of the other stages (for
// the builtin it waits for every direct load in flight before any LDS read, which
// is why a design built on the builtin needs loader waves that never read LDS,
// and loses a third of the register file to them). The kernel waits for its own
// loads explicitly (s_waitcnt vmcnt) before the barrier that ends every K block.
// M0, which the direct load takes its LDS address from, is set in the same asm
// statement; nothing else in this kernel uses M0.
//
// The waves issue their direct loads at two points of the block: waves 0-3 at its
// top, waves 4-7 halfway through their MFMAs, so the two waves of a SIMD (w,
// w + 4) take turns. Issued by all waves at the top of the block they held every
// wave there for ~1,000 clk (the CU moves about 64 B/clk from L2 into LDS, 64 KB
// per block); split, the loads of one half run beside the other half's MFMAs,
// and a wave stalled on a full load queue leaves its SIMD to the other wave.
//
// Per K block and row the fp32 factors s_act[row, kb] * s_w[X1 or X2 block, kb]
// are formed once (wave w: row 64 (w % 4) + lane, X1 for w < 4, X2 above) and
// stored in the stage beside the operands as (X1, X2) pairs, one block ahead; the
// activation scales and the two weight block scales arrive two blocks ahead by
// direct loads into a small LDS buffer.
// ---------------------------------------------------------------------------
constexpr int P1_BM = 256;
constexpr int P1_BNP = 128;
constexpr int P1_NT = I / P1_BNP;          // 16 column-pair tiles
constexpr int P1_WAVES = 8;
constexpr int P1_THREADS = 64 * P1_WAVES;
constexpr int P1_B_BYTES = 2 * P1_BNP * BLK;  // 32 KB: 16 weight fragments (0-7 X1, 8-15 X2)
constexpr int P1_F_BYTES = 2 * P1_BM * 4;     // (X1, X2) factor pairs of the 256 rows
template <int NST>
struct P1Ring {  // the stage layout of an NST-stage ring
  static constexpr int A_BYTES = (NST == 2 ? P1_BM : P1_BM / 2) * BLK;
  static constexpr int B_OFF = A_BYTES;
  static constexpr int F_OFF = A_BYTES + P1_B_BYTES;
  static constexpr int STAGE = F_OFF + P1_F_BYTES;
  static constexpr int BYTES = NST * STAGE;
};
constexpr int P1_SA_OFF = P1Ring<2>::BYTES > P1Ring<3>::BYTES ? P1Ring<2>::BYTES : P1Ring<3>::BYTES;
constexpr int P1_SA_BUF = P1_BM * 4 + 16;  // activation scales of the 256 rows, then the X1 and X2 weight scales
constexpr int P1_LDS = P1_SA_OFF + 2 * P1_SA_BUF;
// 32-item blocks: 4 row tiles x 8 column tiles, or 2 x 16 when no expert has more
// than one row tile (every block then holds all column tiles of 2 experts, whose
// activation rows its 32 workgroups share; with several row tiles per expert the
// 4 x 8 blocks share weight tiles across row tiles instead). Measured per shape
// (GEMM1 us, T=1024 / 8192 / skew / T=14,107): 4 x 8 147.3 / 261.2 / 736.2 /
// 572.5, 2 x 16 140.1 / 263.1 / 745.9 / 577.3, 8 x 4 and 16 x 2 slower.
constexpr int P1_TBM = 4, P1_TBN = 8;
constexpr int P1_TBM1 = 2, P1_TBN1 = 16;
static_assert(P1_BM * BLK == 4 * P1_WAVES * 1024 && P1_B_BYTES == 4 * P1_WAVES * 1024,
              "4 half fragments of each operand per wave");
static_assert(P1_NT % P1_TBN == 0 && P1_TBM * P1_TBN == 32 && P1_NT % P1_TBN1 == 0 && P1_TBM1 * P1_TBN1 == 32,
              "block order");
static_assert(P1_LDS + (int)sizeof(TileMap) <= 160 * 1024, "LDS");
static_assert((size_t)MOE_FP8_CHUNK_TOKENS * H < (1ull << 32) && (size_t)E_LOCAL * N1 * H < (1ull << 32) &&
                  (size_t)E_LOCAL * NB_N1 * NB_H * 4 < (1ull << 32),
              "32-bit load offsets");

// LDS address of p as a scalar (the callers' addresses are uniform; inside a
// lane-divergent branch the compiler may otherwise keep them in a VGPR, which the
// asm's SGPR operand cannot take).
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p);
}

// Direct global -> LDS loads of 16 (4) B per lane from base + voff; lane l's bytes
// land at lds + 16 l (4 l). Untracked by the compiler (see above). s_nop 4 covers
// the wait states after an M0 write and after a VALU write of the base SGPRs.
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, const uint8_t* lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base),
               "s"(lds_addr(lds))
               : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t voff, const uint8_t* lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base),
               "s"(lds_addr(lds))
               : "memory");
}

// Loads of 4 token indices that the compiler does not track, waited for in the
// same asm statement: for a tracked load the compiler would also wait, before the
// first direct load that uses the result, for every direct load in flight.
__device__ __forceinline__ void ld_sync4(const int32_t* p0, const int32_t* p1, const int32_t* p2, const int32_t* p3,
                                         int& v0, int& v1, int& v2, int& v3) {
  asm volatile(
      "global_load_dword %0, %4, off\n\tglobal_load_dword %1, %5, off\n\t"
      "global_load_dword %2, %6, off\n\tglobal_load_dword %3, %7, off\n\ts_waitcnt vmcnt(0)"
      : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
      : "v"(p0), "v"(p1), "v"(p2), "v"(p3)
      : "memory");
}

__device__ __forceinline__ void ld_sync1(const int32_t* p, int& v) {
  asm volatile("global_load_dword %0, %1, off\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
}

// The static deal of block_order_item with the block shape as a parameter.
template <int BMT, int BNT>
__device__ __forceinline__ int block_order_item_t(int i, int total_m, int nt_count) {
  const int nbk = nt_count / BNT, nrb = (total_m + BMT - 1) / BMT;
  const int full = (nrb - 1) * nbk * BMT * BNT;
  int rb, cb, ii, rows;
  if (i < full) {
    const int b = i / (BMT * BNT);
    rb = b / nbk;
    cb = b % nbk;
    ii = i % (BMT * BNT);
    rows = BMT;
  } else {
    rows = total_m - BMT * (nrb - 1);
    rb = nrb - 1;
    cb = (i - full) / (rows * BNT);
    ii = (i - full) % (rows * BNT);
  }
  return (BMT * rb + ii % rows) * nt_count + BNT * cb + ii / rows;
}

struct P1Item {
  int e, m0, valid, nt, seg;
};

// Item of round r of this workgroup (false past the end). All values uniform.
// one_tile: no expert has more than one row tile (selects the 2 x 16 blocks).
__device__ __forceinline__ bool p1_item(const TileMap& map, int r, int slot, int G, int total, bool one_tile,
                                        P1Item& it) {
  const int i = snake_item(r, slot, G);
  if (i >= total) return false;
  const int id = one_tile ? block_order_item_t<P1_TBM1, P1_TBN1>(i, map.total_m, P1_NT)
                          : block_order_item_t<P1_TBM, P1_TBN>(i, map.total_m, P1_NT);
  const int k = id / P1_NT;
  int e, m0;
  tile_row<P1_BM>(map, k, e, m0);
  // values read from LDS are held per lane unless made scalar
  it.e = __builtin_amdgcn_readfirstlane(e);
  it.m0 = __builtin_amdgcn_readfirstlane(m0);
  it.nt = __builtin_amdgcn_readfirstlane(id - k * P1_NT);
  it.valid = __builtin_amdgcn_readfirstlane(min(P1_BM, map.cnt[it.e] - it.m0));
  it.seg = __builtin_amdgcn_readfirstlane(map.seg[it.e]);
  return true;
}

// Address of the token of tile row r; rows at or past the valid count take the first.
__device__ __forceinline__ const int32_t* p1_token_ptr(const int32_t* perm_tok, const P1Item& it, int r) {
  return perm_tok + it.seg + it.m0 + (r < it.valid ? r : 0);
}

struct P1Ctx {
  const uint8_t* hidden;
  const float* hscale;
  int T;
  const uint8_t* w13;
  const float* s13;
  uint16_t* c_act;
  int w, lane, wm, wn, fr, kg, flo, fhi, frow, fkind;
};

// One wave's loads of one item, as byte offsets: A half fragments 4 w + j (tile
// rows 32 w + 8 j + l / 8, from hidden) and B half fragments 4 w + j (fragment
// f = (4 w + j) / 2: X1 rows 128 nt + 16 f + ..., X2 rows for f >= 8, from w13),
// 16 B chunk (l % 8) ^ (l / 8) ^ half, without the K block's 128 B; the
// activation-scale row (waves 0-3, from hscale) and the X1 / X2 weight-scale rows
// (wave 4 lanes 0 / 1, from s13).
struct P1Src {
  uint32_t a[4], b[4];
  int na;          // A half fragments holding valid rows (uniform)
  uint32_t sa;     // activation scale of row 64 w + lane (waves 0-3)
  uint32_t sw;     // weight-scale row (wave 4, lanes 0 and 1)
};

__device__ __forceinline__ void p1_src(const P1Ctx& x, const int32_t* perm_tok, const P1Item& it, P1Src& s) {
  const int rr = x.lane >> 3;
  int tok[4], tsa;
  ld_sync4(p1_token_ptr(perm_tok, it, 32 * x.w + rr), p1_token_ptr(perm_tok, it, 32 * x.w + 8 + rr),
           p1_token_ptr(perm_tok, it, 32 * x.w + 16 + rr), p1_token_ptr(perm_tok, it, 32 * x.w + 24 + rr), tok[0],
           tok[1], tok[2], tok[3]);
  ld_sync1(p1_token_ptr(perm_tok, it, x.frow), tsa);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int h = 4 * x.w + j, half = h & 1, c = (x.lane & 7) ^ rr ^ half;
    s.a[j] = (uint32_t)tok[j] * H + c * 16;
    const int f = h >> 1;
    const int row = (f < 8 ? it.nt * P1_BNP + 16 * f : I + it.nt * P1_BNP + 16 * (f - 8)) + 8 * half + rr;
    s.b[j] = ((uint32_t)it.e * N1 + row) * H + c * 16;
  }
  s.na = min(4, max(0, (it.valid - 32 * x.w + 7) / 8));
  s.sa = (uint32_t)tsa * 4;
  s.sw = ((uint32_t)it.e * NB_N1 + ((x.lane & 1) ? NB_I + it.nt : it.nt)) * NB_H * 4;
}

// Scales of block kb into SA buffer kb % 2.
__device__ __forceinline__ void p1_scales(const P1Ctx& x, const P1Src& s, uint8_t* lds, int kb) {
  uint8_t* sb = lds + P1_SA_OFF + (kb & 1) * P1_SA_BUF;
  if (x.w < 4) dma4(x.hscale + (size_t)kb * x.T, s.sa, sb + 256 * x.w);
  if (x.w == 4 && x.lane < 2) dma4(x.s13 + kb, s.sw, sb + P1_BM * 4);
}

// This wave's factor of block kb (its scales are in SA buffer kb % 2) into the
// factor region f of the block's stage.
__device__ __forceinline__ void p1_factor(const P1Ctx& x, const uint8_t* lds, uint8_t* f, int kb) {
  const uint8_t* sb = lds + P1_SA_OFF + (kb & 1) * P1_SA_BUF;
  const float sa = reinterpret_cast<const float*>(sb)[x.frow];
  const float sw = reinterpret_cast<const float*>(sb + P1_BM * 4)[x.fkind];
  reinterpret_cast<float*>(f)[2 * x.frow + x.fkind] = sa * sw;
}

// This wave's operand loads of block kb into the stage at st.
template <int B_OFF>
__device__ __forceinline__ void p1_operands(const P1Ctx& x, const P1Src& s, uint8_t* st, int kb) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (j < s.na) dma16(x.hidden + kb * BLK, s.a[j], st + (4 * x.w + j) * 1024);
    dma16(x.w13 + kb * BLK, s.b[j], st + B_OFF + (4 * x.w + j) * 1024);
  }
}

// One K block of a wave: NMT valid token fragments (4 mt + wm) x 4 X1 + 4 X2 weight
// fragments, accumulated with the stage's factors. The weight fragment is the
// MFMA's first operand, so lane l's four results are weight columns 4 (l / 16) + r
// of one token (l % 16), and the token's two factors (X1, X2) are one 8-byte LDS
// read per fragment. The next block's operand loads (load(), when any) go out
// before column group DMA_AT; for DMA_AT > 0 empty asm statements that read the
// earlier groups' accumulators come first: asm volatile statements keep their
// order, so those groups' MFMAs stay above the loads (without them the
// instruction DAG sinks every MFMA below the loads).
template <int NMT, int DMA_AT, int B_OFF, int F_OFF, typename Load>
__device__ __forceinline__ void p1_block(const P1Ctx& x, const uint8_t* st, v4f (&au)[4][4], v4f (&ag)[4][4],
                                         const Load& load) {
  v8i a[NMT];
  v2f f[NMT];
#pragma unroll
  for (int mt = 0; mt < NMT; ++mt) {
    a[mt] = lds_frag_sw(st + (4 * mt + x.wm) * FRAG_BYTES, x.flo, x.fhi);
    f[mt] = *reinterpret_cast<const v2f*>(st + F_OFF + ((4 * mt + x.wm) * 16 + x.fr) * 8);
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if (c == DMA_AT) {
#pragma unroll
      for (int cc = 0; cc < DMA_AT; ++cc)
#pragma unroll
        for (int mt = 0; mt < NMT; ++mt) asm volatile("" ::"v"(au[mt][cc]), "v"(ag[mt][cc]));
      load();
    }
    const v8i bu = lds_frag_sw(st + B_OFF + (4 * x.wn + c) * FRAG_BYTES, x.flo, x.fhi);
    const v8i bg = lds_frag_sw(st + B_OFF + (8 + 4 * x.wn + c) * FRAG_BYTES, x.flo, x.fhi);
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) {
      const v4f pu = mfma_fp8_k128(bu, a[mt]);
      const v4f pg = mfma_fp8_k128(bg, a[mt]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        au[mt][c][r] += pu[r] * f[mt][0];
        ag[mt][c][r] += pg[r] * f[mt][1];
      }
    }
  }
}

// s_waitcnt vmcnt(n) for a uniform n in 0..8.
__device__ __forceinline__ void wait_vm(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
  }
}

// One item on an NST-stage ring (a wave with NMT valid token fragments): the
// prologue fills stages 0..NST-2 and the scales of blocks 0 and 1, then each
// block kb computes from stage kb % NST while its waves load block kb + NST - 1.
// Before the barrier that ends block kb each wave waits for all its loads but
// those of block kb + NST - 1 (loads complete in order; the scale loads of the
// block are issued before them), so block kb + 1's operands and kb + 2's scales
// are in place.
template <int NMT, int DMA_AT, int NST>
__device__ __forceinline__ void p1_run_item(const P1Ctx& x, const P1Item& ic, const P1Src& s, uint8_t* lds) {
  using R = P1Ring<NST>;
#pragma unroll
  for (int b = 0; b < NST - 1; ++b) p1_operands<R::B_OFF>(x, s, lds + b * R::STAGE, b);
  p1_scales(x, s, lds, 0);
  p1_scales(x, s, lds, 1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  lds_barrier();
  p1_factor(x, lds, lds + R::F_OFF, 0);
  lds_barrier();

  v4f au[4][4], ag[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      au[mt][c] = v4f{0.f, 0.f, 0.f, 0.f};
      ag[mt][c] = au[mt][c];
    }
  const int n_ld = s.na + 4;  // direct loads of this wave per block
  int cur = 0;
#pragma unroll 1
  for (int kb = 0; kb < NB_H; ++kb) {
    const int nxt = cur == NST - 1 ? 0 : cur + 1;          // stage of block kb + 1
    const int ld = NST == 2 ? nxt : (nxt == NST - 1 ? 0 : nxt + 1);  // stage of block kb + NST - 1
    if (kb + 1 < NB_H) p1_factor(x, lds, lds + nxt * R::STAGE + R::F_OFF, kb + 1);
    if (kb + 2 < NB_H) p1_scales(x, s, lds, kb + 2);
    const int kl = kb + NST - 1;
    const bool loading = kl < NB_H;
    auto load = [&]() {
      if (loading) p1_operands<R::B_OFF>(x, s, lds + ld * R::STAGE, kl);
    };
    if constexpr (NMT > 0) {
      p1_block<NMT, DMA_AT, R::B_OFF, R::F_OFF>(x, lds + cur * R::STAGE, au, ag, load);
    } else {
      load();
    }
    if (kb == NB_H - 1) {
      // SwiGLU and the fp16 C rows (lane l: token row 16 (4 mt + wm) + l % 16, four
      // consecutive columns from 4 (l / 16) of each of its 4 column fragments)
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) {
        const int row = (4 * mt + x.wm) * 16 + x.fr;
        if (row < ic.valid) {
          uint16_t* dst = x.c_act + (size_t)(ic.seg + ic.m0 + row) * I + ic.nt * P1_BNP + 4 * x.kg;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            uint2 v;
            v.x = (uint32_t)c_encode(silu_mul(au[mt][c][0], ag[mt][c][0])) |
                  ((uint32_t)c_encode(silu_mul(au[mt][c][1], ag[mt][c][1])) << 16);
            v.y = (uint32_t)c_encode(silu_mul(au[mt][c][2], ag[mt][c][2])) |
                  ((uint32_t)c_encode(silu_mul(au[mt][c][3], ag[mt][c][3])) << 16);
            *reinterpret_cast<uint2*>(dst + (4 * x.wn + c) * 16) = v;
          }
        }
      }
    }
    if (NST == 2 || !loading)
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else
      wait_vm(n_ld);
    lds_barrier();
    cur = nxt;
  }
}

template <int DMA_AT>
__device__ __forceinline__ void p1_dispatch(const P1Ctx& x, const P1Item& ic, const P1Src& s, uint8_t* lds) {
  const int nf = (ic.valid + 15) / 16;
  const int nmt = nf > x.wm ? (nf - x.wm + 3) / 4 : 0;
  if (ic.valid > P1_BM / 2) {  // nf >= 9: nmt >= 2
    switch (nmt) {
      case 2: p1_run_item<2, DMA_AT, 2>(x, ic, s, lds); break;
      case 3: p1_run_item<3, DMA_AT, 2>(x, ic, s, lds); break;
      default: p1_run_item<4, DMA_AT, 2>(x, ic, s, lds); break;
    }
  } else {  // nf <= 8: nmt <= 2
    switch (nmt) {
      case 0: p1_run_item<0, DMA_AT, 3>(x, ic, s, lds); break;
      case 1: p1_run_item<1, DMA_AT, 3>(x, ic, s, lds); break;
      default: p1_run_item<2, DMA_AT, 3>(x, ic, s, lds); break;
    }
  }
}

__global__ __launch_bounds__(P1_THREADS, 1) void gemm1_prefill_kernel(
    const uint8_t* __restrict__ hidden, const float* __restrict__ hscale, int T, const uint8_t* __restrict__ w13,
    const float* __restrict__ s13, const DispatchHeader* __restrict__ hdr, const int32_t* __restrict__ perm_tok,
    uint16_t* __restrict__ c_act) {
  extern __shared__ __attribute__((aligned(16))) uint8_t p1_lds[];
  __shared__ TileMap map;
  const int tid = threadIdx.x, lane = tid & 63;
  build_tile_map<P1_BM>(hdr, map);
  P1Ctx x;
  x.hidden = hidden; x.hscale = hscale; x.T = T; x.w13 = w13; x.s13 = s13; x.c_act = c_act;
  x.w = __builtin_amdgcn_readfirstlane(tid >> 6);
  x.lane = lane;
  x.wm = x.w & 3; x.wn = x.w >> 2; x.fr = lane & 15; x.kg = lane >> 4;
  frag_sw_offsets(lane, x.flo, x.fhi);
  x.frow = 64 * (x.w & 3) + lane;  // the factor row this wave forms
  x.fkind = x.w >> 2;              // 0: X1, 1: X2
  const int total = __builtin_amdgcn_readfirstlane(map.total_m) * P1_NT, G = gridDim.x;
  const int slot = xcd_remap(blockIdx.x, G);
  const bool one_tile = __builtin_amdgcn_ballot_w64((lane < E_LOCAL ? map.cnt[lane] : 0) > P1_BM) == 0;  // uniform
#pragma unroll 1
  for (int r = 0;; ++r) {
    P1Item ic;
    if (!p1_item(map, r, slot, G, total, one_tile, ic)) break;
    P1Src s;
    p1_src(x, perm_tok, ic, s);
    if (x.w < 4)
      p1_dispatch<0>(x, ic, s, p1_lds);
    else
      p1_dispatch<2>(x, ic, s, p1_lds);
  }
}

// ---------------------------------------------------------------------------
// GEMM2 (+ routing weight), prefill shape: 128 rows x 256 output columns per
// item on the fp16 MFMA v_mfma_f32_32x32x16_f16 (full fp16 rate; the 16x16x32
// form runs at well under half of it), 8 compute waves as 2 (rows) x 4
// (columns), each 64 x 64 = 2 x 2 tiles of 32 x 32 (row blocks 2 i + wm, so
// the two row halves interleave), and 4 loader waves.
//
// One stage is one 128-wide K block (the W2 scale block): the activation tile
// (128 rows x 256 B fp16) and the W2 tile (256 rows x 128 B e4m3), 64 KB, in a
// 2-slot LDS ring; the next block's direct loads fly while this one computes.
// Every load instruction moves 8 whole 128 B row lines, and the LDS holds
// 32-row x 128 B regions with the 16 B chunks XOR-swizzled per row (sw32), so
// the fragment reads are conflict-free. K order inside a block (any bijection
// shared by both operands leaves the MFMA sums unchanged): MFMA step t, lane
// group g takes K 16 (2 (t / 2) + g) + 8 (t % 2) + [0, 8). A lane therefore
// reads one 16 B W2 chunk per pair of steps and widens it exactly to fp16,
// and reads the matching 16 B of fp16 activations per step. The fp32 weight
// block scale is applied once per block.
// ---------------------------------------------------------------------------
constexpr int Q2_BM = 128;
constexpr int Q2_BN = 256;
constexpr int Q2_NT = H / Q2_BN;          // 28 column tiles
constexpr int Q2_REG = 4096;              // 32 rows x 128 B
constexpr int Q2_A_BYTES = Q2_BM * BLK * 2;  // 32 KB: 4 row blocks x 2 lines
constexpr int Q2_B_BYTES = Q2_BN * BLK;      // 32 KB: 8 row blocks
constexpr int Q2_STAGE = Q2_A_BYTES + Q2_B_BYTES;



// ---------------------------------------------------------------------------
// GEMM2 kernel: the item, stage layout and K order above, with the global ->
// LDS traffic (64 load instructions per K block, 16 per loader wave: waves 0-1
// the activation rows, 2-3 the W2 rows) issued by 4 loader waves while the 8
// compute waves read LDS, widen W2 and run MFMAs (as in GEMM1, a wave that
// issues loads would hold back its MFMAs while the memory pipeline is busy). The two 64 KB slots run on across items: after K block kb's barrier
// the loaders fill the other slot with block kb + 1 (of this item or the next).
// The last loader wave also carries the block's two W2 block scales (output
// column blocks 2 nt and 2 nt + 1) into the stage.
// ---------------------------------------------------------------------------
constexpr int W2_CWAVES = 8;
constexpr int W2_PWAVES = 4;
constexpr int W2_THREADS = 64 * (W2_CWAVES + W2_PWAVES);
constexpr int W2_LJOBS = (Q2_A_BYTES + Q2_B_BYTES) / 1024 / W2_PWAVES;  // 16 load instructions per loader wave
constexpr int W2_WSCALE_OFF = Q2_STAGE;
constexpr int W2_STAGE = Q2_STAGE + 16;
static_assert(W2_LJOBS * W2_PWAVES == 64, "64 load instructions per K block");

// One item for a compute wave of the GEMM2 loader kernel: NI of its 32-row
// blocks (2 i + wm, i < NI) against its two 32-column W2 blocks over the 16 K
// blocks, then its rows of the item, times each pair's routing weight, as fp32
// rows. Row blocks past the item's valid rows are skipped; every wave takes
// the barrier of every K block whatever its NI. (Each NI runs the whole item,
// accumulators included, so that no accumulator lives across the choice.)
struct G2Item {
  int m0, cnt, seg, nt;
};
template <int NI>
__device__ __forceinline__ void g2_loader_item(const uint8_t* q2_lds, int& slot, int wm, int wn, int lane,
                                               const G2Item& it, const float* __restrict__ perm_w,
                                               uint16_t* __restrict__ partial) {
  const int lr = lane & 31, lg = lane >> 5;
  v16f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v16f{};
  int boff[4], aoff[2][2];
#pragma unroll
  for (int pp = 0; pp < 4; ++pp) boff[pp] = sw32(lr, 2 * pp + lg);
#pragma unroll
  for (int ph = 0; ph < 2; ++ph)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) aoff[ph][tt] = sw32(lr, 4 * ph + 2 * lg + tt);
#pragma unroll 1
  for (int kb = 0; kb < NB_I; ++kb) {
    __builtin_amdgcn_s_barrier();  // block kb is in its slot
    asm volatile("" ::: "memory");
    const uint8_t* st = q2_lds + slot * W2_STAGE;
    slot ^= 1;
    if constexpr (NI > 0) {
      const uint8_t* sb = st + Q2_A_BYTES + (wn * 2) * Q2_REG;  // this wave's two W2 row blocks
      v16f pacc[NI][2];
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) pacc[i][j] = v16f{};
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        v8h bf[2][2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const v4i raw = *reinterpret_cast<const v4i*>(sb + j * Q2_REG + boff[pp]);
          bf[j][0] = fp8x8_to_f16x8((uint32_t)raw[0], (uint32_t)raw[1]);
          bf[j][1] = fp8x8_to_f16x8((uint32_t)raw[2], (uint32_t)raw[3]);
        }
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          v8h af[NI];
#pragma unroll
          for (int i = 0; i < NI; ++i)  // row block 2 i + wm: two 128 B halves of the K block
            af[i] = *reinterpret_cast<const v8h*>(st + ((2 * i + wm) * 2 + (pp >> 1)) * Q2_REG + aoff[pp & 1][tt]);
#pragma unroll
          for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) pacc[i][j] = mfma_f16_32x32x16(af[i], bf[j][tt], pacc[i][j]);
        }
      }
      const float sc = *reinterpret_cast<const float*>(st + W2_WSCALE_OFF + 4 * (wn >> 1)) * C_LOAD_SCALE;
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] += pacc[i][j][r] * sc;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this block's LDS reads are done
  }
  // epilogue: weight by the pair's routing weight, one row per pair, stored as
  // fp16 of w * O * 2^-8 (c_encode: 11 significant bits, the encoding of C; the
  // combine sums the decoded rows in fp32). The
  // weights of a row block's 32 rows are uniform over the wave and read with
  // scalar loads (counted by lgkmcnt), so no wait covers the stores before them:
  // a vector load here would wait, on vmcnt, for every store in flight. Rows past
  // the valid ones read the next pairs' weights (or the workspace region after
  // the weights), unused. The stores are buffer stores through a resource per
  // row whose range ends at the expert's last valid row, so the stores of rows
  // past it are dropped without a branch, and each lane's address is one 32-bit
  // offset (with 64-bit row pointers the compiler spilled, and every reload's
  // wait also waited for the stores before it).
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int rb = it.m0 + (2 * i + wm) * 32;  // the row block's first row (uniform)
    const float* wp = perm_w + it.seg + rb;
    float wl[16], wh[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      wl[r] = wp[8 * (r / 4) + (r % 4)];
      wh[r] = wp[8 * (r / 4) + 4 + (r % 4)];
    }
    // lane l's row of step r is 8 (r / 4) + r % 4 (uniform) + 4 lg: each step's
    // resource starts at its uniform row, the lane's offset adds 4 lg rows and
    // its column
    const uint32_t off = (uint32_t)((4 * lg * H + lr) * (int)sizeof(uint16_t));
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int r0 = rb + 8 * (r / 4) + (r % 4);
      const __amdgpu_buffer_rsrc_t dst =
          buf_rsrc(partial + (size_t)(it.seg + r0) * H + it.nt * Q2_BN + wn * 64,
                   (uint32_t)(max(it.cnt - r0, 0) * H * (int)sizeof(uint16_t)));
      const float w = lg ? wh[r] : wl[r];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        __builtin_amdgcn_raw_buffer_store_b16(c_encode(acc[i][j][r] * w), dst, off + j * 32 * (int)sizeof(uint16_t),
                                              0, 0);
    }
  }
}

// The GEMM2 kernel body for BM-row items (BM = 128, or 64 when no expert has
// more than 64 rows: the activation waves then load half a stage's activation
// part, 8 of their 16 load instructions, and the compute waves never have more
// than one 32-row block each). The stage layout is the same for both.
template <int BM>
__device__ __forceinline__ void g2_loader_body(const uint16_t* __restrict__ c_act, const uint8_t* __restrict__ w2,
                                               const float* __restrict__ s2, const DispatchHeader* __restrict__ hdr,
                                               const float* __restrict__ perm_w, uint16_t* __restrict__ partial,
                                               uint8_t* q2_lds, TileMap& map) {
  static_assert(BM == Q2_BM || BM == Q2_BM / 2, "128- or 64-row items");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  build_tile_map<BM>(hdr, map);
  const int total = __builtin_amdgcn_readfirstlane(map.total_m) * Q2_NT, G = gridDim.x;
  const int my_slot = xcd_remap(blockIdx.x, G);

  if (wave >= W2_CWAVES) {
    // ----------------------------- loader waves -----------------------------
    // Blocks go global -> registers -> LDS. While block g + 1 is in flight into
    // this wave's other register buffer, block g is written into its LDS slot
    // (the compute waves finished the block that held the slot before the
    // previous barrier) and the freed buffer takes block g + 2: two blocks in
    // flight per CU, where direct global -> LDS loads into the 2-slot ring
    // allow one. The loads are unconditional buffer loads (a zero-byte range
    // once no item is left: zeros, no memory access) so that the compiler
    // counts the loads in flight and waits only for the older block's.
    const int p = wave - W2_CWAVES, ld_row = lane >> 3;
    const bool a_wave = p < 2;
    __amdgpu_buffer_rsrc_t rsrc = buf_rsrc(w2, 0), srsrc = buf_rsrc(s2, 0);
    const uint32_t step_bytes = a_wave ? 2 * BLK : BLK;  // activation rows advance 256 B per K block, W2 rows 128 B
    const int map_total_m = __builtin_amdgcn_readfirstlane(map.total_m);
    const uint32_t row_bytes = a_wave ? I * 2 : I;
    // Job i (8 rows x 128 B, lane l: row l / 8, 16 B chunk (l % 8) ^ (l / 8) ^
    // parity) sits at byte job_off(i) + lane_off[i % 2] of the tile: no
    // per-job registers. Activation jobs: 32-row block 2 p + i / 8, half
    // (i / 4) % 2 of the 256 B row, 8-row group i % 4; W2 jobs: 32-row block
    // 4 (p - 2) + i / 4, 8-row group i % 4.
    uint32_t lane_off[2];
#pragma unroll
    for (int par = 0; par < 2; ++par) lane_off[par] = ld_row * row_bytes + (((lane & 7) ^ ld_row ^ par) * 16);
    auto run = [&](auto nj) {
      constexpr int NJ = decltype(nj)::value;
      const int jbase = a_wave ? p * NJ : p * W2_LJOBS;  // this wave's first job of the stage
      // job i: 8 rows x 128 B at byte job_off(i) + lane_off[i % 2] of the tile
      auto job_off = [&](int i) -> uint32_t {
        const int j = jbase + i;
        return a_wave ? (uint32_t)(((j >> 3) * 32 + (j & 3) * 8) * (I * 2) + ((j >> 2) & 1) * 128)
                      : (uint32_t)((((p - 2) * 4 + (i >> 2)) * 32 + (i & 3) * 8) * I);
      };
      int round = -1, kb = NB_I, nreal = 0;
      bool more = true;
      auto next_item = [&]() -> bool {
        const int i_next = snake_item(++round, my_slot, G);
        if (i_next >= total) {
          rsrc = buf_rsrc(w2, 0);
          srsrc = buf_rsrc(s2, 0);
          return false;
        }
        const int it = block_order_item(i_next, map_total_m, Q2_NT);
        const int k = it / Q2_NT, nt = it % Q2_NT;
        int e, m0;
        tile_row<BM>(map, k, e, m0);
        e = __builtin_amdgcn_readfirstlane(e);
        m0 = __builtin_amdgcn_readfirstlane(m0);
        const int cnt = __builtin_amdgcn_readfirstlane(map.cnt[e]), seg = __builtin_amdgcn_readfirstlane(map.seg[e]);
        const int valid = min(BM, cnt - m0);
        // the activation range ends at the valid rows: rows past it load as zeros
        // (their output rows are dropped)
        rsrc = a_wave ? buf_rsrc(c_act + (size_t)(seg + m0) * I, (uint32_t)valid * I * 2)
                      : buf_rsrc(w2 + ((size_t)e * H + nt * Q2_BN) * I, (uint32_t)Q2_BN * I);
        // the block scales of output column blocks 2 nt and 2 nt + 1
        srsrc = buf_rsrc(s2 + ((size_t)e * NB_H + 2 * nt) * NB_I, 2 * NB_I * 4);
        kb = 0;
        return true;
      };
      auto load_block = [&](v4i (&buf)[NJ], float& sv) {
        if (kb == NB_I && more) more = next_item();
        const int kk = more ? kb : 0;
        // the scale first: a later load into the same register then waits for this
        // small load alone, not for the block's data loads behind it
        // (the order of the loads is pinned: the same in every copy of this code,
        // so that the compiler's count of the loads in flight agrees at the loop head)
        __builtin_amdgcn_sched_barrier(0);
        sv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(srsrc, (uint32_t)(((lane & 1) * NB_I + kk) * 4), 0, 0));
  #pragma unroll
        for (int i = 0; i < NJ; ++i) {
          __builtin_amdgcn_sched_barrier(0);
          buf[i] = __builtin_bit_cast(
              v4i, __builtin_amdgcn_raw_buffer_load_b128(rsrc, lane_off[i & 1] + job_off(i), kk * step_bytes, 0));
        }
        __builtin_amdgcn_sched_barrier(0);
        if (more) {
          ++kb;
          ++nreal;
        }
      };
      auto store_block = [&](int g, const v4i (&buf)[NJ], float sv) {
        uint8_t* st = q2_lds + (g & 1) * W2_STAGE;
  #pragma unroll
        for (int i = 0; i < NJ; ++i) {
          const int job = jbase + i, rg = job & 3;
          const int dst = a_wave ? ((job >> 3) * 2 + ((job >> 2) & 1)) * Q2_REG + rg * 1024
                                 : Q2_A_BYTES + ((job - 32) >> 2) * Q2_REG + rg * 1024;
          *reinterpret_cast<v4i*>(st + dst + 16 * lane) = buf[i];
        }
        if (p == W2_PWAVES - 1 && lane < 2) *reinterpret_cast<float*>(st + W2_WSCALE_OFF + 4 * lane) = sv;
      };
      v4i buf0[NJ], buf1[NJ];
      float sv0, sv1;
      load_block(buf0, sv0);
      load_block(buf1, sv1);
      // Two blocks per pass, every load and store unconditional (one path through
      // the loop for the compiler's count of loads in flight). When block g + 1
      // does not exist its store writes zeros into a slot no wave reads any more
      // (block g - 1's, finished before barrier g), and its barrier is skipped.
      int g = 0;
      if (nreal > 0) {
  #pragma unroll 1
        do {
          store_block(g, buf0, sv0);  // block g; its slot held block g - 2, read before the last barrier
          load_block(buf0, sv0);      // block g + 2
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          __builtin_amdgcn_s_barrier();  // block g is in its slot; block g - 1 is read
          asm volatile("" ::: "memory");
          store_block(g + 1, buf1, sv1);
          load_block(buf1, sv1);  // block g + 3
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if (g + 1 < nreal) __builtin_amdgcn_s_barrier();
          asm volatile("" ::: "memory");
          g += 2;
        } while (g < nreal);
      }
    };
    // the activation waves load BM rows (NJ = 16: 32-row blocks 2 p and 2 p + 1;
    // 8: block p), the W2 waves 256 rows
    if (a_wave) run(std::integral_constant<int, W2_LJOBS * BM / Q2_BM>{});
    else run(std::integral_constant<int, W2_LJOBS>{});
    return;
  }

  // ------------------------------- compute waves -------------------------------
  const int wm = wave & 1, wn = wave >> 1;
  int slot = 0;
  for (int round = 0;; ++round) {
    const int i = snake_item(round, my_slot, G);
    if (i >= total) break;
    const int it = block_order_item(i, map.total_m, Q2_NT);
    const int k = it / Q2_NT, nt = it % Q2_NT;
    int e, m0;
    tile_row<BM>(map, k, e, m0);
    const int cnt = map.cnt[e], seg = map.seg[e];
    // 32-row blocks holding valid rows; this wave's are 2 i + wm for i < ni
    const int nb = (min(BM, cnt - m0) + 31) / 32;
    const int ni = (nb + 1 - wm) / 2;
    const G2Item gi{m0, cnt, seg, nt};
    switch (ni) {
      case 0: g2_loader_item<0>(q2_lds, slot, wm, wn, lane, gi, perm_w, partial); break;
      case 1: g2_loader_item<1>(q2_lds, slot, wm, wn, lane, gi, perm_w, partial); break;
      default: g2_loader_item<2>(q2_lds, slot, wm, wn, lane, gi, perm_w, partial); break;
    }
  }
}

__global__ __launch_bounds__(W2_THREADS, 1) void gemm2_loader_kernel(
    const uint16_t* __restrict__ c_act, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const DispatchHeader* __restrict__ hdr, const float* __restrict__ perm_w, uint16_t* __restrict__ partial) {
  extern __shared__ __attribute__((aligned(16))) uint8_t q2_lds[];
  __shared__ TileMap map;
  // 64-row items when every expert has at most 64 rows (uniform over the grid)
  const int lane = threadIdx.x & 63;
  const bool small = __builtin_amdgcn_ballot_w64(lane < E_LOCAL && hdr->counts[min(lane, E_LOCAL - 1)] > Q2_BM / 2) == 0;
  if (small) g2_loader_body<Q2_BM / 2>(c_act, w2, s2, hdr, perm_w, partial, q2_lds, map);
  else g2_loader_body<Q2_BM>(c_act, w2, s2, hdr, perm_w, partial, q2_lds, map);
}

// ---------------------------------------------------------------------------
// Ordered combine: out[t] = bf16( sum_j pair row(t, j) ) over t's local experts
// in ascending id, the rows decoded from fp16 (x 2^8, exact) and summed in fp32;
// zeros for tokens with none. Each lane takes 8 columns, one 16 B load per pair.
// The token's pair slots that hold a local pair (a uniform bit set) fix the
// number N of loads; a body compiled for each N issues its N loads together and
// then sums (with a branch per slot the compiler waited for each load before
// issuing the next; with all 8 slots loading, a mostly empty token paid for 8
// load instructions). The pair rows are read once: non-temporal loads, which
// leave the caches (the 256 MB memory-side cache above all) to data that is
// used again, such as the expert weights.
// ---------------------------------------------------------------------------
constexpr int CPOL_NT = 2;  // cache-policy operand of the buffer-load builtins: non-temporal
constexpr int COMBINE_THREADS = 128;
constexpr int COMBINE_COLS = 8 * COMBINE_THREADS;  // 1024 columns per workgroup
static_assert(H % COMBINE_COLS == 0, "the combine grid covers H");

// The N pairs of slot set m (ascending slots; lane j of pv holds slot j's pair),
// summed into acc.
template <int N>
__device__ __forceinline__ void combine_pairs(const uint16_t* __restrict__ partial, int pv, uint32_t m,
                                              float (&acc)[8]) {
  v4i v[N];  // 8 fp16 values each
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const int slot = __builtin_ctz(m);  // uniform
    m &= m - 1u;
    const int pr = __builtin_amdgcn_readlane(pv, slot);
    const __amdgpu_buffer_rsrc_t r = buf_rsrc(partial + (size_t)pr * H + blockIdx.y * COMBINE_COLS,
                                              COMBINE_COLS * (uint32_t)sizeof(uint16_t));
    v[k] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, threadIdx.x * 16u, 0, CPOL_NT));
  }
#pragma unroll
  for (int k = 0; k < N; ++k)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // (halves taken with shifts: __builtin_bit_cast of a vector element such
      // as v[k][q] reads element 0 on this compiler)
      const uint32_t w = (uint32_t)v[k][q];
      acc[2 * q] += (float)__builtin_bit_cast(_Float16, (uint16_t)w) * C_LOAD_SCALE;
      acc[2 * q + 1] += (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)) * C_LOAD_SCALE;
    }
}

__global__ __launch_bounds__(COMBINE_THREADS) void combine_kernel(const uint16_t* __restrict__ partial,
                                                                  const int32_t* __restrict__ tok_pair, int T,
                                                                  uint16_t* __restrict__ out) {
  // workgroup (t, c): token t, columns 1024 c .. 1024 c + 1023, 8 per thread
  const int t = blockIdx.x, h = blockIdx.y * COMBINE_COLS + threadIdx.x * 8;
  // The token's 8 pair slots sit in lanes 0-7 (repeated above), and each pair's
  // index is read back with readlane at its uniform slot number. An int[8] copy
  // indexed in a loop was placed in LDS by the compiler, whose per-thread LDS
  // addressing reads the workgroup size from the dispatch packet: one scalar read
  // of that packet per wave held every workgroup 3-12 us at its start.
  const int pv = tok_pair[(size_t)t * TOP_K + (threadIdx.x & (TOP_K - 1))];
  const uint32_t m = (uint32_t)__builtin_amdgcn_ballot_w64(pv >= 0) & ((1u << TOP_K) - 1u);  // slots with a pair
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  switch (__popc(m)) {  // uniform
    case 0: break;
    case 1: combine_pairs<1>(partial, pv, m, acc); break;
    case 2: combine_pairs<2>(partial, pv, m, acc); break;
    case 3: combine_pairs<3>(partial, pv, m, acc); break;
    case 4: combine_pairs<4>(partial, pv, m, acc); break;
    case 5: combine_pairs<5>(partial, pv, m, acc); break;
    case 6: combine_pairs<6>(partial, pv, m, acc); break;
    case 7: combine_pairs<7>(partial, pv, m, acc); break;
    default: combine_pairs<8>(partial, pv, m, acc); break;
  }
  v4i o;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    o[q] = (int)((uint32_t)f32_to_bf16_rne(acc[2 * q]) | ((uint32_t)f32_to_bf16_rne(acc[2 * q + 1]) << 16));
  *reinterpret_cast<v4i*>(out + (size_t)t * H + h) = o;
}

}  // namespace moe

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
namespace moe {

// The decode kernels are built for 64 and for 128 tokens (the LDS dispatch and
// the per-token sums sized to match); a call takes the smaller one that holds T.
template <int TM>
static hipError_t gemm1_decode_set_lds() {
  static PerDeviceOnce<hipError_t> once;
  hipError_t e = hipErrorInvalidDevice;
  once.get([] { return hipFuncSetAttribute(reinterpret_cast<const void*>(gemm1_decode_kernel<TM>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(G1Shared<TM>)); },
           e);
  return e;
}

template <int TM>
static int gemm1_decode_blocks_per_cu_t() {
  static PerDeviceOnce<int> once;
  int n = 1;
  once.get([] {
    int k = 0;
    if (gemm1_decode_set_lds<TM>() != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&k, gemm1_decode_kernel<TM>, 64 * D1_WAVES,
                                                     sizeof(G1Shared<TM>)) != hipSuccess ||
        k < 1)
      k = 1;
    return k;
  }, n);
  return n;
}

int gemm1_decode_blocks_per_cu(int T) {
  return T <= 64 ? gemm1_decode_blocks_per_cu_t<64>() : gemm1_decode_blocks_per_cu_t<SMALL_T>();
}

hipError_t launch_gemm1_decode(const float* logits, const uint16_t* bias, float rsf, bool route_here,
                               const uint8_t* hidden, const float* hscale, int T, int offset, const uint8_t* w13,
                               const float* s13, int32_t* topk_ids, float* topk_w, DispatchHeader* hdr,
                               int32_t* perm_tok, float* perm_w, int32_t* tok_pair, uint16_t* c_act, int grid,
                               hipStream_t stream) {
  if (T <= 0 || T > SMALL_T || (route_here && T > D1_WAVES)) return hipErrorInvalidValue;
  auto launch = [&](auto tm) {
    constexpr int TM = decltype(tm)::value;
    const hipError_t e = gemm1_decode_set_lds<TM>();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(gemm1_decode_kernel<TM>, dim3(grid), dim3(64 * D1_WAVES), sizeof(G1Shared<TM>), stream,
                       logits, bias, rsf, route_here ? 1 : 0, hidden, hscale, T, offset, w13, s13, topk_ids, topk_w,
                       hdr, perm_tok, perm_w, tok_pair, c_act);
    return hipGetLastError();
  };
  return T <= 64 ? launch(std::integral_constant<int, 64>{}) : launch(std::integral_constant<int, SMALL_T>{});
}

hipError_t launch_gemm2_decode(const uint16_t* c_act, const uint8_t* w2, const float* s2, const DispatchHeader* hdr,
                               const int32_t* perm_tok, const float* perm_w, int T, uint16_t* out,
                               hipStream_t stream) {
  if (T <= 0 || T > SMALL_T) return hipErrorInvalidValue;
  if (T <= 64)
    hipLaunchKernelGGL(gemm2_decode_kernel<64>, dim3(D2_NT), dim3(64 * D2_WAVES), 0, stream, c_act, w2, s2, hdr,
                       perm_tok, perm_w, T, out);
  else
    hipLaunchKernelGGL(gemm2_decode_kernel<SMALL_T>, dim3(D2_NT), dim3(64 * D2_WAVES), 0, stream, c_act, w2, s2,
                       hdr, perm_tok, perm_w, T, out);
  return hipGetLastError();
}

hipError_t launch_gemm1_prefill(const uint8_t* hidden, const float* hscale, int T, const uint8_t* w13,
                               const float* s13, const DispatchHeader* hdr, const int32_t* perm_tok,
                               uint16_t* c_act, int grid, hipStream_t stream) {
  static PerDeviceOnce<hipError_t> once;
  hipError_t e = hipErrorInvalidDevice;
  once.get([] { return hipFuncSetAttribute(reinterpret_cast<const void*>(gemm1_prefill_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, P1_LDS); },
           e);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(gemm1_prefill_kernel, dim3(grid), dim3(P1_THREADS), P1_LDS, stream, hidden, hscale, T, w13,
                     s13, hdr, perm_tok, c_act);
  return hipGetLastError();
}

hipError_t launch_gemm2_loader(const uint16_t* c_act, const uint8_t* w2, const float* s2, const DispatchHeader* hdr,
                               const float* perm_w, uint16_t* partial, int grid, hipStream_t stream) {
  static PerDeviceOnce<hipError_t> once;
  hipError_t e = hipErrorInvalidDevice;
  once.get([] { return hipFuncSetAttribute(reinterpret_cast<const void*>(gemm2_loader_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 2 * W2_STAGE); },
           e);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(gemm2_loader_kernel, dim3(grid), dim3(W2_THREADS), 2 * W2_STAGE, stream, c_act, w2, s2, hdr,
                     perm_w, partial);
  return hipGetLastError();
}

hipError_t launch_combine(const uint16_t* partial, const int32_t* tok_pair, int T, uint16_t* out, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(combine_kernel, dim3(T, H / COMBINE_COLS), dim3(COMBINE_THREADS), 0, stream, partial, tok_pair, T,
                     out);
  return hipGetLastError();
}

}  // namespace moe

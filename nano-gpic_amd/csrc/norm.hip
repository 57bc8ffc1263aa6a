// The producer of the FP8 linears' activations at an image block's two norm sites, with the e4m3 cast folded in
// (baselines/PixelGen/src/models/layers/fused_norm.py:64-91, JiT_T2I.py:203-206):
//
//   site 1:  h = RMSNorm(x) * (1 + scale) + shift
//   site 2:  x_new = x + gate * a;  h = RMSNorm(x_new) * (1 + scale) + shift
//
// and then h's tensorwise current-amax e4m3 bytes and dequantization scale (the tcast rule, fp8_native.py:33-49), so
// that the linear that consumes h reads 1 byte per element and h itself never has to exist in bf16 (it may be written
// as well, for a caller that wants it). x_new and the per-row 1 / rms (rstd) are written for the backward.
//
// The arithmetic, row by row, in fp32; fma() is one fused multiply-add (one rounding, as Triton compiles the
// reference's a * b + c on the GPU), every other operation rounds on its own (-ffp-contract=off):
//   xb = bf16(fma(gate, a, x))                  (site 2; site 1: xb = x)
//   ss: lane l of the row's wave accumulates ss = fma(xb, xb, ss) over its elements 4 (l + 64 j) + e < C in the
//       order j, e, then the 64 lane sums are combined by the butterfly v += v[lane ^ o], o = 32, 16, 8, 4, 2, 1
// Rows are C % 4 == 0 elements wide: a lane's group j of 4 elements is either wholly in the row or wholly past its end
// (the last group of a row whose C is not a multiple of 256 covers lanes 0 .. (C % 256) / 4 - 1 only).
//   rstd = 1 / sqrt(ss / C + eps)               (IEEE division and square root)
//   n = bf16(w * (xb * rstd));  h = bf16(fma(n, 1 + scale, shift))
// The reference computes the same expression with Triton's reduction order and libdevice's rsqrt, whose last bits
// are the H100's: this build fixes the order above, which the CPU oracle restates bit for bit.
//
// Two designs, as for the casts: rows that fit the chip's registers (C <= 2048 and at most the single-pass capacity)
// take one launch -- each wave holds the bf16 h of its rows, the workgroups agree on the amax through the tagged
// partials of the cast workspace (gpic_once.h), and each casts from its registers; larger ones, and calls that want
// the bf16 h written as well, take two, the second recomputing h from the x_new (or x) and rstd the first wrote.
#include <algorithm>

#include "gpic_device.h"
#include "gpic_launch.h"
#include "gpic_once.h"

namespace gpic {

struct NormArgs {
  const uint16_t *x;      // [rows, C] bf16
  const uint16_t *a;      // [rows, C] bf16, or null (site 1)
  const uint16_t *gate;   // [B, C] bf16, row stride sg (site 2)
  const float *w;         // [C] fp32, the norm weight
  const uint16_t *shift;  // [B, C] bf16, row stride ssh
  const uint16_t *scale;  // [B, C] bf16, row stride ssc
  uint16_t *xn;           // [rows, C] bf16 x_new (site 2)
  uint16_t *h;            // [rows, C] bf16 h, or null
  float *rstd;            // [rows]
  uint8_t *hq;            // [rows, C] e4m3
  float *dequant;         // [1]
  int64_t rows, ntok, sg, ssh, ssc;
  int C;
  float eps;
};

__device__ __forceinline__ u32x2 ld8(const uint16_t *p) { return *reinterpret_cast<const u32x2 *>(p); }

// Rows whose width C is no multiple of 256 (kTail): a lane holds kJ = ceil(C / 256) groups and its last one may lie
// past the row's end. Such a group loads the row's first group instead (in bounds, the address a per-lane offset from
// the row's base like every other group's) and takes zeros in place of what it read: zeros add exactly nothing to a
// row's sum of squares and give h = 0 (no effect on the maximum), so only the stores need the predicate. Without
// kTail these are the plain loads.
template <int kJ, bool kTail>
__device__ __forceinline__ bool grp_on(int lane, int j, int C) {
  return !kTail || j + 1 < kJ || 4 * (lane + 64 * j) < C;
}
template <int kJ, bool kTail>
__device__ __forceinline__ uint32_t grp_off(int lane, int j, int C) {
  const uint32_t c = 4u * (uint32_t)(lane + 64 * j);
  return grp_on<kJ, kTail>(lane, j, C) ? c : 0u;
}
template <int kJ, bool kTail>
__device__ __forceinline__ u32x2 ld8_grp(const uint16_t *p, int lane, int j, int C) {
  const u32x2 v = ld8(p + grp_off<kJ, kTail>(lane, j, C));
  return grp_on<kJ, kTail>(lane, j, C) ? v : u32x2{0u, 0u};
}
template <int kJ, bool kTail>
__device__ __forceinline__ float4 ld16f_grp(const float *p, int lane, int j, int C) {
  const float4 v = *reinterpret_cast<const float4 *>(p + grp_off<kJ, kTail>(lane, j, C));
  return grp_on<kJ, kTail>(lane, j, C) ? v : float4{0.0f, 0.0f, 0.0f, 0.0f};
}

// No memory access and no instruction moves across this point, neither in the compiler's IR nor in its machine
// scheduler: keeps loads in the phase they belong to (hoisted loads hold registers from the top of the kernel).
__device__ __forceinline__ void phase_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// The four fp32 values of a group's 8 bytes of bf16.
__device__ __forceinline__ void unpack4(u32x2 v, float (&f)[4]) {
  f[0] = bf16_lo(v.x), f[1] = bf16_hi(v.x), f[2] = bf16_lo(v.y), f[3] = bf16_hi(v.y);
}

// x_new = bf16(x + gate * a) of four elements, the product and sum fused (one rounding, as the reference's Triton
// kernel compiles x + g * a), packed.
__device__ __forceinline__ u32x2 xnew_packed(const float (&x)[4], const float (&g)[4], const float (&a)[4]) {
  return u32x2{pack_bf16(__builtin_fmaf(g[0], a[0], x[0]), __builtin_fmaf(g[1], a[1], x[1])),
               pack_bf16(__builtin_fmaf(g[2], a[2], x[2]), __builtin_fmaf(g[3], a[3], x[3]))};
}

// h of four elements, packed bf16 (and in hv before its rounding): n = bf16(w * (x * rstd));
// h = bf16(n * (1 + scale) + shift) with the multiply-add fused.
__device__ __forceinline__ u32x2 h_packed(const float (&x)[4], const float (&w)[4], float rstd, const float (&sc)[4],
                                          const float (&sh)[4], float (&hv)[4]) {
  const u32x2 nw{pack_bf16(w[0] * (x[0] * rstd), w[1] * (x[1] * rstd)),
                 pack_bf16(w[2] * (x[2] * rstd), w[3] * (x[3] * rstd))};
  float n[4];
  unpack4(nw, n);
#pragma unroll
  for (int e = 0; e < 4; e++) hv[e] = __builtin_fmaf(n[e], 1.0f + sc[e], sh[e]);
  return u32x2{pack_bf16(hv[0], hv[1]), pack_bf16(hv[2], hv[3])};
}

__device__ __forceinline__ float wave_sum_butterfly(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

// One row's h (this lane's groups j < J: elements 4 (lane + 64 j) .. + 3) as packed bf16 in H, and its amax bits
// (NaN excluded). kStore: write x_new (site 2), rstd (lane 0) and h (when p.h) as well. The groups are handled with a
// compile-time count when kJ > 0 (held in registers) or a run-time count ceil(C / 256) otherwise (then H is not
// kept); a group past the row's end is skipped.
template <int kJ, bool kStore>
__device__ __forceinline__ uint32_t norm_row(const NormArgs &p, int64_t row, u32x2 *H) {
  const int lane = threadIdx.x & 63;
  const int J = kJ > 0 ? kJ : (p.C + 255) / 256;
  const int64_t b = row / p.ntok;
  const uint16_t *xr = p.x + row * p.C;
  float ss = 0.0f;
  for (int j = 0; j < J; j++) {   // pass over the row: x_new and the sum of squares
    const int c = 4 * (lane + 64 * j);
    if (c >= p.C) break;           // (this lane's groups past the row's end)
    float x[4];
    unpack4(ld8(xr + c), x);
    if (p.a) {
      float av[4], gv[4];
      unpack4(ld8(p.a + row * p.C + c), av);
      unpack4(ld8(p.gate + b * p.sg + c), gv);
      const u32x2 xb = xnew_packed(x, gv, av);
      unpack4(xb, x);
      if (kStore) *reinterpret_cast<u32x2 *>(p.xn + row * p.C + c) = xb;
    }
#pragma unroll
    for (int e = 0; e < 4; e++) ss = __builtin_fmaf(x[e], x[e], ss);
  }
  ss = wave_sum_butterfly(ss);
  // (__builtin_sqrtf is the correctly rounded square root; HIP's __fsqrt_rn maps to the hardware approximation)
  const float rstd = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(ss, (float)p.C) + p.eps));
  if (kStore && lane == 0) p.rstd[row] = rstd;
  uint32_t m = 0;
  for (int j = 0; j < J; j++) {   // h, from x_new as rounded (re-read from the cache for site 2)
    const int c = 4 * (lane + 64 * j);
    if (c >= p.C) break;
    float x[4], sh[4], sc[4];
    if (p.a) {
      float av[4], gv[4];
      unpack4(ld8(xr + c), x);
      unpack4(ld8(p.a + row * p.C + c), av);
      unpack4(ld8(p.gate + b * p.sg + c), gv);
      unpack4(xnew_packed(x, gv, av), x);
    } else {
      unpack4(ld8(xr + c), x);
    }
    const float4 wv = *reinterpret_cast<const float4 *>(p.w + c);
    unpack4(ld8(p.shift + b * p.ssh + c), sh);
    unpack4(ld8(p.scale + b * p.ssc + c), sc);
    const float w4[4] = {wv.x, wv.y, wv.z, wv.w};
    float hv[4];
    const u32x2 hw = h_packed(x, w4, rstd, sc, sh, hv);
    m = max(m, max(bf16x2_absmax_nonan(hw.x), bf16x2_absmax_nonan(hw.y)));
    if (kJ > 0) H[j] = hw;
    if (kStore && p.h) *reinterpret_cast<u32x2 *>(p.h + row * p.C + c) = hw;
  }
  return m << 16;
}

// The same h recomputed from what the first pass stored: x_new (site 2) or x, and rstd -- the same bits.
__device__ __forceinline__ u32x2 h_from_stats(const NormArgs &p, int64_t row, int64_t b, float rstd, int c) {
  float x[4], sh[4], sc[4];
  unpack4(ld8((p.a ? p.xn : p.x) + row * p.C + c), x);
  const float4 wv = *reinterpret_cast<const float4 *>(p.w + c);
  unpack4(ld8(p.shift + b * p.ssh + c), sh);
  unpack4(ld8(p.scale + b * p.ssc + c), sc);
  const float w4[4] = {wv.x, wv.y, wv.z, wv.w};
  float hv[4];
  return h_packed(x, w4, rstd, sc, sh, hv);
}

__device__ __forceinline__ uint32_t cast4_packed(u32x2 hw, float s) {
  return e4m3x4(sat(bf16_lo(hw.x) * s), sat(bf16_hi(hw.x) * s), sat(bf16_lo(hw.y) * s), sat(bf16_hi(hw.y) * s));
}

// A wave's kR consecutive rows from row0 (kJ groups of 4 per lane each) through the norm: x_new (site 2) and rstd
// written, h left as packed bf16 in X, and the largest |h| returned (fp32, before h's rounding; NaN ignored). The rows
// go through each phase together, so that one memory latency covers all of them: every row's x is requested first,
// then (site 2) a and gate are folded in, the kR butterflies run interleaved, and w, shift and scale are read once
// per group and used for all the rows; h replaces x in the same registers. Rows past the end re-read the last row
// (same values, so the same maximum) and store nothing. kUni: every row of a wave lies in one batch (ntok % kR ==
// 0), so gate, shift and scale are one vector per wave. row0 must be wave-uniform (a scalar: the rows' addresses are
// then scalar bases plus one per-lane offset).
template <int kJ, int kR, bool kUni, bool kRes, bool kTail>
__device__ __forceinline__ float norm_rows(const NormArgs &p, int64_t row0, int lane, u32x2 (&X)[kR][kJ]) {
  const int64_t C = p.C;
  auto rowi = [&](int r) { return min(row0 + r, p.rows - 1); };
  auto bat = [&](int r) { return (kUni ? rowi(0) : rowi(r)) / p.ntok; };   // (a wave past the end: the last batch)
#pragma unroll
  for (int r = 0; r < kR; r++)
#pragma unroll
    for (int j = 0; j < kJ; j++) X[r][j] = ld8_grp<kJ, kTail>(p.x + rowi(r) * C, lane, j, p.C);
  const int nr = (int)min<int64_t>(max<int64_t>(p.rows - row0, 0), kR);   // rows of this wave that exist
  // site 2: a (and, per row unless kUni, gate) through a ring of kD rows: the loads of row r + kD - 1 are issued
  // before row r is used, and the fences keep the compiler from hoisting every row's loads to the top (x and a of
  // all rows at once would not fit the registers)
  constexpr int kD = 3;
  u32x2 A[kD][kJ], Gt[kD][kJ], G0[kJ];
  auto load_a = [&](int r) {
#pragma unroll
    for (int j = 0; j < kJ; j++) {
      A[r % kD][j] = ld8_grp<kJ, kTail>(p.a + rowi(r) * C, lane, j, p.C);
      if (!kUni) Gt[r % kD][j] = ld8_grp<kJ, kTail>(p.gate + bat(r) * p.sg, lane, j, p.C);
    }
  };
  if (kRes) {
    if (kUni) {
#pragma unroll
      for (int j = 0; j < kJ; j++) G0[j] = ld8_grp<kJ, kTail>(p.gate + bat(0) * p.sg, lane, j, p.C);
    }
#pragma unroll
    for (int r = 0; r < kD - 1 && r < kR; r++) load_a(r);
  }
  // phase 1: x_new (site 2) and each lane's sum of squares, row by row as the rows come in
  float S[kR];
#pragma unroll
  for (int r = 0; r < kR; r++) {
    S[r] = 0.0f;
    if (kRes) {
      if (r + kD - 1 < kR) load_a(r + kD - 1);
      phase_fence();
    }
#pragma unroll
    for (int j = 0; j < kJ; j++) {
      float x[4];
      unpack4(X[r][j], x);
      if (kRes) {
        float av[4], gv[4];
        unpack4(A[r % kD][j], av);
        unpack4(kUni ? G0[j] : Gt[r % kD][j], gv);
        X[r][j] = xnew_packed(x, gv, av);
        unpack4(X[r][j], x);
      }
#pragma unroll
      for (int e = 0; e < 4; e++) S[r] = __builtin_fmaf(x[e], x[e], S[r]);
    }
    // row r's results are made here, before the next row's fence (the compiler would otherwise sink the arithmetic
    // to its uses and keep every row's a live); the packed words are then the only copy of the row (else phase 1's
    // unpacked fp32 values are reused in phase 3 and the registers double)
#pragma unroll
    for (int j = 0; j < kJ; j++) asm volatile("" : "+v"(X[r][j]));
    asm volatile("" : "+v"(S[r]));
    if (kRes && r < nr) {
#pragma unroll
      for (int j = 0; j < kJ; j++)
        if (grp_on<kJ, kTail>(lane, j, p.C)) *reinterpret_cast<u32x2 *>(p.xn + (row0 + r) * C + 4 * (lane + 64 * j)) = X[r][j];
    }
  }
  // phase 2: the kR butterflies interleaved, rstd
#pragma unroll
  for (int o = 32; o > 0; o >>= 1)
#pragma unroll
    for (int r = 0; r < kR; r++) S[r] = S[r] + __shfl_xor(S[r], o, 64);
  phase_fence();   // w, shift and scale are read below, not hoisted to the top beside the rows
  float rs[kR];
#pragma unroll
  for (int r = 0; r < kR; r++) {
    rs[r] = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(S[r], (float)p.C) + p.eps));
    if (lane == r && r < nr) p.rstd[row0 + r] = rs[r];
  }
  // phase 3: h in place of x, and the largest |h|. Its loads of w, shift and scale come after every row's x (the
  // vector memory counter is in order), so this phase starts once all the rows are in: the reason the rows are not
  // taken in smaller batches.
  float mf = 0.0f;
#pragma unroll
  for (int j = 0; j < kJ; j++) {
    const float4 wv = ld16f_grp<kJ, kTail>(p.w, lane, j, p.C);
    const float w4[4] = {wv.x, wv.y, wv.z, wv.w};
    float sh[4], sc[4];
    if (kUni) {
      unpack4(ld8_grp<kJ, kTail>(p.shift + bat(0) * p.ssh, lane, j, p.C), sh);
      unpack4(ld8_grp<kJ, kTail>(p.scale + bat(0) * p.ssc, lane, j, p.C), sc);
    }
#pragma unroll
    for (int r = 0; r < kR; r++) {
      if (!kUni) {
        unpack4(ld8_grp<kJ, kTail>(p.shift + bat(r) * p.ssh, lane, j, p.C), sh);
        unpack4(ld8_grp<kJ, kTail>(p.scale + bat(r) * p.ssc, lane, j, p.C), sc);
      }
      float x[4], hv[4];
      unpack4(X[r][j], x);
      X[r][j] = h_packed(x, w4, rs[r], sc, sh, hv);
      // the largest |h| in fp32, NaN ignored (maxNum); rounded to bf16 at the end, it is the largest |bf16 h|
      // (rounding is monotonic), in one instruction per element instead of a compare and select on the halves
#pragma unroll
      for (int e = 0; e < 4; e++) mf = fmaxf(mf, fabsf(hv[e]));
    }
  }
  // h is made here and kept only as packed words (the compiler would otherwise carry phase 3's fp32 values into
  // the caller's fold and stores)
#pragma unroll
  for (int r = 0; r < kR; r++)
#pragma unroll
    for (int j = 0; j < kJ; j++) asm volatile("" : "+v"(X[r][j]));
  phase_fence();
  return mf;
}

// Single pass: wave w of workgroup g takes rows (4 g + w) kR .. + kR - 1 through norm_rows, the workgroups fold their
// maxima (gpic_once.h), and each casts its rows from its registers.
template <int kJ, int kR, bool kUni, bool kRes, bool kTail>
__global__ __launch_bounds__(256, 4) void norm_q_once_kernel(NormArgs p, void *ws, uint32_t wait_ticks) {
  const uint32_t ep = once_epoch(ws);   // (before the first loads: its latency passes behind them)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * kR;
  const int64_t C = p.C;
  const int nr = (int)min<int64_t>(max<int64_t>(p.rows - row0, 0), kR);   // rows of this wave that exist
  u32x2 X[kR][kJ];
  const float mf = norm_rows<kJ, kR, kUni, kRes, kTail>(p, row0, lane, X);
  uint32_t tk;
  const uint32_t g = once_fold(block_max_u32(__float_as_uint(bf16_round(mf))), ws, ep, wait_ticks, tk, [&](int cb) {
    // workgroup cb's maximum from its rows (nothing stored): for a partial that did not appear in time
    uint32_t v = 0;
    for (int r = 0; r < kR; r++) {
      const int64_t row = ((int64_t)cb * 4 + wave) * kR + r;
      if (row < p.rows) v = max(v, norm_row<0, false>(p, row, nullptr));
    }
    return block_max_u32(v);
  });
  float scale, deq;
  scales_from_amax(g, scale, deq);
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.dequant = deq;
#pragma unroll
  for (int r = 0; r < kR; r++)
    if (r < nr) {
#pragma unroll
      for (int j = 0; j < kJ; j++)
        if (grp_on<kJ, kTail>(lane, j, p.C))
          __builtin_nontemporal_store(cast4_packed(X[r][j], scale),
                                      reinterpret_cast<uint32_t *>(p.hq + (row0 + r) * C + 4 * (lane + 64 * j)));
    }
  once_done(ws, tk);
}

// Two passes, 1 (rows of at most 2048): workgroup g takes the groups of 4 kR rows g, g + G, ... through norm_rows,
// writes h when asked, and leaves the largest |h| of its rows in partial[g] (float bits of the bf16 value).
// (Two workgroups per CU and 256 registers a lane: it loops over its groups, so it needs no more residency than that,
// and the loop keeps more live than the single pass.) kH: write h.
template <int kJ, int kR, bool kUni, bool kRes, bool kH, bool kTail>
__global__ __launch_bounds__(256, 2) void norm_rows_kernel(NormArgs p, uint32_t *__restrict__ partial, int64_t groups) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t C = p.C;
  float mf = 0.0f;
  for (int64_t g = blockIdx.x; g < groups; g += gridDim.x) {
    const int64_t row0 = (g * 4 + wave) * kR;
    const int nr = (int)min<int64_t>(max<int64_t>(p.rows - row0, 0), kR);
    u32x2 X[kR][kJ];
    mf = fmaxf(mf, norm_rows<kJ, kR, kUni, kRes, kTail>(p, row0, lane, X));
    if (kH) {
#pragma unroll
      for (int r = 0; r < kR; r++)
        if (r < nr) {
#pragma unroll
          for (int j = 0; j < kJ; j++)
            if (grp_on<kJ, kTail>(lane, j, p.C)) *reinterpret_cast<u32x2 *>(p.h + (row0 + r) * C + 4 * (lane + 64 * j)) = X[r][j];
        }
    }
  }
  const uint32_t m = block_max_u32(__float_as_uint(bf16_round(mf)));
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// Two passes, 1: rows strided over the waves of the grid; x_new, rstd (and h) written, one partial maximum per
// workgroup in partial[blockIdx.x].
__global__ __launch_bounds__(256) void norm_stats_kernel(NormArgs p, uint32_t *__restrict__ partial) {
  const int64_t nw = (int64_t)gridDim.x * 4;
  uint32_t m = 0;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < p.rows; row += nw)
    m = max(m, norm_row<0, true>(p, row, nullptr));
  m = block_max_u32(m);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// Two passes, 2: the scale from the first pass's partials; h recomputed from x_new (or x) and rstd and cast.
__global__ __launch_bounds__(256) void norm_cast_kernel(NormArgs p, const uint32_t *__restrict__ partial, int nparts) {
  uint32_t m = 0;
  for (int i = threadIdx.x; i < nparts; i += 256) m = max(m, partial[i]);
  m = block_max_u32(m);
  float scale, deq;
  scales_from_amax(m, scale, deq);
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.dequant = deq;
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * 4;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < p.rows; row += nw) {
    const int64_t b = row / p.ntok;
    const float rstd = p.rstd[row];
    for (int j = 0; j < (p.C + 255) / 256; j++) {
      const int c = 4 * (lane + 64 * j);
      if (c >= p.C) break;
      __builtin_nontemporal_store(cast4_packed(h_from_stats(p, row, b, rstd, c), scale),
                                  reinterpret_cast<uint32_t *>(p.hq + row * p.C + c));
    }
  }
}

// ------------------------------------------------------------------------------------------- host side

static DeviceCache g_cap_norm[9][2][2][2];   // [kJ][kUni][kRes][kTail]
struct NormCacheInit {
  NormCacheInit() {
    for (auto &cj : g_cap_norm)
      for (auto &cu : cj)
        for (auto &cr : cu)
          for (auto &c : cr)
            for (int i = 0; i < kMaxDevices; i++) c[i] = -1;
  }
};
static NormCacheInit g_norm_cache_init;

// Rows per wave held by the single pass: kJ groups of 4 bf16 (kJ * 2 VGPRs) per row, at most 64 VGPRs in all (at
// most 10 rows: more spilled for the narrow rows, whose per-row state then dominates).
template <int kJ>
constexpr int kRowsOnce = kJ >= 3 ? 32 / kJ : 10;

template <int kJ, bool kUni, bool kRes, bool kTail>
static bool launch_norm_once_t(const NormArgs &p, void *ws, hipStream_t st) {
  constexpr int kR = kRowsOnce<kJ>;
  const int cap = once_capacity(reinterpret_cast<const void *>(&norm_q_once_kernel<kJ, kR, kUni, kRes, kTail>),
                                g_cap_norm[kJ][kUni][kRes][kTail], 256);
  const int64_t wgs = (p.rows + 4 * kR - 1) / (4 * kR);
  if (cap <= 0 || wgs > cap) return false;
  norm_q_once_kernel<kJ, kR, kUni, kRes, kTail><<<(int)wgs, 256, 0, st>>>(p, ws, once_wait_ticks());
  return true;
}

// The first of the two passes for rows of at most 2048: one partial maximum per workgroup in `partial` (at most
// kMaxParts workgroups, each taking every G-th group of 4 kR rows). Returns the number of partials.
template <int kJ, bool kUni, bool kRes, bool kTail>
static int launch_norm_rows_t(const NormArgs &p, uint32_t *partial, hipStream_t st) {
  constexpr int kR = kRowsOnce<kJ>;
  const int64_t groups = (p.rows + 4 * kR - 1) / (4 * kR);
  const int g = (int)std::min<int64_t>(groups, kMaxParts);
  if (p.h) norm_rows_kernel<kJ, kR, kUni, kRes, true, kTail><<<g, 256, 0, st>>>(p, partial, groups);
  else norm_rows_kernel<kJ, kR, kUni, kRes, false, kTail><<<g, 256, 0, st>>>(p, partial, groups);
  return g;
}

template <int kJ, bool kTail>
static int launch_norm_rows_w(const NormArgs &p, uint32_t *partial, hipStream_t st) {
  const bool uni = p.ntok % kRowsOnce<kJ> == 0;
  if (p.a)
    return uni ? launch_norm_rows_t<kJ, true, true, kTail>(p, partial, st)
               : launch_norm_rows_t<kJ, false, true, kTail>(p, partial, st);
  return uni ? launch_norm_rows_t<kJ, true, false, kTail>(p, partial, st)
             : launch_norm_rows_t<kJ, false, false, kTail>(p, partial, st);
}

// kJ = ceil(C / 256) groups per lane; rows with C % 256 != 0 take the instances with the partial last group.
template <int kJ>
static int launch_norm_rows(const NormArgs &p, uint32_t *partial, hipStream_t st) {
  return p.C % 256 ? launch_norm_rows_w<kJ, true>(p, partial, st) : launch_norm_rows_w<kJ, false>(p, partial, st);
}

// Pass 1 of the two passes: the multi-row kernel for rows of at most 2048, else the row-at-a-time one. Returns the
// number of partial maxima written to `partial`.
static int norm_first_pass(const NormArgs &p, uint32_t *partial, hipStream_t st) {
  switch ((p.C + 255) / 256) {
    case 1: return launch_norm_rows<1>(p, partial, st);
    case 2: return launch_norm_rows<2>(p, partial, st);
    case 3: return launch_norm_rows<3>(p, partial, st);
    case 4: return launch_norm_rows<4>(p, partial, st);
    case 5: return launch_norm_rows<5>(p, partial, st);
    case 6: return launch_norm_rows<6>(p, partial, st);
    case 7: return launch_norm_rows<7>(p, partial, st);
    case 8: return launch_norm_rows<8>(p, partial, st);
    default: {
      const int g = (int)std::min<int64_t>((p.rows + 3) / 4, kMaxParts);
      norm_stats_kernel<<<g, 256, 0, st>>>(p, partial);
      return g;
    }
  }
}

template <int kJ, bool kTail>
static bool launch_norm_once_w(const NormArgs &p, void *ws, hipStream_t st) {
  const bool uni = p.ntok % kRowsOnce<kJ> == 0;
  if (p.a)
    return uni ? launch_norm_once_t<kJ, true, true, kTail>(p, ws, st) : launch_norm_once_t<kJ, false, true, kTail>(p, ws, st);
  return uni ? launch_norm_once_t<kJ, true, false, kTail>(p, ws, st) : launch_norm_once_t<kJ, false, false, kTail>(p, ws, st);
}

template <int kJ>
static bool launch_norm_once(const NormArgs &p, void *ws, hipStream_t st) {
  if (!once_enabled() || p.h) return false;   // (bf16 h as well: the two passes)
  return p.C % 256 ? launch_norm_once_w<kJ, true>(p, ws, st) : launch_norm_once_w<kJ, false>(p, ws, st);
}


// ------------------------------------------------------------------------------------------- backward

// The norm sites' backward (fused_norm.py:94-147): for each row, with t = xs * rstd (xs = x_new at site 2, x at
// site 1), n = bf16(w t), dn = dh (1 + scale), dt = dn w, mean = sum(dt t) / C:
//   dx = rstd (dt - t mean) (+ dxn at site 2)   -> bf16 dx;   site 2: da = bf16(dx gate)
// and the column sums d_shift[b] = sum dh, d_scale[b] = sum dh n, d_gate[b] = sum dx a (over the rows of batch b),
// d_w = sum dn t (over all rows), in fp32. A workgroup takes kBwdRows consecutive rows of one batch, one wave per row
// (lane l: elements 4 (l + 64 j) + e, as the forward); each wave keeps its column sums in registers, the four waves
// add theirs in LDS in wave order, and the workgroup writes one partial row per sum; norm_bwd_reduce_kernel then adds
// the partials in workgroup order. Every sum has a fixed order: the gradients are deterministic.
constexpr int kBwdRows = 64;   // rows per workgroup (16 per wave)

struct NormBwdArgs {
  const uint16_t *dh, *dxn, *xs, *a, *gate;   // dxn, a, gate: site 2 only (else null)
  const float *w;
  const uint16_t *scale;
  const float *rstd;
  uint16_t *dx, *da;
  float *part;                                // [4][P][C]: shift, scale, w, gate partials
  int64_t rows, ntok, sg, ssc;
  int C, tiles_b, P;
};

template <int kJ, bool kRes, bool kDxn, bool kTail>
__global__ __launch_bounds__(256, 2) void norm_bwd_kernel(NormBwdArgs p) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pid = blockIdx.x;
  const int64_t b = pid / p.tiles_b, tile = pid % p.tiles_b;
  const int64_t r0 = tile * kBwdRows, rend = min<int64_t>(p.ntok, r0 + kBwdRows);   // token range in batch b
  const int64_t C = p.C;
  // the columns' w (fp32) and scale, gate (packed bf16: fewer registers, unpacked where used)
  float w4[kJ][4];
  u32x2 SC[kJ], GT[kJ];
#pragma unroll
  for (int j = 0; j < kJ; j++) {
    const float4 wv = ld16f_grp<kJ, kTail>(p.w, lane, j, p.C);
    w4[j][0] = wv.x, w4[j][1] = wv.y, w4[j][2] = wv.z, w4[j][3] = wv.w;
    SC[j] = ld8_grp<kJ, kTail>(p.scale + b * p.ssc, lane, j, p.C);
    if (kRes) GT[j] = ld8_grp<kJ, kTail>(p.gate + b * p.sg, lane, j, p.C);
  }
  float ash[kJ][4], asc[kJ][4], aw[kJ][4], ag[kJ][4];
#pragma unroll
  for (int j = 0; j < kJ; j++)
#pragma unroll
    for (int e = 0; e < 4; e++) ash[j][e] = asc[j][e] = aw[j][e] = ag[j][e] = 0.0f;
  // A row's loads (packed bf16), issued one row ahead: the next row's are in flight while this one is computed.
  // A group past the row's end (the last one, when C % 256 != 0) loads nothing and takes zeros: every sum and the
  // row's mean then receive exactly zero from it (its dx and da are not stored).
  constexpr int kPre = kJ <= 4 ? 1 : 0;
  u32x2 DH[2][kJ], XS[2][kJ], AV[2][kJ], DX[2][kJ];
  auto load_row = [&](int buf, int64_t r) {
    const int64_t row = b * p.ntok + r;
#pragma unroll
    for (int j = 0; j < kJ; j++) {
      DH[buf][j] = ld8_grp<kJ, kTail>(p.dh + row * C, lane, j, p.C);
      XS[buf][j] = ld8_grp<kJ, kTail>(p.xs + row * C, lane, j, p.C);
      if (kRes) AV[buf][j] = ld8_grp<kJ, kTail>(p.a + row * C, lane, j, p.C);
      if (kDxn) DX[buf][j] = ld8_grp<kJ, kTail>(p.dxn + row * C, lane, j, p.C);
    }
  };
  auto do_row = [&](int buf, int64_t r) {
    // (scale and gate stay packed: the compiler would otherwise unpack them once, out of the row loop, into twice the
    // registers)
#pragma unroll
    for (int j = 0; j < kJ; j++) {
      asm volatile("" : "+v"(SC[j]));
      if (kRes) asm volatile("" : "+v"(GT[j]));
    }
    const int64_t row = b * p.ntok + r;
    const float rs = p.rstd[row];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kJ; j++) {
      float dh[4], x[4], sc[4];
      unpack4(DH[buf][j], dh);
      unpack4(XS[buf][j], x);
      unpack4(SC[j], sc);
      const u32x2 nw{pack_bf16(w4[j][0] * (x[0] * rs), w4[j][1] * (x[1] * rs)),
                     pack_bf16(w4[j][2] * (x[2] * rs), w4[j][3] * (x[3] * rs))};
      float n[4];
      unpack4(nw, n);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float t = x[e] * rs;
        ash[j][e] = ash[j][e] + dh[e];
        asc[j][e] = __builtin_fmaf(dh[e], n[e], asc[j][e]);
        const float dn = dh[e] * (1.0f + sc[e]);
        aw[j][e] = __builtin_fmaf(dn, t, aw[j][e]);
        s = __builtin_fmaf(dn * w4[j][e], t, s);
      }
    }
    const float mean = __fdiv_rn(wave_sum_butterfly(s), (float)p.C);
#pragma unroll
    for (int j = 0; j < kJ; j++) {   // t and dt again from the packed row (fewer registers than keeping them)
      const int c = 4 * (lane + 64 * j);
      const bool on = grp_on<kJ, kTail>(lane, j, p.C);
      float dh[4], x[4], sc[4], dx[4];
      unpack4(DH[buf][j], dh);
      unpack4(XS[buf][j], x);
      unpack4(SC[j], sc);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float t = x[e] * rs;
        const float dt = (dh[e] * (1.0f + sc[e])) * w4[j][e];
        dx[e] = rs * (dt - t * mean);
      }
      if (kDxn) {
        float d[4];
        unpack4(DX[buf][j], d);
#pragma unroll
        for (int e = 0; e < 4; e++) dx[e] = dx[e] + d[e];
      }
      if (kRes) {
        float av[4], g[4];
        unpack4(AV[buf][j], av);
        unpack4(GT[j], g);
#pragma unroll
        for (int e = 0; e < 4; e++) ag[j][e] = __builtin_fmaf(dx[e], av[e], ag[j][e]);
        if (on)
          *reinterpret_cast<u32x2 *>(p.da + row * C + c) =
              u32x2{pack_bf16(dx[0] * g[0], dx[1] * g[1]), pack_bf16(dx[2] * g[2], dx[3] * g[3])};
      }
      if (on) *reinterpret_cast<u32x2 *>(p.dx + row * C + c) = u32x2{pack_bf16(dx[0], dx[1]), pack_bf16(dx[2], dx[3])};
    }
  };
  int64_t r = r0 + wave;
  if (kPre) {
    if (r < rend) load_row(0, r);
    for (; r < rend; r += 8) {   // rows r (buffer 0) and r + 4 (buffer 1)
      if (r + 4 < rend) load_row(1, r + 4);
      do_row(0, r);
      if (r + 4 >= rend) break;
      if (r + 8 < rend) load_row(0, r + 8);
      do_row(1, r + 4);
    }
  } else {
    for (; r < rend; r += 4) {
      load_row(0, r);
      do_row(0, r);
    }
  }
  // the four waves' column sums added in LDS in wave order, then one partial row per sum
  extern __shared__ float red[];   // [4 waves][kNS sums][C]
  constexpr int kNS = kRes ? 4 : 3;
#pragma unroll
  for (int j = 0; j < kJ; j++) {
    const int c = 4 * (lane + 64 * j);
    if (!grp_on<kJ, kTail>(lane, j, p.C)) continue;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      red[(wave * kNS + 0) * C + c + e] = ash[j][e];
      red[(wave * kNS + 1) * C + c + e] = asc[j][e];
      red[(wave * kNS + 2) * C + c + e] = aw[j][e];
      if (kRes) red[(wave * kNS + 3) * C + c + e] = ag[j][e];
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kNS * C; i += 256) {
    const int k = i / (int)C, c = i % (int)C;
    float v = red[(0 * kNS + k) * C + c];
#pragma unroll
    for (int wv = 1; wv < 4; wv++) v = v + red[(wv * kNS + k) * C + c];
    p.part[((int64_t)k * p.P + pid) * C + c] = v;
  }
}

// The partials added in a fixed order. Workgroups [0, nbc): d_shift, d_scale, d_gate [B, C] over the tiles of each
// batch, one thread per (batch, column). The next ceil(C / 16) workgroups: d_w [C] over all P partials, 16 columns
// per workgroup: thread (k, c) adds partials [k P / 16, (k + 1) P / 16) of column c, then the 16 chunk sums of a
// column are added in chunk order (a single thread per column would wait on P dependent loads).
__global__ __launch_bounds__(256) void norm_bwd_reduce_kernel(const float *__restrict__ part, int P, int tiles_b, int B,
                                                              int C, bool res, float *__restrict__ dsh,
                                                              float *__restrict__ dsc, float *__restrict__ dg,
                                                              float *__restrict__ dw) {
  const int64_t nbc = (int64_t)B * C;
  const int64_t wg_bc = (nbc + 255) / 256;
  if (blockIdx.x < wg_bc) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nbc) return;
    const int64_t bb = i / C, c = i % C;
    float s0 = 0.0f, s1 = 0.0f, s3 = 0.0f;
    for (int t = 0; t < tiles_b; t++) {
      const int64_t prow = bb * tiles_b + t;
      s0 = s0 + part[(0 * (int64_t)P + prow) * C + c];
      s1 = s1 + part[(1 * (int64_t)P + prow) * C + c];
      if (res) s3 = s3 + part[(3 * (int64_t)P + prow) * C + c];
    }
    dsh[i] = s0;
    dsc[i] = s1;
    if (res) dg[i] = s3;
    return;
  }
  __shared__ float chunk[16][16];
  const int cl = threadIdx.x & 15, k = threadIdx.x >> 4;
  const int c = (int)(blockIdx.x - wg_bc) * 16 + cl;
  const int per = (P + 15) / 16, q0 = k * per, q1 = min(P, q0 + per);
  float sw = 0.0f;
  if (c < C) {
    const float *pw = part + 2 * (int64_t)P * C + c;
    int q = q0;
    for (; q + 8 <= q1; q += 8) {   // 8 loads in flight, added in order
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = pw[(int64_t)(q + u) * C];
#pragma unroll
      for (int u = 0; u < 8; u++) sw = sw + v[u];
    }
    for (; q < q1; q++) sw = sw + pw[(int64_t)q * C];
  }
  chunk[k][cl] = sw;
  __syncthreads();
  if (k == 0 && c < C) {
    float t = chunk[0][cl];
#pragma unroll
    for (int kk = 1; kk < 16; kk++) t = t + chunk[kk][cl];
    dw[c] = t;
  }
}

template <int kJ, bool kTail>
static void launch_norm_bwd_w(const NormBwdArgs &p, bool res, hipStream_t st) {
  const size_t lds = (size_t)4 * (res ? 4 : 3) * p.C * sizeof(float);
  if (!res) norm_bwd_kernel<kJ, false, false, kTail><<<p.P, 256, lds, st>>>(p);
  else if (p.dxn) norm_bwd_kernel<kJ, true, true, kTail><<<p.P, 256, lds, st>>>(p);
  else norm_bwd_kernel<kJ, true, false, kTail><<<p.P, 256, lds, st>>>(p);
}

template <int kJ>
static void launch_norm_bwd(const NormBwdArgs &p, bool res, hipStream_t st) {
  if (p.C % 256) launch_norm_bwd_w<kJ, true>(p, res, st);
  else launch_norm_bwd_w<kJ, false>(p, res, st);
}

static int64_t norm_bwd_parts(int64_t rows, int64_t ntok) {
  return ntok > 0 ? (rows / ntok) * ((ntok + kBwdRows - 1) / kBwdRows) : 0;
}
}  // namespace gpic

using namespace gpic;

extern "C" {

int gpic_fp8_res_mod_rmsnorm(const uint16_t *x, const uint16_t *a, const uint16_t *gate, int64_t sg, const float *w,
                             const uint16_t *shift, int64_t ssh, const uint16_t *scale, int64_t ssc, int64_t rows,
                             int64_t ntok, int64_t C, float eps, uint16_t *xn, uint16_t *h, float *rstd, uint8_t *hq,
                             float *dequant, void *ws, void *stream) {
  status_scope();
  const bool cast = dequant != nullptr;   // else the norm alone
  if (rows < 0 || C <= 0 || ntok <= 0 || !ws || !w || !shift || !scale) return GPIC_EINVAL;
  if (rows > 0 && (!x || !rstd || (cast ? !hq : !h) || (a && (!gate || !xn)))) return GPIC_EINVAL;
  if (C % 4 != 0 || rows % ntok != 0 || ssh % 4 != 0 || ssc % 4 != 0 || (a && sg % 4 != 0) || ssh < C || ssc < C ||
      (a && sg < C) || C > (1 << 20))
    return GPIC_ESHAPE;
  if (!aligned16(x) || (a && !aligned16(a)) || ((uintptr_t)gate & 7u) || !aligned16(w) || ((uintptr_t)shift & 7u) ||
      ((uintptr_t)scale & 7u) || (xn && !aligned16(xn)) || (h && !aligned16(h)) || (hq && !aligned16(hq)) ||
      !aligned16(ws))
    return GPIC_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  NormArgs p{x, a, gate, w, shift, scale, xn, h, rstd, hq, dequant, rows, ntok, sg, ssh, ssc, (int)C, eps};
  if (rows == 0) {   // nothing but the scale of an empty tensor: 1e-12 / 448
    if (cast) norm_cast_kernel<<<1, 256, 0, st>>>(p, static_cast<const uint32_t *>(ws), 0);
    return (int)hipGetLastError();
  }
  if (!cast) {   // the norm alone (h, x_new, rstd): the first pass of the two-pass path, its partial maxima unused
    norm_first_pass(p, static_cast<uint32_t *>(ws), st);
    return (int)hipGetLastError();
  }
  bool done = false;
  switch ((C + 255) / 256) {
    case 1: done = launch_norm_once<1>(p, ws, st); break;
    case 2: done = launch_norm_once<2>(p, ws, st); break;
    case 3: done = launch_norm_once<3>(p, ws, st); break;
    case 4: done = launch_norm_once<4>(p, ws, st); break;
    case 5: done = launch_norm_once<5>(p, ws, st); break;
    case 6: done = launch_norm_once<6>(p, ws, st); break;
    case 7: done = launch_norm_once<7>(p, ws, st); break;
    case 8: done = launch_norm_once<8>(p, ws, st); break;
    default: break;
  }
  if (done) return (int)hipGetLastError();
  uint32_t *partial = static_cast<uint32_t *>(ws);
  const int g1 = norm_first_pass(p, partial, st);
  const int g2 = (int)std::min<int64_t>((rows + 3) / 4, 2048);
  norm_cast_kernel<<<g2, 256, 0, st>>>(p, partial, g1);
  return (int)hipGetLastError();
}


size_t gpic_fp8_res_mod_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t ntok, int64_t C) {
  if (rows <= 0 || ntok <= 0 || C <= 0 || rows % ntok != 0) return 0;
  return (size_t)4 * norm_bwd_parts(rows, ntok) * C * sizeof(float);
}

int gpic_fp8_res_mod_rmsnorm_bwd(const uint16_t *dh, const uint16_t *dxn, const uint16_t *xs, const uint16_t *a,
                                 const uint16_t *gate, int64_t sg, const float *w, const uint16_t *scale, int64_t ssc,
                                 const float *rstd, int64_t rows, int64_t ntok, int64_t C, uint16_t *dx, uint16_t *da,
                                 float *dshift, float *dscale, float *dgate, float *dw, void *ws, size_t ws_bytes,
                                 void *stream) {
  status_scope();
  const bool res = a != nullptr;
  if (rows < 0 || C <= 0 || ntok <= 0 || !w || !scale || !dshift || !dscale || !dw || (res && (!gate || !dgate)))
    return GPIC_EINVAL;
  if (rows > 0 && (!dh || !xs || !rstd || !dx || (res && !da) || !ws)) return GPIC_EINVAL;
  if (!res && (dxn || dgate)) return GPIC_EINVAL;
  if (C % 4 != 0 || C > 2048 || rows % ntok != 0 || ssc % 4 != 0 || ssc < C || (res && (sg % 4 != 0 || sg < C)))
    return GPIC_ESHAPE;
  if (!aligned16(dh) || (dxn && !aligned16(dxn)) || !aligned16(xs) || (a && !aligned16(a)) || !aligned16(w) ||
      ((uintptr_t)scale & 7u) || ((uintptr_t)gate & 7u) || !aligned16(dx) || (da && !aligned16(da)) ||
      !aligned16(ws))
    return GPIC_EALIGN;
  const int64_t B = rows / ntok;
  hipStream_t st = (hipStream_t)stream;
  if (rows == 0) {   // no rows: d_w is zero (the reduce over no partials writes it; no memset, so a graph can hold it)
    norm_bwd_reduce_kernel<<<(int)((C + 15) / 16), 256, 0, st>>>(nullptr, 0, 0, 0, (int)C, res, dshift, dscale,
                                                                  dgate, dw);
    return (int)hipGetLastError();
  }
  const int64_t P = norm_bwd_parts(rows, ntok);
  if (ws_bytes < (size_t)4 * P * C * sizeof(float)) return GPIC_EWORKSPACE;
  if (P >= (int64_t(1) << 31) / 4 || B * C >= (int64_t(1) << 31)) return GPIC_ESHAPE;
  NormBwdArgs p{dh, dxn, xs, a, gate, w, scale, rstd, dx, da, static_cast<float *>(ws), rows, ntok, sg, ssc, (int)C,
                (int)((ntok + kBwdRows - 1) / kBwdRows), (int)P};
  switch ((C + 255) / 256) {
    case 1: launch_norm_bwd<1>(p, res, st); break;
    case 2: launch_norm_bwd<2>(p, res, st); break;
    case 3: launch_norm_bwd<3>(p, res, st); break;
    case 4: launch_norm_bwd<4>(p, res, st); break;
    case 5: launch_norm_bwd<5>(p, res, st); break;
    case 6: launch_norm_bwd<6>(p, res, st); break;
    case 7: launch_norm_bwd<7>(p, res, st); break;
    default: launch_norm_bwd<8>(p, res, st); break;
  }
  const int64_t grid = (B * C + 255) / 256 + (C + 15) / 16;
  norm_bwd_reduce_kernel<<<(int)grid, 256, 0, st>>>(static_cast<const float *>(ws), (int)P, p.tiles_b, (int)B, (int)C,
                                                     res, dshift, dscale, dgate, dw);
  return (int)hipGetLastError();
}

}  // extern "C"

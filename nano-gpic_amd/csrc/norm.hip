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
// The arithmetic, every fp32 operation rounded on its own (-ffp-contract=off), row by row:
//   xb = bf16(x + gate * a)                     (site 2; site 1: xb = x)
//   ss = sum of xb^2: lane l of the row's wave adds the squares of its elements 4 (l + 64 j) + e in the order j, e,
//        then the 64 lane sums are combined by the butterfly v += v[lane ^ o], o = 32, 16, 8, 4, 2, 1
//   rstd = 1 / sqrt(ss / C + eps)               (IEEE division and square root)
//   n = bf16(w * (xb * rstd));  h = bf16(n * (1 + scale) + shift)
// The reference computes the same expression with Triton's reduction order and libdevice's rsqrt, whose last bits
// are the H100's: this build fixes the order above, which the CPU oracle restates bit for bit.
//
// Two designs, as for the casts: rows that fit the chip's registers (C <= 2048 and at most the single-pass capacity)
// take one launch -- each wave holds the bf16 h of its rows, the workgroups agree on the amax through the tagged
// partials of the cast workspace (gpic_once.h), and each casts from its registers; larger ones take two, the second
// recomputing h from the x_new (or x) and rstd the first wrote.
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

// The four fp32 values of a group's 8 bytes of bf16.
__device__ __forceinline__ void unpack4(u32x2 v, float (&f)[4]) {
  f[0] = bf16_lo(v.x), f[1] = bf16_hi(v.x), f[2] = bf16_lo(v.y), f[3] = bf16_hi(v.y);
}

__device__ __forceinline__ float wave_sum_butterfly(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

// One row's h (this lane's groups j < J: elements 4 (lane + 64 j) .. + 3) as packed bf16 in H, and its amax bits
// (NaN excluded). kStore: write x_new (site 2), rstd (lane 0) and h (when p.h) as well. The groups are handled with a
// compile-time count when kJ > 0 (held in registers) or a run-time count C / 256 otherwise (then H is not kept).
template <int kJ, bool kStore>
__device__ __forceinline__ uint32_t norm_row(const NormArgs &p, int64_t row, u32x2 *H) {
  const int lane = threadIdx.x & 63;
  const int J = kJ > 0 ? kJ : p.C / 256;
  const int64_t b = row / p.ntok;
  const uint16_t *xr = p.x + row * p.C;
  float ss = 0.0f;
  for (int j = 0; j < J; j++) {   // pass over the row: x_new and the sum of squares
    const int c = 4 * (lane + 64 * j);
    float x[4];
    unpack4(ld8(xr + c), x);
    if (p.a) {
      float av[4], gv[4];
      unpack4(ld8(p.a + row * p.C + c), av);
      unpack4(ld8(p.gate + b * p.sg + c), gv);
#pragma unroll
      for (int e = 0; e < 4; e++) x[e] = bf16_round(x[e] + gv[e] * av[e]);
      if (kStore)
        *reinterpret_cast<u32x2 *>(p.xn + row * p.C + c) = u32x2{pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3])};
    }
#pragma unroll
    for (int e = 0; e < 4; e++) ss = ss + x[e] * x[e];
  }
  ss = wave_sum_butterfly(ss);
  // (__builtin_sqrtf is the correctly rounded square root; HIP's __fsqrt_rn maps to the hardware approximation)
  const float rstd = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(ss, (float)p.C) + p.eps));
  if (kStore && lane == 0) p.rstd[row] = rstd;
  uint32_t m = 0;
  for (int j = 0; j < J; j++) {   // h, from x_new as rounded (re-read from the cache for site 2)
    const int c = 4 * (lane + 64 * j);
    float x[4], sh[4], sc[4];
    if (p.a) {
      float av[4], gv[4];
      unpack4(ld8(xr + c), x);
      unpack4(ld8(p.a + row * p.C + c), av);
      unpack4(ld8(p.gate + b * p.sg + c), gv);
#pragma unroll
      for (int e = 0; e < 4; e++) x[e] = bf16_round(x[e] + gv[e] * av[e]);
    } else {
      unpack4(ld8(xr + c), x);
    }
    const float4 wv = *reinterpret_cast<const float4 *>(p.w + c);
    unpack4(ld8(p.shift + b * p.ssh + c), sh);
    unpack4(ld8(p.scale + b * p.ssc + c), sc);
    const float w4[4] = {wv.x, wv.y, wv.z, wv.w};
    float hv[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float n = bf16_round(w4[e] * (x[e] * rstd));
      hv[e] = n * (1.0f + sc[e]) + sh[e];
    }
    const u32x2 hw{pack_bf16(hv[0], hv[1]), pack_bf16(hv[2], hv[3])};
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
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float n = bf16_round(w4[e] * (x[e] * rstd));
    hv[e] = n * (1.0f + sc[e]) + sh[e];
  }
  return u32x2{pack_bf16(hv[0], hv[1]), pack_bf16(hv[2], hv[3])};
}

__device__ __forceinline__ uint32_t cast4_packed(u32x2 hw, float s) {
  return e4m3x4(sat(bf16_lo(hw.x) * s), sat(bf16_hi(hw.x) * s), sat(bf16_lo(hw.y) * s), sat(bf16_hi(hw.y) * s));
}

// Single pass: wave w of workgroup g holds rows (4 g + w) kR .. + kR - 1 (kJ groups of 4 per lane each), the
// workgroups fold their maxima (gpic_once.h), and each casts its rows from its registers.
template <int kJ, int kR>
__global__ __launch_bounds__(256, 4) void norm_q_once_kernel(NormArgs p, void *ws, uint32_t wait_ticks) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  auto row_of = [&](int64_t g, int r) { return (g * 4 + wave) * kR + r; };
  u32x2 H[kR][kJ];
  uint32_t m = 0;
#pragma unroll
  for (int r = 0; r < kR; r++) {
    const int64_t row = row_of(blockIdx.x, r);
    if (row < p.rows) {
      m = max(m, norm_row<kJ, true>(p, row, H[r]));
    } else {
#pragma unroll
      for (int j = 0; j < kJ; j++) H[r][j] = u32x2{0u, 0u};
    }
  }
  const uint32_t g = once_fold(block_max_u32(m), ws, wait_ticks, [&](int c) {
    // workgroup c's maximum from its rows (nothing stored): for a partial that did not appear in time
    uint32_t a = 0;
    for (int r = 0; r < kR; r++) {
      const int64_t row = row_of(c, r);
      if (row < p.rows) a = max(a, norm_row<0, false>(p, row, nullptr));
    }
    return block_max_u32(a);
  });
  float scale, deq;
  scales_from_amax(g, scale, deq);
  if (blockIdx.x == 0 && threadIdx.x == 0) *p.dequant = deq;
#pragma unroll
  for (int r = 0; r < kR; r++) {
    const int64_t row = row_of(blockIdx.x, r);
    if (row < p.rows) {
#pragma unroll
      for (int j = 0; j < kJ; j++)
        __builtin_nontemporal_store(cast4_packed(H[r][j], scale),
                                    reinterpret_cast<uint32_t *>(p.hq + row * p.C + 4 * (lane + 64 * j)));
    }
  }
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
    for (int j = 0; j < p.C / 256; j++) {
      const int c = 4 * (lane + 64 * j);
      __builtin_nontemporal_store(cast4_packed(h_from_stats(p, row, b, rstd, c), scale),
                                  reinterpret_cast<uint32_t *>(p.hq + row * p.C + c));
    }
  }
}

// ------------------------------------------------------------------------------------------- host side

static DeviceCache g_cap_norm[9];
struct NormCacheInit {
  NormCacheInit() {
    for (auto &c : g_cap_norm)
      for (int i = 0; i < kMaxDevices; i++) c[i] = -1;
  }
};
static NormCacheInit g_norm_cache_init;

// Rows per wave held by the single pass: kJ groups of 4 bf16 (kJ * 2 VGPRs) per row, at most 64 VGPRs in all (at
// most 10 rows: more spilled for the narrow rows, whose per-row state then dominates).
template <int kJ>
constexpr int kRowsOnce = kJ >= 3 ? 32 / kJ : 10;

template <int kJ>
static bool launch_norm_once(const NormArgs &p, void *ws, hipStream_t st) {
  constexpr int kR = kRowsOnce<kJ>;
  const int cap = once_capacity(reinterpret_cast<const void *>(&norm_q_once_kernel<kJ, kR>), g_cap_norm[kJ]);
  const int64_t wgs = (p.rows + 4 * kR - 1) / (4 * kR);
  if (!once_enabled() || cap <= 0 || wgs > cap) return false;
  norm_q_once_kernel<kJ, kR><<<(int)wgs, 256, 0, st>>>(p, ws, once_wait_ticks());
  return true;
}

}  // namespace gpic

using namespace gpic;

extern "C" {

int gpic_fp8_res_mod_rmsnorm(const uint16_t *x, const uint16_t *a, const uint16_t *gate, int64_t sg, const float *w,
                             const uint16_t *shift, int64_t ssh, const uint16_t *scale, int64_t ssc, int64_t rows,
                             int64_t ntok, int64_t C, float eps, uint16_t *xn, uint16_t *h, float *rstd, uint8_t *hq,
                             float *dequant, void *ws, void *stream) {
  const bool cast = dequant != nullptr;   // else the norm alone
  if (rows < 0 || C <= 0 || ntok <= 0 || !ws || !w || !shift || !scale) return GPIC_EINVAL;
  if (rows > 0 && (!x || !rstd || (cast ? !hq : !h) || (a && (!gate || !xn)))) return GPIC_EINVAL;
  if (C % 256 != 0 || rows % ntok != 0 || ssh % 4 != 0 || ssc % 4 != 0 || (a && sg % 4 != 0) || ssh < C || ssc < C ||
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
    norm_stats_kernel<<<(int)std::min<int64_t>((rows + 3) / 4, kMaxParts), 256, 0, st>>>(p, static_cast<uint32_t *>(ws));
    return (int)hipGetLastError();
  }
  bool done = false;
  switch (C / 256) {
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
  const int g1 = (int)std::min<int64_t>((rows + 3) / 4, kMaxParts);
  norm_stats_kernel<<<g1, 256, 0, st>>>(p, partial);
  const int g2 = (int)std::min<int64_t>((rows + 3) / 4, 2048);
  norm_cast_kernel<<<g2, 256, 0, st>>>(p, partial, g1);
  return (int)hipGetLastError();
}

}  // extern "C"

// Device-side building blocks of the FP8 linear path for gfx950 (CDNA4): bf16 and e4m3 conversions, the SwiGLU
// sigmoid, wavefront reductions. Everything here is compiled with -ffp-contract=off, so each float operation
// rounds exactly as written; fused multiply-adds appear only where __builtin_fmaf is called.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gpic {

constexpr float kFmax = 448.0f;  // the largest finite e4m3fn value (fp8_native.py:25)
constexpr float kTiny = 1e-12f;  // the amax floor (fp8_native.py:26)

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------- bf16

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16, round to nearest even; a NaN becomes a quiet NaN (torch's rounding rule). gfx950's
// v_cvt_pk_bf16_f32 does this in one instruction for two values; it gives the same bits as the integer rule
// (u + 0x7fff + ((u >> 16) & 1)) >> 16, NaN -> (u >> 16) | 0x40, on every one of the 2^32 fp32 inputs (the test
// suite's bf16 self-check runs that comparison on the GPU).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Packed bf16 pair: `lo` in bits 0..15, `hi` in bits 16..31.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// bf16 bits of one value (in bits 0..15).
__device__ __forceinline__ uint32_t bf16_rne(float f) { return pack_bf16(f, 0.0f) & 0xffffu; }

__device__ __forceinline__ float bf16_round(float f) { return __uint_as_float(bf16_rne(f) << 16); }

// Packed maximum of two u16 pairs (v_pk_max_u16).
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  u16x2 x = __builtin_bit_cast(u16x2, a), y = __builtin_bit_cast(u16x2, b);
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(x, y));
}

// |bf16| magnitudes of a word's two halves, NaNs dropped (set to 0): the amax ignores NaN as Triton's tl.max
// (maxnum) does in fp8_native.py:36.
__device__ __forceinline__ uint32_t bf16x2_absmax_nonan(uint32_t w) {
  uint32_t lo = w & 0x7fffu, hi = (w >> 16) & 0x7fffu;
  lo = lo > 0x7f80u ? 0u : lo;
  hi = hi > 0x7f80u ? 0u : hi;
  return lo > hi ? lo : hi;
}

// ------------------------------------------------------------------------------------------- e4m3

// q = e4m3(min(max(x * scale, -448), 448)) (fp8_native.py:47). fmaxf/fminf are IEEE maxNum/minNum as Triton's
// tl.maximum/tl.minimum: a NaN product saturates to -448. The narrowing is gfx950's v_cvt_pk_fp8_f32 (OCP e4m3fn,
// round to nearest even), which the GPU tests check against torch's conversion over every fp32 magnitude <= 448.
__device__ __forceinline__ float sat(float y) { return fminf(fmaxf(y, -kFmax), kFmax); }

__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
}

// Eight bf16 (one 16-byte word) -> eight e4m3 bytes.
__device__ __forceinline__ u32x2 cast8_bf16(u32x4 w, float s) {
  u32x2 o;
  o.x = e4m3x4(sat(bf16_lo(w.x) * s), sat(bf16_hi(w.x) * s), sat(bf16_lo(w.y) * s), sat(bf16_hi(w.y) * s));
  o.y = e4m3x4(sat(bf16_lo(w.z) * s), sat(bf16_hi(w.z) * s), sat(bf16_lo(w.w) * s), sat(bf16_hi(w.w) * s));
  return o;
}

// Four fp32 (one 16-byte word) -> four e4m3 bytes.
__device__ __forceinline__ uint32_t cast4_f32(u32x4 w, float s) {
  return e4m3x4(sat(__uint_as_float(w.x) * s), sat(__uint_as_float(w.y) * s), sat(__uint_as_float(w.z) * s),
                sat(__uint_as_float(w.w) * s));
}

// a = max(amax, 1e-12); scale = RN(448 / a); dequant = RN(a / 448) (fp8_native.py:43-44,49; IEEE division).
__device__ __forceinline__ void scales_from_amax(uint32_t amax_bits, float &scale, float &dequant) {
  float a = __uint_as_float(amax_bits);
  a = a < kTiny ? kTiny : a;
  scale = __fdiv_rn(kFmax, a);
  dequant = __fdiv_rn(a, kFmax);
}

// ------------------------------------------------------------------------------------------- SwiGLU sigmoid

// e^t: Cody-Waite reduction t = n ln2 + r with n = rint(t log2 e), r from two fused multiply-adds with a split ln2;
// e^r by its degree-7 Taylor polynomial (Horner, fused multiply-adds); ldexp(p, n). sigmoid(x) = 1 / (1 + e^-x)
// with IEEE division. This is the build's definition of the SwiGLU sigmoid (the reference's tl.sigmoid rounds as
// the H100 does); the CPU oracle states the same sequence and the tests check both over every bf16 input.
__device__ __forceinline__ float exp_cw(float t) {
  if (t != t) return t;
  if (t > 88.8f) return __builtin_huge_valf();
  if (t < -104.0f) return 0.0f;
  float n = __builtin_rintf(t * 1.44269502f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, t);
  r = __builtin_fmaf(-n, 1.42860682e-06f, r);
  float p = 1.98412698e-04f;
  p = __builtin_fmaf(p, r, 1.38888889e-03f);
  p = __builtin_fmaf(p, r, 8.33333377e-03f);
  p = __builtin_fmaf(p, r, 4.16666679e-02f);
  p = __builtin_fmaf(p, r, 1.66666672e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

__device__ __forceinline__ float sigmoid(float x) { return __fdiv_rn(1.0f, 1.0f + exp_cw(-x)); }

// ------------------------------------------------------------------------------------------- reductions

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t t = (uint32_t)__shfl_xor((int)v, o, 64);
    v = v > t ? v : t;
  }
  return v;
}

// Block-wide maximum (blockDim.x a multiple of 64, at most 1024); every thread gets the result.
// Workgroup barrier for LDS communication only: waits for this wave's LDS operations, not for its global loads, so
// loads issued before it stay in flight (__syncthreads' fence would wait for them).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v) {
  __shared__ uint32_t red[16];
  v = wave_max_u32(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  lds_barrier();  // red[] may still be read by a previous call
  if (lane == 0) red[wave] = v;
  lds_barrier();
  uint32_t m = 0;
  for (int i = 0; i < nw; i++) m = red[i] > m ? red[i] : m;
  return m;
}

}  // namespace gpic

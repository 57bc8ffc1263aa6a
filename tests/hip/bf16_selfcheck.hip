// Test-only library: checks the library's fp32 -> bf16 rounding (pack_bf16 in gpic_device.h, gfx950's
// v_cvt_pk_bf16_f32) against the integer round-to-nearest-even rule on all 2^32 fp32 bit patterns, both halves of
// the packed result. Built by __graft_entry__.build(); called by tests/test_gpu_bf16.py.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../nano-gpic_amd/csrc/gpic_device.h"

namespace {

// The rule the reference's rounding follows (torch's round_to_nearest_even): RNE on the bits; NaN -> quiet NaN.
__device__ uint32_t rne_int(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// One launch covers the patterns [hi << 24, (hi + 1) << 24): 65536 workgroups x 256 threads, one pattern each.
// The high half of the pair gets a different pattern (sign and lowest bit flipped) so both halves are exercised.
__global__ __launch_bounds__(256) void check(uint32_t hi, unsigned long long *mismatch) {
  const uint32_t u = (hi << 24) | (blockIdx.x << 8) | threadIdx.x;
  const float f = __uint_as_float(u), g = __uint_as_float(u ^ 0x80000001u);
  const uint32_t got = gpic::pack_bf16(f, g);
  const uint32_t want = rne_int(f) | (rne_int(g) << 16);
  if (got != want) atomicAdd(mismatch, 1ull);
}

}  // namespace

extern "C" int gpic_selfcheck_bf16(unsigned long long *mismatch, void *stream) {
  for (uint32_t hi = 0; hi < 256; hi++) check<<<65536, 256, 0, (hipStream_t)stream>>>(hi, mismatch);
  return (int)hipGetLastError();
}

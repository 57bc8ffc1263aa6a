// Measurement-only library: the FP8 MFMA throughput the device sustains when every SIMD issues MFMAs back to back,
// on constant and on random e4m3 operands, for the two f8f6f4 forms: v_mfma_f32_16x16x128_f8f6f4 (the one the GEMM
// uses) and v_mfma_f32_32x32x64_f8f6f4. It is the ceiling the GEMM's roofline fraction should be read against: the
// published dense peak (5.0 PFLOP/s at 2.4 GHz) holds for operands whose bits barely toggle, while random operands
// draw enough power that the clock drops, and the two forms draw different power for the same work.
//
// One workgroup of 4 waves per CU (160 KiB of LDS keeps it alone there), one wave per SIMD, each wave with 16
// independent 32 x 32 accumulator tiles (or 32 of 16 x 16) and 4 A x 4 B operand fragments of random (or constant)
// e4m3 bytes in registers, consecutive MFMAs taking a different pair, so the operands toggle as a GEMM's do.
// (Fragments read from LDS instead measured the same rates: the LDS and register traffic costs next to nothing beside
// the MFMA array.) No memory traffic, no barriers in the loop. Built by __graft_entry__.build(); called by
// tests/test_gpu_ceiling.py and bench.py.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

__device__ uint32_t hash_e4m3x4(uint32_t x) {   // 4 random e4m3 bytes, the exponent's lowest bit cleared (no NaN)
  x ^= x >> 15;
  x *= 0x2c1b3c6du;
  x ^= x >> 12;
  x *= 0x297a2d39u;
  x ^= x >> 15;
  return x & 0xf7f7f7f7u;
}

// K step: 128 x 128 x 64 x 2 FLOP per wave either way -- 16 MFMAs of 32 x 32 x 64 (64 cycles each) or 32 of
// 16 x 16 x 128 (32 cycles each): 1024 cycles of one SIMD's MFMA pipe.
template <int kShape>
__global__ __launch_bounds__(256, 1) void mfma_loop(int steps, int random, const uint32_t *src, int64_t src_words,
                                                     float *out, unsigned long long *cycles) {
  __shared__ uint8_t hold[160 * 1024];
  if (threadIdx.x == 0) hold[blockIdx.x & 1023] = 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v8i fa[4], fb[4];
#pragma unroll
  for (int f = 0; f < 4; f++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint32_t seed = ((blockIdx.x * 4 + wave) * 64 + lane) * 64 + f * 8 + e;
      if (src) {   // words of the caller's operand bytes
        fa[f][e] = (int)src[(2 * (int64_t)seed) % src_words];
        fb[f][e] = (int)src[(2 * (int64_t)seed + 1) % src_words];
      } else {
        fa[f][e] = random ? (int)hash_e4m3x4(2 * seed) : 0x38383838;
        fb[f][e] = random ? (int)hash_e4m3x4(2 * seed + 1) : 0x38383838;
      }
    }
  __syncthreads();
  float sum = 0.f;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  if constexpr (kShape == 32) {
    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[i][j] = v16f{};
    for (int s = 0; s < steps; s++) {
#pragma unroll
      for (int j = 0; j < 16; j++)
        acc[j >> 2][j & 3] =
            __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[j >> 2], fa[j & 3], acc[j >> 2][j & 3], 0, 0, 0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) sum += acc[i][j][e];
  } else {
    v4f acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[i][j] = v4f{};
    for (int s = 0; s < steps; s++) {
#pragma unroll
      for (int j = 0; j < 32; j++)
        acc[j >> 2][j & 3] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fb[(j >> 2) & 3], fa[j & 3],
                                                                              acc[j >> 2][j & 3], 0, 0, 0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) sum += acc[i][j][e];
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  out[blockIdx.x * 256 + threadIdx.x] = sum;
  if (lane == 0) cycles[blockIdx.x * 4 + wave] = t1 - t0;
}

}  // namespace

// Runs the loop of MFMA form `shape` (16: 16 x 16 x 128, 32: 32 x 32 x 64) for `steps` K steps on every CU of the
// current device, after one untimed launch. Operands: words of the device buffer `src` (src_bytes bytes, 4-byte
// aligned: e.g. the e4m3 bytes of a real tensor) when it is given, else random (random != 0) or constant bytes. Returns the kernel's
// time in ms, its TFLOP/s, the shader clock the waves saw (s_memtime cycles over the time) and the MFMA-busy fraction
// (1024 MFMA cycles per K step over the cycles).
extern "C" int gpic_probe_mfma_ceiling(int shape, int random, const void *src, int64_t src_bytes, int steps, double *ms,
                                       double *tflops, double *ghz, double *busy) {
  if ((shape != 16 && shape != 32) || steps < 1 || !ms || !tflops || !ghz || !busy) return 1;
  if (src && (src_bytes < 8 || ((uintptr_t)src & 3))) return 1;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 2;
  float *out = nullptr;
  unsigned long long *cyc = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = 0;
  auto launch = [&]() {
    const uint32_t *w = static_cast<const uint32_t *>(src);
    if (shape == 16) mfma_loop<16><<<cus, 256>>>(steps, random, w, src_bytes / 4, out, cyc);
    else mfma_loop<32><<<cus, 256>>>(steps, random, w, src_bytes / 4, out, cyc);
  };
  if (hipMalloc(&out, (size_t)cus * 256 * sizeof(float)) != hipSuccess ||
      hipMalloc(&cyc, (size_t)cus * 4 * sizeof(unsigned long long)) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
      hipEventCreate(&e1) != hipSuccess) {
    rc = 3;
  } else {
    launch();
    const hipError_t r0 = hipEventRecord(e0, nullptr);
    launch();
    const hipError_t r1 = hipEventRecord(e1, nullptr);
    float t = 0.f;
    if (r0 != hipSuccess || r1 != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
        hipEventElapsedTime(&t, e0, e1) != hipSuccess) {
      rc = 4;
    } else {
      unsigned long long *h = new unsigned long long[(size_t)cus * 4];
      if (hipMemcpy(h, cyc, (size_t)cus * 4 * sizeof(unsigned long long), hipMemcpyDeviceToHost) != hipSuccess) {
        rc = 5;
      } else {
        double mean = 0.0;
        for (int i = 0; i < cus * 4; i++) mean += (double)h[i];
        mean /= (double)(cus * 4);
        *ms = t;
        *tflops = 2.0 * 128 * 128 * 64 * 4 * (double)steps * cus / (t * 1e-3) / 1e12;
        *ghz = mean / (t * 1e-3) / 1e9;
        *busy = 1024.0 * steps / mean;
      }
      delete[] h;
    }
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (out) (void)hipFree(out);
  if (cyc) (void)hipFree(cyc);
  return rc ? rc : (int)hipGetLastError();
}

// Measurement-only library: the FP8 MFMA throughput the device sustains when every SIMD issues
// v_mfma_f32_32x32x64_f8f6f4 back to back, on constant and on random e4m3 operands. It is the ceiling the GEMM's
// roofline fraction should be read against: the published dense peak (5.0 PFLOP/s at 2.4 GHz) holds for operands
// whose bits barely toggle, while random operands draw enough power that the clock drops.
//
// One workgroup of 4 waves per CU (160 KiB of LDS keeps it alone there), one wave per SIMD. Each wave owns 4 x 4
// independent 32 x 32 accumulator tiles (256 AGPRs) and runs K steps of 16 MFMAs; between its MFMAs it reads the next
// step's 16 fragment registers from LDS (two fragment buffers, as the GEMM's K loop does), so the only traffic is LDS
// reads. No global loads, no barriers in the loop. Built by __graft_entry__.build(); called by
// tests/test_gpu_ceiling.py and bench.py.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#define LDS_AS __attribute__((address_space(3)))

constexpr int kLds = 160 * 1024;

__global__ __launch_bounds__(256, 1) void mfma_loop(int steps, int random, float *out, unsigned long long *cycles) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kLds];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // operands: random e4m3 bytes (bit 3, the exponent's lowest bit, cleared: no NaN / inf pattern, magnitudes up to
  // 240) or one constant pattern
  for (int i = threadIdx.x; i < kLds / 4; i += 256) {
    uint32_t x = 0x38383838u;
    if (random) {
      x = (uint32_t)i * 2654435761u ^ (uint32_t)blockIdx.x * 40503u ^ 0x9e3779b9u;
      x ^= x >> 15;
      x *= 0x2c1b3c6du;
      x ^= x >> 12;
      x *= 0x297a2d39u;
      x ^= x >> 15;
      x &= 0xf7f7f7f7u;
    }
    reinterpret_cast<uint32_t *>(smem)[i] = x;
  }
  __syncthreads();

  // fragment f of a K step: 32 rows x 64 bytes of K; lane l reads 32 bytes of row (l & 31) as two 16-byte reads
  // (A fragments from the first 64 KiB of LDS, B fragments from the next 64 KiB; rows of 128 bytes, two K steps per
  // row, 16-byte slots XOR-swizzled by (row >> 1) & 7 so that 16 lanes read 16 distinct slots)
  v8i fa[2][4], fb[2][4];
  const int row = lane & 31, c0 = 2 * (lane >> 5), sw = (row >> 1) & 7;
  auto read = [&](int b, int ks, int j) {
    const int f = (j >> 1) & 3;
    const bool isA = j < 8;
    const int r = (isA ? 0 : 512) + wave * 128 + f * 32 + row;   // 1024 rows of 128 bytes = 128 KiB
    const int off = r * 128 + 16 * ((4 * ks + c0 + (j & 1)) ^ sw);
    const u32x4 x = *(const LDS_AS u32x4 *)((const LDS_AS uint8_t *)smem + off);
    v8i &d = isA ? fa[b][f] : fb[b][f];
    if (j & 1) {
      d[4] = (int)x.x, d[5] = (int)x.y, d[6] = (int)x.z, d[7] = (int)x.w;
    } else {
      d[0] = (int)x.x, d[1] = (int)x.y, d[2] = (int)x.z, d[3] = (int)x.w;
    }
  };
#pragma unroll
  for (int j = 0; j < 16; j++) read(0, 0, j);
  v16f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = v16f{};
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int s = 0; s < steps; s += 2) {
#pragma unroll
    for (int u = 0; u < 2; u++) {   // K step s + u: MFMAs on buffer u, the next step's fragments into buffer u ^ 1
#pragma unroll
      for (int j = 0; j < 16; j++) {
        acc[j >> 2][j & 3] =
            __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[u][j >> 2], fa[u][j & 3], acc[j >> 2][j & 3], 0, 0, 0, 0,
                                                            0, 0);
        read(u ^ 1, u ^ 1, j);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) sum += acc[i][j][e];
  out[blockIdx.x * 256 + threadIdx.x] = sum;
  if (lane == 0) cycles[blockIdx.x * 4 + wave] = t1 - t0;
}

}  // namespace

// Runs the loop for `steps` K steps (even, >= 2) on every CU of the current device, with random (random != 0) or
// constant operands, after one untimed launch. Returns the kernel's time in ms, its TFLOP/s, the shader clock the
// waves saw (s_memtime cycles over the time) and the MFMA-busy fraction (64 cycles per MFMA over the cycles).
extern "C" int gpic_probe_mfma_ceiling(int random, int steps, double *ms, double *tflops, double *ghz, double *busy) {
  if (steps < 2 || steps % 2 || !ms || !tflops || !ghz || !busy) return 1;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 2;
  float *out = nullptr;
  unsigned long long *cyc = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = 0;
  if (hipMalloc(&out, (size_t)cus * 256 * sizeof(float)) != hipSuccess ||
      hipMalloc(&cyc, (size_t)cus * 4 * sizeof(unsigned long long)) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
      hipEventCreate(&e1) != hipSuccess) {
    rc = 3;
  } else {
    mfma_loop<<<cus, 256>>>(steps, random, out, cyc);
    const hipError_t r0 = hipEventRecord(e0, nullptr);
    mfma_loop<<<cus, 256>>>(steps, random, out, cyc);
    const hipError_t r1 = hipEventRecord(e1, nullptr);
    float t = 0.f;
    if (r0 != hipSuccess || r1 != hipSuccess || hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&t, e0, e1) != hipSuccess) {
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
        *tflops = 2.0 * 256 * 256 * 64 * (double)steps * cus / (t * 1e-3) / 1e12;
        *ghz = mean / (t * 1e-3) / 1e9;
        *busy = 16.0 * 64.0 * steps / mean;
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

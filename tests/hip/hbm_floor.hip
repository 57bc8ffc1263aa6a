// Measurement-only library: how long one launch takes to read a buffer from HBM into registers, to write one, or to
// do both with the traffic of a cast (read 16 bytes, write 8 for each word) -- floors under any single-pass cast of
// that buffer, which has to read all of its input, agree on the maximum, then write all of its output. bench.py
// reports the config-2 cast against them (the 64 MiB bf16 read and the 32 MiB e4m3 write of [32768 x 1024]), with
// L2 / MALL flushed as for the cast.
//
// Launch shapes (cfg): 0 = 1024 threads x 16 words of 16 bytes per thread (the cast's own: one workgroup per CU),
// 1 = 512 x 16 (two per CU), 2 = 256 x 8, 3 = 512 x 32. A thread's words lie one grid's worth apart
// (word (j G + b) T + t), as in the cast; reads are non-temporal loads whose maximum is written once per workgroup,
// writes are non-temporal 16-byte stores of a constant. Built by __graft_entry__.build(); called by bench.py and
// tests/test_gpu_ceiling.py.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int kT, int kW>
__global__ __launch_bounds__(kT) void read_kernel(const u32x4 *__restrict__ x, uint32_t nw, uint32_t *__restrict__ out) {
  const uint32_t t = threadIdx.x, b = blockIdx.x, G = gridDim.x;
  u32x4 w[kW];
#pragma unroll
  for (int j = 0; j < kW; j++) {
    const uint32_t i = ((uint32_t)j * G + b) * kT + t;
    w[j] = __builtin_nontemporal_load(x + (i < nw ? i : 0u));
  }
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < kW; j++) m = max(m, max(max(w[j].x, w[j].y), max(w[j].z, w[j].w)));
  __shared__ uint32_t s;
  if (t == 0) s = 0;
  __syncthreads();
  atomicMax(&s, m);
  __syncthreads();
  if (t == 0) out[b] = s;
}

template <int kT, int kW>
__global__ __launch_bounds__(kT) void write_kernel(u32x4 *__restrict__ y, uint32_t nw, uint32_t v) {
  const uint32_t t = threadIdx.x, b = blockIdx.x, G = gridDim.x;
#pragma unroll
  for (int j = 0; j < kW; j++) {
    const uint32_t i = ((uint32_t)j * G + b) * kT + t;
    if (i < nw) __builtin_nontemporal_store(u32x4{v, v, v, v}, y + i);
  }
}

// The cast's traffic in one launch without its cross-chip step: each thread reads its kW words of 16 bytes, then
// writes 8 bytes for each (dst word i of 8 bytes for source word i, as the cast writes e4m3), a workgroup's writes
// starting as soon as its own reads are in. A single-pass cast must also wait for every workgroup's maximum before
// its first write, so this launch's time is a floor under it.
template <int kT, int kW>
__global__ __launch_bounds__(kT) void read_write_kernel(const u32x4 *__restrict__ x, uint32_t nw,
                                                        uint32_t *__restrict__ y) {
  const uint32_t t = threadIdx.x, b = blockIdx.x, G = gridDim.x;
  u32x4 w[kW];
#pragma unroll
  for (int j = 0; j < kW; j++) {
    const uint32_t i = ((uint32_t)j * G + b) * kT + t;
    w[j] = __builtin_nontemporal_load(x + (i < nw ? i : 0u));
  }
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int j = 0; j < kW; j++) {
    const uint32_t i = ((uint32_t)j * G + b) * kT + t;
    if (i < nw) __builtin_nontemporal_store(u32x2{w[j].x ^ w[j].y, w[j].z ^ w[j].w}, reinterpret_cast<u32x2 *>(y) + i);
  }
}

template <int kT, int kW>
int launch_rw(const void *src, uint64_t bytes, void *dst, hipStream_t st) {
  const uint32_t nw = (uint32_t)(bytes / 16);
  const int grid = (int)((nw + kT * kW - 1) / (kT * kW));
  read_write_kernel<kT, kW><<<grid, kT, 0, st>>>(static_cast<const u32x4 *>(src), nw, static_cast<uint32_t *>(dst));
  return (int)hipGetLastError();
}

template <int kT, int kW>
int launch(bool rd, void *p, uint64_t bytes, void *out, hipStream_t st) {
  const uint32_t nw = (uint32_t)(bytes / 16);
  const uint32_t per = kT * kW;
  const int grid = (int)((nw + per - 1) / per);
  if (rd) read_kernel<kT, kW><<<grid, kT, 0, st>>>(static_cast<const u32x4 *>(p), nw, static_cast<uint32_t *>(out));
  else write_kernel<kT, kW><<<grid, kT, 0, st>>>(static_cast<u32x4 *>(p), nw, 0x38383838u);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

// Workgroups the read of `bytes` launches in shape cfg (the size of the `out` buffer it needs, in words).
int gpic_probe_hbm_groups(int cfg, uint64_t bytes) {
  static const int per[4] = {1024 * 16, 512 * 16, 256 * 8, 512 * 32};
  if (cfg < 0 || cfg > 3) return -1;
  return (int)((bytes / 16 + per[cfg] - 1) / per[cfg]);
}

// One read (rd != 0; out: gpic_probe_hbm_groups words) or write (rd == 0) launch over `bytes` (a multiple of 16, below
// 2^35) of p on `stream`. Returns a hipError_t, or -1 for a bad argument.
int gpic_probe_hbm(int rd, int cfg, void *p, uint64_t bytes, void *out, void *stream) {
  (void)hipGetLastError();
  if (!p || bytes % 16 != 0 || bytes / 16 >= (1ull << 31) || (rd && !out)) return -1;
  hipStream_t st = (hipStream_t)stream;
  switch (cfg) {
    case 0: return launch<1024, 16>(rd != 0, p, bytes, out, st);
    case 1: return launch<512, 16>(rd != 0, p, bytes, out, st);
    case 2: return launch<256, 8>(rd != 0, p, bytes, out, st);
    case 3: return launch<512, 32>(rd != 0, p, bytes, out, st);
    default: return -1;
  }
}

// One launch reading `bytes` of src (16-byte words) and writing bytes / 2 to dst (8 bytes per source word), in shape
// cfg: the cast's traffic without its cross-chip maximum. Returns a hipError_t, or -1 for a bad argument.
int gpic_probe_hbm_rw(int cfg, const void *src, uint64_t bytes, void *dst, void *stream) {
  (void)hipGetLastError();
  if (!src || !dst || bytes % 16 != 0 || bytes / 16 >= (1ull << 31)) return -1;
  hipStream_t st = (hipStream_t)stream;
  switch (cfg) {
    case 0: return launch_rw<1024, 16>(src, bytes, dst, st);
    case 1: return launch_rw<512, 16>(src, bytes, dst, st);
    case 2: return launch_rw<256, 8>(src, bytes, dst, st);
    case 3: return launch_rw<512, 32>(src, bytes, dst, st);
    default: return -1;
  }
}

}  // extern "C"

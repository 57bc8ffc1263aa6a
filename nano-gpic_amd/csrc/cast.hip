// Per-tensor current-amax e4m3 casts for gfx950: the flat cast (tcast), the cast with a transposed copy (for the
// dgrad / wgrad operands), the SwiGLU product cast and the SwiGLU backward.
//
// Every cast is two stream-ordered launches with no state between calls:
//   1. an amax pass: each workgroup reduces its share to one partial maximum (|x| bit patterns, NaN ignored) and
//      writes it to partial[blockIdx.x] -- no atomics, so nothing has to be zeroed beforehand;
//   2. a cast pass: each workgroup folds all partials (<= kMaxParts words, served from L2), derives the scale with
//      IEEE division and streams its share: 128-bit loads, 128-bit e4m3 stores.
// Workgroup 0 of pass 2 writes the dequantization scale.
#include "gpic_device.h"
#include "gpic_launch.h"

namespace gpic {

// ------------------------------------------------------------------------------------------- pass 1: amax

// x: n elements of T (bf16 as uint16_t, or float), 16-byte aligned. Units of 16 elements; the n % 16 tail is read
// by the first threads of workgroup 0.
template <typename T>
__global__ __launch_bounds__(kCastThreads) void amax_kernel(const T *__restrict__ x, int64_t n,
                                                             uint32_t *__restrict__ partial) {
  constexpr int kWords = 16 * sizeof(T) / 16;  // 16-byte words per unit: 2 (bf16) or 4 (fp32)
  const int64_t units = n / 16;
  const u32x4 *xv = reinterpret_cast<const u32x4 *>(x);
  uint32_t m = 0;
  bool nan = false;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += (int64_t)gridDim.x * blockDim.x) {
    u32x4 w[kWords];
#pragma unroll
    for (int i = 0; i < kWords; i++) w[i] = __builtin_nontemporal_load(xv + u * kWords + i);
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int i = 0; i < kWords; i++) {
        m = pk_max_u16(m, w[i].x & 0x7fff7fffu);
        m = pk_max_u16(m, w[i].y & 0x7fff7fffu);
        m = pk_max_u16(m, w[i].z & 0x7fff7fffu);
        m = pk_max_u16(m, w[i].w & 0x7fff7fffu);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kWords; i++) {
        uint32_t a = max(max(w[i].x & 0x7fffffffu, w[i].y & 0x7fffffffu), max(w[i].z & 0x7fffffffu, w[i].w & 0x7fffffffu));
        m = max(m, a);
      }
    }
  }
  if constexpr (sizeof(T) == 2) {
    m = max(m & 0xffffu, m >> 16);
    nan = m > 0x7f80u;
    m <<= 16;
  } else {
    nan = m > 0x7f800000u;
  }
  if (nan) {  // rare: this thread saw a NaN; fold its elements again without them (tl.max is maxnum)
    m = 0;
    for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += (int64_t)gridDim.x * blockDim.x)
      for (int i = 0; i < 16; i++) {
        uint32_t a = sizeof(T) == 2 ? ((uint32_t)(reinterpret_cast<const uint16_t *>(x)[u * 16 + i] & 0x7fffu) << 16)
                                    : (__float_as_uint(reinterpret_cast<const float *>(x)[u * 16 + i]) & 0x7fffffffu);
        if (a <= 0x7f800000u) m = max(m, a);
      }
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 15)) {
    const int64_t i = units * 16 + threadIdx.x;
    uint32_t a = sizeof(T) == 2 ? ((uint32_t)(reinterpret_cast<const uint16_t *>(x)[i] & 0x7fffu) << 16)
                                : (__float_as_uint(reinterpret_cast<const float *>(x)[i]) & 0x7fffffffu);
    if (a <= 0x7f800000u) m = max(m, a);
  }
  m = block_max_u32(m);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// Fold the partial maxima of pass 1 (every thread gets the amax bits).
__device__ __forceinline__ uint32_t fold_partials(const uint32_t *__restrict__ partial, int nparts) {
  uint32_t m = 0;
  for (int i = threadIdx.x; i < nparts; i += blockDim.x) m = max(m, partial[i]);
  return block_max_u32(m);
}

// ------------------------------------------------------------------------------------------- pass 2: flat cast

template <typename T>
__global__ __launch_bounds__(kCastThreads) void cast_kernel(const T *__restrict__ x, int64_t n,
                                                             const uint32_t *__restrict__ partial, int nparts,
                                                             uint8_t *__restrict__ q, float *__restrict__ dequant) {
  constexpr int kWords = 16 * sizeof(T) / 16;
  float scale, deq;
  scales_from_amax(fold_partials(partial, nparts), scale, deq);
  if (blockIdx.x == 0 && threadIdx.x == 0) *dequant = deq;
  const int64_t units = n / 16;
  const u32x4 *xv = reinterpret_cast<const u32x4 *>(x);
  u32x4 *qv = reinterpret_cast<u32x4 *>(q);
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += (int64_t)gridDim.x * blockDim.x) {
    u32x4 w[kWords];
#pragma unroll
    for (int i = 0; i < kWords; i++) w[i] = __builtin_nontemporal_load(xv + u * kWords + i);
    u32x4 o;
    if constexpr (sizeof(T) == 2) {
      u32x2 a = cast8_bf16(w[0], scale), b = cast8_bf16(w[1], scale);
      o = u32x4{a.x, a.y, b.x, b.y};
    } else {
      o = u32x4{cast4_f32(w[0], scale), cast4_f32(w[1], scale), cast4_f32(w[2], scale), cast4_f32(w[3], scale)};
    }
    __builtin_nontemporal_store(o, qv + u);
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 15)) {
    const int64_t i = units * 16 + threadIdx.x;
    float v = sizeof(T) == 2 ? bf16_lo(reinterpret_cast<const uint16_t *>(x)[i])
                             : reinterpret_cast<const float *>(x)[i];
    q[i] = (uint8_t)e4m3x4(sat(v * scale), 0.f, 0.f, 0.f);
  }
}

// ------------------------------------------------------------------------------------------- pass 2: cast + transpose

// Sources of the transposing cast: 8 consecutive elements (row r, columns c..c+7) as fp32.
struct SrcBF16 {
  const uint16_t *x;
  int64_t ld;
  __device__ __forceinline__ void load8(int64_t r, int64_t c, float (&v)[8]) const {
    const u32x4 w = *reinterpret_cast<const u32x4 *>(x + r * ld + c);
    const uint32_t a[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[2 * i] = bf16_lo(a[i]);
      v[2 * i + 1] = bf16_hi(a[i]);
    }
  }
};

struct SrcF32 {
  const float *x;
  int64_t ld;
  __device__ __forceinline__ void load8(int64_t r, int64_t c, float (&v)[8]) const {
    const u32x4 w0 = *reinterpret_cast<const u32x4 *>(x + r * ld + c);
    const u32x4 w1 = *reinterpret_cast<const u32x4 *>(x + r * ld + c + 4);
    v[0] = __uint_as_float(w0.x), v[1] = __uint_as_float(w0.y), v[2] = __uint_as_float(w0.z);
    v[3] = __uint_as_float(w0.w), v[4] = __uint_as_float(w1.x), v[5] = __uint_as_float(w1.y);
    v[6] = __uint_as_float(w1.z), v[7] = __uint_as_float(w1.w);
  }
};

struct SrcSwiGLU;  // defined with the SwiGLU kernels below

// src [rows, cols] (cols % 8 == 0) -> q [rows, cols] (row stride ldq; skipped when q == nullptr) and the transposed
// bytes qt [cols, ldt] (ldt % 16 == 0, ldt >= rows), whose columns rows..ldt-1 are written as zeros so a GEMM can
// reduce over the padded length. Tile: 64 rows x 64 cols per workgroup of 256 threads; the transpose goes through
// LDS. The scale comes from the partial maxima of the matching amax pass.
template <class Src>
__global__ __launch_bounds__(256) void cast_t_kernel(Src src, int64_t rows, int64_t cols,
                                                      const uint32_t *__restrict__ partial, int nparts,
                                                      uint8_t *__restrict__ q, int64_t ldq, uint8_t *__restrict__ qt,
                                                      int64_t ldt, float *__restrict__ dequant) {
  __shared__ uint32_t tile[64][64 / 4 + 1];  // [row][col / 4] e4m3 bytes; one word of padding per row
  float scale, deq;
  scales_from_amax(fold_partials(partial, nparts), scale, deq);
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *dequant = deq;
  const int64_t c0 = (int64_t)blockIdx.x * 64, r0 = (int64_t)blockIdx.y * 64;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int ci = threadIdx.x + 256 * i;
    const int r = ci >> 3, cc = ci & 7;
    const int64_t gr = r0 + r, gc = c0 + cc * 8;
    u32x2 o = {0u, 0u};
    if (gr < rows && gc < cols) {
      float v[8];
      src.load8(gr, gc, v);
      o.x = e4m3x4(sat(v[0] * scale), sat(v[1] * scale), sat(v[2] * scale), sat(v[3] * scale));
      o.y = e4m3x4(sat(v[4] * scale), sat(v[5] * scale), sat(v[6] * scale), sat(v[7] * scale));
      if (q) *reinterpret_cast<u32x2 *>(q + gr * ldq + gc) = o;
    }
    tile[r][cc * 2] = o.x;
    tile[r][cc * 2 + 1] = o.y;
  }
  __syncthreads();
  // qt row c0 + c gets bytes r0 + 16p .. r0 + 16p + 15: thread t -> c = t / 4, p = t % 4
  const int c = threadIdx.x >> 2, p = threadIdx.x & 3;
  const int64_t gc = c0 + c, gr = r0 + 16 * p;
  if (gc < cols && gr < ldt) {
    const uint8_t *tb = reinterpret_cast<const uint8_t *>(&tile[0][0]);
    constexpr int kRowBytes = (64 / 4 + 1) * 4;
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint32_t v = 0;
#pragma unroll
      for (int b = 0; b < 4; b++) v |= (uint32_t)tb[(16 * p + 4 * j + b) * kRowBytes + c] << (8 * b);
      o[j] = v;
    }
    *reinterpret_cast<u32x4 *>(qt + gc * ldt + gr) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// ------------------------------------------------------------------------------------------- SwiGLU

// a = bf16(bf16(z1 * sigmoid(z1)) * z2) for one z1 / z2 pair of bf16 (fp8_native.py:55-58).
__device__ __forceinline__ float swiglu1(float z1, float z2) {
  float sl = bf16_round(z1 * sigmoid(z1));
  return bf16_round(sl * z2);
}

// Eight products from 16-byte words of z1 and z2; returns them as fp32 (exact bf16 values).
__device__ __forceinline__ void swiglu8(u32x4 z1, u32x4 z2, float (&a)[8]) {
  const uint32_t w1[4] = {z1.x, z1.y, z1.z, z1.w}, w2[4] = {z2.x, z2.y, z2.z, z2.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    a[2 * i] = swiglu1(bf16_lo(w1[i]), bf16_lo(w2[i]));
    a[2 * i + 1] = swiglu1(bf16_hi(w1[i]), bf16_hi(w2[i]));
  }
}

struct SrcSwiGLU {
  const uint16_t *z;
  int64_t sz, H;
  __device__ __forceinline__ void load8(int64_t r, int64_t c, float (&v)[8]) const {
    const u32x4 z1 = *reinterpret_cast<const u32x4 *>(z + r * sz + c);
    const u32x4 z2 = *reinterpret_cast<const u32x4 *>(z + r * sz + H + c);
    swiglu8(z1, z2, v);
  }
};

__device__ __forceinline__ uint32_t absbits_nonan(float v) {
  uint32_t a = __float_as_uint(v) & 0x7fffffffu;
  return a > 0x7f800000u ? 0u : a;
}

// z [M, 2H] bf16 (row stride sz, H % 8 == 0): rows strided over workgroups, 8-element units over threads.
__global__ __launch_bounds__(kCastThreads) void swiglu_amax_kernel(const uint16_t *__restrict__ z, int64_t M, int64_t H,
                                                                    int64_t sz, uint32_t *__restrict__ partial) {
  const int64_t units = H / 8;
  uint32_t m = 0;
  for (int64_t r = blockIdx.x; r < M; r += gridDim.x) {
    const uint16_t *zr = z + r * sz;
    for (int64_t u = threadIdx.x; u < units; u += blockDim.x) {
      u32x4 z1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + 8 * u));
      u32x4 z2 = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + H + 8 * u));
      float a[8];
      swiglu8(z1, z2, a);
#pragma unroll
      for (int i = 0; i < 8; i++) m = max(m, absbits_nonan(a[i]));
    }
  }
  m = block_max_u32(m);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

__global__ __launch_bounds__(kCastThreads) void swiglu_cast_kernel(const uint16_t *__restrict__ z, int64_t M, int64_t H,
                                                                    int64_t sz, const uint32_t *__restrict__ partial,
                                                                    int nparts, uint8_t *__restrict__ q, int64_t sq,
                                                                    float *__restrict__ dequant) {
  float scale, deq;
  scales_from_amax(fold_partials(partial, nparts), scale, deq);
  if (blockIdx.x == 0 && threadIdx.x == 0) *dequant = deq;
  const int64_t units = H / 8;
  for (int64_t r = blockIdx.x; r < M; r += gridDim.x) {
    const uint16_t *zr = z + r * sz;
    for (int64_t u = threadIdx.x; u < units; u += blockDim.x) {
      u32x4 z1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + 8 * u));
      u32x4 z2 = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + H + 8 * u));
      float a[8];
      swiglu8(z1, z2, a);
      u32x2 o;
      o.x = e4m3x4(sat(a[0] * scale), sat(a[1] * scale), sat(a[2] * scale), sat(a[3] * scale));
      o.y = e4m3x4(sat(a[4] * scale), sat(a[5] * scale), sat(a[6] * scale), sat(a[7] * scale));
      *reinterpret_cast<u32x2 *>(q + r * sq + 8 * u) = o;
    }
  }
}

// dz = [d1 | d2] (fp8_native.py:88-96), each operation rounded on its own, left to right:
//   sg = sigmoid(z1); sl = bf16(z1 * sg); d1 = bf16((da * z2) * (sg * (1 + z1 * (1 - sg)))); d2 = bf16(da * sl)
__global__ __launch_bounds__(kCastThreads) void swiglu_bwd_kernel(const uint16_t *__restrict__ z,
                                                                   const uint16_t *__restrict__ da, int64_t M, int64_t H,
                                                                   int64_t sz, int64_t sda, uint16_t *__restrict__ dz,
                                                                   int64_t sdz, uint32_t *__restrict__ partial) {
  const int64_t units = H / 8;
  uint32_t m = 0;
  for (int64_t r = blockIdx.x; r < M; r += gridDim.x) {
    const uint16_t *zr = z + r * sz;
    for (int64_t u = threadIdx.x; u < units; u += blockDim.x) {
      u32x4 z1v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + 8 * u));
      u32x4 z2v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + H + 8 * u));
      u32x4 dav = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(da + r * sda + 8 * u));
      const uint32_t w1[4] = {z1v.x, z1v.y, z1v.z, z1v.w}, w2[4] = {z2v.x, z2v.y, z2v.z, z2v.w},
                     wd[4] = {dav.x, dav.y, dav.z, dav.w};
      uint32_t o1[4], o2[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        uint32_t h1[2], h2[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
          const float z1 = j ? bf16_hi(w1[i]) : bf16_lo(w1[i]);
          const float z2 = j ? bf16_hi(w2[i]) : bf16_lo(w2[i]);
          const float dv = j ? bf16_hi(wd[i]) : bf16_lo(wd[i]);
          const float sg = sigmoid(z1);
          const float sl = bf16_round(z1 * sg);
          const float t1 = 1.0f - sg;
          const float t2 = z1 * t1;
          const float t3 = 1.0f + t2;
          const float g = sg * t3;
          const float pr = dv * z2;
          h1[j] = bf16_rne(pr * g);
          h2[j] = bf16_rne(dv * sl);
          m = max(m, absbits_nonan(__uint_as_float(h1[j] << 16)));
          m = max(m, absbits_nonan(__uint_as_float(h2[j] << 16)));
        }
        o1[i] = h1[0] | (h1[1] << 16);
        o2[i] = h2[0] | (h2[1] << 16);
      }
      *reinterpret_cast<u32x4 *>(dz + r * sdz + 8 * u) = u32x4{o1[0], o1[1], o1[2], o1[3]};
      *reinterpret_cast<u32x4 *>(dz + r * sdz + H + 8 * u) = u32x4{o2[0], o2[1], o2[2], o2[3]};
    }
  }
  m = block_max_u32(m);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// ------------------------------------------------------------------------------------------- host side

static inline int grid_for(int64_t units, int cap) {
  int64_t g = (units + kCastThreads - 1) / kCastThreads;
  return (int)(g < 1 ? 1 : (g > cap ? cap : g));
}

template <typename T>
static int launch_tcast(const T *x, int64_t n, uint8_t *q, float *dequant, uint32_t *partial, hipStream_t st) {
  const int64_t units = n / 16;
  const int ga = grid_for((units + 3) / 4, kMaxParts);
  amax_kernel<T><<<ga, kCastThreads, 0, st>>>(x, n, partial);
  const int gc = grid_for(units, kMaxCastBlocks);
  cast_kernel<T><<<gc, kCastThreads, 0, st>>>(x, n, partial, ga, q, dequant);
  return (int)hipGetLastError();
}

template <class Src>
static void launch_cast_t(Src src, int64_t rows, int64_t cols, int nparts, uint8_t *q, int64_t ldq, uint8_t *qt,
                          int64_t ldt, float *dequant, const uint32_t *partial, hipStream_t st) {
  dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((ldt + 63) / 64));
  cast_t_kernel<Src><<<grid, 256, 0, st>>>(src, rows, cols, partial, nparts, q, ldq, qt, ldt, dequant);
}

static inline int swiglu_grid(int64_t M) { return (int)(M < 1 ? 1 : (M > kMaxParts ? kMaxParts : M)); }

}  // namespace gpic

using namespace gpic;

extern "C" {

size_t gpic_fp8_cast_workspace_bytes(void) { return kCastWorkspaceBytes; }

int gpic_fp8_tcast(const void *x, int dtype, int64_t n, uint8_t *q, float *dequant, void *ws, void *stream) {
  if (n < 0 || !dequant || !ws || (n > 0 && (!x || !q))) return GPIC_EINVAL;
  if (dtype != GPIC_DTYPE_BF16 && dtype != GPIC_DTYPE_F32) return GPIC_EDTYPE;
  if (!aligned16(x) || !aligned16(q) || !aligned16(ws)) return GPIC_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  uint32_t *partial = static_cast<uint32_t *>(ws);
  if (dtype == GPIC_DTYPE_BF16) return launch_tcast(static_cast<const uint16_t *>(x), n, q, dequant, partial, st);
  return launch_tcast(static_cast<const float *>(x), n, q, dequant, partial, st);
}

int gpic_fp8_tcast_t(const void *x, int dtype, int64_t rows, int64_t cols, uint8_t *q, uint8_t *qt, int64_t ldt,
                     float *dequant, void *ws, void *stream) {
  if (rows < 0 || cols < 0 || !dequant || !ws || (rows > 0 && cols > 0 && !x) || (cols > 0 && ldt > 0 && !qt))
    return GPIC_EINVAL;
  if (cols % 16 != 0 || ldt % 16 != 0 || ldt < rows) return GPIC_ESHAPE;
  if (dtype != GPIC_DTYPE_BF16 && dtype != GPIC_DTYPE_F32) return GPIC_EDTYPE;
  if (!aligned16(x) || (q && !aligned16(q)) || !aligned16(qt) || !aligned16(ws)) return GPIC_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  uint32_t *partial = static_cast<uint32_t *>(ws);
  const int64_t n = rows * cols;
  const int ga = grid_for((n / 16 + 3) / 4, kMaxParts);
  if (dtype == GPIC_DTYPE_BF16)
    amax_kernel<uint16_t><<<ga, kCastThreads, 0, st>>>(static_cast<const uint16_t *>(x), n, partial);
  else
    amax_kernel<float><<<ga, kCastThreads, 0, st>>>(static_cast<const float *>(x), n, partial);
  if (cols == 0 || ldt == 0) {  // nothing to write but the scale (the amax of an empty tensor is 0)
    cast_kernel<uint16_t><<<1, kCastThreads, 0, st>>>(nullptr, 0, partial, ga, nullptr, dequant);
  } else if (dtype == GPIC_DTYPE_BF16) {
    launch_cast_t(SrcBF16{static_cast<const uint16_t *>(x), cols}, rows, cols, ga, q, cols, qt, ldt, dequant, partial,
                  st);
  } else {
    launch_cast_t(SrcF32{static_cast<const float *>(x), cols}, rows, cols, ga, q, cols, qt, ldt, dequant, partial, st);
  }
  return (int)hipGetLastError();
}

int gpic_fp8_swiglu_tcast(const uint16_t *z, int64_t M, int64_t H, int64_t sz, uint8_t *q, int64_t sq, float *dequant,
                          void *ws, void *stream) {
  if (M < 0 || H < 0 || !dequant || !ws || (M > 0 && H > 0 && (!z || !q))) return GPIC_EINVAL;
  if (H % 8 != 0 || sz % 8 != 0 || sq % 8 != 0 || sz < 2 * H || sq < H) return GPIC_ESHAPE;
  if (!aligned16(z) || !aligned16(q) || !aligned16(ws)) return GPIC_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  uint32_t *partial = static_cast<uint32_t *>(ws);
  const int g = swiglu_grid(M);
  swiglu_amax_kernel<<<g, kCastThreads, 0, st>>>(z, M, H, sz, partial);
  swiglu_cast_kernel<<<g, kCastThreads, 0, st>>>(z, M, H, sz, partial, g, q, sq, dequant);
  return (int)hipGetLastError();
}

int gpic_fp8_swiglu_tcast_t(const uint16_t *z, int64_t M, int64_t H, int64_t sz, uint8_t *q, int64_t sq, uint8_t *qt,
                            int64_t ldt, float *dequant, void *ws, void *stream) {
  if (M < 0 || H < 0 || !dequant || !ws || (M > 0 && H > 0 && (!z || !q)) || (H > 0 && ldt > 0 && !qt))
    return GPIC_EINVAL;
  if (H % 16 != 0 || sz % 8 != 0 || sq % 8 != 0 || sz < 2 * H || sq < H || ldt % 16 != 0 || ldt < M)
    return GPIC_ESHAPE;
  if (!aligned16(z) || !aligned16(q) || !aligned16(qt) || !aligned16(ws)) return GPIC_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  uint32_t *partial = static_cast<uint32_t *>(ws);
  const int g = swiglu_grid(M);
  swiglu_amax_kernel<<<g, kCastThreads, 0, st>>>(z, M, H, sz, partial);
  if (H == 0 || ldt == 0)
    cast_kernel<uint16_t><<<1, kCastThreads, 0, st>>>(nullptr, 0, partial, g, nullptr, dequant);
  else
    launch_cast_t(SrcSwiGLU{z, sz, H}, M, H, g, q, sq, qt, ldt, dequant, partial, st);
  return (int)hipGetLastError();
}

static int swiglu_bwd_common(const uint16_t *z, const uint16_t *da, int64_t M, int64_t H, int64_t sz, int64_t sda,
                             uint16_t *dz, uint8_t *dzq, uint8_t *dzqt, int64_t ldt, float *dequant, void *ws,
                             hipStream_t st) {
  uint32_t *partial = static_cast<uint32_t *>(ws);
  const int g = swiglu_grid(M);
  swiglu_bwd_kernel<<<g, kCastThreads, 0, st>>>(z, da, M, H, sz, sda, dz, 2 * H, partial);
  const int64_t n = M * 2 * H;
  if (dzqt && H > 0 && ldt > 0) {
    launch_cast_t(SrcBF16{dz, 2 * H}, M, 2 * H, g, dzq, 2 * H, dzqt, ldt, dequant, partial, st);
  } else {
    const int gc = grid_for(n / 16, kMaxCastBlocks);
    cast_kernel<uint16_t><<<gc, kCastThreads, 0, st>>>(dz, n, partial, g, dzq, dequant);
  }
  return (int)hipGetLastError();
}

int gpic_fp8_swiglu_bwd(const uint16_t *z, const uint16_t *da, int64_t M, int64_t H, int64_t sz, int64_t sda,
                        uint16_t *dz, uint8_t *dzq, float *dequant, void *ws, void *stream) {
  if (M < 0 || H < 0 || !dequant || !ws || (M > 0 && H > 0 && (!z || !da || !dz || !dzq))) return GPIC_EINVAL;
  if (H % 8 != 0 || sz % 8 != 0 || sda % 8 != 0 || sz < 2 * H || sda < H) return GPIC_ESHAPE;
  if (!aligned16(z) || !aligned16(da) || !aligned16(dz) || !aligned16(dzq) || !aligned16(ws)) return GPIC_EALIGN;
  return swiglu_bwd_common(z, da, M, H, sz, sda, dz, dzq, nullptr, 0, dequant, ws, (hipStream_t)stream);
}

int gpic_fp8_swiglu_bwd_t(const uint16_t *z, const uint16_t *da, int64_t M, int64_t H, int64_t sz, int64_t sda,
                          uint16_t *dz, uint8_t *dzq, uint8_t *dzqt, int64_t ldt, float *dequant, void *ws,
                          void *stream) {
  if (M < 0 || H < 0 || !dequant || !ws || (M > 0 && H > 0 && (!z || !da || !dz || !dzq)) ||
      (H > 0 && ldt > 0 && !dzqt))
    return GPIC_EINVAL;
  if (H % 8 != 0 || sz % 8 != 0 || sda % 8 != 0 || sz < 2 * H || sda < H || ldt % 16 != 0 || ldt < M)
    return GPIC_ESHAPE;
  if (!aligned16(z) || !aligned16(da) || !aligned16(dz) || !aligned16(dzq) || !aligned16(dzqt) || !aligned16(ws))
    return GPIC_EALIGN;
  return swiglu_bwd_common(z, da, M, H, sz, sda, dz, dzq, dzqt, ldt, dequant, ws, (hipStream_t)stream);
}

}  // extern "C"

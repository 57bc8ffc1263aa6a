// Per-tensor current-amax e4m3 casts for gfx950: the flat cast (tcast), the cast with a transposed copy (for the
// dgrad / wgrad operands), the SwiGLU product cast and the SwiGLU backward.
//
// Two designs, chosen per call by size:
//  * Single pass (flat bf16 tensors of at most 100 MiB, fp32 of 48 MiB, transposing bf16 casts of 64 MiB; hybrids up
//    to 8x that; the SwiGLU casts, whose limits are stated with their kernels): ONE launch. Each workgroup holds its
//    share of x on chip, publishes a partial maximum tagged with the call's number, folds every workgroup's partial and
//    casts from what it holds (3 B/elem moved for bf16). The call number lives in the
//    workspace (an epoch word the last workgroup of each call advances), so the workspace carries state from call to
//    call: it is zeroed once when created, and calls that may run at the same time (different streams) need
//    different workspaces. Graph capture is fine: a replayed launch reads the epoch the previous call left.
//  * Two passes (larger tensors, the SwiGLU kernels past their single passes, fp32 transposing casts): two
//    stream-ordered launches,
//      1. an amax pass: each workgroup reduces its share to one partial maximum (|x| bit patterns, NaN ignored) and
//         writes it to partial[blockIdx.x] -- no atomics, so nothing has to be zeroed beforehand;
//      2. a cast pass: each workgroup folds all partials (<= kMaxParts words, served from L2), derives the scale with
//         IEEE division and streams its share: 128-bit loads, 128-bit e4m3 stores.
//    Workgroup 0 of pass 2 writes the dequantization scale. The partials are scratch of the call in the workspace.
#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "gpic_device.h"
#include "gpic_launch.h"
#include "gpic_once.h"

namespace gpic {

constexpr int kUnroll = 4;    // 16-element units per thread in flight in the streaming passes

// ------------------------------------------------------------------------------------------- source maps
//
// The flat casts read output word i (8 bf16 or 4 fp32 elements) from source word map(i). FlatMap: the source is the
// output's shape, contiguous. HeadMap: the attention output o [B, H, N, D] with any strides, cast into the rows of
// [B N, H D] (o.transpose(1, 2).reshape(B N, H D)) -- the head-merging layout change folded into the cast.
struct FlatMap {
  __device__ __forceinline__ int64_t operator()(int64_t i) const { return i; }
  __device__ __forceinline__ uint32_t operator()(uint32_t i) const { return i; }
};

// Division by a divisor d fixed for a launch, for dividends below 2^31: q = (n m) >> (31 + s), s = ceil(log2 d),
// m = ceil(2^(31 + s) / d) < 2^32. Exact: with m d = 2^(31 + s) + e, 0 <= e < d <= 2^s, the error n e / (d 2^(31 + s))
// stays below 1 / d for n < 2^31, so it never carries past the next multiple of d.
struct FastDiv {
  uint32_t d, m, s;
};
static inline FastDiv fast_div(uint32_t d) {
  uint32_t s = 0;
  while ((1ull << s) < d) s++;
  return FastDiv{d, (uint32_t)(((1ull << (31 + s)) + d - 1) / d), s};
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) {
  return (uint32_t)(((uint64_t)n * f.m) >> (31 + f.s));
}

// Output word i = ((b N + n) H + h) D/8 + dw lies at source word b sb + h sh + n sn + dw (strides in 16-byte words;
// the host checks every source word index and the output's word count below 2^31).
struct HeadMap {
  FastDiv dw8, heads, tokens;   // D / 8, H, N
  uint32_t sb, sh, sn;
  __device__ __forceinline__ uint32_t operator()(uint32_t i) const {
    const uint32_t g = fdiv(i, dw8), dw = i - g * dw8.d;   // head row g = (b N + n) H + h
    const uint32_t r = fdiv(g, heads), h = g - r * heads.d;
    const uint32_t b = fdiv(r, tokens), n = r - b * tokens.d;
    return b * sb + h * sh + n * sn + dw;
  }
  __device__ __forceinline__ int64_t operator()(int64_t i) const { return (*this)((uint32_t)i); }
};

// ------------------------------------------------------------------------------------------- pass 1: amax

__device__ __forceinline__ uint32_t absbits_bf16(uint16_t h) { return (uint32_t)(h & 0x7fffu) << 16; }
__device__ __forceinline__ uint32_t absbits_f32(float f) { return __float_as_uint(f) & 0x7fffffffu; }

// Max of |x| over a 16-byte word: packed u16 maxima for bf16 (NaN included; caught by the caller), u32 for fp32.
template <typename T>
__device__ __forceinline__ uint32_t word_max(uint32_t m, u32x4 w) {
  if constexpr (sizeof(T) == 2) {
    m = pk_max_u16(m, w.x & 0x7fff7fffu);
    m = pk_max_u16(m, w.y & 0x7fff7fffu);
    m = pk_max_u16(m, w.z & 0x7fff7fffu);
    return pk_max_u16(m, w.w & 0x7fff7fffu);
  } else {
    const uint32_t a = max(max(w.x & 0x7fffffffu, w.y & 0x7fffffffu), max(w.z & 0x7fffffffu, w.w & 0x7fffffffu));
    return max(m, a);
  }
}

// x: n elements of T (bf16 as uint16_t, or float), 16-byte aligned, read as units of 16 elements (kUnroll units per
// thread per iteration, all loads issued first); the n % 16 tail is read by the first threads of workgroup 0.
// Writes max |x| over the non-NaN elements of this workgroup's share to partial[blockIdx.x].
// kKeep: ordinary loads, which leave x in the MALL for the cast pass (used when x fits it, kMallBytes); otherwise
// non-temporal loads (measured: for x of 192 MiB and more, ordinary loads slow both passes).
// Map: the source of each 16-byte word (a 16-element unit's words are consecutive in the source); the n % 16 tail is
// read flat (HeadMap sources have none).
template <typename T, bool kKeep, class Map = FlatMap>
__global__ __launch_bounds__(kCastThreads) void amax_kernel(const T *__restrict__ x, int64_t n,
                                                             uint32_t *__restrict__ partial, const Map map = Map()) {
  constexpr int kWords = sizeof(T);   // 16-byte words per 16-element unit: 2 (bf16) or 4 (fp32)
  const int64_t units = n / 16;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const u32x4 *xv = reinterpret_cast<const u32x4 *>(x);
  uint32_t m = 0;
  int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; u + (kUnroll - 1) * stride < units; u += kUnroll * stride) {
    u32x4 w[kUnroll][kWords];
#pragma unroll
    for (int k = 0; k < kUnroll; k++)
#pragma unroll
      for (int i = 0; i < kWords; i++) {
        const u32x4 *p = xv + map((u + k * stride) * kWords) + i;
        w[k][i] = kKeep ? *p : __builtin_nontemporal_load(p);
      }
#pragma unroll
    for (int k = 0; k < kUnroll; k++)
#pragma unroll
      for (int i = 0; i < kWords; i++) m = word_max<T>(m, w[k][i]);
  }
  for (; u < units; u += stride)
#pragma unroll
    for (int i = 0; i < kWords; i++) m = word_max<T>(m, __builtin_nontemporal_load(xv + map(u * kWords) + i));
  bool nan;
  if constexpr (sizeof(T) == 2) {
    m = max(m & 0xffffu, m >> 16);
    nan = m > 0x7f80u;
    m <<= 16;
  } else {
    nan = m > 0x7f800000u;
  }
  if (nan) {  // rare: this thread saw a NaN; fold its elements again without them (tl.max is maxnum)
    m = 0;
    for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < units; v += stride)
      for (int i = 0; i < 16; i++) {
        const u32x4 *p = xv + map(v * kWords);
        const uint32_t a = sizeof(T) == 2 ? absbits_bf16(reinterpret_cast<const uint16_t *>(p)[i])
                                          : absbits_f32(reinterpret_cast<const float *>(p)[i]);
        if (a <= 0x7f800000u) m = max(m, a);
      }
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 15)) {
    const int64_t i = units * 16 + threadIdx.x;
    const uint32_t a = sizeof(T) == 2 ? absbits_bf16(reinterpret_cast<const uint16_t *>(x)[i])
                                      : absbits_f32(reinterpret_cast<const float *>(x)[i]);
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
__device__ __forceinline__ u32x4 cast_unit(const u32x4 (&w)[sizeof(T)], float scale) {
  if constexpr (sizeof(T) == 2) {
    const u32x2 a = cast8_bf16(w[0], scale), b = cast8_bf16(w[1], scale);
    return u32x4{a.x, a.y, b.x, b.y};
  } else {
    return u32x4{cast4_f32(w[0], scale), cast4_f32(w[1], scale), cast4_f32(w[2], scale), cast4_f32(w[3], scale)};
  }
}

template <typename T, class Map = FlatMap>
__global__ __launch_bounds__(kCastThreads) void cast_kernel(const T *__restrict__ x, int64_t n,
                                                             const uint32_t *__restrict__ partial, int nparts,
                                                             uint8_t *__restrict__ q, float *__restrict__ dequant,
                                                             const Map map = Map()) {
  constexpr int kWords = sizeof(T);
  float scale, deq;
  scales_from_amax(fold_partials(partial, nparts), scale, deq);
  if (blockIdx.x == 0 && threadIdx.x == 0) *dequant = deq;
  const int64_t units = n / 16;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const u32x4 *xv = reinterpret_cast<const u32x4 *>(x);
  u32x4 *qv = reinterpret_cast<u32x4 *>(q);
  int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; u + (kUnroll - 1) * stride < units; u += kUnroll * stride) {
    u32x4 w[kUnroll][kWords];
#pragma unroll
    for (int k = 0; k < kUnroll; k++)
#pragma unroll
      for (int i = 0; i < kWords; i++) w[k][i] = __builtin_nontemporal_load(xv + map((u + k * stride) * kWords) + i);
#pragma unroll
    for (int k = 0; k < kUnroll; k++) __builtin_nontemporal_store(cast_unit<T>(w[k], scale), qv + u + k * stride);
  }
  for (; u < units; u += stride) {
    u32x4 w[kWords];
#pragma unroll
    for (int i = 0; i < kWords; i++) w[i] = __builtin_nontemporal_load(xv + map(u * kWords) + i);
    __builtin_nontemporal_store(cast_unit<T>(w, scale), qv + u);
  }
  if (blockIdx.x == 0 && threadIdx.x < (n & 15)) {
    const int64_t i = units * 16 + threadIdx.x;
    const float v = sizeof(T) == 2 ? bf16_lo(reinterpret_cast<const uint16_t *>(x)[i])
                                   : reinterpret_cast<const float *>(x)[i];
    q[i] = (uint8_t)e4m3x4(sat(v * scale), 0.f, 0.f, 0.f);
  }
}

// ------------------------------------------------------------------------------------------- SwiGLU sigmoid table

// sigmoid(z1) for the bf16 values z1 with exponent field in [kLutELo, kLutEHi], i.e. 2^-16 <= |z1| < 2^8, both signs
// (6144 floats = 24 KiB of LDS). Each workgroup fills its table with the same sigmoid() the other values use, so a
// lookup returns exactly what the computation would; values outside the range (rare: tiny, huge, zero, NaN) are
// computed directly. Entry r holds the value whose bf16 bits, rotated left by one (sign to bit 0), are
// r + (kLutELo << 8): the index of a value is then a 16-bit rotate, subtract and clamp, done for both halves of a
// 32-bit word of bf16 at once with packed 16-bit instructions. The clamp sends values outside the table to entry
// kLutSize, which the LDS copy holds as -1 (no sigmoid is negative): that marks them for direct computation.
constexpr int kLutELo = 111, kLutEHi = 134;
constexpr int kLutHalf = (kLutEHi - kLutELo + 1) * 128;
constexpr int kLutSize = 2 * kLutHalf;
constexpr int kLutLds = kLutSize + 4;   // LDS copy: the table, the sentinel, padding
static_assert(kMaxParts * 4 + kLutSize * 4 <= (int)kCastWorkspaceBytes, "cast workspace too small");
static_assert((kLutELo << 8) + kLutSize <= 0x10000, "table indices are 16-bit");

// The workspace: partial maxima at the start, the sigmoid table after them.
__host__ __device__ inline float *ws_table(void *ws) { return reinterpret_cast<float *>((char *)ws + kMaxParts * 4); }

__device__ __forceinline__ void lut_build(float *lut) {
  for (int i = threadIdx.x; i < kLutSize; i += blockDim.x) {
    const uint32_t h = (uint32_t)(i + (kLutELo << 8));        // rotated bits
    lut[i] = sigmoid(bf16_lo((h >> 1) | ((h & 1u) << 15)));
  }
  if (threadIdx.x == 0) lut[kLutSize] = -1.0f;
  __syncthreads();
}

// The same table copied from global memory (written by an earlier pass of the same call).
__device__ __forceinline__ void lut_load(float *lut, const float *__restrict__ g) {
  for (int i = threadIdx.x; i < kLutSize / 4; i += blockDim.x)
    reinterpret_cast<u32x4 *>(lut)[i] = reinterpret_cast<const u32x4 *>(g)[i];
  if (threadIdx.x == 0) lut[kLutSize] = -1.0f;
  __syncthreads();
}

// Eight sigmoids of the eight bf16 values of a 16-byte word; z holds their fp32 values.
__device__ __forceinline__ void sigmoid8(const float *lut, u32x4 w, const float (&z)[8], float (&sg)[8]) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  bool slow = false;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    u16x2 h = __builtin_bit_cast(u16x2, ws[j]);
    h = (h << (uint16_t)1) | (h >> (uint16_t)15);
    h = h - (uint16_t)(kLutELo << 8);                            // below the table wraps high
    h = __builtin_elementwise_min(h, (u16x2)(uint16_t)kLutSize);  // past it: the sentinel
    const uint32_t r = __builtin_bit_cast(uint32_t, h);
    sg[2 * j] = lut[r & 0xffffu];
    sg[2 * j + 1] = lut[r >> 16];
  }
#pragma unroll
  for (int i = 0; i < 8; i++) slow |= sg[i] < 0.0f;
  if (slow) {
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (sg[i] < 0.0f) sg[i] = sigmoid(z[i]);
  }
}

__device__ __forceinline__ void unpack8(u32x4 w, float (&v)[8]) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    v[2 * i] = bf16_lo(ws[i]);
    v[2 * i + 1] = bf16_hi(ws[i]);
  }
}

// a = bf16(bf16(z1 * sigmoid(z1)) * z2) for 8 pairs (fp8_native.py:55-58) as 4 words of packed bf16 (each
// rounding done for two values by one v_cvt_pk_bf16_f32).
__device__ __forceinline__ u32x4 swiglu8_words(const float *lut, u32x4 z1w, u32x4 z2w) {
  float z1[8], z2[8], sg[8];
  unpack8(z1w, z1);
  unpack8(z2w, z2);
  sigmoid8(lut, z1w, z1, sg);
  u32x4 a;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t sl = pack_bf16(z1[2 * j] * sg[2 * j], z1[2 * j + 1] * sg[2 * j + 1]);
    a[j] = pack_bf16(bf16_lo(sl) * z2[2 * j], bf16_hi(sl) * z2[2 * j + 1]);
  }
  return a;
}

// The same as exact bf16 values in fp32.
__device__ __forceinline__ void swiglu8(const float *lut, u32x4 z1w, u32x4 z2w, float (&a)[8]) {
  unpack8(swiglu8_words(lut, z1w, z2w), a);
}

__device__ __forceinline__ uint32_t absbits_nonan(float v) {
  const uint32_t a = __float_as_uint(v) & 0x7fffffffu;
  return a > 0x7f800000u ? 0u : a;
}

// ------------------------------------------------------------------------------------------- pass 2: cast + transpose

// Sources of the transposing cast: 8 consecutive elements (row r, columns c..c+7) as fp32.
struct SrcBF16 {
  static constexpr bool kLut = false;
  const uint16_t *x;
  int64_t ld;
  __device__ __forceinline__ void load8(int64_t r, int64_t c, float (&v)[8], const float *) const {
    unpack8(*reinterpret_cast<const u32x4 *>(x + r * ld + c), v);
  }
};

struct SrcF32 {
  static constexpr bool kLut = false;
  const float *x;
  int64_t ld;
  __device__ __forceinline__ void load8(int64_t r, int64_t c, float (&v)[8], const float *) const {
    const u32x4 w0 = *reinterpret_cast<const u32x4 *>(x + r * ld + c);
    const u32x4 w1 = *reinterpret_cast<const u32x4 *>(x + r * ld + c + 4);
    v[0] = __uint_as_float(w0.x), v[1] = __uint_as_float(w0.y), v[2] = __uint_as_float(w0.z);
    v[3] = __uint_as_float(w0.w), v[4] = __uint_as_float(w1.x), v[5] = __uint_as_float(w1.y);
    v[6] = __uint_as_float(w1.z), v[7] = __uint_as_float(w1.w);
  }
};

// The SwiGLU product a of z [M, 2H] (row stride sz), as a source of H columns.
struct SrcSwiGLU {
  static constexpr bool kLut = true;
  const uint16_t *z;
  int64_t sz, H;
  const float *table;   // the sigmoid table the amax pass of this call wrote
  __device__ __forceinline__ void load8(int64_t r, int64_t c, float (&v)[8], const float *lut) const {
    const u32x4 z1 = *reinterpret_cast<const u32x4 *>(z + r * sz + c);
    const u32x4 z2 = *reinterpret_cast<const u32x4 *>(z + r * sz + H + c);
    swiglu8(lut, z1, z2, v);
  }
};
// The z1 half of dz for one element (fp8_native.py:88-96), before its bf16 rounding: da * z2 * sg * (1 + z1 * (1 - sg)),
// each operation rounded on its own (the z2 half, da * bf16(z1 * sg), is formed in dz_words).
__device__ __forceinline__ float dz1_of(float z1, float z2, float dv, float sg) {
  const float t1 = 1.0f - sg;
  const float t2 = z1 * t1;
  const float t3 = 1.0f + t2;
  const float g = sg * t3;
  const float pr = dv * z2;
  return pr * g;
}


// src [rows, cols] (cols % 8 == 0) -> q [rows, cols] (row stride ldq; skipped when q == nullptr) and the transposed
// bytes qt [cols, ldt] (ldt % 16 == 0, ldt >= rows), whose columns rows..ldt-1 are written as zeros so a GEMM can
// reduce over the padded length. Tile: 128 rows x 128 columns per workgroup of 256 threads, so both outputs are
// stored as whole 128-byte lines (q: 16 lanes x 8 bytes per row; qt: 8 lanes x 16 bytes per row); the transpose goes
// through LDS. Each thread has its 8 loads in flight at once. The scale comes from the partial maxima of the
// matching amax pass.
constexpr int kTT = 128;   // transposing tile side

template <class Src>
__global__ __launch_bounds__(256) void cast_t_kernel(Src src, int64_t rows, int64_t cols,
                                                      const uint32_t *__restrict__ partial, int nparts,
                                                      uint8_t *__restrict__ q, int64_t ldq, uint8_t *__restrict__ qt,
                                                      int64_t ldt, float *__restrict__ dequant) {
  constexpr int kPitch = kTT / 4 + 1;          // words per LDS row (one word of padding)
  __shared__ uint32_t tile[kTT * kPitch];      // [row][col / 4] e4m3 bytes
  const float *lut = nullptr;
  if constexpr (Src::kLut) {
    __shared__ float table[kLutLds];
    lut_load(table, src.table);
    lut = table;
  }
  // The persistent (SwiGLU) workgroups fold the partial maxima once; the one-tile workgroups fold them after
  // issuing their tile's loads, so the two latencies overlap (the fold's barriers wait for LDS only).
  float scale = 0.0f, deq = 0.0f;
  if constexpr (Src::kLut) scales_from_amax(fold_partials(partial, nparts), scale, deq);
  const int64_t tiles_c = (cols + kTT - 1) / kTT, tiles = tiles_c * ((ldt + kTT - 1) / kTT);
  constexpr int kPer = kTT * (kTT / 8) / 256;  // 8-element chunks per thread per tile: 8
  // The SwiGLU source walks tiles (persistent workgroups); the others take exactly one tile each.
  const int64_t tstep = Src::kLut ? (int64_t)gridDim.x : tiles;
  for (int64_t t = blockIdx.x; t < tiles; t += tstep) {   // tiles walked column-block fastest
    const int64_t tr = tiles - 1 - t;   // reverse order: see cast_t_bf16_kernel
    const int64_t c0 = (tr % tiles_c) * kTT, r0 = (tr / tiles_c) * kTT;
    float v[kPer][8];
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int id = threadIdx.x + 256 * i;
      const int r = id >> 4, cc = id & 15;
      const int64_t gr = r0 + r, gc = c0 + 8 * cc;
      if (gr < rows && gc < cols) src.load8(gr, gc, v[i], lut);
    }
    if constexpr (!Src::kLut) scales_from_amax(fold_partials(partial, nparts), scale, deq);
#pragma unroll
    for (int i = 0; i < kPer; i++) {
      const int id = threadIdx.x + 256 * i;
      const int r = id >> 4, cc = id & 15;
      const int64_t gr = r0 + r, gc = c0 + 8 * cc;
      u32x2 o = {0u, 0u};
      if (gr < rows && gc < cols) {
        o.x = e4m3x4(sat(v[i][0] * scale), sat(v[i][1] * scale), sat(v[i][2] * scale), sat(v[i][3] * scale));
        o.y = e4m3x4(sat(v[i][4] * scale), sat(v[i][5] * scale), sat(v[i][6] * scale), sat(v[i][7] * scale));
        if (q) *reinterpret_cast<u32x2 *>(q + gr * ldq + gc) = o;
      }
      tile[r * kPitch + 2 * cc] = o.x;
      tile[r * kPitch + 2 * cc + 1] = o.y;
    }
    lds_barrier();
    // qt rows c0 + 4k .. c0 + 4k + 3 get bytes r0 + 16p .. r0 + 16p + 15 of their columns, k = tid / 8, p = tid % 8:
    // four 4 x 4 byte blocks (rows 16p + 4g .. + 3, word k of the tile) transposed with v_perm_b32. Eight lanes
    // write the 128 bytes of one qt row chunk.
    {
      const int k = threadIdx.x >> 3, p = threadIdx.x & 7;
      u32x4 out[4];
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const uint32_t *w = tile + (16 * p + 4 * g) * kPitch + k;
        const uint32_t w0 = w[0], w1 = w[kPitch], w2 = w[2 * kPitch], w3 = w[3 * kPitch];
        const uint32_t lo01 = __builtin_amdgcn_perm(w1, w0, 0x05010400u);   // w0.b0 w1.b0 w0.b1 w1.b1
        const uint32_t hi01 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);   // w0.b2 w1.b2 w0.b3 w1.b3
        const uint32_t lo23 = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
        const uint32_t hi23 = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
        out[0][g] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);         // byte 0 of w0..w3
        out[1][g] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);         // byte 1
        out[2][g] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);         // byte 2
        out[3][g] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);         // byte 3
      }
      const int64_t gr = r0 + 16 * p;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int64_t gc = c0 + 4 * k + j;
        if (gc < cols && gr < ldt) *reinterpret_cast<u32x4 *>(qt + gc * ldt + gr) = out[j];
      }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0 && t == 0) *dequant = deq;
    if constexpr (!Src::kLut) break;
    lds_barrier();   // the tile buffer is rewritten by the next tile
  }
}

// ------------------------------------------------------------------------------------------- SwiGLU kernels

// z [M, 2H] bf16 (row stride sz, H % 8 == 0): rows strided over workgroups (kRowsPer rows at a time, all their
// loads issued first), 8-element units over threads. Workgroup 0 also publishes its sigmoid table to `table` for the
// cast pass of the same call.
constexpr int kRowsPer = 4;

// Partial maxima of the SwiGLU product a; when `a` is given, also writes a ([M, H] bf16, contiguous; its values are
// bf16 already, so the write is exact) for a cast that then reads it instead of recomputing it. The maximum is taken
// on the packed bf16 magnitudes (one v_pk_max_u16 per two values); a thread whose maximum is a NaN pattern folds its
// rows again element by element without the NaNs (tl.max is maxnum).
__global__ __launch_bounds__(kCastThreads) void swiglu_amax_kernel(const uint16_t *__restrict__ z, int64_t M, int64_t H,
                                                                    int64_t sz, uint32_t *__restrict__ partial,
                                                                    float *__restrict__ table, uint16_t *__restrict__ a) {
  __shared__ float lut[kLutLds];
  lut_build(lut);
  if (blockIdx.x == 0 && table)
    for (int i = threadIdx.x; i < kLutSize; i += blockDim.x) table[i] = lut[i];
  const int64_t units = H / 8;
  const int64_t rstride = gridDim.x;
  uint32_t m16 = 0;   // packed maxima of |bf16 a| (NaN patterns included)
  auto unit = [&](int64_t r, int64_t u, u32x4 z1, u32x4 z2) {
    const u32x4 aw = swiglu8_words(lut, z1, z2);
#pragma unroll
    for (int j = 0; j < 4; j++) m16 = pk_max_u16(m16, aw[j] & 0x7fff7fffu);
    if (a) *reinterpret_cast<u32x4 *>(a + r * H + 8 * u) = aw;
  };
  for (int64_t u = threadIdx.x; u < units; u += blockDim.x) {
    int64_t r = blockIdx.x;
    for (; r + (kRowsPer - 1) * rstride < M; r += kRowsPer * rstride) {
      u32x4 z1[kRowsPer], z2[kRowsPer];
#pragma unroll
      for (int k = 0; k < kRowsPer; k++) {
        const uint16_t *zr = z + (r + k * rstride) * sz;
        z1[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + 8 * u));
        z2[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + H + 8 * u));
      }
#pragma unroll
      for (int k = 0; k < kRowsPer; k++) unit(r + k * rstride, u, z1[k], z2[k]);
    }
    for (; r < M; r += rstride) {
      const uint16_t *zr = z + r * sz;
      unit(r, u, __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + 8 * u)),
           __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + H + 8 * u)));
    }
  }
  uint32_t m = max(m16 & 0xffffu, m16 >> 16);
  if (m > 0x7f80u) {   // rare: a NaN among this thread's products; fold them again without it
    m = 0;
    for (int64_t u = threadIdx.x; u < units; u += blockDim.x)
      for (int64_t r = blockIdx.x; r < M; r += rstride) {
        const uint16_t *zr = z + r * sz;
        float v[8];
        swiglu8(lut, *reinterpret_cast<const u32x4 *>(zr + 8 * u), *reinterpret_cast<const u32x4 *>(zr + H + 8 * u), v);
#pragma unroll
        for (int i = 0; i < 8; i++) m = max(m, absbits_nonan(v[i]));
      }
  } else {
    m <<= 16;
  }
  m = block_max_u32(m);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

__global__ __launch_bounds__(kCastThreads) void swiglu_cast_kernel(const uint16_t *__restrict__ z, int64_t M, int64_t H,
                                                                    int64_t sz, const uint32_t *__restrict__ partial,
                                                                    int nparts, uint8_t *__restrict__ q, int64_t sq,
                                                                    float *__restrict__ dequant,
                                                                    const float *__restrict__ table) {
  __shared__ float lut[kLutLds];
  lut_load(lut, table);
  float scale, deq;
  scales_from_amax(fold_partials(partial, nparts), scale, deq);
  if (blockIdx.x == 0 && threadIdx.x == 0) *dequant = deq;
  const int64_t units = H / 8;
  for (int64_t r = blockIdx.x; r < M; r += gridDim.x) {
    const uint16_t *zr = z + r * sz;
    for (int64_t u = threadIdx.x; u < units; u += blockDim.x) {
      const u32x4 z1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + 8 * u));
      const u32x4 z2 = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + H + 8 * u));
      float a[8];
      swiglu8(lut, z1, z2, a);
      u32x2 o;
      o.x = e4m3x4(sat(a[0] * scale), sat(a[1] * scale), sat(a[2] * scale), sat(a[3] * scale));
      o.y = e4m3x4(sat(a[4] * scale), sat(a[5] * scale), sat(a[6] * scale), sat(a[7] * scale));
      *reinterpret_cast<u32x2 *>(q + r * sq + 8 * u) = o;
    }
  }
}

// dz = [d1 | d2] (fp8_native.py:88-96), each operation rounded on its own, left to right:
//   sg = sigmoid(z1); sl = bf16(z1 * sg); d1 = bf16((da * z2) * (sg * (1 + z1 * (1 - sg)))); d2 = bf16(da * sl)
// for the 8 elements of one 16-byte word of z1, z2 and da: h1, h2 are the bf16 words of d1 and d2.
__device__ __forceinline__ void dz_words(const float *lut, u32x4 z1v, u32x4 z2v, u32x4 dav, u32x4 &h1, u32x4 &h2) {
  float z1[8], z2[8], dv[8], sg[8];
  unpack8(z1v, z1);
  unpack8(z2v, z2);
  unpack8(dav, dv);
  sigmoid8(lut, z1v, z1, sg);
  float d1[8], d2[8];
#pragma unroll
  for (int i = 0; i < 8; i++) d1[i] = dz1_of(z1[i], z2[i], dv[i], sg[i]);
#pragma unroll
  for (int j = 0; j < 4; j++) {   // d2 = da * bf16(z1 * sg), the roundings of two values by one instruction
    const uint32_t sl = pack_bf16(z1[2 * j] * sg[2 * j], z1[2 * j + 1] * sg[2 * j + 1]);
    d2[2 * j] = dv[2 * j] * bf16_lo(sl);
    d2[2 * j + 1] = dv[2 * j + 1] * bf16_hi(sl);
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    h1[j] = pack_bf16(d1[2 * j], d1[2 * j + 1]);
    h2[j] = pack_bf16(d2[2 * j], d2[2 * j + 1]);
  }
}

// dz = [dz1 | dz2] (written when kStore) and the partial maxima of its bf16 values; workgroup 0 also publishes its
// sigmoid table to `table` (when given) for a later pass of the same call. Rows are strided over workgroups. Without
// stores, kRowsPer rows at a time with all their loads issued first (the dz arithmetic, ~30 VALU operations per
// element, needs several rows of loads in flight: 8% faster); with stores, one row at a time (measured faster: the
// batched stores of four rows slowed it by 7%). The maximum is taken on packed 16-bit magnitudes; a thread whose
// maximum is a NaN pattern folds its rows again element by element without them.
template <bool kStore>
__global__ __launch_bounds__(kCastThreads) void swiglu_bwd_kernel(const uint16_t *__restrict__ z,
                                                                   const uint16_t *__restrict__ da, int64_t M, int64_t H,
                                                                   int64_t sz, int64_t sda, uint16_t *__restrict__ dz,
                                                                   int64_t sdz, uint32_t *__restrict__ partial,
                                                                   float *__restrict__ table) {
  __shared__ float lut[kLutLds];
  lut_build(lut);
  if (blockIdx.x == 0 && table)
    for (int i = threadIdx.x; i < kLutSize; i += blockDim.x) table[i] = lut[i];
  const int64_t units = H / 8;
  const int64_t rstride = gridDim.x;
  auto unit = [&](int64_t r, int64_t u, u32x4 &h1, u32x4 &h2) {
    const uint16_t *zr = z + r * sz + 8 * u;
    dz_words(lut, __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr)),
             __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + H)),
             __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(da + r * sda + 8 * u)), h1, h2);
  };
  auto store = [&](int64_t r, int64_t u, u32x4 h1, u32x4 h2) {
    if constexpr (kStore) {
      *reinterpret_cast<u32x4 *>(dz + r * sdz + 8 * u) = h1;
      *reinterpret_cast<u32x4 *>(dz + r * sdz + H + 8 * u) = h2;
    }
  };
  uint32_t m16 = 0;   // packed maxima of |bf16| (NaN patterns included)
  auto fold = [&](u32x4 h1, u32x4 h2) {
#pragma unroll
    for (int j = 0; j < 4; j++) m16 = pk_max_u16(pk_max_u16(m16, h1[j] & 0x7fff7fffu), h2[j] & 0x7fff7fffu);
  };
  for (int64_t u = threadIdx.x; u < units; u += blockDim.x) {
    int64_t r = blockIdx.x;
    for (; !kStore && r + (kRowsPer - 1) * rstride < M; r += kRowsPer * rstride) {
      u32x4 Z1[kRowsPer], Z2[kRowsPer], D[kRowsPer];
#pragma unroll
      for (int k = 0; k < kRowsPer; k++) {
        const uint16_t *zr = z + (r + k * rstride) * sz + 8 * u;
        Z1[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr));
        Z2[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + H));
        D[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(da + (r + k * rstride) * sda + 8 * u));
      }
#pragma unroll
      for (int k = 0; k < kRowsPer; k++) {
        u32x4 h1, h2;
        dz_words(lut, Z1[k], Z2[k], D[k], h1, h2);
        fold(h1, h2);
        store(r + k * rstride, u, h1, h2);
      }
    }
    for (; r < M; r += rstride) {
      u32x4 h1, h2;
      unit(r, u, h1, h2);
      fold(h1, h2);
      store(r, u, h1, h2);
    }
  }
  uint32_t m = max(m16 & 0xffffu, m16 >> 16);
  if (m > 0x7f80u) {   // rare: a NaN among this thread's dz values; fold them again without it (tl.max is maxnum)
    m = 0;
    for (int64_t u = threadIdx.x; u < units; u += blockDim.x)
      for (int64_t r = blockIdx.x; r < M; r += rstride) {
        u32x4 h1, h2;
        unit(r, u, h1, h2);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          m = max(m, max(absbits_nonan(bf16_lo(h1[j])), absbits_nonan(bf16_hi(h1[j]))));
          m = max(m, max(absbits_nonan(bf16_lo(h2[j])), absbits_nonan(bf16_hi(h2[j]))));
        }
      }
  } else {
    m <<= 16;
  }
  m = block_max_u32(m);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// The flat cast of dz without dz in memory: dz recomputed from z and da (the same bf16 values as swiglu_bwd_kernel)
// and cast to dzq [M, 2H] (contiguous) with the scale from swiglu_bwd_kernel<false>'s partial maxima and its
// sigmoid table. Rows strided over workgroups, walked row-major two rows at a time: each thread has the loads of
// two rows x two units in flight (12 x 16 bytes). Measured on the d12 shape: 18% faster than walking each unit
// down all of the workgroup's rows first (that order left the dzq stores at 4.5 TB/s of combined traffic).
__global__ __launch_bounds__(kCastThreads) void swiglu_bwd_cast_kernel(const uint16_t *__restrict__ z,
                                                                        const uint16_t *__restrict__ da, int64_t M,
                                                                        int64_t H, int64_t sz, int64_t sda,
                                                                        const uint32_t *__restrict__ partial, int nparts,
                                                                        const float *__restrict__ table,
                                                                        uint8_t *__restrict__ dzq,
                                                                        float *__restrict__ dequant) {
  __shared__ float lut[kLutLds];
  lut_load(lut, table);
  float scale, deq;
  scales_from_amax(fold_partials(partial, nparts), scale, deq);
  if (blockIdx.x == 0 && threadIdx.x == 0) *dequant = deq;
  const int64_t units = H / 8;
  const int64_t rstride = gridDim.x;
  auto emit = [&](int64_t r, int64_t u, u32x4 z1, u32x4 z2, u32x4 d) {
    u32x4 h1, h2;
    dz_words(lut, z1, z2, d, h1, h2);
    uint8_t *o = dzq + r * 2 * H + 8 * u;
    __builtin_nontemporal_store(cast8_bf16(h1, scale), reinterpret_cast<u32x2 *>(o));
    __builtin_nontemporal_store(cast8_bf16(h2, scale), reinterpret_cast<u32x2 *>(o + H));
  };
  auto ld = [](const uint16_t *p) { return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p)); };
  int64_t r = blockIdx.x;
  for (; r + rstride < M; r += 2 * rstride) {
    for (int64_t u = threadIdx.x; u < units; u += 2 * blockDim.x) {
      const bool two = u + blockDim.x < units;   // the thread's second unit of the row exists
      u32x4 Z1[4], Z2[4], D[4];                  // k: row r + (k / 2) rstride, unit u + (k % 2) blockDim.x
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int64_t rk = r + (k >> 1) * rstride, uk = u + (k & 1) * blockDim.x;
        const bool ok = (k & 1) == 0 || two;
        const uint16_t *zr = z + rk * sz + 8 * uk;
        Z1[k] = ok ? ld(zr) : u32x4{0u, 0u, 0u, 0u};
        Z2[k] = ok ? ld(zr + H) : u32x4{0u, 0u, 0u, 0u};
        D[k] = ok ? ld(da + rk * sda + 8 * uk) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int k = 0; k < 4; k++)
        if ((k & 1) == 0 || two) emit(r + (k >> 1) * rstride, u + (k & 1) * blockDim.x, Z1[k], Z2[k], D[k]);
    }
  }
  for (; r < M; r += rstride)   // the workgroup's last row when it has an odd count
    for (int64_t u = threadIdx.x; u < units; u += blockDim.x) {
      const uint16_t *zr = z + r * sz + 8 * u;
      emit(r, u, ld(zr), ld(zr + H), ld(da + r * sda + 8 * u));
    }
}

// ------------------------------------------------------------------------------------------- host side

static inline int grid_for(int64_t units, int cap) {
  int64_t g = (units + kCastThreads - 1) / kCastThreads;
  return (int)(g < 1 ? 1 : (g > cap ? cap : g));
}

constexpr int64_t kMallBytes = 128ll << 20;   // x at most this large stays in the 256 MiB MALL between the passes

template <typename T, class Map = FlatMap>
static void launch_amax(const T *x, int64_t n, int grid, uint32_t *partial, hipStream_t st, const Map map = Map()) {
  if (n * (int64_t)sizeof(T) <= kMallBytes) amax_kernel<T, true, Map><<<grid, kCastThreads, 0, st>>>(x, n, partial, map);
  else amax_kernel<T, false, Map><<<grid, kCastThreads, 0, st>>>(x, n, partial, map);
}

template <typename T, class Map = FlatMap>
static int launch_tcast(const T *x, int64_t n, uint8_t *q, float *dequant, uint32_t *partial, hipStream_t st,
                        const Map map = Map()) {
  const int64_t units = n / 16;
  const int ga = grid_for((units + kUnroll - 1) / kUnroll, kAmaxBlocks);
  launch_amax(x, n, ga, partial, st, map);
  const int gc = grid_for((units + kUnroll - 1) / kUnroll, kMaxCastBlocks);
  cast_kernel<T, Map><<<gc, kCastThreads, 0, st>>>(x, n, partial, ga, q, dequant, map);
  return (int)hipGetLastError();
}

template <class Src>
static void launch_cast_t(Src src, int64_t rows, int64_t cols, int nparts, uint8_t *q, int64_t ldq, uint8_t *qt,
                          int64_t ldt, float *dequant, const uint32_t *partial, hipStream_t st) {
  // One tile per workgroup, except for the SwiGLU source: its workgroups copy the 24 KiB sigmoid table first, so
  // they stay resident and walk the tiles.
  const int64_t tiles = ((cols + kTT - 1) / kTT) * ((ldt + kTT - 1) / kTT);
  const int grid = (int)(!Src::kLut || tiles < kCastTBlocks ? tiles : kCastTBlocks);
  cast_t_kernel<Src><<<grid, 256, 0, st>>>(src, rows, cols, partial, nparts, q, ldq, qt, ldt, dequant);
}

// A 128 x 128 bf16 tile (rows r0.., columns c0..) as thread tid's 8 raw chunks: chunk i is row id / 16, columns
// 8 (id % 16) .. + 7 of the tile, id = tid + 256 i; zero outside x.
constexpr int kTPitch = kTT / 4 + 1;            // words per LDS row of the e4m3 tile (one word of padding)
constexpr int kTPer = kTT * (kTT / 8) / 256;    // 8-element chunks per thread per tile: 8
__device__ __forceinline__ void load_tile_bf16(const uint16_t *__restrict__ x, int64_t ld, int64_t rows, int64_t cols,
                                               int64_t r0, int64_t c0, u32x4 (&R)[kTPer]) {
#pragma unroll
  for (int i = 0; i < kTPer; i++) {
    const int id = threadIdx.x + 256 * i;
    const int64_t gr = r0 + (id >> 4), gc = c0 + 8 * (id & 15);
    R[i] = gr < rows && gc < cols ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(x + gr * ld + gc))
                                  : u32x4{0u, 0u, 0u, 0u};
  }
}

// The tile held in R (as load_tile_bf16 left it) as e4m3 bytes with `scale`: 8 bytes per chunk.
__device__ __forceinline__ void cvt_tile_bf16(const u32x4 (&R)[kTPer], float scale, u32x2 (&E)[kTPer]) {
#pragma unroll
  for (int i = 0; i < kTPer; i++) {
    float v[8];
    unpack8(R[i], v);
    E[i].x = e4m3x4(sat(v[0] * scale), sat(v[1] * scale), sat(v[2] * scale), sat(v[3] * scale));
    E[i].y = e4m3x4(sat(v[4] * scale), sat(v[5] * scale), sat(v[6] * scale), sat(v[7] * scale));
  }
}

// Stores a tile's e4m3 bytes E (from cvt_tile_bf16): q rows from registers, qt through the LDS buffer `tile`
// ([row][col / 4] e4m3 words), which is free again when this returns. Same bytes as cast_t_kernel.
__device__ __forceinline__ void emit_tile(const u32x2 (&E)[kTPer], int64_t r0, int64_t c0, int64_t rows, int64_t cols,
                                          uint8_t *__restrict__ q, int64_t ldq, uint8_t *__restrict__ qt, int64_t ldt,
                                          uint32_t *tile) {
#pragma unroll
  for (int i = 0; i < kTPer; i++) {
    const int id = threadIdx.x + 256 * i;
    const int r = id >> 4, cc = id & 15;
    const int64_t gr = r0 + r, gc = c0 + 8 * cc;
    if (q && gr < rows && gc < cols) *reinterpret_cast<u32x2 *>(q + gr * ldq + gc) = E[i];
    tile[r * kTPitch + 2 * cc] = E[i].x;
    tile[r * kTPitch + 2 * cc + 1] = E[i].y;
  }
  lds_barrier();
  // qt rows c0 + 4k .. c0 + 4k + 3 get bytes r0 + 16p .. r0 + 16p + 15 of their columns, k = tid / 8, p = tid % 8
  // (as in cast_t_kernel)
  {
    const int k = threadIdx.x >> 3, p = threadIdx.x & 7;
    u32x4 out[4];
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const uint32_t *w = tile + (16 * p + 4 * g) * kTPitch + k;
      const uint32_t w0 = w[0], w1 = w[kTPitch], w2 = w[2 * kTPitch], w3 = w[3 * kTPitch];
      const uint32_t lo01 = __builtin_amdgcn_perm(w1, w0, 0x05010400u);
      const uint32_t hi01 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);
      const uint32_t lo23 = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
      const uint32_t hi23 = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
      out[0][g] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
      out[1][g] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
      out[2][g] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
      out[3][g] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
    }
    const int64_t gr = r0 + 16 * p;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int64_t gc = c0 + 4 * k + j;
      if (gc < cols && gr < ldt) *reinterpret_cast<u32x4 *>(qt + gc * ldt + gr) = out[j];
    }
  }
  lds_barrier();   // the tile buffer is rewritten by the next tile
}

// The transposing cast of a bf16 source, persistent: each workgroup folds the partial maxima once, then walks its
// tiles, loading the next tile's bf16 (kept raw: 32 VGPRs) while it casts, transposes and stores the current one.
// Same tile layout and bytes as cast_t_kernel. Both transposing kernels walk the tiles last to first: the pass before
// (amax, SwiGLU) streamed x first to last, so the first tiles read here are those most likely still in the MALL
// (measured 2-4% faster for x of 128-512 MiB).
__global__ __launch_bounds__(256) void cast_t_bf16_kernel(const uint16_t *__restrict__ x, int64_t ld, int64_t rows,
                                                          int64_t cols, const uint32_t *__restrict__ partial, int nparts,
                                                          uint8_t *__restrict__ q, int64_t ldq, uint8_t *__restrict__ qt,
                                                          int64_t ldt, float *__restrict__ dequant) {
  __shared__ uint32_t tile[kTT * kTPitch];
  const int64_t tiles_c = (cols + kTT - 1) / kTT, tiles = tiles_c * ((ldt + kTT - 1) / kTT);
  int64_t t = blockIdx.x;   // < tiles: the grid never exceeds the tile count
  u32x4 R[kTPer];
  load_tile_bf16(x, ld, rows, cols, ((tiles - 1 - t) / tiles_c) * kTT, ((tiles - 1 - t) % tiles_c) * kTT, R);
  float scale, deq;
  scales_from_amax(fold_partials(partial, nparts), scale, deq);   // its barriers wait for LDS only
  if (blockIdx.x == 0 && threadIdx.x == 0) *dequant = deq;
  for (; t < tiles; t += gridDim.x) {
    const int64_t tn = t + gridDim.x;
    u32x4 Rn[kTPer];
    if (tn < tiles) {
      load_tile_bf16(x, ld, rows, cols, ((tiles - 1 - tn) / tiles_c) * kTT, ((tiles - 1 - tn) % tiles_c) * kTT, Rn);
    } else {
#pragma unroll
      for (int i = 0; i < kTPer; i++) Rn[i] = u32x4{0u, 0u, 0u, 0u};
    }
    u32x2 E[kTPer];
    cvt_tile_bf16(R, scale, E);
    emit_tile(E, ((tiles - 1 - t) / tiles_c) * kTT, ((tiles - 1 - t) % tiles_c) * kTT, rows, cols, q, ldq, qt, ldt, tile);
#pragma unroll
    for (int i = 0; i < kTPer; i++) R[i] = Rn[i];
  }
}

// The SwiGLU backward's cast without dz in memory: dz is recomputed from z and da (the same bf16 values as
// swiglu_bwd_kernel) tile by tile and cast to dzq [M, 2H] and dzqt [2H, ldt] at once. A tile is 128 rows x 128
// columns h of BOTH halves, so z1, z2 and da are read once for dz1 and dz2; each half leaves through emit_tile. The
// scale comes from the partial maxima of swiglu_bwd_kernel run without dz, which also published the sigmoid table.
// Persistent workgroups (each copies the 24 KiB table once) walk the tiles last to first (the amax pass streamed z
// and da first to last).
__global__ __launch_bounds__(256) void swiglu_bwd_cast_t_kernel(const uint16_t *__restrict__ z,
                                                                const uint16_t *__restrict__ da, int64_t M, int64_t H,
                                                                int64_t sz, int64_t sda,
                                                                const uint32_t *__restrict__ partial, int nparts,
                                                                const float *__restrict__ table, uint8_t *__restrict__ dzq,
                                                                uint8_t *__restrict__ dzqt, int64_t ldt,
                                                                float *__restrict__ dequant) {
  __shared__ float lut[kLutLds];
  __shared__ uint32_t tile[kTT * kTPitch];
  lut_load(lut, table);
  float scale, deq;
  scales_from_amax(fold_partials(partial, nparts), scale, deq);
  if (blockIdx.x == 0 && threadIdx.x == 0) *dequant = deq;
  const int64_t tiles_h = (H + kTT - 1) / kTT, tiles = tiles_h * ((ldt + kTT - 1) / kTT);
  for (int64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
    const int64_t tr = tiles - 1 - t;
    const int64_t r0 = (tr / tiles_h) * kTT, h0 = (tr % tiles_h) * kTT;
    u32x2 E1[kTPer], E2[kTPer];
#pragma unroll
    for (int b = 0; b < kTPer; b += 4) {   // two batches of 4 chunks: 12 loads in flight per thread
      u32x4 Z1[4], Z2[4], D[4];
      bool ok[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int id = threadIdx.x + 256 * (b + i);
        const int64_t gr = r0 + (id >> 4), gh = h0 + 8 * (id & 15);
        ok[i] = gr < M && gh < H;
        const uint16_t *zr = z + gr * sz + gh;
        Z1[i] = ok[i] ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr)) : u32x4{0u, 0u, 0u, 0u};
        Z2[i] = ok[i] ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(zr + H)) : u32x4{0u, 0u, 0u, 0u};
        D[i] = ok[i] ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(da + gr * sda + gh))
                     : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        u32x4 h1, h2;
        dz_words(lut, Z1[i], Z2[i], D[i], h1, h2);
        E1[b + i] = ok[i] ? cast8_bf16(h1, scale) : u32x2{0u, 0u};
        E2[b + i] = ok[i] ? cast8_bf16(h2, scale) : u32x2{0u, 0u};
      }
    }
    emit_tile(E1, r0, h0, M, H, dzq, 2 * H, dzqt, ldt, tile);
    emit_tile(E2, r0, h0, M, H, dzq + H, 2 * H, dzqt + H * ldt, ldt, tile);
  }
}

// bf16 sources take the persistent kernel above up to 8 tiles per workgroup, the one-tile kernel beyond (measured on
// [32768, C]: persistent 7-15% faster for C = 2048..4096, 5% slower for C = 8192)
constexpr int64_t kCastTPersistentTiles = 8 * kCastTBlocks;
static void launch_cast_t(SrcBF16 src, int64_t rows, int64_t cols, int nparts, uint8_t *q, int64_t ldq, uint8_t *qt,
                          int64_t ldt, float *dequant, const uint32_t *partial, hipStream_t st) {
  const int64_t tiles = ((cols + kTT - 1) / kTT) * ((ldt + kTT - 1) / kTT);
  if (tiles > kCastTPersistentTiles) {
    cast_t_kernel<SrcBF16><<<(int)tiles, 256, 0, st>>>(src, rows, cols, partial, nparts, q, ldq, qt, ldt, dequant);
    return;
  }
  const int grid = (int)(tiles < kCastTBlocks ? tiles : kCastTBlocks);
  cast_t_bf16_kernel<<<grid, 256, 0, st>>>(src.x, src.ld, rows, cols, partial, nparts, q, ldq, qt, ldt, dequant);
}


// ------------------------------------------------------------------------------------------- single pass
//
// A tensor that fits in the registers of the whole chip is cast in one launch: each workgroup loads its share into
// registers, reduces it to a partial maximum and publishes it, takes the maximum of all workgroups' partials, and
// casts from its registers. x is read once: 3 B/elem moved for bf16 instead of 5.
//
// The partials' layout and the fold: gpic_once.h.
static_assert(kMaxParts * 4 + kLutSize * 4 <= (int)kOnceTagged, "two-pass scratch overlaps the single-pass words");
template <typename T>
constexpr int kOnceWords = sizeof(T) == 2 ? 16 : 12;   // 16-byte words a thread of the flat kernel holds (fp32: 12,
                                                        // which its wider narrowing code needs to fit 128 VGPRs)
constexpr int kOnceTiles = 2;       // 128 x 128 bf16 tiles a workgroup of the transposing kernel holds (64 VGPRs)
constexpr int kHybridTiles = 8;     // the transposing kernel takes up to this many tiles per workgroup (2 held)
constexpr int kHybridFlat = 8;      // the flat kernel takes up to this many times the words it can hold
constexpr int kStream = 8;          // streamed words in flight per thread (flat hybrid)

// A uniform index the compiler must treat as new here, so it recomputes the addresses derived from it instead of
// keeping (and spilling) them across the fold's wait.
__device__ __forceinline__ int64_t opaque_s64(int64_t v) {
  asm volatile("" : "+s"(v));
  return v;
}

// Marks held words as redefined here, so the compiler cannot hoist their conversion above the fold's wait (it would
// widen all of them to fp32 at once and spill).
template <int W>
__device__ __forceinline__ void hold(u32x4 (&w)[W]) {
#pragma unroll
  for (int i = 0; i < W; i++) asm volatile("" : "+v"(w[i]));
}

// max |x| bits of one 16-byte word, NaN excluded (the rule of amax_kernel, element by element).
template <typename T>
__device__ __forceinline__ uint32_t word_amax_exact(u32x4 w) {
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t v = w[j];
    if constexpr (sizeof(T) == 2) {
      const uint32_t a0 = (v & 0x7fffu) << 16, a1 = v & 0x7fff0000u;
      if (a0 <= 0x7f800000u) m = max(m, a0);
      if (a1 <= 0x7f800000u) m = max(m, a1);
    } else {
      const uint32_t a = v & 0x7fffffffu;
      if (a <= 0x7f800000u) m = max(m, a);
    }
  }
  return m;
}

// max |x| over a thread's words: packed maxima first; a thread that saw a NaN folds its words again exactly. Zero
// words (outside x) change nothing.
template <typename T, int W>
__device__ __forceinline__ uint32_t words_amax(const u32x4 (&w)[W]) {
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < W; i++) m = word_max<T>(m, w[i]);
  bool nan;
  if constexpr (sizeof(T) == 2) {
    m = max(m & 0xffffu, m >> 16);
    nan = m > 0x7f80u;
    m <<= 16;
  } else {
    nan = m > 0x7f800000u;
  }
  if (nan) {
    m = 0;
#pragma unroll
    for (int i = 0; i < W; i++) m = max(m, word_amax_exact<T>(w[i]));
  }
  return m;
}

// Flat single-pass cast. x as nw 16-byte words (8 bf16 or 4 fp32 elements) plus `tail` (< 8 or < 4) elements;
// workgroup b holds words [b P, (b + 1) P), P = 256 wpt, thread t words b P + 256 j + t, j < wpt <= kOnceWords<T>.
// Hybrid (sgroups > 0, x larger than the grid holds): the 256-word groups past the held words, G P + 256 s + t, are
// streamed by workgroup s % G twice -- for the maximum, then (last first, for MALL hits) for the cast -- so only
// what does not fit is read twice. Map: the source word of each output word (the tail is read flat: HeadMap sources
// have none).
template <typename T, class Map = FlatMap>
__global__ __launch_bounds__(256, 4) void cast_once_kernel(const T *__restrict__ x, int64_t n, int wpt,
                                                           int64_t sgroups, uint8_t *__restrict__ q,
                                                           float *__restrict__ dequant, void *ws,
                                                           uint32_t wait_ticks, const Map map = Map()) {
  const uint32_t ep = once_epoch(ws);   // (before the first loads: its latency passes behind them)
  constexpr int kE = 16 / sizeof(T);   // elements per word
  const int64_t nw = n / kE;
  const int tail = (int)(n % kE);
  const u32x4 *xv = reinterpret_cast<const u32x4 *>(x);
  const int64_t P = 256 * (int64_t)wpt;
  const int64_t G = gridDim.x;
  auto word = [&](int64_t b, int j) { return b * P + 256 * j + threadIdx.x; };
  // streamed word index (below 2^31: a hybrid x is at most kHybridFlat x 4 Mi words)
  auto sword = [&](int64_t s) { return (uint32_t)(G * P + 256 * s) + threadIdx.x; };
  // the streamed groups' maximum of workgroup b
  auto stream_amax = [&](int64_t b) {
    uint32_t a = 0;
    for (int64_t s = b; s < sgroups; s += kStream * G) {
      u32x4 S[kStream];
#pragma unroll
      for (int k = 0; k < kStream; k++) {
        const int64_t sk = s + k * G, i = sword(sk);
        S[k] = sk < sgroups && i < nw ? __builtin_nontemporal_load(xv + map(i)) : u32x4{0u, 0u, 0u, 0u};
      }
      a = max(a, words_amax<T, kStream>(S));
    }
    return a;
  };
  constexpr int kW = kOnceWords<T>;
  u32x4 w[kW];
#pragma unroll
  for (int j = 0; j < kW; j++) {
    const int64_t i = word(blockIdx.x, j);
    w[j] = j < wpt && i < nw ? __builtin_nontemporal_load(xv + map(i)) : u32x4{0u, 0u, 0u, 0u};
  }
  // every workgroup folds the tail elements into its partial, so a partial computed from x includes them as well
  auto tail_amax = [&]() {
    uint32_t a = 0;
    if (threadIdx.x < tail) {
      const float v = sizeof(T) == 2 ? bf16_lo(reinterpret_cast<const uint16_t *>(x)[nw * kE + threadIdx.x])
                                     : reinterpret_cast<const float *>(x)[nw * kE + threadIdx.x];
      a = __float_as_uint(v) & 0x7fffffffu;
      a = a <= 0x7f800000u ? a : 0u;
    }
    return a;
  };
  uint32_t m0 = max(words_amax<T, kW>(w), tail_amax());
  if (sgroups > 0) m0 = max(m0, stream_amax(blockIdx.x));
  const uint32_t m = block_max_u32(m0);
  uint32_t tk;
  const uint32_t g = once_fold(m, ws, ep, wait_ticks, tk, [&](int c) {
    uint32_t a = tail_amax();
    for (int j = 0; j < wpt; j++) {
      const int64_t i = word(c, j);
      if (i < nw) a = max(a, word_amax_exact<T>(__builtin_nontemporal_load(xv + map(i))));
    }
    if (sgroups > 0) a = max(a, stream_amax(c));
    return block_max_u32(a);
  });
  hold(w);
  float scale, deq;
  scales_from_amax(g, scale, deq);
  if (blockIdx.x == 0 && threadIdx.x == 0) *dequant = deq;
  const int64_t b2 = opaque_s64(blockIdx.x);   // the store addresses are recomputed, not kept from the loads
#pragma unroll
  for (int j = 0; j < kW; j++) {
    const int64_t i = word(b2, j);
    if (j < wpt && i < nw) {
      if constexpr (sizeof(T) == 2) __builtin_nontemporal_store(cast8_bf16(w[j], scale), reinterpret_cast<u32x2 *>(q) + i);
      else __builtin_nontemporal_store(cast4_f32(w[j], scale), reinterpret_cast<uint32_t *>(q) + i);
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < tail) {
    const int64_t i = nw * kE + threadIdx.x;
    const float v = sizeof(T) == 2 ? bf16_lo(reinterpret_cast<const uint16_t *>(x)[i]) : reinterpret_cast<const float *>(x)[i];
    q[i] = (uint8_t)e4m3x4(sat(v * scale), 0.f, 0.f, 0.f);
  }
  // hybrid: the streamed groups again, this workgroup's last first, kStream loads in flight
  if (sgroups > (int64_t)blockIdx.x) {
    const int64_t cnt = (sgroups - 1 - blockIdx.x) / G + 1;   // streamed groups of this workgroup
    for (int64_t k0 = cnt - 1; k0 >= 0; k0 -= kStream) {
      u32x4 S[kStream];
#pragma unroll
      for (int k = 0; k < kStream; k++) {
        const int64_t i = sword(blockIdx.x + (k0 - k) * G);
        S[k] = k0 - k >= 0 && i < nw ? __builtin_nontemporal_load(xv + map(i)) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int k = 0; k < kStream; k++) {
        const int64_t i = sword(blockIdx.x + (k0 - k) * G);
        if (k0 - k >= 0 && i < nw) {
          if constexpr (sizeof(T) == 2) __builtin_nontemporal_store(cast8_bf16(S[k], scale), reinterpret_cast<u32x2 *>(q) + i);
          else __builtin_nontemporal_store(cast4_f32(S[k], scale), reinterpret_cast<uint32_t *>(q) + i);
        }
      }
    }
  }
  once_done(ws, tk);
}

// Transposing single-pass cast of a bf16 source, run by the G workgroups [first, first + G) of a launch: workgroup b of
// them holds tiles b and b + G (when there is one) in registers.
// A larger x (at most kHybridTiles tiles) takes the same kernel as a hybrid: workgroup b's further tiles b + k G,
// k >= 2, are streamed once for the maximum and once more, last first, for the cast, so only the part of x that does
// not fit is read twice.
__device__ __forceinline__ void cast_t_once_run(const uint16_t *__restrict__ x, int64_t ld, int64_t rows, int64_t cols,
                                                uint8_t *__restrict__ q, int64_t ldq, uint8_t *__restrict__ qt,
                                                int64_t ldt, float *__restrict__ dequant, void *ws, uint32_t wait_ticks,
                                                uint32_t ep, int64_t b, int64_t G, int first) {
  static_assert(kOnceTiles == 2, "two tiles per workgroup");
  __shared__ uint32_t tile[kTT * kTPitch];
  const int64_t tiles_c = (cols + kTT - 1) / kTT, tiles = tiles_c * ((ldt + kTT - 1) / kTT);
  const int64_t t0 = b, t1 = b + G;   // t0 < tiles: the grid never exceeds the tile count
  auto r0_of = [&](int64_t t) { return (t / tiles_c) * kTT; };
  auto c0_of = [&](int64_t t) { return (t % tiles_c) * kTT; };
  u32x4 R[2 * kTPer];
  u32x4(&R0)[kTPer] = *reinterpret_cast<u32x4(*)[kTPer]>(R);
  u32x4(&R1)[kTPer] = *reinterpret_cast<u32x4(*)[kTPer]>(R + kTPer);
  load_tile_bf16(x, ld, rows, cols, r0_of(t0), c0_of(t0), R0);
  if (t1 < tiles) {
    load_tile_bf16(x, ld, rows, cols, r0_of(t1), c0_of(t1), R1);
  } else {
#pragma unroll
    for (int i = 0; i < kTPer; i++) R1[i] = u32x4{0u, 0u, 0u, 0u};
  }
  uint32_t m = words_amax<uint16_t, 2 * kTPer>(R);
  for (int64_t t = b + 2 * G; t < tiles; t += G) {   // hybrid: the tiles that are not held
    u32x4 S[kTPer];
    load_tile_bf16(x, ld, rows, cols, r0_of(t), c0_of(t), S);
    m = max(m, words_amax<uint16_t, kTPer>(S));
  }
  uint32_t tk;
  const uint32_t g = once_fold_range(block_max_u32(m), ws, ep, wait_ticks, tk, first, (int)G, [&](int c) {
    uint32_t a = 0;
    for (int64_t t = c; t < tiles; t += G) {
      const int64_t r0 = r0_of(t), c0 = c0_of(t);
      for (int i = 0; i < kTPer; i++) {
        const int id = threadIdx.x + 256 * i;
        const int64_t gr = r0 + (id >> 4), gc = c0 + 8 * (id & 15);
        if (gr < rows && gc < cols) a = max(a, word_amax_exact<uint16_t>(*reinterpret_cast<const u32x4 *>(x + gr * ld + gc)));
      }
    }
    return block_max_u32(a);
  });
  hold(R);
  float scale, deq;
  scales_from_amax(g, scale, deq);
  if (b == 0 && threadIdx.x == 0) *dequant = deq;
  u32x2 E0[kTPer], E1[kTPer];   // both tiles narrowed first: 32 VGPRs live instead of 64
  cvt_tile_bf16(R0, scale, E0);
  cvt_tile_bf16(R1, scale, E1);
  // hybrid: the streamed tiles again, last first (the most recently read are the likeliest still in the MALL), the
  // next one's loads in flight while the current one is cast
  int64_t ts = b + 2 * G;
  if (ts < tiles) ts += ((tiles - 1 - ts) / G) * G;   // the last tile of this workgroup
  u32x4 S[kTPer];
  if (ts < tiles) load_tile_bf16(x, ld, rows, cols, r0_of(ts), c0_of(ts), S);
  const int64_t u0 = opaque_s64(t0), u1 = u0 + G;
  emit_tile(E0, r0_of(u0), c0_of(u0), rows, cols, q, ldq, qt, ldt, tile);
  if (u1 < tiles) emit_tile(E1, r0_of(u1), c0_of(u1), rows, cols, q, ldq, qt, ldt, tile);
  for (; ts >= 2 * G && ts < tiles; ts -= G) {
    u32x2 E[kTPer];
    cvt_tile_bf16(S, scale, E);
    if (ts - G >= 2 * G) load_tile_bf16(x, ld, rows, cols, r0_of(ts - G), c0_of(ts - G), S);
    emit_tile(E, r0_of(ts), c0_of(ts), rows, cols, q, ldq, qt, ldt, tile);
  }
  once_done(ws, tk);
}

__global__ __launch_bounds__(256, 4) void cast_t_once_kernel(const uint16_t *__restrict__ x, int64_t ld, int64_t rows,
                                                             int64_t cols, uint8_t *__restrict__ q, int64_t ldq,
                                                             uint8_t *__restrict__ qt, int64_t ldt,
                                                             float *__restrict__ dequant, void *ws,
                                                             uint32_t wait_ticks) {
  const uint32_t ep = once_epoch(ws);   // (before the first loads: its latency passes behind them)
  cast_t_once_run(x, ld, rows, cols, q, ldq, qt, ldt, dequant, ws, wait_ticks, ep, blockIdx.x, gridDim.x, 0);
}

// Several transposing casts in one launch: tensor i takes workgroups [first[i], first[i + 1]), each holding at most
// two of its tiles (no hybrid), and folds over its own workgroups' partials; one epoch and one done count for the
// launch. The same bytes and scales as one cast_t_once_kernel launch per tensor.
constexpr int kMaxTGroup = 8;
struct TGroup {
  const uint16_t *x[kMaxTGroup];
  uint8_t *q[kMaxTGroup];
  uint8_t *qt[kMaxTGroup];
  float *dequant[kMaxTGroup];
  int64_t rows[kMaxTGroup], cols[kMaxTGroup], ldt[kMaxTGroup];
  int first[kMaxTGroup + 1];
  int count;
};
__global__ __launch_bounds__(256, 4) void cast_t_group_kernel(const TGroup g, void *ws,
                                                              uint32_t wait_ticks) {
  const uint32_t ep = once_epoch(ws);
  int i = 0;
  while (i + 1 < g.count && (int)blockIdx.x >= g.first[i + 1]) i++;
  i = __builtin_amdgcn_readfirstlane(i);
  const int first = g.first[i];
  cast_t_once_run(g.x[i], g.cols[i], g.rows[i], g.cols[i], g.q[i], g.cols[i], g.qt[i], g.ldt[i], g.dequant[i], ws,
                  wait_ticks, ep, (int)blockIdx.x - first, g.first[i + 1] - first, first);
}

// ------------------------------------------------------------------------------------------- single-pass SwiGLU

// Single-pass SwiGLU product cast, flat (q [M, H] contiguous): one launch of one 1024-thread workgroup per CU. Word i
// of the product (8 values: row i / (H / 8), columns 8 (i % (H / 8)) + [0, 8)) is computed from 16 bytes of z1 and
// 16 of z2. The words go in groups of 1024, one word per thread; workgroup b takes groups j G + b, j = 0, 1, ...: at
// each step the grid reads one contiguous window of z. Groups j < wpt are held as bf16 until the fold: j < kSwHeldR in
// registers, the rest in LDS (128 KiB beside the 24 KiB sigmoid table; 96 MiB over 256 CUs). A product larger than the
// grid holds is a hybrid: the sgroups groups past wpt G are streamed -- computed, taken into the maximum and written
// to `a`; after the fold read back, last first, and cast. Moved per element: 4 B of z read and 1 B of q written, plus
// 2 B written and 2 B read back for the streamed part (the two-pass cast: 4 + 2 + 2 + 1). The thread that writes a
// streamed word is the one that reads it back: the XCDs' L2 caches are not coherent with each other within a kernel.
constexpr int kSwThreads = 1024;   // 16 waves, 4 per SIMD: at most 128 VGPRs each
constexpr int kSwHeldR = 16;       // product words a thread holds in registers (64 VGPRs)
constexpr int kSwHeldL = 8;        // product words a thread holds in LDS (128 KiB per workgroup)
constexpr int kSwHeld = kSwHeldR + kSwHeldL;
constexpr int kSwBatch = 2;        // words whose z loads are issued together (4 words' loads spill at 128 VGPRs)
constexpr int kSwHybrid = 8;       // the single pass takes products up to this many times what the grid holds
static_assert(kSwHeldR % kSwBatch == 0 && kSwHeldL % kSwBatch == 0, "a batch lies in registers or in LDS");

// Row and 8-column unit of product word i, stepped along words a fixed distance apart: one division at the start,
// then per step an add and at most one wrap (the step's remainder is below `units`).
struct SwCursor {
  uint32_t r, u;
  __device__ __forceinline__ SwCursor(uint32_t i, uint32_t units) : r(i / units), u(i % units) {}
  __device__ __forceinline__ void step(uint32_t dq, uint32_t dr, uint32_t units) {
    r += dq;
    u += dr;
    if (u >= units) {
      u -= units;
      r++;
    }
  }
};

// nw = M H / 8 product words (below 2^31: the host bounds it); a is needed only when sgroups > 0.
__global__ __launch_bounds__(kSwThreads) void swiglu_once_kernel(const uint16_t *__restrict__ z, int64_t H, int64_t sz,
                                                                  uint32_t nw, int wpt, uint32_t sgroups,
                                                                  uint16_t *__restrict__ a, uint8_t *__restrict__ q,
                                                                  float *__restrict__ dequant, void *ws,
                                                                  uint32_t wait_ticks) {
  const uint32_t ep = once_epoch(ws);   // (before the first loads: its latency passes behind them)
  __shared__ float lut[kLutLds];
  __shared__ u32x4 held[kSwHeldL * kSwThreads];
  lut_build(lut);
  const uint32_t t = threadIdx.x, units = (uint32_t)(H / 8), G = gridDim.x;
  const uint32_t base_s = G * kSwThreads * (uint32_t)wpt;   // the first streamed word
  // word of thread t in held group j of workgroup b
  auto hword = [&](uint32_t b, int j) { return ((uint32_t)j * G + b) * kSwThreads + t; };
  const u32x4 zero{0u, 0u, 0u, 0u};
  auto zp = [&](uint32_t r, uint32_t u) { return z + (int64_t)r * sz + 8 * u; };
  auto ld = [](const uint16_t *p) { return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p)); };
  auto product = [&](uint32_t i) {
    const uint32_t r = i / units;
    const uint16_t *p = zp(r, i - r * units);
    return swiglu8_words(lut, ld(p), ld(p + H));
  };

  // held words, kSwBatch at a time: loads branch-free (a word past the product reads z's first word and is then
  // zeroed), products kept (registers, then LDS) and folded into m. The 16 waves of the workgroup overlap one
  // another's loads and arithmetic (2 waves per SIMD holding twice the words, with a software pipeline: 3.7 TB/s
  // against ~6 here).
  u32x4 w[kSwHeldR];
#pragma unroll
  for (int j = 0; j < kSwHeldR; j++) w[j] = zero;
  uint32_t m = 0;
  {
    SwCursor c(hword(blockIdx.x, 0), units);
    const uint32_t d = kSwThreads * G, dq = d / units, dr = d % units;
#pragma unroll
    for (int j0 = 0; j0 < kSwHeld; j0 += kSwBatch) {
      if (j0 < wpt) {   // (a small product: fewer words per thread)
        u32x4 z1[kSwBatch], z2[kSwBatch];
        bool ok[kSwBatch];
#pragma unroll
        for (int k = 0; k < kSwBatch; k++) {
          ok[k] = j0 + k < wpt && hword(blockIdx.x, j0 + k) < nw;
          const uint16_t *p = ok[k] ? zp(c.r, c.u) : z;
          z1[k] = ld(p);
          z2[k] = ld(p + H);
          c.step(dq, dr, units);
        }
        u32x4 A[kSwBatch];
#pragma unroll
        for (int k = 0; k < kSwBatch; k++)
          A[k] = swiglu8_words(lut, ok[k] ? z1[k] : zero, ok[k] ? z2[k] : zero);   // zero words: zero products
        m = max(m, words_amax<uint16_t, kSwBatch>(A));
#pragma unroll
        for (int k = 0; k < kSwBatch; k++) {
          if (j0 + k < kSwHeldR) w[j0 + k] = A[k];
          else held[(j0 + k - kSwHeldR) * kSwThreads + t] = A[k];
        }
      }
    }
  }
  // hybrid: this workgroup's streamed groups s = b, b + G, ..., computed, folded into m and written to a
  if (blockIdx.x < sgroups) {
    SwCursor c(base_s + kSwThreads * blockIdx.x + t, units);
    const uint32_t d = kSwThreads * G, dq = d / units, dr = d % units;
    for (uint32_t s0 = blockIdx.x; s0 < sgroups; s0 += kSwBatch * G) {
      u32x4 z1[kSwBatch], z2[kSwBatch];
      bool ok[kSwBatch];
#pragma unroll
      for (int k = 0; k < kSwBatch; k++) {
        const uint32_t s = s0 + k * G, i = base_s + kSwThreads * s + t;
        ok[k] = s < sgroups && i < nw;
        const uint16_t *p = zp(c.r, c.u);
        z1[k] = ok[k] ? ld(p) : zero;
        z2[k] = ok[k] ? ld(p + H) : zero;
        c.step(dq, dr, units);
      }
      u32x4 A[kSwBatch];
#pragma unroll
      for (int k = 0; k < kSwBatch; k++) A[k] = swiglu8_words(lut, z1[k], z2[k]);
      m = max(m, words_amax<uint16_t, kSwBatch>(A));
#pragma unroll
      for (int k = 0; k < kSwBatch; k++)
        if (ok[k]) reinterpret_cast<u32x4 *>(a)[base_s + kSwThreads * (s0 + k * G) + t] = A[k];
    }
  }

  uint32_t tk;
  const uint32_t g = once_fold(block_max_u32(m), ws, ep, wait_ticks, tk, [&](int cb) {
    uint32_t v = 0;
    for (int j = 0; j < wpt; j++) {
      const uint32_t i = hword((uint32_t)cb, j);
      if (i < nw) v = max(v, word_amax_exact<uint16_t>(product(i)));
    }
    for (uint32_t s = cb; s < sgroups; s += G) {
      const uint32_t i = base_s + kSwThreads * s + t;
      if (i < nw) v = max(v, word_amax_exact<uint16_t>(product(i)));
    }
    return block_max_u32(v);
  });
  hold(w);
  float scale, deq;
  scales_from_amax(g, scale, deq);
  if (blockIdx.x == 0 && t == 0) *dequant = deq;
  u32x2 *qv = reinterpret_cast<u32x2 *>(q);
  const uint32_t b2 = (uint32_t)opaque_s64(blockIdx.x);   // store addresses recomputed, not kept from the loads
#pragma unroll
  for (int j = 0; j < kSwHeldR; j++) {
    const uint32_t i = hword(b2, j);
    if (j < wpt && i < nw) __builtin_nontemporal_store(cast8_bf16(w[j], scale), qv + i);
  }
  if (wpt > kSwHeldR) {
    u32x4 L[kSwHeldL];
#pragma unroll
    for (int j = 0; j < kSwHeldL; j++) L[j] = held[j * kSwThreads + t];
#pragma unroll
    for (int j = 0; j < kSwHeldL; j++) {
      const uint32_t i = hword(b2, kSwHeldR + j);
      if (kSwHeldR + j < wpt && i < nw) __builtin_nontemporal_store(cast8_bf16(L[j], scale), qv + i);
    }
  }
  // hybrid: the streamed groups back from a, this workgroup's last first, kStream loads in flight
  if (blockIdx.x < sgroups) {
    const u32x4 *av = reinterpret_cast<const u32x4 *>(a);
    const int64_t cnt = (sgroups - 1 - blockIdx.x) / G + 1;
    for (int64_t k0 = cnt - 1; k0 >= 0; k0 -= kStream) {
      u32x4 S[kStream];
#pragma unroll
      for (int k = 0; k < kStream; k++) {
        const uint32_t i = base_s + kSwThreads * (uint32_t)(blockIdx.x + (k0 - k) * G) + t;
        S[k] = k0 - k >= 0 && i < nw ? __builtin_nontemporal_load(av + i) : zero;
      }
#pragma unroll
      for (int k = 0; k < kStream; k++) {
        const uint32_t i = base_s + kSwThreads * (uint32_t)(blockIdx.x + (k0 - k) * G) + t;
        if (k0 - k >= 0 && i < nw) __builtin_nontemporal_store(cast8_bf16(S[k], scale), qv + i);
      }
    }
  }
  once_done(ws, tk);
}

// Single-pass SwiGLU backward cast without dz in memory (dzq [M, 2H] contiguous): one launch of one 1024-thread
// workgroup per CU. Unit i (row i / (H / 8), columns 8 (i % (H / 8)) + [0, 8) of each half) takes 16 bytes each of
// z1, z2 and da and gives two dz words (d1, d2: 8 bf16 each, dz_words). Units go in groups of 1024, one per thread;
// workgroup b takes groups j G + b. Groups j < wpt are held as dz words until the fold: j < kBwHeldR in registers,
// the rest in LDS (128 KiB beside the 24 KiB sigmoid table; 80 MiB of dz over 256 CUs). Past that (sgroups further
// groups) the units are computed for the maximum only and computed again from z and da after the fold, as the
// two-pass cast does. Moved per unit: 48 B read and 16 B written held, 96 B read and 16 B written streamed (the
// two-pass cast: 96 + 16).
constexpr int kBwHeldR = 6;     // units a thread holds in registers (2 words each: 48 VGPRs)
constexpr int kBwHeldL = 4;     // units a thread holds in LDS (128 KiB per workgroup)
constexpr int kBwHeld = kBwHeldR + kBwHeldL;
constexpr int kBwBatch = 2;     // units whose loads are issued together
constexpr int kBwHybrid = 16;   // the single pass takes up to this many times what the grid holds (d18: 11x)
static_assert(kBwHeldR % kBwBatch == 0 && kBwHeldL % kBwBatch == 0, "a batch lies in registers or in LDS");

// nu = M H / 8 units (below 2^31: the host bounds it).
__global__ __launch_bounds__(kSwThreads) void swiglu_bwd_once_kernel(const uint16_t *__restrict__ z,
                                                                      const uint16_t *__restrict__ da, int64_t H,
                                                                      int64_t sz, int64_t sda, uint32_t nu, int wpt,
                                                                      uint32_t sgroups, uint8_t *__restrict__ dzq,
                                                                      float *__restrict__ dequant, void *ws,
                                                                      uint32_t wait_ticks) {
  const uint32_t ep = once_epoch(ws);   // (before the first loads: its latency passes behind them)
  __shared__ float lut[kLutLds];
  __shared__ u32x4 held[2 * kBwHeldL * kSwThreads];
  lut_build(lut);
  const uint32_t t = threadIdx.x, units = (uint32_t)(H / 8), G = gridDim.x;
  const uint32_t base_s = G * kSwThreads * (uint32_t)wpt;   // the first streamed unit
  const u32x4 zero{0u, 0u, 0u, 0u};
  auto hunit = [&](uint32_t b, int j) { return ((uint32_t)j * G + b) * kSwThreads + t; };
  auto ld = [](const uint16_t *p) { return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p)); };
  // the three input words of the unit at (r, u), or of unit 0 when !ok (then zeroed by the caller)
  auto load3 = [&](bool ok, uint32_t r, uint32_t u, u32x4 &z1, u32x4 &z2, u32x4 &d) {
    const uint16_t *zr = ok ? z + (int64_t)r * sz + 8 * u : z;
    z1 = ld(zr);
    z2 = ld(zr + H);
    d = ld(ok ? da + (int64_t)r * sda + 8 * u : da);
  };
  auto dz_of = [&](uint32_t i, u32x4 &h1, u32x4 &h2) {
    const uint32_t r = i / units, u = i - r * units;
    u32x4 z1, z2, d;
    load3(true, r, u, z1, z2, d);
    dz_words(lut, z1, z2, d, h1, h2);
  };

  // held units, kBwBatch at a time: loads branch-free, dz kept (registers, then LDS) and folded into m
  u32x4 w1[kBwHeldR], w2[kBwHeldR];
#pragma unroll
  for (int j = 0; j < kBwHeldR; j++) w1[j] = w2[j] = zero;
  uint32_t m = 0;
  {
    SwCursor c(hunit(blockIdx.x, 0), units);
    const uint32_t d = kSwThreads * G, dq = d / units, dr = d % units;
#pragma unroll
    for (int j0 = 0; j0 < kBwHeld; j0 += kBwBatch) {
      if (j0 < wpt) {   // (a small tensor: fewer units per thread)
        u32x4 Z1[kBwBatch], Z2[kBwBatch], D[kBwBatch];
        bool ok[kBwBatch];
#pragma unroll
        for (int k = 0; k < kBwBatch; k++) {
          ok[k] = j0 + k < wpt && hunit(blockIdx.x, j0 + k) < nu;
          load3(ok[k], c.r, c.u, Z1[k], Z2[k], D[k]);
          c.step(dq, dr, units);
        }
        u32x4 Hh[2 * kBwBatch];
#pragma unroll
        for (int k = 0; k < kBwBatch; k++)
          dz_words(lut, ok[k] ? Z1[k] : zero, ok[k] ? Z2[k] : zero, ok[k] ? D[k] : zero, Hh[2 * k], Hh[2 * k + 1]);
        m = max(m, words_amax<uint16_t, 2 * kBwBatch>(Hh));   // zero inputs: zero dz
#pragma unroll
        for (int k = 0; k < kBwBatch; k++) {
          const int j = j0 + k;
          if (j < kBwHeldR) {
            w1[j] = Hh[2 * k];
            w2[j] = Hh[2 * k + 1];
          } else {
            held[(2 * (j - kBwHeldR)) * kSwThreads + t] = Hh[2 * k];
            held[(2 * (j - kBwHeldR) + 1) * kSwThreads + t] = Hh[2 * k + 1];
          }
        }
      }
    }
  }
  // hybrid: this workgroup's streamed groups s = b, b + G, ..., computed and folded into m (not kept)
  if (blockIdx.x < sgroups) {
    SwCursor c(base_s + kSwThreads * blockIdx.x + t, units);
    const uint32_t d = kSwThreads * G, dq = d / units, dr = d % units;
    for (uint32_t s0 = blockIdx.x; s0 < sgroups; s0 += kBwBatch * G) {
      u32x4 Z1[kBwBatch], Z2[kBwBatch], D[kBwBatch];
      bool ok[kBwBatch];
#pragma unroll
      for (int k = 0; k < kBwBatch; k++) {
        const uint32_t s = s0 + k * G;
        ok[k] = s < sgroups && base_s + kSwThreads * s + t < nu;
        load3(ok[k], c.r, c.u, Z1[k], Z2[k], D[k]);
        c.step(dq, dr, units);
      }
      u32x4 Hh[2 * kBwBatch];
#pragma unroll
      for (int k = 0; k < kBwBatch; k++)
        dz_words(lut, ok[k] ? Z1[k] : zero, ok[k] ? Z2[k] : zero, ok[k] ? D[k] : zero, Hh[2 * k], Hh[2 * k + 1]);
      m = max(m, words_amax<uint16_t, 2 * kBwBatch>(Hh));
    }
  }

  uint32_t tk;
  const uint32_t g = once_fold(block_max_u32(m), ws, ep, wait_ticks, tk, [&](int cb) {
    uint32_t v = 0;
    for (int j = 0; j < wpt; j++) {
      const uint32_t i = hunit((uint32_t)cb, j);
      if (i < nu) {
        u32x4 h1, h2;
        dz_of(i, h1, h2);
        v = max(v, max(word_amax_exact<uint16_t>(h1), word_amax_exact<uint16_t>(h2)));
      }
    }
    for (uint32_t s = cb; s < sgroups; s += G) {
      const uint32_t i = base_s + kSwThreads * s + t;
      if (i < nu) {
        u32x4 h1, h2;
        dz_of(i, h1, h2);
        v = max(v, max(word_amax_exact<uint16_t>(h1), word_amax_exact<uint16_t>(h2)));
      }
    }
    return block_max_u32(v);
  });
  hold(w1);
  hold(w2);
  float scale, deq;
  scales_from_amax(g, scale, deq);
  if (blockIdx.x == 0 && t == 0) *dequant = deq;
  auto out = [&](uint32_t i) {   // dzq bytes of unit i's d1 (d2: + H)
    const uint32_t r = i / units;
    return dzq + (int64_t)r * 2 * H + 8 * (i - r * units);
  };
  auto emit = [&](uint32_t i, u32x4 h1, u32x4 h2) {
    uint8_t *o = out(i);
    __builtin_nontemporal_store(cast8_bf16(h1, scale), reinterpret_cast<u32x2 *>(o));
    __builtin_nontemporal_store(cast8_bf16(h2, scale), reinterpret_cast<u32x2 *>(o + H));
  };
  const uint32_t b2 = (uint32_t)opaque_s64(blockIdx.x);   // addresses recomputed, not kept from the loads
#pragma unroll
  for (int j = 0; j < kBwHeldR; j++) {
    const uint32_t i = hunit(b2, j);
    if (j < wpt && i < nu) emit(i, w1[j], w2[j]);
  }
  if (wpt > kBwHeldR) {
    u32x4 L1[kBwHeldL], L2[kBwHeldL];
#pragma unroll
    for (int j = 0; j < kBwHeldL; j++) {
      L1[j] = held[(2 * j) * kSwThreads + t];
      L2[j] = held[(2 * j + 1) * kSwThreads + t];
    }
#pragma unroll
    for (int j = 0; j < kBwHeldL; j++) {
      const uint32_t i = hunit(b2, kBwHeldR + j);
      if (kBwHeldR + j < wpt && i < nu) emit(i, L1[j], L2[j]);
    }
  }
  // hybrid: the streamed groups again, this workgroup's last first, dz computed again from z and da and cast
  if (blockIdx.x < sgroups) {
    const int64_t cnt = (sgroups - 1 - blockIdx.x) / G + 1;
    for (int64_t k0 = cnt - 1; k0 >= 0; k0 -= kBwBatch) {
      u32x4 Z1[kBwBatch], Z2[kBwBatch], D[kBwBatch];
      bool ok[kBwBatch];
      uint32_t ii[kBwBatch];
#pragma unroll
      for (int k = 0; k < kBwBatch; k++) {
        ii[k] = base_s + kSwThreads * (uint32_t)(blockIdx.x + (k0 - k) * G) + t;
        ok[k] = k0 - k >= 0 && ii[k] < nu;
        const uint32_t r = ok[k] ? ii[k] / units : 0u;
        load3(ok[k], r, ok[k] ? ii[k] - r * units : 0u, Z1[k], Z2[k], D[k]);
      }
#pragma unroll
      for (int k = 0; k < kBwBatch; k++) {
        if (ok[k]) {
          u32x4 h1, h2;
          dz_words(lut, Z1[k], Z2[k], D[k], h1, h2);
          emit(ii[k], h1, h2);
        }
      }
    }
  }
  once_done(ws, tk);
}

// Single-pass flat cast of a bf16 tensor above 48 MiB (cast_once_kernel holds 64 MiB): one 1024-thread workgroup per
// CU, each thread holding kWideR words in registers and kWideL in LDS -- 400 KiB per CU, 100 MiB over 256 CUs. Words
// go in groups of 1024, one per thread, workgroup b taking groups j G + b (j < wpt held); a larger x is a hybrid as in
// cast_once_kernel: the sgroups groups past wpt G, workgroup s % G taking group s, are read for the maximum and read
// again, last first, for the cast. The n % 8 tail elements: folded into every workgroup's partial, cast by workgroup 0
// (read flat). Map: the source word of each output word.
constexpr int kWideR = 16;   // words a thread holds in registers (64 VGPRs)
constexpr int kWideL = 9;    // words a thread holds in LDS (144 KiB per workgroup)
constexpr int kWide = kWideR + kWideL;

template <class Map = FlatMap>
__global__ __launch_bounds__(kSwThreads) void cast_wide_kernel(const uint16_t *__restrict__ x, int64_t n, int wpt,
                                                                uint32_t sgroups, uint8_t *__restrict__ q,
                                                                float *__restrict__ dequant, void *ws,
                                                                uint32_t wait_ticks, const Map map = Map()) {
  const uint32_t ep = once_epoch(ws);   // (before the first loads: its latency passes behind them)
  __shared__ u32x4 held[kWideL * kSwThreads];
  const uint32_t nw = (uint32_t)(n / 8), t = threadIdx.x, G = gridDim.x;
  const int tail = (int)(n % 8);
  const u32x4 *xv = reinterpret_cast<const u32x4 *>(x);
  const uint32_t base_s = G * kSwThreads * (uint32_t)wpt;   // the first streamed word
  const u32x4 zero{0u, 0u, 0u, 0u};
  auto hword = [&](uint32_t b, int j) { return ((uint32_t)j * G + b) * kSwThreads + t; };
  auto sword = [&](uint32_t s) { return base_s + kSwThreads * s + t; };
  // branch-free: a word past x reads source word 0 and is zeroed
  auto ld = [&](bool ok, uint32_t i) {
    const u32x4 v = __builtin_nontemporal_load(xv + (ok ? map(i) : 0u));
    return ok ? v : zero;
  };
  auto tail_amax = [&]() {
    uint32_t a = 0;
    if ((int)t < tail) {
      a = __float_as_uint(bf16_lo(x[(int64_t)nw * 8 + t])) & 0x7fffffffu;
      a = a <= 0x7f800000u ? a : 0u;
    }
    return a;
  };
  u32x4 w[kWideR], L[kWideL];
#pragma unroll
  for (int j = 0; j < kWideR; j++) w[j] = ld(j < wpt && hword(blockIdx.x, j) < nw, hword(blockIdx.x, j));
#pragma unroll
  for (int j = 0; j < kWideL; j++)
    L[j] = ld(kWideR + j < wpt && hword(blockIdx.x, kWideR + j) < nw, hword(blockIdx.x, kWideR + j));
  uint32_t m = max(max(words_amax<uint16_t, kWideR>(w), words_amax<uint16_t, kWideL>(L)), tail_amax());
#pragma unroll
  for (int j = 0; j < kWideL; j++) held[j * kSwThreads + t] = L[j];
  // the streamed groups' maximum of workgroup b, kStream words in flight
  auto stream_amax = [&](uint32_t b) {
    uint32_t a = 0;
    for (uint32_t s0 = b; s0 < sgroups; s0 += kStream * G) {
      u32x4 S[kStream];
#pragma unroll
      for (int k = 0; k < kStream; k++) S[k] = ld(s0 + k * G < sgroups && sword(s0 + k * G) < nw, sword(s0 + k * G));
      a = max(a, words_amax<uint16_t, kStream>(S));
    }
    return a;
  };
  if (blockIdx.x < sgroups) m = max(m, stream_amax(blockIdx.x));
  uint32_t tk;
  const uint32_t g = once_fold(block_max_u32(m), ws, ep, wait_ticks, tk, [&](int cb) {
    uint32_t a = tail_amax();
    for (int j = 0; j < wpt; j++) {
      const uint32_t i = hword((uint32_t)cb, j);
      if (i < nw) a = max(a, word_amax_exact<uint16_t>(__builtin_nontemporal_load(xv + map(i))));
    }
    for (uint32_t s = cb; s < sgroups; s += G) {
      const uint32_t i = sword(s);
      if (i < nw) a = max(a, word_amax_exact<uint16_t>(__builtin_nontemporal_load(xv + map(i))));
    }
    return block_max_u32(a);
  });
  hold(w);
  float scale, deq;
  scales_from_amax(g, scale, deq);
  if (blockIdx.x == 0 && t == 0) *dequant = deq;
  u32x2 *qv = reinterpret_cast<u32x2 *>(q);
  const uint32_t b2 = (uint32_t)opaque_s64(blockIdx.x);   // store addresses recomputed, not kept from the loads
#pragma unroll
  for (int j = 0; j < kWideR; j++) {
    const uint32_t i = hword(b2, j);
    if (j < wpt && i < nw) __builtin_nontemporal_store(cast8_bf16(w[j], scale), qv + i);
  }
  if (wpt > kWideR) {
#pragma unroll
    for (int j = 0; j < kWideL; j++) L[j] = held[j * kSwThreads + t];
#pragma unroll
    for (int j = 0; j < kWideL; j++) {
      const uint32_t i = hword(b2, kWideR + j);
      if (kWideR + j < wpt && i < nw) __builtin_nontemporal_store(cast8_bf16(L[j], scale), qv + i);
    }
  }
  if (blockIdx.x == 0 && (int)t < tail) {
    const int64_t i = (int64_t)nw * 8 + t;
    q[i] = (uint8_t)e4m3x4(sat(bf16_lo(x[i]) * scale), 0.f, 0.f, 0.f);
  }
  // hybrid: the streamed groups again, this workgroup's last first, kStream loads in flight
  if (blockIdx.x < sgroups) {
    const int64_t cnt = (sgroups - 1 - blockIdx.x) / G + 1;
    for (int64_t k0 = cnt - 1; k0 >= 0; k0 -= kStream) {
      u32x4 S[kStream];
#pragma unroll
      for (int k = 0; k < kStream; k++) {
        const uint32_t i = sword((uint32_t)(blockIdx.x + (k0 - k) * G));
        S[k] = ld(k0 - k >= 0 && i < nw, i);
      }
#pragma unroll
      for (int k = 0; k < kStream; k++) {
        const uint32_t i = sword((uint32_t)(blockIdx.x + (k0 - k) * G));
        if (k0 - k >= 0 && i < nw) __builtin_nontemporal_store(cast8_bf16(S[k], scale), qv + i);
      }
    }
  }
  once_done(ws, tk);
}

// Host side. The single-pass settings (a process-wide tuning and test knob, gpic_fp8_set_single_pass): on / off and
// the wait bound in microseconds. Atomic: a call on another thread reads either the old or the new setting.
static std::atomic<int> g_once_enabled{1};
static std::atomic<int> g_once_wait_us{kOnceWaitUs};

// Workgroups of `kernel` (`threads` threads each) the current device holds at once, capped at kMaxOnceBlocks; cached
// per device in `cache` (one per kernel, slots initialised to -1).
int once_capacity(const void *kernel, DeviceCache &cache, int threads) {
  return per_device(cache, [kernel, threads](int dev) {
    int per = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, 0) != hipSuccess) per = 0;
    (void)hipGetLastError();
    return std::min(per * device_cus(dev), kMaxOnceBlocks);
  });
}

// s_memrealtime counts at 100 MHz on this target
uint32_t once_wait_ticks() { return (uint32_t)std::max(0, g_once_wait_us.load(std::memory_order_relaxed)) * 100u; }

bool once_enabled() { return g_once_enabled.load(std::memory_order_relaxed) != 0; }

static DeviceCache g_cap_flat_bf16, g_cap_flat_f32, g_cap_t, g_cap_sw, g_cap_bw, g_cap_wide, g_cap_tg, g_cap_heads,
    g_cap_heads_wide;
struct DeviceCacheInit {   // every slot starts at -1 (not yet computed)
  DeviceCacheInit() {
    for (int i = 0; i < kMaxDevices; i++)
      g_cap_flat_bf16[i] = g_cap_flat_f32[i] = g_cap_t[i] = g_cap_sw[i] = g_cap_bw[i] = g_cap_wide[i] = g_cap_tg[i] =
          g_cap_heads[i] = g_cap_heads_wide[i] = -1;
  }
};
static DeviceCacheInit g_device_cache_init;

// The single-pass flat cast when x fits, as a hybrid up to kHybridFlat times that (false, nothing launched, above).
// Map: where each output word's source lies (FlatMap: x itself; HeadMap: bf16 attention heads).
template <typename T, class Map = FlatMap>
static bool launch_tcast_once(const T *x, int64_t n, uint8_t *q, float *dequant, void *ws, hipStream_t st,
                              const Map map = Map()) {
  constexpr bool kFlat = std::is_same<Map, FlatMap>::value;
  const int cap = once_capacity(reinterpret_cast<const void *>(&cast_once_kernel<T, Map>),
                                !kFlat ? g_cap_heads : sizeof(T) == 2 ? g_cap_flat_bf16 : g_cap_flat_f32, 256);
  constexpr int kE = 16 / sizeof(T);
  const int64_t nw = n / kE;
  const int64_t held = (int64_t)kOnceWords<T> * 256 * cap;   // words the grid holds in registers
  if (!once_enabled() || cap <= 0 || n <= 0) return false;
  if constexpr (sizeof(T) == 2) {   // bf16 past 3/4 of what this kernel holds (48 MiB): the wide kernel, up to
                                     // kHybridFlat x its hold (flushed caches: 64 MiB 23.8 us against 24.8, 32 MiB
                                     // 18.3 against 16.4, 192 MiB 74 against 88 as this kernel's hybrid)
    if (4 * nw > 3 * held) {
      const int capw = once_capacity(reinterpret_cast<const void *>(&cast_wide_kernel<Map>),
                                     kFlat ? g_cap_wide : g_cap_heads_wide, kSwThreads);
      const int64_t heldw = (int64_t)kWide * kSwThreads * capw;
      if (capw <= 0 || nw > kHybridFlat * heldw) return false;
      int grid = capw, wpt = kWide;
      int64_t sgroups = 0;
      if (nw > heldw) {
        sgroups = (nw - heldw + kSwThreads - 1) / kSwThreads;
      } else {
        const int64_t groups = (nw + kSwThreads - 1) / kSwThreads;
        grid = (int)std::min<int64_t>(groups, capw);
        wpt = (int)((groups + grid - 1) / grid);
      }
      cast_wide_kernel<Map><<<grid, kSwThreads, 0, st>>>(reinterpret_cast<const uint16_t *>(x), n, wpt,
                                                         (uint32_t)sgroups, q, dequant, ws, once_wait_ticks(), map);
      return true;
    }
  }
  if (nw > kHybridFlat * held) return false;
  if (nw > held) {   // hybrid: every workgroup holds its full share, the rest is streamed
    const int64_t sgroups = (nw - held + 255) / 256;
    cast_once_kernel<T, Map><<<cap, 256, 0, st>>>(x, n, kOnceWords<T>, sgroups, q, dequant, ws, once_wait_ticks(),
                                                  map);
    return true;
  }
  const int64_t groups = std::max<int64_t>(1, (nw + 255) / 256);   // 256-word groups
  const int grid = (int)std::min<int64_t>(groups, cap);
  const int wpt = (int)((groups + grid - 1) / grid);
  cast_once_kernel<T, Map><<<grid, 256, 0, st>>>(x, n, wpt, 0, q, dequant, ws, once_wait_ticks(), map);
  return true;
}

// The single-pass SwiGLU product cast of z [M, 2H] (row stride sz) into q [M, H] contiguous, when the product fits the
// grid, or as a hybrid up to kSwHybrid times that when the product buffer `a` is given (false, nothing launched,
// otherwise).
static bool launch_swiglu_once(const uint16_t *z, int64_t M, int64_t H, int64_t sz, uint16_t *a, uint8_t *q,
                               float *dequant, void *ws, hipStream_t st) {
  const int cap = once_capacity(reinterpret_cast<const void *>(&swiglu_once_kernel), g_cap_sw, kSwThreads);
  const int64_t nw = M * (H / 8);
  const int64_t held = (int64_t)kSwHeld * kSwThreads * cap;   // words the grid holds
  if (!once_enabled() || cap <= 0 || nw <= 0 || nw > kSwHybrid * held) return false;
  if (nw > held) {   // hybrid: every workgroup holds its full share, the rest goes through a
    if (!a) return false;
    const int64_t sgroups = (nw - held + kSwThreads - 1) / kSwThreads;
    swiglu_once_kernel<<<cap, kSwThreads, 0, st>>>(z, H, sz, (uint32_t)nw, kSwHeld, (uint32_t)sgroups, a, q, dequant,
                                                   ws, once_wait_ticks());
    return true;
  }
  const int64_t groups = (nw + kSwThreads - 1) / kSwThreads;   // groups of kSwThreads words
  const int grid = (int)std::min<int64_t>(groups, cap);
  const int wpt = (int)((groups + grid - 1) / grid);
  swiglu_once_kernel<<<grid, kSwThreads, 0, st>>>(z, H, sz, (uint32_t)nw, wpt, 0u, a, q, dequant, ws,
                                                  once_wait_ticks());
  return true;
}

// The single-pass SwiGLU backward cast of z [M, 2H], da [M, H] into dzq [M, 2H] contiguous (no dz), up to kBwHybrid
// times what the grid holds (false, nothing launched, above).
static bool launch_swiglu_bwd_once(const uint16_t *z, const uint16_t *da, int64_t M, int64_t H, int64_t sz,
                                   int64_t sda, uint8_t *dzq, float *dequant, void *ws, hipStream_t st) {
  const int cap = once_capacity(reinterpret_cast<const void *>(&swiglu_bwd_once_kernel), g_cap_bw, kSwThreads);
  const int64_t nu = M * (H / 8);
  const int64_t held = (int64_t)kBwHeld * kSwThreads * cap;   // units the grid holds
  if (!once_enabled() || cap <= 0 || nu <= 0 || nu > kBwHybrid * held) return false;
  int grid = cap, wpt = kBwHeld;
  int64_t sgroups = 0;
  if (nu > held) {   // hybrid: every workgroup holds its full share, the rest is computed twice
    sgroups = (nu - held + kSwThreads - 1) / kSwThreads;
  } else {
    const int64_t groups = (nu + kSwThreads - 1) / kSwThreads;
    grid = (int)std::min<int64_t>(groups, cap);
    wpt = (int)((groups + grid - 1) / grid);
  }
  swiglu_bwd_once_kernel<<<grid, kSwThreads, 0, st>>>(z, da, H, sz, sda, (uint32_t)nu, wpt, (uint32_t)sgroups, dzq,
                                                      dequant, ws, once_wait_ticks());
  return true;
}

// The single-pass transposing cast of a bf16 source when it fits (false, nothing launched, otherwise).
static bool launch_tcast_t_once(const uint16_t *x, int64_t rows, int64_t cols, uint8_t *q, uint8_t *qt, int64_t ldt,
                                float *dequant, void *ws, hipStream_t st) {
  const int cap = once_capacity(reinterpret_cast<const void *>(&cast_t_once_kernel), g_cap_t, 256);
  const int64_t tiles = ((cols + kTT - 1) / kTT) * ((ldt + kTT - 1) / kTT);
  if (!once_enabled() || cap <= 0 || tiles <= 0 || tiles > (int64_t)kHybridTiles * cap)
    return false;
  const int grid = (int)std::min<int64_t>(tiles, cap);
  cast_t_once_kernel<<<grid, 256, 0, st>>>(x, cols, rows, cols, q, cols, qt, ldt, dequant, ws, once_wait_ticks());
  return true;
}

// The grouped transposing cast when every tensor fits (false, nothing launched, otherwise): one tile per workgroup
// when the tiles fit the device at once, else two.
static bool launch_tcast_t_group(int count, const uint16_t *const *x, const int64_t *rows, const int64_t *cols,
                                 uint8_t *const *q, uint8_t *const *qt, const int64_t *ldt, float *const *dequant,
                                 void *ws, hipStream_t st) {
  const int cap = once_capacity(reinterpret_cast<const void *>(&cast_t_group_kernel), g_cap_tg, 256);
  if (!once_enabled() || cap <= 0 || count < 1 || count > kMaxTGroup) return false;
  int64_t tiles[kMaxTGroup], all = 0, halves = 0;
  for (int i = 0; i < count; i++) {
    tiles[i] = ((cols[i] + kTT - 1) / kTT) * ((ldt[i] + kTT - 1) / kTT);
    if (rows[i] <= 0 || tiles[i] <= 0) return false;
    all += tiles[i];
    halves += (tiles[i] + 1) / 2;
  }
  if (halves > cap) return false;
  TGroup g{};
  g.count = count;
  g.first[0] = 0;
  for (int i = 0; i < count; i++) {
    g.x[i] = x[i];
    g.q[i] = q[i];
    g.qt[i] = qt[i];
    g.dequant[i] = dequant[i];
    g.rows[i] = rows[i];
    g.cols[i] = cols[i];
    g.ldt[i] = ldt[i];
    g.first[i + 1] = g.first[i] + (int)(all <= cap ? tiles[i] : (tiles[i] + 1) / 2);
  }
  cast_t_group_kernel<<<g.first[count], 256, 0, st>>>(g, ws, once_wait_ticks());
  return true;
}

// ------------------------------------------------------------------------------------------- allocation-free cast
//
// gpic_fp8_tcast_noalloc: gpic_fp8_tcast with its workspace in this file's static device array `scratch` (one copy per
// GPU, held until the process ends) instead of a caller's buffer, for callers that cannot allocate. The host name
// `scratch` is only a stand-in for the device array: its device address is taken once per device with
// hipGetSymbolAddress (below) and only that address is ever passed to a kernel. The cast workspace has a fixed size
// (kCastWorkspaceBytes, whatever n is), which the array holds. Every call on one GPU shares the array and keeps what
// the last call left in it (the single-pass casts' epoch and tagged partials: state they expect to persist); calls
// that overlap on one GPU (several streams, or a graph replayed beside other casts on that GPU) race.
constexpr size_t kScratchBytes = kCastWorkspaceBytes;   // 44 KiB per GPU
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
static_assert(kCastWorkspaceBytes <= kScratchBytes, "the cast workspace must fit the static scratch array");

static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];   // the array's device address per device (guarded by g_scratch_mu)

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t *__restrict__ p, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

// The current device's scratch address, set up on the first call on that device: the symbol's address, then a
// clearing of the array on `st` (a fill kernel, not a memset: a caller may be capturing a graph) so that the
// single-pass state starts at zero, stream-ordered before the cast that follows on `st`.
static int scratch_address(hipStream_t st, void **out) {
  const int dev = current_device();
  if (dev < 0 || dev >= kMaxDevices) return GPIC_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!ptr || !aligned16(ptr)) return GPIC_EALIGN;
    zero_words_kernel<<<(int)(kScratchBytes / 4 + 255) / 256, 256, 0, st>>>(static_cast<uint32_t *>(ptr),
                                                                          (int)(kScratchBytes / 4));
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return GPIC_OK;
}

// SwiGLU kernels: rows strided over at most kSwigluBlocks workgroups (each builds its 24 KiB sigmoid table once).
static inline int swiglu_grid(int64_t M) { return (int)(M < 1 ? 1 : (M > kSwigluBlocks ? kSwigluBlocks : M)); }

}  // namespace gpic

using namespace gpic;

extern "C" {

size_t gpic_fp8_cast_workspace_bytes(void) { return kCastWorkspaceBytes; }

void gpic_fp8_set_single_pass(int enabled, int wait_us) {
  g_once_enabled.store(enabled != 0, std::memory_order_relaxed);
  g_once_wait_us.store(wait_us < 0 ? kOnceWaitUs : wait_us, std::memory_order_relaxed);
}

int gpic_fp8_tcast(const void *x, int dtype, int64_t n, uint8_t *q, float *dequant, void *ws, void *stream) {
  status_scope();
  if (n < 0 || !dequant || !ws || (n > 0 && (!x || !q))) return GPIC_EINVAL;
  if (dtype != GPIC_DTYPE_BF16 && dtype != GPIC_DTYPE_F32) return GPIC_EDTYPE;
  if (!aligned16(x) || !aligned16(q) || !aligned16(ws)) return GPIC_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  uint32_t *partial = static_cast<uint32_t *>(ws);
  if (dtype == GPIC_DTYPE_BF16) {
    const uint16_t *xb = static_cast<const uint16_t *>(x);
    if (launch_tcast_once(xb, n, q, dequant, ws, st)) return (int)hipGetLastError();
    return launch_tcast(xb, n, q, dequant, partial, st);
  }
  const float *xf = static_cast<const float *>(x);
  if (launch_tcast_once(xf, n, q, dequant, ws, st)) return (int)hipGetLastError();
  return launch_tcast(xf, n, q, dequant, partial, st);
}

int gpic_fp8_tcast_heads(const uint16_t *o, int64_t B, int64_t H, int64_t N, int64_t D, int64_t sb, int64_t sh,
                         int64_t sn, uint8_t *q, float *dequant, void *ws, void *stream) {
  status_scope();
  if (B < 0 || H < 0 || N < 0 || D < 0 || sb < 0 || sh < 0 || sn < 0 || !dequant || !ws) return GPIC_EINVAL;
  const int64_t big = 1ll << 31;   // every extent and stride below 2^31, so the products below stay exact
  if (D % 16 != 0 || B >= big || H >= big || N >= big || D >= big || sb >= big || sh >= big || sn >= big)
    return GPIC_ESHAPE;
  if (sb % 8 != 0 || sh % 8 != 0 || sn % 8 != 0) return GPIC_EALIGN;
  int64_t n = 0;
  if (__builtin_mul_overflow(B, H, &n) || __builtin_mul_overflow(n, N, &n) || __builtin_mul_overflow(n, D, &n))
    return GPIC_ESHAPE;
  if (n == 0) return gpic_fp8_tcast(o, GPIC_DTYPE_BF16, 0, q, dequant, ws, stream);
  if (!o || !q) return GPIC_EINVAL;
  if (!aligned16(o) || !aligned16(q) || !aligned16(ws)) return GPIC_EALIGN;
  // one past the last source word (each product below 2^62: the sum fits 64 unsigned bits)
  const uint64_t last = ((uint64_t)(B - 1) * sb + (uint64_t)(H - 1) * sh + (uint64_t)(N - 1) * sn + D) / 8;
  if (n / 8 >= big || last >= (uint64_t)big) return GPIC_ESHAPE;
  // [B, N, H, D] contiguous (a stride of a dimension of extent 1 does not matter): the flat cast of o
  if ((H == 1 || sh == D) && (N == 1 || sn == H * D) && (B == 1 || sb == N * H * D))
    return gpic_fp8_tcast(o, GPIC_DTYPE_BF16, n, q, dequant, ws, stream);
  const HeadMap map{fast_div((uint32_t)(D / 8)), fast_div((uint32_t)H), fast_div((uint32_t)N),
                    (uint32_t)(sb / 8), (uint32_t)(sh / 8), (uint32_t)(sn / 8)};
  hipStream_t st = (hipStream_t)stream;
  if (launch_tcast_once<uint16_t, HeadMap>(o, n, q, dequant, ws, st, map)) return (int)hipGetLastError();
  return launch_tcast<uint16_t, HeadMap>(o, n, q, dequant, static_cast<uint32_t *>(ws), st, map);
}

int gpic_fp8_tcast_noalloc(const void *x, int dtype, int64_t n, uint8_t *q, float *dequant, void *stream) {
  status_scope();
  // the arguments gpic_fp8_tcast checks, before the first call on a device sets its scratch up
  if (n < 0 || !dequant || (n > 0 && (!x || !q))) return GPIC_EINVAL;
  if (dtype != GPIC_DTYPE_BF16 && dtype != GPIC_DTYPE_F32) return GPIC_EDTYPE;
  if (!aligned16(x) || !aligned16(q)) return GPIC_EALIGN;
  if (gpic_fp8_cast_workspace_bytes() > kScratchBytes) return GPIC_EWORKSPACE;
  void *ws = nullptr;
  const int rc = scratch_address((hipStream_t)stream, &ws);
  if (rc != GPIC_OK) return rc;
  return gpic_fp8_tcast(x, dtype, n, q, dequant, ws, stream);
}

int gpic_fp8_tcast_t_group(int count, const void *const *x, int dtype, const int64_t *rows, const int64_t *cols,
                           uint8_t *const *q, uint8_t *const *qt, const int64_t *ldt, float *const *dequant, void *ws,
                           void *stream) {
  status_scope();
  if (count < 0 || (count > 0 && (!x || !rows || !cols || !q || !qt || !ldt || !dequant))) return GPIC_EINVAL;
  for (int i = 0; i < count; i++) {   // every tensor checked as gpic_fp8_tcast_t checks it, before anything is launched
    if (rows[i] < 0 || cols[i] < 0 || !dequant[i] || !ws || (rows[i] > 0 && cols[i] > 0 && !x[i]) ||
        (cols[i] > 0 && ldt[i] > 0 && !qt[i]))
      return GPIC_EINVAL;
    if (cols[i] % 16 != 0 || ldt[i] % 16 != 0 || ldt[i] < rows[i]) return GPIC_ESHAPE;
    if (dtype != GPIC_DTYPE_BF16 && dtype != GPIC_DTYPE_F32) return GPIC_EDTYPE;
    if (!aligned16(x[i]) || (q[i] && !aligned16(q[i])) || !aligned16(qt[i]) || !aligned16(ws)) return GPIC_EALIGN;
  }
  if (dtype == GPIC_DTYPE_BF16 &&
      launch_tcast_t_group(count, reinterpret_cast<const uint16_t *const *>(x), rows, cols, q, qt, ldt, dequant, ws,
                           (hipStream_t)stream))
    return (int)hipGetLastError();
  for (int i = 0; i < count; i++) {   // otherwise one call per tensor, in order
    const int rc = gpic_fp8_tcast_t(x[i], dtype, rows[i], cols[i], q[i], qt[i], ldt[i], dequant[i], ws, stream);
    if (rc != GPIC_OK) return rc;
  }
  return GPIC_OK;
}

int gpic_fp8_tcast_t(const void *x, int dtype, int64_t rows, int64_t cols, uint8_t *q, uint8_t *qt, int64_t ldt,
                     float *dequant, void *ws, void *stream) {
  status_scope();
  if (rows < 0 || cols < 0 || !dequant || !ws || (rows > 0 && cols > 0 && !x) || (cols > 0 && ldt > 0 && !qt))
    return GPIC_EINVAL;
  if (cols % 16 != 0 || ldt % 16 != 0 || ldt < rows) return GPIC_ESHAPE;
  if (dtype != GPIC_DTYPE_BF16 && dtype != GPIC_DTYPE_F32) return GPIC_EDTYPE;
  if (!aligned16(x) || (q && !aligned16(q)) || !aligned16(qt) || !aligned16(ws)) return GPIC_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  uint32_t *partial = static_cast<uint32_t *>(ws);
  if (dtype == GPIC_DTYPE_BF16 && rows > 0 && cols > 0 &&
      launch_tcast_t_once(static_cast<const uint16_t *>(x), rows, cols, q, qt, ldt, dequant, ws, st))
    return (int)hipGetLastError();
  const int64_t n = rows * cols;
  const int ga = grid_for((n / 16 + kUnroll - 1) / kUnroll, kAmaxBlocks);
  if (dtype == GPIC_DTYPE_BF16)
    launch_amax(static_cast<const uint16_t *>(x), n, ga, partial, st);
  else
    launch_amax(static_cast<const float *>(x), n, ga, partial, st);
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
  status_scope();
  if (M < 0 || H < 0 || !dequant || !ws || (M > 0 && H > 0 && (!z || !q))) return GPIC_EINVAL;
  if (H % 8 != 0 || sz % 8 != 0 || sq % 8 != 0 || sz < 2 * H || sq < H) return GPIC_ESHAPE;
  if (!aligned16(z) || !aligned16(q) || !aligned16(ws)) return GPIC_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  if (sq == H && launch_swiglu_once(z, M, H, sz, nullptr, q, dequant, ws, st)) return (int)hipGetLastError();
  uint32_t *partial = static_cast<uint32_t *>(ws);
  const int g = swiglu_grid(M);
  swiglu_amax_kernel<<<g, kCastThreads, 0, st>>>(z, M, H, sz, partial, ws_table(ws), nullptr);
  swiglu_cast_kernel<<<g, kCastThreads, 0, st>>>(z, M, H, sz, partial, g, q, sq, dequant, ws_table(ws));
  return (int)hipGetLastError();
}

int gpic_fp8_swiglu_tcast_t(const uint16_t *z, int64_t M, int64_t H, int64_t sz, uint16_t *a, uint8_t *q, int64_t sq,
                            uint8_t *qt, int64_t ldt, float *dequant, void *ws, void *stream) {
  status_scope();
  if (M < 0 || H < 0 || !dequant || !ws || (M > 0 && H > 0 && (!z || !q)) || (H > 0 && ldt > 0 && !qt))
    return GPIC_EINVAL;
  if (!qt && ldt != 0) return GPIC_EINVAL;
  if ((qt ? H % 16 : H % 8) != 0 || sz % 8 != 0 || sq % 8 != 0 || sz < 2 * H || sq < H || ldt % 16 != 0 ||
      (qt && ldt < M))
    return GPIC_ESHAPE;
  if (!aligned16(z) || !aligned16(a) || !aligned16(q) || !aligned16(qt) || !aligned16(ws)) return GPIC_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  uint32_t *partial = static_cast<uint32_t *>(ws);
  const int g = swiglu_grid(M);
  if (!qt) {   // q only, contiguous: the single pass (a hybrid through `a` when the product is larger than the grid
               // holds); else, with `a`, the product written once and cast flat; else recomputed
    if (sq == H && launch_swiglu_once(z, M, H, sz, a, q, dequant, ws, st)) return (int)hipGetLastError();
    const bool flat = a && sq == H;
    swiglu_amax_kernel<<<g, kCastThreads, 0, st>>>(z, M, H, sz, partial, ws_table(ws), flat ? a : nullptr);
    if (flat) {
      const int64_t n = M * H;
      const int gc = grid_for((n / 16 + kUnroll - 1) / kUnroll, kMaxCastBlocks);
      cast_kernel<uint16_t><<<gc, kCastThreads, 0, st>>>(a, n, partial, g, q, dequant);
    } else {
      swiglu_cast_kernel<<<g, kCastThreads, 0, st>>>(z, M, H, sz, partial, g, q, sq, dequant, ws_table(ws));
    }
    return (int)hipGetLastError();
  }
  // with `a`, the first pass writes the product and the cast reads it; without, the cast recomputes it from z
  swiglu_amax_kernel<<<g, kCastThreads, 0, st>>>(z, M, H, sz, partial, ws_table(ws), a);
  if (H == 0 || ldt == 0)
    cast_kernel<uint16_t><<<1, kCastThreads, 0, st>>>(nullptr, 0, partial, g, nullptr, dequant);
  else if (a)
    launch_cast_t(SrcBF16{a, H}, M, H, g, q, sq, qt, ldt, dequant, partial, st);
  else
    launch_cast_t(SrcSwiGLU{z, sz, H, ws_table(ws)}, M, H, g, q, sq, qt, ldt, dequant, partial, st);
  return (int)hipGetLastError();
}

static int swiglu_bwd_common(const uint16_t *z, const uint16_t *da, int64_t M, int64_t H, int64_t sz, int64_t sda,
                             uint16_t *dz, uint8_t *dzq, uint8_t *dzqt, int64_t ldt, float *dequant, void *ws,
                             hipStream_t st) {
  uint32_t *partial = static_cast<uint32_t *>(ws);
  const int g = swiglu_grid(M);
  if (!dz && !dzqt) {   // dzq straight from z and da: the single pass, or an amax pass and the recomputing flat cast
    if (launch_swiglu_bwd_once(z, da, M, H, sz, sda, dzq, dequant, ws, st)) return (int)hipGetLastError();
    swiglu_bwd_kernel<false><<<g, kCastThreads, 0, st>>>(z, da, M, H, sz, sda, nullptr, 0, partial, ws_table(ws));
    swiglu_bwd_cast_kernel<<<g, kCastThreads, 0, st>>>(z, da, M, H, sz, sda, partial, g, ws_table(ws), dzq, dequant);
    return (int)hipGetLastError();
  }
  if (!dz) {   // dzq and dzqt straight from z and da: an amax pass, then the recomputing transposing cast
    swiglu_bwd_kernel<false><<<g, kCastThreads, 0, st>>>(z, da, M, H, sz, sda, nullptr, 0, partial, ws_table(ws));
    const int64_t tiles = ((H + kTT - 1) / kTT) * ((ldt + kTT - 1) / kTT);
    const int grid = (int)std::min<int64_t>(std::max<int64_t>(tiles, 1), kSwigluCastTBlocks);
    swiglu_bwd_cast_t_kernel<<<grid, 256, 0, st>>>(z, da, M, H, sz, sda, partial, g, ws_table(ws), dzq, dzqt, ldt,
                                                   dequant);
    return (int)hipGetLastError();
  }
  swiglu_bwd_kernel<true><<<g, kCastThreads, 0, st>>>(z, da, M, H, sz, sda, dz, 2 * H, partial, nullptr);
  const int64_t n = M * 2 * H;
  if (dzqt && H > 0 && ldt > 0) {
    launch_cast_t(SrcBF16{dz, 2 * H}, M, 2 * H, g, dzq, 2 * H, dzqt, ldt, dequant, partial, st);
  } else {
    const int gc = grid_for((n / 16 + kUnroll - 1) / kUnroll, kMaxCastBlocks);
    cast_kernel<uint16_t><<<gc, kCastThreads, 0, st>>>(dz, n, partial, g, dzq, dequant);
  }
  return (int)hipGetLastError();
}

int gpic_fp8_swiglu_bwd(const uint16_t *z, const uint16_t *da, int64_t M, int64_t H, int64_t sz, int64_t sda,
                        uint16_t *dz, uint8_t *dzq, float *dequant, void *ws, void *stream) {
  status_scope();
  if (M < 0 || H < 0 || !dequant || !ws || (M > 0 && H > 0 && (!z || !da || !dzq))) return GPIC_EINVAL;
  if (H % 8 != 0 || sz % 8 != 0 || sda % 8 != 0 || sz < 2 * H || sda < H) return GPIC_ESHAPE;
  if (!aligned16(z) || !aligned16(da) || (dz && !aligned16(dz)) || !aligned16(dzq) || !aligned16(ws))
    return GPIC_EALIGN;
  return swiglu_bwd_common(z, da, M, H, sz, sda, dz, dzq, nullptr, 0, dequant, ws, (hipStream_t)stream);
}

int gpic_fp8_swiglu_bwd_t(const uint16_t *z, const uint16_t *da, int64_t M, int64_t H, int64_t sz, int64_t sda,
                          uint16_t *dz, uint8_t *dzq, uint8_t *dzqt, int64_t ldt, float *dequant, void *ws,
                          void *stream) {
  status_scope();
  if (M < 0 || H < 0 || !dequant || !ws || (M > 0 && H > 0 && (!z || !da || !dzq)) || (H > 0 && ldt > 0 && !dzqt) ||
      (!dz && M > 0 && H > 0 && ldt == 0))
    return GPIC_EINVAL;
  if (H % 8 != 0 || sz % 8 != 0 || sda % 8 != 0 || sz < 2 * H || sda < H || ldt % 16 != 0 || ldt < M)
    return GPIC_ESHAPE;
  if (!aligned16(z) || !aligned16(da) || (dz && !aligned16(dz)) || !aligned16(dzq) || !aligned16(dzqt) ||
      !aligned16(ws))
    return GPIC_EALIGN;
  return swiglu_bwd_common(z, da, M, H, sz, sda, dz, dzq, dzqt, ldt, dequant, ws, (hipStream_t)stream);
}

}  // extern "C"

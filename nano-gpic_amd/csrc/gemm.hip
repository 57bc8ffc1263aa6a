// Scaled FP8 (e4m3fn) GEMM for gfx950, "TN" layout: C[M, N] = bf16(sa * sb * A[M, K] . B[N, K]^T) (+ bias).
//
// Design (CDNA4):
//  * Macro tile BM x BN x 128 per workgroup; waves arranged WM x WN, each owning a (BM/WM) x (BN/WN) sub-tile made
//    of 16 x 16 MFMA tiles (v_mfma_f32_16x16x128_f8f6f4, both operands e4m3, fp32 accumulators).
//  * Global -> LDS with buffer_load_dwordx4 ... lds (no VGPR round trip). One wave instruction fills 1 KiB of LDS
//    = 8 rows x 128 bytes of K. Out-of-range rows / K chunks are handled by the buffer descriptor's range check
//    (they read as zeros), so any M and any K % 16 == 0 work without branches in the main loop.
//  * LDS rows are XOR-swizzled: 16-byte chunk c of row r lives in slot c ^ (r & 7), so the ds_read_b128 of 8
//    consecutive rows at the same K chunk hit 8 different bank groups.
//  * Two LDS stages: the loads of K tile t+1 are in flight while tile t is multiplied.
//  * The MFMA is issued as B-fragment x A-fragment, so each lane's 4 accumulators are 4 consecutive columns n of
//    one row m of C: the epilogue writes 8-byte (bf16) or 16-byte (fp32 partial) chunks.
//  * Tile order: workgroups are dealt to the 8 XCDs round robin; the id is remapped so each XCD walks a contiguous
//    range of tiles in groups of kGroupM tile rows (neighbouring workgroups share A and B panels in that XCD's L2).
//  * Split-K (for the small-output wgrad shapes): each split writes fp32 partials; a second kernel sums them in
//    split order (deterministic) and applies scale, bias and the bf16 rounding.
#include "gpic_device.h"
#include "gpic_launch.h"

namespace gpic {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
#define GPIC_LDS __attribute__((address_space(3)))

constexpr int kBK = 128;
constexpr int kGroupM = 4;
constexpr int kBufferFlags = 0x00020000;  // raw buffer descriptor word 3 for gfx9-family targets

template <int BM, int BN, int WM, int WN>
struct GemmCfg {
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kWTM = BM / WM, kWTN = BN / WN;
  static constexpr int kTM = kWTM / 16, kTN = kWTN / 16;
  static constexpr int kStageBytes = (BM + BN) * kBK;
  static constexpr int kLoadsPerWave = (BM + BN) / 8 / kWaves;
  static_assert((BM + BN) % (8 * kWaves) == 0, "rows per stage must split evenly over the waves");
  static_assert(kWTM % 16 == 0 && kWTN % 16 == 0, "wave tile must be a multiple of the 16x16 MFMA");
};

// Logical tile id for workgroup `bid` out of G: XCD x (= bid % 8) gets the contiguous range of ids
// [start_x, start_x + count_x).
__device__ __forceinline__ int xcd_remap(int bid, int G) {
  const int q = G >> 3, r = G & 7, x = bid & 7, i = bid >> 3;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + i;
}

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM *WN * 64) void gemm_tn_kernel(const uint8_t *__restrict__ A, int lda,
                                                               const uint8_t *__restrict__ B, int ldb,
                                                               const float *__restrict__ sa,
                                                               const float *__restrict__ sb,
                                                               const uint16_t *__restrict__ bias,
                                                               uint16_t *__restrict__ C, int64_t ldc,
                                                               float *__restrict__ P, int M, int N, int K, int ksplit,
                                                               int tiles_m, int tiles_n, int splits) {
  using Cfg = GemmCfg<BM, BN, WM, WN>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * Cfg::kStageBytes];
  // Declaring an AGPR clobber makes the compiler select the MFMA form that keeps accumulators in AGPRs, leaving
  // the 256 architectural VGPRs for operands and addresses.
  asm volatile("" ::: "a0");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;

  // ---- which tile / split this workgroup owns
  const int tiles = tiles_m * tiles_n;
  const int lid = xcd_remap(blockIdx.x, tiles * splits);
  const int split = lid / tiles;
  const int tile = lid % tiles;
  const int per_group = kGroupM * tiles_n;
  const int first_m = (tile / per_group) * kGroupM;
  const int gsz = min(tiles_m - first_m, kGroupM);
  const int tm = first_m + (tile % per_group) % gsz;
  const int tn = (tile % per_group) / gsz;
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = split * ksplit;
  const int kend = min(K, kbeg + ksplit);

  // ---- buffer descriptors covering this tile's rows of A and B (rows past M / N read as zero)
  const int rows_a = min(M - m0, BM), rows_b = min(N - n0, BN);
  const __amdgpu_buffer_rsrc_t rA =
      __builtin_amdgcn_make_buffer_rsrc((void *)(A + (int64_t)m0 * lda), 0, rows_a * lda, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rB =
      __builtin_amdgcn_make_buffer_rsrc((void *)(B + (int64_t)n0 * ldb), 0, rows_b * ldb, kBufferFlags);

  // ---- global -> LDS for one stage: wave instruction i covers stacked rows [R0, R0 + 8) of [A tile; B tile]
  auto issue = [&](int stage, int k0) {
    GPIC_LDS uint8_t *sbase = (GPIC_LDS uint8_t *)smem + stage * Cfg::kStageBytes;
#pragma unroll
    for (int i = 0; i < Cfg::kLoadsPerWave; i++) {
      const int R0 = (i * Cfg::kWaves + wave) * 8;
      const int s = lane & 7;
      if (R0 < BM) {
        const int r = R0 + (lane >> 3);
        const int kk = k0 + 16 * (s ^ (r & 7));
        const int voff = kk < kend ? r * lda + kk : (int)0x80000000;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (GPIC_LDS void *)(sbase + R0 * kBK), 16, voff, 0, 0, 0);
      } else {
        const int r = R0 - BM + (lane >> 3);
        const int kk = k0 + 16 * (s ^ (r & 7));
        const int voff = kk < kend ? r * ldb + kk : (int)0x80000000;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (GPIC_LDS void *)(sbase + R0 * kBK), 16, voff, 0, 0, 0);
      }
    }
  };

  // ---- one MFMA operand: row `row` of a stage's A or B area, K chunks 2g and 2g+1 (g = lane / 16)
  auto frag = [&](const GPIC_LDS uint8_t *base, int row) -> v8i {
    const int g = lane >> 4;
    const GPIC_LDS uint8_t *p = base + row * kBK;
    const u32x4 lo = *(const GPIC_LDS u32x4 *)(p + 16 * ((2 * g) ^ (row & 7)));
    const u32x4 hi = *(const GPIC_LDS u32x4 *)(p + 16 * ((2 * g + 1) ^ (row & 7)));
    return v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  };

  v4f acc[Cfg::kTN][Cfg::kTM];
#pragma unroll
  for (int i = 0; i < Cfg::kTN; i++)
#pragma unroll
    for (int j = 0; j < Cfg::kTM; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  const int nk = (kend - kbeg + kBK - 1) / kBK;
  if (nk > 0) issue(0, kbeg);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int st = kt & 1;
    if (kt + 1 < nk) issue(st ^ 1, kbeg + (kt + 1) * kBK);
    const GPIC_LDS uint8_t *sA = (const GPIC_LDS uint8_t *)smem + st * Cfg::kStageBytes;
    const GPIC_LDS uint8_t *sB = sA + BM * kBK;
    v8i af[Cfg::kTM];
#pragma unroll
    for (int mi = 0; mi < Cfg::kTM; mi++) af[mi] = frag(sA, wm * Cfg::kWTM + mi * 16 + (lane & 15));
#pragma unroll
    for (int ni = 0; ni < Cfg::kTN; ni++) {
      const v8i bf = frag(sB, wn * Cfg::kWTN + ni * 16 + (lane & 15));
#pragma unroll
      for (int mi = 0; mi < Cfg::kTM; mi++)
        acc[ni][mi] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf, af[mi], acc[ni][mi], 0, 0, 0, 0, 0, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

  // ---- epilogue: lane holds C[m][n..n+3] for each MFMA tile
  const float s = sa[0] * sb[0];
#pragma unroll
  for (int ni = 0; ni < Cfg::kTN; ni++) {
    const int n = n0 + wn * Cfg::kWTN + ni * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int mi = 0; mi < Cfg::kTM; mi++) {
      const int m = m0 + wm * Cfg::kWTM + mi * 16 + (lane & 15);
      if (m >= M || n >= N) continue;
      const v4f v = acc[ni][mi];
      if (P) {
        *reinterpret_cast<v4f *>(P + ((int64_t)split * M + m) * N + n) = v;
      } else {
        uint32_t h[4];
#pragma unroll
        for (int j = 0; j < 4; j++) h[j] = bf16_rne(v[j] * s);
        if (bias) {
          const u32x2 bw = *reinterpret_cast<const u32x2 *>(bias + n);
          h[0] = bf16_rne(bf16_lo(h[0]) + bf16_lo(bw.x));
          h[1] = bf16_rne(bf16_lo(h[1]) + bf16_hi(bw.x));
          h[2] = bf16_rne(bf16_lo(h[2]) + bf16_lo(bw.y));
          h[3] = bf16_rne(bf16_lo(h[3]) + bf16_hi(bw.y));
        }
        *reinterpret_cast<u32x2 *>(C + (int64_t)m * ldc + n) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
      }
    }
  }
}

// Sum of the split-K partials in split order, then the same epilogue as the single-pass kernel.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ P, int splits, int M, int N,
                                                            const float *__restrict__ sa, const float *__restrict__ sb,
                                                            const uint16_t *__restrict__ bias, uint16_t *__restrict__ C,
                                                            int64_t ldc) {
  const int64_t quads = (int64_t)M * (N / 4);
  const float s = sa[0] * sb[0];
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < quads; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / (N / 4);
    const int n = (int)(i % (N / 4)) * 4;
    v4f sum = *reinterpret_cast<const v4f *>(P + m * N + n);
    for (int z = 1; z < splits; z++) sum += *reinterpret_cast<const v4f *>(P + ((int64_t)z * M + m) * N + n);
    uint32_t h[4];
#pragma unroll
    for (int j = 0; j < 4; j++) h[j] = bf16_rne(sum[j] * s);
    if (bias) {
      const u32x2 bw = *reinterpret_cast<const u32x2 *>(bias + n);
      h[0] = bf16_rne(bf16_lo(h[0]) + bf16_lo(bw.x));
      h[1] = bf16_rne(bf16_lo(h[1]) + bf16_hi(bw.x));
      h[2] = bf16_rne(bf16_lo(h[2]) + bf16_lo(bw.y));
      h[3] = bf16_rne(bf16_lo(h[3]) + bf16_hi(bw.y));
    }
    *reinterpret_cast<u32x2 *>(C + m * ldc + n) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
  }
}

// ------------------------------------------------------------------------------------------- host side

constexpr int kBM = 256, kBN = 256, kWM = 2, kWN = 2;
using MainCfg = GemmCfg<kBM, kBN, kWM, kWN>;

struct Plan {
  int tiles_m, tiles_n, splits, ksplit;
};

static int num_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  }
  return cus;
}

// Split K only when the output has too few tiles to fill the chip and each split keeps >= 8 K tiles.
static Plan plan_gemm(int64_t M, int64_t N, int64_t K) {
  Plan p;
  p.tiles_m = (int)((M + kBM - 1) / kBM);
  p.tiles_n = (int)((N + kBN - 1) / kBN);
  const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
  const int64_t ktiles = (K + kBK - 1) / kBK;
  int splits = 1;
  const int cus = num_cus();
  while (tiles * splits < cus && ktiles / (splits * 2) >= 8) splits *= 2;
  const int64_t kt_per = (ktiles + splits - 1) / splits;
  p.ksplit = (int)(kt_per * kBK);
  p.splits = (int)((ktiles + kt_per - 1) / kt_per);
  return p;
}

}  // namespace gpic

using namespace gpic;

extern "C" {

size_t gpic_fp8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const Plan p = plan_gemm(M, N, K);
  return p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
}

int gpic_fp8_gemm(const uint8_t *A, int64_t lda, const float *sa, const uint8_t *B, int64_t ldb, const float *sb,
                  const uint16_t *bias, uint16_t *C, int64_t ldc, int64_t M, int64_t N, int64_t K, int fast_accum,
                  void *ws, size_t ws_bytes, void *stream) {
  (void)fast_accum;
  if (M < 0 || N < 0 || K < 0 || !sa || !sb || (M > 0 && N > 0 && !C)) return GPIC_EINVAL;
  if (K % 16 != 0 || N % 16 != 0 || lda % 16 != 0 || ldb % 16 != 0 || ldc % 8 != 0) return GPIC_ESHAPE;
  if (lda < K || ldb < K || ldc < N || lda >= (1 << 23) || ldb >= (1 << 23) || M >= (1 << 30) || N >= (1 << 30))
    return GPIC_ESHAPE;
  if (M == 0 || N == 0) return GPIC_OK;
  if (K > 0 && (!A || !B)) return GPIC_EINVAL;
  if (!aligned16(A) || !aligned16(B) || !aligned16(C) || (bias && ((uintptr_t)bias & 7u))) return GPIC_EALIGN;
  hipStream_t st = (hipStream_t)stream;
  const Plan p = K > 0 ? plan_gemm(M, N, K) : Plan{(int)((M + kBM - 1) / kBM), (int)((N + kBN - 1) / kBN), 1, kBK};
  float *P = nullptr;
  if (p.splits > 1) {
    const size_t need = (size_t)p.splits * M * N * sizeof(float);
    if (!ws || ws_bytes < need) return GPIC_EWORKSPACE;
    if (!aligned16(ws)) return GPIC_EALIGN;
    P = static_cast<float *>(ws);
  }
  const int grid = p.tiles_m * p.tiles_n * p.splits;
  gemm_tn_kernel<kBM, kBN, kWM, kWN><<<grid, MainCfg::kThreads, 0, st>>>(
      A, (int)lda, B, (int)ldb, sa, sb, bias, C, ldc, P, (int)M, (int)N, (int)K, p.ksplit, p.tiles_m, p.tiles_n,
      p.splits);
  if (P) {
    const int64_t quads = M * (N / 4);
    int64_t g = (quads + 255) / 256;
    if (g > 8192) g = 8192;
    splitk_reduce_kernel<<<(int)g, 256, 0, st>>>(P, p.splits, (int)M, (int)N, sa, sb, bias, C, ldc);
  }
  return (int)hipGetLastError();
}

}  // extern "C"

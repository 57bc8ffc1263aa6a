// Scaled FP8 (e4m3fn) GEMM for gfx950, "TN" layout: C[M, N] = bf16(sa * sb * A[M, K] . B[N, K]^T) (+ bias), and
// its "MN-major" instance for the wgrad, C = bf16(sa * sb * A[K, M]^T . B[K, N]) from operands stored with K as their row
// index: the same kernel, whose K tiles are then 128 K rows x 256 bytes in LDS and whose fragments are read with the
// transposing ds_read_b64_tr_b8 (bit-identical to the TN instance on the transposed operands).
//
// Design (CDNA4):
//  * Macro tile 256 x 256 x 128 per workgroup of 8 waves, two per SIMD. Wave w owns the 64 x 128 sub-tile
//    (rows 64 * (w >> 1), columns 128 * (w & 1)) as 4 x 8 MFMA tiles of v_mfma_f32_16x16x128_f8f6f4, one instruction
//    per tile and K tile (both operands e4m3, fp32 accumulators in VGPRs, so the epilogue's VALU work reads them
//    without AGPR copies). The 16 x 16 x 128 form does the 32 x 32 x 64 form's work per cycle at lower power, and this
//    kernel is power-bound on real data: repeated back-to-back MFMA-only loops on random e4m3 operands held the clock
//    at 1.87-1.95 GHz against 1.59-1.68 (single runs: within ~3%); this kernel, 20 calls per d12 shape, ran each shape
//    0.13-0.24 GHz faster and in 3-5% less time than with the 32 x 32 x 64 form.
//  * A narrow class, 256 x 128, for shapes whose 256 x 256 tiles leave CUs idle: each wave then owns 64 x 64, the B
//    K tile is 16 KiB; the host picks the width and the K split per shape, the same for both operand layouts.
//  * Ping-pong: waves 0-3 (group 0) and 4-7 (group 1) share the SIMDs pairwise and run one phase apart. In each
//    phase one group issues its 32 MFMAs of a K tile while the other reads its 12 fragments of that K tile from LDS,
//    with its share of a later K tile's loads between the reads (group 0 sends B one K tile ahead, group 1 sends A
//    two ahead); a workgroup barrier separates phases. The MFMA pipe of every SIMD sees the two groups' MFMA blocks
//    back to back. LDS: 3 A stages and 2 B stages of 32 KiB, all of gfx950's 160 KiB.
//  * Global -> LDS with buffer_load_dwordx4 ... lds (no VGPR round trip): one wave instruction fills 1 KiB of LDS =
//    8 rows x 128 bytes of K. Rows past M / N read as zeros through the buffer descriptor's range check; the last,
//    partial K tile masks its chunks the same way, so any M and any K % 16 == 0 need no branches in the main loop.
//    Per-lane offsets are computed once; the K position travels in the scalar soffset.
//  * LDS rows are XOR-swizzled: 16-byte chunk c of row r lives in slot c ^ ((r >> 1) & 7). gfx950's LDS serves
//    256 B per clock to 16 lanes at a time; the fragment reads of 16 consecutive rows at one chunk then hit 16
//    different 16-byte bank groups (measured: no SQ_LDS_BANK_CONFLICT cycles).
//  * The MFMA is issued as B-fragment x A-fragment with B's rows permuted in LDS (col_of), so each lane's
//    accumulators hold, for each pair of 16-column tiles, a run of 8 consecutive columns of one row of C. The bf16
//    epilogue rounds them, passes each 32-row block through LDS and stores 16 bytes per lane, whole 256-byte row
//    segments per 16 lanes; split-K partials go out as 16-byte fp32 stores straight from the accumulators.
//  * Persistent grid: work items (tile, K split) are dealt to the workgroups round robin and the id is remapped so
//    each XCD walks a contiguous range of tiles in groups of kGroupM tile rows (neighbouring workgroups share A and B
//    panels in that XCD's L2). The next item's first loads are issued before the current item's epilogue.
//  * Split-K (for the small-output wgrad shapes): each split writes fp32 partials; a second kernel sums them in
//    split order (deterministic) and applies scale, bias and the bf16 rounding.
#include <algorithm>

#include "gpic_device.h"
#include "gpic_launch.h"

namespace gpic {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
// Types for the C staging block in LDS and the bf16 stores: may_alias, since LDS holding fragments of A and B as
// one type is reused for C as another, and type-based alias analysis must not separate the two.
typedef float f4a_t __attribute__((ext_vector_type(4), __may_alias__));
typedef uint32_t st16_t __attribute__((ext_vector_type(4), __may_alias__));
typedef uint32_t st8_t __attribute__((ext_vector_type(2), __may_alias__));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
#define GPIC_LDS __attribute__((address_space(3)))

constexpr int kBM = 256, kBN = 256, kBK = 128;         // the wide tile (the narrow one is 256 x 128: kBNt)
constexpr int kThreads = 512;                          // 8 waves: 2 groups x 4
constexpr int kWTM = 64;                               // wave tile rows (columns: kWTNt, 128 or 64)
constexpr int kTM = kWTM / 16;                         // 16 x 16 MFMA tiles per wave in M: 4
constexpr int kHalfBytes = kBM * kBK;                  // 32 KiB: an A K tile (and a wide tile's B K tile)
constexpr int kAStages = 3, kBStages = 2;              // A is sent two K tiles ahead, B one
constexpr int kBBase = kAStages * kHalfBytes;          // B stages follow the A stages (160 KiB in all for the wide tile)
constexpr int kLoaders = 4;                            // waves of a group
constexpr int kLoads = kBM / 8 / kLoaders;             // 8 wave-instructions (1 KiB each) per A K tile per wave
constexpr int kGroupM = 4;
constexpr int kBufferFlags = 0x00020000;               // raw buffer descriptor word 3 for gfx9-family targets
constexpr int kOOB = (int)0x80000000;                  // an offset past any descriptor's range: reads zeros
// Cache policy of the bf16 C stores: nt (non-temporal). C is not read again by the kernel, and the streaming policy
// keeps each round's 32 MiB burst of C from displacing the A and B panels the XCD's other tiles still read from L2
// (12 d12 shapes: -3% GEMM time, the block step -2.3%, same process). The split-K partials keep the default policy:
// the reduce reads them back, and with nt it missed the cache (wgrads +30-80%).
constexpr int kStoreNT = 2;

__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }
// MN-major K tiles (rows of 256 bytes): 16-byte chunk c of K row r lives in slot c ^ mn_swz(r). A 16-lane group of a
// transposing read takes one chunk of 8 consecutive rows, and the two groups of a half-wave take the same chunk 32
// rows apart (K bytes 32 g of the fragment); the XOR with 2 (r & 7) | (r >> 5) & 1 sends those 16 chunks to 16
// different slots, i.e. all 64 banks.
__device__ __forceinline__ int mn_swz(int r) { return ((r & 7) << 1) | ((r >> 5) & 1); }
// The narrow tile's MN-major B K tile has rows of 128 bytes (8 chunks): chunk c of K row r lives in slot
// c ^ mn_swz_n(r). Two rows share a 256-byte bank window, so the 8 rows of a group hit 8 different 16-byte slots when
// the 4 rows of each parity XOR the chunk with 4 different even masks, and the two groups 32 rows apart differ in
// the lowest bit.
__device__ __forceinline__ int mn_swz_n(int r) { return (((r >> 1) & 3) << 1) | ((r >> 5) & 1); }

// The column of C that MFMA output row i of a pair of 16 x 16 tiles (i = 0..31: tile i / 16, row i % 16) stands for.
// Lane l holds output rows 4 (l / 16) + v, v = 0..3, of each tile; through this map those of tiles 2p and 2p + 1 are
// the columns 32 p + 8 (l / 16) + [0, 8), one run of 8. In bits: i = (h, g, v) with h = bit 4, g = bits 2-3,
// v = bits 0-1 maps to (g, h, v). A permutation of each aligned group of 32 rows; the loads take B row col_of(r) for
// LDS row r, and rows past N read as zeros through the descriptor's range whichever LDS row they land in.
__host__ __device__ constexpr int col_of(int i) {
  return (i & ~31) | (((i >> 2) & 3) << 3) | (((i >> 4) & 1) << 2) | (i & 3);
}
static_assert(col_of(3) == 3 && col_of(4) == 8 && col_of(16) == 4 && col_of(20) == 12 && col_of(31) == 31 &&
                  col_of(32 + 17) == 32 + 5,
              "col_of: tile bit 4 and row bits 2-3 of a pair of 16 x 16 tiles to column bits 2 and 3-4");

// Raw buffer descriptor (stride 0) over [base, base + bytes): offsets at or past `bytes` read as zero.
__device__ __forceinline__ v4i buffer_rsrc(const void *base, int bytes) {
  const uint64_t a = (uint64_t)base;
  return v4i{__builtin_amdgcn_readfirstlane((int)(uint32_t)a), __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffff)),
             __builtin_amdgcn_readfirstlane(bytes), kBufferFlags};
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const GPIC_LDS void *)p;
}

// LDS DMA: lane j loads 16 bytes at buffer offset voffset + soffset (range-checked on voffset) and the wave writes
// them to LDS [lds, lds + 1 KiB) in lane order. Written as asm so the compiler does not count it as an LDS store it
// has to order against later LDS reads: it would otherwise wait for every load in flight before reading the other
// stage. The waits these loads need are explicit at their uses (s_waitcnt vmcnt then a barrier). hipcc warns that
// the clobbered m0 is a reserved register: the compiler keeps no value in m0 across instructions (it sets m0 right
// before each instruction that reads it), so the clobber only states what the asm does.
__device__ __forceinline__ void lds_dma16(v4i rsrc, int voffset, int soffset, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voffset), "s"(rsrc), "s"(soffset), "s"(lds)
               : "memory", "m0");
}

// A uniform value the compiler must recompute where it is used: keeps it from hoisting the 16 per-load row offsets
// out of the K loop as 16 live registers (a scalar multiply and a v_add beside each load are free; registers are not).
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+s"(v));
  return v;
}

// The same for a per-lane value: the epilogue derives its addresses from an opaque copy of the lane index, so they
// are computed in the epilogue instead of being hoisted out of the tile loop and spilled across it.
__device__ __forceinline__ int opaque_v(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Logical tile id for workgroup `bid` out of G: XCD x (= bid % 8) gets the contiguous range of ids
// [start_x, start_x + count_x).
__device__ __forceinline__ int xcd_remap(int bid, int G) {
  const int q = G >> 3, r = G & 7, x = bid & 7, i = bid >> 3;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + i;
}

// kMN: both operands stored with K as their row index ("MN-major"): A [K, M] (row stride lda), B [K, N] (row stride
// ldb), C[m, n] = bf16(sa * sb * sum_k A[k, m] B[k, n]) -- the FP8 wgrad reading the untransposed e4m3 activations
// and gradients. A K tile of an operand is then 128 rows (K) x 256 bytes (MN) in LDS and its fragments are read with
// the transposing ds_read_b64_tr_b8.
// kBNt: the tile's width, 256 or 128 -- the narrow tile class for shapes whose 256 x 256 tiles leave CUs idle or end
// on a partial round: each wave then owns 64 x 64 of C, a B K tile is 16 KiB (MN-major: 128 K rows x 128 bytes).
template <bool kTail, bool kMN, int kBNt>
__global__ __launch_bounds__(kThreads) void gemm_tn_kernel(const uint8_t *__restrict__ A, int lda,
                                                            const uint8_t *__restrict__ B, int ldb,
                                                            const float *__restrict__ sa, const float *__restrict__ sb,
                                                            const uint16_t *__restrict__ bias, uint16_t *__restrict__ C,
                                                            int64_t ldc, float *__restrict__ P, int M, int N, int K,
                                                            int ksplit, int tiles_m, int tiles_n, int splits) {
  static_assert(kBNt == 256 || kBNt == 128, "tile widths: 256 or 128");
  constexpr int kWTNt = kBNt / 2;                 // wave tile columns
  constexpr int kTNt = kWTNt / 16;                // 16-column MFMA tiles per wave: 8 or 4
  constexpr int kHalfB = kBNt * kBK;              // one B K tile: 32 or 16 KiB
  constexpr int kLoadsB = kBNt / 8 / kLoaders;    // B loads per wave per K tile: 8 or 4
  constexpr int kRowB = kWTNt * 2;                // bytes of a row of a wave's bf16 C block: 256 or 128
  constexpr int kCStage = 32 * kRowB;             // a wave's 32-row C block on its way out
  static_assert(4 * kCStage <= kHalfBytes && 4 * kCStage <= kHalfB, "each group's C blocks fit one stage");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kAStages * kHalfBytes + kBStages * kHalfB];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = wave >> 2;
  const int wm = wave >> 1, wn = wave & 1;

  // ---- loads. A K tile of one operand is 256 rows x 128 bytes = 32 wave-instructions of 1 KiB, 8 per wave of a
  // group (the narrow tile's B K tile: 128 rows, 4 per wave). Instruction i of a wave fills rows [R0, R0 + 8), R0 = (i * 4 + wave % 4) * 8; lane j writes slot j & 7
  // of row R0 + j / 8, i.e. K chunk (j & 7) ^ swz(row). swz(row) does not depend on i, so every instruction's offset
  // is a per-lane base plus i * 32 rows. Row offsets stay in the VGPR offset (the part the descriptor
  // range-checks); only the K position goes to the scalar offset.
  const int lrow = (wave & 3) * 8 + (lane >> 3);
  const int kchunk = 16 * ((lane & 7) ^ swz(lrow));
  // B rows are permuted inside each group of 32: LDS row r holds B row col_of(r), so that each lane's accumulators
  // hold runs of 8 consecutive columns of C (see the epilogue).
  // MN-major: instruction i of a wave fills K rows [R0, R0 + 4), R0 = (i * 4 + wave % 4) * 4 = 16 i + mrow - lane / 16;
  // lane j writes 16-byte slot j & 15 of row 16 i + mrow, i.e. MN chunk (j & 15) ^ mn_swz(row), and mn_swz depends on
  // row & 7 = mrow & 7 only.
  const int mrow = (wave & 3) * 4 + (lane >> 4);
  const int mchunk = (lane & 15) ^ mn_swz(mrow);   // for K rows with bit 5 clear (i & 2 == 0); else mchunk ^ 1
  // MN-major B of the narrow tile: instruction i fills K rows [R0, R0 + 8), R0 = (i * 4 + wave % 4) * 8 =
  // 32 i + mrowB - lane / 8; lane j writes slot j & 7 of row 32 i + mrowB, i.e. MN chunk (j & 7) ^ mn_swz_n(row), and
  // mn_swz_n depends on (row / 2) & 3 = (mrowB / 2) & 3 and on bit 5 of the row, i & 1.
  const int mrowB = kBNt == 256 ? mrow : (wave & 3) * 8 + (lane >> 3);
  const int mchunkB = kBNt == 256 ? mchunk : (lane & 7) ^ mn_swz_n(mrowB);
  const int baseA = kMN ? mrow * lda + 16 * mchunk : lrow * lda + kchunk;
  const int baseB = kMN ? mrowB * ldb + 16 * mchunkB : col_of(lrow) * ldb + kchunk;
  // MN-major: the same loads for K rows with bit 5 set, whose chunks are swizzled with one more bit
  const int baseA1 = mrow * lda + 16 * (mchunk ^ 1);
  const int baseB1 = mrowB * ldb + 16 * (mchunkB ^ 1);
  const float s = sa[0] * sb[0];

  // ---- persistent: work item `it` (a tile and a K split) goes to workgroup it % gridDim.x. The grid is a multiple
  // of 8 (or covers every item in one pass), so it & 7 is the XCD the workgroup runs on and xcd_remap gives each
  // XCD a contiguous range of tiles.
  const int tiles = tiles_m * tiles_n;
  const int work = tiles * splits;
  struct Item {
    int m0, n0, split, kbeg, kend, nk;
    v4i rA, rB;   // buffer descriptors over the item's rows of A and B (rows past M / N read as zero)
    int voA, voB; // MN-major: this lane's load offsets, or kOOB where its chunk lies past M / N
    int voA1, voB1; // the same for K rows with bit 5 set
  };
  auto item = [&](int it) {
    Item w;
    const int lid = xcd_remap(it, work);
    w.split = lid / tiles;
    const int tile = lid % tiles;
    const int per_group = kGroupM * tiles_n;
    const int first_m = (tile / per_group) * kGroupM;
    const int gsz = min(tiles_m - first_m, kGroupM);
    w.m0 = (first_m + (tile % per_group) % gsz) * kBM;
    w.n0 = ((tile % per_group) / gsz) * kBNt;
    w.kbeg = w.split * ksplit;
    w.kend = min(K, w.kbeg + ksplit);
    w.nk = (w.kend - w.kbeg + kBK - 1) / kBK;
    if constexpr (kMN) {   // descriptors from the item's first column to the end of the matrix (K x ld bytes)
      w.rA = buffer_rsrc(A + w.m0, K * lda - w.m0);
      w.rB = buffer_rsrc(B + w.n0, K * ldb - w.n0);
      w.voA = w.m0 + 16 * mchunk < M ? baseA : kOOB;
      w.voB = w.n0 + 16 * mchunkB < N ? baseB : kOOB;
      w.voA1 = w.m0 + 16 * (mchunk ^ 1) < M ? baseA1 : kOOB;
      w.voB1 = w.n0 + 16 * (mchunkB ^ 1) < N ? baseB1 : kOOB;
    } else {
      w.rA = buffer_rsrc(A + (int64_t)w.m0 * lda, min(M - w.m0, kBM) * lda);
      w.rB = buffer_rsrc(B + (int64_t)w.n0 * ldb, min(N - w.n0, kBNt) * ldb);
      w.voA = w.voB = w.voA1 = w.voB1 = 0;
    }
    return w;
  };

  // Load i (of 8) of this wave's share of operand `isA ? A : B`'s K tile at k0 of item w, into the LDS half stage at
  // byte offset `dst`. The stride of 32 rows is opaque, so each load's offset is a scalar multiply here rather than a
  // register held across the loop for each load. In the last, partial K tile (kTail instance only), chunks at or past
  // kend read zeros.
  auto load = [&](const Item &w, bool isA, int dst, int k0, int i) {
    if constexpr (kMN && kBNt == 128) {
      if (!isA) {   // the narrow B K tile: K rows k0 + 32 i + mrowB, 128 bytes each
        const int R0 = (i * kLoaders + (wave & 3)) * 8;
        const int vo = ((i & 1) ? w.voB1 : w.voB) + i * opaque(32 * ldb);   // (K row bit 5 = i & 1)
        const uint32_t to = lds_addr(smem) + dst + R0 * 128;
        if (!kTail || k0 + kBK <= w.kend) lds_dma16(w.rB, vo, k0 * ldb, to);
        else lds_dma16(w.rB, k0 + 32 * i + mrowB < w.kend ? vo + k0 * ldb : kOOB, 0, to);
        return;
      }
    }
    if constexpr (kMN) {
      // K rows k0 + 16 i + mrow; the K position goes to the scalar offset (k0 * ld), the row within the tile and the
      // chunk to the lane's; lanes whose chunk lies past M / N start from kOOB
      const int ld = isA ? lda : ldb;
      const int R0 = (i * kLoaders + (wave & 3)) * 4;
      // (kOOB + these offsets stays in [2^31, 2^32): still past the range, which is below 2^31)
      const int vo = ((i & 2) ? (isA ? w.voA1 : w.voB1) : (isA ? w.voA : w.voB)) + i * opaque(16 * ld);   // (bit 5 = i & 2)
      const uint32_t to = lds_addr(smem) + dst + R0 * 256;
      if (!kTail || k0 + kBK <= w.kend) lds_dma16(isA ? w.rA : w.rB, vo, k0 * ld, to);
      else lds_dma16(isA ? w.rA : w.rB, k0 + 16 * i + mrow < w.kend ? vo + k0 * ld : kOOB, 0, to);
    } else {
      const int R0 = (i * kLoaders + (wave & 3)) * 8;
      const int vo = isA ? baseA + i * opaque(32 * lda) : baseB + i * opaque(32 * ldb);
      const uint32_t to = lds_addr(smem) + dst + R0 * kBK;
      if (!kTail || k0 + kBK <= w.kend) lds_dma16(isA ? w.rA : w.rB, vo, k0, to);
      else lds_dma16(isA ? w.rA : w.rB, k0 + kchunk < w.kend ? vo + k0 : kOOB, 0, to);
    }
  };
  auto a_half = [](int stage) { return stage * kHalfBytes; };
  auto b_half = [](int stage) { return kBBase + stage * kHalfB; };
  // Group 0 sends an item's first loads: A(0), B(0) and, with a second K tile, A(1) (16 + 8 per wave).
  auto send_prologue = [&](const Item &w) {
    if (w.nk > 0) {
#pragma unroll
      for (int i = 0; i < kLoads; i++) load(w, true, a_half(0), w.kbeg, i);
#pragma unroll
      for (int i = 0; i < kLoadsB; i++) load(w, false, b_half(0), w.kbeg, i);
    }
    if (w.nk > 1) {
#pragma unroll
      for (int i = 0; i < kLoads; i++) load(w, true, a_half(1), w.kbeg + kBK, i);
    }
  };

  // ---- fragments of one K tile: 16 x 16 x 128 operands, row (lane & 15), 32 bytes at K 32 * (lane >> 4).
  // Fragment j: j < kTM is A fragment j, otherwise B fragment j - kTM; two ds_read_b128 each.
  v8i fa[kTM], fb[kTNt];
  const int frow = lane & 15;
  const int fsw = swz(frow);                 // swz of every fragment row: the tile offsets are multiples of 16
  const int c0 = 2 * (lane >> 4);
  // MN-major: a fragment is 4 ds_read_b64_tr_b8. In each 16-lane group g = lane / 16, source lane s = lane % 16 reads
  // 8 bytes of K row 32 g + 8 q + s / 2, MN bytes mnb + 8 (s % 2) + [0, 8); the transposing read hands output lane j
  // of the group byte r of source lane 2 r + j / 8, i.e. K row 32 g + 8 q + r of MN index mnb + j: lane l gets MN
  // index mnb + (l & 15) and K 32 (l / 16) + 8 q + [0, 8) in bytes 8 q .. 8 q + 7 of its operand -- the layout of the
  // K-major fragment. The chunk mnb / 16 of K row 32 g + 8 q + s / 2 sits in slot (mnb / 16) ^ mn_swz(row), and
  // mn_swz of those rows does not depend on q.
  const int tr_g = lane >> 4, tr_s = lane & 15;
  const int tr_row = 32 * tr_g + (tr_s >> 1);
  const int tr_off = tr_row * 256 + 8 * (tr_s & 1);
  const int tr_x = 16 * mn_swz(tr_row);
  // (the narrow tile's B: rows of 128 bytes, chunk (mnb / 16) ^ mn_swz_n(row))
  const int tr_offB = kBNt == 256 ? tr_off : tr_row * 128 + 8 * (tr_s & 1);
  const int tr_xB = kBNt == 256 ? tr_x : 16 * mn_swz_n(tr_row);
  auto read_frag = [&](int ast, int bst, int j) {
    const int f = j;
    if constexpr (kMN) {
      const int mnb = f < kTM ? wm * kWTM + f * 16 : wn * kWTNt + (f - kTM) * 16;
      const int rowb = f < kTM ? 256 : kBNt;   // bytes per K row of the operand's K tile
      const GPIC_LDS uint8_t *p =
          kBNt == 256 ? (const GPIC_LDS uint8_t *)smem + (f < kTM ? a_half(ast) : b_half(bst)) + tr_off + (mnb ^ tr_x)
                      : (const GPIC_LDS uint8_t *)smem +
                            (f < kTM ? a_half(ast) + tr_off + (mnb ^ tr_x) : b_half(bst) + tr_offB + (mnb ^ tr_xB));
      v2i r[4];
#pragma unroll
      for (int q = 0; q < 4; q++) r[q] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((GPIC_LDS v2i *)(p + q * 8 * rowb));
      const v8i v{r[0].x, r[0].y, r[1].x, r[1].y, r[2].x, r[2].y, r[3].x, r[3].y};
      if (f < kTM) fa[f] = v;
      else fb[f - kTM] = v;
      return;
    }
    const int lo = 16 * (c0 ^ fsw), hi = 16 * ((c0 + 1) ^ fsw);
    const GPIC_LDS uint8_t *p = (const GPIC_LDS uint8_t *)smem +
                                (f < kTM ? a_half(ast) + (wm * kWTM + f * 16 + frow) * kBK
                                         : b_half(bst) + (wn * kWTNt + (f - kTM) * 16 + frow) * kBK);
    const u32x4 x0 = *(const GPIC_LDS u32x4 *)(p + lo), x1 = *(const GPIC_LDS u32x4 *)(p + hi);
    const v8i v{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
    if (f < kTM) fa[f] = v;
    else fb[f - kTM] = v;
  };
  // A memory phase: the wave's 12 fragment reads of K tile (ast, bst), with its 8 loads of one operand's later K
  // tile between them when `send`. A load issue waits while the texture unit's queue is full; with the reads in
  // between, the LDS works through the reads during those waits.
  // (The narrow tile: 8 fragment reads, with the 8 A or 4 B loads spread evenly between them.)
  auto mem_phase = [&](const Item &w, int ast, int bst, bool send, bool isA, int dst, int k0) {
    if constexpr (kBNt == 256) {
      static_assert(kTM + kTNt == 12 && kLoads == 8 && kLoadsB == 8, "interleave pattern: 3 fragments per 2 loads");
#pragma unroll
      for (int j = 0; j < 4; j++) {
        read_frag(ast, bst, 3 * j);
        if (send) load(w, isA, dst, k0, 2 * j);
        read_frag(ast, bst, 3 * j + 1);
        read_frag(ast, bst, 3 * j + 2);
        if (send) load(w, isA, dst, k0, 2 * j + 1);
      }
    } else {
      constexpr int R = kTM + kTNt;
#pragma unroll
      for (int j = 0; j < R; j++) {
        read_frag(ast, bst, j);
        if (send) {
          if (isA) {
#pragma unroll
            for (int i = j * kLoads / R; i < (j + 1) * kLoads / R; i++) load(w, true, dst, k0, i);
          } else {
#pragma unroll
            for (int i = j * kLoadsB / R; i < (j + 1) * kLoadsB / R; i++) load(w, false, dst, k0, i);
          }
        }
      }
    }
  };

  // Phase boundary: a bare s_barrier (no fence: the waits each side needs are explicit, so the loads issued in a
  // memory phase stay in flight through it), pinned with sched_barrier so the compiler cannot move MFMAs
  // (register-only instructions) across it into the other group's phase.
  auto phase_barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // The waits below count vector-memory operations: on this target (no separate store counter) loads, LDS-DMA
  // loads and stores all retire in issue order through one vmcnt, as the compiler itself assumes for gfx9 targets.
  // Group 0's prologue wait: its A(0) and B(0) have landed once at most the 8 loads of A(1) (when sent) and the
  // `pend` stores it issued after them are still in flight; the stores of the previous item drain meanwhile.
  auto wait_prologue = [](bool two, int pend) {
    if (pend == 0) {
      if (two) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else if (kBNt == 128 && pend == 8) {   // (the narrow tile's pend is 0, 8 or 16; the wide one's 0, 16 or 32)
      if (two) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    } else if (kBNt == 128 || pend == 16) {
      if (two) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    } else {
      if (two) asm volatile("s_waitcnt vmcnt(40)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
    }
  };
  constexpr int kStoresBF16 = (kTM / 2) * (32 * kRowB / 1024);   // bf16 epilogue: 16 (narrow: 8) buffer stores per wave, always issued
  constexpr int kStoresF32 = kTNt * kTM;                         // split-K partials: 32 (narrow: 16)

  int it = blockIdx.x;
  Item cur = item(it);
  if (group == 0) send_prologue(cur);
  int pend = 0;   // stores group 0 issued after the current item's prologue loads
  for (;;) {
    v4f acc[kTNt][kTM];
#pragma unroll
    for (int i = 0; i < kTNt; i++)
#pragma unroll
      for (int j = 0; j < kTM; j++) acc[i][j] = v4f{};

    // K tile t: A half in A stage t % 3, B half in B stage t % 2. Group 0 reads tile kt in phase 2 kt and multiplies
    // in 2 kt + 1; group 1 reads it in 2 kt + 1 and multiplies in 2 kt + 2. The loads are spread over both kinds of
    // phase, each side's between its own fragment reads: group 0 sends B(kt + 1) in phase 2 kt and waits for it at
    // the end of 2 kt + 1; group 1 sends A(kt + 2) in phase 2 kt + 1 and waits for it at the end of 2 kt + 3 (after
    // sending A(kt + 3): vmcnt(8) leaves only those 8 in flight). Every stage written in a phase was last read two
    // phases before: B stage (kt + 1) % 2 held tile kt - 1 (read in 2 kt - 2, 2 kt - 1); A stage (kt + 2) % 3 held
    // tile kt - 1 as well.
    // Prologue: group 0 sent A(0), B(0) and A(1) (before the previous item's epilogue, or above for the first) and
    // waits for the first two; all meet; group 1 then passes one extra barrier to run one phase behind group 0. A(1)
    // is waited for by group 0 with B(1), at the end of phase 1.
    if (group == 0) wait_prologue(cur.nk > 1, pend);
    phase_barrier();
    if (group == 1) phase_barrier();
    int ast = 0;   // A stage of K tile kt
    for (int kt = 0; kt < cur.nk; ++kt) {
      const int bst = kt & 1;
      // memory phase
      if (group == 0) {
        mem_phase(cur, ast, bst, kt + 1 < cur.nk, false, b_half(bst ^ 1), cur.kbeg + (kt + 1) * kBK);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // done reading the stages before anyone overwrites them
      } else {
        mem_phase(cur, ast, bst, kt + 2 < cur.nk, true, a_half(ast == 0 ? 2 : ast - 1), cur.kbeg + (kt + 2) * kBK);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (opaque(kt) > 0) {   // A(kt + 1) has landed (A(1) is group 0's, waited for by group 0); opaque: no peeled copy of the first iteration
          if (kt + 2 < cur.nk) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
          else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
      }
      phase_barrier();
      // MFMA phase
#pragma unroll
      for (int ni = 0; ni < kTNt; ni++)
#pragma unroll
        for (int mi = 0; mi < kTM; mi++)
          acc[ni][mi] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fb[ni], fa[mi], acc[ni][mi], 0, 0, 0, 0, 0, 0);
      if (group == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // B(kt + 1) (and A(1)) have landed
      phase_barrier();
      ast = ast == 2 ? 0 : ast + 1;
    }
    if (group == 0) phase_barrier();

    // ---- the next item's first loads go out now (into A stages 0, 1 and B stage 0: nothing reads them any more),
    // so their latency passes during this item's epilogue
    const int nit = it + gridDim.x;
    const bool more = nit < work;
    if (more && group == 0) send_prologue(item(nit));

    // ---- epilogue: acc[ni][mi] lane l holds C[m][n + v], v = 0..3, for m = mi * 16 + (l & 15) and, through col_of,
    // n = 32 (ni / 2) + 8 (l >> 4) + 4 (ni % 2) (MN-major, in natural order: n = 16 ni + 4 (l >> 4)): 4 consecutive
    // columns per tile, a run of 8 per pair of tiles in the K-major instance. Every store is a buffer store issued by
    // every wave (lanes outside M x N get an offset past the descriptor's range and write nothing), so group 0 knows
    // exactly how many stores follow its prologue loads.
    const int el = opaque_v(lane);
    const int rows_c = min(M - cur.m0, kBM);
    const int wr = el & 15, wg = el >> 4;
    if (P) {   // split-K fp32 partials
      const __amdgpu_buffer_rsrc_t rP = __builtin_amdgcn_make_buffer_rsrc(
          (void *)(P + ((int64_t)cur.split * M + cur.m0) * N), 0, rows_c * N * 4, kBufferFlags);
#pragma unroll
      for (int ni = 0; ni < kTNt; ni++)
#pragma unroll
        for (int mi = 0; mi < kTM; mi++) {
          const int r = wm * kWTM + mi * 16 + wr;
          const int n = cur.n0 + wn * kWTNt + (kMN ? 16 * ni + 4 * wg : 32 * (ni >> 1) + 8 * wg + 4 * (ni & 1));
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[ni][mi]), rP,
                                                 r < rows_c && n < N ? (r * N + n) * 4 : kOOB, 0, 0);
        }
      pend = kStoresF32;
    } else {
      // bf16 output through LDS: each lane rounds its runs of 8 columns (scaled) to bf16 and writes them to LDS as
      // 16 bytes (MN-major: its runs of 4 as 8 bytes), one 32 x 128 block (two 16-row tile rows) of the wave at a
      // time; each lane then reads back 16 bytes of one row, adds the bias (a second rounding, as the reference) and
      // stores them, 16 lanes to a 256-byte row segment of C. A block row is 256 bytes; 16-byte chunk c of row r sits
      // in slot c ^ (r & 15) (conflict-free both ways). Each wave uses its own 8 KiB: group 0 in A stage 2, group 1 in
      // B stage 1. The next item's prologue loads go to A stages 0, 1 and B stage 0; the first loads into A stage 2
      // and B stage 1 come after the next item's first barrier, which group 1 reaches only when its epilogue is done.
      // The narrow tile's block rows are 128 bytes (8 chunks): chunk c of row r sits in slot c ^ ((r / 2) & 7), so the
      // 16 lanes of a write (rows r..r+15 at one chunk) or of a read-back (two rows) cover all 64 banks.
      GPIC_LDS uint8_t *cst =
          (GPIC_LDS uint8_t *)smem + (group == 0 ? a_half(2) : b_half(1)) + (wave & 3) * kCStage;
      const __amdgpu_buffer_rsrc_t rC =
          __builtin_amdgcn_make_buffer_rsrc((void *)(C + (int64_t)cur.m0 * ldc), 0, rows_c * (int)ldc * 2, kBufferFlags);
      constexpr int kLPR = kRowB / 16, kRPI = 64 / kLPR;   // read-back: lanes per row, rows per instruction
      auto slot = [](int c, int r) { return kBNt == 256 ? c ^ (r & 15) : c ^ ((r >> 1) & 7); };
      const int rr = (unsigned)el / kLPR, rc = (unsigned)el % kLPR;   // read-back: rows kRPI j + rr, chunk rc
      const int n = cur.n0 + wn * kWTNt + 8 * rc;   // the read-back lane's 8 columns
      uint32_t b[4] = {0, 0, 0, 0};
      if (bias && n < N) {
        const u32x2 b0 = *reinterpret_cast<const u32x2 *>(bias + n), b1 = *reinterpret_cast<const u32x2 *>(bias + n + 4);
        b[0] = b0.x, b[1] = b0.y, b[2] = b1.x, b[3] = b1.y;
      }
#pragma unroll
      for (int mq = 0; mq < kTM / 2; mq++) {
#pragma unroll
        for (int h2 = 0; h2 < 2; h2++) {   // the block's two 16-row tile rows
          const int mi = 2 * mq + h2, row = 16 * h2 + wr;
          if constexpr (kMN) {
            // natural column order: a run of 4 (columns 16 ni + 4 wg + [0, 4)) per tile, 8 bytes into half wg % 2 of
            // chunk 2 ni + wg / 2
#pragma unroll
            for (int ni = 0; ni < kTNt; ni++) {
              const v4f &v = acc[ni][mi];
              *(GPIC_LDS st8_t *)(cst + row * kRowB + 16 * slot(2 * ni + (wg >> 1), row) + 8 * (wg & 1)) =
                  st8_t{pack_bf16(v[0] * s, v[1] * s), pack_bf16(v[2] * s, v[3] * s)};
            }
          } else {
            // tiles 2 p and 2 p + 1: columns 32 p + 8 wg + [0, 8), chunk 4 p + wg
#pragma unroll
            for (int pp = 0; pp < kTNt / 2; pp++) {
              const v4f &a = acc[2 * pp][mi], &b2 = acc[2 * pp + 1][mi];
              *(GPIC_LDS st16_t *)(cst + row * kRowB + 16 * slot(4 * pp + wg, row)) =
                  st16_t{pack_bf16(a[0] * s, a[1] * s), pack_bf16(a[2] * s, a[3] * s), pack_bf16(b2[0] * s, b2[1] * s),
                         pack_bf16(b2[2] * s, b2[3] * s)};
            }
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the block is complete before any lane reads it back
        // all 8 rows read back first (their latencies overlap; a store between them would order them), then stored
        constexpr int kNI = 32 / kRPI;   // read-back instructions per block: 8 (narrow: 4)
        st16_t wv[kNI];
#pragma unroll
        for (int j = 0; j < kNI; j++) {
          const int r = kRPI * j + rr;
          wv[j] = *(const GPIC_LDS st16_t *)(cst + r * kRowB + 16 * slot(rc, r));
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // read back before the next block overwrites it
        const int rl0 = wm * kWTM + mq * 32 + rr;   // row within the tile of j = 0; row j is rl0 + kRPI j
        int off = (rl0 * (int)ldc + n) * 2;
#pragma unroll
        for (int j = 0; j < kNI; j++) {
          st16_t w = wv[j];
          if (bias) {   // bf16(bf16(acc * s) + bias)
#pragma unroll
            for (int e = 0; e < 4; e++) w[e] = pack_bf16(bf16_lo(w[e]) + bf16_lo(b[e]), bf16_hi(w[e]) + bf16_hi(b[e]));
          }
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, w), rC,
                                                 rl0 + kRPI * j < rows_c && n < N ? off : kOOB, 0, kStoreNT);
          off += 2 * kRPI * (int)ldc;
        }
      }
      pend = kStoresBF16;
    }
    if (!more) break;
    it = nit;
    cur = item(opaque(nit));   // recomputed rather than kept live through the epilogue
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
    u32x2 w{pack_bf16(sum[0] * s, sum[1] * s), pack_bf16(sum[2] * s, sum[3] * s)};
    if (bias) {   // the output is rounded, then the bias add is rounded again
      const u32x2 bw = *reinterpret_cast<const u32x2 *>(bias + n);
      w.x = pack_bf16(bf16_lo(w.x) + bf16_lo(bw.x), bf16_hi(w.x) + bf16_hi(bw.x));
      w.y = pack_bf16(bf16_lo(w.y) + bf16_lo(bw.y), bf16_hi(w.y) + bf16_hi(bw.y));
    }
    *reinterpret_cast<u32x2 *>(C + m * ldc + n) = w;
  }
}

// ------------------------------------------------------------------------------------------- host side

struct Plan {
  int tiles_m, tiles_n, splits, ksplit, bn;   // bn: the tile width, 256 or 128
};

// Compute units of the current device (cached per device).
static DeviceCache g_cus;
struct CusInit {
  CusInit() {
    for (int i = 0; i < kMaxDevices; i++) g_cus[i] = -1;
  }
};
static CusInit g_cus_init;
static int num_cus() { return per_device(g_cus, device_cus); }

// The plan: for each tile width, the number of K splits s (and K tiles per split) that minimises a model of the run
// time; then the width. Work items
// (tiles x splits) run in rounds of one per CU; a round lasts as long as its items' K tiles plus a fixed cost per
// item (prologue, epilogue); splitting adds the reduce, which reads s fp32 partials of C and writes C. Model constants
// from measured d12 and text-block shapes: a K tile takes ~1.45 us with every CU busy and less when a single round
// leaves CUs idle (1.0 + 0.45 x the busy fraction: 1.03-1.18 us measured at 104 of 256), ~4 us per item (5 with fp32
// partials), and the reduce ~4 us plus its bytes at ~5 TB/s. Split-K also needs N < 2^21 (the partials' 32-bit
// buffer offsets).
// The tile width: the 256 x 128 tile does half the work per item at ~0.59 of the time per K tile (measured over
// full rounds of d12 shapes: 0.57-0.60) and ~3 us per item, so it wins where it fills CUs that 256 x 256 tiles leave
// idle (text-block shapes: 104 tiles of 256 x 256 on 256 CUs), evens out a partial last round, or needs fewer K
// splits. The best narrow plan (over its own split counts) is taken only for a predicted gain of 10% or more over the
// best wide one: the model treats a partial last round of several as a full one, and near-ties went either way when
// measured (text qkv.fwd: 3 narrow rounds vs 2 wide ones, 29.4 vs 30.0 us on one box, 33.3 vs 31.1 on another). Both
// operand layouts use the same plan, so they sum the same partials in the same order: their results are the same bits.
constexpr double kNarrowKTile = 0.59, kNarrowItem = 3.0, kNarrowGain = 0.9;
static Plan plan_gemm(int64_t M, int64_t N, int64_t K) {
  const int64_t ktiles = (K + kBK - 1) / kBK;
  const int64_t cus = num_cus();
  const int64_t tiles_m = (M + kBM - 1) / kBM;
  const int64_t max_splits = N < (1 << 21) ? std::min<int64_t>(ktiles, 64) : 1;
  Plan best[2];
  double tbest[2] = {0.0, 0.0};
  for (int c = 0; c < 2; c++) {
    const int bn = c == 0 ? 256 : 128;
    const double ktile = c == 0 ? 1.0 : kNarrowKTile, fixed = c == 0 ? 4.0 : kNarrowItem;
    const int64_t tiles = tiles_m * ((N + bn - 1) / bn);
    best[c] = Plan{(int)tiles_m, (int)((N + bn - 1) / bn), 1, (int)(std::max<int64_t>(ktiles, 1) * kBK), bn};
    for (int64_t s = 1; s <= max_splits; s++) {
      const int64_t per = (ktiles + s - 1) / s;          // K tiles per split
      const int64_t splits = (ktiles + per - 1) / per;   // splits actually needed
      if (splits != s) continue;
      const int64_t items = tiles * splits;
      const int64_t rounds = (items + cus - 1) / cus;
      const double busy = rounds == 1 ? (double)items / (double)cus : 1.0;
      double t = (double)rounds * ((double)per * ktile * (1.0 + 0.45 * busy) + fixed + (splits > 1 ? 1.0 : 0.0));
      if (splits > 1) t += 4.0 + ((double)splits * 4.0 + 2.0) * (double)M * (double)N / 5.0e6;
      if (s == 1 || t < tbest[c]) {
        tbest[c] = t;
        best[c].splits = (int)splits;
        best[c].ksplit = (int)(per * kBK);
      }
    }
  }
  return ktiles > 0 && tbest[1] < kNarrowGain * tbest[0] ? best[1] : best[0];
}

// The launch shared by both operand layouts (arguments checked by the entry points).
template <bool kMN>
static int launch_gemm(const uint8_t *A, int64_t lda, const float *sa, const uint8_t *B, int64_t ldb, const float *sb,
                       const uint16_t *bias, uint16_t *C, int64_t ldc, int64_t M, int64_t N, int64_t K, void *ws,
                       size_t ws_bytes, hipStream_t st) {
  if (M == 0 || N == 0) return GPIC_OK;
  if (K > 0 && (!A || !B)) return GPIC_EINVAL;
  if (!aligned16(A) || !aligned16(B) || !aligned16(C) || (bias && ((uintptr_t)bias & 7u))) return GPIC_EALIGN;
  const Plan p = K > 0 ? plan_gemm(M, N, K) : Plan{(int)((M + kBM - 1) / kBM), (int)((N + kBN - 1) / kBN), 1, kBK, kBN};
  float *P = nullptr;
  if (p.splits > 1) {
    const size_t need = (size_t)p.splits * M * N * sizeof(float);
    if (!ws || ws_bytes < need) return GPIC_EWORKSPACE;
    if (!aligned16(ws)) return GPIC_EALIGN;
    P = static_cast<float *>(ws);
  }
  // One workgroup per CU at most (160 KiB of LDS each); a persistent grid is a multiple of 8, one per XCD.
  const int work = p.tiles_m * p.tiles_n * p.splits;
  const int slots = num_cus() & ~7;
  const int grid = work <= slots || slots < 8 ? work : slots;
  // the partial-K-tile load path is compiled only into the instance that needs it
  auto *kernel = p.bn == 128 ? (K % kBK ? gemm_tn_kernel<true, kMN, 128> : gemm_tn_kernel<false, kMN, 128>)
                              : (K % kBK ? gemm_tn_kernel<true, kMN, 256> : gemm_tn_kernel<false, kMN, 256>);
  kernel<<<grid, kThreads, 0, st>>>(
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
  status_scope();
  (void)fast_accum;
  if (M < 0 || N < 0 || K < 0 || !sa || !sb || (M > 0 && N > 0 && !C)) return GPIC_EINVAL;
  if (K % 16 != 0 || N % 16 != 0 || lda % 16 != 0 || ldb % 16 != 0 || ldc % 8 != 0) return GPIC_ESHAPE;
  // (the epilogue's C offsets, row within the tile x ldc x 2 bytes, are 32-bit: ldc < 2^22)
  if (lda < K || ldb < K || ldc < N || lda >= (1 << 23) || ldb >= (1 << 23) || ldc >= (1 << 22) || M >= (1 << 30))
    return GPIC_ESHAPE;
  return launch_gemm<false>(A, lda, sa, B, ldb, sb, bias, C, ldc, M, N, K, ws, ws_bytes, (hipStream_t)stream);
}

int gpic_fp8_gemm_mn(const uint8_t *A, int64_t lda, const float *sa, const uint8_t *B, int64_t ldb, const float *sb,
                     const uint16_t *bias, uint16_t *C, int64_t ldc, int64_t M, int64_t N, int64_t K, void *ws,
                     size_t ws_bytes, void *stream) {
  status_scope();
  if (M < 0 || N < 0 || K < 0 || !sa || !sb || (M > 0 && N > 0 && !C)) return GPIC_EINVAL;
  if (M % 16 != 0 || N % 16 != 0 || lda % 16 != 0 || ldb % 16 != 0 || ldc % 8 != 0) return GPIC_ESHAPE;
  // every load offset (K row x row stride) is a 32-bit buffer offset, and so is every C offset (ldc < 2^22)
  if (lda < M || ldb < N || ldc < N || K * lda >= (int64_t(1) << 31) || K * ldb >= (int64_t(1) << 31) ||
      ldc >= (1 << 22) || M >= (1 << 30))
    return GPIC_ESHAPE;
  return launch_gemm<true>(A, lda, sa, B, ldb, sb, bias, C, ldc, M, N, K, ws, ws_bytes, (hipStream_t)stream);
}

}  // extern "C"

/*
 * libgpic_fp8 -- the C ABI of the MI355X (gfx950) FP8 linear path of nano-gpic's JiT-T2I transformer.
 *
 * The reference path is baselines/PixelGen/src/models/layers/fp8_native.py (Python + Triton, with the GEMM in
 * torch._scaled_mm). Each entry point below names the reference interface it replaces. The reference's "FFI" for
 * this path is torch.library: its ops gpic::fp8_tcast / gpic::fp8_swiglu_tcast / gpic::fp8_swiglu_bwd and the
 * aten::_scaled_mm call in _mm. The Python package gpic_fp8 registers ops of the same names and schemas over these
 * functions (ctypes).
 *
 * Conventions
 *   - Every pointer is a device pointer (HBM), except where noted. bf16 tensors are passed as uint16_t bit patterns,
 *     e4m3fn tensors as uint8_t bytes, scales as one fp32 each.
 *   - `stream` is a hipStream_t (void * here so this header needs no HIP headers). Work is enqueued on it; nothing
 *     synchronises with the host, nothing is allocated, and scales stay on the device.
 *   - `ws` is a caller-provided device workspace of at least the size the matching *_workspace_bytes() returns,
 *     16-byte aligned. The cast workspace carries state from call to call and must be zeroed once, when it is created
 *     (by any means; it is never to be cleared again while it is in use): the single-pass casts tag their partial
 *     maxima with a call number kept in the workspace itself (an epoch word that each call's last workgroup advances
 *     on the device), so a stale word from an earlier call never matches a later one. Because the number lives on the
 *     device, a cast captured in a HIP graph takes a new number on every replay. Calls that may run at the same time
 *     (different streams, or graphs replayed concurrently) need different workspaces; calls ordered on one stream may
 *     share one. The GEMM workspace (split-K partials) is scratch of one call.
 *   - Tensor data pointers are 16-byte aligned; leading dimensions are in elements.
 *   - Return value: 0 on success, a negative GPIC_E* code for invalid arguments (nothing was launched), or a positive
 *     hipError_t from the launch.
 */
#ifndef GPIC_FP8_H
#define GPIC_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GPIC_OK 0
#define GPIC_EINVAL (-1)  /* null pointer, negative size */
#define GPIC_EDTYPE (-2)  /* unsupported dtype code */
#define GPIC_ESHAPE (-3)  /* a size or leading dimension breaks the alignment rules (multiples of 16 / 8) */
#define GPIC_EALIGN (-4)  /* a pointer is not 16-byte aligned */
#define GPIC_EWORKSPACE (-5) /* the workspace is smaller than required */

#define GPIC_DTYPE_BF16 0
#define GPIC_DTYPE_F32 1

/* Library version string and a message for a status code (host memory, static). */
const char *gpic_fp8_version(void);
const char *gpic_fp8_status_string(int status);

/* Bytes of workspace the cast entry points need (the partial maxima of the amax pass, the SwiGLU sigmoid table and
 * the single-pass casts' tagged partials). */
size_t gpic_fp8_cast_workspace_bytes(void);

/* Tuning and test knob (process-wide; a call made on another thread at the same time sees the old or the new
 * setting; no counterpart in the reference, whose casts are always two Triton launches). gpic_fp8_tcast and gpic_fp8_tcast_t cast a bf16 (or, flat, fp32) tensor
 * that fits in the chip's registers in one launch (x read once) and larger ones in two (amax pass, then cast pass).
 * enabled = 0 forces the two-pass path; wait_us bounds how long a workgroup of the single pass waits for another's
 * partial maximum before computing it from x itself (< 0: the default, 200 us; 0 makes every missing partial a direct
 * computation, which tests use to exercise that path). The results are the same bytes either way. */
void gpic_fp8_set_single_pass(int enabled, int wait_us);

/*
 * Tensorwise current-amax cast to e4m3fn.
 * Replaces gpic::fp8_tcast (fp8_native.py:114-122: _amax_kernel :33-37, _cast_kernel :40-49, _cast_flat :105-111).
 *   x        n contiguous elements, bf16 (dtype GPIC_DTYPE_BF16) or fp32 (GPIC_DTYPE_F32)
 *   q        n bytes: e4m3(min(max(RN(x * scale), -448), 448)), scale = RN(448 / max(amax, 1e-12))
 *   dequant  1 fp32: RN(max(amax, 1e-12) / 448); amax = max |x| over the non-NaN elements
 * n == 0 writes only dequant (1e-12 / 448).
 */
int gpic_fp8_tcast(const void *x, int dtype, int64_t n, uint8_t *q, float *dequant, void *ws, void *stream);

/*
 * gpic_fp8_tcast without a workspace argument, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation). No counterpart in the reference. It allocates
 * nothing: its workspace is a static 44 KiB device array of the library, one per GPU, held until the process ends,
 * set up on the first call on each device (its address taken, and the array cleared by a kernel on `stream`). The
 * array's size does not depend on n, so every n gpic_fp8_tcast takes is accepted; a build whose cast workspace
 * outgrew the array would return GPIC_EWORKSPACE. The same bytes and scale as gpic_fp8_tcast. Every call on one GPU
 * shares the array and keeps the state the last call left there: calls that overlap on one GPU (several streams, or
 * a captured graph replayed beside other such calls) race; calls ordered on one stream do not.
 */
int gpic_fp8_tcast_noalloc(const void *x, int dtype, int64_t n, uint8_t *q, float *dequant, void *stream);

/*
 * The same cast of x [rows, cols] (row-major, cols % 16 == 0), writing q [rows, cols] (skipped when q is NULL) and
 * the transposed bytes qt [cols, ldt] (ldt % 16 == 0, ldt >= rows; columns rows..ldt-1 are written as zero bytes).
 * Replaces the reference's tcast(w.t().contiguous()) (fp8_native.py:259,262), which has the same amax and therefore
 * the same bytes transposed; qt is also the K-major operand of the FP8 wgrad (an extension of the reference, whose
 * wgrads are bf16, fp8_native.py:202,225,264-265).
 */
int gpic_fp8_tcast_t(const void *x, int dtype, int64_t rows, int64_t cols, uint8_t *q, uint8_t *qt, int64_t ldt,
                     float *dequant, void *ws, void *stream);

/*
 * count transposing casts in one call: tensor i is x[i] [rows[i], cols[i]] -> q[i] (or NULL), qt[i] [cols[i], ldt[i]],
 * dequant[i], each with its own amax: the same bytes and scales as gpic_fp8_tcast_t on each tensor in order. No
 * counterpart in the reference, whose linears cast their weights one at a time inside each forward; this is for a
 * caller that casts a block's weights together before the block runs. bf16 tensors that fit the device together
 * (d12: the four weights, 1024 tiles of 128 x 128) are cast in ONE launch, each tensor over its own workgroups;
 * otherwise (fp32, more than 8 tensors, empty or larger tensors) the call makes the per-tensor calls. Every tensor is
 * checked first, as gpic_fp8_tcast_t checks it; on an error nothing is launched.
 */
int gpic_fp8_tcast_t_group(int count, const void *const *x, int dtype, const int64_t *rows, const int64_t *cols,
                           uint8_t *const *q, uint8_t *const *qt, const int64_t *ldt, float *const *dequant, void *ws,
                           void *stream);

/*
 * The attention output's cast with its head merge folded in: the cast of proj's input, read from the attention's own
 * output. Replaces, at the attention output feeding proj (baselines/PixelGen/src/models/transformer/JiT_T2I.py:183-185:
 * x = attention(q, k, v); x.transpose(1, 2).reshape(B, N, C); self.proj(x)), the head-merging copy plus the FP8
 * linear's tcast of its result (fp8_native.py:114-122, 187) with one producer of proj's e4m3 input (an extension:
 * the reference keeps them apart, fp8_native.py:3-6):
 *   o        [B, H, N, D] bf16, element (b, h, n, d) at o + b sb + h sh + n sn + d (strides in elements, multiples of
 *            8, >= 0; D % 16 == 0; 16-byte aligned) -- e.g. scaled_dot_product_attention's output in either of the
 *            layouts its backends write ([B, H, N, D] or [B, N, H, D] in memory)
 *   q        [B N, H D] e4m3, row b N + n, column h D + d: the bytes gpic_fp8_tcast gives for the contiguous
 *            o.transpose(1, 2).reshape(B N, H D), with the same amax, scale and dequant
 * The source's word indices (16 bytes) and the output's words must stay below 2^31 (else GPIC_ESHAPE). When the
 * strides already describe [B, N, H, D] contiguous, the call is gpic_fp8_tcast of o. Same single-pass / two-pass
 * choice, workspace and empty-tensor rule as gpic_fp8_tcast.
 */
int gpic_fp8_tcast_heads(const uint16_t *o, int64_t B, int64_t H, int64_t N, int64_t D, int64_t sb, int64_t sh,
                         int64_t sn, uint8_t *q, float *dequant, void *ws, void *stream);

/*
 * SwiGLU product cast. Replaces gpic::fp8_swiglu_tcast (fp8_native.py:130-144; _swiglu_tile :53-58,
 * _swiglu_amax_kernel :61-66, _swiglu_cast_kernel :69-78).
 *   z        [M, 2H] bf16, row stride sz (H % 8 == 0, sz % 8 == 0)
 *   q        [M, H] e4m3 of a = bf16(bf16(z1 * sigmoid(z1)) * z2), row stride sq (sq % 8 == 0)
 *   dequant  1 fp32
 * With sq == H and a product of at most 96 MiB (on 256 CUs) one single-pass launch (see gpic_fp8_tcast: the
 * workspace carries its call counter); otherwise an amax pass and a cast pass that recomputes the product.
 */
int gpic_fp8_swiglu_tcast(const uint16_t *z, int64_t M, int64_t H, int64_t sz, uint8_t *q, int64_t sq, float *dequant,
                          void *ws, void *stream);

/*
 * SwiGLU backward with the cast of its output. Replaces gpic::fp8_swiglu_bwd (fp8_native.py:153-166;
 * _swiglu_bwd_kernel :83-98, then _cast_flat).
 *   z [M, 2H] (row stride sz), da [M, H] (row stride sda) bf16 ->
 *   dz [M, 2H] bf16 contiguous, dzq [M, 2H] e4m3 contiguous, dequant 1 fp32
 *   dz may be NULL: dz is not written and dzq is cast from dz recomputed from z and da (the same bytes; less memory
 *      traffic than writing dz and reading it back) -- for a caller whose weight gradient takes dzq, not dz. Then one
 *      single-pass launch (see gpic_fp8_tcast: the workspace carries its call counter) holds up to 80 MiB of dz on
 *      chip (on 256 CUs) and computes the rest twice, up to 16x that (d12's [32768, 4096]: 307 us against 336 for an
 *      amax pass and a recomputing cast pass, flushed caches); beyond, or with single-pass casts disabled, the latter.
 */
int gpic_fp8_swiglu_bwd(const uint16_t *z, const uint16_t *da, int64_t M, int64_t H, int64_t sz, int64_t sda,
                        uint16_t *dz, uint8_t *dzq, float *dequant, void *ws, void *stream);

/*
 * gpic_fp8_swiglu_tcast plus the transposed bytes qt [H, ldt] (H % 16 == 0, ldt % 16 == 0, ldt >= M; columns
 * M..ldt-1 zero): the K-major operand of w3's FP8 wgrad. Same bytes and scale as gpic_fp8_swiglu_tcast.
 *   a  [M, H] bf16, contiguous, or NULL. With qt given, or in the two-pass casts: the SwiGLU product is written there
 *      by the amax pass and the cast reads it instead of recomputing it (the same bytes; faster: the product is
 *      computed once), so `a` holds the whole product afterwards. In the q-only single pass (qt == NULL, sq == H,
 *      below) `a` is scratch: the pass writes only the rows of the product that do not fit on chip (none when the
 *      whole product fits), and the contents of `a` afterwards are unspecified. A caller that needs the bf16 product
 *      itself must pass qt, or disable the single pass (gpic_fp8_set_single_pass).
 *   qt may be NULL (then ldt == 0, and H % 8 == 0 suffices): q only. With sq == H the single pass: one launch that
 *      holds up to 96 MiB of the product on chip (on 256 CUs) and, given `a`, streams the rest through a -- up to 8x
 *      that (d12's [32768, 8192]: 190 us against 246 for the amax pass writing a and a flat cast of it, flushed
 *      caches); the same bytes as gpic_fp8_swiglu_tcast. With single-pass casts disabled (gpic_fp8_set_single_pass)
 *      or past 8x: the two-pass casts, through `a` when given.
 * No counterpart in the reference (its w3 wgrad is bf16, fp8_native.py:225,265); the FP8-wgrad extension.
 */
int gpic_fp8_swiglu_tcast_t(const uint16_t *z, int64_t M, int64_t H, int64_t sz, uint16_t *a, uint8_t *q, int64_t sq,
                            uint8_t *qt, int64_t ldt, float *dequant, void *ws, void *stream);

/*
 * gpic_fp8_swiglu_bwd plus the transposed bytes dzqt [2H, ldt] (ldt % 16 == 0, ldt >= M; columns M..ldt-1 zero):
 * the K-major operand of w12's FP8 wgrad. Same dz, dzq and scale as gpic_fp8_swiglu_bwd.
 *   dz may be NULL (then ldt > 0 and dzqt are required): dz is not written; dzq and dzqt, the same bytes, are cast from
 *      dz recomputed from z and da tile by tile (less memory traffic than writing dz and reading it back).
 * No counterpart in the reference (its w12 wgrad is bf16, fp8_native.py:264); the FP8-wgrad extension.
 */
int gpic_fp8_swiglu_bwd_t(const uint16_t *z, const uint16_t *da, int64_t M, int64_t H, int64_t sz, int64_t sda,
                          uint16_t *dz, uint8_t *dzq, uint8_t *dzqt, int64_t ldt, float *dequant, void *ws,
                          void *stream);

/*
 * The norm sites' producer with the cast of its output folded in. Replaces gpic::res_mod_rmsnorm_fwd
 * (baselines/PixelGen/src/models/layers/fused_norm.py:150-175, kernel :64-91) followed by the FP8 linear's tcast of
 * its output h (fp8_native.py:114-122), as one producer (the reference keeps them apart, fp8_native.py:3-6):
 *   site 2 (a != NULL): x_new = bf16(fma(gate, a, x)) -> xn;   site 1 (a == NULL): x_new = x
 *   rstd = 1 / sqrt(sum(x_new^2) / C + eps) -> rstd [rows];  n = bf16(w * (x_new * rstd))
 *   h = bf16(fma(n, 1 + scale, shift)) -> h (when h != NULL), and its tensorwise e4m3 bytes -> hq, dequant (the
 *   tcast rule: amax over the non-NaN values, IEEE scales, saturating round-to-nearest-even)
 *   x, a, xn, h: [rows, C] bf16 (C % 4 == 0, 16-byte aligned); hq [rows, C] e4m3; w [C] fp32 (16-byte aligned)
 *   gate, shift, scale: [B, C] bf16 rows with strides sg, ssh, ssc (multiples of 4, >= C; 8-byte aligned); row r of
 *   x uses row r / ntok of them (rows % ntok == 0)
 * dequant == NULL (then h != NULL, hq unused): the norm alone, as the reference's op (one pass writing h).
 * fma is one fused multiply-add (as Triton compiles the reference's expressions on the GPU), every other fp32
 * operation is rounded on its own, and the sum of squares is taken in a fixed order (norm.hip states it); the
 * reference's order and rsqrt are Triton's and libdevice's. Uses the cast workspace (its single-pass partials); a
 * call with both h and dequant runs the two-pass kernels (the single pass does not write h).
 */
int gpic_fp8_res_mod_rmsnorm(const uint16_t *x, const uint16_t *a, const uint16_t *gate, int64_t sg, const float *w,
                             const uint16_t *shift, int64_t ssh, const uint16_t *scale, int64_t ssc, int64_t rows,
                             int64_t ntok, int64_t C, float eps, uint16_t *xn, uint16_t *h, float *rstd, uint8_t *hq,
                             float *dequant, void *ws, void *stream);

/*
 * The norm sites' backward. Replaces gpic::res_mod_rmsnorm_bwd (fused_norm.py:249-275, kernel :94-147) with its
 * column sums done on the device in a fixed order (the reference adds its partials with torch.sum):
 *   t = xs * rstd, n = bf16(w t), dn = dh (1 + scale), dt = dn w, mean = sum_row(dt t) / C
 *   dx = bf16(rstd (dt - t mean) + dxn);   site 2 (a != NULL): da = bf16(dx_fp32 gate)
 *   d_shift[b] = sum dh, d_scale[b] = sum dh n, d_gate[b] = sum dx_fp32 a  (over the rows of batch b)  [B, C] fp32
 *   d_w = sum dn t (over all rows)  [C] fp32
 *   dh, dxn, xs (x_new at site 2, x at site 1), a, dx, da: [rows, C] bf16 (16-byte aligned); dxn may be NULL at site 2
 *   and must be NULL at site 1 (as gate, d_gate); gate, scale: [B, C] bf16 rows (strides sg, ssc); w [C] fp32;
 *   rstd [rows] fp32 (the forward's); C % 4 == 0, C <= 2048, rows % ntok == 0.
 *   ws: gpic_fp8_res_mod_rmsnorm_bwd_workspace_bytes(rows, ntok, C) bytes (the partial column sums).
 * Deterministic: every sum is taken in a fixed order.
 */
size_t gpic_fp8_res_mod_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t ntok, int64_t C);
int gpic_fp8_res_mod_rmsnorm_bwd(const uint16_t *dh, const uint16_t *dxn, const uint16_t *xs, const uint16_t *a,
                                 const uint16_t *gate, int64_t sg, const float *w, const uint16_t *scale, int64_t ssc,
                                 const float *rstd, int64_t rows, int64_t ntok, int64_t C, uint16_t *dx, uint16_t *da,
                                 float *dshift, float *dscale, float *dgate, float *dw, void *ws, size_t ws_bytes,
                                 void *stream);

/* Bytes of workspace gpic_fp8_gemm needs for this problem (0 when it runs without split-K). */
size_t gpic_fp8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * Scaled FP8 GEMM, "TN": both operands K-contiguous.
 * Replaces _mm (fp8_native.py:175-178) = torch._scaled_mm(A, B.t(), scale_a, scale_b, out_dtype=bf16), and folds the
 * bias add of _Fp8Linear.forward (fp8_native.py:189-190) into the epilogue with the same two roundings:
 *   C[m, n] = bf16(sa * sb * sum_k A[m, k] * B[n, k]);  if bias: C[m, n] = bf16(C[m, n] + bias[n])
 *   A [M, K] e4m3, row stride lda;  B [N, K] e4m3, row stride ldb;  C [M, N] bf16, row stride ldc
 *   sa, sb   device fp32 scalars (the dequantization scales);  bias: [N] bf16 or NULL
 *   K % 16 == 0, N % 16 == 0, lda / ldb % 16 == 0, ldc % 8 == 0; lda, ldb < 2^23, ldc < 2^22; any M.
 *   fast_accum is accepted for interface parity with use_fast_accum: MFMA accumulates in fp32 either way.
 * The fp32 accumulation is the MFMA's; the result matches the scaled matmul of the same operands within the
 * relative Frobenius error the path promises (1e-2), and is deterministic (split-K partials are summed in a fixed
 * order).
 */
int gpic_fp8_gemm(const uint8_t *A, int64_t lda, const float *sa, const uint8_t *B, int64_t ldb, const float *sb,
                  const uint16_t *bias, uint16_t *C, int64_t ldc, int64_t M, int64_t N, int64_t K, int fast_accum,
                  void *ws, size_t ws_bytes, void *stream);

/*
 * Scaled FP8 GEMM with both operands "MN-major" (K is their row index): the weight gradient straight from the
 * untransposed e4m3 bytes of the layer's output gradient and input.
 *   C[m, n] = bf16(sa * sb * sum_k A[k, m] * B[k, n]);  if bias: C[m, n] = bf16(C[m, n] + bias[n])
 *   A [K, M] e4m3, row stride lda;  B [K, N] e4m3, row stride ldb;  C [M, N] bf16, row stride ldc
 *   M % 16 == 0, N % 16 == 0, lda / ldb % 16 == 0, ldc % 8 == 0, K * lda and K * ldb < 2^31, ldc < 2^22; any K.
 * Bit-identical to gpic_fp8_gemm on the transposed operands (A^T [M, K], B^T [N, K]): the same products summed in
 * the same order, with the same workspace (gpic_fp8_gemm_workspace_bytes(M, N, K)).
 * No counterpart in the reference (its wgrads are bf16, fp8_native.py:202, 264-265); the FP8-wgrad extension.
 */
int gpic_fp8_gemm_mn(const uint8_t *A, int64_t lda, const float *sa, const uint8_t *B, int64_t ldb, const float *sb,
                     const uint16_t *bias, uint16_t *C, int64_t ldc, int64_t M, int64_t N, int64_t K, void *ws,
                     size_t ws_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GPIC_FP8_H */

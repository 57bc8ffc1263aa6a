/*
 * CPU restatement of nano-gpic's native FP8 linear path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this code, and only as the checker
 * (or as the timed CPU baseline). The product (nano-gpic_amd/) never links, loads or calls it.
 *
 * Every function restates one piece of baselines/PixelGen/src/models/layers/fp8_native.py (cited per function)
 * as scalar C with the same rounding steps, so that it can be pinned against torch's own CPU routines and
 * against closed forms (tests/test_oracle.py) and then used to check the HIP kernels bit for bit.
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off: every multiply and add is rounded on its own unless the code
 * calls fmaf explicitly, which is what the device code does too). The element loops are split over threads with
 * OpenMP (-fopenmp; OMP_NUM_THREADS sets how many): each element's arithmetic is the same scalar code whatever thread
 * runs it, and the maxima are reduced with max, which does not depend on order, so the results do not depend on the
 * thread count.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define FMAX 448.0f   /* fp8_native.py:25, the largest finite e4m3fn value */
#define TINY 1e-12f   /* fp8_native.py:26, the amax floor */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* bf16 bits -> fp32 (exact). */
float gpo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* fp32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN of the same sign (torch's rule). */
uint16_t gpo_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* fp32 -> OCP e4m3fn byte (bias 7, no infinities, 0x7f/0xff NaN, subnormals m * 2^-9), round to nearest even.
 * Values whose rounding would exceed 448 become NaN, as torch's .to(float8_e4m3fn) does; the path never feeds
 * such a value because fp8_native.py:47 clamps to +-448 first. Written from the OCP 8-bit FP spec v1.0. */
uint8_t gpo_e4m3(float f) {
    uint32_t u = f2u(f);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint8_t)(sign | 0x7f);          /* NaN */
    if (a < 0x3c800000u) {                                          /* |f| < 2^-6: subnormal range, unit 2^-9 */
        float m = rintf(u2f(a) * 512.0f);                           /* exact scaling, then RNE to an integer */
        return (uint8_t)(sign | (uint8_t)m);                        /* m == 8 is the encoding of 2^-6 itself */
    }
    uint32_t r = a - (120u << 23);                                  /* rebias the exponent 127 -> 7 */
    r = (r + 0x7ffffu + ((r >> 20) & 1u)) >> 20;                    /* keep 3 mantissa bits, RNE */
    if (r > 0x7eu) return (uint8_t)(sign | 0x7f);                   /* beyond 448 after rounding: NaN */
    return (uint8_t)(sign | r);
}

void gpo_e4m3_n(const float *x, int64_t n, uint8_t *q) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) q[i] = gpo_e4m3(x[i]);
}

/* e4m3fn byte -> fp32 (exact). */
float gpo_e4m3_to_f32(uint8_t b) {
    int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
    float v;
    if (e == 15 && m == 7) v = NAN;
    else if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf((float)(8 + m), e - 10);
    return s ? -v : v;
}

/* _amax_kernel, fp8_native.py:33-37: max |fp32(x)| over the tensor, gathered as the maximum of the non-negative
 * float bit patterns (the kernel's atomic_max on the int32 bits); returns those bits. tl.max reduces with maxnum,
 * so NaN elements take no part (an all-NaN tensor has amax 0). */
uint32_t gpo_amax_bf16(const uint16_t *x, int64_t n) {
    uint32_t m = 0;
#pragma omp parallel for schedule(static) reduction(max : m)
    for (int64_t i = 0; i < n; i++) {
        uint32_t a = ((uint32_t)(x[i] & 0x7fffu)) << 16;
        if (a > 0x7f800000u) continue;
        if (a > m) m = a;
    }
    return m;
}

uint32_t gpo_amax_f32(const float *x, int64_t n) {
    uint32_t m = 0;
#pragma omp parallel for schedule(static) reduction(max : m)
    for (int64_t i = 0; i < n; i++) {
        uint32_t a = f2u(x[i]) & 0x7fffffffu;
        if (a > 0x7f800000u) continue;
        if (a > m) m = a;
    }
    return m;
}

/* _cast_kernel, fp8_native.py:43-44,49: a = max(amax, 1e-12); scale = RN(448 / a) (IEEE division, div_rn);
 * dequant = RN(a / 448). */
void gpo_scales(uint32_t amax_bits, float *scale, float *dequant) {
    float a = u2f(amax_bits);
    if (a < TINY) a = TINY;   /* tl.maximum(amax, 1e-12); the amax is never NaN */
    *scale = FMAX / a;
    *dequant = a / FMAX;
}

/* _cast_kernel, fp8_native.py:46-47: q = e4m3(min(max(RN(x * scale), -448), 448)). tl.maximum / tl.minimum are
 * maxNum / minNum (C's fmaxf / fminf): a NaN product saturates to -448. */
static inline uint8_t cast1(float x, float scale) {
    float y = x * scale;
    y = fmaxf(y, -FMAX);
    y = fminf(y, FMAX);
    return gpo_e4m3(y);
}

void gpo_cast_bf16(const uint16_t *x, int64_t n, float scale, uint8_t *q) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) q[i] = cast1(gpo_bf16_to_f32(x[i]), scale);
}

void gpo_cast_f32(const float *x, int64_t n, float scale, uint8_t *q) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) q[i] = cast1(x[i], scale);
}

/* tcast, fp8_native.py:114-122: amax pass then cast pass; an empty tensor keeps amax 0 -> dequant 1e-12/448. */
void gpo_tcast_bf16(const uint16_t *x, int64_t n, uint8_t *q, float *dequant, uint32_t *amax_out) {
    float scale;
    uint32_t am = gpo_amax_bf16(x, n);
    gpo_scales(am, &scale, dequant);
    gpo_cast_bf16(x, n, scale, q);
    if (amax_out) *amax_out = am;
}

void gpo_tcast_f32(const float *x, int64_t n, uint8_t *q, float *dequant, uint32_t *amax_out) {
    float scale;
    uint32_t am = gpo_amax_f32(x, n);
    gpo_scales(am, &scale, dequant);
    gpo_cast_f32(x, n, scale, q);
    if (amax_out) *amax_out = am;
}

/* The sigmoid of the SwiGLU kernels (fp8_native.py:57,91 use Triton's tl.sigmoid, whose rounding is the H100's and
 * is not reproducible here). This build fixes one definition, shared bit for bit with the device code:
 *   e^t by Cody-Waite reduction t = n ln2 + r (n = rint(t log2 e), r by two fused multiply-adds with a split ln2),
 *   e^r by its degree-7 Taylor polynomial in Horner form with fused multiply-adds, then ldexp(p, n);
 *   sigmoid(x) = 1 / (1 + e^-x) with IEEE division.
 * It is pinned against torch.sigmoid within 1 bf16 ulp of the SwiGLU values that use it. */
float gpo_exp(float t) {
    if (t != t) return t;
    if (t > 88.8f) return INFINITY;
    if (t < -104.0f) return 0.0f;
    float n = rintf(t * 1.44269502f);
    float r = fmaf(-n, 0.693145751953125f, t);
    r = fmaf(-n, 1.42860682e-06f, r);
    float p = 1.98412698e-04f;            /* 1/7! */
    p = fmaf(p, r, 1.38888889e-03f);      /* 1/6! */
    p = fmaf(p, r, 8.33333377e-03f);      /* 1/5! */
    p = fmaf(p, r, 4.16666679e-02f);      /* 1/4! */
    p = fmaf(p, r, 1.66666672e-01f);      /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

float gpo_sigmoid(float x) { return 1.0f / (1.0f + gpo_exp(-x)); }

/* _swiglu_tile, fp8_native.py:55-58: sl = bf16(z1 * sigmoid(z1)); a = bf16(sl * z2); returns a's bf16 bits. */
uint16_t gpo_swiglu1(uint16_t z1h, uint16_t z2h) {
    float z1 = gpo_bf16_to_f32(z1h), z2 = gpo_bf16_to_f32(z2h);
    float sl = gpo_bf16_to_f32(gpo_f32_to_bf16(z1 * gpo_sigmoid(z1)));
    return gpo_f32_to_bf16(sl * z2);
}

/* swiglu_tcast, fp8_native.py:61-78,130-144: z [M, 2H] (row stride sz) -> aq [M, H] (row stride sq), dequant. */
void gpo_swiglu_tcast(const uint16_t *z, int64_t M, int64_t H, int64_t sz, uint8_t *q, int64_t sq, float *dequant,
                      uint32_t *amax_out) {
    uint32_t m = 0;
#pragma omp parallel for schedule(static) reduction(max : m)
    for (int64_t r = 0; r < M; r++)
        for (int64_t k = 0; k < H; k++) {
            uint32_t a = ((uint32_t)(gpo_swiglu1(z[r * sz + k], z[r * sz + H + k]) & 0x7fffu)) << 16;
            if (a > 0x7f800000u) continue;
            if (a > m) m = a;
        }
    float scale;
    gpo_scales(m, &scale, dequant);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < M; r++)
        for (int64_t k = 0; k < H; k++)
            q[r * sq + k] = cast1(gpo_bf16_to_f32(gpo_swiglu1(z[r * sz + k], z[r * sz + H + k])), scale);
    if (amax_out) *amax_out = m;
}

/* _swiglu_bwd_kernel, fp8_native.py:88-94 (the same expression as the eager backward, fp8_native.py:226-231):
 *   sg = sigmoid(z1); sl = bf16(z1 * sg)
 *   d1 = bf16((da * z2) * (sg * (1 + z1 * (1 - sg))))     every operation rounded on its own, left to right
 *   d2 = bf16(da * sl)
 * then swiglu_bwd, fp8_native.py:153-166: amax over dz and the flat cast of dz. */
void gpo_swiglu_bwd1(uint16_t z1h, uint16_t z2h, uint16_t dah, uint16_t *d1, uint16_t *d2) {
    float z1 = gpo_bf16_to_f32(z1h), z2 = gpo_bf16_to_f32(z2h), da = gpo_bf16_to_f32(dah);
    float sg = gpo_sigmoid(z1);
    float sl = gpo_bf16_to_f32(gpo_f32_to_bf16(z1 * sg));
    float t1 = 1.0f - sg;
    float t2 = z1 * t1;
    float t3 = 1.0f + t2;
    float g = sg * t3;
    float p = da * z2;
    *d1 = gpo_f32_to_bf16(p * g);
    *d2 = gpo_f32_to_bf16(da * sl);
}

void gpo_swiglu_bwd(const uint16_t *z, const uint16_t *da, int64_t M, int64_t H, int64_t sz, int64_t sda,
                    uint16_t *dz, int64_t sdz, uint8_t *dzq, float *dequant, uint32_t *amax_out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < M; r++)
        for (int64_t k = 0; k < H; k++)
            gpo_swiglu_bwd1(z[r * sz + k], z[r * sz + H + k], da[r * sda + k], &dz[r * sdz + k], &dz[r * sdz + H + k]);
    /* _cast_flat over the contiguous dz [M, 2H] */
    uint32_t m = 0;
#pragma omp parallel for schedule(static) reduction(max : m)
    for (int64_t r = 0; r < M; r++)
        for (int64_t k = 0; k < 2 * H; k++) {
            uint32_t a = ((uint32_t)(dz[r * sdz + k] & 0x7fffu)) << 16;
            if (a > 0x7f800000u) continue;
            if (a > m) m = a;
        }
    float scale;
    gpo_scales(m, &scale, dequant);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < M; r++)
        for (int64_t k = 0; k < 2 * H; k++)
            dzq[r * 2 * H + k] = cast1(gpo_bf16_to_f32(dz[r * sdz + k]), scale);
    if (amax_out) *amax_out = m;
}

/* The norm sites' producer (fused_norm.py:64-91, res_mod_rmsnorm forward) as this build defines its arithmetic
 * (nano-gpic_amd/csrc/norm.hip), row by row in fp32; fmaf is one fused multiply-add (one rounding, as Triton
 * compiles the reference's a * b + c on the GPU), every other operation rounds on its own:
 *   xb = bf16(fmaf(gate, a, x)) (a != NULL; else xb = x);  rstd = 1 / sqrt(ss / C + eps)  (IEEE);
 *   n = bf16(w * (xb * rstd));  h = bf16(fmaf(n, 1 + scale, shift))
 * with ss accumulated in the device's order: lane l (0..63) takes ss = fmaf(xb, xb, ss) over elements
 * 4 (l + 64 j) + e < C in the order j, e; then the 64 lane sums are combined by the butterfly v_l += v_{l ^ o},
 * o = 32, 16, ..., 1 (C % 4 == 0: a lane's group of 4 is wholly inside the row or wholly past its end).
 * The reference sums in Triton's order and takes libdevice's rsqrt; its own eager formula (fused_norm.py:305-313)
 * rounds gate * a to bf16 before the add. gate, shift, scale are [B, C] rows (strides sg, ssh, ssc), row r in batch
 * r / ntok. Writes xn (a != NULL), h and rstd. */
static inline float norm_xb(const uint16_t *x, const uint16_t *a, const uint16_t *gate, int64_t i, int64_t gi) {
    float v = gpo_bf16_to_f32(x[i]);
    if (a) v = gpo_bf16_to_f32(gpo_f32_to_bf16(fmaf(gpo_bf16_to_f32(gate[gi]), gpo_bf16_to_f32(a[i]), v)));
    return v;
}

void gpo_mod_rmsnorm(const uint16_t *x, const uint16_t *a, const uint16_t *gate, int64_t sg, const float *w,
                     const uint16_t *shift, int64_t ssh, const uint16_t *scale, int64_t ssc, int64_t rows, int64_t ntok,
                     int64_t C, float eps, uint16_t *xn, uint16_t *h, float *rstd) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const int64_t b = r / ntok, J = (C + 255) / 256;
        float part[64], nxt[64];
        for (int l = 0; l < 64; l++) {
            float s = 0.0f;
            for (int64_t j = 0; j < J; j++)
                for (int e = 0; e < 4; e++) {
                    const int64_t c = 4 * (l + 64 * j) + e;
                    if (c >= C) break;
                    const float v = norm_xb(x, a, gate, r * C + c, b * sg + c);
                    s = fmaf(v, v, s);
                }
            part[l] = s;
        }
        for (int o = 32; o > 0; o >>= 1) {
            for (int l = 0; l < 64; l++) nxt[l] = part[l] + part[l ^ o];
            memcpy(part, nxt, sizeof part);
        }
        const float rs = 1.0f / sqrtf(part[0] / (float)C + eps);
        rstd[r] = rs;
        for (int64_t c = 0; c < C; c++) {
            const float v = norm_xb(x, a, gate, r * C + c, b * sg + c);
            if (a) xn[r * C + c] = gpo_f32_to_bf16(v);
            const float n = gpo_bf16_to_f32(gpo_f32_to_bf16(w[c] * (v * rs)));
            const float sc = gpo_bf16_to_f32(scale[b * ssc + c]), sh = gpo_bf16_to_f32(shift[b * ssh + c]);
            h[r * C + c] = gpo_f32_to_bf16(fmaf(n, 1.0f + sc, sh));
        }
    }
}

/*
 * psq_oracle.c -- CPU oracle for the quantized linear path (TEST INFRASTRUCTURE ONLY).
 *
 * It checks the product and is never part of it: only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it.  The HIP library must never call into it.
 *
 * It restates, in plain C with OpenMP, the arithmetic of PowerShard's quantized linear
 * path (powershard/quant_linear.py QuantLinear.forward, powershard/operations.py ConvRot
 * helpers) plus the conventions the reference leaves to comfy-kitchen (activation
 * quantization, int32 GEMM epilogue, fp8 per-token scaling, uint4 group layout).
 *
 * Conventions fixed here (the GPU kernels must reproduce them bit for bit where stated):
 *  - ConvRot "regular" Hadamard of size g = 4^k: H = H4^{(x)k} / sqrt(g),
 *    H4[a][b] = -1 iff a + b == 3 (powershard/operations.py:72-81).
 *    Fast transform T (unnormalized, so x H = 2^-k T(x)): one radix-4 stage per base-4
 *    digit, digit 0 (least significant) first.  Within a stage, S = (x0 + x1) + (x2 + x3)
 *    and y_j = S - 2*x_{3-j} rounded once (fmaf(-2, x_{3-j}, S); 2x is exact, so this is the
 *    rounding of the two-step form wherever 2x does not overflow), all in fp32.  The 2^-k
 *    normalization is folded into the
 *    scales below (multiplying by a power of two is exact).
 *  - int8 activation quantization per row (token), u = T(x) (or x when not rotated):
 *    a = max|u|; if a == 0: s = 1, q = 0; else r = 127 / a (fp32 IEEE division, once per
 *    row), s = (a / 127) * 2^-k, q = clamp(rint(u * r), -127, 127), ties to even.
 *    With a static input scale s_in: s = s_in, r = (1 / s_in) * 2^-k.
 *    NaN: a row holding a NaN has a = NaN (torch's amax propagates NaN), hence s = r = NaN, so
 *    its dequantized output is NaN wherever the scale reaches it; a NaN product clamps to the
 *    lower bound, clamp(v) = fmin(fmax(v, -LIM), LIM) with C's fmax/fmin (the non-NaN operand).
 *  - fp8 e4m3fn (OCP) activation quantization per row: the same with 448 in place of 127,
 *    v = clamp(u * r, -448, 448), q = e4m3_rne(v).
 *  - int8 GEMM: acc[m][n] = sum_k a[m][k] * w[n][k] in int32 (exact, order free).
 *  - fp8 GEMM: e4m3fn activation codes times e4m3fn or e5m2 weight codes, decoded exactly
 *    and summed in double, then rounded to fp32 for the epilogue.
 *  - Epilogue (int8 and fp8): y = round_out(fmaf((float)acc, a_s[m] * w_s[n], bias[n])),
 *    bias = 0 when absent, round_out = RNE to bf16 / fp16, or identity for fp32.
 *  - uint4 asymmetric group weights (two per byte, low nibble = even k, group g along K,
 *    fp16 scale s and zero z per (row, group)):  w = (float(q) - float(z)) * float(s),
 *    then rounded to the compute dtype (bf16) before the matmul, as the reference's
 *    dequantize branch does (powershard/quant_linear.py:219-220).
 *
 * Build: see oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off; never -ffast-math).
 */
#include <stdint.h>
#include <string.h>
#include <math.h>
#include <stdlib.h>

#define EXPORT __attribute__((visibility("default")))

enum { PSQ_BF16 = 0, PSQ_F16 = 1, PSQ_F32 = 2 };

/* ------------------------------------------------------------------ scalar formats */

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static inline float bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

static inline uint16_t f32_to_bf16(float f)
{
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline float f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1f) return bits_f32(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return bits_f32(sign);
        /* subnormal: m * 2^-24, exact in fp32 */
        float v = (float)m * 0x1p-24f;
        return sign ? -v : v;
    }
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

static inline uint16_t f32_to_f16(float f)
{
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;            /* NaN */
    if (a >= 0x477ff000u) return sign | 0x7c00u;           /* rounds to >= 65520 -> inf */
    if (a < 0x38800000u) {                                 /* below 2^-14: subnormal half */
        /* value = a * 2^24 in units of the half subnormal step; RNE via rint on exact float */
        float v = bits_f32(a) * 0x1p24f;                   /* exact scaling by power of 2 */
        uint32_t q = (uint32_t)rintf(v);                   /* 0..1024 */
        return sign | (uint16_t)q;                         /* q == 1024 is min normal 0x0400 */
    }
    uint32_t e = (a >> 23) - 112u, m = a & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return sign | (uint16_t)h;
}

static inline float load_act(const void *p, int64_t i, int dtype)
{
    if (dtype == PSQ_BF16) return bf16_to_f32(((const uint16_t *)p)[i]);
    if (dtype == PSQ_F16) return f16_to_f32(((const uint16_t *)p)[i]);
    return ((const float *)p)[i];
}

static inline void store_out(void *p, int64_t i, int dtype, float v)
{
    if (dtype == PSQ_BF16) ((uint16_t *)p)[i] = f32_to_bf16(v);
    else if (dtype == PSQ_F16) ((uint16_t *)p)[i] = f32_to_f16(v);
    else ((float *)p)[i] = v;
}

/* OCP FP8 E4M3FN: bias 7, no infinities, NaN = S.1111.111, max 448. */
static inline float e4m3_to_f32(uint8_t c)
{
    uint32_t s = c >> 7, e = (c >> 3) & 0xfu, m = c & 7u;
    float v;
    if (e == 0xf && m == 7) return NAN;
    if (e == 0) v = (float)m * 0x1p-9f;
    else v = ldexpf(1.0f + (float)m * 0.125f, (int)e - 7);
    return s ? -v : v;
}

/* OCP FP8 E5M2 (bf8): bias 15, 2 mantissa bits, IEEE-style infinities (S.11111.00) and NaNs
 * (S.11111.mm, mm != 0); subnormals m * 2^-16.  From the format's definition. */
static inline float e5m2_to_f32(uint8_t c)
{
    uint32_t s = c >> 7, e = (c >> 2) & 0x1fu, m = c & 3u;
    float v;
    if (e == 0x1f) v = m ? NAN : INFINITY;
    else if (e == 0) v = (float)m * 0x1p-16f;
    else v = ldexpf(1.0f + (float)m * 0.25f, (int)e - 15);
    return s ? -v : v;
}

/* round-to-nearest-even, saturating to +-448; NaN -> 0x7f. */
static inline uint8_t f32_to_e4m3(float x)
{
    if (isnan(x)) return 0x7f;
    uint8_t sign = signbit(x) ? 0x80 : 0;
    float a = fabsf(x);
    if (a >= 448.0f) return sign | 0x7e;
    if (a < 0x1p-6f) {                        /* subnormal range: step 2^-9 */
        float q = rintf(a * 512.0f);           /* exact scale, 0..8; 8 == min normal */
        return sign | (uint8_t)q;
    }
    int e;
    float m = frexpf(a, &e);                   /* a = m * 2^e, m in [0.5, 1) */
    /* a = (2m) * 2^(e-1); mantissa steps of 1/8 on [1, 2) */
    float f = rintf((2.0f * m - 1.0f) * 8.0f); /* exact operations; 0..8 */
    int E = e - 1 + 7;
    int q = (int)f;
    if (q == 8) { q = 0; E += 1; }
    if (E > 15 || (E == 15 && q > 6)) return sign | 0x7e;
    return sign | (uint8_t)((E << 3) | q);
}

EXPORT float psq_or_bf16_round(float x) { return bf16_to_f32(f32_to_bf16(x)); }
EXPORT uint16_t psq_or_f32_to_bf16(float x) { return f32_to_bf16(x); }
EXPORT uint16_t psq_or_f32_to_f16(float x) { return f32_to_f16(x); }
EXPORT float psq_or_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
EXPORT uint8_t psq_or_f32_to_e4m3(float x) { return f32_to_e4m3(x); }
EXPORT float psq_or_e4m3_to_f32(uint8_t c) { return e4m3_to_f32(c); }
EXPORT float psq_or_e5m2_to_f32(uint8_t c) { return e5m2_to_f32(c); }

/* --------------------------------------------------------------- regular Hadamard */

static int log4_of(int g)
{
    if (g < 4 || (g & (g - 1))) return -1;
    int b = 0;
    while ((1 << b) < g) b++;
    return (b % 2) ? -1 : b / 2;
}

/* Closed form: H[i][j] = g^-1/2 * (-1)^{#digits d with i_d + j_d == 3}. */
EXPORT int psq_or_regular_hadamard(int g, float *h)
{
    int k = log4_of(g);
    if (k < 0) return -1;
    float inv = ldexpf(1.0f, -k);
    for (int i = 0; i < g; i++)
        for (int j = 0; j < g; j++) {
            int neg = 0;
            for (int d = 0, a = i, b = j; d < k; d++, a >>= 2, b >>= 2)
                neg ^= ((a & 3) + (b & 3)) == 3;
            h[(int64_t)i * g + j] = neg ? -inv : inv;
        }
    return 0;
}

/* In-place unnormalized fast transform T of one group of g = 4^k fp32 values (x H = 2^-k T(x)),
 * fixed stage order. */
static void fwht4_group(float *v, int g, int k)
{
    for (int d = 0, stride = 1; d < k; d++, stride *= 4) {
        for (int base = 0; base < g; base++) {
            if ((base / stride) % 4) continue;    /* digit d of base is 0 */
            float x0 = v[base], x1 = v[base + stride];
            float x2 = v[base + 2 * stride], x3 = v[base + 3 * stride];
            float s01 = x0 + x1;
            float s23 = x2 + x3;
            float s = s01 + s23;
            v[base]              = fmaf(-2.0f, x3, s);
            v[base + stride]     = fmaf(-2.0f, x2, s);
            v[base + 2 * stride] = fmaf(-2.0f, x1, s);
            v[base + 3 * stride] = fmaf(-2.0f, x0, s);
        }
    }
}

/* Rotate rows of x (dtype) in groups of g along K into fp32 out [M, K]. g == 0: no rotation. */
EXPORT int psq_or_rotate_rows(const void *x, int in_dtype, int64_t M, int64_t K, int64_t ldx,
                              int g, float *out)
{
    int k = g ? log4_of(g) : 0;
    if (g && (k < 0 || K % g)) return -1;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; m++) {
        float *row = out + m * K;
        for (int64_t c = 0; c < K; c++) row[c] = load_act(x, m * ldx + c, in_dtype);
        if (g) {
            float post = ldexpf(1.0f, -k);
            for (int64_t c = 0; c < K; c += g) fwht4_group(row + c, g, k);
            for (int64_t c = 0; c < K; c++) row[c] = row[c] * post;
        }
    }
    return 0;
}

/* Row scale of the activation quantizers: r multiplies the (unnormalized) transform output,
 * s dequantizes the codes.  lim = 127 (int8) or 448 (e4m3); k = log4 of the rotation group. */
static void row_scale(const float *row, int64_t K, float lim, int k, const float *static_scale, float *r,
                      float *s)
{
    const float post = ldexpf(1.0f, -k);
    if (static_scale) {
        *s = static_scale[0];
        *r = (1.0f / *s) * post;
        return;
    }
    float amax = 0.0f;
    for (int64_t c = 0; c < K; c++) {
        const float a = fabsf(row[c]);
        if (isnan(a)) {
            amax = a;
            break;
        }
        amax = a > amax ? a : amax;
    }
    if (amax == 0.0f) {
        *s = 1.0f;
        *r = 1.0f;
    } else {
        *r = lim / amax;
        *s = (amax / lim) * post;
    }
}

/* fmin(fmax(v, -lim), lim): C's fmax/fmin return the non-NaN operand, so NaN -> -lim. */
static inline float clamp_lim(float v, float lim) { return fminf(fmaxf(v, -lim), lim); }

/* Per-row int8 quantization of (optionally rotated) activations.
 * q [M, ldq] int8, scale [M] fp32.  static_scale: NULL for dynamic per-row absmax. */
EXPORT int psq_or_quantize_rows_i8(const void *x, int in_dtype, int64_t M, int64_t K, int64_t ldx,
                                   int g, const float *static_scale, int8_t *q, int64_t ldq,
                                   float *scale)
{
    int k = g ? log4_of(g) : 0;
    if (g && (k < 0 || K % g)) return -1;
    int err = 0;
#pragma omp parallel
    {
        float *row = (float *)malloc(sizeof(float) * (size_t)(K ? K : 1));
        if (!row) {
#pragma omp atomic write
            err = -2;
        }
#pragma omp for schedule(static)
        for (int64_t m = 0; m < M; m++) {
            if (!row) continue;
            for (int64_t c = 0; c < K; c++) row[c] = load_act(x, m * ldx + c, in_dtype);
            if (g)
                for (int64_t c = 0; c < K; c += g) fwht4_group(row + c, g, k);
            float s, r;
            row_scale(row, K, 127.0f, k, static_scale, &r, &s);
            for (int64_t c = 0; c < K; c++)
                q[m * ldq + c] = (int8_t)clamp_lim(rintf(row[c] * r), 127.0f);
            scale[m] = s;
        }
        free(row);
    }
    return err;
}

/* Per-row fp8 e4m3fn quantization (optionally rotated). */
EXPORT int psq_or_quantize_rows_fp8(const void *x, int in_dtype, int64_t M, int64_t K, int64_t ldx,
                                    int g, const float *static_scale, uint8_t *q, int64_t ldq,
                                    float *scale)
{
    int k = g ? log4_of(g) : 0;
    if (g && (k < 0 || K % g)) return -1;
    int err = 0;
#pragma omp parallel
    {
        float *row = (float *)malloc(sizeof(float) * (size_t)(K ? K : 1));
        if (!row) {
#pragma omp atomic write
            err = -2;
        }
#pragma omp for schedule(static)
        for (int64_t m = 0; m < M; m++) {
            if (!row) continue;
            for (int64_t c = 0; c < K; c++) row[c] = load_act(x, m * ldx + c, in_dtype);
            if (g)
                for (int64_t c = 0; c < K; c += g) fwht4_group(row + c, g, k);
            float s, r;
            row_scale(row, K, 448.0f, k, static_scale, &r, &s);
            for (int64_t c = 0; c < K; c++) q[m * ldq + c] = f32_to_e4m3(clamp_lim(row[c] * r, 448.0f));
            scale[m] = s;
        }
        free(row);
    }
    return err;
}

/* ------------------------------------------------------------------------- GEMMs */

/* acc[m][n] = sum_k a[m][k] * w[n][k], int32.  Rows of a given by row_ids (NULL = 0..M-1). */
EXPORT void psq_or_gemm_i8_i32(const int8_t *a, int64_t lda, const int8_t *w, int64_t ldw,
                               int32_t *c, int64_t ldc, int64_t M, int64_t N, int64_t K,
                               const int64_t *row_ids)
{
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t i = 0; i < M; i++)
        for (int64_t n = 0; n < N; n++) {
            const int8_t *ar = a + (row_ids ? row_ids[i] : i) * lda;
            const int8_t *wr = w + n * ldw;
            int32_t acc = 0;
            for (int64_t k = 0; k < K; k++) acc += (int32_t)ar[k] * (int32_t)wr[k];
            c[i * ldc + n] = acc;
        }
}

/* Shared epilogue: y[i][n] = round_out(fmaf(acc, a_s * w_s, bias)).  acc as float. */
static inline float epilogue(float acc, float a_s, float w_s, float bias)
{
    return fmaf(acc, a_s * w_s, bias);
}

EXPORT void psq_or_epilogue_i32(const int32_t *c, int64_t ldc, const float *a_scale,
                                const float *w_scale, int w_scale_per_row, const void *bias,
                                int bias_dtype, void *y, int out_dtype, int64_t ldy, int64_t M,
                                int64_t N, const int64_t *row_ids)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M; i++) {
        float as = a_scale[row_ids ? row_ids[i] : i];
        for (int64_t n = 0; n < N; n++) {
            float ws = w_scale[w_scale_per_row ? n : 0];
            float b = bias ? load_act(bias, n, bias_dtype) : 0.0f;
            store_out(y, i * ldy + n, out_dtype, epilogue((float)c[i * ldc + n], as, ws, b));
        }
    }
}

/* fp8 x fp8 GEMM, accumulated in double (exact products, nearly exact sum); the epilogue
 * then uses the double sum rounded to fp32.  Output rows follow row_ids.  The activations are
 * e4m3fn codes; the weights e4m3fn (w_e5m2 = 0) or e5m2 codes (1). */
static void gemm_fp8_any(const uint8_t *a, int64_t lda, const float *a_scale, const uint8_t *w,
                         int64_t ldw, const float *w_scale, int w_scale_per_row, const void *bias,
                         int bias_dtype, void *y, int out_dtype, int64_t ldy, int64_t M, int64_t N,
                         int64_t K, const int64_t *row_ids, int w_e5m2)
{
    float alut[256], wlut[256];
    for (int i = 0; i < 256; i++) {
        alut[i] = e4m3_to_f32((uint8_t)i);
        wlut[i] = w_e5m2 ? e5m2_to_f32((uint8_t)i) : e4m3_to_f32((uint8_t)i);
    }
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M; i++) {
        int64_t m = row_ids ? row_ids[i] : i;
        const uint8_t *ar = a + m * lda;
        for (int64_t n = 0; n < N; n++) {
            const uint8_t *wr = w + n * ldw;
            double acc = 0.0;
            for (int64_t k = 0; k < K; k++) acc += (double)alut[ar[k]] * (double)wlut[wr[k]];
            float ws = w_scale[w_scale_per_row ? n : 0];
            float b = bias ? load_act(bias, n, bias_dtype) : 0.0f;
            store_out(y, i * ldy + n, out_dtype, epilogue((float)acc, a_scale[m], ws, b));
        }
    }
}

EXPORT void psq_or_gemm_fp8(const uint8_t *a, int64_t lda, const float *a_scale,
                            const uint8_t *w, int64_t ldw, const float *w_scale,
                            int w_scale_per_row, const void *bias, int bias_dtype, void *y,
                            int out_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K,
                            const int64_t *row_ids)
{
    gemm_fp8_any(a, lda, a_scale, w, ldw, w_scale, w_scale_per_row, bias, bias_dtype, y, out_dtype,
                 ldy, M, N, K, row_ids, 0);
}

/* The same with e5m2 weight codes. */
EXPORT void psq_or_gemm_fp8_e5m2w(const uint8_t *a, int64_t lda, const float *a_scale,
                                  const uint8_t *w, int64_t ldw, const float *w_scale,
                                  int w_scale_per_row, const void *bias, int bias_dtype, void *y,
                                  int out_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K,
                                  const int64_t *row_ids)
{
    gemm_fp8_any(a, lda, a_scale, w, ldw, w_scale, w_scale_per_row, bias, bias_dtype, y, out_dtype,
                 ldy, M, N, K, row_ids, 1);
}

/* -------------------------------------------------------- uint4 group weights */

/* Dequantize uint4 asym group weights to fp32 then round to out_dtype (bf16/f16/f32).
 * wq [N, K/2] bytes (low nibble = even k), scale/zero fp16 [N, K/gs]. */
EXPORT int psq_or_dequant_uint4(const uint8_t *wq, const uint16_t *scale, const uint16_t *zero,
                                int64_t N, int64_t K, int gs, void *out, int out_dtype)
{
    if (K % 2 || gs <= 0 || K % gs) return -1;
    int64_t G = K / gs;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; n++)
        for (int64_t k = 0; k < K; k++) {
            uint8_t b = wq[n * (K / 2) + k / 2];
            int q = (k & 1) ? (b >> 4) : (b & 15);
            float s = f16_to_f32(scale[n * G + k / gs]);
            float z = f16_to_f32(zero[n * G + k / gs]);
            store_out(out, n * K + k, out_dtype, ((float)q - z) * s);
        }
    return 0;
}

/* Dequantize int8 row-scaled weights: v = (float)q * s[n]; with rot_group g = 4^k the
 * ConvRot inverse (v @ H^T = v @ H) as 2^-k * T(v) in fp32; then round_out
 * (powershard/operations.py:84-93). */
EXPORT int psq_or_dequant_i8_rows(const int8_t *q, const float *scale, int64_t N, int64_t K,
                                  int g, void *out, int out_dtype)
{
    int k = g ? log4_of(g) : 0;
    if (g && (k < 0 || K % g)) return -1;
    float post = ldexpf(1.0f, -k);
#pragma omp parallel
    {
        float *row = (float *)malloc(sizeof(float) * (size_t)(K ? K : 1));
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; n++) {
            if (!row) continue;
            for (int64_t c = 0; c < K; c++) row[c] = (float)q[n * K + c] * scale[n];
            if (g) {
                for (int64_t c = 0; c < K; c += g) fwht4_group(row + c, g, k);
                for (int64_t c = 0; c < K; c++) row[c] = row[c] * post;
            }
            for (int64_t c = 0; c < K; c++) store_out(out, n * K + c, out_dtype, row[c]);
        }
        free(row);
    }
    return 0;
}

/* fp8 weights: out = round_out(e4m3(q) * s[n or 0]). */
EXPORT void psq_or_dequant_fp8(const uint8_t *q, const float *scale, int per_row, int64_t N,
                               int64_t K, void *out, int out_dtype)
{
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; n++)
        for (int64_t k = 0; k < K; k++)
            store_out(out, n * K + k, out_dtype, e4m3_to_f32(q[n * K + k]) * scale[per_row ? n : 0]);
}

/* e5m2 weights: out = round_out(e5m2(q) * s[n or 0]). */
EXPORT void psq_or_dequant_e5m2(const uint8_t *q, const float *scale, int per_row, int64_t N,
                                int64_t K, void *out, int out_dtype)
{
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; n++)
        for (int64_t k = 0; k < K; k++)
            store_out(out, n * K + k, out_dtype, e5m2_to_f32(q[n * K + k]) * scale[per_row ? n : 0]);
}

/* Weight-only GEMM over an already dequantized weight wd [N, K] (in wd_dtype), activations
 * x [M, K] (x_dtype): acc in double, then y = round_out(fmaf(acc, col_scale[n] or 1, bias)). */
EXPORT void psq_or_gemm_wonly(const void *x, int x_dtype, int64_t ldx, const void *wd,
                              int wd_dtype, const float *col_scale, const void *bias,
                              int bias_dtype, void *y, int out_dtype, int64_t ldy, int64_t M,
                              int64_t N, int64_t K, const int64_t *row_ids)
{
#pragma omp parallel
    {
        float *xr = (float *)malloc(sizeof(float) * (size_t)(K ? K : 1));
#pragma omp for schedule(static)
        for (int64_t i = 0; i < M; i++) {
            if (!xr) continue;
            int64_t m = row_ids ? row_ids[i] : i;
            for (int64_t k = 0; k < K; k++) xr[k] = load_act(x, m * ldx + k, x_dtype);
            for (int64_t n = 0; n < N; n++) {
                double acc = 0.0;
                for (int64_t k = 0; k < K; k++)
                    acc += (double)xr[k] * (double)load_act(wd, n * K + k, wd_dtype);
                float b = bias ? load_act(bias, n, bias_dtype) : 0.0f;
                float cs = col_scale ? col_scale[n] : 1.0f;
                store_out(y, i * ldy + n, out_dtype, fmaf((float)acc, cs, b));
            }
        }
        free(xr);
    }
}

EXPORT int psq_or_version(void) { return 1; }

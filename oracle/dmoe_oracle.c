/*
 * dmoe_oracle.c — CPU oracle for the LLaDA2 block-routed MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY (the checker): loaded by tests/, by the smoke entry
 * and by the CPU-baseline leg of bench.py; never by the product library.
 *
 * Build with -ffp-contract=off and without fast-math: every float expression
 * below is meant as written (one IEEE rounding per operation); fused
 * multiply-adds appear only as explicit fma()/fmaf() calls.
 *
 * References are to files of Akicou/diffuse-cpp.  "ggml-internal" marks
 * semantics of the ggml CPU kernels the reference calls; ggml's sources are
 * not in the reference checkout, so those parts restate ggml's published
 * algorithms.
 */
#include "dmoe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32 (IEEE binary16, round to nearest even)                      */
/* ------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float dmo_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in binary32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return u2f(f2u(v) | sign);
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t dmo_f32_to_f16(float f)
{
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);      /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                        /* below 2^-14     */
        if (ax <= 0x33000000u) return (uint16_t)sign;              /* <= 2^-25 -> 0   */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = (ax >> 13) - (112u << 10);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

void dmo_f16_to_f32_n(const uint16_t *h, float *f, int64_t n)
{
    for (int64_t i = 0; i < n; i++) f[i] = dmo_f16_to_f32(h[i]);
}

void dmo_f32_to_f16_n(const float *f, uint16_t *h, int64_t n)
{
    for (int64_t i = 0; i < n; i++) h[i] = dmo_f32_to_f16(f[i]);
}

/* ------------------------------------------------------------------------ */
/* exp / sigmoid                                                             */
/* ------------------------------------------------------------------------ */
/* exp(x) evaluated in binary64 and rounded once to binary32.  Method:
 * Cody-Waite reduction x = k ln2 + r with ln2 split in a 32-bit head (exact
 * k*ln2_hi for |k| < 2^21) and a tail, |r| <= ln2/2; exp(r) by its Taylor
 * series to degree 13 in Horner form with fma (truncation < 5e-18 relative);
 * scaling by 2^k through the exponent field.  The result is the correctly
 * rounded expf except when exp(x) lies within ~1e-16 relative of a binary32
 * rounding boundary.  Only IEEE add/mul/fma/rint are used, so the same
 * sequence gives the same bits on any IEEE-754 machine.
 * The reference's sigmoid calls ggml's expf (ggml-internal); this function
 * stands for it. */
static double dmo_exp_f64(double x)
{
    const double inv_ln2 = 1.4426950408889634;
    const double ln2_hi  = 6.93147180369123816490e-01; /* 0x3fe62e42fee00000 */
    const double ln2_lo  = 1.90821492927058770002e-10; /* 0x3dea39ef35793c76 */
    double kd = rint(x * inv_ln2);
    double r = fma(-kd, ln2_hi, x);
    r = fma(-kd, ln2_lo, r);
    double p = 1.0 / 6227020800.0;          /* 1/13! */
    p = fma(p, r, 1.0 / 479001600.0);       /* 1/12! */
    p = fma(p, r, 1.0 / 39916800.0);        /* 1/11! */
    p = fma(p, r, 1.0 / 3628800.0);         /* 1/10! */
    p = fma(p, r, 1.0 / 362880.0);          /* 1/9!  */
    p = fma(p, r, 1.0 / 40320.0);           /* 1/8!  */
    p = fma(p, r, 1.0 / 5040.0);            /* 1/7!  */
    p = fma(p, r, 1.0 / 720.0);             /* 1/6!  */
    p = fma(p, r, 1.0 / 120.0);             /* 1/5!  */
    p = fma(p, r, 1.0 / 24.0);              /* 1/4!  */
    p = fma(p, r, 1.0 / 6.0);               /* 1/3!  */
    p = fma(p, r, 0.5);                     /* 1/2!  */
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    int64_t k = (int64_t)kd;
    uint64_t bits = (uint64_t)(k + 1023) << 52;
    double two_k;
    memcpy(&two_k, &bits, 8);
    return p * two_k;
}

float dmo_expf(float x)
{
    if (x != x) return x;
    /* exp(100) overflows binary32 and exp(-110) rounds to 0 in binary32, so
     * clamping keeps every result and keeps k inside the normal exponent range */
    if (x > 100.0f) x = 100.0f;
    if (x < -110.0f) x = -110.0f;
    return (float)dmo_exp_f64((double)x);
}

void dmo_expf_n(const float *x, float *y, int64_t n)
{
    for (int64_t i = 0; i < n; i++) y[i] = dmo_expf(x[i]);
}

/* ggml_sigmoid (diffuse-moe-graph.cpp:204): 1/(1+exp(-x)) (ggml-internal form) */
float dmo_sigmoid(float x)
{
    return 1.0f / (1.0f + dmo_expf(-x));
}

/* ------------------------------------------------------------------------ */
/* block formats                                                             */
/* ------------------------------------------------------------------------ */
size_t dmo_row_size(int32_t type, int64_t n)
{
    switch (type) {
    case DMOE_TYPE_F32:  return (size_t)n * 4;
    case DMOE_TYPE_F16:  return (size_t)n * 2;
    case DMOE_TYPE_Q8_0: return (n % 32) ? 0 : (size_t)(n / 32) * sizeof(dmo_block_q8_0);
    case DMOE_TYPE_Q4_K: return (n % 256) ? 0 : (size_t)(n / 256) * sizeof(dmo_block_q4_K);
    case DMO_TYPE_Q8_K:  return (n % 256) ? 0 : (size_t)(n / 256) * sizeof(dmo_block_q8_K);
    case DMOE_TYPE_Q6_K: return (n % 256) ? 0 : (size_t)(n / 256) * sizeof(dmo_block_q6_K);
    default: return 0;
    }
}

/* ggml type_traits_cpu[type].vec_dot_type (ggml-internal): the type the
 * activations are converted to before mul_mat / mul_mat_id dots. */
int32_t dmo_vec_dot_type(int32_t type)
{
    switch (type) {
    case DMOE_TYPE_F32:  return DMOE_TYPE_F32;
    case DMOE_TYPE_F16:  return DMOE_TYPE_F16;
    case DMOE_TYPE_Q8_0: return DMOE_TYPE_Q8_0;
    case DMOE_TYPE_Q4_K: return DMO_TYPE_Q8_K;
    case DMOE_TYPE_Q6_K: return DMO_TYPE_Q8_K;
    default: return -1;
    }
}

/* 6-bit scale / min of sub-block j (0..7) of a Q4_K super-block
 * (GGUF Q4_K layout: 12 bytes hold eight 6-bit scales and eight 6-bit mins). */
void dmo_q4K_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *m  = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        *m  = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* The 6-bit quant of weight i (0..255) of a Q6_K super-block, in 0..63
 * (ggml-internal block_q6_K layout): in half h = i / 128, at r = i % 128,
 * quarter k = r / 32 and l = r % 32, the low 4 bits are the low (k < 2) or
 * high (k >= 2) nibble of ql[64 h + l + 32 (k & 1)] and the high 2 bits are
 * bits 2k, 2k + 1 of qh[32 h + l].  Weight i belongs to sub-block i / 16,
 * whose scale is scales[i / 16]. */
int dmo_q6K_quant(const dmo_block_q6_K *b, int i)
{
    const int h = i >> 7, r = i & 127, k = r >> 5, l = r & 31;
    const uint8_t lb = b->ql[64 * h + l + 32 * (k & 1)];
    const int lo = (k >> 1) ? (lb >> 4) : (lb & 0x0f);
    const int hi = (b->qh[32 * h + l] >> (2 * k)) & 3;
    return lo | (hi << 4);
}

int dmo_dequant_row(int32_t type, const void *src, float *dst, int64_t n)
{
    switch (type) {
    case DMOE_TYPE_F32:
        memcpy(dst, src, (size_t)n * 4);
        return 0;
    case DMOE_TYPE_F16:
        dmo_f16_to_f32_n((const uint16_t *)src, dst, n);
        return 0;
    case DMOE_TYPE_Q8_0: {
        if (n % 32) return -1;
        const dmo_block_q8_0 *b = (const dmo_block_q8_0 *)src;
        for (int64_t i = 0; i < n / 32; i++) {
            float d = dmo_f16_to_f32(b[i].d);
            for (int j = 0; j < 32; j++) dst[i * 32 + j] = d * (float)b[i].qs[j];
        }
        return 0;
    }
    case DMOE_TYPE_Q4_K: {
        if (n % 256) return -1;
        const dmo_block_q4_K *b = (const dmo_block_q4_K *)src;
        for (int64_t i = 0; i < n / 256; i++) {
            float d = dmo_f16_to_f32(b[i].d), dmin = dmo_f16_to_f32(b[i].dmin);
            float *y = dst + i * 256;
            for (int c = 0; c < 4; c++) {             /* 64-weight chunk c      */
                uint8_t sc0, m0, sc1, m1;
                dmo_q4K_scale_min(2 * c, b[i].scales, &sc0, &m0);
                dmo_q4K_scale_min(2 * c + 1, b[i].scales, &sc1, &m1);
                float d0 = d * (float)sc0, mm0 = dmin * (float)m0;
                float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
                const uint8_t *q = b[i].qs + 32 * c;
                for (int l = 0; l < 32; l++) y[64 * c + l]      = d0 * (float)(q[l] & 0x0f) - mm0;
                for (int l = 0; l < 32; l++) y[64 * c + 32 + l] = d1 * (float)(q[l] >> 4) - mm1;
            }
        }
        return 0;
    }
    case DMOE_TYPE_Q6_K: {
        /* w = d * sc * (q - 32), as ggml's dequantize_row_q6_K evaluates it:
         * (d * sc) first, then times the signed quant (ggml-internal) */
        if (n % 256) return -1;
        const dmo_block_q6_K *b = (const dmo_block_q6_K *)src;
        for (int64_t i = 0; i < n / 256; i++) {
            const float d = dmo_f16_to_f32(b[i].d);
            for (int v = 0; v < 256; v++) {
                const float ds = d * (float)b[i].scales[v >> 4];
                dst[i * 256 + v] = ds * (float)(dmo_q6K_quant(&b[i], v) - 32);
            }
        }
        return 0;
    }
    default:
        return -1;
    }
}

/* ------------------------------------------------------------------------ */
/* quantisers                                                                */
/* ------------------------------------------------------------------------ */
/* round half to even for |v| < 2^22 (ggml's nearest_int, ggml-internal) */
static inline int dmo_nearest_int(float v)
{
    float t = v + 12582912.0f;
    uint32_t i = f2u(t);
    return (int)(i & 0x007fffffu) - 0x00400000;
}

/* Q8_0 block: d = amax/127, q = roundf(x/d) (half away from zero), d stored
 * as fp16 — ggml's quantize_row_q8_0_ref (ggml-internal); used both for the
 * Q8_0 vec_dot_type of activations and for synthetic Q8_0 weights. */
static void quant_q8_0_block(const float *x, dmo_block_q8_0 *y)
{
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) {
        float a = fabsf(x[j]);
        if (a > amax) amax = a;
    }
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    y->d = dmo_f32_to_f16(d);
    for (int j = 0; j < 32; j++) y->qs[j] = (int8_t)roundf(x[j] * id);
}

/* Q8_K block: the signed value of largest magnitude (first one on ties)
 * maps to -127; iscale = -127/max, q = min(127, nearest(iscale*x)),
 * d = 1/iscale, bsums = sums of 16 — ggml's quantize_row_q8_K_ref
 * (ggml-internal).  An all-zero block gets d = 0, q = 0, bsums = 0. */
static void quant_q8_K_block(const float *x, dmo_block_q8_K *y)
{
    float amax = 0.0f, vmax = 0.0f;
    for (int j = 0; j < 256; j++) {
        float a = fabsf(x[j]);
        if (a > amax) { amax = a; vmax = x[j]; }
    }
    if (amax == 0.0f) {
        memset(y, 0, sizeof(*y));
        return;
    }
    float iscale = -127.0f / vmax;
    for (int j = 0; j < 256; j++) {
        int v = dmo_nearest_int(iscale * x[j]);
        y->qs[j] = (int8_t)(v < 127 ? v : 127);
    }
    for (int j = 0; j < 16; j++) {
        int s = 0;
        for (int l = 0; l < 16; l++) s += y->qs[16 * j + l];
        y->bsums[j] = (int16_t)s;
    }
    y->d = 1.0f / iscale;
}

/* Synthetic Q4_K quantiser (min/max per 32-weight sub-block).  Not ggml's
 * make_qkx2_quants: it only has to produce valid, realistic Q4_K blocks.
 * The same steps run on the GPU in dmoe_quantize_device. */
static void quant_q4_K_block(const float *x, dmo_block_q4_K *y)
{
    float scale[8], mn[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int l = 1; l < 32; l++) {
            float v = x[32 * j + l];
            if (v < lo) lo = v;
            if (v > hi) hi = v;
        }
        if (lo > 0.0f) lo = 0.0f;
        scale[j] = (hi - lo) / 15.0f;
        mn[j] = -lo;
        if (scale[j] > max_scale) max_scale = scale[j];
        if (mn[j] > max_min) max_min = mn[j];
    }
    uint16_t dh = dmo_f32_to_f16(max_scale / 63.0f);
    uint16_t mh = dmo_f32_to_f16(max_min / 63.0f);
    float d = dmo_f16_to_f32(dh), dmin = dmo_f16_to_f32(mh);
    float id = d > 0.0f ? 1.0f / d : 0.0f;
    float imin = dmin > 0.0f ? 1.0f / dmin : 0.0f;
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; j++) {
        int a = dmo_nearest_int(scale[j] * id);
        int b = dmo_nearest_int(mn[j] * imin);
        sc[j] = (uint8_t)(a < 0 ? 0 : a > 63 ? 63 : a);
        m[j]  = (uint8_t)(b < 0 ? 0 : b > 63 ? 63 : b);
    }
    memset(y->scales, 0, 12);
    for (int j = 0; j < 4; j++) {
        y->scales[j]     = sc[j];
        y->scales[j + 4] = m[j];
    }
    for (int j = 4; j < 8; j++) {
        y->scales[j + 4] = (uint8_t)((sc[j] & 0x0f) | ((m[j] & 0x0f) << 4));
        y->scales[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
        y->scales[j]     |= (uint8_t)((m[j] >> 4) << 6);
    }
    y->d = dh;
    y->dmin = mh;
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
        float ed = d * (float)sc[j];
        float em = dmin * (float)m[j];
        for (int l = 0; l < 32; l++) {
            int v = 0;
            if (ed > 0.0f) v = dmo_nearest_int((x[32 * j + l] + em) / ed);
            q[32 * j + l] = (uint8_t)(v < 0 ? 0 : v > 15 ? 15 : v);
        }
    }
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++)
            y->qs[32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
}

/* Writes the 6-bit quant q (0..63) of weight i into a Q6_K block (the
 * inverse of dmo_q6K_quant). */
static void q6K_put(dmo_block_q6_K *b, int i, int q)
{
    const int h = i >> 7, r = i & 127, k = r >> 5, l = r & 31;
    uint8_t *lb = &b->ql[64 * h + l + 32 * (k & 1)];
    if (k >> 1)
        *lb = (uint8_t)((*lb & 0x0f) | ((q & 15) << 4));
    else
        *lb = (uint8_t)((*lb & 0xf0) | (q & 15));
    uint8_t *hb = &b->qh[32 * h + l];
    *hb = (uint8_t)((*hb & ~(3 << (2 * k))) | (((q >> 4) & 3) << (2 * k)));
}

/* Synthetic Q6_K quantiser.  Not ggml's make_qx_quants search: per 16-weight
 * sub-block the value of largest magnitude (first on ties) v_j sets the
 * signed scale s_j = -v_j / 32 (so v_j maps to quant -32, as ggml's
 * quantiser maps its extreme value); the super-block's s of largest
 * magnitude sets d = -s_max / 128 (f16), sc_j = min(127, nearest(s_j / d))
 * in -128..127, q = clamp(nearest(x / (d sc_j)), -32, 31) + 32.  Scales and
 * d take both signs, as ggml's do.  The same steps run on the GPU in
 * dmoe_quantize_device. */
static void quant_q6_K_block(const float *x, dmo_block_q6_K *y)
{
    float sj[16];
    float smax = 0.0f, samax = 0.0f;
    for (int j = 0; j < 16; j++) {
        float amax = 0.0f, vmax = 0.0f;
        for (int l = 0; l < 16; l++) {
            const float a = fabsf(x[16 * j + l]);
            if (a > amax) { amax = a; vmax = x[16 * j + l]; }
        }
        sj[j] = -vmax / 32.0f;
        if (amax / 32.0f > samax) { samax = amax / 32.0f; smax = sj[j]; }
    }
    memset(y, 0, sizeof(*y));
    if (samax == 0.0f) return;
    const uint16_t dh = dmo_f32_to_f16(-smax / 128.0f);
    const float d = dmo_f16_to_f32(dh);
    y->d = dh;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    for (int j = 0; j < 16; j++) {
        int sc = dmo_nearest_int(sj[j] * id);
        sc = sc < -128 ? -128 : sc > 127 ? 127 : sc;
        y->scales[j] = (int8_t)sc;
        const float ds = d * (float)sc;
        for (int l = 0; l < 16; l++) {
            int q = 0;
            if (ds != 0.0f) q = dmo_nearest_int(x[16 * j + l] / ds);
            q = q < -32 ? -32 : q > 31 ? 31 : q;
            q6K_put(y, 16 * j + l, q + 32);
        }
    }
}

int dmo_quantize_rows(int32_t type, const float *src, void *dst,
                      int64_t nrows, int64_t n_per_row, int n_threads)
{
    size_t rs = dmo_row_size(type, n_per_row);
    if (rs == 0) return -1;
#ifdef _OPENMP
    if (n_threads <= 0) n_threads = omp_get_max_threads();
#pragma omp parallel for num_threads(n_threads) schedule(static)
#endif
    for (int64_t r = 0; r < nrows; r++) {
        const float *x = src + r * n_per_row;
        uint8_t *y = (uint8_t *)dst + (size_t)r * rs;
        switch (type) {
        case DMOE_TYPE_F32: memcpy(y, x, rs); break;
        case DMOE_TYPE_F16: dmo_f32_to_f16_n(x, (uint16_t *)y, n_per_row); break;
        case DMOE_TYPE_Q8_0:
            for (int64_t b = 0; b < n_per_row / 32; b++)
                quant_q8_0_block(x + 32 * b, (dmo_block_q8_0 *)y + b);
            break;
        case DMOE_TYPE_Q4_K:
            for (int64_t b = 0; b < n_per_row / 256; b++)
                quant_q4_K_block(x + 256 * b, (dmo_block_q4_K *)y + b);
            break;
        case DMOE_TYPE_Q6_K:
            for (int64_t b = 0; b < n_per_row / 256; b++)
                quant_q6_K_block(x + 256 * b, (dmo_block_q6_K *)y + b);
            break;
        default: break;
        }
    }
    (void)n_threads;
    return 0;
}

int dmo_quantize_row_act(int32_t act_type, const float *src, void *dst, int64_t n)
{
    switch (act_type) {
    case DMOE_TYPE_F32: memcpy(dst, src, (size_t)n * 4); return 0;
    case DMOE_TYPE_F16: dmo_f32_to_f16_n(src, (uint16_t *)dst, n); return 0;
    case DMOE_TYPE_Q8_0:
        if (n % 32) return -1;
        for (int64_t b = 0; b < n / 32; b++) quant_q8_0_block(src + 32 * b, (dmo_block_q8_0 *)dst + b);
        return 0;
    case DMO_TYPE_Q8_K:
        if (n % 256) return -1;
        for (int64_t b = 0; b < n / 256; b++) quant_q8_K_block(src + 256 * b, (dmo_block_q8_K *)dst + b);
        return 0;
    default: return -1;
    }
}

/* ------------------------------------------------------------------------ */
/* dots (ggml vec_dot semantics, ggml-internal)                              */
/* ------------------------------------------------------------------------ */
/* F32 x F32 and F16 x F16: products rounded to binary32 (exact for F16),
 * accumulated in binary64 (ggml's scalar ggml_vec_dot_f32/_f16). */
static float dot_f32(int64_t n, const float *w, const float *x)
{
    double s = 0.0;
    for (int64_t i = 0; i < n; i++) s += (double)(w[i] * x[i]);
    return (float)s;
}

static float dot_f16(int64_t n, const uint16_t *w, const uint16_t *x)
{
    double s = 0.0;
    for (int64_t i = 0; i < n; i++) s += (double)(dmo_f16_to_f32(w[i]) * dmo_f16_to_f32(x[i]));
    return (float)s;
}

/* Q8_0 x Q8_0: per block integer dot times fp16(dw)*fp16(dx). */
static float dot_q8_0(int64_t n, const dmo_block_q8_0 *w, const dmo_block_q8_0 *x)
{
    float s = 0.0f;
    for (int64_t b = 0; b < n / 32; b++) {
        int32_t si = 0;
        for (int j = 0; j < 32; j++) si += (int32_t)w[b].qs[j] * (int32_t)x[b].qs[j];
        s += (float)si * (dmo_f16_to_f32(w[b].d) * dmo_f16_to_f32(x[b].d));
    }
    return s;
}

/* Q4_K x Q8_K: per super-block
 *   sumi  = sum_j sc_j * sum_{i in j} q_i * xq_i        (exact int)
 *   summs = sum_j m_j * (bsums[2j] + bsums[2j+1])        (exact int)
 *   s    += (xd*d) * sumi - (xd*dmin) * summs            (binary32) */
static float dot_q4K(int64_t n, const dmo_block_q4_K *w, const dmo_block_q8_K *x)
{
    float s = 0.0f;
    for (int64_t b = 0; b < n / 256; b++) {
        int32_t sumi = 0, summs = 0;
        for (int c = 0; c < 4; c++) {
            uint8_t sc0, m0, sc1, m1;
            dmo_q4K_scale_min(2 * c, w[b].scales, &sc0, &m0);
            dmo_q4K_scale_min(2 * c + 1, w[b].scales, &sc1, &m1);
            const uint8_t *q = w[b].qs + 32 * c;
            const int8_t *xa = x[b].qs + 64 * c;
            int32_t lo = 0, hi = 0;
            for (int l = 0; l < 32; l++) {
                lo += (int32_t)(q[l] & 0x0f) * xa[l];
                hi += (int32_t)(q[l] >> 4) * xa[32 + l];
            }
            sumi += (int32_t)sc0 * lo + (int32_t)sc1 * hi;
            summs += (int32_t)m0 * (x[b].bsums[4 * c] + x[b].bsums[4 * c + 1])
                   + (int32_t)m1 * (x[b].bsums[4 * c + 2] + x[b].bsums[4 * c + 3]);
        }
        float d = x[b].d * dmo_f16_to_f32(w[b].d);
        float dmin = x[b].d * dmo_f16_to_f32(w[b].dmin);
        s += d * (float)sumi;
        s -= dmin * (float)summs;
    }
    return s;
}

/* Q6_K x Q8_K: per super-block
 *   sumi = sum_j sc_j * sum_{i in j} (q_i - 32) * xq_i     (exact int; 16
 *          sub-blocks of 16, |sumi| < 2^31)
 *   s   += (fp16(d) * xd) * sumi                          (binary32)
 * ggml's vec_dot_q6_K_q8_K forms the same integers; the float accumulation
 * order of its SIMD versions is not pinned (ggml-internal). */
static float dot_q6K(int64_t n, const dmo_block_q6_K *w, const dmo_block_q8_K *x)
{
    float s = 0.0f;
    for (int64_t b = 0; b < n / 256; b++) {
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) {
            int32_t sj = 0;
            for (int l = 0; l < 16; l++)
                sj += (int32_t)(dmo_q6K_quant(&w[b], 16 * j + l) - 32) * x[b].qs[16 * j + l];
            sumi += (int32_t)w[b].scales[j] * sj;
        }
        const float d = dmo_f16_to_f32(w[b].d) * x[b].d;
        s += d * (float)sumi;
    }
    return s;
}

/* The AVX-512 dots of dmoe_cpu_simd.c, used once dmo_set_simd(1) has found
 * them supported (the CPU baseline): bit-identical results for the
 * quantised types; binary32 sums for F32 / F16 (ggml's SIMD order, within
 * tolerance of the binary64 sums here). */
static int g_simd = 0;

int dmo_set_simd(int on)
{
    g_simd = on && dmo_simd_available();
    return g_simd;
}

float dmo_vec_dot(int32_t wtype, int64_t n, const void *wrow, const void *xrow)
{
    if (g_simd) {
        if (wtype == DMOE_TYPE_Q4_K)
            return dmo_dot_q4K_simd(n, (const dmo_block_q4_K *)wrow, (const dmo_block_q8_K *)xrow);
        if (wtype == DMOE_TYPE_Q8_0)
            return dmo_dot_q8_0_simd(n, (const dmo_block_q8_0 *)wrow, (const dmo_block_q8_0 *)xrow);
        if (wtype == DMOE_TYPE_F16)
            return dmo_dot_f16_simd(n, (const uint16_t *)wrow, (const uint16_t *)xrow);
        if (wtype == DMOE_TYPE_F32)
            return dmo_dot_f32_simd(n, (const float *)wrow, (const float *)xrow);
    }
    switch (wtype) {
    case DMOE_TYPE_F32:  return dot_f32(n, (const float *)wrow, (const float *)xrow);
    case DMOE_TYPE_F16:  return dot_f16(n, (const uint16_t *)wrow, (const uint16_t *)xrow);
    case DMOE_TYPE_Q8_0: return dot_q8_0(n, (const dmo_block_q8_0 *)wrow, (const dmo_block_q8_0 *)xrow);
    case DMOE_TYPE_Q4_K: return dot_q4K(n, (const dmo_block_q4_K *)wrow, (const dmo_block_q8_K *)xrow);
    case DMOE_TYPE_Q6_K: return dot_q6K(n, (const dmo_block_q6_K *)wrow, (const dmo_block_q8_K *)xrow);
    default: return NAN;
    }
}

/* ------------------------------------------------------------------------ */
/* router                                                                    */
/* ------------------------------------------------------------------------ */
/* Router logits L[t][e] = sum_k W[e][k] x[t][k] (diffuse-moe-graph.cpp:203).
 * ggml's own summation order is ggml-internal; this oracle and the GPU share
 * one canonical order instead (n_embd % 256 == 0):
 *   64 partial sums a_l, l = 0..63; a_l = fma(W[k], x[k], a_l) over
 *   k = 256*i + 4*l + j, i ascending, then j = 0..3;
 *   then six butterfly rounds a_l <- a_l + a_{l xor m}, m = 32,16,8,4,2,1;
 *   L = a_0. */
void dmo_router_logits(const float *W, int64_t w_row_stride, const float *x,
                       int n_tokens, int n_embd, int n_experts, float *logits)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int t = 0; t < n_tokens; t++) {
        const float *xt = x + (size_t)t * n_embd;
        for (int e = 0; e < n_experts; e++) {
            const float *we = W + (size_t)e * w_row_stride;
            float a[64];
            for (int l = 0; l < 64; l++) {
                float acc = 0.0f;
                for (int i = 0; i < n_embd / 256; i++)
                    for (int j = 0; j < 4; j++) {
                        int k = 256 * i + 4 * l + j;
                        acc = fmaf(we[k], xt[k], acc);
                    }
                a[l] = acc;
            }
            for (int m = 32; m >= 1; m >>= 1) {
                float b[64];
                for (int l = 0; l < 64; l++) b[l] = a[l] + a[l ^ m];
                memcpy(a, b, sizeof(a));
            }
            logits[(size_t)t * n_experts + e] = a[0];
        }
    }
}

/* diffuse-moe-graph.cpp:215-216 */
int dmo_use_block_routing(const dmoe_hparams *hp, int n_tokens)
{
    return hp->block_size > 1 && hp->capacity > 0 && hp->capacity < hp->n_experts &&
           n_tokens % hp->block_size == 0;
}

/* Total order used for every "largest" choice: descending float value, ties
 * to the lower expert id, NaN below everything, -0 equal to +0.  ggml's
 * argsort / top_k tie order is ggml-internal; this is the build's rule. */
static inline uint32_t order_key(float f)
{
    if (f != f) return 0u;
    if (f == 0.0f) f = 0.0f;
    uint32_t u = f2u(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static inline int ranks_before(uint32_t ka, int ea, uint32_t kb, int eb)
{
    return ka > kb || (ka == kb && ea < eb);
}

/* :221-229  max over a block's tokens folded as m <- s_j + relu(m - s_j),
 * j = 1..n-1, starting from s_0 (ggml has no elementwise max).  In binary32
 * this is not an exact max and not associative. */
float dmo_block_fold(const float *s, int n, int stride)
{
    float m = s[0];
    for (int j = 1; j < n; j++) {
        float sj = s[(size_t)j * stride];
        float r = m - sj;
        r = r > 0.0f ? r : 0.0f;      /* ggml_relu */
        m = sj + r;
    }
    return m;
}

int dmo_route(const dmoe_hparams *hp, const float *bias, const float *logits,
              int n_tokens, float *probs, float *bmax, float *thr,
              uint8_t *allowed, int32_t *idx, float *weights)
{
    const int E = hp->n_experts, K = hp->top_k, N = n_tokens;
    const int cap = hp->capacity, blk = hp->block_size;
    if (K <= 0 || K > E) return -1;
    float *sel = (float *)malloc((size_t)N * E * sizeof(float));
    float *p = probs ? probs : (float *)malloc((size_t)N * E * sizeof(float));
    if (!sel || !p) return -1;

    /* :204 probs = sigmoid(logits); :207-210 sel = probs + bias */
    for (size_t i = 0; i < (size_t)N * E; i++) {
        p[i] = dmo_sigmoid(logits[i]);
        sel[i] = bias ? p[i] + bias[i % E] : p[i];
    }

    if (dmo_use_block_routing(hp, N)) {
        const int nb = N / blk;
        uint32_t *key = (uint32_t *)malloc((size_t)E * sizeof(uint32_t));
        float *bm = (float *)malloc((size_t)E * sizeof(float));
        for (int b = 0; b < nb; b++) {
            /* :223-229 bmax = fold_j (s_j + relu(bmax - s_j)), sequential in j */
            for (int e = 0; e < E; e++) {
                float m = dmo_block_fold(sel + (size_t)(b * blk) * E + e, blk, E);
                bm[e] = m;
                key[e] = order_key(m);
            }
            /* :232-236 thr = value at position cap-1 of the descending sort */
            int pick = -1;
            for (int e = 0; e < E && pick < 0; e++) {
                int rank = 0;
                for (int f = 0; f < E; f++)
                    if (f != e && ranks_before(key[f], f, key[e], e)) rank++;
                if (rank == cap - 1) pick = e;
            }
            float th = bm[pick];
            /* :241-243 allowed = step(bmax - (thr - 1e-6)); bias 0 / -1e30 */
            float tp = th + (-1e-6f);
            for (int e = 0; e < E; e++) {
                float diff = bm[e] - tp;
                int keep = diff > 0.0f;
                float add = (float)keep * 1e30f + (-1e30f);
                if (bmax) bmax[(size_t)b * E + e] = bm[e];
                if (allowed) allowed[(size_t)b * E + e] = (uint8_t)keep;
                /* :246-248 the block mask is added to every token of the block */
                for (int j = 0; j < blk; j++) {
                    size_t i = (size_t)(b * blk + j) * E + e;
                    sel[i] = sel[i] + add;
                }
            }
            if (thr) thr[b] = th;
        }
        free(key);
        free(bm);
    }

    /* :252 idx = top_k(sel); :253-262 weights from the unbiased probs */
    for (int t = 0; t < N; t++) {
        const float *st = sel + (size_t)t * E;
        int32_t *it = idx + (size_t)t * K;
        for (int s = 0; s < K; s++) {
            int best = -1;
            uint32_t bk = 0;
            for (int e = 0; e < E; e++) {
                int taken = 0;
                for (int q = 0; q < s; q++) taken |= (it[q] == e);
                if (taken) continue;
                uint32_t k = order_key(st[e]);
                if (best < 0 || ranks_before(k, e, bk, best)) { best = e; bk = k; }
            }
            it[s] = best;
        }
        float *wt = weights + (size_t)t * K;
        for (int s = 0; s < K; s++) wt[s] = p[(size_t)t * E + it[s]];
        if (hp->norm_topk_prob) {
            double acc = 0.0;                     /* ggml_sum_rows: binary64 sum */
            for (int s = 0; s < K; s++) acc += (double)wt[s];
            float S = (float)acc;
            for (int s = 0; s < K; s++) wt[s] = wt[s] / S;
        }
        if (hp->routed_scaling != 1.0f)
            for (int s = 0; s < K; s++) wt[s] = wt[s] * hp->routed_scaling;
    }
    free(sel);
    if (!probs) free(p);
    return 0;
}

/* Grouping of (token, slot) pairs by expert inside ggml_mul_mat_id
 * (ggml-internal): a stable counting sort of the t-major, slot-minor pair
 * list.  perm holds pair ids t*K + slot. */
void dmo_dispatch(const int32_t *idx, int n_tokens, int top_k, int n_experts,
                  int32_t *counts, int32_t *offsets, int32_t *perm)
{
    int P = n_tokens * top_k;
    int32_t *cur = (int32_t *)calloc((size_t)n_experts, sizeof(int32_t));
    memset(counts, 0, (size_t)n_experts * sizeof(int32_t));
    for (int i = 0; i < P; i++) counts[idx[i]]++;
    int run = 0;
    for (int e = 0; e < n_experts; e++) { offsets[e] = run; run += counts[e]; }
    for (int i = 0; i < P; i++) {
        int e = idx[i];
        perm[offsets[e] + cur[e]++] = i;
    }
    free(cur);
}

/* ------------------------------------------------------------------------ */
/* whole segment                                                             */
/* ------------------------------------------------------------------------ */
static float silu_f32(float v)  /* ggml_silu: x / (1 + exp(-x)) */
{
    return v / (1.0f + expf(-v));
}

static const uint8_t *tensor_row(const dmoe_tensor *t, int64_t row, int64_t mat)
{
    return (const uint8_t *)t->data + (size_t)mat * t->nb[2] + (size_t)row * t->nb[1];
}

/* Rows [r0,r1) of matrix `mat` of tensor t times a list of activation rows. */
static void matvec_rows(const dmoe_tensor *t, int64_t mat, int64_t r0, int64_t r1,
                        int64_t n, const uint8_t *act, size_t act_stride,
                        const int32_t *rows_in, int n_in, float *out, size_t out_stride)
{
    if (g_simd && t->type == DMOE_TYPE_Q4_K) {
        for (int64_t r = r0; r < r1; r++)
            dmo_rows_q4K_simd(n, (const dmo_block_q4_K *)tensor_row(t, r, mat), act, act_stride, rows_in, n_in,
                              out + r, out_stride);
        return;
    }
    for (int64_t r = r0; r < r1; r++) {
        const void *w = tensor_row(t, r, mat);
        for (int i = 0; i < n_in; i++)
            out[(size_t)i * out_stride + r] =
                dmo_vec_dot(t->type, n, w, act + (size_t)rows_in[i] * act_stride);
    }
}

/* y = W_down (silu(W_gate x) * (W_up x)) with every weight cast to F32
 * (ensure_f32_moe, src/diffuse-moe-graph.cpp:8-12) and F32 activations: the
 * shared expert (:280-286) and the dense MLP (:181-187) build the same ops. */
static void swiglu_f32(int H, int FF, const dmoe_tensor *gate, const dmoe_tensor *up,
                       const dmoe_tensor *down, const float *x, int N, float *y)
{
    float *sg = (float *)malloc((size_t)N * FF * 4);
    float *su = (float *)malloc((size_t)N * FF * 4);
    /* the CPU baseline's dots (dmo_set_simd) or the binary64 sums */
    float (*dotf)(int64_t, const float *, const float *) = g_simd ? dmo_dot_f32_simd : dot_f32;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic)
#endif
    for (int r = 0; r < FF; r++) {
        float *wg = (float *)malloc((size_t)H * 4);
        float *wu = (float *)malloc((size_t)H * 4);
        dmo_dequant_row(gate->type, tensor_row(gate, r, 0), wg, H);
        dmo_dequant_row(up->type, tensor_row(up, r, 0), wu, H);
        for (int t = 0; t < N; t++) {
            float gv = dotf(H, wg, x + (size_t)t * H);
            float uv = dotf(H, wu, x + (size_t)t * H);
            sg[(size_t)t * FF + r] = silu_f32(gv);        /* ggml_silu(g) */
            su[(size_t)t * FF + r] = uv;
        }
        free(wg);
        free(wu);
    }
    for (size_t i = 0; i < (size_t)N * FF; i++) sg[i] = sg[i] * su[i];   /* ggml_mul(g, u) */
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic)
#endif
    for (int r = 0; r < H; r++) {
        float *wd = (float *)malloc((size_t)FF * 4);
        dmo_dequant_row(down->type, tensor_row(down, r, 0), wd, FF);
        for (int t = 0; t < N; t++)
            y[(size_t)t * H + r] = dotf(FF, wd, sg + (size_t)t * FF);
        free(wd);
    }
    free(sg);
    free(su);
}

int dmo_dense_forward(int n_embd, int n_ff, const dmoe_tensor *gate, const dmoe_tensor *up,
                      const dmoe_tensor *down, const float *x, int n_tokens, float *y,
                      int n_threads)
{
    if (n_embd <= 0 || n_ff <= 0 || n_tokens <= 0 || !gate || !up || !down) return -1;
#ifdef _OPENMP
    if (n_threads <= 0) n_threads = omp_get_max_threads();
    int saved_threads = omp_get_max_threads();
    omp_set_num_threads(n_threads);
#else
    (void)n_threads;
#endif
    /* :181-187 g = silu(W_gate cur); u = W_up cur; cur = W_down (g * u) */
    swiglu_f32(n_embd, n_ff, gate, up, down, x, n_tokens, y);
#ifdef _OPENMP
    omp_set_num_threads(saved_threads);
#endif
    return 0;
}

/* ggml_rms_norm (CPU definition): the f32 squares summed in binary64
 * sequentially, mean = (float)(sum / n), scale = 1 / sqrtf(mean + eps),
 * out = x * scale; then ggml_mul by the norm weight. */
void dmo_rms_norm(const float *x, const float *w, int n, float eps, float *out)
{
    double sum = 0.0;
    for (int i = 0; i < n; i++) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < n; i++) {
        const float v = x[i] * scale;
        out[i] = w ? v * w[i] : v;
    }
}

/* The temperature-0 branch of sample_token (src/diffuse-sampler.cpp:29-49):
 * the first index of the largest logit (strict >, so a NaN never wins and a
 * NaN logits[0] stays the answer), prob = 1 / sum of expf(l - max) added
 * sequentially in float. */
void dmo_argmax_prob(const float *logits, int n_vocab, int32_t *token, float *prob)
{
    int best = 0;
    float best_val = logits[0];
    for (int v = 1; v < n_vocab; v++)
        if (logits[v] > best_val) {
            best_val = logits[v];
            best = v;
        }
    float sum = 0.0f;
    for (int v = 0; v < n_vocab; v++) sum += dmo_expf(logits[v] - best_val);
    *token = best;
    *prob = 1.0f / sum;
}

int dmo_head_forward(int n_embd, int n_vocab, const float *norm_w, const dmoe_tensor *output,
                     const float *h, int n_tokens, float eps, int32_t *tokens, float *probs,
                     float *logits_out, int n_threads)
{
    const int H = n_embd, V = n_vocab, N = n_tokens;
    if (H <= 0 || V <= 0 || N <= 0 || !output || !h || !tokens || !probs) return -1;
#ifdef _OPENMP
    if (n_threads <= 0) n_threads = omp_get_max_threads();
    int saved_threads = omp_get_max_threads();
    omp_set_num_threads(n_threads);
#else
    (void)n_threads;
#endif
    /* :296-297 cur = rms_norm(cur) * output_norm */
    float *xn = (float *)malloc((size_t)N * H * 4);
    float *logits = logits_out ? logits_out : (float *)malloc((size_t)N * V * 4);
    for (int t = 0; t < N; t++) dmo_rms_norm(h + (size_t)t * H, norm_w, H, eps, xn + (size_t)t * H);
    /* :299 logits = output x, the output weight cast to F32 (ensure_f32_moe) */
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 64)
#endif
    for (int v = 0; v < V; v++) {
        float *wrow = (float *)malloc((size_t)H * 4);
        dmo_dequant_row(output->type, tensor_row(output, v, 0), wrow, H);
        for (int t = 0; t < N; t++) logits[(size_t)t * V + v] = dot_f32(H, wrow, xn + (size_t)t * H);
        free(wrow);
    }
    for (int t = 0; t < N; t++) dmo_argmax_prob(logits + (size_t)t * V, V, tokens + t, probs + t);
    free(xn);
    if (!logits_out) free(logits);
#ifdef _OPENMP
    omp_set_num_threads(saved_threads);
#endif
    return 0;
}

/* ggml_rope_ext in NEOX mode with n_dims = rotary_dim (freq_scale 1,
 * ext_factor 0, attn_factor 1, no frequency factors), ggml's CPU algorithm:
 * theta_scale = powf(base, -2/n_dims); per position p the angle of pair ic is
 * p * theta_scale^ic formed by repeated float multiplication (theta *=
 * theta_scale); x0 = x[ic], x1 = x[ic + n_dims/2] ->
 * (x0 cos - x1 sin, x0 sin + x1 cos); dims from n_dims on are copied. */
void dmo_rope_neox(float *x, int head_dim, int n_dims, int pos, float base)
{
    const float theta_scale = powf(base, -2.0f / (float)n_dims);
    float theta = (float)pos;
    for (int i0 = 0; i0 < n_dims; i0 += 2) {
        const float c = cosf(theta), sn = sinf(theta);
        const int ic = i0 / 2;
        const float x0 = x[ic], x1 = x[ic + n_dims / 2];
        x[ic] = x0 * c - x1 * sn;
        x[ic + n_dims / 2] = x0 * sn + x1 * c;
        theta *= theta_scale;
    }
    (void)head_dim;
}

/* ggml_flash_attn_ext on the CPU for one query row, F32 K and V: keys in
 * order, s = (q . k) * scale + mask (mask 0 or -inf; -inf keys skipped),
 * online softmax (running max M and sum S, the accumulator rescaled by
 * expf(M_old - M_new) when the max grows), result VKQ / S. */
static void attn_row(const float *q, const float *K, const float *V, size_t kstride, int n_keys,
                     const uint8_t *allowed, int hd, float scale, float *out)
{
    float M = -INFINITY, S = 0.0f;
    float *acc = (float *)calloc((size_t)hd, 4);
    for (int j = 0; j < n_keys; j++) {
        if (!allowed[j]) continue;
        const float *k = K + (size_t)j * kstride, *v = V + (size_t)j * kstride;
        const float s = dot_f32(hd, q, k) * scale;
        float ms = 1.0f, vs = 1.0f;
        if (s > M) {
            ms = dmo_expf(M - s);
            M = s;
            for (int d = 0; d < hd; d++) acc[d] = acc[d] * ms;
        } else {
            vs = dmo_expf(s - M);
        }
        for (int d = 0; d < hd; d++) acc[d] = acc[d] + v[d] * vs;
        S = S * ms + vs;
    }
    for (int d = 0; d < hd; d++) out[d] = acc[d] / S;
    free(acc);
}

int dmo_attn_forward(const dmoe_attn_hparams *ap, const dmoe_attn_desc *desc, const float *h,
                     int n_tokens, float *h_out, float *moe_in, int n_threads)
{
    const int N = n_tokens, H = ap->n_embd, NH = ap->n_head, NKV = ap->n_head_kv;
    const int HD = ap->head_dim, RD = ap->rotary_dim;
    const int QD = NH * HD, KD = NKV * HD, QKV = QD + 2 * KD;
    if (N <= 0 || H <= 0 || NH <= 0 || NKV <= 0 || NH % NKV || HD <= 0 || RD > HD || RD % 2) return -1;
#ifdef _OPENMP
    if (n_threads <= 0) n_threads = omp_get_max_threads();
    int saved_threads = omp_get_max_threads();
    omp_set_num_threads(n_threads);
#else
    (void)n_threads;
#endif
    const float eps = ap->rms_eps;
    float *xn = (float *)malloc((size_t)N * H * 4);
    float *qkv = (float *)malloc((size_t)N * QKV * 4);
    float *att = (float *)malloc((size_t)N * QD * 4);
    float *proj = (float *)malloc((size_t)N * H * 4);
    /* :120-121 input layernorm */
    for (int t = 0; t < N; t++)
        dmo_rms_norm(h + (size_t)t * H, (const float *)desc->attn_norm.data, H, eps, xn + (size_t)t * H);
    /* :124 fused QKV, the weight cast to F32 */
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 16)
#endif
    for (int r = 0; r < QKV; r++) {
        float *w = (float *)malloc((size_t)H * 4);
        dmo_dequant_row(desc->qkv.type, tensor_row(&desc->qkv, r, 0), w, H);
        for (int t = 0; t < N; t++) qkv[(size_t)t * QKV + r] = dot_f32(H, w, xn + (size_t)t * H);
        free(w);
    }
    /* :141-146 QK norm (RMSNorm over head_dim, times q_norm / k_norm), then
     * :154-155 partial NEOX RoPE at position t (inp_pos = 0..N-1, :93-99) */
    for (int t = 0; t < N; t++) {
        float *row = qkv + (size_t)t * QKV;
        for (int hh = 0; hh < NH + NKV; hh++) {
            float *x = row + (size_t)hh * HD;
            if (ap->use_qk_norm) {
                const float *w = (const float *)(hh < NH ? desc->q_norm.data : desc->k_norm.data);
                dmo_rms_norm(x, w, HD, eps, x);
            }
            dmo_rope_neox(x, HD, RD, t, ap->rope_base);
        }
    }
    /* :165-167 flash attention with the block-causal mask (:19-55): query i
     * sees key j iff j / B <= i / B (all keys when B <= 0); query head hh
     * reads kv head hh / (NH / NKV); scale 1 / sqrt(head_dim) */
    const float scale = 1.0f / sqrtf((float)HD);
    const int B = ap->block_length;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic)
#endif
    for (int i = 0; i < N * NH; i++) {
        const int t = i / NH, hh = i % NH, g = hh / (NH / NKV);
        uint8_t *allowed = (uint8_t *)malloc((size_t)N);
        for (int j = 0; j < N; j++) allowed[j] = B <= 0 || j / B <= t / B;
        attn_row(qkv + (size_t)t * QKV + (size_t)hh * HD, qkv + QD + (size_t)g * HD,
                 qkv + QD + KD + (size_t)g * HD, (size_t)QKV, N, allowed, HD, scale,
                 att + (size_t)t * QD + (size_t)hh * HD);
        free(allowed);
    }
    /* :172 output projection (cast to F32), :175 residual */
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 16)
#endif
    for (int r = 0; r < H; r++) {
        float *w = (float *)malloc((size_t)QD * 4);
        dmo_dequant_row(desc->wo.type, tensor_row(&desc->wo, r, 0), w, QD);
        for (int t = 0; t < N; t++) proj[(size_t)t * H + r] = dot_f32(QD, w, att + (size_t)t * QD);
        free(w);
    }
    for (size_t i = 0; i < (size_t)N * H; i++) h_out[i] = proj[i] + h[i];
    /* :177-178 post-attention layernorm: the MoE segment's input */
    if (moe_in)
        for (int t = 0; t < N; t++)
            dmo_rms_norm(h_out + (size_t)t * H, (const float *)desc->post_attn_norm.data, H, eps,
                         moe_in + (size_t)t * H);
    free(xn); free(qkv); free(att); free(proj);
#ifdef _OPENMP
    omp_set_num_threads(saved_threads);
#endif
    return 0;
}

int dmo_layer_forward(const dmoe_hparams *hp, const dmoe_layer_desc *desc,
                      const float *x, int n_tokens, float *y,
                      dmoe_debug *dbg, int n_threads)
{
    const int N = n_tokens, H = hp->n_embd, E = hp->n_experts, K = hp->top_k;
    const int FF = hp->moe_ff;
    const int P = N * K;
#ifdef _OPENMP
    if (n_threads <= 0) n_threads = omp_get_max_threads();
    int saved_threads = omp_get_max_threads();
    omp_set_num_threads(n_threads);
#else
    (void)n_threads;
#endif
    int rc = -1;
    float *logits = (float *)malloc((size_t)N * E * 4);
    float *probs = (float *)malloc((size_t)N * E * 4);
    int32_t *idx = (int32_t *)malloc((size_t)P * 4);
    float *wts = (float *)malloc((size_t)P * 4);
    int32_t *counts = (int32_t *)malloc((size_t)E * 4);
    int32_t *offsets = (int32_t *)malloc((size_t)E * 4);
    int32_t *perm = (int32_t *)malloc((size_t)P * 4);
    int nb = dmo_use_block_routing(hp, N) ? N / hp->block_size : 0;

    /* router weight: F32 as stored, or cast to F32 (ensure_f32_moe, :8-12, :203) */
    const dmoe_tensor *gw = &desc->gate_w;
    float *W = (float *)malloc((size_t)E * H * 4);
    for (int e = 0; e < E; e++)
        dmo_dequant_row(gw->type, tensor_row(gw, e, 0), W + (size_t)e * H, H);
    dmo_router_logits(W, H, x, N, H, E, logits);
    free(W);

    if (dmo_route(hp, desc->gate_bias.data ? (const float *)desc->gate_bias.data : NULL,
                  logits, N, probs,
                  dbg ? dbg->bmax : NULL, dbg ? dbg->thr : NULL,
                  dbg ? dbg->allowed : NULL, idx, wts) != 0)
        goto done;
    dmo_dispatch(idx, N, K, E, counts, offsets, perm);

    {
        /* :264-269 routed experts through mul_mat_id; activations converted to
         * the weight's vec_dot_type first (ggml-internal) */
        const int32_t T = desc->exp_gate.type;
        const int32_t AT = dmo_vec_dot_type(T);
        const size_t xrs = AT == DMOE_TYPE_F32 ? (size_t)H * 4 : dmo_row_size(AT, H);
        const size_t hrs = AT == DMOE_TYPE_F32 ? (size_t)FF * 4 : dmo_row_size(AT, FF);
        uint8_t *xq = (uint8_t *)malloc((size_t)N * xrs);
        float *g = (float *)malloc((size_t)P * FF * 4);
        float *u = (float *)malloc((size_t)P * FF * 4);
        uint8_t *hq = (uint8_t *)malloc((size_t)P * hrs);
        float *ye = (float *)malloc((size_t)P * H * 4);
        int32_t *tok = (int32_t *)malloc((size_t)P * 4);
        for (int t = 0; t < N; t++)
            dmo_quantize_row_act(AT, x + (size_t)t * H, xq + (size_t)t * xrs, H);
        for (int i = 0; i < P; i++) tok[i] = perm[i] / K;

        /* gate / up: work items (expert, 64-row chunk) */
        const int RC = 64;
        const int nck_ff = (FF + RC - 1) / RC;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic)
#endif
        for (int it = 0; it < E * nck_ff; it++) {
            int e = it / nck_ff, c = it % nck_ff;
            if (!counts[e]) continue;
            int r0 = c * RC, r1 = r0 + RC < FF ? r0 + RC : FF;
            const int32_t *tl = tok + offsets[e];
            float *gbuf = (float *)malloc((size_t)counts[e] * FF * 4);
            float *ubuf = (float *)malloc((size_t)counts[e] * FF * 4);
            matvec_rows(&desc->exp_gate, e, r0, r1, H, xq, xrs, tl, counts[e], gbuf, FF);
            matvec_rows(&desc->exp_up, e, r0, r1, H, xq, xrs, tl, counts[e], ubuf, FF);
            for (int i = 0; i < counts[e]; i++) {
                int pr = perm[offsets[e] + i];
                for (int r = r0; r < r1; r++) {
                    g[(size_t)pr * FF + r] = gbuf[(size_t)i * FF + r];
                    u[(size_t)pr * FF + r] = ubuf[(size_t)i * FF + r];
                }
            }
            free(gbuf);
            free(ubuf);
        }
        /* :266-268 inter = silu(gate) * up, then converted for the down dots */
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
        for (int pr = 0; pr < P; pr++) {
            float *hrow = (float *)malloc((size_t)FF * 4);
            for (int r = 0; r < FF; r++)
                hrow[r] = silu_f32(g[(size_t)pr * FF + r]) * u[(size_t)pr * FF + r];
            dmo_quantize_row_act(AT, hrow, hq + (size_t)pr * hrs, FF);
            free(hrow);
        }
        /* :269 down: work items (expert, 256-row chunk of n_embd) */
        const int RD = 256;
        const int nck_h = (H + RD - 1) / RD;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic)
#endif
        for (int it = 0; it < E * nck_h; it++) {
            int e = it / nck_h, c = it % nck_h;
            if (!counts[e]) continue;
            int r0 = c * RD, r1 = r0 + RD < H ? r0 + RD : H;
            const int32_t *pl = perm + offsets[e];
            float *ybuf = (float *)malloc((size_t)counts[e] * H * 4);
            matvec_rows(&desc->exp_down, e, r0, r1, FF, hq, hrs, pl, counts[e], ybuf, H);
            for (int i = 0; i < counts[e]; i++)
                memcpy(ye + (size_t)pl[i] * H + r0, ybuf + (size_t)i * H + r0,
                       (size_t)(r1 - r0) * 4);
            free(ybuf);
        }
        /* :270-278 y = sum over slots of (expert_out * weight), left fold */
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
        for (int t = 0; t < N; t++) {
            float *yt = y + (size_t)t * H;
            for (int r = 0; r < H; r++) {
                float acc = ye[(size_t)(t * K) * H + r] * wts[t * K];
                for (int s = 1; s < K; s++)
                    acc = acc + ye[(size_t)(t * K + s) * H + r] * wts[t * K + s];
                yt[r] = acc;
            }
        }
        free(xq); free(g); free(u); free(hq); free(ye); free(tok);
    }

    if (hp->n_shared > 0 && desc->sh_gate.data) {
        /* :280-286 shared expert on the MoE input with weights cast to F32
         * (ensure_f32_moe) and F32 activations, added to the routed sum */
        float *sd = (float *)malloc((size_t)N * H * 4);
        swiglu_f32(H, hp->shared_ff, &desc->sh_gate, &desc->sh_up, &desc->sh_down, x, N, sd);
        for (size_t i = 0; i < (size_t)N * H; i++) y[i] = y[i] + sd[i];
        free(sd);
    }

    if (dbg) {
        if (dbg->logits) memcpy(dbg->logits, logits, (size_t)N * E * 4);
        if (dbg->probs) memcpy(dbg->probs, probs, (size_t)N * E * 4);
        if (dbg->idx) memcpy(dbg->idx, idx, (size_t)P * 4);
        if (dbg->weights) memcpy(dbg->weights, wts, (size_t)P * 4);
        if (dbg->counts) memcpy(dbg->counts, counts, (size_t)E * 4);
        if (dbg->offsets) memcpy(dbg->offsets, offsets, (size_t)E * 4);
        if (dbg->perm) memcpy(dbg->perm, perm, (size_t)P * 4);
        if (dbg->use_block_routing) *dbg->use_block_routing = nb > 0;
    }
    rc = 0;
done:
    free(logits); free(probs); free(idx); free(wts);
    free(counts); free(offsets); free(perm);
#ifdef _OPENMP
    omp_set_num_threads(saved_threads);
#endif
    return rc;
}

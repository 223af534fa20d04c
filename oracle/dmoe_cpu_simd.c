/* dmoe_cpu_simd.c -- AVX-512 VNNI versions of the oracle's quantised dots,
 * and AVX-512 fp32 / f16 dots, for the CPU baseline that bench.py times
 * (test infrastructure: the checker's fast twin, never the product).
 *
 * ggml's vec_dot_q4_K_q8_K and vec_dot_q8_0_q8_0 have SIMD kernels of their
 * own in the ggml submodule, which is absent from the reference checkout;
 * these are written from the block formats and the dot's definition
 * (dmoe_oracle.c, dot_q4K / dot_q8_0).  The integer parts are exact in any
 * order (sub-block sums of nibble x int8 products by vpdpbusd, 64 per
 * instruction; int8 x int8 block sums by vpmaddwd), and the float steps run
 * in the scalar functions' order, so every result equals the scalar
 * oracle's bit for bit (tests/test_oracle_simd.py).
 *
 * The F32 and F16 dots follow ggml's SIMD ggml_vec_dot_f32 / _f16 on
 * AVX-512 (products and sums in binary32: four 16-lane fused multiply-add
 * accumulators, added and reduced at the end); they round differently from
 * the scalar oracle's binary64 sums, within the tolerance the tests state
 * (tests/test_oracle_simd.py).
 *
 * Functions carry their target attributes and run only when the CPU reports
 * AVX-512 F / BW and VNNI (dmo_simd_available); the library itself stays
 * x86-64-v3.
 */
#include <immintrin.h>
#include <stdint.h>

#include "dmoe_oracle.h"

int dmo_simd_available(void)
{
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vnni");
}

#define SIMD_TARGET __attribute__((target("avx512f,avx512bw,avx512vnni,avx2")))

/* sum of the 16 int32 lanes */
SIMD_TARGET static inline int32_t hsum_epi32(__m512i v)
{
    return _mm512_reduce_add_epi32(v);
}

/* Q4_K x Q8_K, as dot_q4K: per super-block
 *   sumi  = sum_j sc_j * S_j,  S_j = sum_{i in j} q_i x_i     (exact int)
 *   summs = sum_j m_j * (bsums[2j] + bsums[2j+1])             (exact int)
 *   s += (xd * d) * sumi;  s -= (xd * dmin) * summs            (binary32)
 * Chunk c (32 quant bytes: low nibbles = sub-block 2c, high = 2c + 1)
 * against the 64 activation bytes of those sub-blocks is one vpdpbusd:
 * int32 lanes 0..7 sum sub-block 2c, lanes 8..15 sub-block 2c + 1; the
 * lanes are scaled by sc and accumulated, one horizontal sum per block. */
SIMD_TARGET float dmo_dot_q4K_simd(int64_t n, const dmo_block_q4_K *w, const dmo_block_q8_K *x)
{
    float s = 0.0f;
    const __m256i m4 = _mm256_set1_epi8(0x0f);
    for (int64_t b = 0; b < n / 256; b++) {
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) dmo_q4K_scale_min(j, w[b].scales, &sc[j], &mn[j]);
        __m512i acc = _mm512_setzero_si512();
        for (int c = 0; c < 4; c++) {
            const __m256i q = _mm256_loadu_si256((const __m256i *)(w[b].qs + 32 * c));
            const __m256i lo = _mm256_and_si256(q, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
            const __m512i u = _mm512_inserti64x4(_mm512_castsi256_si512(lo), hi, 1);
            const __m512i a = _mm512_loadu_si512((const void *)(x[b].qs + 64 * c));
            const __m512i d = _mm512_dpbusd_epi32(_mm512_setzero_si512(), u, a);
            const __m512i scv = _mm512_inserti64x4(_mm512_castsi256_si512(_mm256_set1_epi32(sc[2 * c])),
                                                   _mm256_set1_epi32(sc[2 * c + 1]), 1);
            acc = _mm512_add_epi32(acc, _mm512_mullo_epi32(d, scv));
        }
        const int32_t sumi = hsum_epi32(acc);
        int32_t summs = 0;
        for (int j = 0; j < 8; j++) summs += (int32_t)mn[j] * (x[b].bsums[2 * j] + x[b].bsums[2 * j + 1]);
        const float dd = x[b].d * dmo_f16_to_f32(w[b].d);
        const float dm = x[b].d * dmo_f16_to_f32(w[b].dmin);
        s += dd * (float)sumi;
        s -= dm * (float)summs;
    }
    return s;
}

/* Q8_0 x Q8_0, as dot_q8_0: per 32-value block the exact int32 dot (int16
 * products summed in pairs by vpmaddwd, 16 lanes), times fp16(dw) * fp16(dx),
 * added in block order. */
SIMD_TARGET float dmo_dot_q8_0_simd(int64_t n, const dmo_block_q8_0 *w, const dmo_block_q8_0 *x)
{
    float s = 0.0f;
    for (int64_t b = 0; b < n / 32; b++) {
        const __m512i a = _mm512_cvtepi8_epi16(_mm256_loadu_si256((const __m256i *)w[b].qs));
        const __m512i v = _mm512_cvtepi8_epi16(_mm256_loadu_si256((const __m256i *)x[b].qs));
        const int32_t si = hsum_epi32(_mm512_madd_epi16(a, v));
        s += (float)si * (dmo_f16_to_f32(w[b].d) * dmo_f16_to_f32(x[b].d));
    }
    return s;
}

/* One Q4_K row against n_in activation rows (out[i * out_stride] for row i
 * of the list): the row's scales and nibble operands are unpacked once per
 * super-block and reused for every activation row; each result is
 * dmo_dot_q4K_simd's (the same integers, the same float steps in block
 * order), so still the scalar dot's bit for bit. */
SIMD_TARGET void dmo_rows_q4K_simd(int64_t n, const dmo_block_q4_K *w, const uint8_t *act, size_t act_stride,
                                   const int32_t *rows_in, int n_in, float *out, size_t out_stride)
{
    const int64_t nb = n / 256;
    const __m256i m4 = _mm256_set1_epi8(0x0f);
    /* per super-block: 4 nibble operands, 4 scale vectors, mins, d, dmin */
    enum { MAXB = 64 };
    __m512i u[MAXB][4], scv[MAXB][4];
    uint8_t mn[MAXB][8];
    float wd[MAXB], wdm[MAXB];
    if (nb > MAXB) {
        for (int i = 0; i < n_in; i++)
            out[(size_t)i * out_stride] =
                dmo_dot_q4K_simd(n, w, (const dmo_block_q8_K *)(act + (size_t)rows_in[i] * act_stride));
        return;
    }
    for (int64_t b = 0; b < nb; b++) {
        uint8_t sc[8];
        for (int j = 0; j < 8; j++) dmo_q4K_scale_min(j, w[b].scales, &sc[j], &mn[b][j]);
        for (int c = 0; c < 4; c++) {
            const __m256i q = _mm256_loadu_si256((const __m256i *)(w[b].qs + 32 * c));
            const __m256i lo = _mm256_and_si256(q, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
            u[b][c] = _mm512_inserti64x4(_mm512_castsi256_si512(lo), hi, 1);
            scv[b][c] = _mm512_inserti64x4(_mm512_castsi256_si512(_mm256_set1_epi32(sc[2 * c])),
                                           _mm256_set1_epi32(sc[2 * c + 1]), 1);
        }
        wd[b] = dmo_f16_to_f32(w[b].d);
        wdm[b] = dmo_f16_to_f32(w[b].dmin);
    }
    for (int i = 0; i < n_in; i++) {
        const dmo_block_q8_K *x = (const dmo_block_q8_K *)(act + (size_t)rows_in[i] * act_stride);
        float s = 0.0f;
        for (int64_t b = 0; b < nb; b++) {
            __m512i acc = _mm512_setzero_si512();
            for (int c = 0; c < 4; c++) {
                const __m512i a = _mm512_loadu_si512((const void *)(x[b].qs + 64 * c));
                acc = _mm512_add_epi32(acc, _mm512_mullo_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), u[b][c], a),
                                                               scv[b][c]));
            }
            const int32_t sumi = hsum_epi32(acc);
            int32_t summs = 0;
            for (int j = 0; j < 8; j++) summs += (int32_t)mn[b][j] * (x[b].bsums[2 * j] + x[b].bsums[2 * j + 1]);
            const float dd = x[b].d * wd[b];
            const float dm = x[b].d * wdm[b];
            s += dd * (float)sumi;
            s -= dm * (float)summs;
        }
        out[(size_t)i * out_stride] = s;
    }
}

/* F32 x F32: four accumulators of 16 lanes over steps of 64 values, fused
 * multiply-adds, then the accumulators added and the lanes reduced; the
 * tail (n % 64) one lane at a time. */
SIMD_TARGET float dmo_dot_f32_simd(int64_t n, const float *w, const float *x)
{
    __m512 a0 = _mm512_setzero_ps(), a1 = _mm512_setzero_ps(), a2 = _mm512_setzero_ps(),
           a3 = _mm512_setzero_ps();
    int64_t i = 0;
    for (; i + 64 <= n; i += 64) {
        a0 = _mm512_fmadd_ps(_mm512_loadu_ps(w + i), _mm512_loadu_ps(x + i), a0);
        a1 = _mm512_fmadd_ps(_mm512_loadu_ps(w + i + 16), _mm512_loadu_ps(x + i + 16), a1);
        a2 = _mm512_fmadd_ps(_mm512_loadu_ps(w + i + 32), _mm512_loadu_ps(x + i + 32), a2);
        a3 = _mm512_fmadd_ps(_mm512_loadu_ps(w + i + 48), _mm512_loadu_ps(x + i + 48), a3);
    }
    float s = _mm512_reduce_add_ps(_mm512_add_ps(_mm512_add_ps(a0, a1), _mm512_add_ps(a2, a3)));
    for (; i < n; i++) s += w[i] * x[i];
    return s;
}

/* F16 x F16: the same on values converted to binary32 (exactly). */
SIMD_TARGET float dmo_dot_f16_simd(int64_t n, const uint16_t *w, const uint16_t *x)
{
    __m512 acc[4] = {_mm512_setzero_ps(), _mm512_setzero_ps(), _mm512_setzero_ps(), _mm512_setzero_ps()};
    int64_t i = 0;
    for (; i + 64 <= n; i += 64)
        for (int k = 0; k < 4; k++) {
            const __m512 wv = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i *)(w + i + 16 * k)));
            const __m512 xv = _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i *)(x + i + 16 * k)));
            acc[k] = _mm512_fmadd_ps(wv, xv, acc[k]);
        }
    float s = _mm512_reduce_add_ps(_mm512_add_ps(_mm512_add_ps(acc[0], acc[1]), _mm512_add_ps(acc[2], acc[3])));
    for (; i < n; i++) s += dmo_f16_to_f32(w[i]) * dmo_f16_to_f32(x[i]);
    return s;
}

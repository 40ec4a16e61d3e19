/*
 * cpu_simd.c -- the SIMD tier of the reference's CPU matmul, restated for
 * the literal int8 format (int8 weights [rows][cols], fp16 scale per 32
 * columns, int8 activations with one fp32 scale per token).
 *
 * TEST INFRASTRUCTURE ONLY: the timed CPU baseline of bench.py (the tier the
 * reference would run on the host), never the checker of a GPU result.
 *
 * Structure of Gemv.Rows / Gemv.Block / Gemv.Single (src/Needle/Gemv.cs:
 * 204-317): rows in blocks of Quant.RowBlock = 4, one 8-lane float
 * accumulator per row; per group the int32 dot of the group's bytes with
 * the activations in eight lanes (Tiers.cs's IInt8Dot: Avx2Dot =
 * maddubs + madd with ones, VnniDot = vpdpbusd), converted and accumulated
 * with one FMA by the group's factor (HalfToSingle(scale) * token scale,
 * the reference's `scaled` array); the four accumulators of a block end in
 * the HorizontalAdd tree of Gemv.Block, a single row in a horizontal sum.
 * The literal weights are signed, so the u8 x s8 instructions take |w| and
 * the activations with w's sign (exact for |q| <= 127, which QuantizeInt8's
 * absmax / 127 scaling always gives).  The int32 group sums are exact; the
 * float association is the SIMD tier's, not Scalar.MatMulRows' (the
 * reference allows 1e-3 between tiers).
 *
 * The tier is picked as Tiers.Best does (src/Needle/Tiers.cs:127-138):
 * AVX-VNNI when the CPU has it, else AVX2 + FMA, else the scalar oracle.
 */
#define _GNU_SOURCE
#include <cpuid.h>
#include <immintrin.h>
#include <string.h>

#include "needle_oracle.h"

int or_simd_tier(void)
{
    unsigned a, b, c, d;
    if (!__get_cpuid_count(1, 0, &a, &b, &c, &d)) return OR_TIER_SCALAR;
    const int fma = (c >> 12) & 1, osxsave = (c >> 27) & 1, f16c = (c >> 29) & 1;
    if (!osxsave || !fma || !f16c) return OR_TIER_SCALAR;
    unsigned xa, xd;
    __asm__("xgetbv" : "=a"(xa), "=d"(xd) : "c"(0));
    if ((xa & 6) != 6) return OR_TIER_SCALAR; /* the OS saves ymm state */
    if (!__get_cpuid_count(7, 0, &a, &b, &c, &d) || !((b >> 5) & 1)) return OR_TIER_SCALAR;
    if (__get_cpuid_count(7, 1, &a, &b, &c, &d) && ((a >> 4) & 1)) return OR_TIER_AVX_VNNI;
    return OR_TIER_AVX2;
}

#define TARGET_AVX2 __attribute__((target("avx2,fma,f16c")))
#define TARGET_VNNI __attribute__((target("avx2,fma,f16c,avxvnni")))

/* Avx2Dot (src/Needle/Tiers.cs:31-41) of one 32-byte group */
TARGET_AVX2 static inline __m256i dot_avx2(__m256i w, __m256i x)
{
    const __m256i pairs = _mm256_maddubs_epi16(_mm256_sign_epi8(w, w), _mm256_sign_epi8(x, w));
    return _mm256_madd_epi16(pairs, _mm256_set1_epi16(1));
}

/* VnniDot (src/Needle/Tiers.cs:44-55) of one 32-byte group */
TARGET_VNNI static inline __m256i dot_vnni(__m256i w, __m256i x)
{
    return _mm256_dpbusd_avx_epi32(_mm256_setzero_si256(), _mm256_sign_epi8(w, w), _mm256_sign_epi8(x, w));
}

/* factor[g] = HalfToSingle(scale[n][g]) * token scale: the reference's
 * `scaled` array (Gemv.Corrections / TileCorrections, with ByteScale 1 and
 * no offsets in the literal format). */
#define SIMD_KERNELS(SUFFIX, TARGET, DOT)                                                                      \
    TARGET static inline void factors_##SUFFIX(const uint16_t* s, int groups, float qs, float* f)           \
    {                                                                                                         \
        for (int g = 0; g < groups; g++) f[g] = _cvtsh_ss(s[g]) * qs;                                         \
    }                                                                                                         \
    TARGET static inline __m256 group_##SUFFIX(const int8_t* w, const int8_t* x, float f, __m256 acc)         \
    {                                                                                                         \
        const __m256i d = DOT(_mm256_loadu_si256((const __m256i*)w), _mm256_loadu_si256((const __m256i*)x)); \
        return _mm256_fmadd_ps(_mm256_cvtepi32_ps(d), _mm256_set1_ps(f), acc);                                \
    }                                                                                                         \
    /* Gemv.Block (4 rows, one token) and Gemv.Single */                                                      \
    TARGET static void rows1_##SUFFIX(const int8_t* w, const uint16_t* scales, int cols, const int8_t* x,      \
                                      float qs, float* y, int r0, int r1, float* f)                           \
    {                                                                                                         \
        const int G = cols / 32;                                                                              \
        int n = r0;                                                                                           \
        for (; n + 4 <= r1; n += 4) {                                                                         \
            for (int i = 0; i < 4; i++) factors_##SUFFIX(scales + (size_t)(n + i) * G, G, qs, f + i * G);     \
            const int8_t* w0 = w + (size_t)n * cols;                                                          \
            __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;                                       \
            for (int g = 0; g < G; g++) {                                                                     \
                a0 = group_##SUFFIX(w0 + 32 * g, x + 32 * g, f[g], a0);                                       \
                a1 = group_##SUFFIX(w0 + cols + 32 * g, x + 32 * g, f[G + g], a1);                            \
                a2 = group_##SUFFIX(w0 + 2 * cols + 32 * g, x + 32 * g, f[2 * G + g], a2);                    \
                a3 = group_##SUFFIX(w0 + 3 * cols + 32 * g, x + 32 * g, f[3 * G + g], a3);                    \
            }                                                                                                 \
            const __m256 q = _mm256_hadd_ps(_mm256_hadd_ps(a0, a1), _mm256_hadd_ps(a2, a3));                  \
            _mm_storeu_ps(y + n, _mm_add_ps(_mm256_castps256_ps128(q), _mm256_extractf128_ps(q, 1)));         \
        }                                                                                                     \
        for (; n < r1; n++) {                                                                                 \
            factors_##SUFFIX(scales + (size_t)n * G, G, qs, f);                                               \
            const int8_t* wr = w + (size_t)n * cols;                                                          \
            __m256 a = _mm256_setzero_ps();                                                                   \
            for (int g = 0; g < G; g++) a = group_##SUFFIX(wr + 32 * g, x + 32 * g, f[g], a);                 \
            const __m128 h = _mm_add_ps(_mm256_castps256_ps128(a), _mm256_extractf128_ps(a, 1));              \
            const __m128 h2 = _mm_hadd_ps(h, h);                                                              \
            y[n] = _mm_cvtss_f32(_mm_hadd_ps(h2, h2));                                                        \
        }                                                                                                     \
    }                                                                                                         \
    /* Gemv.Tile4 / Tile2 (Pair4 / Pair2: two rows x T tokens per pass over the weights; Row4 / Row2 for an   \
     * odd last row): the accumulators of a row's T tokens end in one HorizontalAdd tree. */                  \
    TARGET static void tile_##SUFFIX(int T, const int8_t* w, const uint16_t* scales, int cols, const int8_t* x, \
                                     const float* qs, float* y, int ldy, int r0, int r1, float* f)           \
    {                                                                                                         \
        const int G = cols / 32;                                                                              \
        for (int n = r0; n < r1; n += 2) {                                                                    \
            const int R = n + 2 <= r1 ? 2 : 1;                                                                \
            for (int r = 0; r < R; r++)                                                                       \
                for (int t = 0; t < T; t++)                                                                   \
                    factors_##SUFFIX(scales + (size_t)(n + r) * G, G, qs[t], f + (r * 4 + t) * G);            \
            __m256 acc[2][4];                                                                                 \
            for (int r = 0; r < 2; r++)                                                                       \
                for (int t = 0; t < 4; t++) acc[r][t] = _mm256_setzero_ps();                                  \
            for (int g = 0; g < G; g++)                                                                       \
                for (int r = 0; r < R; r++) {                                                                 \
                    const int8_t* wg = w + (size_t)(n + r) * cols + 32 * g;                                   \
                    for (int t = 0; t < T; t++)                                                               \
                        acc[r][t] = group_##SUFFIX(wg, x + (size_t)t * cols + 32 * g, f[(r * 4 + t) * G + g],  \
                                                   acc[r][t]);                                                \
                }                                                                                             \
            for (int r = 0; r < R; r++) {                                                                     \
                __m256 q;                                                                                     \
                if (T == 4)                                                                                   \
                    q = _mm256_hadd_ps(_mm256_hadd_ps(acc[r][0], acc[r][1]), _mm256_hadd_ps(acc[r][2], acc[r][3])); \
                else {                                                                                        \
                    const __m256 p = _mm256_hadd_ps(acc[r][0], acc[r][1]);                                    \
                    q = _mm256_hadd_ps(p, p);                                                                 \
                }                                                                                             \
                float sums[4];                                                                                \
                _mm_storeu_ps(sums, _mm_add_ps(_mm256_castps256_ps128(q), _mm256_extractf128_ps(q, 1)));      \
                for (int t = 0; t < T; t++) y[(size_t)t * ldy + n + r] = sums[t];                             \
            }                                                                                                 \
        }                                                                                                     \
    }

SIMD_KERNELS(avx2, TARGET_AVX2, dot_avx2)
SIMD_KERNELS(vnni, TARGET_VNNI, dot_vnni)

/* One member's share of Quant.MatMulRows' SIMD branch (src/Needle/Quant.cs:
 * 627-632): tokens in tiles of 4 (Gemv.Tile4), then one tile of 2
 * (Gemv.Tile2), then single tokens (Gemv.Rows), over rows [row_start,
 * row_end).  Group 32; cols a multiple of 32, at most 8192 (otherwise the
 * scalar oracle runs). */
void or_simd_matmul_i8(int tier, const int8_t* w, const uint16_t* scales, int rows, int cols, const int8_t* q,
                       const float* qscale, int tokens, float* y, int ldy, int row_start, int row_end)
{
    float f[8 * 256];
    if (tier == OR_TIER_SCALAR || cols % 32 || cols > 8192) {
        or_matmul_rows_i8(w, scales, rows, cols, 32, q, qscale, tokens, y, ldy, row_start, row_end);
        return;
    }
    const int vnni = tier == OR_TIER_AVX_VNNI;
    int t = 0;
    for (; t + 4 <= tokens; t += 4) {
        if (vnni)
            tile_vnni(4, w, scales, cols, q + (size_t)t * cols, qscale + t, y + (size_t)t * ldy, ldy, row_start,
                      row_end, f);
        else
            tile_avx2(4, w, scales, cols, q + (size_t)t * cols, qscale + t, y + (size_t)t * ldy, ldy, row_start,
                      row_end, f);
    }
    if (tokens - t >= 2) {
        if (vnni)
            tile_vnni(2, w, scales, cols, q + (size_t)t * cols, qscale + t, y + (size_t)t * ldy, ldy, row_start,
                      row_end, f);
        else
            tile_avx2(2, w, scales, cols, q + (size_t)t * cols, qscale + t, y + (size_t)t * ldy, ldy, row_start,
                      row_end, f);
        t += 2;
    }
    for (; t < tokens; t++) {
        if (vnni)
            rows1_vnni(w, scales, cols, q + (size_t)t * cols, qscale[t], y + (size_t)t * ldy, row_start, row_end, f);
        else
            rows1_avx2(w, scales, cols, q + (size_t)t * cols, qscale[t], y + (size_t)t * ldy, row_start, row_end, f);
    }
}

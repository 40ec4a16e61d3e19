/*
 * needle_oracle.c -- CPU restatement of the needle-cs quantized decode path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  Each function cites the reference file:line it restates (paths
 * relative to the IAFahim/needle-cs root).  Build with -ffp-contract=off and
 * without -ffast-math: every float operation below is one IEEE binary32
 * operation in the written order, as the C# reference evaluates it.
 *
 * Parity pinning (how each function is checked, tests/test_oracle.py):
 *   xorshift / fills / half_bits  - reference known-answer semantics, closed form
 *   half_to_single                - all 65536 patterns vs the IEEE rule
 *                                   (tests/Needle.Tests/MatMulTests.cs:88-113)
 *   codebook_fill                 - closed form + Bytes in [0,126]
 *                                   (tests/Needle.Tests/MatMulTests.cs:270-285)
 *   hadamard                      - orthonormal + self-inverse + numpy FWHT
 *                                   (tests/Needle.Tests/KernelTests.cs:10-22)
 *   quantize_int8 / round_trip    - goldens (KernelConformanceTests.cs:312-329,
 *                                   1138-1156; tools/conformance_fixtures.py:81-84)
 *   planes / prepare              - zero-input golden (KernelConformanceTests.cs:280-309),
 *                                   numpy brute force of the permutation and sums
 *   matmul_rows (cq, i8)          - int64 numpy brute force of every group sum,
 *                                   float64 dequantised product, untouched rows
 *   softmax / exp_poly            - softmax goldens (tools/conformance_fixtures.py:71-72),
 *                                   exp_poly vs libm exp within 2 ulp
 *   attention_head / merge        - float64 numpy attention, merge == whole
 *                                   (tests/Needle.Tests/KernelTests.cs:242-282)
 *   argmax / topk_log_softmax     - numpy argmax / sorted log-softmax
 */
#include "needle_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>

#define GROUP 128

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* MathF.Max / MathF.Min (.NET Core 3.0+): NaN propagates, +0 > -0. */
static inline float fmax_ref(float a, float b)
{
    if (a > b) return a;
    if (b > a) return b;
    if (a != a) return a;
    if (b != b) return b;
    return signbit(a) ? b : a;
}
static inline float fmin_ref(float a, float b)
{
    if (a < b) return a;
    if (b < a) return b;
    if (a != a) return a;
    if (b != b) return b;
    return signbit(a) ? a : b;
}

/* ------------------------------------------------------------------ RNG -- */

/* tests/Needle.Tests/Conformance/Conformance.cs:14-17 */
uint64_t or_xs_seed(uint64_t seed) { return seed != 0 ? seed : 0x9E3779B97F4A7C15ull; }

/* tests/Needle.Tests/Conformance/Conformance.cs:19-27 */
uint64_t or_xs_next(uint64_t* state)
{
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x;
}

/* tests/Needle.Tests/Conformance/Conformance.cs:29-32 */
int or_xs_next_int(uint64_t* state, int lo, int hi)
{
    return lo + (int)(or_xs_next(state) % (uint64_t)(hi - lo));
}

/* tests/Needle.Tests/Conformance/Conformance.cs:34-37: ulong -> float is one
 * rounding (the value is < 2^53), then float arithmetic left to right. */
float or_xs_next_float(uint64_t* state, float scale)
{
    float u = (float)(or_xs_next(state) >> 11) * (1.0f / 9007199254740992.0f);
    return ((u - 0.5f) * 2.0f) * scale;
}

/* tests/Needle.Tests/Conformance/Conformance.cs:42-48 */
void or_fill_uniform(float* x, int n, uint64_t* state, float scale)
{
    for (int i = 0; i < n; i++) x[i] = or_xs_next_float(state, scale);
}

/* tests/Needle.Tests/Conformance/Conformance.cs:50-68 */
void or_fill_edges(float* x, int n, uint64_t* state, float scale)
{
    for (int i = 0; i < n; i++) x[i] = or_xs_next_float(state, scale);
    for (int i = 0; i < n; i += 7) x[i] = 0.0f;
    for (int i = 3; i < n; i += 11) x[i] = 1e-38f * (i % 2 == 0 ? 1.0f : -1.0f);
    for (int i = 5; i < n; i += 13) x[i] = (i % 26 < 13 ? 0.5f : -0.5f) * scale;
}

/* tests/Needle.Tests/Conformance/Conformance.cs:70-88 */
void or_fill_sbyte(int8_t* x, int n, uint64_t* state, int extremes)
{
    for (int i = 0; i < n; i++) x[i] = (int8_t)or_xs_next_int(state, -128, 128);
    if (extremes && n > 0) {
        x[0] = -128;
        if (n > 1) x[1] = 127;
        for (int i = 2; i < n; i += 5) x[i] = (i % 2 == 0) ? (int8_t)-128 : (int8_t)127;
    }
}

/* tests/Needle.Tests/Conformance/Conformance.cs:90-101 */
void or_fill_bytes(uint8_t* x, int n, uint64_t* state, int extremes)
{
    for (int i = 0; i < n; i++) x[i] = (uint8_t)or_xs_next_int(state, 0, 256);
    if (extremes && n >= 2) { x[0] = 0x00; x[1] = 0xFF; }
}

/* tests/Needle.Tests/Conformance/Conformance.cs:103-118 */
uint16_t or_half_bits(float value)
{
    uint32_t bits = f2u(value);
    uint32_t sign = (bits >> 16) & 0x8000u;
    uint32_t magnitude = bits & 0x7FFFFFFFu;
    if (magnitude >= 0x47800000u) return (uint16_t)(sign | 0x7BFFu);
    if (magnitude <= 0x38000000u) return (uint16_t)sign;
    uint32_t rounded = (magnitude >> 13) + ((magnitude >> 12) & 1u);
    return (uint16_t)(sign | (rounded - 0x1C000u));
}

/* ------------------------------------------------- synthetic workloads -- */

double or_synth_u53(uint64_t* state)
{
    return (double)(or_xs_next(state) >> 11) * (1.0 / 9007199254740992.0);
}

void or_synth_normal(float* x, size_t n, uint64_t* state)
{
    for (size_t i = 0; i < n; i++) {
        double u1 = 1.0 - or_synth_u53(state);
        double u2 = or_synth_u53(state);
        x[i] = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
    }
}

void or_synth_uniform(float* x, size_t n, uint64_t* state, float lo, float hi)
{
    for (size_t i = 0; i < n; i++) x[i] = (float)((double)lo + ((double)hi - (double)lo) * or_synth_u53(state));
}

void or_synth_int8(int8_t* x, size_t n, uint64_t* state)
{
    for (size_t i = 0; i < n; i++) x[i] = (int8_t)or_xs_next_int(state, -127, 128);
}

/* IEEE binary32 -> binary16, round to nearest even, subnormals and
 * overflow to infinity included. */
uint16_t or_single_to_half_rne(float f)
{
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t)(sign | (a > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);           /* >= 65520 rounds to inf */
    if (a >= 0x38800000u) {                                           /* normal half */
        uint32_t mant = a & 0x7FFFFFu;
        uint32_t exp = (a >> 23) - 112u;
        uint32_t h = (exp << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (a < 0x33000000u) return (uint16_t)sign;                       /* < 2^-25: rounds to 0 */
    {                                                                 /* subnormal half */
        uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
        int shift = 126 - (int)(a >> 23);                             /* 14..24 */
        uint32_t h = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
}

void or_synth_half_uniform(uint16_t* x, size_t n, uint64_t* state, float lo, float hi)
{
    for (size_t i = 0; i < n; i++) {
        float v = (float)((double)lo + ((double)hi - (double)lo) * or_synth_u53(state));
        x[i] = or_single_to_half_rne(v);
    }
}

/* ------------------------------------------------------ scalar kernels -- */

/* src/Needle/Scalar.cs:121-128 */
float or_half_to_single(uint16_t half)
{
    int magnitude = half & 0x7FFF;
    if (magnitude == 0) return 0.0f;
    if (magnitude < 0x0400)
        return (half & 0x8000) != 0 ? (float)(-magnitude) * 5.9604645e-8f : (float)magnitude * 5.9604645e-8f;
    uint32_t bits = (((uint32_t)magnitude << 13) + 0x38000000u) | ((uint32_t)(half & 0x8000) << 16);
    return u2f(bits);
}

/* src/Needle/Scalar.cs:113-119 */
float or_half_to_single_upstream(uint16_t half)
{
    int magnitude = half & 0x7FFF;
    if (magnitude == 0) return 0.0f;
    uint32_t bits = (((uint32_t)magnitude << 13) + 0x38000000u) | ((uint32_t)(half & 0x8000) << 16);
    return u2f(bits);
}

/* src/Needle/Model.cs:44-52.  MathF.Round is round-half-to-even. */
void or_codebook_fill(or_codebook* book, const float* levels, int count)
{
    float peak = 0.0f;
    for (int i = 0; i < count; i++) peak = fmax_ref(peak, fabsf(levels[i]));
    book->byte_scale = peak / 63.0f;
    for (int i = 0; i < 16; i++) book->levels[i] = levels[i % count];
    for (int i = 0; i < 32; i++)
        book->bytes[i] = i % 16 < count ? (uint8_t)(rintf(levels[i % 16] / book->byte_scale) + 63.0f) : (uint8_t)0;
}

/* src/Needle/Scalar.cs:76-89 */
void or_hadamard(const float* source, float* p)
{
    if (source != p) for (int i = 0; i < GROUP; i++) p[i] = source[i];
    for (int stride = 1; stride < GROUP; stride <<= 1)
        for (int block = 0; block < GROUP; block += stride * 2)
            for (int i = block; i < block + stride; i++) {
                float a = p[i];
                float b = p[i + stride];
                p[i] = a + b;
                p[i + stride] = a - b;
            }
    for (int i = 0; i < GROUP; i++) p[i] *= 0.08838834764831845f;
}

/* src/Needle/Scalar.cs:51-53: (x + 1.5*2^23) - 1.5*2^23 */
static inline float round_even(float x)
{
    return (x + 12582912.0f) - 12582912.0f;
}

/* src/Needle/Scalar.cs:55-60 */
float or_abs_max(const float* x, int n)
{
    float peak = 0.0f;
    for (int i = 0; i < n; i++) peak = fmax_ref(peak, fabsf(x[i]));
    return peak;
}

/* src/Needle/Scalar.cs:62-65 */
void or_round_trip(float* x, int n, float inverse, float scale)
{
    for (int i = 0; i < n; i++) x[i] = fmin_ref(fmax_ref(round_even(x[i] * inverse), -128.0f), 127.0f) * scale;
}

/* src/Needle/Scalar.cs:67-74 */
float or_quantize_int8(const float* x, int n, int8_t* destination)
{
    float peak = or_abs_max(x, n);
    float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    float inverse = 1.0f / scale;
    for (int i = 0; i < n; i++)
        destination[i] = (int8_t)fmin_ref(fmax_ref(round_even(x[i] * inverse), -128.0f), 127.0f);
    return scale;
}

/* src/Needle/Scalar.cs:91-111 */
void or_planes(const int8_t* quantized, int bits, int8_t* destination, int* sum)
{
    int s = 0;
    if (bits == 2) {
        for (int j = 0; j < 32; j++)
            for (int p = 0; p < 4; p++) {
                int8_t q = quantized[4 * j + p];
                destination[p * 32 + j] = q;
                s += q;
            }
    } else {
        for (int half = 0; half < 2; half++)
            for (int j = 0; j < 32; j++)
                for (int p = 0; p < 2; p++) {
                    int8_t q = quantized[half * 64 + 2 * j + p];
                    destination[half * 64 + p * 32 + j] = q;
                    s += q;
                }
    }
    *sum = s;
}

/* src/Needle/Quant.cs:473-488 */
void or_prepare(const float* x, int tokens, int cols, int bits, const or_activations* a)
{
    float rotated[GROUP];
    int8_t quantized[GROUP];
    for (int t = 0; t < tokens; t++)
        for (int g = 0; g < a->groups; g++) {
            int slot = t * a->stride + g;
            int sum;
            or_hadamard(x + (long)t * cols + g * GROUP, rotated);
            a->scales[slot] = or_quantize_int8(rotated, GROUP, quantized);
            or_planes(quantized, bits, a->values + ((long)t * a->groups + g) * GROUP, &sum);
            a->offsets[slot] = 63.0f * (float)sum;
        }
}

/* src/Needle/Scalar.cs:130-144 */
void or_decode_row(const or_cq* w, int row, float* destination)
{
    int groups = w->cols / GROUP;
    int row_bytes = w->cols * w->bits / 8;
    const uint8_t* indices = w->indices + (long)row * row_bytes;
    const uint16_t* norms = w->norms + (long)row * groups;
    const float* levels = w->book->levels;
    for (int g = 0; g < groups; g++) {
        float norm = or_half_to_single(norms[g]);
        float* d = destination + g * GROUP;
        if (w->bits == 2)
            for (int i = 0; i < GROUP; i++) d[i] = levels[indices[g * 32 + i / 4] >> (i % 4 * 2) & 3] * norm;
        else
            for (int i = 0; i < GROUP; i++) d[i] = levels[indices[g * 64 + i / 2] >> (i % 2 * 4) & 15] * norm;
    }
}

/* Scalar.cs:166-184: the exact int32 dot of one (token, row, group). */
static int cq_group_dot(const or_cq* w, const uint8_t* packed, const int8_t* x, int g)
{
    const uint8_t* table = w->book->bytes;
    int dot = 0;
    if (w->bits == 2) {
        const uint8_t* p = packed + g * 32;
        for (int j = 0; j < 32; j++) {
            int b = p[j];
            dot += table[b & 3] * x[j] + table[b >> 2 & 3] * x[32 + j] + table[b >> 4 & 3] * x[64 + j] + table[b >> 6 & 3] * x[96 + j];
        }
    } else {
        const uint8_t* p = packed + g * 64;
        for (int half = 0; half < 2; half++)
            for (int j = 0; j < 32; j++) {
                int b = p[half * 32 + j];
                dot += table[b & 15] * x[2 * half * 32 + j] + table[b >> 4] * x[(2 * half + 1) * 32 + j];
            }
    }
    return dot;
}

/* src/Needle/Scalar.cs:146-192 */
void or_matmul_rows(const or_cq* w, const or_activations* a, int tokens, float* y, int ldy,
                    int row_start, int row_end)
{
    int groups = w->cols / GROUP;
    int row_bytes = w->cols * w->bits / 8;
    float byte_scale = w->book->byte_scale;
    for (int t = 0; t < tokens; t++) {
        const int8_t* values = a->values + (long)t * a->cols;
        const float* scales = a->scales + t * a->stride;
        const float* offsets = a->offsets + t * a->stride;
        for (int n = row_start; n < row_end; n++) {
            const uint8_t* packed = w->indices + (long)n * row_bytes;
            const uint16_t* norms = w->norms + (long)n * groups;
            float accumulator = 0.0f;
            float bias = 0.0f;
            for (int g = 0; g < groups; g++) {
                int dot = cq_group_dot(w, packed, values + g * GROUP, g);
                float scaled = or_half_to_single(norms[g]) * byte_scale * scales[g];
                accumulator += scaled * (float)dot;
                bias += scaled * offsets[g];
            }
            y[(long)t * ldy + n] = accumulator - bias;
        }
    }
}

void or_group_dots_cq(const or_cq* w, const or_activations* a, int tokens, int row_start,
                      int row_end, int32_t* dots)
{
    int groups = w->cols / GROUP;
    int row_bytes = w->cols * w->bits / 8;
    long rows = row_end - row_start;
    for (int t = 0; t < tokens; t++) {
        const int8_t* values = a->values + (long)t * a->cols;
        for (int n = row_start; n < row_end; n++) {
            const uint8_t* packed = w->indices + (long)n * row_bytes;
            for (int g = 0; g < groups; g++)
                dots[((long)t * rows + (n - row_start)) * groups + g] = cq_group_dot(w, packed, values + g * GROUP, g);
        }
    }
}

static int i8_group_dot(const int8_t* wrow, const int8_t* x, int group, int g)
{
    int dot = 0;
    for (int j = 0; j < group; j++) dot += (int)wrow[g * group + j] * (int)x[g * group + j];
    return dot;
}

void or_matmul_rows_i8(const int8_t* w, const uint16_t* scales, int rows, int cols, int group,
                       const int8_t* q, const float* qscale, int tokens, float* y, int ldy,
                       int row_start, int row_end)
{
    (void)rows;
    int groups = cols / group;
    const float byte_scale = 1.0f;
    for (int t = 0; t < tokens; t++) {
        const int8_t* values = q + (long)t * cols;
        for (int n = row_start; n < row_end; n++) {
            const int8_t* wrow = w + (long)n * cols;
            const uint16_t* norms = scales + (long)n * groups;
            float accumulator = 0.0f;
            float bias = 0.0f;
            for (int g = 0; g < groups; g++) {
                int dot = i8_group_dot(wrow, values, group, g);
                float scaled = or_half_to_single(norms[g]) * byte_scale * qscale[t];
                accumulator += scaled * (float)dot;
                bias += scaled * 0.0f;
            }
            y[(long)t * ldy + n] = accumulator - bias;
        }
    }
}

void or_group_dots_i8(const int8_t* w, int rows, int cols, int group, const int8_t* q,
                      int tokens, int row_start, int row_end, int32_t* dots)
{
    (void)rows;
    int groups = cols / group;
    long nrows = row_end - row_start;
    for (int t = 0; t < tokens; t++)
        for (int n = row_start; n < row_end; n++)
            for (int g = 0; g < groups; g++)
                dots[((long)t * nrows + (n - row_start)) * groups + g] =
                    i8_group_dot(w + (long)n * cols, q + (long)t * cols, group, g);
}

void or_quantize_rows(const float* x, int tokens, int cols, int8_t* q, float* scales)
{
    for (int t = 0; t < tokens; t++) scales[t] = or_quantize_int8(x + (long)t * cols, cols, q + (long)t * cols);
}

/* ----------------------------------------------------------- softmax -- */

/* x86 MAXPS / MINPS on one lane (Avx.Max / Avx.Min): the first operand when
 * it compares greater (less), else the second -- so a NaN first operand
 * gives the second. */
static inline float max_ps(float a, float b) { return a > b ? a : b; }
static inline float min_ps(float a, float b) { return a < b ? a : b; }

/* src/Needle/Ops.cs:16-31 (one lane; Fma.MultiplyAddNegated(a,b,c) = c - a*b
 * fused).  The clamp is Avx.Min(Avx.Max(x, -87.3), 88.7) (Ops.cs:18): a NaN
 * argument becomes -87.3. */
float or_exp_poly(float x)
{
    x = min_ps(max_ps(x, -87.3f), 88.7f);
    float n = rintf(x * 1.44269504f);
    float r = fmaf(-n, 0.693359375f, x);
    r = fmaf(-n, -2.12194440e-4f, r);
    float p = 1.9875691500e-4f;
    p = fmaf(p, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    float y = fmaf(p, r * r, r + 1.0f);
    float scale = u2f((uint32_t)((int)n + 127) << 23);
    return y * scale;
}

static inline float exp_sel(float x, int use_poly) { return use_poly ? or_exp_poly(x) : expf(x); }

/* src/Needle/Scalar.cs:220-231 */
void or_softmax(float* s, int n, int use_poly)
{
    float peak = -INFINITY;
    for (int i = 0; i < n; i++) peak = fmax_ref(peak, s[i]);
    float total = 0.0f;
    for (int i = 0; i < n; i++) {
        s[i] = exp_sel(s[i] - peak, use_poly);
        total += s[i];
    }
    for (int i = 0; i < n; i++) s[i] /= total;
}

/* src/Needle/Scalar.cs:290-312 (qk dimension generalised) */
void or_attention_head(const int8_t* query, float query_scale, const int8_t* keys,
                       const float* key_scales, const int8_t* values, const float* value_scales,
                       int key_stride, int value_stride, int scale_stride, int first, int last,
                       float* scores, float* output, float* probabilities, int qk_dim,
                       int use_poly)
{
    int count = last - first + 1;
    float inv_sqrt = (float)(1.0 / sqrt((double)qk_dim));
    float scale = query_scale * inv_sqrt;
    for (int s = 0; s < count; s++) {
        const int8_t* key = keys + (long)(first + s) * key_stride;
        int dot = 0;
        for (int d = 0; d < qk_dim; d++) dot += query[d] * key[d];
        scores[s] = (float)dot * key_scales[(long)(first + s) * scale_stride] * scale;
    }
    or_softmax(scores, count, use_poly);
    if (probabilities) for (int s = 0; s < count; s++) probabilities[first + s] = scores[s];
    for (int d = 0; d < 64; d++) output[d] = 0.0f;
    for (int s = 0; s < count; s++) {
        const int8_t* row = values + (long)(first + s) * value_stride;
        float weight = scores[s] * value_scales[(long)(first + s) * scale_stride];
        for (int d = 0; d < 64; d++) output[d] += weight * (float)row[d];
    }
}

void or_attention_partial(const int8_t* query, float query_scale, const int8_t* keys,
                          const float* key_scales, const int8_t* values, const float* value_scales,
                          int key_stride, int value_stride, int scale_stride, int first, int count,
                          int qk_dim, int use_poly, float* output, float* peak_out, float* sum_out)
{
    float inv_sqrt = (float)(1.0 / sqrt((double)qk_dim));
    float scale = query_scale * inv_sqrt;
    float peak = -INFINITY;
    for (int s = 0; s < count; s++) {
        const int8_t* key = keys + (long)(first + s) * key_stride;
        int dot = 0;
        for (int d = 0; d < qk_dim; d++) dot += query[d] * key[d];
        float sc = (float)dot * key_scales[(long)(first + s) * scale_stride] * scale;
        peak = fmax_ref(peak, sc);
    }
    float total = 0.0f;
    for (int d = 0; d < 64; d++) output[d] = 0.0f;
    for (int s = 0; s < count; s++) {
        const int8_t* key = keys + (long)(first + s) * key_stride;
        int dot = 0;
        for (int d = 0; d < qk_dim; d++) dot += query[d] * key[d];
        float sc = (float)dot * key_scales[(long)(first + s) * scale_stride] * scale;
        float e = exp_sel(sc - peak, use_poly);
        total += e;
        const int8_t* row = values + (long)(first + s) * value_stride;
        float weight = e * value_scales[(long)(first + s) * scale_stride];
        for (int d = 0; d < 64; d++) output[d] += weight * (float)row[d];
    }
    *peak_out = peak;
    *sum_out = total;
}

/* src/Needle/Scalar.cs:314-321 */
void or_attention_tile_run(const or_attention_tile* tile, int use_poly)
{
    for (int h = 0; h < tile->heads; h++)
        or_attention_head(tile->queries + h * 48, tile->query_scales[h], tile->keys, tile->key_scales,
                          tile->values, tile->value_scales, tile->key_stride, tile->value_stride,
                          tile->scale_stride, tile->first, tile->first + tile->count - 1, tile->scores,
                          tile->output + h * 64,
                          tile->probabilities ? tile->probabilities + h * tile->probability_stride : NULL,
                          48, use_poly);
}

#define MAX_TILE_HEADS 6
#define PARTIAL_FLOATS (MAX_TILE_HEADS * 64 + 16)

/* src/Needle/Blocks.cs:750-817, non-SIMD branch */
void or_merge_partials(const float* partials, int count, int heads, float* output, int use_poly)
{
    float weights[8];
    for (int h = 0; h < heads; h++) {
        if (count == 2) {
            float peak0 = partials[MAX_TILE_HEADS * 64 + h];
            float peak1 = partials[PARTIAL_FLOATS + MAX_TILE_HEADS * 64 + h];
            float pk = fmax_ref(peak0, peak1);
            float w0 = exp_sel(peak0 - pk, use_poly);
            float w1 = exp_sel(peak1 - pk, use_poly);
            float tot = 0.0f;
            tot += w0 * partials[MAX_TILE_HEADS * 64 + 8 + h];
            tot += w1 * partials[PARTIAL_FLOATS + MAX_TILE_HEADS * 64 + 8 + h];
            float inv = 1.0f / tot;
            for (int d = 0; d < 64; d++)
                output[h * 64 + d] = (w0 * partials[h * 64 + d] + w1 * partials[PARTIAL_FLOATS + h * 64 + d]) * inv;
            continue;
        }
        float peak = -INFINITY;
        for (int c = 0; c < count; c++) peak = fmax_ref(peak, partials[c * PARTIAL_FLOATS + MAX_TILE_HEADS * 64 + h]);
        float total = 0.0f;
        for (int c = 0; c < count; c++) {
            weights[c] = exp_sel(partials[c * PARTIAL_FLOATS + MAX_TILE_HEADS * 64 + h] - peak, use_poly);
            total += weights[c] * partials[c * PARTIAL_FLOATS + MAX_TILE_HEADS * 64 + 8 + h];
        }
        float inverse = 1.0f / total;
        for (int d = 0; d < 64; d++) {
            float sum = 0.0f;
            for (int c = 0; c < count; c++) sum += weights[c] * partials[c * PARTIAL_FLOATS + h * 64 + d];
            output[h * 64 + d] = sum * inverse;
        }
    }
}

/* tests/Needle.Tests/Conformance/KernelConformanceTests.cs:498-525 */
void or_merge_partials_double(const float* partials, int count, int heads, float* output)
{
    for (int h = 0; h < heads; h++) {
        float peak = -INFINITY;
        for (int c = 0; c < count; c++) peak = fmax_ref(peak, partials[c * PARTIAL_FLOATS + MAX_TILE_HEADS * 64 + h]);
        double total = 0;
        for (int c = 0; c < count; c++)
            total += exp((double)(partials[c * PARTIAL_FLOATS + MAX_TILE_HEADS * 64 + h] - peak))
                     * partials[c * PARTIAL_FLOATS + MAX_TILE_HEADS * 64 + 8 + h];
        double inverse = 1.0 / total;
        for (int d = 0; d < 64; d++) {
            double sum = 0;
            for (int c = 0; c < count; c++) {
                double w = exp((double)(partials[c * PARTIAL_FLOATS + MAX_TILE_HEADS * 64 + h] - peak));
                sum += w * partials[c * PARTIAL_FLOATS + h * 64 + d];
            }
            output[h * 64 + d] = (float)(sum * inverse);
        }
    }
}

/* src/Needle/Blocks.cs:973-978 */
void or_attention_span(int position, int window, int frames, int* first, int* count)
{
    *first = window == 0 ? 0 : (position - window + 1 > 0 ? position - window + 1 : 0);
    *count = (frames > 0 ? frames - 1 : position) - *first + 1;
}

/* src/Needle/Blocks.cs:934-938 */
int or_attention_plan(int count, int max_chunks, int* length)
{
    int needed = count / 16;
    if (needed < 1) needed = 1;
    if (needed > max_chunks) needed = max_chunks;
    int len = ((count + needed - 1) / needed + 3) & ~3;
    *length = len;
    return (count + len - 1) / len;
}

/* src/Needle/Blocks.cs:760-815, non-SIMD branch, any count */
void or_merge_head(const float* outs, int out_stride, const float* peaks, const float* sums,
                   int stride, int count, float* output, int use_poly)
{
    if (count == 2) {
        float peak0 = peaks[0], peak1 = peaks[stride];
        float pk = fmax_ref(peak0, peak1);
        float w0 = exp_sel(peak0 - pk, use_poly);
        float w1 = exp_sel(peak1 - pk, use_poly);
        float tot = 0.0f;
        tot += w0 * sums[0];
        tot += w1 * sums[stride];
        float inv = 1.0f / tot;
        for (int d = 0; d < 64; d++) output[d] = (w0 * outs[d] + w1 * outs[out_stride + d]) * inv;
        return;
    }
    float peak = -INFINITY;
    for (int c = 0; c < count; c++) peak = fmax_ref(peak, peaks[(long)c * stride]);
    float total = 0.0f;
    for (int c = 0; c < count; c++) total += exp_sel(peaks[(long)c * stride] - peak, use_poly) * sums[(long)c * stride];
    float inverse = 1.0f / total;
    for (int d = 0; d < 64; d++) {
        float sum = 0.0f;
        for (int c = 0; c < count; c++)
            sum += exp_sel(peaks[(long)c * stride] - peak, use_poly) * outs[(long)c * out_stride + d];
        output[d] = sum * inverse;
    }
}

/* src/Needle/Blocks.cs:927-966 (ExecuteChunk + MergePartials) over a ragged
 * batch with pooled per-slot caches */
void or_attention_decode(const int8_t* q, const float* q_scales, int rows, int heads, int kv_heads,
                         int qk_dim, const int8_t* keys, const float* key_scales,
                         const int8_t* values, const float* value_scales, int capacity,
                         const int* row_slot, const int* row_first, const int* row_count,
                         int max_chunks, float* out)
{
    int group = heads / kv_heads;
    if (max_chunks > 256) max_chunks = 256;
    float* outs = (float*)malloc(sizeof(float) * 64 * (size_t)max_chunks);
    float peaks[256], sums[256];
    for (int r = 0; r < rows; r++) {
        int count = row_count[r];
        size_t base = (size_t)row_slot[r] * capacity;
        for (int h = 0; h < heads; h++) {
            float* dst = out + ((size_t)r * heads + h) * 64;
            if (count <= 0) {
                for (int d = 0; d < 64; d++) dst[d] = 0.0f;
                continue;
            }
            int kv = h / group, length;
            int chunks = or_attention_plan(count, max_chunks, &length);
            for (int c = 0; c < chunks; c++) {
                int begin = c * length;
                int n = count - begin < length ? count - begin : length;
                or_attention_partial(q + ((size_t)r * heads + h) * qk_dim, q_scales[(size_t)r * heads + h],
                                     keys + base * kv_heads * qk_dim + (size_t)kv * qk_dim,
                                     key_scales + base * kv_heads + kv,
                                     values + base * kv_heads * 64 + (size_t)kv * 64,
                                     value_scales + base * kv_heads + kv, kv_heads * qk_dim,
                                     kv_heads * 64, kv_heads, row_first[r] + begin, n, qk_dim, 1,
                                     outs + (size_t)c * 64, &peaks[c], &sums[c]);
            }
            or_merge_head(outs, 64, peaks, sums, 1, chunks, dst, 1);
        }
    }
    free(outs);
}

/* ----------------------------------- Needle 3 attention inputs (rows) -- */

/* Scalar.SumOfSquares (src/Needle/Scalar.cs:206-211) and Ops.InverseRms /
 * ZeroCenteredRms's scalar branch (src/Needle/Ops.cs:209, 233-244):
 * destination = ((1 + scale) * x) * (1 / sqrt(sum x^2 / n + 1e-6)). */
/* The row order of the Needle 3 engine's reductions: 0 (the default) is
 * Scalar.cs's sequential sums, 1 the AVX2 tier's (Ops.cs, the Vector256
 * branches that Tiers.Best takes on AVX2 / AVX-VNNI hosts). */
static int row_tier;
void or_n3_set_tier(int tier) { row_tier = tier; }
int or_n3_tier(void) { return row_tier; }

/* Ops.SumOfSquares / Ops.Dot on the Vector256 tier (Ops.cs:123-205; RmsStats
 * and CenteredRmsStats, :513-630, sum the same way): four 8-lane
 * accumulators take x[i .. i + 32) by FMA, a remaining 16-block goes to s0
 * and s1 and an 8-block to s2, the rest to a sequential FMA tail; the result
 * is Vector256.Sum((s0 + s1) + (s2 + s3)) + tail, where Vector256.Sum(v) =
 * ((v0 + v1) + (v2 + v3)) + ((v4 + v5) + (v6 + v7)) (.NET's Sum(lower) +
 * Sum(upper)).  b == NULL: the squares of a. */
float or_v256_sum(const float* a, const float* b, int n)
{
    float s[4][8] = {{0.0f}};
    int i = 0, bulk = n & ~31;
    if (!b) b = a;
    for (; i < bulk; i += 32)
        for (int k = 0; k < 4; k++)
            for (int j = 0; j < 8; j++) s[k][j] = fmaf(a[i + 8 * k + j], b[i + 8 * k + j], s[k][j]);
    for (; i + 16 <= n; i += 16)
        for (int k = 0; k < 2; k++)
            for (int j = 0; j < 8; j++) s[k][j] = fmaf(a[i + 8 * k + j], b[i + 8 * k + j], s[k][j]);
    if (i + 8 <= n) {
        for (int j = 0; j < 8; j++) s[2][j] = fmaf(a[i + j], b[i + j], s[2][j]);
        i += 8;
    }
    float tail = 0.0f;
    for (; i < n; i++) tail = fmaf(a[i], b[i], tail);
    float v[8];
    for (int j = 0; j < 8; j++) v[j] = (s[0][j] + s[1][j]) + (s[2][j] + s[3][j]);
    return (((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]))) + tail;
}

/* Ops.SumOfSquares in the row tier: Scalar.SumOfSquares or the Vector256 sum */
float or_tier_sum_of_squares(const float* x, int n)
{
    if (row_tier) return or_v256_sum(x, NULL, n);
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += x[i] * x[i];
    return sum;
}

/* Ops.ZeroCenteredRms (Ops.cs:233-255): the elementwise form is the same on
 * both tiers, ((1 + scale) * x) * inverse */
void or_zero_centered_rms(const float* x, const float* scale, int n, float* destination)
{
    float sum = or_tier_sum_of_squares(x, n);
    float inverse = 1.0f / sqrtf(sum / (float)n + 1e-6f);
    for (int i = 0; i < n; i++) destination[i] = (1.0f + scale[i]) * x[i] * inverse;
}

/* Scalar.Rope for one head (src/Needle/Scalar.cs:233-248): rotate-half
 * pairs (i, i + n/2) by the table's cos / sin of the position. */
void or_rope_rotate(float* x, int n, const float* cos_row, const float* sin_row)
{
    int half = n / 2;
    for (int i = 0; i < half; i++) {
        float a = x[i], b = x[half + i];
        x[i] = a * cos_row[i] - b * sin_row[i];
        x[half + i] = b * cos_row[i] + a * sin_row[i];
    }
}

/* EngineCore.TapsAndAttentionHeadsSingle (src/Needle/Engine.cs:1332-1387)
 * with TapsHead (:1302-1330, scalar branch), one row at a time in order:
 * for each query head, key head and value head the three-tap convolution of
 * the current raw frame with the slot's two previous frames
 *   conv = taps[c] * x_t + taps[W + c] * x_{t-1} + taps[2W + c] * x_{t-2}
 * (W = the part's width), then for queries and keys ZeroCenteredRms (QNorm /
 * KNorm, shared by the heads), Rope at the row's position and QuantizeInt8
 * per head -- queries to q / q_scales, keys to the slot's cache row -- and
 * for values QuantizeInt8 per head to the cache; then the slot's history
 * moves on one frame (frame 0 <- frame 1, frame 1 <- the raw row).
 * raw: [rows][qw + kw + vw]; history: [slots][2][qw], [2][kw], [2][vw]
 * (frame 1 the latest); rope tables [capacity][qk/2].  Rows whose slot or
 * position is out of range get q = 0, scale 1 and touch nothing. */
void or_needle3_attention_inputs(const float* raw, int rows, int heads, int kv_heads, int qk, int vd,
                                 const float* q_taps, const float* k_taps, const float* v_taps,
                                 const float* q_norm, const float* k_norm, const float* rope_cos,
                                 const float* rope_sin, float* history, const int* row_slot, const int* row_pos,
                                 int slots, int capacity, int8_t* q, float* q_scales, int8_t* keys,
                                 float* key_scales, int8_t* values, float* value_scales)
{
    int qw = heads * qk, kw = kv_heads * qk, vw = kv_heads * vd, all = qw + kw + vw, half = qk / 2;
    float buf[256];
    for (int r = 0; r < rows; r++) {
        int slot = row_slot[r], pos = row_pos[r];
        const float* x = raw + (long)r * all;
        if (slot < 0 || slot >= slots || pos < 0 || pos >= capacity) {
            memset(q + (long)r * qw, 0, (size_t)qw);
            for (int h = 0; h < heads; h++) q_scales[(long)r * heads + h] = 1.0f;
            continue;
        }
        float* hist = history + (long)slot * 2 * all;
        const float* cs = rope_cos + (long)pos * half;
        const float* sn = rope_sin + (long)pos * half;
        int parts[3] = {qw, kw, vw};
        const float* taps[3] = {q_taps, k_taps, v_taps};
        int base = 0;
        for (int part = 0; part < 3; part++) {
            int W = parts[part], n = part == 2 ? vd : qk, count = W / n;
            const float* cur = x + base;
            const float* f0 = hist + 2 * base;
            const float* f1 = f0 + W;
            for (int h = 0; h < count; h++) {
                int off = h * n;
                for (int c = 0; c < n; c++)
                    buf[c] = taps[part][off + c] * cur[off + c] + taps[part][W + off + c] * f1[off + c] +
                             taps[part][2 * W + off + c] * f0[off + c];
                if (part == 0) {
                    or_zero_centered_rms(buf, q_norm, n, buf);
                    or_rope_rotate(buf, n, cs, sn);
                    q_scales[(long)r * heads + h] = or_quantize_int8(buf, n, q + (long)r * qw + off);
                } else if (part == 1) {
                    or_zero_centered_rms(buf, k_norm, n, buf);
                    or_rope_rotate(buf, n, cs, sn);
                    long cell = (long)slot * capacity + pos;
                    key_scales[cell * kv_heads + h] = or_quantize_int8(buf, n, keys + cell * kw + off);
                } else {
                    long cell = (long)slot * capacity + pos;
                    value_scales[cell * kv_heads + h] = or_quantize_int8(buf, n, values + cell * vw + off);
                }
            }
            base += W;
        }
        /* the history moves on one frame */
        base = 0;
        for (int part = 0; part < 3; part++) {
            int W = parts[part];
            float* f0 = hist + 2 * base;
            float* f1 = f0 + W;
            memcpy(f0, f1, sizeof(float) * W);
            memcpy(f1, x + base, sizeof(float) * W);
            base += W;
        }
    }
}

/* ---------------------------------------------------------- selection -- */

/* src/Needle/Ops.cs:1086-1089 */
int or_argmax(const float* x, int n)
{
    int best = 0;
    for (int i = 1; i < n; i++) if (x[i] > x[best]) best = i;
    return best;
}

/* src/Needle/Ops.cs:1236-1266 (ArgMaxMaskedScalar): ids in ascending order,
 * bit id%32 of mask word id/32, ids >= length skipped; a value replaces the
 * best only when strictly greater (the first id of the maximum wins, -inf
 * and NaN never do); -1 when nothing is selected. */
int or_argmax_masked(const float* x, const uint32_t* mask, int words, int length)
{
    int best = -1;
    float peak = -INFINITY;
    for (int w = 0; w < words; w++) {
        uint32_t bits = mask[w];
        while (bits != 0) {
            int id = w * 32 + __builtin_ctz(bits);
            bits &= bits - 1;
            if (id >= length) continue;
            float value = x[id];
            if (value > peak) { peak = value; best = id; }
        }
    }
    return best;
}

/* src/Needle/Ops.cs:1092-1221, scalar branch (k <= 16) */
/* The selection of src/Needle/Ops.cs:1094-1166 (scalar loop; the AVX loop
 * selects the same ids for NaN-free rows): slots start as (-inf, -1); with
 * the mask and n > 1, id 1 is placed in slot 0 whatever its value and the
 * scan starts at id 4; a value enters when it is above the last slot's
 * value, or equal to it with a lower id than the last slot's (INT_MAX
 * before the first entry), and moves up past larger-or-equal-with-higher-id
 * entries.  So the first scanned value enters even at -inf, later -inf
 * values never do, and slots left over keep (-inf, -1). */
void or_topk_select(const float* x, int n, int k, int mask_special_023, int* top_idx, float* top_val)
{
    for (int i = 0; i < k; i++) { top_val[i] = -INFINITY; top_idx[i] = -1; }
    float min_val = -INFINITY;
    int min_idx = 0x7FFFFFFF;
    int start = 0;
    if (mask_special_023 && n > 1) {
        top_val[0] = x[1];
        top_idx[0] = 1;
        if (k == 1) { min_val = top_val[0]; min_idx = 1; }
        start = 4;
    }
    for (int i = start; i < n; i++) {
        if (mask_special_023 && (i == 0 || i == 2 || i == 3)) continue;
        float v = x[i];
        if (v > min_val || (v == min_val && i < min_idx)) {
            int pos = k - 1;
            while (pos > 0 && (v > top_val[pos - 1] || (v == top_val[pos - 1] && i < top_idx[pos - 1]))) {
                top_val[pos] = top_val[pos - 1];
                top_idx[pos] = top_idx[pos - 1];
                pos--;
            }
            top_val[pos] = v;
            top_idx[pos] = i;
            min_val = top_val[k - 1];
            min_idx = top_idx[k - 1];
        }
    }
}

void or_topk_log_softmax(const float* x, int n, int k, int* indices, float* log_probs,
                         float* probs, int mask_special_023)
{
    float top_val[16];
    int top_idx[16];
    or_topk_select(x, n, k, mask_special_023, top_idx, top_val);
    float peak = top_val[0];
    double total = 0;
    for (int i = 0; i < n; i++) {
        float v = mask_special_023 && (i == 0 || i == 2 || i == 3) ? -1e30f : x[i];
        total += exp((double)(v - peak));
    }
    float log_shift = peak + (float)log(total);
    for (int m = 0; m < k; m++) {
        indices[m] = top_idx[m];
        float lp = top_val[m] - log_shift;
        log_probs[m] = lp;
        if (probs) probs[m] = expf(lp);
    }
}

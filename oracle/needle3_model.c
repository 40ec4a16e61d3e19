/*
 * needle3_model.c -- CPU restatement of Needle 3's batched decode step.
 *
 * TEST INFRASTRUCTURE ONLY: the checker of the GPU Needle 3 engine.
 *
 * EngineCore.ForwardBatch (src/Needle/Engine.cs:2303-2350) with
 * RunLayerBatch (:2352-2398), ApplyEngramBatch (:2399-2463),
 * RunAttentionBatch (:2480-2596), RunMlp (:2146-2156) and PrepareHead
 * (:2188-2189, :920-928), every row operation in the order of its scalar
 * kernel (src/Needle/Scalar.cs) or of the scalar branch of its Ops / Quant
 * dispatcher.  Where the scalar code calls MathF.Exp (Sigmoid, Softmax,
 * Sinkhorn) the reference's polynomial Ops.Exp (Ops.cs:16-31, the exp its
 * AVX paths run) is used instead, since MathF.Exp's bits are the platform
 * libm's; the model's load-time constants (AttnGate = Sigmoid of a stored
 * scalar, the RoPE tables, sqrt(dim)) use the host libm as .NET's MathF does
 * on Linux.
 */
#define _POSIX_C_SOURCE 199309L
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "needle_oracle.h"

#define N3_LANES 4
#define N3_ENGRAM_HISTORY 9
#define N3_ENGRAM_TAPS 4

static inline float round_even(float x) { return (x + 12582912.0f) - 12582912.0f; }
static inline float fmax_(float a, float b) { return a > b ? a : b; }
static inline float fmin_(float a, float b) { return a < b ? a : b; }
/* MathF.Max / MathF.Min on the non-NaN values these kernels see */
static inline float clamp_q(float v) { return fmin_(fmax_(round_even(v), -128.0f), 127.0f); }

/* LayerWeights' AttnGate (Model.cs:147): 1 / (1 + MathF.Exp(-x)) of the
 * stored scalar, computed once at load with the host libm expf. */
float or_n3_attn_gate(float x) { return 1.0f / (1.0f + expf(-x)); }

/* Sigmoid (Scalar.cs:193) with the polynomial exp */
float or_sigmoid(float x) { return 1.0f / (1.0f + or_exp_poly(-x)); }

/* SumOfSquares + InverseRms (Scalar.cs:206-211 or the Vector256 sum, by the
 * row tier; Ops.cs:209).  RmsFakeA8, CenteredRmsFakeA8, RmsUnit and
 * ZeroCenteredRms have the same elementwise form on both tiers; on the
 * Vector256 tier the fused norms take the peak of x (times inverse, which
 * rounds to the same value as the peak of x * inverse: inverse > 0 and
 * rounding is monotone), Ops.cs:632-723. */
static float inverse_rms(const float* x, int n)
{
    return 1.0f / sqrtf(or_tier_sum_of_squares(x, n) / (float)n + 1e-6f);
}

/* Scalar.RmsFakeA8 (Scalar.cs:~367-381) */
void or_rms_fake_a8(const float* x, int n, float* d)
{
    float inverse = inverse_rms(x, n), peak = 0.0f;
    for (int i = 0; i < n; i++) {
        d[i] = x[i] * inverse;
        peak = fmax_(peak, fabsf(d[i]));
    }
    float scale = peak > 0.0f ? peak / 127.0f : 1.0f, round = 1.0f / scale;
    for (int i = 0; i < n; i++) d[i] = clamp_q(d[i] * round) * scale;
}

/* Scalar.CenteredRmsFakeA8 */
void or_centered_rms_fake_a8(const float* x, const float* s, int n, float* d)
{
    float inverse = inverse_rms(x, n), peak = 0.0f;
    for (int i = 0; i < n; i++) {
        d[i] = (1.0f + s[i]) * x[i] * inverse;
        peak = fmax_(peak, fabsf(d[i]));
    }
    float factor = peak > 0.0f ? peak / 127.0f : 1.0f, round = 1.0f / factor;
    for (int i = 0; i < n; i++) d[i] = clamp_q(d[i] * round) * factor;
}

/* Scalar.GateFakeA8, in place */
void or_gate_fake_a8(float* x, const float* gate, int n)
{
    float peak = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] *= or_sigmoid(gate[i]);
        peak = fmax_(peak, fabsf(x[i]));
    }
    float scale = peak > 0.0f ? peak / 127.0f : 1.0f, round = 1.0f / scale;
    for (int i = 0; i < n; i++) x[i] = clamp_q(x[i] * round) * scale;
}

/* Quant.FakeA8 (Quant.cs:69-79): AbsMax, then Scalar.RoundTrip */
float or_fake_a8(float* x, int n)
{
    float peak = or_abs_max(x, n);
    float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    or_round_trip(x, n, 1.0f / scale, scale);
    return scale;
}

/* Scalar.PostNormAdd, or Ops.PostNormAdd's Vector256 branch (Ops.cs:904-
 * 928): residual = fma(gate, ((1 + s) * x) * inverse, residual) in 8-blocks,
 * the tail as ((gate * (1 + s)) * x) * inverse added */
void or_post_norm_add(float* residual, const float* x, const float* s, float gate, int n)
{
    float inverse = inverse_rms(x, n);
    if (or_n3_tier()) {
        int i = 0;
        for (; i + 8 <= n; i += 8)
            for (int j = i; j < i + 8; j++) residual[j] = fmaf(gate, (1.0f + s[j]) * x[j] * inverse, residual[j]);
        for (; i < n; i++) residual[i] += gate * (1.0f + s[i]) * x[i] * inverse;
        return;
    }
    for (int i = 0; i < n; i++) residual[i] += gate * ((1.0f + s[i]) * x[i] * inverse);
}

/* Scalar.Mix4 */
void or_mix4(const float* s, int dim, float w0, float w1, float w2, float w3, float* d)
{
    for (int c = 0; c < dim; c++) d[c] = w0 * s[c] + w1 * s[dim + c] + w2 * s[2 * dim + c] + w3 * s[3 * dim + c];
}

/* Ops.CombineDiff4x4's scalar branch (Ops.cs:800-812): Scalar.CombineDiff4
 * per lane i with mix row i and postGate[i] */
void or_combine_diff4x4(const float* s, int dim, const float* mix, const float* x, const float* u,
                        const float* post_gate, float* d)
{
    for (int i = 0; i < 4; i++) {
        const float* w = mix + 4 * i;
        float post = post_gate[i];
        float* o = d + (size_t)i * dim;
        for (int c = 0; c < dim; c++)
            o[c] = post * (x[c] - u[c]) + w[0] * s[c] + w[1] * s[dim + c] + w[2] * s[2 * dim + c] + w[3] * s[3 * dim + c];
    }
}

/* Scalar.Sinkhorn4x4 */
void or_sinkhorn4x4(const float* logits, float* r)
{
    for (int a = 0; a < 4; a++) {
        float peak = fmax_(fmax_(logits[a * 4], logits[a * 4 + 1]), fmax_(logits[a * 4 + 2], logits[a * 4 + 3]));
        for (int c = 0; c < 4; c++) r[a * 4 + c] = or_exp_poly(logits[a * 4 + c] - peak);
    }
    for (int it = 0; it < 20; it++) {
        for (int a = 0; a < 4; a++) {
            float sum = r[a * 4] + r[a * 4 + 1] + r[a * 4 + 2] + r[a * 4 + 3];
            for (int c = 0; c < 4; c++) r[a * 4 + c] /= sum;
        }
        for (int c = 0; c < 4; c++) {
            float sum = r[c] + r[4 + c] + r[8 + c] + r[12 + c];
            if (sum > 0.0f)
                for (int a = 0; a < 4; a++) r[a * 4 + c] /= sum;
        }
    }
}

/* Ops.RmsUnit's scalar branch (Ops.cs:211-225) */
void or_rms_unit(const float* x, int n, float* d)
{
    float inverse = inverse_rms(x, n);
    for (int i = 0; i < n; i++) d[i] = x[i] * inverse;
}

/* Scalar.Dot, or Ops.Dot's Vector256 branch (Ops.cs:167-205) */
float or_dot(const float* a, const float* b, int n)
{
    if (or_n3_tier()) return or_v256_sum(a, b, n);
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* HadamardMlp.ConditionWeights (Blocks.cs:1104-1125): Scalar.ConditionWeights,
 * or the Vector256 branch -- accumulator k takes the inputs i = k (mod 4) by
 * FMA (a remainder of dim % 4 goes to l0), weights = (l0 + l1) + (l2 + l3),
 * then Ops.Softmax's 8-wide branch (Ops.cs:269-276): e = Exp(v - max),
 * total = Vector256.Sum(e), weights = e * (1 / total). */
static void condition_weights(const float* cond_v, const float* input, int dim, float* weights)
{
    if (!or_n3_tier()) {
        for (int j = 0; j < 8; j++) {
            float sum = 0.0f;
            for (int i = 0; i < dim; i++) sum += input[i] * cond_v[i * 8 + j];
            weights[j] = sum;
        }
        or_softmax(weights, 8, 1);
        return;
    }
    float l[4][8] = {{0.0f}};
    int i = 0;
    for (; i + 4 <= dim; i += 4)
        for (int k = 0; k < 4; k++)
            for (int j = 0; j < 8; j++) l[k][j] = fmaf(input[i + k], cond_v[(i + k) * 8 + j], l[k][j]);
    for (; i < dim; i++)
        for (int j = 0; j < 8; j++) l[0][j] = fmaf(input[i], cond_v[i * 8 + j], l[0][j]);
    float peak = -INFINITY;
    for (int j = 0; j < 8; j++) {
        weights[j] = (l[0][j] + l[1][j]) + (l[2][j] + l[3][j]);
        peak = fmax_(peak, weights[j]);
    }
    float e[8];
    for (int j = 0; j < 8; j++) e[j] = or_exp_poly(weights[j] - peak);
    float total = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
    float inverse = 1.0f / total;
    for (int j = 0; j < 8; j++) weights[j] = e[j] * inverse;
}

/* Quant.GatherRow (Quant.cs:566-575): Scalar.DecodeRow, then Scalar.Hadamard
 * on every 128-group */
void or_gather_row(const or_cq* w, int row, float* d)
{
    or_decode_row(w, row, d);
    for (int g = 0; g < w->cols / 128; g++) or_hadamard(d + g * 128, d + g * 128);
}

/* Scalar.Kron: result[k][c] = sum_j (sum_i left[i][k] z[i][c]) right[j][c],
 * each sum in ascending order from +0.  The vectorised tiers (KronAvx2,
 * Kron32Avx2Range, Kron32Avx2Range4, KronAvx512Range; Blocks.cs:1243-1700)
 * form every output's two sums in the same order, each step one FMA: the
 * row tier's form. */
static void kron(const float* z, int active_rows, const float* left, const float* right, int rows, int cols,
                 int result_rows, float* result, float* scratch)
{
    int fused = or_n3_tier();
    for (int k = 0; k < result_rows; k++) {
        for (int c = 0; c < cols; c++) {
            float sum = 0.0f;
            for (int i = 0; i < active_rows; i++)
                sum = fused ? fmaf(left[i * rows + k], z[i * cols + c], sum) : sum + left[i * rows + k] * z[i * cols + c];
            scratch[c] = sum;
        }
        for (int c = 0; c < cols; c++) {
            float sum = 0.0f;
            for (int j = 0; j < cols; j++)
                sum = fused ? fmaf(scratch[j], right[j * cols + c], sum) : sum + scratch[j] * right[j * cols + c];
            result[k * cols + c] = sum;
        }
    }
}

/* HadamardMlp.Apply's scalar kernels (Blocks.cs:1067-1101 with
 * Scalar.ConditionWeights, ScaleInput, Kron, PermuteModulateActivate,
 * PermuteScale, AccumulateOutput), Scale 1, on one residual row. */
void or_hadamard_mlp(const or_n3_mlp* w, const float* pre_norm, const int* perm_a, const int* perm_b, int dim,
                     int rows, int cols, float* residual)
{
    int width = rows * cols, input_rows = (dim + cols - 1) / cols;
    int output_rows = (input_rows + 3) / 4 * 4;
    if (output_rows > rows) output_rows = rows;
    float* normalized = (float*)malloc(sizeof(float) * dim);
    float* front = (float*)malloc(sizeof(float) * width);
    float* back = (float*)malloc(sizeof(float) * width);
    float* scratch = (float*)malloc(sizeof(float) * cols);
    float weights[8];
    or_zero_centered_rms(residual, pre_norm, dim, normalized);
    condition_weights(w->cond_v, normalized, dim, weights);
    for (int i = 0; i < dim; i++) front[i] = normalized[i] * w->d1[i];
    for (int i = dim; i < input_rows * cols; i++) front[i] = 0.0f;
    kron(front, input_rows, w->w1a, w->w1b, rows, cols, rows, back, scratch);
    for (int n = 0; n < width; n++) {
        float condition = 1.0f;
        for (int j = 0; j < 8; j++) condition += weights[j] * w->cond_u[j * width + n];
        float v = w->d2[n] * condition * back[perm_a[n]] + w->b2[n];
        front[n] = v * or_sigmoid(v);
    }
    kron(front, rows, w->w2a, w->w2b, rows, cols, rows, back, scratch);
    for (int n = 0; n < width; n++) front[n] = back[perm_b[n]] * w->d3[n];
    kron(front, rows, w->w3a, w->w3b, rows, cols, output_rows, back, scratch);
    for (int i = 0; i < dim; i++) residual[i] += 1.0f * (back[i] * w->d4[i]);
    free(normalized);
    free(front);
    free(back);
    free(scratch);
}

/* EngineCore.EngramHashRowsBatch (Engine.cs:2631-2656): the engram table row
 * of every (row, table), -1 before the order's first full n-gram. */
void or_n3_engram_rows(const or_n3_dims* g, const int* tokens, const int* row_slots, int rows, const int* lengths,
                       const int* prev, int* out)
{
    int heads = g->engram_tables / g->order_count, run_start = 0;
    for (int t = 0; t < rows; t++) {
        if (t == 0 || row_slots[t] != row_slots[t - 1]) run_start = t;
        int slot = row_slots[t], position = lengths[slot] + t - run_start;
        const int* pv = prev + 2 * slot;
        for (int o = 0; o < g->order_count; o++)
            for (int h = 0; h < heads; h++) {
                int table = o * heads + h, order = g->orders[o];
                if (position < order - 1) {
                    out[t * g->engram_tables + table] = -1;
                    continue;
                }
                uint32_t acc = 0x9E3779B9u * (uint32_t)(table + 1);
                for (int j = 0; j < order; j++) {
                    int back = t - run_start - j;
                    int token = back >= 0 ? tokens[run_start + back] : pv[back + 2];
                    acc = (acc ^ (uint32_t)token) * 0x01000193u;
                }
                acc ^= acc >> 15;
                out[t * g->engram_tables + table] = table * g->engram_slots + (int)(acc % (uint32_t)g->engram_slots);
            }
    }
}

/* ---------------------------------------------------------- engine -- */

static size_t qkv_all(const or_n3_dims* g)
{
    return (size_t)g->heads * g->qk + (size_t)g->kv_heads * g->qk + (size_t)g->kv_heads * g->vd;
}

int or_n3_init(or_n3_engine* e)
{
    const or_n3_dims* g = &e->m->g;
    int half = g->qk / 2;
    size_t all = qkv_all(g);
    size_t cells = (size_t)g->layers * e->slots * e->capacity;
    size_t hist = (size_t)g->layers * e->slots * 2 * all;
    size_t ehist = (size_t)(g->site_count > 0 ? g->site_count : 1) * e->slots * N3_ENGRAM_HISTORY * g->dim;
    e->rope_cos = (float*)malloc(sizeof(float) * (size_t)e->capacity * half);
    e->rope_sin = (float*)malloc(sizeof(float) * (size_t)e->capacity * half);
    e->keys = (int8_t*)calloc(cells * g->kv_heads * g->qk, 1);
    e->values = (int8_t*)calloc(cells * g->kv_heads * g->vd, 1);
    e->key_scales = (float*)calloc(cells * g->kv_heads, sizeof(float));
    e->value_scales = (float*)calloc(cells * g->kv_heads, sizeof(float));
    e->qkv_hist = (float*)calloc(hist, sizeof(float));
    e->engram_hist = (float*)calloc(ehist, sizeof(float));
    e->snap_qkv = (float*)calloc(hist, sizeof(float));
    e->snap_engram = (float*)calloc(ehist, sizeof(float));
    e->length = (int*)calloc(e->slots, sizeof(int));
    e->marked = (int*)calloc(e->slots, sizeof(int));
    e->prev = (int*)calloc(2 * e->slots, sizeof(int));
    e->snap_prev = (int*)calloc(2 * e->slots, sizeof(int));
    if (!e->rope_cos || !e->rope_sin || !e->keys || !e->values || !e->key_scales || !e->value_scales ||
        !e->qkv_hist || !e->engram_hist || !e->snap_qkv || !e->snap_engram || !e->length || !e->marked ||
        !e->prev || !e->snap_prev)
        return -1;
    or_n3_rope_tables(g->rope_theta, g->qk, e->capacity, e->rope_cos, e->rope_sin);
    return 0;
}

void or_n3_free(or_n3_engine* e)
{
    free(e->rope_cos); free(e->rope_sin); free(e->keys); free(e->values); free(e->key_scales);
    free(e->value_scales); free(e->qkv_hist); free(e->engram_hist); free(e->snap_qkv); free(e->snap_engram);
    free(e->length); free(e->marked); free(e->prev); free(e->snap_prev);
    memset(e, 0, sizeof(*e));
}

/* EngineCore.RopeFrequencies + BuildRopeTables (Engine.cs:336-356): host
 * libm powf / cosf / sinf in float, as MathF on Linux. */
void or_n3_rope_tables(float theta, int qk, int capacity, float* cos_t, float* sin_t)
{
    int half = qk / 2;
    float freq[64];
    for (int i = 0; i < half; i++) freq[i] = 1.0f / powf(theta, 2.0f * (float)i / (float)qk);
    for (int p = 0; p < capacity; p++)
        for (int i = 0; i < half; i++) {
            float angle = (float)p * freq[i];
            cos_t[p * half + i] = cosf(angle);
            sin_t[p * half + i] = sinf(angle);
        }
}

/* ResetView / MarkView / RewindView (Engine.cs:2227-2255): the rewind
 * restores the histories eagerly (the reference marks them pending). */
void or_n3_reset(or_n3_engine* e, int slot)
{
    const or_n3_dims* g = &e->m->g;
    size_t all = qkv_all(g);
    for (int l = 0; l < g->layers; l++)
        memset(e->qkv_hist + ((size_t)l * e->slots + slot) * 2 * all, 0, sizeof(float) * 2 * all);
    for (int s = 0; s < g->site_count; s++)
        memset(e->engram_hist + ((size_t)s * e->slots + slot) * N3_ENGRAM_HISTORY * g->dim, 0,
               sizeof(float) * N3_ENGRAM_HISTORY * g->dim);
    e->prev[2 * slot] = e->prev[2 * slot + 1] = 0;
    e->length[slot] = 0;
    e->marked[slot] = 0;
}

static void copy_slot_state(or_n3_engine* e, int slot, int to_snapshot)
{
    const or_n3_dims* g = &e->m->g;
    size_t all = qkv_all(g), eh = (size_t)N3_ENGRAM_HISTORY * g->dim;
    for (int l = 0; l < g->layers; l++) {
        size_t o = ((size_t)l * e->slots + slot) * 2 * all;
        if (to_snapshot) memcpy(e->snap_qkv + o, e->qkv_hist + o, sizeof(float) * 2 * all);
        else memcpy(e->qkv_hist + o, e->snap_qkv + o, sizeof(float) * 2 * all);
    }
    for (int s = 0; s < g->site_count; s++) {
        size_t o = ((size_t)s * e->slots + slot) * eh;
        if (to_snapshot) memcpy(e->snap_engram + o, e->engram_hist + o, sizeof(float) * eh);
        else memcpy(e->engram_hist + o, e->snap_engram + o, sizeof(float) * eh);
    }
    if (to_snapshot) memcpy(e->snap_prev + 2 * slot, e->prev + 2 * slot, 2 * sizeof(int));
    else memcpy(e->prev + 2 * slot, e->snap_prev + 2 * slot, 2 * sizeof(int));
}

void or_n3_mark(or_n3_engine* e, int slot)
{
    copy_slot_state(e, slot, 1);
    e->marked[slot] = e->length[slot];
}

void or_n3_rewind(or_n3_engine* e, int slot)
{
    copy_slot_state(e, slot, 0);
    e->length[slot] = e->marked[slot];
}

/* Threads of or_n3_forward's matmuls, attention rows and MLP rows (1 by
 * default).  Every output element is still computed by one thread in the
 * scalar order, so the results do not depend on the count. */
static int n3_threads = 1;
void or_n3_set_threads(int n) { n3_threads = n > 0 ? n : 1; }

static void matmul(const or_cq* w, int row0, int rows, const float* x, int tokens, float* y, int ldy, int bits)
{
    int cols = w->cols, groups = cols / 128, stride = (groups + 7) / 8 * 8;
    or_activations a;
    a.values = (int8_t*)malloc((size_t)tokens * cols);
    a.scales = (float*)calloc((size_t)tokens * stride, sizeof(float));
    a.offsets = (float*)calloc((size_t)tokens * stride, sizeof(float));
    a.cols = cols;
    a.groups = groups;
    a.stride = stride;
    or_prepare(x, tokens, cols, bits, &a);
    or_cq slice = *w;
    slice.indices = w->indices + (size_t)row0 * cols * w->bits / 8;
    slice.norms = w->norms + (size_t)row0 * groups;
    slice.rows = rows;
    int blocks = rows / 32 < n3_threads ? rows / 32 : n3_threads;
    if (blocks < 1) blocks = 1;
#pragma omp parallel for num_threads(blocks) schedule(static)
    for (int b = 0; b < blocks; b++)
        or_matmul_rows(&slice, &a, tokens, y, ldy, (int)((long)rows * b / blocks), (int)((long)rows * (b + 1) / blocks));
    free(a.values);
    free(a.scales);
    free(a.offsets);
}

/* Planted composition mistakes, the controls of the tests that hold this
 * forward to the reference's own numpy forward (0, the default: none):
 *   1  hpre's +4 lane bias on lane (l + 1) % 4 instead of l % 4
 *   2  every engram site applied one layer late
 *   3  the MLP run before PostNormAdd instead of after it
 *   4  the Sinkhorn mix applied transposed
 *   5  PostNorm and PreHada exchanged (each layer's records read one slot off) */
static int plant;
void or_n3_set_plant(int which) { plant = which; }

void or_n3_forward(or_n3_engine* e, const int* tokens, const int* row_slots, int rows, const int* head_rows,
                   int heads, float* logits)
{
    const or_n3_model* m = e->m;
    const or_n3_dims* g = &m->g;
    int dim = g->dim, sw = N3_LANES * dim, H = g->heads, KV = g->kv_heads, qk = g->qk, vd = g->vd;
    int qw = H * qk, kw = KV * qk, vw = KV * vd, ow = H * vd, all = qw + kw + vw, ET = g->engram_tables;
    float* stream = (float*)malloc(sizeof(float) * (size_t)rows * sw);
    float* next = (float*)malloc(sizeof(float) * (size_t)rows * sw);
    float* normed = (float*)malloc(sizeof(float) * (size_t)rows * sw);
    float* input = (float*)malloc(sizeof(float) * (size_t)rows * dim);
    float* residual = (float*)malloc(sizeof(float) * (size_t)rows * dim);
    float* buf = (float*)malloc(sizeof(float) * (size_t)rows * (dim > ow ? dim : ow));
    float* raw = (float*)malloc(sizeof(float) * (size_t)rows * all);
    float* gate = (float*)malloc(sizeof(float) * (size_t)rows * ow);
    float* att = (float*)malloc(sizeof(float) * (size_t)rows * ow);
    float* proj = (float*)malloc(sizeof(float) * (size_t)rows * dim);
    float* key = (float*)malloc(sizeof(float) * (size_t)rows * dim);
    float* stage = (float*)malloc(sizeof(float) * (size_t)rows * (N3_ENGRAM_HISTORY + 1) * dim);
    float* conv = (float*)malloc(sizeof(float) * (size_t)rows * dim);
    float* unit_a = (float*)malloc(sizeof(float) * dim);
    float* unit_b = (float*)malloc(sizeof(float) * dim);
    float pre[16 * 4], post[16 * 4], res[16 * 16];
    float* pre_out = (float*)malloc(sizeof(float) * (size_t)rows * 4);
    float* post_out = (float*)malloc(sizeof(float) * (size_t)rows * 4);
    float* res_out = (float*)malloc(sizeof(float) * (size_t)rows * 16);
    float* post_gate = (float*)malloc(sizeof(float) * (size_t)rows * 4);
    float* mix = (float*)malloc(sizeof(float) * (size_t)rows * 16);
    int8_t* q8 = (int8_t*)malloc((size_t)rows * qw);
    float* qs = (float*)malloc(sizeof(float) * (size_t)rows * H);
    int* pos = (int*)malloc(sizeof(int) * rows);
    int* first = (int*)malloc(sizeof(int) * rows);
    int* count = (int*)malloc(sizeof(int) * rows);
    int* erows = (int*)malloc(sizeof(int) * (size_t)rows * (ET > 0 ? ET : 1));
    (void)pre; (void)post; (void)res;
    int run_start = 0;
    for (int t = 0; t < rows; t++) {
        if (t == 0 || row_slots[t] != row_slots[t - 1]) run_start = t;
        pos[t] = e->length[row_slots[t]] + t - run_start;
    }
    if (g->site_count > 0) or_n3_engram_rows(g, tokens, row_slots, rows, e->length, e->prev, erows);
    /* embedding: GatherRow, x += (sqrt(dim) - 1) x, copied to the four lanes */
    float emb_scale = sqrtf((float)dim) - 1.0f;
    for (int t = 0; t < rows; t++) {
        or_gather_row(&m->embedding, tokens[t], buf);
        for (int i = 0; i < dim; i++) buf[i] += emb_scale * buf[i];
        for (int lane = 0; lane < N3_LANES; lane++) memcpy(stream + (size_t)t * sw + lane * dim, buf, sizeof(float) * dim);
    }
    if (e->trace) memcpy(e->trace, stream, sizeof(float) * (size_t)rows * sw);
    for (int l = 0; l < g->layers; l++) {
        const or_n3_layer* w = &m->layer[l];
        int lane = l % N3_LANES, bias_lane = plant == 1 ? (l + 1) % N3_LANES : lane;
        /* hyper-connection phi (RunLayerBatch, Engine.cs:2356-2364) */
        for (int t = 0; t < rows; t++) or_rms_fake_a8(stream + (size_t)t * sw, sw, normed + (size_t)t * sw);
        matmul(&m->phi_pre, l * 4, 4, normed, rows, pre_out, 4, 4);
        matmul(&m->phi_post, l * 4, 4, normed, rows, post_out, 4, 4);
        matmul(&m->phi_res, l * 16, 16, normed, rows, res_out, 16, 4);
        for (int t = 0; t < rows; t++) {
            float hpre[4], logits_mix[16];
            for (int i = 0; i < 4; i++) {
                hpre[i] = or_sigmoid(m->a_pre[l] * pre_out[t * 4 + i] + m->b_pre[l * 4 + i] + (i == bias_lane ? 4.0f : -4.0f));
                post_gate[t * 4 + i] =
                    2.0f * or_sigmoid(m->a_post[l] * post_out[t * 4 + i] + m->b_post[l * 4 + i] + (i == lane ? 0.0f : -4.0f));
            }
            or_mix4(stream + (size_t)t * sw, dim, hpre[0], hpre[1], hpre[2], hpre[3], input + (size_t)t * dim);
            for (int i = 0; i < 16; i++) logits_mix[i] = m->a_res[l] * res_out[t * 16 + i] + m->b_res[l * 16 + i];
            or_sinkhorn4x4(logits_mix, mix + t * 16);
            if (plant == 4)
                for (int i = 0; i < 4; i++)
                    for (int j = i + 1; j < 4; j++) {
                        float a = mix[t * 16 + i * 4 + j];
                        mix[t * 16 + i * 4 + j] = mix[t * 16 + j * 4 + i];
                        mix[t * 16 + j * 4 + i] = a;
                    }
            memcpy(residual + (size_t)t * dim, input + (size_t)t * dim, sizeof(float) * dim);
        }
        /* engram (ApplyEngramBatch, Engine.cs:2399-2463) */
        int site = -1;
        for (int s = 0; s < g->site_count; s++)
            if (g->sites[s] + (plant == 2) == l) site = s;
        if (site >= 0) {
            const or_n3_site* S = &m->site[site];
            int sub = g->engram_sub, stride = N3_ENGRAM_HISTORY + 1;
            for (int t = 0; t < rows; t++) {
                float* ein = buf + (size_t)t * dim;
                for (int table = 0; table < ET; table++) {
                    int row = erows[t * ET + table];
                    if (row < 0) memset(ein + table * sub, 0, sizeof(float) * sub);
                    else or_gather_row(&S->tables, row, ein + table * sub);
                }
                or_fake_a8(ein, dim);
            }
            matmul(&S->key, 0, dim, buf, rows, key, dim, 2);
            matmul(&S->value, 0, dim, buf, rows, stage + N3_ENGRAM_HISTORY * dim, stride * dim, 2);
            for (int rs = 0; rs < rows;) {
                int slot = row_slots[rs], rk = rs;
                while (rk + 1 < rows && row_slots[rk + 1] == slot) rk++;
                float* hist = e->engram_hist + ((size_t)site * e->slots + slot) * N3_ENGRAM_HISTORY * dim;
                memcpy(stage + (size_t)rs * stride * dim, hist, sizeof(float) * N3_ENGRAM_HISTORY * dim);
                for (int t = rs; t <= rk; t++) {
                    float* cur = stage + (size_t)t * stride * dim;
                    if (t > rs) memcpy(cur, cur - (size_t)stride * dim + dim, sizeof(float) * N3_ENGRAM_HISTORY * dim);
                    float* o = conv + (size_t)t * dim;
                    memset(o, 0, sizeof(float) * dim);
                    for (int j = 0; j < N3_ENGRAM_TAPS; j++) {
                        const float* a = S->taps + (size_t)j * dim;
                        const float* b = cur + (size_t)(N3_ENGRAM_HISTORY - j * g->engram_dilation) * dim;
                        for (int i = 0; i < dim; i++) o[i] += a[i] * b[i];
                    }
                }
                memcpy(hist, stage + ((size_t)rk * stride + 1) * dim, sizeof(float) * N3_ENGRAM_HISTORY * dim);
                rs = rk + 1;
            }
            float inverse_root = 1.0f / sqrtf((float)dim);
            for (int t = 0; t < rows; t++) {
                or_rms_unit(input + (size_t)t * dim, dim, unit_a);
                or_rms_unit(key + (size_t)t * dim, dim, unit_b);
                float alpha = or_sigmoid(or_dot(unit_a, unit_b, dim) * inverse_root);
                float* r = residual + (size_t)t * dim;
                const float* v = conv + (size_t)t * dim;
                for (int i = 0; i < dim; i++) r[i] += alpha * v[i];
            }
        }
        /* attention (RunAttentionBatch, Engine.cs:2480-2596) */
        for (int t = 0; t < rows; t++)
            or_centered_rms_fake_a8(residual + (size_t)t * dim, w->norm_in, dim, buf + (size_t)t * dim);
        matmul(&w->q, 0, qw, buf, rows, raw, all, 2);
        matmul(&w->k, 0, kw, buf, rows, raw + qw, all, 2);
        matmul(&w->v, 0, vw, buf, rows, raw + qw + kw, all, 2);
        matmul(&w->gate, 0, ow, buf, rows, gate, ow, 2);
        size_t lcell = (size_t)l * e->slots * e->capacity;
        or_needle3_attention_inputs(raw, rows, H, KV, qk, vd, w->q_taps, w->k_taps, w->v_taps, w->q_norm, w->k_norm,
                                    e->rope_cos, e->rope_sin, e->qkv_hist + (size_t)l * e->slots * 2 * all, row_slots,
                                    pos, e->slots, e->capacity, q8, qs, e->keys + lcell * kw,
                                    e->key_scales + lcell * KV, e->values + lcell * vw, e->value_scales + lcell * KV);
        int window = (g->global_mask >> l & 1) ? 0 : g->window;
        for (int t = 0; t < rows; t++) {
            first[t] = window == 0 ? 0 : (pos[t] - window + 1 > 0 ? pos[t] - window + 1 : 0);
            count[t] = pos[t] - first[t] + 1;
        }
#pragma omp parallel for num_threads(n3_threads) schedule(dynamic, 1)
        for (int t = 0; t < rows; t++)
            or_attention_decode(q8 + (size_t)t * qw, qs + (size_t)t * H, 1, H, KV, qk, e->keys + lcell * kw,
                                e->key_scales + lcell * KV, e->values + lcell * vw, e->value_scales + lcell * KV,
                                e->capacity, row_slots + t, first + t, count + t, e->max_chunks, att + (size_t)t * ow);
        for (int t = 0; t < rows; t++) or_gate_fake_a8(att + (size_t)t * ow, gate + (size_t)t * ow, ow);
        matmul(&w->out, 0, dim, att, rows, proj, dim, 2);
        const float* post_norm = plant == 5 ? w->pre_hada : w->post_norm;
        const float* pre_hada = plant == 5 ? w->post_norm : w->pre_hada;
        for (int t = 0; t < rows && plant == 3; t++)
            or_hadamard_mlp(&w->mlp, pre_hada, m->perm_a, m->perm_b, dim, g->hada_rows, g->hada_cols,
                            residual + (size_t)t * dim);
        for (int t = 0; t < rows; t++)
            or_post_norm_add(residual + (size_t)t * dim, proj + (size_t)t * dim, post_norm, w->attn_gate, dim);
        /* Kronecker-Hadamard MLP (RunMlp) */
#pragma omp parallel for num_threads(n3_threads) schedule(static)
        for (int t = 0; t < (plant != 3 ? rows : 0); t++)
            or_hadamard_mlp(&w->mlp, pre_hada, m->perm_a, m->perm_b, dim, g->hada_rows, g->hada_cols,
                            residual + (size_t)t * dim);
        /* the four lanes of the next stream */
        for (int t = 0; t < rows; t++)
            or_combine_diff4x4(stream + (size_t)t * sw, dim, mix + t * 16, residual + (size_t)t * dim,
                               input + (size_t)t * dim, post_gate + t * 4, next + (size_t)t * sw);
        float* swap = stream;
        stream = next;
        next = swap;
        if (e->trace) memcpy(e->trace + (size_t)(l + 1) * rows * sw, stream, sizeof(float) * (size_t)rows * sw);
    }
    /* the slots' lengths and previous tokens (ForwardBatch, Engine.cs:2326-2340) */
    for (int rs = 0; rs < rows;) {
        int slot = row_slots[rs], rk = rs;
        while (rk + 1 < rows && row_slots[rk + 1] == slot) rk++;
        int* pv = e->prev + 2 * slot;
        if (rk > rs) {
            pv[0] = tokens[rk - 1];
            pv[1] = tokens[rk];
        } else {
            pv[0] = pv[1];
            pv[1] = tokens[rk];
        }
        e->length[slot] += rk - rs + 1;
        rs = rk + 1;
    }
    /* the head rows: PrepareHeadVectors + the tied 4-bit embedding */
    for (int i = 0; i < heads; i++) {
        const float* s = stream + (size_t)head_rows[i] * sw;
        or_mix4(s, dim, 0.25f, 0.25f, 0.25f, 0.25f, unit_a);
        or_zero_centered_rms(unit_a, m->final_norm, dim, unit_b);
        or_fake_a8(unit_b, dim);
        matmul(&m->embedding, 0, g->vocab, unit_b, 1, logits + (size_t)i * g->vocab, g->vocab, 4);
    }
    free(stream); free(next); free(normed); free(input); free(residual); free(buf); free(raw); free(gate);
    free(att); free(proj); free(key); free(stage); free(conv); free(unit_a); free(unit_b); free(pre_out);
    free(post_out); free(res_out); free(post_gate); free(mix); free(q8); free(qs); free(pos); free(first);
    free(count); free(erows);
}

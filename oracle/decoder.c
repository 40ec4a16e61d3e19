/*
 * decoder.c -- CPU restatement of the synthetic int8 decoder's decode loop.
 *
 * TEST INFRASTRUCTURE ONLY: the CPU path that the GPU decoder's token streams
 * are checked against (and the timed CPU baseline of that loop).  The model
 * is the plain pre-norm decoder of the benchmark (the reference engine runs
 * Needle 3 / Whistle, not this geometry): embedding, per layer RMSNorm ->
 * fused QKV -> RoPE -> int8 KV cache -> ragged attention -> output
 * projection -> residual, RMSNorm -> gate/up -> SwiGLU -> down -> residual,
 * final RMSNorm -> LM head -> TopKLogSoftmax -> beam search.  Every linear is
 * the literal int8 matmul (or_matmul_rows_i8, Scalar.MatMulRows' order; or,
 * for the timed CPU path only, the SIMD tier of cpu_simd.c) on
 * activations quantized per row with QuantizeInt8 (Scalar.cs:67-74);
 * attention is or_attention_decode (AttentionBatch + MergePartials order);
 * the beam driver follows Whistle.BeamSearch (src/Needle/Whistle.Decode.cs:
 * 226-350).  The element-wise operations below have no counterpart in the
 * reference; their order (written out in each function) is the canonical
 * one that the GPU kernels reproduce operation for operation.
 */
#define _POSIX_C_SOURCE 199309L
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "needle_oracle.h"

static inline float u2f_(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u_(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* Natural logarithm for x > 0 (normal): x = m * 2^e with m in
 * [sqrt(1/2), sqrt(2)), log(m) = 2 atanh(s), s = (m-1)/(m+1), by the odd
 * series to s^9 (|s| <= 0.1716), e*ln2 with ln2 split as in Ops.Exp. */
float or_log_poly(float x)
{
    uint32_t u = f2u_(x);
    int e = (int)(u >> 23) - 127;
    float m = u2f_((u & 0x7FFFFFu) | 0x3F800000u);
    if (m > 1.41421356f) {
        m = m * 0.5f;
        e = e + 1;
    }
    float f = m - 1.0f;
    float s = f / (2.0f + f);
    float z = s * s;
    float p = 0.11111111f;
    p = fmaf(p, z, 0.14285715f);
    p = fmaf(p, z, 0.2f);
    p = fmaf(p, z, 0.33333334f);
    p = fmaf(p, z, 1.0f);
    float r = (2.0f * s) * p;
    float fe = (float)e;
    return fmaf(fe, 0.693359375f, fmaf(fe, -2.12194440e-4f, r));
}

/* The canonical 256-way reduction of a row's terms: partial p[t] (t < 256)
 * adds the terms of the elements i with (i / 4) % 256 == t in ascending i
 * from +0 (CANON_LANE); q[m] (m < 16) = p[16m] + p[16m+1] + ... + p[16m+15]
 * left to right; the total is q folded with strides 8, 4, 2, 1
 * (q[m] = q[m] + q[m + stride]).  On the GPU lane t of a 256-thread block
 * holds p[t], and the last two levels run in one 16-lane DPP row. */
#define CANON_LANE(i) (((i) >> 2) & 255)

static float tree_fold(const float* p)
{
    float q[16];
    for (int m = 0; m < 16; m++) {
        q[m] = p[16 * m];
        for (int k = 1; k < 16; k++) q[m] = q[m] + p[16 * m + k];
    }
    for (int stride = 8; stride > 0; stride >>= 1)
        for (int m = 0; m < stride; m++) q[m] = q[m] + q[m + stride];
    return q[0];
}

/* x += delta (if given); h = (x * inv) * gain with inv = 1 / sqrt(ss / d +
 * eps), ss = sum x^2 by the canonical reduction; q, scale = QuantizeInt8(h). */
float or_add_rmsnorm_quant(float* x, const float* delta, const float* gain, int d, float eps, float* h,
                           int8_t* q)
{
    float s[256];
    for (int t = 0; t < 256; t++) s[t] = 0.0f;
    if (delta)
        for (int i = 0; i < d; i++) x[i] = x[i] + delta[i];
    for (int i = 0; i < d; i++) s[CANON_LANE(i)] = s[CANON_LANE(i)] + x[i] * x[i];
    float ss = tree_fold(s);
    float inv = 1.0f / sqrtf(ss / (float)d + eps);
    for (int i = 0; i < d; i++) h[i] = (x[i] * inv) * gain[i];
    return or_quantize_int8(h, d, q);
}

/* cos/sin of position p times theta^(-2i/dim), i < dim/2, rounded from
 * double to float. */
void or_rope_table(int positions, int dim, double theta, float* cos_t, float* sin_t)
{
    int half = dim / 2;
    for (int p = 0; p < positions; p++)
        for (int i = 0; i < half; i++) {
            double angle = (double)p * pow(theta, -2.0 * i / dim);
            cos_t[(long)p * half + i] = (float)cos(angle);
            sin_t[(long)p * half + i] = (float)sin(angle);
        }
}

/* Rotate-half RoPE of one 64-element head: (x_i, x_{i+32}) -> (x_i c - x_{i+32}
 * s, x_{i+32} c + x_i s). */
void or_rope_head(float* v, const float* c, const float* s)
{
    for (int i = 0; i < 32; i++) {
        float x0 = v[i], x1 = v[i + 32];
        v[i] = x0 * c[i] - x1 * s[i];
        v[i + 32] = x1 * c[i] + x0 * s[i];
    }
}

/* a = silu(g) * u with silu(g) = g / (1 + Exp(-g)), then QuantizeInt8. */
float or_swiglu_quant(const float* g, const float* u, int n, float* a, int8_t* q)
{
    for (int i = 0; i < n; i++) a[i] = (g[i] / (1.0f + or_exp_poly(-g[i]))) * u[i];
    return or_quantize_int8(a, n, q);
}

/* TopKLogSoftmax (src/Needle/Ops.cs:1092-1221) in the canonical float form:
 * the reference's own selection (or_topk_select: the top k of the allowed
 * ids by value, ties to the lower id, one -inf id at most, (-inf, -1) for
 * slots left over); log_shift = peak + log(S) with peak the top value
 * and S summed over blocks of OR_TOPK_BLOCK ids: for block b with masked
 * values v_i = -1e30 and block maximum m_b, S_b = sum_i Exp(v_i - m_b) by
 * the canonical reduction over the block's ids (relative to its start),
 * and S = sum_b Exp(m_b - peak) * S_b in ascending b.  The blocks let the
 * GPU reduce one block per workgroup. */
#define OR_TOPK_BLOCK 2048

void or_topk_lse(const float* x, int n, int k, int mask, int* idx, float* lp)
{
    float top_val[16];
    int top_idx[16];
    or_topk_select(x, n, k, mask, top_idx, top_val);
    float peak = top_val[0];
    float total = 0.0f;
    for (int b0 = 0; b0 < n; b0 += OR_TOPK_BLOCK) {
        int b1 = b0 + OR_TOPK_BLOCK < n ? b0 + OR_TOPK_BLOCK : n;
        float mb = -INFINITY;
        for (int i = b0; i < b1; i++) {
            float v = mask && (i == 0 || i == 2 || i == 3) ? -1e30f : x[i];
            mb = fmaxf(mb, v);
        }
        float s[256];
        for (int t = 0; t < 256; t++) s[t] = 0.0f;
        for (int i = b0; i < b1; i++) {
            float v = mask && (i == 0 || i == 2 || i == 3) ? -1e30f : x[i];
            s[CANON_LANE(i - b0)] = s[CANON_LANE(i - b0)] + or_exp_poly(v - mb);
        }
        total = total + or_exp_poly(mb - peak) * tree_fold(s);
    }
    float log_shift = peak + or_log_poly(total);
    for (int m = 0; m < k; m++) {
        idx[m] = top_idx[m];
        lp[m] = top_val[m] - log_shift;
    }
}

/* ------------------------------------------------------------ model -- */

static void linear(const or_decoder* m, const int8_t* w, const uint16_t* s, int rows, int cols, const int8_t* q,
                   const float* qs, int tokens, float* y)
{
    if (m->simd != OR_TIER_SCALAR)
        or_baseline_simd_matmul_i8(m->simd, w, s, rows, cols, q, qs, tokens, y, rows, 0, rows);
    else if (m->threads > 1)
        or_baseline_matmul_i8(w, s, rows, cols, 32, q, qs, tokens, y, rows, 0, rows);
    else
        or_matmul_rows_i8(w, s, rows, cols, 32, q, qs, tokens, y, rows, 0, rows);
}

int or_decoder_init(or_decoder* m)
{
    const or_decoder_dims* D = &m->dims;
    int half = D->head_dim / 2;
    size_t cells = (size_t)D->layers * D->slots * D->capacity * D->kv_heads;
    m->rope_cos = (float*)malloc(sizeof(float) * (size_t)D->capacity * half);
    m->rope_sin = (float*)malloc(sizeof(float) * (size_t)D->capacity * half);
    m->keys = (int8_t*)calloc(cells * D->head_dim, 1);
    m->values = (int8_t*)calloc(cells * D->head_dim, 1);
    m->key_scales = (float*)calloc(cells, sizeof(float));
    m->value_scales = (float*)calloc(cells, sizeof(float));
    if (!m->rope_cos || !m->rope_sin || !m->keys || !m->values || !m->key_scales || !m->value_scales) return -1;
    or_rope_table(D->capacity, D->head_dim, D->theta, m->rope_cos, m->rope_sin);
    if (m->threads > 1) m->threads = or_baseline_start(m->threads);
    return 0;
}

void or_decoder_free(or_decoder* m)
{
    free(m->rope_cos);
    free(m->rope_sin);
    free(m->keys);
    free(m->values);
    free(m->key_scales);
    free(m->value_scales);
    m->rope_cos = m->rope_sin = m->key_scales = m->value_scales = NULL;
    m->keys = m->values = NULL;
    if (m->threads > 1) or_baseline_stop();
}

/* Cache region of (layer, slot): [capacity][kv_heads*head_dim] / [capacity][kv_heads]. */
static size_t region(const or_decoder_dims* D, int layer, int slot)
{
    return ((size_t)layer * D->slots + slot) * D->capacity;
}

void or_decoder_forward(or_decoder* m, const int* tokens, const int* slots, const int* positions, int rows,
                        float* logits, int k, int* topk_idx, float* topk_lp)
{
    const or_decoder_dims* D = &m->dims;
    int d = D->d, H = D->heads, KV = D->kv_heads, hd = D->head_dim, F = D->ffn, half = hd / 2;
    int qkv_n = (H + 2 * KV) * hd;
    float* x = (float*)malloc(sizeof(float) * (size_t)rows * d);
    float* h = (float*)malloc(sizeof(float) * (size_t)(d > F ? d : F));
    int qw = F > d ? F : d;
    if (H * hd > qw) qw = H * hd;
    int8_t* q8 = (int8_t*)malloc((size_t)rows * qw);
    float* qs = (float*)malloc(sizeof(float) * rows);
    float* qkv = (float*)malloc(sizeof(float) * (size_t)rows * qkv_n);
    int8_t* qh = (int8_t*)malloc((size_t)rows * H * hd);
    float* qhs = (float*)malloc(sizeof(float) * (size_t)rows * H);
    float* att = (float*)malloc(sizeof(float) * (size_t)rows * H * hd);
    float* delta = (float*)malloc(sizeof(float) * (size_t)rows * d);
    float* gu = (float*)malloc(sizeof(float) * (size_t)rows * 2 * F);
    float* lg = logits ? logits : (float*)malloc(sizeof(float) * (size_t)rows * D->vocab);
    int* first = (int*)calloc(rows, sizeof(int));
    int* count = (int*)malloc(sizeof(int) * rows);
    for (int r = 0; r < rows; r++) {
        memcpy(x + (size_t)r * d, m->embedding + (size_t)tokens[r] * d, sizeof(float) * d);
        count[r] = positions[r] + 1;
    }
    for (int l = 0; l < D->layers; l++) {
        const or_layer_weights* W = &m->layers[l];
        for (int r = 0; r < rows; r++)
            qs[r] = or_add_rmsnorm_quant(x + (size_t)r * d, l == 0 ? NULL : delta + (size_t)r * d, W->attn_norm, d,
                                         D->eps, h, q8 + (size_t)r * d);
        linear(m, W->wqkv, W->sqkv, qkv_n, d, q8, qs, rows, qkv);
        for (int r = 0; r < rows; r++) {
            float* v = qkv + (size_t)r * qkv_n;
            const float* c = m->rope_cos + (size_t)positions[r] * half;
            const float* s = m->rope_sin + (size_t)positions[r] * half;
            for (int hh = 0; hh < H; hh++) {
                or_rope_head(v + hh * hd, c, s);
                qhs[(size_t)r * H + hh] = or_quantize_int8(v + hh * hd, hd, qh + ((size_t)r * H + hh) * hd);
            }
            size_t cell = region(D, l, slots[r]) + positions[r];
            for (int kv = 0; kv < KV; kv++) {
                float* kp = v + (size_t)(H + kv) * hd;
                float* vp = v + (size_t)(H + KV + kv) * hd;
                or_rope_head(kp, c, s);
                m->key_scales[cell * KV + kv] = or_quantize_int8(kp, hd, m->keys + (cell * KV + kv) * hd);
                m->value_scales[cell * KV + kv] = or_quantize_int8(vp, hd, m->values + (cell * KV + kv) * hd);
            }
        }
        size_t base = region(D, l, 0);
        int* slot_rel = (int*)malloc(sizeof(int) * rows);
        for (int r = 0; r < rows; r++) slot_rel[r] = slots[r];
        or_attention_decode(qh, qhs, rows, H, KV, hd, m->keys + base * KV * hd, m->key_scales + base * KV,
                            m->values + base * KV * hd, m->value_scales + base * KV, D->capacity, slot_rel, first,
                            count, D->max_chunks, att);
        free(slot_rel);
        for (int r = 0; r < rows; r++)
            qs[r] = or_quantize_int8(att + (size_t)r * H * hd, H * hd, q8 + (size_t)r * H * hd);
        linear(m, W->wo, W->so, d, H * hd, q8, qs, rows, delta);
        for (int r = 0; r < rows; r++)
            qs[r] = or_add_rmsnorm_quant(x + (size_t)r * d, delta + (size_t)r * d, W->ffn_norm, d, D->eps, h,
                                         q8 + (size_t)r * d);
        linear(m, W->wgu, W->sgu, 2 * F, d, q8, qs, rows, gu);
        for (int r = 0; r < rows; r++) {
            const float* g = gu + (size_t)r * 2 * F;
            qs[r] = or_swiglu_quant(g, g + F, F, h, q8 + (size_t)r * F);
        }
        linear(m, W->wd, W->sd, d, F, q8, qs, rows, delta);
    }
    for (int r = 0; r < rows; r++)
        qs[r] = or_add_rmsnorm_quant(x + (size_t)r * d, delta + (size_t)r * d, m->final_norm, d, D->eps, h,
                                     q8 + (size_t)r * d);
    linear(m, m->wlm, m->slm, D->vocab, d, q8, qs, rows, lg);
    if (k > 0)
        for (int r = 0; r < rows; r++)
            or_topk_lse(lg + (size_t)r * D->vocab, D->vocab, k, 1, topk_idx + (size_t)r * k, topk_lp + (size_t)r * k);
    free(x); free(h); free(q8); free(qs); free(qkv); free(qh); free(qhs); free(att); free(delta); free(gu);
    free(first); free(count);
    if (!logits) free(lg);
}

void or_decoder_copy_slot(or_decoder* m, int dst, int src, int length)
{
    const or_decoder_dims* D = &m->dims;
    for (int l = 0; l < D->layers; l++) {
        size_t a = region(D, l, dst) * D->kv_heads, b = region(D, l, src) * D->kv_heads;
        size_t n = (size_t)length * D->kv_heads;
        memmove(m->keys + a * D->head_dim, m->keys + b * D->head_dim, n * D->head_dim);
        memmove(m->values + a * D->head_dim, m->values + b * D->head_dim, n * D->head_dim);
        memmove(m->key_scales + a, m->key_scales + b, n * sizeof(float));
        memmove(m->value_scales + a, m->value_scales + b, n * sizeof(float));
    }
}

/* ------------------------------------------------------------ greedy -- */

static double now_s(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}


int or_greedy(or_decoder* m, const int* prompt, int prompt_len, int max_new, int stop, int* out_tokens,
              double* seconds)
{
    double t0 = now_s();
    int V = m->dims.vocab;
    float* lg = (float*)malloc(sizeof(float) * (size_t)prompt_len * V);
    int* pos = (int*)malloc(sizeof(int) * prompt_len);
    int* sl = (int*)calloc(prompt_len, sizeof(int));
    for (int i = 0; i < prompt_len; i++) pos[i] = i;
    or_decoder_forward(m, prompt, sl, pos, prompt_len, lg, 0, NULL, NULL);
    double t1 = now_s();
    const float* last = lg + (size_t)(prompt_len - 1) * V;
    int n = 0;
    for (int step = 0; step < max_new; step++) {
        int next = or_argmax(last, V);
        if (next == stop) break;
        out_tokens[n++] = next;
        int slot = 0, p = prompt_len + step;
        or_decoder_forward(m, &next, &slot, &p, 1, lg, 0, NULL, NULL);
        last = lg;
    }
    double t2 = now_s();
    if (seconds) {
        seconds[0] = t1 - t0;
        seconds[1] = t2 - t1;
    }
    free(lg); free(pos); free(sl);
    return n;
}

/* ------------------------------------------------------- beam search -- */

typedef struct { float score; int parent, token; } cand_t;

/* Whistle.BeamSearch (src/Needle/Whistle.Decode.cs:226-350) for one prompt
 * on this decoder, length penalty 1, no keyword bias: slot of beam j is
 * tracked instead of engines (the last child of a parent keeps the parent's
 * slot, the others get a copy -- Engine.CopyFrom); candidates are sorted by
 * score with ties in insertion order (a stable sort; List.Sort leaves ties
 * unspecified).  Returns the winner's length; tokens[], score, and the
 * number of forward rows fed after the prompt (for tokens/s). */

int or_beam_search(or_decoder* m, const int* prompt, int prompt_len, int width, int max_new, int eos,
                   int* out_tokens, float* out_score, long* fed_rows, double* seconds)
{
    double t0 = now_s();
    int W = width, V = m->dims.vocab;
    int slots_live[16], slots_next[16];
    int* live_tok = (int*)malloc(sizeof(int) * W * (max_new + 1));
    int* next_tok = (int*)malloc(sizeof(int) * W * (max_new + 1));
    int live_len[16], next_len[16];
    float live_score[16];
    int* fin_tok = (int*)malloc(sizeof(int) * (size_t)(W * max_new + W) * (max_new + 1));
    int fin_len[1024];
    float fin_score[1024];
    int fin_count = 0;
    int topk_idx[16 * 16];
    float topk_lp[16 * 16];
    cand_t cand[256];
    int* pos = (int*)malloc(sizeof(int) * (prompt_len > W ? prompt_len : W));
    int* sl = (int*)malloc(sizeof(int) * (prompt_len > W ? prompt_len : W));
    int feed_tok[16], feed_slot[16], feed_pos[16];
    (void)V;
    /* prefill the prompt into slot 0; the logits of its last token start the search */
    for (int i = 0; i < prompt_len; i++) { pos[i] = i; sl[i] = 0; }
    {
        float* lg = (float*)malloc(sizeof(float) * (size_t)prompt_len * m->dims.vocab);
        or_decoder_forward(m, prompt, sl, pos, prompt_len, lg, 0, NULL, NULL);
        or_topk_lse(lg + (size_t)(prompt_len - 1) * m->dims.vocab, m->dims.vocab, W, 1, topk_idx, topk_lp);
        free(lg);
    }
    double t1 = now_s();
    int live_count = 1;
    slots_live[0] = 0;
    live_len[0] = 0;
    live_score[0] = 0.0f;
    long fed = 0;
    for (int step = 0; step < max_new; step++) {
        int nc = 0;
        for (int i = 0; i < live_count; i++)
            for (int kk = 0; kk < W; kk++) {
                cand[nc].score = live_score[i] + topk_lp[i * W + kk];
                cand[nc].parent = i;
                cand[nc].token = topk_idx[i * W + kk];
                nc++;
            }
        /* stable sort by score, descending */
        for (int a = 1; a < nc; a++) {
            cand_t c = cand[a];
            int b = a - 1;
            while (b >= 0 && cand[b].score < c.score) { cand[b + 1] = cand[b]; b--; }
            cand[b + 1] = c;
        }
        int kept = 0, parents[16], picks[16];
        float pick_scores[16];
        for (int a = 0; a < nc; a++) {
            cand_t c = cand[a];
            if (c.token == eos) {
                memcpy(fin_tok + (size_t)fin_count * (max_new + 1), live_tok + (size_t)c.parent * (max_new + 1),
                       sizeof(int) * live_len[c.parent]);
                fin_len[fin_count] = live_len[c.parent];
                fin_score[fin_count] = c.score;
                fin_count++;
            } else {
                parents[kept] = c.parent;
                picks[kept] = c.token;
                pick_scores[kept] = c.score;
                kept++;
            }
            if (kept >= W) break;
        }
        if (kept == 0) break;
        if (fin_count >= W) {
            float best_fin = -INFINITY, best_live = -INFINITY;
            for (int f = 0; f < fin_count; f++) {
                float sc = fin_score[f] / (float)(fin_len[f] + 1);
                best_fin = best_fin > sc ? best_fin : sc;
            }
            for (int j = 0; j < kept; j++) {
                float sc = pick_scores[j] / (float)(live_len[parents[j]] + 1);
                best_live = best_live > sc ? best_live : sc;
            }
            if (best_fin >= best_live) break;
        }
        int last_child[16];
        for (int p = 0; p < live_count; p++) last_child[p] = -1;
        for (int j = 0; j < kept; j++) last_child[parents[j]] = j;
        /* slots: a last child keeps its parent's slot, the others take a
         * free slot holding a copy of the parent's cache */
        int used[64] = {0};
        for (int j = 0; j < kept; j++)
            if (j == last_child[parents[j]]) used[slots_live[parents[j]]] = 1;
        for (int j = 0; j < kept; j++) {
            int p = parents[j];
            if (j == last_child[p]) {
                slots_next[j] = slots_live[p];
            } else {
                int f = 0;
                while (used[f]) f++;
                used[f] = 1;
                or_decoder_copy_slot(m, f, slots_live[p], prompt_len + live_len[p]);
                slots_next[j] = f;
            }
            memcpy(next_tok + (size_t)j * (max_new + 1), live_tok + (size_t)p * (max_new + 1), sizeof(int) * live_len[p]);
            next_tok[(size_t)j * (max_new + 1) + live_len[p]] = picks[j];
            next_len[j] = live_len[p] + 1;
            feed_tok[j] = picks[j];
            feed_slot[j] = slots_next[j];
            feed_pos[j] = prompt_len + live_len[p];
        }
        or_decoder_forward(m, feed_tok, feed_slot, feed_pos, kept, NULL, W, topk_idx, topk_lp);
        fed += kept;
        for (int j = 0; j < kept; j++) {
            slots_live[j] = slots_next[j];
            live_len[j] = next_len[j];
            live_score[j] = pick_scores[j];
        }
        int* t = live_tok; live_tok = next_tok; next_tok = t;
        live_count = kept;
    }
    double t2 = now_s();
    if (seconds) {
        seconds[0] = t1 - t0;
        seconds[1] = t2 - t1;
    }
    int winner_len = 0;
    float winner_score = -INFINITY;
    const int* winner = NULL;
    for (int f = 0; f < fin_count; f++) {
        float sc = fin_score[f] / (float)(fin_len[f] + 1);
        if (sc > winner_score) { winner_score = sc; winner = fin_tok + (size_t)f * (max_new + 1); winner_len = fin_len[f]; }
    }
    if (!winner)
        for (int j = 0; j < live_count; j++) {
            float sc = live_score[j] / (float)live_len[j];
            if (sc > winner_score) { winner_score = sc; winner = live_tok + (size_t)j * (max_new + 1); winner_len = live_len[j]; }
        }
    if (winner) memcpy(out_tokens, winner, sizeof(int) * winner_len);
    *out_score = winner_score;
    if (fed_rows) *fed_rows = fed;
    free(live_tok); free(next_tok); free(fin_tok); free(pos); free(sl);
    return winner_len;
}

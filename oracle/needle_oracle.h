/*
 * needle_oracle.h -- CPU restatement of the needle-cs quantized decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  Nothing in the product (needle_cs_amd/, include/) links or
 * calls it.
 *
 * Every function restates one reference function; the citation is given at
 * the declaration.  Paths are relative to the reference repository root
 * (IAFahim/needle-cs).  Where the reference has no counterpart (the literal
 * int8/group-32 weight format, head dimension 64, the plain decoder used for
 * the full decode loop), the function says so and names the reference
 * function it generalises.
 *
 * Arithmetic rules: float is IEEE binary32, no contraction (built with
 * -ffp-contract=off); explicit fmaf() only where the reference uses an FMA
 * (Fma.MultiplyAdd / MultiplyAddNegated).
 */
#ifndef NEEDLE_ORACLE_H
#define NEEDLE_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- reference struct layouts (C# sequential layout == C natural layout) ---- */

/* src/Needle/Model.cs:36-42 */
typedef struct or_codebook {
    float levels[16];
    uint8_t bytes[32];
    float byte_scale;
} or_codebook;

/* src/Needle/Model.cs:8-34; GroupSize 128 (Model.cs:10) */
typedef struct or_cq {
    const uint8_t* indices;
    const uint16_t* norms;
    const or_codebook* book;
    int rows, cols, bits;
} or_cq;

/* src/Needle/Quant.cs:11-28 */
typedef struct or_activations {
    int8_t* values;
    float* scales;
    float* offsets;
    int cols, groups, stride;
} or_activations;

/* src/Needle/Blocks.cs:11-27 */
typedef struct or_attention_tile {
    const int8_t* queries;
    const float* query_scales;
    int heads;
    const int8_t* keys;
    const float* key_scales;
    const int8_t* values;
    const float* value_scales;
    int key_stride, value_stride, scale_stride, first, count;
    float* scores;
    float* output;
    float* probabilities;
    int probability_stride;
    float* peaks;
    float* sums;
} or_attention_tile;

/* ---- generators ---- */

/* tests/Needle.Tests/Conformance/Conformance.cs:10-38 (XorShift64) */
uint64_t or_xs_seed(uint64_t seed);
uint64_t or_xs_next(uint64_t* state);
int or_xs_next_int(uint64_t* state, int lo, int hi);
float or_xs_next_float(uint64_t* state, float scale);
/* tests/Needle.Tests/Conformance/Conformance.cs:42-68 */
void or_fill_uniform(float* x, int n, uint64_t* state, float scale);
void or_fill_edges(float* x, int n, uint64_t* state, float scale);
/* tests/Needle.Tests/Conformance/Conformance.cs:70-101 */
void or_fill_sbyte(int8_t* x, int n, uint64_t* state, int extremes);
void or_fill_bytes(uint8_t* x, int n, uint64_t* state, int extremes);
/* tests/Needle.Tests/Conformance/Conformance.cs:103-118 */
uint16_t or_half_bits(float value);

/* Synthetic workload distributions (no reference counterpart; the workload
 * definition of the decode benchmarks): one XorShift64 stream, 53-bit
 * uniforms u = (next >> 11) * 2^-53, N(0,1) by Box-Muller on (1-u1, u2),
 * U(a,b) = a + (b-a)*u, int8 U[-127,127] = NextInt(-127,128), fp16 by RNE. */
double or_synth_u53(uint64_t* state);
void or_synth_normal(float* x, size_t n, uint64_t* state);
void or_synth_uniform(float* x, size_t n, uint64_t* state, float lo, float hi);
void or_synth_int8(int8_t* x, size_t n, uint64_t* state);
void or_synth_half_uniform(uint16_t* x, size_t n, uint64_t* state, float lo, float hi);
uint16_t or_single_to_half_rne(float f);

/* ---- scalar kernels ---- */

/* src/Needle/Scalar.cs:121-128 */
float or_half_to_single(uint16_t half);
/* src/Needle/Scalar.cs:113-119 */
float or_half_to_single_upstream(uint16_t half);
/* src/Needle/Model.cs:44-52 */
void or_codebook_fill(or_codebook* book, const float* levels, int count);
/* src/Needle/Scalar.cs:76-89 (128-element Walsh-Hadamard) */
void or_hadamard(const float* source, float* p);
/* src/Needle/Scalar.cs:55-60 */
float or_abs_max(const float* x, int n);
/* src/Needle/Scalar.cs:62-65 */
void or_round_trip(float* x, int n, float inverse, float scale);
/* src/Needle/Scalar.cs:67-74 */
float or_quantize_int8(const float* x, int n, int8_t* destination);
/* src/Needle/Scalar.cs:91-111 */
void or_planes(const int8_t* quantized, int bits, int8_t* destination, int* sum);
/* src/Needle/Quant.cs:473-488 (scalar branch of PrepareRange) */
void or_prepare(const float* x, int tokens, int cols, int bits, const or_activations* a);
/* src/Needle/Scalar.cs:130-144 */
void or_decode_row(const or_cq* w, int row, float* destination);
/* src/Needle/Scalar.cs:146-192 */
void or_matmul_rows(const or_cq* w, const or_activations* a, int tokens, float* y, int ldy,
                    int row_start, int row_end);
/* Int32 group sums D[t][n][g] of Scalar.cs:162-184 (the accumulators the
 * parity bar requires bit-exact), for rows [row_start,row_end). */
void or_group_dots_cq(const or_cq* w, const or_activations* a, int tokens, int row_start,
                      int row_end, int32_t* dots);

/* Literal int8 format: int8 weights [rows][cols], one fp16 scale per
 * `group` elements [rows][cols/group], activations quantized per row by
 * or_quantize_int8 (one scale per token).  No reference counterpart: this is
 * Scalar.MatMulRows (Scalar.cs:146-192) with the codebook replaced by the
 * identity (Bytes[i] = i, ByteScale = 1), Cq.GroupSize = `group`, every
 * group's activation scale equal to the row scale and zero offsets.  The
 * epilogue keeps Scalar.cs:185-189's exact order. */
void or_matmul_rows_i8(const int8_t* w, const uint16_t* scales, int rows, int cols, int group,
                       const int8_t* q, const float* qscale, int tokens, float* y, int ldy,
                       int row_start, int row_end);
void or_group_dots_i8(const int8_t* w, int rows, int cols, int group, const int8_t* q,
                      int tokens, int row_start, int row_end, int32_t* dots);
/* Per-row activation quantization of the literal path: or_quantize_int8 over
 * each of `tokens` rows of `cols` floats. */
void or_quantize_rows(const float* x, int tokens, int cols, int8_t* q, float* scales);

/* ---- softmax / exp / attention ---- */

/* src/Needle/Ops.cs:16-31, one lane of the AVX polynomial exp. */
float or_exp_poly(float x);
/* src/Needle/Scalar.cs:220-231; use_poly selects or_exp_poly instead of
 * libm expf (MathF.Exp). */
void or_softmax(float* s, int n, int use_poly);
/* src/Needle/Scalar.cs:290-312, generalised to qk_dim in {48, 64} and
 * v_dim 64 (the reference hard-codes 48; Blocks.cs:45-46).  The score scale
 * is 1/sqrt(qk_dim) rounded to float (0.14433756729740643f for 48, as
 * Scalar.cs:50). */
void or_attention_head(const int8_t* query, float query_scale, const int8_t* keys,
                       const float* key_scales, const int8_t* values, const float* value_scales,
                       int key_stride, int value_stride, int scale_stride, int first, int last,
                       float* scores, float* output, float* probabilities, int qk_dim,
                       int use_poly);
/* One head's position-split partial: the un-normalised output
 * sum_s (e_s * valueScale_s) * v_s with e_s = exp(score_s - peak), plus the
 * peak and sum_s e_s (src/Needle/Blocks.cs:188-199 with Peaks set and
 * ValuesFloat, Blocks.cs:415-435, restated with scalar operations). */
void or_attention_partial(const int8_t* query, float query_scale, const int8_t* keys,
                          const float* key_scales, const int8_t* values, const float* value_scales,
                          int key_stride, int value_stride, int scale_stride, int first, int count,
                          int qk_dim, int use_poly, float* output, float* peak, float* sum);
/* src/Needle/Scalar.cs:314-321 */
void or_attention_tile_run(const or_attention_tile* tile, int use_poly);
/* src/Needle/Blocks.cs:750-817, the non-SIMD branch (count == 2 special
 * case included).  Partial layout: PartialFloats = 6*64+16 floats per chunk,
 * out [6][64], peaks at +384, sums at +392 (Blocks.cs:42-43,956-957). */
void or_merge_partials(const float* partials, int count, int heads, float* output,
                       int use_poly);
/* tests/Needle.Tests/Conformance/KernelConformanceTests.cs:498-525 (double
 * reference). */
void or_merge_partials_double(const float* partials, int count, int heads, float* output);
/* src/Needle/Blocks.cs:973-978 */
void or_attention_span(int position, int window, int frames, int* first, int* count);

/* Position-split plan of AttentionBatch.ExecuteChunk (Blocks.cs:934-938)
 * with the chunk cap as a parameter (the reference's MaxChunks is 8,
 * MinChunkPositions 16, Blocks.cs:832-833): returns the chunk count, sets
 * the chunk length (a multiple of 4). */
int or_attention_plan(int count, int max_chunks, int* length);
/* One head's merge of `count` partials in the order of
 * Attention.MergePartials' non-SIMD branch (Blocks.cs:760-815), any count:
 * outs [count][out_stride] (64 used), peaks/sums [count] at their strides. */
void or_merge_head(const float* outs, int out_stride, const float* peaks, const float* sums,
                   int stride, int count, float* output, int use_poly);
/* Ragged decode attention over a pooled int8 KV cache:
 *   keys   int8 [slots][capacity][kv_heads*qk_dim], key_scales   [slots][capacity][kv_heads]
 *   values int8 [slots][capacity][kv_heads*64],     value_scales [slots][capacity][kv_heads]
 *   q int8 [rows][heads][qk_dim], q_scales [rows][heads], out [rows][heads][64].
 * Row r attends positions row_first[r] .. +row_count[r]-1 of slot
 * row_slot[r]; query head h reads kv head h / (heads/kv_heads).  Each
 * (row, head) is split by or_attention_plan, every chunk is
 * or_attention_partial with the polynomial exp, and the chunks are merged by
 * or_merge_head -- AttentionBatch.ExecuteChunk + MergePartials
 * (Blocks.cs:927-966) for every row of a ragged batch. */
void or_attention_decode(const int8_t* q, const float* q_scales, int rows, int heads, int kv_heads,
                         int qk_dim, const int8_t* keys, const float* key_scales,
                         const int8_t* values, const float* value_scales, int capacity,
                         const int* row_slot, const int* row_first, const int* row_count,
                         int max_chunks, float* out);

/* src/Needle/Ops.cs:1086-1089 (first index of the maximum) */
int or_argmax(const float* x, int n);
/* src/Needle/Ops.cs:1094-1166: the ids and values TopKLogSoftmax selects
 * (slots left over: (-inf, -1)) */
void or_topk_select(const float* x, int n, int k, int mask_special_023, int* top_idx, float* top_val);
/* src/Needle/Ops.cs:1092-1221, scalar branch (the double log-sum-exp) */
void or_topk_log_softmax(const float* x, int n, int k, int* indices, float* log_probs,
                         float* probs, int mask_special_023);

/* ---- threaded CPU baseline (cpu_baseline.c) ---- */

int or_baseline_start(int members);
void or_baseline_stop(void);
/* or_matmul_rows_i8 split over the pool's members (bit-identical results). */
void or_baseline_matmul_i8(const int8_t* w, const uint16_t* scales, int rows, int cols, int group,
                           const int8_t* q, const float* qscale, int tokens, float* y, int ldy,
                           int row_start, int row_end);

/* ---- SIMD tier of the CPU matmul (cpu_simd.c): the timed baseline ---- */

enum { OR_TIER_SCALAR = 0, OR_TIER_AVX2 = 1, OR_TIER_AVX_VNNI = 2 };
/* Tiers.Best on this CPU (src/Needle/Tiers.cs:127-138): AVX-VNNI, else
 * AVX2 + FMA (+ F16C), else scalar. */
int or_simd_tier(void);
/* Quant.MatMulRows' SIMD branch (Quant.cs:627-632, Gemv.cs Tile4 / Tile2 /
 * Rows) for the literal int8 format (group 32): exact int32 group sums, the
 * SIMD tier's float association. */
void or_simd_matmul_i8(int tier, const int8_t* w, const uint16_t* scales, int rows, int cols, const int8_t* q,
                       const float* qscale, int tokens, float* y, int ldy, int row_start, int row_end);
/* or_simd_matmul_i8 split over the pool's members (4-row blocks). */
void or_baseline_simd_matmul_i8(int tier, const int8_t* w, const uint16_t* scales, int rows, int cols,
                                const int8_t* q, const float* qscale, int tokens, float* y, int ldy,
                                int row_start, int row_end);

/* ---- synthetic int8 decoder (decoder.c) ---- */

/* Canonical element-wise operations of the decoder (no reference
 * counterpart; the GPU kernels repeat them operation for operation). */
float or_log_poly(float x);
float or_add_rmsnorm_quant(float* x, const float* delta, const float* gain, int d, float eps, float* h,
                           int8_t* q);
void or_rope_table(int positions, int dim, double theta, float* cos_t, float* sin_t);
void or_rope_head(float* v, const float* c, const float* s);
float or_swiglu_quant(const float* g, const float* u, int n, float* a, int8_t* q);
void or_topk_lse(const float* x, int n, int k, int mask, int* idx, float* lp);

typedef struct or_decoder_dims {
    int layers, d, heads, kv_heads, head_dim, ffn, vocab, capacity, slots, max_chunks;
    double theta;
    float eps;
} or_decoder_dims;

/* int8 weights [rows][cols] with fp16 group-32 scales [rows][cols/32]:
 * wqkv [(heads+2*kv_heads)*head_dim][d], wo [d][heads*head_dim],
 * wgu [2*ffn][d] (gate rows, then up rows), wd [d][ffn]. */
typedef struct or_layer_weights {
    const int8_t* wqkv;
    const uint16_t* sqkv;
    const int8_t* wo;
    const uint16_t* so;
    const int8_t* wgu;
    const uint16_t* sgu;
    const int8_t* wd;
    const uint16_t* sd;
    const float* attn_norm;
    const float* ffn_norm;
} or_layer_weights;

typedef struct or_decoder {
    or_decoder_dims dims;
    const or_layer_weights* layers;
    const float* embedding;  /* [vocab][d] */
    const float* final_norm; /* [d] */
    const int8_t* wlm;       /* [vocab][d] */
    const uint16_t* slm;
    int threads;             /* > 1: linears on the baseline pool */
    int simd;                /* OR_TIER_*: linears in the SIMD tier (the timed CPU path), 0: the scalar order */
    float* rope_cos;         /* owned: [capacity][head_dim/2] */
    float* rope_sin;
    int8_t* keys;            /* owned: [layer][slot][capacity][kv_heads*head_dim] */
    int8_t* values;
    float* key_scales;       /* owned: [layer][slot][capacity][kv_heads] */
    float* value_scales;
} or_decoder;

int or_decoder_init(or_decoder* m);
void or_decoder_free(or_decoder* m);
/* One forward over `rows` rows (token, slot, position each): writes every
 * layer's K/V at the row's position, fills logits [rows][vocab] if given
 * and the top-k (masked ids 0,2,3) ids/log-probabilities if k > 0. */
void or_decoder_forward(or_decoder* m, const int* tokens, const int* slots, const int* positions, int rows,
                        float* logits, int k, int* topk_idx, float* topk_lp);
void or_decoder_copy_slot(or_decoder* m, int dst, int src, int length);
/* ToolCaller.Complete's loop (src/Needle/ToolCaller.cs:59-77) on this
 * decoder: prefill the prompt into slot 0, then up to max_new times take
 * Ops.ArgMax of the last logits (or_argmax), stop before a token equal to
 * `stop` (-1: none), record it and feed it.  Returns the number of tokens. */
int or_greedy(or_decoder* m, const int* prompt, int prompt_len, int max_new, int stop, int* out_tokens,
              double* seconds);
/* seconds (if given): [prefill, decode] wall time. */
int or_beam_search(or_decoder* m, const int* prompt, int prompt_len, int width, int max_new, int eos,
                   int* out_tokens, float* out_score, long* fed_rows, double* seconds);

/* ---- Needle 3's batched decode step (needle3_model.c) ---- */

/* Needle 3 row kernels in the scalar order (src/Needle/Scalar.cs), the
 * polynomial Ops.Exp in place of MathF.Exp. */
float or_sigmoid(float x);
float or_n3_attn_gate(float x);                                                       /* Model.cs:147 */
void or_rms_fake_a8(const float* x, int n, float* d);                                 /* Scalar.RmsFakeA8 */
void or_centered_rms_fake_a8(const float* x, const float* s, int n, float* d);        /* Scalar.CenteredRmsFakeA8 */
void or_gate_fake_a8(float* x, const float* gate, int n);                             /* Scalar.GateFakeA8 */
float or_fake_a8(float* x, int n);                                                    /* Quant.FakeA8 (Quant.cs:69-79) */
void or_post_norm_add(float* residual, const float* x, const float* s, float gate, int n); /* Scalar.PostNormAdd */
void or_mix4(const float* s, int dim, float w0, float w1, float w2, float w3, float* d);  /* Scalar.Mix4 */
void or_combine_diff4x4(const float* s, int dim, const float* mix, const float* x, const float* u,
                        const float* post_gate, float* d);                            /* Ops.CombineDiff4x4 */
void or_sinkhorn4x4(const float* logits, float* r);                                   /* Scalar.Sinkhorn4x4 */
void or_rms_unit(const float* x, int n, float* d);                                    /* Ops.RmsUnit (scalar) */
float or_dot(const float* a, const float* b, int n);                                  /* Scalar.Dot */
void or_gather_row(const or_cq* w, int row, float* d);                                /* Quant.GatherRow */

/* Geometry (src/Needle/Model.cs:65-121) */
typedef struct or_n3_dims {
    int vocab, dim, heads, kv_heads, layers, qk, vd, hada_n, hada_rows, hada_cols, window;
    int engram_slots, engram_sub, engram_tables, engram_dilation, order_count, orders[4];
    int site_count, sites[16];
    uint64_t global_mask;
    float rope_theta;
} or_n3_dims;

/* MlpWeights (src/Needle/Audio.cs:5-27) */
typedef struct or_n3_mlp {
    const float *d1, *d2, *b2, *d3, *d4, *w1a, *w1b, *w2a, *w2b, *w3a, *w3b, *cond_v, *cond_u;
} or_n3_mlp;

/* LayerWeights (src/Needle/Model.cs:123-152); attn_gate already the
 * sigmoid of the stored value */
typedef struct or_n3_layer {
    const float* norm_in;
    or_cq q, k, v;
    const float *q_taps, *k_taps, *v_taps, *q_norm, *k_norm;
    or_cq gate, out;
    const float* post_norm;
    float attn_gate;
    const float* pre_hada;
    or_n3_mlp mlp;
} or_n3_layer;

/* EngramSite (src/Needle/Model.cs:176-188) */
typedef struct or_n3_site {
    or_cq tables, key, value;
    const float* taps; /* [4][dim] */
} or_n3_site;

typedef struct or_n3_model {
    or_n3_dims g;
    or_cq embedding;                                   /* [vocab][dim], 4-bit (the tied head) */
    const or_n3_layer* layer;                          /* [layers] */
    const float *a_pre, *a_post, *a_res, *b_pre, *b_post, *b_res;
    or_cq phi_pre, phi_post, phi_res;                  /* [L*4|L*4|L*16][4*dim], 4-bit */
    const int *perm_a, *perm_b;                        /* [hada_n] */
    const or_n3_site* site;                            /* [site_count] */
    const float* final_norm;
} or_n3_model;

/* A batched engine's state (EngineCore with slots, Engine.cs:2197-2283):
 * per slot the KV caches of every layer, the three-tap histories, the
 * engram histories, the two previous tokens, the length and the mark. */
typedef struct or_n3_engine {
    const or_n3_model* m;
    int slots, capacity, max_chunks;
    float *rope_cos, *rope_sin;                        /* [capacity][qk/2] */
    int8_t *keys, *values;                             /* [layers][slots][capacity][kv*qk | kv*vd] */
    float *key_scales, *value_scales;                  /* [layers][slots][capacity][kv] */
    float* qkv_hist;                                   /* [layers][slots][2*(qw+kw+vw)] */
    float* engram_hist;                                /* [sites][slots][9][dim] */
    float *snap_qkv, *snap_engram;
    int *length, *marked, *prev, *snap_prev;
    /* optional: when set, or_n3_forward copies the stream [rows][4][dim]
     * after the embedding to trace[0] and after layer l to trace[l + 1]
     * (the states tools/golden.py:253-267 dumps as x0 and streamNN) */
    float* trace;
} or_n3_engine;

/* HadamardMlp.Apply (Blocks.cs:1067-1101), scalar kernels, Scale 1 */
void or_hadamard_mlp(const or_n3_mlp* w, const float* pre_norm, const int* perm_a, const int* perm_b, int dim,
                     int rows, int cols, float* residual);
/* EngineCore.EngramHashRowsBatch (Engine.cs:2631-2656) */
void or_n3_engram_rows(const or_n3_dims* g, const int* tokens, const int* row_slots, int rows, const int* lengths,
                       const int* prev, int* out);
/* EngineCore.RopeFrequencies + BuildRopeTables (Engine.cs:336-356) */
void or_n3_rope_tables(float theta, int qk, int capacity, float* cos_t, float* sin_t);
int or_n3_init(or_n3_engine* e);
void or_n3_free(or_n3_engine* e);
void or_n3_reset(or_n3_engine* e, int slot);
void or_n3_mark(or_n3_engine* e, int slot);
void or_n3_rewind(or_n3_engine* e, int slot);
/* EngineCore.ForwardBatch (Engine.cs:2303-2350): logits [heads][vocab] of
 * the head rows. */
void or_n3_forward(or_n3_engine* e, const int* tokens, const int* row_slots, int rows, const int* head_rows,
                   int heads, float* logits);
/* The Needle 3 row ops' reduction order: 0 Scalar.cs, 1 the AVX2 tier's
 * Vector256 sums (and the elementwise forms of the ops that own them). */
void or_n3_set_tier(int tier);
int or_n3_tier(void);
float or_v256_sum(const float* a, const float* b, int n);
float or_tier_sum_of_squares(const float* x, int n);
/* A planted composition mistake for the tests' controls (0: none). */
void or_n3_set_plant(int which);
/* Threads of or_n3_forward's row-parallel loops (results do not depend on it). */
void or_n3_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif

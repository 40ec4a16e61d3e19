/*
 * needle_hip.h -- C ABI of libneedle_hip.so, the MI355X (gfx950) quantized
 * decode hot path of needle-cs.
 *
 * Two groups of entry points:
 *
 *  1. Kernel-table entries.  Same signatures and semantics as the reference's
 *     cdecl KernelTable slots (src/Needle/Kernels/KernelTable.cs:6-47, filled
 *     by src/Needle/Kernels/Net10KernelExports.cs:118-150): host pointers,
 *     synchronous, void (the reference has no error channel), rows outside
 *     [rowStart,rowEnd) untouched, tokens == 0 or an empty range a no-op.
 *     Weights are resolved to device-resident copies through a host-pointer ->
 *     device-pointer cache filled on first use, so a model's weights cross
 *     PCIe once.  A failure leaves the outputs untouched and sets
 *     nhip_last_error().
 *
 *  2. Device-resident API (the performance path).  Weights are uploaded once
 *     and stay in HBM; activations, outputs and KV caches are device pointers;
 *     every call is asynchronous on the given stream (NULL = the library's
 *     default stream) and returns 0 on success or a negative nhip_status.
 *
 * Every struct below matches the reference's C# sequential layout on x86-64
 * (natural alignment, 8-byte pointers).
 */
#ifndef NEEDLE_HIP_H
#define NEEDLE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ status ---- */

typedef enum nhip_status {
    NHIP_OK = 0,
    NHIP_ERR_ARG = -1,      /* invalid argument (shape, range, null pointer) */
    NHIP_ERR_HIP = -2,      /* a HIP runtime call failed */
    NHIP_ERR_NODEV = -3,    /* no usable gfx950 device */
    NHIP_ERR_FORMAT = -4,   /* malformed .cact archive */
    NHIP_ERR_CAPACITY = -5, /* KV capacity or slot count exceeded */
    NHIP_ERR_UNSUPPORTED = -6
} nhip_status;

/* Text of the last error on the calling thread ("" if none). */
const char* nhip_last_error(void);
/* Library and device description, e.g. "needle_hip 0.1 gfx950 (256 CUs)". */
const char* nhip_describe(void);

/* --------------------------------------------- reference struct layouts */

/* src/Needle/Model.cs:36-42 (Codebook: 100 bytes) */
typedef struct nhip_codebook {
    float levels[16];
    uint8_t bytes[32];
    float byte_scale;
} nhip_codebook;

/* src/Needle/Model.cs:8-34 (Cq: codebook-quantized weight view, 40 bytes).
 * indices: rows x (cols*bits/8) bytes; norms: fp16 [rows][cols/128]. */
typedef struct nhip_cq {
    const uint8_t* indices;
    const uint16_t* norms;
    const nhip_codebook* book;
    int32_t rows, cols, bits;
} nhip_cq;

/* src/Needle/Quant.cs:11-28 (Activations, 40 bytes).  values: int8
 * [tokens][cols] in planes order; scales/offsets: fp32 [tokens][stride],
 * stride = roundup8(cols/128). */
typedef struct nhip_activations {
    int8_t* values;
    float* scales;
    float* offsets;
    int32_t cols, groups, stride;
} nhip_activations;

/* src/Needle/Blocks.cs:11-27 (AttentionTile, 128 bytes) */
typedef struct nhip_attn_tile {
    const int8_t* queries;
    const float* query_scales;
    int32_t heads;
    const int8_t* keys;
    const float* key_scales;
    const int8_t* values;
    const float* value_scales;
    int32_t key_stride, value_stride, scale_stride, first, count;
    float* scores;
    float* output;
    float* probabilities;
    int32_t probability_stride;
    float* peaks;
    float* sums;
} nhip_attn_tile;

/* ------------------------------------------------- kernel-table entries */

/* Replaces slot 0, Quant.MatMulRows (src/Needle/Quant.cs:615-633; scalar
 * semantics src/Needle/Scalar.cs:146-192).  Results are bit-identical to the
 * reference's scalar kernel. */
void nhip_matmul_rows(const nhip_cq* w, const nhip_activations* a, int32_t tokens, float* y,
                      int32_t ldy, int32_t row_start, int32_t row_end);

/* Replaces slot 1, Quant.Prepare (src/Needle/Quant.cs:439-502; scalar branch
 * Quant.cs:473-488): per 128-group Walsh-Hadamard, int8 quantization,
 * planes permutation and offsets 63*sum(q). */
void nhip_prepare(float* x, int32_t tokens, int32_t cols, int32_t bits, const nhip_activations* a);

/* Replaces slot 3, Attention.Run (src/Needle/Blocks.cs:65-84; scalar
 * src/Needle/Scalar.cs:290-321).  With peaks/sums set, writes the
 * un-normalised partial (output, peak, sum per head) as the position-split
 * path expects (Blocks.cs:188-199, 950-958). */
void nhip_attention_tile(const nhip_attn_tile* tile);

/* Replaces slot 4, Attention.MergePartials (src/Needle/Blocks.cs:750-817). */
void nhip_merge_partials(const float* partials, int32_t count, int32_t heads, float* output);

/* Replaces slot 22, Quant.QuantizeInt8 (src/Needle/Quant.cs:103-132;
 * scalar src/Needle/Scalar.cs:67-74).  Returns the scale. */
float nhip_quantize_int8(const float* x, int32_t n, int8_t* destination);

/* The kernel-table entries above return void, as the reference's do: a
 * failure (no device, a HIP error, an argument the reference's caller would
 * have rejected) leaves the outputs untouched and sets nhip_last_error(), so
 * a host installs the table only after a probe call leaves nhip_last_error()
 * empty.  Weights are looked up in a cache by their view's host pointers and
 * shape; nhip_table_release drops every cached device copy whose index
 * pointer lies in [base, base + bytes) (all of them when base is NULL) and
 * frees its HBM -- call it when the host disposes of the model that owns
 * those bytes (Model.Dispose), with no entry running on its weights, so that
 * a later model mapped at the same addresses is uploaded afresh.
 * nhip_table_cached reports the cached entries and their HBM bytes. */
int32_t nhip_table_release(const void* base, size_t bytes, int32_t* released);
int32_t nhip_table_cached(int32_t* entries, size_t* device_bytes);

/* Mirror of Net10KernelExports.Fill (src/Needle/Kernels/Net10KernelExports.cs:118-150):
 * writes this library's entries into a 27-slot KernelTable (slots 0, 1, 3, 4,
 * 22; every other slot is set to NULL so the reference falls back to its own
 * kernels).  Returns NHIP_ERR_ARG if count < 27 or table is NULL. */
int32_t nhip_fill_kernel_table(void** table, int32_t count);

/* ------------------------------------------------ runtime plumbing ------ */

int32_t nhip_init(int32_t device);
int32_t nhip_device_count(int32_t* count);
int32_t nhip_malloc(void** ptr, size_t bytes);
int32_t nhip_free(void* ptr);
int32_t nhip_memcpy_htod(void* dst, const void* src, size_t bytes);
int32_t nhip_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int32_t nhip_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream);
/* Device-to-device copy by a kernel on `stream` (NULL = the library stream);
 * asynchronous and capturable in a graph.  Used for KV-slot copies. */
int32_t nhip_copy_dev(void* dst, const void* src, size_t bytes, void* stream);
int32_t nhip_memset(void* dst, int32_t value, size_t bytes);
int32_t nhip_stream_create(void** stream);
int32_t nhip_stream_destroy(void* stream);
int32_t nhip_stream_sync(void* stream);
int32_t nhip_device_sync(void);
int32_t nhip_event_create(void** event);
int32_t nhip_event_destroy(void* event);
int32_t nhip_event_record(void* event, void* stream);
int32_t nhip_event_elapsed_ms(void* start, void* stop, float* ms);

/* HIP graphs: capture the device-resident calls issued on `stream` between
 * begin and end into an executable graph, then replay it with one launch.
 * The library records no memset nodes into captured work. */
int32_t nhip_graph_begin(void* stream);
int32_t nhip_graph_end(void* stream, void** graph_exec);
int32_t nhip_graph_launch(void* graph_exec, void* stream);
int32_t nhip_graph_destroy(void* graph_exec);

/* --------------------------------------------- device-resident weights */

typedef struct nhip_weights nhip_weights;

/* Literal int8 format: int8 weights [rows][cols] row-major, one fp16 scale
 * per 32 consecutive elements [rows][cols/32].  cols must be a multiple of
 * 32.  Uploaded once and re-tiled in HBM for 1 KB coalesced loads. */
int32_t nhip_weights_i8_create(const int8_t* w, const uint16_t* scales, int32_t rows,
                               int32_t cols, nhip_weights** out);
/* Same from device buffers (no host copy; the inputs may be freed after). */
int32_t nhip_weights_i8_create_dev(const int8_t* d_w, const uint16_t* d_scales, int32_t rows,
                                   int32_t cols, nhip_weights** out);
/* Codebook format of .cact (Model.cs:257-267): indices + fp16 norms +
 * codebook, host pointers, 2- or 4-bit, cols a multiple of 128. */
int32_t nhip_weights_cq_create(const nhip_cq* w, nhip_weights** out);
int32_t nhip_weights_destroy(nhip_weights* w);
/* rows, cols, bits (8 for the literal format), HBM bytes held. */
int32_t nhip_weights_info(const nhip_weights* w, int32_t* rows, int32_t* cols, int32_t* bits,
                          size_t* device_bytes);

/* ------------------------------------------------ device-resident ops -- */

/* Per-row dynamic quantization (Scalar.QuantizeInt8 on each row):
 * x fp32 [tokens][cols] -> q int8 [tokens][cols], scales fp32 [tokens]. */
int32_t nhip_quantize_rows_dev(const float* d_x, int32_t tokens, int32_t cols, int8_t* d_q,
                               float* d_scales, void* stream);

/* Quant.Prepare on device (Quant.cs:473-488): x fp32 [tokens][cols] ->
 * values int8 [tokens][cols] (planes order), scales/offsets fp32
 * [tokens][stride]. */
int32_t nhip_prepare_dev(const float* d_x, int32_t tokens, int32_t cols, int32_t bits,
                         int8_t* d_values, float* d_scales, float* d_offsets, int32_t stride,
                         void* stream);

/* y[t*ldy+n] = sum_g (h(scale[n][g]) * qscale[t]) * dot_g(w[n], q[t]) for
 * n in [row_start,row_end), t < tokens, in Scalar.MatMulRows' order
 * (Scalar.cs:160-189).  Literal int8 weights. */
int32_t nhip_matmul_i8_dev(const nhip_weights* w, const int8_t* d_q, const float* d_qscale,
                           int32_t tokens, float* d_y, int32_t ldy, int32_t row_start,
                           int32_t row_end, void* stream);

/* Bandwidth calibration, no reference counterpart: reads `bytes` (a multiple
 * of 16) from d_src with the decode GEMV's access pattern (16-byte
 * non-temporal loads, 1 KB per wave instruction, 32 KB per 256-thread
 * workgroup) and writes each workgroup's XOR of the words it read to
 * d_sink[ceil(bytes / 32768)].  The time of one launch is the read ceiling
 * of a GEMV over the same bytes. */
int32_t nhip_read_stream_dev(const void* d_src, size_t bytes, uint32_t* d_sink, void* stream);

/* Prefill form of nhip_matmul_i8_dev with a fused epilogue: the same exact
 * int32 group sums D_g, accumulated as acc = fma(h(scale[n][g]), D_g, acc)
 * and scaled once, y = acc * qscale[t] -- two VALU operations per (token,
 * row, group) instead of the reference's four, so the fp32 outputs agree with
 * Scalar.MatMulRows to 1e-4 of RMS(y), not bit for bit.  For prefill
 * throughput; nhip_matmul_i8_dev stays bit-exact for every token count. */
int32_t nhip_matmul_i8_fused_dev(const nhip_weights* w, const int8_t* d_q, const float* d_qscale,
                                 int32_t tokens, float* d_y, int32_t ldy, int32_t row_start,
                                 int32_t row_end, void* stream);

/* Scalar.MatMulRows on device for codebook weights (Scalar.cs:146-192):
 * activations as produced by nhip_prepare_dev. */
int32_t nhip_matmul_cq_dev(const nhip_weights* w, const int8_t* d_values, const float* d_scales,
                           const float* d_offsets, int32_t stride, int32_t tokens, float* d_y,
                           int32_t ldy, int32_t row_start, int32_t row_end, void* stream);

/* Quant.MatMulBatch (src/Needle/Quant.cs:679-816): `count` (1..4) weight
 * matrices of one format and one K that share the activations (Needle 3's
 * Q, K, V and Gate projections), each job j computing all of its rows into
 * d_y[j] with row stride ldy[j] (>= its rows), as nhip_matmul_i8_dev
 * (literal: d_scales [tokens], d_offsets and stride unused) or
 * nhip_matmul_cq_dev (codebook) would.  Decode sizes (literal up to 16
 * tokens, codebook up to 4) run as one launch over every job's row tiles;
 * other token counts run the jobs in turn.  Bit-identical with the
 * single-matrix calls.  w and d_y / ldy are host arrays of `count` entries. */
int32_t nhip_matmul_batch_dev(const nhip_weights* const* w, int32_t count, const int8_t* d_q,
                              const float* d_scales, const float* d_offsets, int32_t stride,
                              int32_t tokens, float* const* d_y, const int32_t* ldy, void* stream);

/* The int32 group sums D[t][n-row_start][g] (Scalar.cs:162-184) that the
 * matmuls accumulate, for checking them bit-exactly.  Literal / codebook. */
int32_t nhip_group_dots_i8_dev(const nhip_weights* w, const int8_t* d_q, int32_t tokens,
                               int32_t row_start, int32_t row_end, int32_t* d_dots,
                               void* stream);
int32_t nhip_group_dots_cq_dev(const nhip_weights* w, const int8_t* d_values, int32_t tokens,
                               int32_t row_start, int32_t row_end, int32_t* d_dots,
                               void* stream);

/* ------------------------------------------ decode attention (KV cache) -- */

/* Ragged decode attention over a pooled int8 KV cache (one launch for a
 * batch of rows from independent slots).  Replaces the per-row
 * AttentionBatch.Run / ExecuteChunk + MergePartials path
 * (src/Needle/Blocks.cs:849-966, 750-817) that EngineCore.RunAttentionBatch
 * drives (src/Needle/Engine.cs:2480-2596).  Layout per layer, as the
 * reference's KV cache (src/Needle/Engine.cs:127-136, 184-187) with one
 * region per slot:
 *   keys   int8 [slots][capacity][kv_heads*qk_dim], key_scales   fp32 [slots][capacity][kv_heads]
 *   values int8 [slots][capacity][kv_heads*64],     value_scales fp32 [slots][capacity][kv_heads]
 *   q int8 [rows][heads][qk_dim] with q_scales [rows][heads] (QuantizeInt8
 *   per head), out fp32 [rows][heads][64].
 * Row r attends positions row_first[r] .. row_first[r]+row_count[r]-1 of
 * slot row_slot[r] (device arrays, so a captured graph can be replayed with
 * new spans); query head h reads kv head h / (heads/kv_heads).  Each (row,
 * head) is split into at most max_chunks chunks by the reference's plan
 * (8 reproduces the reference; 64 fills the GPU), each chunk is the
 * reference tile in partial form and the chunks are merged in
 * MergePartials' order, with the polynomial Ops.Exp.  Rows whose slot or
 * span is out of range produce zeros.  qk_dim is 48 or 64, v dim 64,
 * heads/kv_heads <= 16; q, keys, values and out 16-byte aligned.
 * The workspace (nhip_attention_decode_workspace bytes) holds the chunk
 * partials; it needs no initialisation (nhip_attention_decode_workspace_init
 * zeroes it, for callers that want defined contents).  Calls that share a
 * workspace must not overlap. */
size_t nhip_attention_decode_workspace(int32_t rows, int32_t heads, int32_t max_chunks);
int32_t nhip_attention_decode_workspace_init(void* d_workspace, size_t bytes, void* stream);
int32_t nhip_attention_decode_dev(const int8_t* d_q, const float* d_q_scales, int32_t rows,
                                  int32_t heads, int32_t kv_heads, int32_t qk_dim,
                                  const int8_t* d_keys, const float* d_key_scales,
                                  const int8_t* d_values, const float* d_value_scales,
                                  int32_t slots, int32_t capacity, const int32_t* d_row_slot,
                                  const int32_t* d_row_first, const int32_t* d_row_count,
                                  int32_t max_chunks, void* d_workspace, size_t workspace_bytes,
                                  float* d_out, void* stream);

/* No counterpart in the reference: nhip_attention_decode_dev for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, semantics and results,
 * without the workspace: the chunk partials go to a fixed 8 MiB device
 * scratch array that the library holds on each GPU until the process ends
 * (its address is looked up at nhip_init, which must have been called).
 * Calls whose partials (nhip_attention_decode_workspace(rows, heads,
 * max_chunks) bytes) exceed 8 MiB fail with NHIP_ERR_ARG.  No allocation
 * happens in the call.  Every call on a GPU shares that GPU's scratch:
 * calls that overlap on one GPU (other streams or threads) race, so
 * serialise them. */
int32_t nhip_attention_decode_noalloc_dev(const int8_t* d_q, const float* d_q_scales, int32_t rows,
                                          int32_t heads, int32_t kv_heads, int32_t qk_dim,
                                          const int8_t* d_keys, const float* d_key_scales,
                                          const int8_t* d_values, const float* d_value_scales,
                                          int32_t slots, int32_t capacity, const int32_t* d_row_slot,
                                          const int32_t* d_row_first, const int32_t* d_row_count,
                                          int32_t max_chunks, float* d_out, void* stream);

/* ------------------------------------ Needle 3 attention inputs (rows) -- */

/* Needle 3's step from a row's raw Q/K/V projections to its int8 query heads
 * and KV-cache row (EngineCore.TapsAndAttentionHeadsSingle,
 * src/Needle/Engine.cs:1302-1387, and Scalar.Taps3's multi-frame form,
 * src/Needle/Scalar.cs:285-288): for every query, key and value head the
 * three-tap convolution over time with the slot's two previous frames
 * (taps [3][width] per part: current, previous, two back), then for queries
 * and keys ZeroCenteredRms (q_norm / k_norm [qk_dim], shared by the heads),
 * Rope at the row's position (cos / sin tables [capacity][qk_dim/2]) and
 * QuantizeInt8 per head; values QuantizeInt8 per head.  Queries go to
 * d_q [rows][heads*qk_dim] / d_q_scales [rows][heads]; keys and values to the
 * cache at (slot, position): keys [slots][capacity][kv_heads*qk_dim],
 * values [slots][capacity][kv_heads*v_dim], scales [slots][capacity][kv_heads].
 * d_raw: [rows][qw + kw + vw] (qw = heads*qk_dim, kw = kv_heads*qk_dim,
 * vw = kv_heads*v_dim); d_history: [slots] x ([2][qw], [2][kw], [2][vw]),
 * frame 1 the latest, moved on to each slot's last two frames.  The rows of a
 * slot must be one contiguous run of consecutive positions (a row takes its
 * previous frames from the rows before it in the run); rows with an
 * out-of-range slot or position get q = 0, scale 1 and touch nothing.
 * qk_dim even and <= 64, v_dim <= 64.  Bit-identical with the reference's
 * scalar row-by-row step on the same tables. */
int32_t nhip_needle3_attention_inputs_dev(const float* d_raw, int32_t rows, int32_t heads, int32_t kv_heads,
                                          int32_t qk_dim, int32_t v_dim, const float* d_q_taps,
                                          const float* d_k_taps, const float* d_v_taps, const float* d_q_norm,
                                          const float* d_k_norm, const float* d_rope_cos,
                                          const float* d_rope_sin, float* d_history,
                                          const int32_t* d_row_slot, const int32_t* d_row_pos, int32_t slots,
                                          int32_t capacity, int8_t* d_q, float* d_q_scales, int8_t* d_keys,
                                          float* d_key_scales, int8_t* d_values, float* d_value_scales,
                                          void* stream);

/* ---------------------------------------------- decode loop (engine) -- */

/* The beam/ragged-batched decode step of a pre-norm int8 decoder (RMSNorm,
 * fused QKV, rotary positions, int8 KV cache per slot, SwiGLU FFN, LM head)
 * with every linear in the literal int8 format.  One forward packs `rows`
 * rows from independent cache slots, as EngineCore.ForwardBatch does
 * (src/Needle/Engine.cs:2303-2350, 2480-2596); beam search drives it as
 * Whistle.BeamSearch does (src/Needle/Whistle.Decode.cs:226-350) but with
 * the beams batched into one forward per step, which is the step API of the
 * performance path (nhip_step / slot copy).  Element-wise operations follow
 * the canonical order the CPU restatement shares, so logits and token streams
 * are bit-identical with it. */
typedef struct nhip_decoder nhip_decoder;

typedef struct nhip_decoder_dims {
    int32_t layers, d, heads, kv_heads, head_dim, ffn, vocab;
    int32_t capacity;   /* positions per cache slot */
    int32_t slots;      /* cache slots (beams, sequences) */
    int32_t max_rows;   /* rows per forward (prompt length for prefill) */
    int32_t max_chunks; /* attention position-split cap (64 fills the GPU) */
    double theta;       /* RoPE base */
    float eps;          /* RMSNorm epsilon */
} nhip_decoder_dims;

typedef struct nhip_decode_stats {
    double prefill_seconds, decode_seconds;
    int64_t fed_rows; /* rows fed after the prompt (row-tokens) */
    int32_t steps;
} nhip_decode_stats;

int32_t nhip_decoder_create(const nhip_decoder_dims* dims, nhip_decoder** out);
/* Host weights of one layer, uploaded and re-tiled: wqkv [(heads+2kv)*64][d],
 * wo [d][heads*64], wgu [2*ffn][d] (gate rows then up rows), wd [d][ffn],
 * each int8 with fp16 group-32 scales; RMSNorm gains [d]. */
int32_t nhip_decoder_set_layer(nhip_decoder* m, int32_t layer, const int8_t* wqkv, const uint16_t* sqkv,
                               const int8_t* wo, const uint16_t* so, const int8_t* wgu, const uint16_t* sgu,
                               const int8_t* wd, const uint16_t* sd, const float* attn_norm,
                               const float* ffn_norm);
/* Embedding fp32 [vocab][d], final RMSNorm gain [d], LM head [vocab][d]. */
int32_t nhip_decoder_set_head(nhip_decoder* m, const float* embedding, const float* final_norm,
                              const int8_t* wlm, const uint16_t* slm);
/* One synchronous forward of `rows` rows (host token/slot/position arrays):
 * writes each layer's K/V at the row's position in its slot, returns logits
 * [rows][vocab] if non-NULL and the top-k ids / log-probabilities
 * (TopKLogSoftmax, ids 0,2,3 masked) if k > 0 (k <= 8). */
int32_t nhip_decoder_forward(nhip_decoder* m, const int32_t* tokens, const int32_t* slots,
                             const int32_t* positions, int32_t rows, float* logits, int32_t k,
                             int32_t* topk_idx, float* topk_lp);
/* Grammar-constrained greedy step: one forward whose LM head computes only
 * the 16-row vocab tiles that hold an id allowed by some row's mask
 * (Engine.LogitsForRows' sparse head, src/Needle/Engine.cs:2191-2195,
 * 2683-2700), then Ops.ArgMaxMasked per row (src/Needle/Ops.cs:1223-1266):
 * best[r] = the lowest allowed id holding row r's largest allowed logit
 * above -inf, or -1.  masks: host [rows][words] bitsets, bit id%32 of word
 * id/32 (ids from vocab on are ignored); best_logit optional.  rows <= 16.
 * The allowed logits are bit-identical with the dense head's. */
int32_t nhip_decoder_forward_masked(nhip_decoder* m, const int32_t* tokens, const int32_t* slots,
                                    const int32_t* positions, int32_t rows, const uint32_t* masks,
                                    int32_t words, int32_t* best, float* best_logit);
/* Ops.ArgMaxMasked (src/Needle/Ops.cs:1223-1266; kernel-table slot 25's
 * operation) over `rows` device rows: row r reads d_x + r*ldx and the mask
 * d_mask + r*mask_ld ([words] bitsets, ids >= length ignored) and writes the
 * chosen id (or -1) to d_index[r] and, if d_value is non-NULL, its value
 * (-inf for -1).  Asynchronous on `stream`. */
int32_t nhip_argmax_masked_dev(const float* d_x, int32_t ldx, const uint32_t* d_mask, int32_t mask_ld,
                               int32_t words, int32_t length, int32_t rows, int32_t* d_index, float* d_value,
                               void* stream);
/* Ops.TopKLogSoftmax (src/Needle/Ops.cs:1092-1221) as the decoder's head
 * runs it, over `rows` device rows of n logits (row r at d_logits + r*n):
 * the k (1..8) best ids by value, ties to the lower id, ids 0, 2 and 3
 * excluded, and their log-probabilities v - (peak + log S), with S summed
 * over blocks of 2048 ids in the canonical order.  d_idx / d_lp: [rows][k].
 * n <= 524288.  The workspace (nhip_topk_lse_workspace bytes) holds the
 * per-block partial lists; nothing needs clearing.  Asynchronous on
 * `stream`. */
size_t nhip_topk_lse_workspace(int32_t rows, int32_t n);
int32_t nhip_topk_lse_dev(const float* d_logits, int32_t rows, int32_t n, int32_t k, void* d_workspace,
                          size_t workspace_bytes, int32_t* d_idx, float* d_lp, void* stream);
/* Ops.ArgMax (src/Needle/Ops.cs:1052-1090; Engine.Greedy, Engine.cs:103)
 * over `rows` device rows of n values (row r at d_x + r*ldx): d_index[r] =
 * the lowest id holding the row's largest non-NaN value, 0 when x[0] is NaN
 * (the scalar loop's `x[i] > x[best]` from best = 0: +0 and -0 are equal, an
 * all -inf row gives 0; the AVX path gives the same ids on NaN-free rows);
 * d_value[r] (optional) = that value.  Asynchronous on `stream`. */
int32_t nhip_argmax_dev(const float* d_x, int32_t ldx, int32_t n, int32_t rows, int32_t* d_index, float* d_value,
                        void* stream);
/* Engine.CopyFrom (src/Needle/Engine.cs:367-379): positions [0, length) of
 * slot src into slot dst, whose length (for nhip_decoder_step) becomes
 * `length`. */
int32_t nhip_decoder_copy_slot(nhip_decoder* m, int32_t dst, int32_t src, int32_t length);
/* The step API of the batched engine: BatchedEngine.ForwardBatch /
 * EngineCore.ForwardBatch (src/Needle/BatchEngine.cs:38-39,
 * src/Needle/Engine.cs:2303-2350).  Rows carry tokens[r] into slot
 * row_slots[r]; the rows of a slot form one contiguous run and sit at the
 * slot's length + their offset in the run (Engine.cs:2655-2661), and every
 * slot's length grows by its run (NHIP_ERR_ARG past the capacity, before any
 * device work).  The LM head runs only over head_rows[0..heads) (rows of
 * this call): row i of the outputs is row head_rows[i] -- logits [heads][vocab]
 * (BatchLogitsRow), the top-k ids / log-probabilities [heads][k] if k > 0,
 * Ops.ArgMax of each head row into argmax[heads] if non-NULL.  rows <= 16
 * replay a graph captured per (rows, heads, k, argmax).  Synchronous.
 * nhip_decoder_forward (explicit positions) leaves the lengths alone. */
int32_t nhip_decoder_step(nhip_decoder* m, const int32_t* tokens, const int32_t* row_slots, int32_t rows,
                          const int32_t* head_rows, int32_t heads, float* logits, int32_t k, int32_t* topk_idx,
                          float* topk_lp, int32_t* argmax);
/* BatchedEngine.ResetSlot / MarkSlot / RewindSlot / SlotLength
 * (src/Needle/BatchEngine.cs:25-30): reset sets a slot's length (and mark) to
 * 0, mark records its length, rewind returns to the mark; the next step
 * overwrites the cache from there. */
int32_t nhip_decoder_slot_reset(nhip_decoder* m, int32_t slot);
int32_t nhip_decoder_slot_mark(nhip_decoder* m, int32_t slot);
int32_t nhip_decoder_slot_rewind(nhip_decoder* m, int32_t slot);
int32_t nhip_decoder_slot_length(const nhip_decoder* m, int32_t slot, int32_t* length);
/* Greedy decoding, ToolCaller.Complete's loop (src/Needle/ToolCaller.cs:
 * 59-77) on slot 0: reset it, feed the prompt (chunks of max_rows rows, the
 * head on the last row only), then up to max_new times take Ops.ArgMax of
 * the last logits on the device, stop before a token equal to `stop` (-1:
 * none), otherwise record it and feed it.  Writes the tokens (without the
 * prompt) and their count. */
int32_t nhip_decoder_greedy(nhip_decoder* m, const int32_t* prompt, int32_t prompt_len, int32_t max_new,
                            int32_t stop, int32_t* out_tokens, int32_t* out_len, nhip_decode_stats* stats);
/* Prefill `prompt` into slot 0, then beam search of `width` beams for up to
 * max_new tokens (length penalty 1, EOS `eos`); writes the winner's tokens
 * (without the prompt), its length and normalised score. */
int32_t nhip_decoder_beam_search(nhip_decoder* m, const int32_t* prompt, int32_t prompt_len, int32_t width,
                                 int32_t max_new, int32_t eos, int32_t* out_tokens, int32_t* out_len,
                                 float* out_score, nhip_decode_stats* stats);
int32_t nhip_decoder_destroy(nhip_decoder* m);

/* ------------------------------------------------- .cact archives (Model) -- */

/* Model.Open / Model.FromMemory (src/Needle/Model.cs:307-389, 400-411): the
 * archive is parsed in place and every tensor is uploaded to HBM once.  The
 * layout is the reference's (Model.cs:190-276 Record / Reader;
 * ModelInfo.cs:7-8 magic 0x05E12A84 and the 196-byte header): 48 uint32
 * header words + the RoPE theta float, header[2] codebook floats, header[1]
 * packed 44-byte records, then the data.  Malformed archives (Model.cs:372-389's
 * checks, plus each record's data inside the archive) give NHIP_ERR_FORMAT
 * before any device work.  Codebook-quantized records become weights for
 * nhip_matmul_cq_dev (2-bit book = Codebook.Fill(levels 0..3), 4-bit =
 * Codebook.Fill(levels 12..27)); fp16 / fp32 records become fp32 device
 * arrays (fp16 by Scalar.HalfToSingle); raw records (the tokenizer blob)
 * stay in the caller's bytes at record.offset.  The model holds no pointer
 * into the archive after nhip_open returns. */
enum { NHIP_CACT_FP16 = 1, NHIP_CACT_FP32 = 2, NHIP_CACT_CQ = 3, NHIP_CACT_RAW = 4 };

typedef struct nhip_record_info {
    int32_t dtype, ndim;
    uint32_t shape[4];
    uint64_t offset, bytes; /* in the archive */
    uint32_t group, bits;   /* codebook-quantized records: 128, 2 or 4 */
} nhip_record_info;

typedef struct nhip_model nhip_model;

int32_t nhip_open(const uint8_t* cact, size_t length, nhip_model** out);
/* header words [48] (geometry: Model.cs:65-105), RoPE theta, record count;
 * any output may be NULL */
int32_t nhip_model_info(const nhip_model* m, uint32_t* header48, float* rope_theta, int32_t* records);
int32_t nhip_model_record(const nhip_model* m, int32_t index, nhip_record_info* info);
/* the device weights of a codebook-quantized record, else NULL */
nhip_weights* nhip_model_weights(const nhip_model* m, int32_t index);
/* the fp32 device array of an fp16 / fp32 record, else NULL */
const float* nhip_model_dense(const nhip_model* m, int32_t index);
/* the record's bytes (indices, then fp16 norms) on the device, for row
 * gathers (Quant.GatherRow, src/Needle/Quant.cs:566-575), of a
 * codebook-quantized record, else NULL */
const uint8_t* nhip_model_raw(const nhip_model* m, int32_t index);
/* the archive's 2-bit and 4-bit codebooks (Model.cs:318-321); either may be NULL */
int32_t nhip_model_codebooks(const nhip_model* m, nhip_codebook* book2, nhip_codebook* book4);
int32_t nhip_model_close(nhip_model* m);

/* ----------------------------------- Needle 3 batched engine (step API) -- */

/* BatchedEngine over an opened Needle 3 archive (src/Needle/BatchEngine.cs:5-50,
 * EngineCore.ForwardBatch, src/Needle/Engine.cs:2285-2350): `slots` (1..16)
 * independent sequences of up to `capacity` positions each, steps of up to
 * `chunk` rows (0: the reference's default 64).  Attention splits a row's
 * span into at most `max_chunks` chunks by the reference's plan (0: 8, the
 * reference's MaxChunks, Blocks.cs:832).  The model must stay open while the
 * context lives.  One context is single-threaded; it owns a HIP stream and
 * its device state (KV cache, convolution and engram histories, snapshots). */
typedef struct nhip_ctx nhip_ctx;

int32_t nhip_ctx_create(const nhip_model* model, int32_t capacity, int32_t slots, int32_t chunk,
                        int32_t max_chunks, nhip_ctx** out);
int32_t nhip_ctx_destroy(nhip_ctx* c);
/* any output may be NULL */
int32_t nhip_ctx_info(const nhip_ctx* c, int32_t* vocab, int32_t* slots, int32_t* capacity, int32_t* chunk);
/* ForwardBatch (Engine.cs:2303-2350): row r feeds tokens[r] to slot
 * row_slots[r]; a slot's rows form one contiguous run at the slot's length +
 * their offset in it, and every slot's length grows by its run (NHIP_ERR_ARG
 * past the capacity, before any device work).  The LM head runs only over
 * head_rows[0..heads): output row i is row head_rows[i] -- logits
 * [heads][vocab] if non-NULL (BatchLogitsRow), the top-k ids and
 * log-probabilities [heads][k] if k > 0 (Ops.TopKLogSoftmax as
 * nhip_topk_lse_dev), Ops.ArgMax of each head row into argmax[heads] if
 * non-NULL.  Synchronous.  After a failed step the slots it named must be
 * reset. */
int32_t nhip_step(nhip_ctx* c, const int32_t* tokens, const int32_t* row_slots, int32_t rows,
                  const int32_t* head_rows, int32_t heads, float* logits, int32_t k, int32_t* topk_idx,
                  float* topk_lp, int32_t* argmax);
/* FeedSlot (Engine.cs:2285-2301): `count` tokens into one slot in steps of
 * `chunk` rows; logits [vocab] of the last token if non-NULL. */
int32_t nhip_slot_feed(nhip_ctx* c, int32_t slot, const int32_t* tokens, int32_t count, float* logits);
/* ResetSlot / MarkSlot / RewindSlot / SlotLength (BatchEngine.cs:24-29,
 * Engine.cs:2224-2283): reset clears the slot's histories and sets its length
 * and mark to 0; mark snapshots the histories and records the length; rewind
 * restores the snapshot and the length. */
int32_t nhip_slot_reset(nhip_ctx* c, int32_t slot);
int32_t nhip_slot_mark(nhip_ctx* c, int32_t slot);
int32_t nhip_slot_rewind(nhip_ctx* c, int32_t slot);
int32_t nhip_slot_length(const nhip_ctx* c, int32_t slot, int32_t* length);
/* Engine.CopyFrom (Engine.cs:367-379) between two slots of one context (a
 * beam reorder): dst becomes a clone of src -- KV positions [0, length of
 * src), histories, snapshot, previous tokens, length and mark. */
int32_t nhip_slot_copy(nhip_ctx* c, int32_t dst, int32_t src);

/* ------------------------------------------ synthetic workload inputs -- */

/* Deterministic host-side generators for the benchmark workloads: one
 * XorShift64 stream (tests/Needle.Tests/Conformance/Conformance.cs:10-38),
 * 53-bit uniforms, N(0,1) by Box-Muller, fp16 by round-to-nearest-even.
 * The state is updated in place. */
void nhip_synth_normal(uint64_t* state, float* x, size_t n);
void nhip_synth_uniform(uint64_t* state, float* x, size_t n, float lo, float hi);
void nhip_synth_int8(uint64_t* state, int8_t* x, size_t n);
void nhip_synth_half_uniform(uint64_t* state, uint16_t* x, size_t n, float lo, float hi);

#ifdef __cplusplus
}
#endif
#endif

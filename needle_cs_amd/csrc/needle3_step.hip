// needle3_step.hip -- Needle 3's batched decode step on gfx950, driven from an
// opened .cact archive: the step API of the batched engine (nhip_ctx_*,
// nhip_step, nhip_slot_*).
//
// One step is EngineCore.ForwardBatch (src/Needle/Engine.cs:2303-2350): rows
// from up to `slots` independent sequences, each slot's rows one contiguous
// run at the slot's length + their offset, through
//   embedding (Quant.GatherRow of the 4-bit table, times sqrt(dim), copied to
//   the four hyper-connection lanes),
//   per layer (RunLayerBatch, :2352-2398)
//     RmsFakeA8 of the 4-lane stream, Prepare 4-bit, the phi matmuls,
//     sigmoid gates, Mix4 and Sinkhorn4x4 (the hyper-connection mix),
//     the engram at its layers (ApplyEngramBatch, :2399-2463),
//     attention (RunAttentionBatch, :2480-2596): CenteredRmsFakeA8, Prepare
//     2-bit, the Q/K/V/Gate MatMulBatch, the three-tap convolution +
//     ZeroCenteredRms + RoPE + QuantizeInt8 into the KV cache, ragged
//     attention over the window (global layers: the whole span), GateFakeA8,
//     Prepare, the output matmul and PostNormAdd,
//     the Kronecker-Hadamard MLP (HadamardMlp.Apply, Blocks.cs:1067-1101),
//     CombineDiff4x4 into the next stream;
//   the head rows: Mix4 of the lanes, ZeroCenteredRms, FakeA8, Prepare 4-bit
//   and the tied embedding (PrepareHeadVectors, :920-928).
// Every row kernel below follows its scalar kernel's operation order
// (src/Needle/Scalar.cs) with the polynomial Ops.Exp where that code calls
// MathF.Exp; sums are sequential chains (one lane over the row staged in
// LDS), maxima are order-free, element-wise work runs in parallel with the
// same per-element arithmetic.  The results are bit-identical with the CPU
// restatement.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "common.hpp"

namespace nhip {

int32_t attention_decode_impl(const int8_t* d_q, const float* d_qscale, int32_t rows, int32_t heads,
                              int32_t kv_heads, int32_t qk_dim, const int8_t* d_keys, const float* d_key_scales,
                              const int8_t* d_values, const float* d_value_scales, int32_t slots, int32_t capacity,
                              const int32_t* d_row_slot, const int32_t* d_row_first, const int32_t* d_row_count,
                              int32_t max_chunks, void* d_workspace, size_t workspace_bytes, float* d_out,
                              int8_t* d_q_out, float* d_qs_out, hipStream_t stream);
int32_t matmul_cq_split_internal(const DeviceWeights* w, const int8_t* values, const float* scales,
                                 const float* offsets, int32_t stride, int32_t tokens, float* const* ys,
                                 const int32_t* ldys, const int32_t* firsts, int32_t parts, hipStream_t stream);
int32_t weights_cq_create_internal(const nhip_cq* cq, nhip_weights** out);

namespace {

constexpr int kLanes = 4;
constexpr int kEngramHistory = 9;
constexpr int kEngramTaps = 4;
constexpr int kThreads = 1024;  // one workgroup per row: 16 waves share each row's phases
constexpr int kWaves = kThreads / 64;
constexpr int kMaxDim = 1024;
constexpr int kPer = kMaxDim / kThreads;    // elements of a dim-row per thread: c = threadIdx.x + kThreads * q
constexpr int kMaxStream = kLanes * kMaxDim;
constexpr int kCondPer = 8 * kMaxDim / kThreads;  // condition-weight entries per thread
constexpr int kHistPer = (2560 + kThreads - 1) / kThreads;  // Q/K/V frame entries per thread (qw + kw + vw <= 2560)
constexpr int kMaxPhiGroups = kLanes * kMaxDim / 128;       // groups of a phi row (K = 4 * dim)

__device__ __forceinline__ float sigmoid_poly(float x) { return 1.0f / (1.0f + exp_poly(-x)); }

__device__ __forceinline__ float clamp_q(float v)
{
    return fminf(fmaxf(ref_round_even(v), -128.0f), 127.0f);
}

__device__ __forceinline__ int col_of(int q) { return (int)threadIdx.x + kThreads * q; }

// Ops.InverseRms of a sum of squares over n elements
__device__ __forceinline__ float inverse_rms_of(float sum, int n) { return 1.0f / sqrtf(sum / (float)n + 1e-6f); }

// Quant.Prepare (Quant.cs:473-488) of an LDS row of `cols` floats into row t
// of act: wave w takes groups w, w + 4, ...
__device__ __forceinline__ void prepare_row(const float* v, int cols, int bits, const Act& act, int stride, int t)
{
    const int lane = threadIdx.x & 63;
    for (int g = threadIdx.x >> 6; g < cols / 128; g += kWaves) {
        float v0 = v[g * 128 + lane], v1 = v[g * 128 + 64 + lane];
        hadamard_wave(v0, v1);
        prepare_group_wave(v0, v1, bits, act.values + (size_t)t * cols + g * 128, act.scales + (size_t)t * stride + g,
                           act.offsets + (size_t)t * stride + g);
    }
}

// prepare_row of the row that RmsUnit and Quant.FakeA8 make of the LDS row
// v: element i is clamp(RoundEven((v[i] * inverse) * round)) * scale, formed
// by the wave that prepares its group (no pass and barrier of its own).  The
// caller takes FakeA8's scale = peak > 0 ? peak / 127 : 1 and round =
// 1 / scale (Scalar.cs:55-65) from the row's peak of v * inverse, which is
// RoundNearest(max |v| * inverse) since inverse > 0 and rounding is monotone.
__device__ __forceinline__ void prepare_row_fake(const float* v, int cols, int bits, const Act& act, int stride, int t,
                                                 float inverse, float round, float scale)
{
    const int lane = threadIdx.x & 63;
    for (int g = threadIdx.x >> 6; g < cols / 128; g += kWaves) {
        float v0 = clamp_q((v[g * 128 + lane] * inverse) * round) * scale;
        float v1 = clamp_q((v[g * 128 + 64 + lane] * inverse) * round) * scale;
        hadamard_wave(v0, v1);
        prepare_group_wave(v0, v1, bits, act.values + (size_t)t * cols + g * 128, act.scales + (size_t)t * stride + g,
                           act.offsets + (size_t)t * stride + g);
    }
}

// Ops.InverseRms of an LDS row x[0..n) (written before the call and
// synchronised), its sum of squares in the AVX2 tier's order by wave 0.
__device__ __forceinline__ float row_inverse_rms(const float* x, int n, float* slot)
{
    if (threadIdx.x < 64) {
        const float sum = wave_v256_sum(x, x, n);
        if (threadIdx.x == 0) *slot = inverse_rms_of(sum, n);
    }
    __syncthreads();
    return *slot;
}

// The same, with `beside()` run by waves 1.. while wave 0 sums.
template <typename F>
__device__ __forceinline__ float row_inverse_rms_beside(const float* x, int n, float* slot, F&& beside)
{
    if (threadIdx.x < 64) {
        const float sum = wave_v256_sum(x, x, n);
        if (threadIdx.x == 0) *slot = inverse_rms_of(sum, n);
    } else {
        beside();
    }
    __syncthreads();
    return *slot;
}

// ---------------------------------------------------------- gathers --

struct Book {
    float levels[16];
};

// Quant.GatherRow of group `group` of row `row` (Scalar.DecodeRow, then
// Scalar.Hadamard), held by a wave as hadamard_wave leaves it.
__device__ __forceinline__ void gather_group_wave(const uint8_t* raw, int rows, int cols, int bits, const Book& book,
                                                  int row, int group, float& v0, float& v1)
{
    const int lane = threadIdx.x & 63;
    const int groups = cols / 128;
    const uint8_t* idx = raw + (size_t)row * cols * bits / 8;
    const uint16_t* norms = reinterpret_cast<const uint16_t*>(raw + (size_t)rows * cols * bits / 8);
    const float norm = ref_half_to_single(norms[(size_t)row * groups + group]);
    int c0, c1;
    if (bits == 2) {
        c0 = (idx[group * 32 + lane / 4] >> (lane % 4 * 2)) & 3;
        c1 = (idx[group * 32 + (lane + 64) / 4] >> (lane % 4 * 2)) & 3;
    } else {
        c0 = (idx[group * 64 + lane / 2] >> (lane % 2 * 4)) & 15;
        c1 = (idx[group * 64 + (lane + 64) / 2] >> (lane % 2 * 4)) & 15;
    }
    v0 = book.levels[c0] * norm;
    v1 = book.levels[c1] * norm;
    hadamard_wave(v0, v1);
}


// ----------------------------------------------- hyper-connection mix --

struct HyperArgs {
    const float* stream;
    PhiRows phi;
    const float *a_pre, *a_post, *a_res, *b_pre, *b_post, *b_res;  // the layer's entries
    int lane, dim;
    float* input;
    float* residual;
    float* post_gate;  // [rows][4]
    float* mix;        // [rows][16]
    const float* norm_in;
    // engram layers: the gathered engram input instead of the attention norm
    const uint8_t* tables;
    int table_rows, table_cols, table_bits, tables_count;
    Book book;
    const int32_t* erows;
    Act act;
    int stride;
    int rows;
};

// Thread i < 8's phi output affine map, z = ga * y + gb: i < 4 the pre
// outputs (a_pre, b_pre[i]), then the post ones (a_post, b_post[i - 4]).
__device__ __forceinline__ void phi_affine(const HyperArgs& a, float& ga, float& gb)
{
    const int i = threadIdx.x;
    const global_ptr<float> a0 = scalar_ptr(a.a_pre), a1 = scalar_ptr(a.a_post);
    const global_ptr<float> b0 = scalar_ptr(a.b_pre), b1 = scalar_ptr(a.b_post);
    ga = 0.0f;
    gb = 0.0f;
    if (i < 8) {
        const bool post = i >= 4;
        ga = (post ? a1 : a0)[0];
        gb = (post ? b1 : b0)[i & 3];
    }
}

// The rest of row t's mix once thread i < 8 holds its phi output y (i < 4:
// pre, else post) and its affine map ga, gb: hpre / postGate by Sigmoid,
// Mix4 of the stream lanes sv into input and residual, then on layers
// without an engram the attention input's CenteredRmsFakeA8 and 2-bit
// Prepare, on engram layers the gathered engram input's FakeA8 and 2-bit
// Prepare (RunLayerBatch, Engine.cs:2356-2414).  The attention input's
// FakeA8 peak is taken with the mix, before the norm: with v = (1 + s) * u
// and inverse > 0, max |v * inverse| is RoundNearest(max |v| * inverse), as
// rounding is monotone, so the scaling and the int8 round trip run inside
// the Prepare waves after the sum of squares.
__device__ __forceinline__ void hyper_mix_row(const HyperArgs& a, int t, float y, float ga, float gb,
                                              const float (&sv)[kPer][kLanes], const float (&sn)[kPer], float* x,
                                              float* sq, float* hpre, float* red, float* inv_s)
{
    const int dim = a.dim;
    const int i = threadIdx.x;
    if (i < 4) hpre[i] = sigmoid_poly(ga * y + gb + (i == a.lane ? 4.0f : -4.0f));
    if (i >= 4 && i < 8) a.post_gate[t * 4 + i - 4] = 2.0f * sigmoid_poly(ga * y + gb + (i - 4 == a.lane ? 0.0f : -4.0f));
    __syncthreads();
    float peak = 0.0f;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = col_of(q);
        if (c < dim) {
            const float u = hpre[0] * sv[q][0] + hpre[1] * sv[q][1] + hpre[2] * sv[q][2] + hpre[3] * sv[q][3];
            a.input[(size_t)t * dim + c] = u;
            a.residual[(size_t)t * dim + c] = u;
            x[c] = u;
            const float v = (1.0f + sn[q]) * u;
            sq[c] = v;  // the scaled row, for the Prepare waves (sq serves the engram input otherwise)
            peak = fmaxf(peak, fabsf(v));
        }
    }
    if (!a.tables) {
        peak = wave_max(peak);
        if ((i & 63) == 0) red[i >> 6] = peak;
    }
    __syncthreads();
    if (a.tables) {
        // wave u gathers group u of the row (table u / per, its group u %
        // per; dim <= 1024: at most 8 groups) in the Hadamard's lane layout,
        // then FakeA8 at the row's peak, Hadamard and Prepare from registers
        const int sub = a.table_cols, per = sub / 128, units = a.tables_count * per;
        const int unit = i >> 6;
        float v0 = 0.0f, v1 = 0.0f;
        if (unit < units) {
            const int table = unit / per, g = unit % per;
            const int r = a.erows[t * a.tables_count + table];
            if (r >= 0) gather_group_wave(a.tables, a.table_rows, sub, a.table_bits, a.book, r, g, v0, v1);
            const float m = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
            if ((i & 63) == 0) red[unit] = m;
        }
        __syncthreads();
        if (unit < units) {
            float m = 0.0f;
            for (int j = 0; j < units; j++) m = fmaxf(m, red[j]);
            const float scale = m > 0.0f ? m / 127.0f : 1.0f;
            const float round = 1.0f / scale;
            v0 = clamp_q(v0 * round) * scale;
            v1 = clamp_q(v1 * round) * scale;
            hadamard_wave(v0, v1);
            prepare_group_wave(v0, v1, 2, a.act.values + (size_t)t * dim + unit * 128,
                               a.act.scales + (size_t)t * a.stride + unit, a.act.offsets + (size_t)t * a.stride + unit);
        }
        return;
    }
    const float inverse = row_inverse_rms(x, dim, inv_s);
    float m = red[0];
    for (int w = 1; w < kWaves; w++) m = fmaxf(m, red[w]);
    const float top = m * inverse;
    const float scale = top > 0.0f ? top / 127.0f : 1.0f;
    const float round = 1.0f / scale;
    prepare_row_fake(sq, dim, 2, a.act, a.stride, t, inverse, round, scale);
}

// RunLayerBatch's per-row mix (Engine.cs:2356-2381): the phi rows, hpre /
// postGate by Sigmoid, Mix4 of the lanes into input and residual, Sinkhorn4x4
// of the residual-mix logits.  Workgroup t < rows takes row t's 4 pre and 4
// post outputs and the mix; only the layer's tail reads the Sinkhorn matrix,
// so workgroup rows + t (launched for steps whose attention launch does not
// form it) forms row t's 16 residual-mix outputs and its Sinkhorn
// (Engine.cs:2374-2378) beside it.  Then, on layers without an engram,
// RunAttentionBatch's CenteredRmsFakeA8 of the residual and its 2-bit Prepare
// (Engine.cs:2487-2490); on engram layers, ApplyEngramBatch's input
// (Engine.cs:2404-2414): every table's GatherRow (zeros for row -1),
// Quant.FakeA8 and the 2-bit Prepare.
__global__ __launch_bounds__(kThreads) void n3_hyper_kernel(HyperArgs a)
{
    __shared__ __align__(16) float prod[2 * 16 * kMaxPhiGroups];
    __shared__ float logits[16];
    const int dim = a.dim, K = kLanes * dim;
    if ((int)blockIdx.x >= a.rows) {
        const int t = (int)blockIdx.x - a.rows;
        const int first[4] = {0, 16, 16, 16};
        const PhiUnit unit = phi_load(a.phi, K, 2, first);
        const float ga = a.a_res[0], gb = a.b_res[threadIdx.x & 15];
        const float y = phi_outputs(a.phi, unit, a.phi.in.values + (size_t)t * K,
                                    a.phi.in.scales + (size_t)t * a.phi.stride,
                                    a.phi.in.offsets + (size_t)t * a.phi.stride, K, first, prod);
        if (threadIdx.x < 16) logits[threadIdx.x] = ga * y + gb;
        __syncthreads();
        if (threadIdx.x < 64) sinkhorn4x4_wave(logits, a.mix + t * 16);
        return;
    }
    __shared__ __align__(16) float x[kMaxDim];
    __shared__ __align__(16) float sq[kMaxDim];
    __shared__ float hpre[4];
    __shared__ float red[kWaves];
    __shared__ float inv_s;
    const int t = blockIdx.x;
    const int first[4] = {0, 4, 8, 8};
    const PhiUnit unit = phi_load(a.phi, K, 0, first);
    float ga, gb;
    phi_affine(a, ga, gb);
    const float* s = a.stream + (size_t)t * kLanes * dim;
    float sv[kPer][kLanes], sn[kPer];
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = col_of(q);
        if (c < dim) {
#pragma unroll
            for (int l = 0; l < kLanes; l++) sv[q][l] = s[l * dim + c];
            sn[q] = a.norm_in[c];
        }
    }
    const float y = phi_outputs(a.phi, unit, a.phi.in.values + (size_t)t * K,
                                a.phi.in.scales + (size_t)t * a.phi.stride, a.phi.in.offsets + (size_t)t * a.phi.stride,
                                K, first, prod);
    hyper_mix_row(a, t, y, ga, gb, sv, sn, x, sq, hpre, red, &inv_s);
}

// Embedding (ForwardBatch, Engine.cs:2310-2316): GatherRow of the token's
// row, x += (sqrt(dim) - 1) * x, copied to the four lanes of the stream; then
// the first layer's RmsFakeA8 of the stream and its 4-bit Prepare.
// HYPER: for a decode step (rows one per slot), the workgroup goes on into
// layer 0's mix (h, as n3_tail_kernel<true> does for later layers): the
// stream row stays in LDS and its 4-bit prepared activations too, with a copy
// in act for the attention launch's residual-mix rows.
template <bool HYPER>
__global__ __launch_bounds__(kThreads) void n3_embed_kernel(const uint8_t* raw, int rows, int dim, int bits, Book book,
                                                            const int32_t* tokens, float scale_m1, float* stream,
                                                            Act act, int stride, HyperArgs h)
{
    __shared__ __align__(16) float s[kMaxStream];
    __shared__ float red[kWaves];
    __shared__ float inv_s;
    __shared__ __align__(16) int8_t a4v[HYPER ? kMaxStream : 16];
    __shared__ __align__(16) float a4s[HYPER ? 2 * kMaxPhiGroups : 4];
    __shared__ __align__(16) float hprod[HYPER ? 2 * 8 * kMaxPhiGroups : 4];
    __shared__ __align__(16) float hx[HYPER ? kMaxDim : 4];
    __shared__ __align__(16) float hsq[HYPER ? kMaxDim : 4];
    __shared__ float hpre[4];
    constexpr int kPhiFirst[4] = {0, 4, 8, 8};
    constexpr int kPhiBase = 8 * 64;  // waves 8.. take the phi units
    PhiUnit hunit{};
    float hga = 0.0f, hgb = 0.0f, hsn[kPer];
    if constexpr (HYPER) {
        hunit = phi_load(h.phi, kLanes * dim, 0, kPhiFirst, kPhiBase);
        phi_affine(h, hga, hgb);
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int c = col_of(q);
            if (c < dim) hsn[q] = h.norm_in[c];
        }
    }
    const int t = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int token = tokens[t];
    float* row = stream + (size_t)t * kLanes * dim;
    for (int g = threadIdx.x >> 6; g < dim / 128; g += kWaves) {
        float v0, v1;
        gather_group_wave(raw, rows, dim, bits, book, token, g, v0, v1);
        const float x0 = v0 + scale_m1 * v0, x1 = v1 + scale_m1 * v1;
        for (int l = 0; l < kLanes; l++) {
            const int c = l * dim + g * 128 + lane;
            row[c] = x0;
            row[c + 64] = x1;
            s[c] = x0;
            s[c + 64] = x1;
        }
        // the group's peak (dim <= 1024: one group a wave, at most 8)
        const float m = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
        if (lane == 0) red[g] = m;
    }
    __syncthreads();
    const int n = kLanes * dim;
    const float inverse = row_inverse_rms(s, n, &inv_s);
    // RmsUnit then FakeA8: the peak of x * inverse is RoundNearest(max |x| *
    // inverse), so the Prepare waves form the scaled, int8 round-tripped row
    float m = 0.0f;
    for (int g = 0; g < dim / 128; g++) m = fmaxf(m, red[g]);
    const float top = m * inverse;
    const float scale = top > 0.0f ? top / 127.0f : 1.0f;
    const float round = 1.0f / scale;
    if constexpr (HYPER) {
        const int g4 = n / 128;
        prepare_row_fake(s, n, 4, Act{a4v, a4s, a4s + g4}, 0, 0, inverse, round, scale);
        __syncthreads();
        for (int e = threadIdx.x; e < n / 16; e += kThreads)
            reinterpret_cast<uint4*>(act.values + (size_t)t * n)[e] = reinterpret_cast<const uint4*>(a4v)[e];
        if ((int)threadIdx.x < 2 * g4) {
            const int g = (int)threadIdx.x % g4;
            float* dst = (int)threadIdx.x < g4 ? act.scales : act.offsets;
            dst[(size_t)t * stride + g] = a4s[threadIdx.x];
        }
        const float y = phi_outputs(h.phi, hunit, a4v, a4s, a4s + g4, n, kPhiFirst, hprod, kPhiBase);
        float sv[kPer][kLanes];
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int c = col_of(q);
            if (c < dim) {
#pragma unroll
                for (int l = 0; l < kLanes; l++) sv[q][l] = s[l * dim + c];
            }
        }
        hyper_mix_row(h, t, y, hga, hgb, sv, hsn, hx, hsq, hpre, red, &inv_s);
    } else {
        prepare_row_fake(s, n, 4, act, stride, t, inverse, round, scale);
    }
}

// ----------------------------------------------------------- engram --

struct EngramArgs {
    const float* stage;        // [rows][10][dim]: row 9 the new value projection
    float* history;            // [slots][9][dim] of this site
    const int32_t* row_slot;
    const int32_t* run_start;  // first row of each row's run
    const int32_t* run_end;    // whether the row ends its run
    const float* taps;         // [4][dim]
    int dilation, dim;
    const float* input;
    const float* key;
    float* residual;
    float inverse_root;        // 1 / sqrt(dim)
    const float* norm_in;
    Act act;
    int stride;
};

// Row t's convolution input j (0..9): the slot's history followed by the
// value rows of its run (Engine.cs:2430-2437): sequence index (t - rs) + j.
__device__ __forceinline__ const float* engram_frame(const EngramArgs& a, int t, int j)
{
    const int rs = a.run_start[t];
    const int idx = (t - rs) + j;
    if (j == kEngramHistory) return a.stage + ((size_t)t * (kEngramHistory + 1) + kEngramHistory) * a.dim;
    if (idx < kEngramHistory) return a.history + ((size_t)a.row_slot[t] * kEngramHistory + idx) * a.dim;
    return a.stage + ((size_t)(rs + idx - kEngramHistory) * (kEngramHistory + 1) + kEngramHistory) * a.dim;
}

// The engram's convolution, RmsUnit of the input and the key, their Dot,
// alpha = Sigmoid(dot / sqrt(dim)) and residual += alpha * conv
// (Engine.cs:2437-2462), then RunAttentionBatch's CenteredRmsFakeA8 of the
// residual and its 2-bit Prepare.  Waves 0 and 1 run the two sums of squares
// at once; every sum is in the AVX2 tier's order.
__global__ __launch_bounds__(kThreads) void n3_engram_mix_kernel(EngramArgs a)
{
    __shared__ __align__(16) float ua[kMaxDim];
    __shared__ __align__(16) float ub[kMaxDim];
    __shared__ float inv[2];
    __shared__ float red[kWaves];
    __shared__ float alpha_s;
    const int t = blockIdx.x;
    const int dim = a.dim;
    const float* f[kEngramTaps];
#pragma unroll
    for (int j = 0; j < kEngramTaps; j++) f[j] = engram_frame(a, t, kEngramHistory - j * a.dilation);
    float tp[kPer][kEngramTaps], fr[kPer][kEngramTaps], xv[kPer], kv[kPer], rv[kPer], sn[kPer];
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = col_of(q);
        if (c < dim) {
#pragma unroll
            for (int j = 0; j < kEngramTaps; j++) {
                tp[q][j] = a.taps[(size_t)j * dim + c];
                fr[q][j] = f[j][c];
            }
            xv[q] = a.input[(size_t)t * dim + c];
            kv[q] = a.key[(size_t)t * dim + c];
            rv[q] = a.residual[(size_t)t * dim + c];
            sn[q] = a.norm_in[c];
        }
    }
    float cv[kPer];
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = col_of(q);
        if (c < dim) {
            float o = 0.0f;
#pragma unroll
            for (int j = 0; j < kEngramTaps; j++) o = o + tp[q][j] * fr[q][j];
            cv[q] = o;
            ua[c] = xv[q];
            ub[c] = kv[q];
        }
    }
    __syncthreads();
    // Ops.RmsUnit of the input (wave 0) and of the key (wave 1)
    if (threadIdx.x < 128) {
        const float* v = threadIdx.x < 64 ? ua : ub;
        const float sum = wave_v256_sum(v, v, dim);
        if ((threadIdx.x & 63) == 0) inv[threadIdx.x >> 6] = inverse_rms_of(sum, dim);
    }
    __syncthreads();
    const float ia = inv[0], ib = inv[1];
    for (int c = threadIdx.x; c < dim; c += kThreads) {
        ua[c] = ua[c] * ia;
        ub[c] = ub[c] * ib;
    }
    __syncthreads();
    // alpha = Sigmoid(Ops.Dot(unitA, unitB) / sqrt(dim))
    if (threadIdx.x < 64) {
        const float dot = wave_v256_sum(ua, ub, dim);
        if (threadIdx.x == 0) alpha_s = sigmoid_poly(dot * a.inverse_root);
    }
    __syncthreads();
    const float alpha = alpha_s;
    // the attention norm's FakeA8 peak with the residual (the scaled row
    // (1 + s) * r into ub, whose dot is done): max |v * inverse| is
    // RoundNearest(max |v| * inverse), so the Prepare waves form the int8
    // round trip themselves
    float peak = 0.0f;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = col_of(q);
        if (c < dim) {
            const float r = rv[q] + alpha * cv[q];
            a.residual[(size_t)t * dim + c] = r;
            ua[c] = r;
            const float v = (1.0f + sn[q]) * r;
            ub[c] = v;
            peak = fmaxf(peak, fabsf(v));
        }
    }
    peak = wave_max(peak);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = peak;
    __syncthreads();
    const float inverse = row_inverse_rms(ua, dim, &inv[0]);
    float m = red[0];
    for (int w = 1; w < kWaves; w++) m = fmaxf(m, red[w]);
    const float top = m * inverse;
    const float scale = top > 0.0f ? top / 127.0f : 1.0f;
    const float round = 1.0f / scale;
    prepare_row_fake(ub, dim, 2, a.act, a.stride, t, inverse, round, scale);
}

// ------------------------------------------------- attention epilogue --

// The slots' Q/K/V frames (the three-tap convolution's history) of a layer.
struct QkvHistArgs {
    float* history;  // [slots] x ([2][qw], [2][kw], [2][vw]), frame 1 the latest
    const float* raw;  // [rows][qw + kw + vw]: this step's projections
    const int32_t* row_slot;
    const int32_t* run_start;
    const int32_t* run_end;
    int qw, kw, vw;
};

// The run's last row moves its slot's Q/K/V frames on: frame 0 takes the row
// before it (the old frame 1 for a one-row run), frame 1 the row itself
// (Scalar.Taps3's history, TapsAndAttentionHeadsSingle).  qkv_hist_load reads
// the new frames (true when row t ends its run), qkv_hist_store writes them.
__device__ __forceinline__ bool qkv_hist_load(const QkvHistArgs& h, int t, float* hv0, float* hv1)
{
    if (h.run_end[t] == 0) return false;
    const int all = h.qw + h.kw + h.vw;
    const float* hist = h.history + (size_t)h.row_slot[t] * 2 * all;
    const bool run1 = t > h.run_start[t];
#pragma unroll
    for (int q = 0; q < kHistPer; q++) {
        const int c = col_of(q);
        if (c < all) {
            const int base = c < h.qw ? 0 : (c < h.qw + h.kw ? h.qw : h.qw + h.kw);
            const int width = c < h.qw ? h.qw : (c < h.qw + h.kw ? h.kw : h.vw);
            hv0[q] = run1 ? h.raw[(size_t)(t - 1) * all + c] : hist[2 * base + (c - base) + width];
            hv1[q] = h.raw[(size_t)t * all + c];
        }
    }
    return true;
}

__device__ __forceinline__ void qkv_hist_store(const QkvHistArgs& h, int t, const float* hv0, const float* hv1)
{
    const int all = h.qw + h.kw + h.vw;
    float* hist = h.history + (size_t)h.row_slot[t] * 2 * all;
#pragma unroll
    for (int q = 0; q < kHistPer; q++) {
        const int c = col_of(q);
        if (c < all) {
            const int base = c < h.qw ? 0 : (c < h.qw + h.kw ? h.qw : h.qw + h.kw);
            const int width = c < h.qw ? h.qw : (c < h.qw + h.kw ? h.kw : h.vw);
            hist[2 * base + (c - base)] = hv0[q];
            hist[2 * base + (c - base) + width] = hv1[q];
        }
    }
}

// On engram layers a run-end row moves its slot's engram history on
// (Engine.cs:2439): the nine frames before the sequence's end.
__device__ __forceinline__ void engram_hist_move(const EngramArgs& e, int t)
{
    if (!e.history || !e.run_end[t]) return;
    const int len = t - e.run_start[t] + 1;  // the run's length
    float* hist = e.history + (size_t)e.row_slot[t] * kEngramHistory * e.dim;
    for (int c = threadIdx.x; c < e.dim; c += kThreads) {
        float v[kEngramHistory];
#pragma unroll
        for (int j = 0; j < kEngramHistory; j++) {
            const int idx = len + j;  // sequence index of the new frame j
            v[j] = idx < kEngramHistory
                       ? hist[(size_t)idx * e.dim + c]
                       : e.stage[((size_t)(e.run_start[t] + idx - kEngramHistory) * (kEngramHistory + 1) +
                                  kEngramHistory) * e.dim + c];
        }
#pragma unroll
        for (int j = 0; j < kEngramHistory; j++) hist[(size_t)j * e.dim + c] = v[j];
    }
}

// Scalar.GateFakeA8 on row t of the attention output: x *= Sigmoid(gate),
// the fake int8 round trip at the row's peak, and the 2-bit Prepare of the
// output matmul.  Row t's Q/K/V frames and, on engram layers, its engram
// history move on here, after every row's attention and engram mix have read
// the old ones.
__global__ __launch_bounds__(kThreads) void n3_gate_kernel(const float* att, const float* gate, int n, Act act,
                                                           int stride, EngramArgs e, QkvHistArgs h)
{
    __shared__ float peak_g[kMaxDim / 128];
    const int t = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int g = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);  // wave g takes group g
    const int groups = n >> 7;
    // lane e holds elements e and e + 64 of the group, as hadamard_wave wants
    // them; the history's loads go out with the row's own
    float x0 = 0.0f, x1 = 0.0f, s0 = 0.0f, s1 = 0.0f;
    if (g < groups) {
        const size_t at = (size_t)t * n + g * 128 + lane;
        x0 = att[at];
        x1 = att[at + 64];
        s0 = gate[at];
        s1 = gate[at + 64];
    }
    float hv0[kHistPer], hv1[kHistPer];
    const bool hist_end = qkv_hist_load(h, t, hv0, hv1);
    if (g < groups) {
        x0 = x0 * sigmoid_poly(s0);
        x1 = x1 * sigmoid_poly(s1);
        const float m = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
        if (lane == 0) peak_g[g] = m;
    }
    __syncthreads();
    if (g < groups) {
        // Quant.FakeA8 at the row's peak (the maximum of the groups' maxima),
        // then the group's Hadamard and Prepare
        float peak = 0.0f;
        for (int j = 0; j < groups; j++) peak = fmaxf(peak, peak_g[j]);
        const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
        const float round = 1.0f / scale;
        float v0 = clamp_q(x0 * round) * scale;
        float v1 = clamp_q(x1 * round) * scale;
        hadamard_wave(v0, v1);
        prepare_group_wave(v0, v1, 2, act.values + (size_t)t * n + g * 128, act.scales + (size_t)t * stride + g,
                           act.offsets + (size_t)t * stride + g);
    }
    if (hist_end) qkv_hist_store(h, t, hv0, hv1);
    engram_hist_move(e, t);
}

// n3_gate_kernel and the output matmul in one launch, for steps of up to
// kGateOutRows rows: workgroup b computes output columns 16b .. 16b + 15 of
// every row.  Each workgroup forms the prepared activations itself
// (GateFakeA8 and the 2-bit Prepare, its waves taking the (row, group)
// pairs); wave g then takes group g of the workgroup's 16 weight rows
// (row-major 2-bit codes: element 4j + p in byte j, bits 2p) through four
// i8 MFMAs, one per plane, as the codebook decode kernels do, and the group
// dots D_g go into Scalar.MatMulRows' chain (Scalar.cs:146-192):
//   scaled = (HalfToSingle(norm[n][g]) * ByteScale) * scale[t][g]
//   acc += scaled * D_g;  bias += scaled * offset[t][g]   (g ascending)
//   y = acc - bias
// The Q/K/V and engram history moves of n3_gate_kernel are spread over the
// workgroups, an element each for the last waves' threads.
constexpr int kGateOutRows = 4;
constexpr int kMaxGroups = kMaxDim / 128;
typedef int v4i __attribute__((ext_vector_type(4)));

struct GateOutArgs {
    const uint16_t* norms;  // [columns][k / 128] fp16: the record's scales
    float* y;               // [rows][ldy]
    int ldy;
    uint32_t table;         // the 2-bit codebook's four level bytes
    float byte_scale;
    EngramArgs e;
    QkvHistArgs h;
};

__global__ __launch_bounds__(kThreads) void n3_gate_out_kernel(const uint8_t* codes, const float* att,
                                                               const float* gate, uint64_t h_rows_k, GateOutArgs a)
{
    __shared__ __align__(16) int8_t act[kGateOutRows * kMaxDim];  // [t][k], planes order within each group
    __shared__ float peak_g[kGateOutRows * kMaxGroups];
    __shared__ float g_scale[kGateOutRows * kMaxGroups], g_offset[kGateOutRows * kMaxGroups];
    __shared__ __align__(16) float pa[kGateOutRows * 16 * kMaxGroups], pb[kGateOutRows * 16 * kMaxGroups];
    const int rows = (int)(uint32_t)h_rows_k, k = (int)(h_rows_k >> 32);
    const int groups = k >> 7;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    // wave g < groups: lane l's MFMA B operand, bytes 8 * (l / 16) .. + 7 of
    // group g of weight row l % 16, and that row's group scale (lanes < 16)
    const int nr = lane & 15, kq = lane >> 4;
    const bool dots = wave < groups;
    uint2 code = make_uint2(0u, 0u);
    uint32_t norm = 0u;
    if (dots) {
        const size_t row = (size_t)blockIdx.x * 16 + nr;
        code = *reinterpret_cast<const uint2*>(codes + row * (k >> 2) + wave * 32 + kq * 8);
        if (lane < 16) norm = a.norms[row * groups + wave];
    }
    // the gate's (row, group) pairs: wave v takes v and v + kWaves; lane e
    // holds elements e and e + 64 of the group, as hadamard_wave wants them
    const int tasks = rows * groups;
    float x0[2], x1[2], s0[2], s1[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int task = wave + kWaves * u;
        if (task < tasks) {
            const int t = task / groups, gg = task - t * groups;
            const size_t at = (size_t)t * k + gg * 128 + lane;
            x0[u] = att[at];
            x1[u] = att[at + 64];
            s0[u] = gate[at];
            s1[u] = gate[at + 64];
        }
    }
    // the history moves: row t's element c for flat index t * width + c, a
    // run of `per` indices for each workgroup, from its last thread down
    const int hi = kThreads - 1 - (int)threadIdx.x;
    const int all = a.h.qw + a.h.kw + a.h.vw;
    const int qkv_per = (rows * all + (int)gridDim.x - 1) / (int)gridDim.x;
    const int qkv_e = (int)blockIdx.x * qkv_per + hi;
    const bool qkv_on = hi < qkv_per && qkv_e < rows * all;
    float hv0 = 0.0f, hv1 = 0.0f;
    float* qkv_dst = nullptr;
    int qkv_width = 0;
    if (qkv_on) {
        const int t = qkv_e / all, c = qkv_e - t * all;
        if (a.h.run_end[t] != 0) {
            const int base = c < a.h.qw ? 0 : (c < a.h.qw + a.h.kw ? a.h.qw : a.h.qw + a.h.kw);
            qkv_width = c < a.h.qw ? a.h.qw : (c < a.h.qw + a.h.kw ? a.h.kw : a.h.vw);
            qkv_dst = a.h.history + (size_t)a.h.row_slot[t] * 2 * all + 2 * base + (c - base);
            hv0 = t > a.h.run_start[t] ? a.h.raw[(size_t)(t - 1) * all + c] : qkv_dst[qkv_width];
            hv1 = a.h.raw[(size_t)t * all + c];
        }
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int task = wave + kWaves * u;
        if (task < tasks) {
            x0[u] = x0[u] * sigmoid_poly(s0[u]);
            x1[u] = x1[u] * sigmoid_poly(s1[u]);
            const float m = wave_max(fmaxf(fabsf(x0[u]), fabsf(x1[u])));
            if (lane == 0) peak_g[task] = m;
        }
    }
    __syncthreads();
    // Quant.FakeA8 at the row's peak, then the Hadamard and Prepare of the group
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int task = wave + kWaves * u;
        if (task < tasks) {
            const int t = task / groups, gg = task - t * groups;
            float peak = 0.0f;
            for (int j = 0; j < groups; j++) peak = fmaxf(peak, peak_g[t * groups + j]);
            const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
            const float round = 1.0f / scale;
            float v0 = clamp_q(x0[u] * round) * scale;
            float v1 = clamp_q(x1[u] * round) * scale;
            hadamard_wave(v0, v1);
            prepare_group_wave(v0, v1, 2, act + t * k + gg * 128, &g_scale[task], &g_offset[task]);
        }
    }
    __syncthreads();
    if (dots) {
        // D_g for tokens 0..3 (MFMA rows; rows of tokens >= rows read nothing)
        v4i d = {0, 0, 0, 0};
#pragma unroll
        for (int pl = 0; pl < 4; pl++) {
            long av = 0;
            if (nr < rows) av = *reinterpret_cast<const long*>(act + nr * k + wave * 128 + 32 * pl + 8 * kq);
            const uint32_t b0 = lut2((code.x >> (2 * pl)) & 0x03030303u, a.table);
            const uint32_t b1 = lut2((code.y >> (2 * pl)) & 0x03030303u, a.table);
            d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, (long)(((uint64_t)b1 << 32) | b0), d, 0, 0, 0);
        }
        // lane l < 16 holds D[t][row l] in d[t]
        if (lane < 16) {
            const float hb = ref_half_to_single(norm) * a.byte_scale;
            const int dv[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
            for (int t = 0; t < kGateOutRows; t++) {
                if (t < rows) {
                    const float scaled = hb * g_scale[t * groups + wave];
                    pa[(t * 16 + nr) * kMaxGroups + wave] = scaled * static_cast<float>(dv[t]);
                    pb[(t * 16 + nr) * kMaxGroups + wave] = scaled * g_offset[t * groups + wave];
                }
            }
        }
    }
    __syncthreads();
    if ((int)threadIdx.x < rows * 16) {
        const int i = threadIdx.x;
        const float4* ra = reinterpret_cast<const float4*>(pa + i * kMaxGroups);
        const float4* rb = reinterpret_cast<const float4*>(pb + i * kMaxGroups);
        const float4 a0 = ra[0], a1 = ra[1], b0 = rb[0], b1 = rb[1];
        const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const float bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
        float acc = 0.0f, bias = 0.0f;
#pragma unroll
        for (int gg = 0; gg < kMaxGroups; gg++) {
            if (gg < groups) {
                acc = acc + av[gg];
                bias = bias + bv[gg];
            }
        }
        a.y[(size_t)(i >> 4) * a.ldy + blockIdx.x * 16 + (i & 15)] = acc - bias;
    }
    if (qkv_dst) {
        qkv_dst[0] = hv0;
        qkv_dst[qkv_width] = hv1;
    }
    // engram: row t's column c, its nine frames
    const EngramArgs& e = a.e;
    if (e.history) {
        const int per = (rows * e.dim + (int)gridDim.x - 1) / (int)gridDim.x;
        const int f = (int)blockIdx.x * per + hi;
        if (hi < per && f < rows * e.dim) {
            const int t = f / e.dim, c = f - t * e.dim;
            if (e.run_end[t]) {
                const int len = t - e.run_start[t] + 1;  // the run's length
                float* hist = e.history + (size_t)e.row_slot[t] * kEngramHistory * e.dim;
                float v[kEngramHistory];
#pragma unroll
                for (int j = 0; j < kEngramHistory; j++) {
                    const int idx = len + j;  // sequence index of the new frame j
                    v[j] = idx < kEngramHistory
                               ? hist[(size_t)idx * e.dim + c]
                               : e.stage[((size_t)(e.run_start[t] + idx - kEngramHistory) * (kEngramHistory + 1) +
                                          kEngramHistory) * e.dim + c];
                }
#pragma unroll
                for (int j = 0; j < kEngramHistory; j++) hist[(size_t)j * e.dim + c] = v[j];
            }
        }
    }
}

// -------------------------------------------------------------- tail --

struct TailArgs {
    float* residual;
    const float* proj;
    const float* post_norm;
    float attn_gate;
    const float* pre_norm;
    const int32_t *perm_a, *perm_b;
    const float *d1, *d2, *b2, *d3, *d4, *w1a, *w1b, *w2a, *w2b, *w3a, *w3b, *cond_v, *cond_u;
    int dim, rows, cols;
    const float* stream;     // this layer's stream
    const float* mix;        // [rows][16]
    const float* input;      // u
    const float* post_gate;  // [rows][4]
    float* next;             // the next stream
    // the next layer's RmsFakeA8 + 4-bit Prepare (head_of == NULL), or the
    // head rows' PrepareHeadVectors + 4-bit Prepare into row head_of[t]
    const int32_t* head_of;
    const float* final_norm;
    Act act;
    int stride;
};

// The padded row stride of the condition weights' lane-major copies (dim % 64
// == 0): input[i] at (i % 4) * stride + i / 4, cond_v[8i + j] at
// ((i % 4) * 8 + j) * stride + i / 4.
__host__ __device__ constexpr int cond_stride(int dim) { return dim / 4 + 4; }

// The row stride of a transposed Kronecker left factor in LDS (16-byte aligned).
__host__ __device__ constexpr int krows_t(int rows) { return rows + 4; }

// Bytes of LDS n3_tail_kernel takes for a geometry.
size_t tail_lds_bytes(int dim, int rows, int cols)
{
    const size_t width = (size_t)rows * cols;
    return sizeof(float) * (2 * width + (size_t)rows * (cols + 4) + 2 * (size_t)dim + 36 * (size_t)cond_stride(dim) +
                            3 * (size_t)rows * krows_t(rows) + 3 * (size_t)cols * cols + (size_t)kLanes * dim +
                            32 * (size_t)v256_stride(kLanes * dim));
}

// HadamardMlp.ConditionWeights' Vector256 branch (Blocks.cs:1104-1125) by one
// wave, from the lane-major copies: lane 8k + j (k < 4, j < 8) accumulates
// fma(input[i], cond_v[8i + j], acc) over i = k (mod 4) ascending (dim % 4
// == 0: no remainder); weight j = (l0 + l1) + (l2 + l3); then Ops.Softmax's
// 8-wide branch (Ops.cs:269-276): e = Exp(w - max), total =
// Vector256.Sum(e), w = e * (1 / total).  Lane j < 8 returns weight j.
__device__ __forceinline__ float wave_condition_weights(const float* input_t, const float* cond_t, int dim)
{
    const int lane = threadIdx.x & 63;
    const int k = (lane >> 3) & 3;
    const int stride = cond_stride(dim);
    float acc = 0.0f;
    if (lane < 32) acc = lds_fma_chain(input_t + k * stride, cond_t + lane * stride, dim / 4, 0.0f);
    // lanes 0-7: their xor-partners 8, 16, 24 are lanes j + 8, j + 16, j + 24,
    // and xor-partners 1, 2, 4 span the eight weights
    const float a16 = lane_xor<16>(acc);
    const float w = (acc + lane_xor<8>(acc)) + (a16 + lane_xor<8>(a16));
    float peak = w;
    peak = fmaxf(peak, lane_xor<1>(peak));
    peak = fmaxf(peak, lane_xor<2>(peak));
    peak = fmaxf(peak, lane_xor<4>(peak));
    const float e = exp_poly(w - peak);
    const float p2 = e + lane_xor<1>(e);
    const float p4 = p2 + lane_xor<2>(p2);
    const float p8 = p4 + lane_xor<4>(p4);
    const float total = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(p8)));
    return e * (1.0f / total);
}

// Kron in LDS in the vectorised tiers' form (Blocks.cs:1243-1700): scratch[k][c]
// = sum_{i < active} left[i][k] z[i][c] (an FMA chain over i per (k, c)),
// then result[k][c] = sum_j scratch[k][j] right[j][c] (an FMA chain over j),
// for k < result_rows.  Thread u owns the four
// elements 4u .. 4u+3 (one k, four consecutive c; cols % 4 == 0) and runs
// their chains together; each step's operands are loaded 8 steps at a time.
// The passes are bound by the LDS reads, so the scalar operand of 4 steps
// comes in one 16-byte read as well: left is staged transposed (leftT[k][i],
// rows krows_t(rows) apart) and scratch rows are cols + 4 apart (both
// 16-byte aligned; kron_scratch floats in all).
__device__ __forceinline__ int kron_scratch(int rows, int cols) { return rows * (cols + 4); }

// The two chains of output element e0..e0+3 (row k = e0 / cols, columns c..c+3).
// active is a multiple of 8 (the caller zero-fills z's rows up to it: a
// zero product leaves a sum that starts at +0 unchanged).
__device__ __forceinline__ void kron_first(const float* z, int active, const float* left, int lt, int cols, int e0,
                                           float* scratch)
{
    const int k = e0 / cols, c = e0 - k * cols, ss = cols + 4;
    float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int i0 = 0; i0 < active; i0 += 8) {
        float lv[8];
        float4 zv[8];
        const float4 l0 = *reinterpret_cast<const float4*>(left + k * lt + i0);
        const float4 l1 = *reinterpret_cast<const float4*>(left + k * lt + i0 + 4);
        lv[0] = l0.x; lv[1] = l0.y; lv[2] = l0.z; lv[3] = l0.w;
        lv[4] = l1.x; lv[5] = l1.y; lv[6] = l1.z; lv[7] = l1.w;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            zv[u] = *reinterpret_cast<const float4*>(z + (i0 + u) * cols + c);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            sum.x = fmaf(lv[u], zv[u].x, sum.x);
            sum.y = fmaf(lv[u], zv[u].y, sum.y);
            sum.z = fmaf(lv[u], zv[u].z, sum.z);
            sum.w = fmaf(lv[u], zv[u].w, sum.w);
        }
    }
    float* srow = scratch + k * ss + c;
    srow[0] = sum.x;
    srow[1] = sum.y;
    srow[2] = sum.z;
    srow[3] = sum.w;
}

__device__ __forceinline__ void kron_second(const float* right, int cols, int e0, const float* scratch, float* result)
{
    const int k = e0 / cols, c = e0 - k * cols, ss = cols + 4;
    float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int j0 = 0; j0 < cols; j0 += 8) {
        float sv[8];
        float4 rv[8];
        const float4 s0 = *reinterpret_cast<const float4*>(scratch + k * ss + j0);
        const float4 s1 = *reinterpret_cast<const float4*>(scratch + k * ss + j0 + 4);
        sv[0] = s0.x; sv[1] = s0.y; sv[2] = s0.z; sv[3] = s0.w;
        sv[4] = s1.x; sv[5] = s1.y; sv[6] = s1.z; sv[7] = s1.w;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            rv[u] = *reinterpret_cast<const float4*>(right + (j0 + u) * cols + c);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            sum.x = fmaf(sv[u], rv[u].x, sum.x);
            sum.y = fmaf(sv[u], rv[u].y, sum.y);
            sum.z = fmaf(sv[u], rv[u].z, sum.z);
            sum.w = fmaf(sv[u], rv[u].w, sum.w);
        }
    }
    *reinterpret_cast<float4*>(result + e0) = sum;
}

__device__ __forceinline__ void kron_lds(const float* z, int active, const float* left, const float* right, int rows,
                                         int cols, int result_rows, float* scratch, float* result)
{
    const int e0 = 4 * (int)threadIdx.x;
    const bool on = e0 < result_rows * cols;
    if (on) kron_first(z, active, left, rows, cols, e0, scratch);
    __syncthreads();
    if (on) kron_second(right, cols, e0, scratch, result);
    __syncthreads();
}

// kron_lds by the first `nthreads` threads (a multiple of 64) with no block
// barrier: thread u owns the outputs 4f.. for f = u, u + nthreads, ...  A
// row's cols / 4 outputs are consecutive f in one wave (cols / 4 divides
// 64), which writes that row of scratch and then reads it, so a wave-scope
// fence orders the passes.  The caller synchronises before result is read.
__device__ __forceinline__ void kron_rows(const float* z, int active, const float* left, const float* right,
                                          int rows, int cols, int result_rows, float* scratch, float* result,
                                          int nthreads)
{
    const int total4 = result_rows * cols / 4;
    for (int f = threadIdx.x; f < total4; f += nthreads) kron_first(z, active, left, rows, cols, 4 * f, scratch);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int f = threadIdx.x; f < total4; f += nthreads) kron_second(right, cols, 4 * f, scratch, result);
}

// The end of a layer for one row, in RunLayerBatch's order
// (Engine.cs:2382-2397): Scalar.PostNormAdd of the attention output into the
// residual, HadamardMlp.Apply (Blocks.cs:1067-1101, scalar kernels, Scale 1),
// CombineDiff4x4's scalar branch (Ops.cs:800-812) into the next stream; then
// the next layer's RmsFakeA8 + 4-bit Prepare of that stream, or after the
// last layer PrepareHeadVectors (Engine.cs:920-928: Mix4 by 0.25,
// ZeroCenteredRms, FakeA8) + 4-bit Prepare for the head rows.  The Kronecker
// factors are staged in LDS.  The sums of PostNormAdd, the norms and the
// condition weights run in the AVX2 tier's order (wave_v256_sum,
// wave_condition_weights), and PostNormAdd adds with its Vector256 FMA.
// The first loads' pointers also travel as leading arguments, which gfx950
// preloads into SGPRs (kernarg preload; a struct argument is never
// preloaded), so those loads issue without an argument-segment round trip.
// LDS the fused tail's next-layer mix adds to tail_lds_bytes: the 4-bit
// prepared stream row (values, scales, offsets), the phi products of 8
// outputs and the mix kernel's two dim rows.
size_t tail_hyper_lds_bytes(int dim)
{
    const size_t n4 = (size_t)kLanes * dim, groups = n4 / 128;
    return 16 + n4 + sizeof(float) * (2 * groups + 2 * 8 * groups + 2 * (size_t)dim);
}

// HYPER: for a layer l < L - 1 of a step whose rows are one per slot (whose
// attention launch forms the residual-mix logits and their Sinkhorn), the
// workgroup goes on into layer l + 1's mix (h, as n3_hyper_kernel's row
// part): the next stream row stays in registers and its 4-bit prepared
// activations in LDS, with a copy in act for the attention launch.
template <bool HYPER>
__global__ __launch_bounds__(kThreads) void n3_tail_kernel(const float* h_proj, float* h_residual,
                                                           const float* h_post_norm, const float* h_pre_norm,
                                                           const float* h_mix, const float* h_post_gate, TailArgs a,
                                                           HyperArgs h)
{
    a.proj = h_proj;
    a.residual = h_residual;
    a.post_norm = h_post_norm;
    a.pre_norm = h_pre_norm;
    a.mix = h_mix;
    a.post_gate = h_post_gate;
    extern __shared__ __align__(16) float lds[];
    const int width = a.rows * a.cols, dim = a.dim, rr = a.rows * a.rows, cc = a.cols * a.cols, n4 = kLanes * dim;
    float* front = lds;               // width (>= the padded input)
    float* back = front + width;      // width
    float* scratch = back + width;    // kron_scratch
    float* res = scratch + kron_scratch(a.rows, a.cols);  // dim
    float* norm = res + dim;          // dim
    const int cs = cond_stride(dim), ts = v256_stride(n4);
    float* cvt = norm + dim;          // CondV, lane-major [32][cs]
    float* int_ = cvt + 32 * cs;      // the condition input, lane-major [4][cs]
    float* wl = int_ + 4 * cs;        // W1A, W2A, W3A
    const int lt = krows_t(a.rows);   // W1A, W2A, W3A transposed ([k][i], rows lt apart)
    float* wr = wl + 3 * a.rows * lt; // W1B, W2B, W3B
    float* ns = wr + 3 * cc;          // the next stream row, 4 * dim
    float* nst = ns + n4;             // its lane-major copy [32][ts]
    const int g4 = n4 / 128;
    // HYPER: the 4-bit prepared next stream row, 16-byte aligned
    int8_t* a4v = reinterpret_cast<int8_t*>(lds + ((int)(nst + 32 * ts - lds) + 3) / 4 * 4);
    float* a4s = reinterpret_cast<float*>(a4v + n4);          // its group scales, then offsets
    float* hprod = a4s + 2 * g4;                              // phi products [8][g4][2]
    float* hx = hprod + 2 * 8 * g4;                           // the mix kernel's rows
    float* hsq = hx + dim;
    __shared__ float weights[8];
    __shared__ float red[kWaves];
    __shared__ float inv_s;
    const int t = blockIdx.x;
    // every global load of the row up front
    float rv[kPer], pv[kPer], psv[kPer], prv[kPer], d1v[kPer], d4v[kPer], uv[kPer], sv[kPer][kLanes];
    float hsn[kPer], nsv[kPer][kLanes];  // HYPER: layer l + 1's NormIn, the next stream row
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = col_of(q);
        if (c < dim) {
            rv[q] = a.residual[(size_t)t * dim + c];
            pv[q] = a.proj[(size_t)t * dim + c];
            psv[q] = a.post_norm[c];
            prv[q] = a.pre_norm[c];
            d1v[q] = a.d1[c];
            d4v[q] = a.d4[c];
            uv[q] = a.input[(size_t)t * dim + c];
#pragma unroll
            for (int l = 0; l < kLanes; l++) sv[q][l] = a.stream[(size_t)t * n4 + l * dim + c];
            if constexpr (HYPER) hsn[q] = h.norm_in[c];
        }
    }
    float cu[kPer][8], d2v[kPer], b2v[kPer], d3v[kPer];
    int pa[kPer], pb[kPer];
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int n = col_of(q);
        if (n < width) {
#pragma unroll
            for (int j = 0; j < 8; j++) cu[q][j] = a.cond_u[j * width + n];
            d2v[q] = a.d2[n];
            b2v[q] = a.b2[n];
            d3v[q] = a.d3[n];
            pa[q] = a.perm_a[n];
            pb[q] = a.perm_b[n];
        }
    }
    // the row's lane mix and post gates (wave-uniform), for CombineDiff4x4
    float mix[16], pgate[kLanes];
#pragma unroll
    for (int e = 0; e < 16; e++) mix[e] = a.mix[t * 16 + e];
#pragma unroll
    for (int l = 0; l < kLanes; l++) pgate[l] = a.post_gate[t * kLanes + l];
    float cvv[kCondPer], wv[kPer][6];
#pragma unroll
    for (int q = 0; q < kCondPer; q++) {
        const int e = col_of(q);
        if (e < dim * 8) cvv[q] = a.cond_v[e];
    }
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int e = col_of(q);
        if (e < rr) {
            wv[q][0] = a.w1a[e];
            wv[q][1] = a.w2a[e];
            wv[q][2] = a.w3a[e];
        }
        if (e < cc) {
            wv[q][3] = a.w1b[e];
            wv[q][4] = a.w2b[e];
            wv[q][5] = a.w3b[e];
        }
    }
    // Scalar.PostNormAdd: residual += gate * ((1 + s) * x * (1 / rms(x))), x = the attention projection
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = col_of(q);
        if (c < dim) norm[c] = pv[q];
    }
    __syncthreads();
    float inverse = row_inverse_rms(norm, dim, &inv_s);
    // Ops.PostNormAdd's Vector256 branch: fma(gate, ((1 + s) * x) * inverse,
    // residual) over whole 8-blocks, the scalar expression on the rest
    const int blocks8 = dim & ~7;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = col_of(q);
        if (c < dim) {
            const float v = (1.0f + psv[q]) * pv[q] * inverse;
            rv[q] = c < blocks8 ? fmaf(a.attn_gate, v, rv[q]) : rv[q] + a.attn_gate * (1.0f + psv[q]) * pv[q] * inverse;
            res[c] = rv[q];
        }
    }
    __syncthreads();
    // HadamardMlp.Apply
    inverse = row_inverse_rms(res, dim, &inv_s);
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = col_of(q);
        if (c < dim) {
            const float v = (1.0f + prv[q]) * rv[q] * inverse;
            norm[c] = v;
            int_[(c & 3) * cs + (c >> 2)] = v;
        }
    }
    // no barrier: what follows writes CondV and the Kronecker factors from
    // registers and the first product's input from the thread's own norm[c];
    // int_ is read after the next one
#pragma unroll
    for (int q = 0; q < kCondPer; q++) {  // CondV for the condition weights
        const int e = col_of(q);
        if (e < dim * 8) cvt[(((e >> 3) & 3) * 8 + (e & 7)) * cs + (e >> 5)] = cvv[q];
    }
    // the Kronecker factors into LDS only now: stored earlier, their loads
    // (issued last) would hold up the two norm chains above
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int e = col_of(q);
        if (e < rr) {
            const int et = (e % a.rows) * lt + e / a.rows;
            wl[et] = wv[q][0];
            wl[a.rows * lt + et] = wv[q][1];
            wl[2 * a.rows * lt + et] = wv[q][2];
        }
        if (e < cc) {
            wr[e] = wv[q][3];
            wr[cc + e] = wv[q][4];
            wr[2 * cc + e] = wv[q][5];
        }
    }
    const int input_rows = (dim + a.cols - 1) / a.cols;
    const int output_rows = min(a.rows, (input_rows + 3) / 4 * 4);
    const int active_rows = (input_rows + 7) / 8 * 8;  // <= rows (rows % 8 == 0): zero rows past the input
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = col_of(q);
        if (c < active_rows * a.cols) front[c] = c < dim ? norm[c] * d1v[q] : 0.0f;
    }
    __syncthreads();
    // the last wave forms the condition weights while the others run the
    // first Kronecker product, which does not depend on them
    constexpr int kKronThreads = (kWaves - 1) * 64;
    if (threadIdx.x >= kKronThreads) {
        const float w = wave_condition_weights(int_, cvt, dim);
        if (threadIdx.x - kKronThreads < 8) weights[threadIdx.x - kKronThreads] = w;
    } else {
        kron_rows(front, active_rows, wl, wr, lt, a.cols, a.rows, scratch, back, kKronThreads);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kPer; q++) {  // Scalar.PermuteModulateActivate
        const int n = col_of(q);
        if (n < width) {
            float condition = 1.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) condition = condition + weights[j] * cu[q][j];
            const float v = d2v[q] * condition * back[pa[q]] + b2v[q];
            front[n] = v * sigmoid_poly(v);
        }
    }
    __syncthreads();
    kron_lds(front, a.rows, wl + a.rows * lt, wr + cc, lt, a.cols, a.rows, scratch, back);
#pragma unroll
    for (int q = 0; q < kPer; q++) {  // Scalar.PermuteScale
        const int n = col_of(q);
        if (n < width) front[n] = back[pb[q]] * d3v[q];
    }
    __syncthreads();
    kron_lds(front, a.rows, wl + 2 * a.rows * lt, wr + 2 * cc, lt, a.cols, output_rows, scratch, back);
    // Scalar.AccumulateOutput, then CombineDiff4x4 into the next stream
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = col_of(q);
        if (c < dim) {
            const float x = rv[q] + 1.0f * (back[c] * d4v[q]);
            const float y = x - uv[q];
#pragma unroll
            for (int l = 0; l < kLanes; l++) {
                const float o = pgate[l] * y + mix[4 * l] * sv[q][0] + mix[4 * l + 1] * sv[q][1] +
                                mix[4 * l + 2] * sv[q][2] + mix[4 * l + 3] * sv[q][3];
                const int i = l * dim + c;
                a.next[(size_t)t * n4 + i] = o;
                if constexpr (HYPER) nsv[q][l] = o;
                ns[i] = o;
                nst[(i & 31) * ts + (i >> 5)] = o;
            }
        }
    }
    __syncthreads();
    // HYPER: layer l + 1's phi rows, 4 pre and 4 post (the attention launch
    // forms the 16 residual-mix ones); their codes and affine maps load under
    // the next layer's RmsFakeA8 and Prepare
    constexpr int kPhiFirst[4] = {0, 4, 8, 8};
    constexpr int kPhiBase = 8 * 64;  // waves 8.. take the units: wave 0 sums the squares first
    PhiUnit hunit{};
    float hga = 0.0f, hgb = 0.0f;
    if constexpr (HYPER) {
        hunit = phi_load(h.phi, n4, 0, kPhiFirst, kPhiBase);
        phi_affine(h, hga, hgb);
    }
    if (!a.head_of) {  // the next layer's RmsFakeA8 and 4-bit Prepare
        // RmsUnit then FakeA8 with one barrier: the peak of x * inverse is
        // RoundNearest(max |x| * inverse) (inverse > 0 and rounding is
        // monotone), so the row's max |x| is taken with the squares, before
        // the chain, and the scaling and the int8 round trip run inside the
        // Prepare waves
        float peak_x = 0.0f;
        for (int c = threadIdx.x; c < n4; c += kThreads) peak_x = fmaxf(peak_x, fabsf(ns[c]));
        peak_x = wave_max(peak_x);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = peak_x;
        if (threadIdx.x < 64) {
            const float sum = wave_v256_squares(nst, n4);
            if (threadIdx.x == 0) inv_s = inverse_rms_of(sum, n4);
        }
        __syncthreads();
        inverse = inv_s;
        float m = red[0];
        for (int w = 1; w < kWaves; w++) m = fmaxf(m, red[w]);
        const float peak = m * inverse;
        const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
        const float round = 1.0f / scale;
        if constexpr (HYPER) {
            prepare_row_fake(ns, n4, 4, Act{a4v, a4s, a4s + g4}, 0, 0, inverse, round, scale);
            __syncthreads();
            // and into the row's global copy, which layer l + 1's attention
            // launch reads for the residual-mix logits
            for (int e = threadIdx.x; e < n4 / 16; e += kThreads)
                reinterpret_cast<uint4*>(a.act.values + (size_t)t * n4)[e] = reinterpret_cast<const uint4*>(a4v)[e];
            if ((int)threadIdx.x < 2 * g4) {
                const int g = (int)threadIdx.x % g4;
                float* dst = threadIdx.x < g4 ? a.act.scales : a.act.offsets;
                dst[(size_t)t * a.stride + g] = a4s[threadIdx.x];
            }
            const float y = phi_outputs(h.phi, hunit, a4v, a4s, a4s + g4, n4, kPhiFirst, hprod, kPhiBase);
            __shared__ float hpre[4];
            hyper_mix_row(h, t, y, hga, hgb, nsv, hsn, hx, hsq, hpre, red, &inv_s);
        } else {
            prepare_row_fake(ns, n4, 4, a.act, a.stride, t, inverse, round, scale);
        }
        return;
    }
    const int head = a.head_of[t];
    if (head < 0) return;
    // the scaled row (1 + s) * x into res with its peak: FakeA8's peak of
    // v * inverse is RoundNearest(max |v| * inverse), so the Prepare waves
    // form the int8 round trip themselves
    float peak_h = 0.0f;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = col_of(q);
        if (c < dim) {
            const float x = 0.25f * ns[c] + 0.25f * ns[dim + c] + 0.25f * ns[2 * dim + c] + 0.25f * ns[3 * dim + c];
            norm[c] = x;
            const float v = (1.0f + a.final_norm[c]) * x;
            res[c] = v;
            peak_h = fmaxf(peak_h, fabsf(v));
        }
    }
    peak_h = wave_max(peak_h);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = peak_h;
    __syncthreads();
    inverse = row_inverse_rms(norm, dim, &inv_s);
    float m = red[0];
    for (int w = 1; w < kWaves; w++) m = fmaxf(m, red[w]);
    const float top = m * inverse;
    const float scale = top > 0.0f ? top / 127.0f : 1.0f;
    const float round = 1.0f / scale;
    prepare_row_fake(res, dim, 4, a.act, a.stride, head, inverse, round, scale);
}

}  // namespace
}  // namespace nhip

using namespace nhip;

// ------------------------------------------------------------- model --

namespace {

struct N3Layer {
    const float *norm_in = nullptr, *q_taps = nullptr, *k_taps = nullptr, *v_taps = nullptr, *q_norm = nullptr,
                *k_norm = nullptr, *post_norm = nullptr, *pre_hada = nullptr;
    nhip_weights *q = nullptr, *k = nullptr, *v = nullptr, *gate = nullptr, *out = nullptr;
    nhip_weights* qkvg = nullptr;  // Q, K, V and Gate stacked by rows (the context's own)
    const uint8_t* out_raw = nullptr;  // Out's archive bytes on the device: row-major codes, then the norms
    const uint8_t* qkvg_raw[4] = {};   // Q, K, V and Gate's, the same way
    float attn_gate = 0.0f;
    const float *d1 = nullptr, *d2 = nullptr, *b2 = nullptr, *d3 = nullptr, *d4 = nullptr, *w1a = nullptr,
                *w1b = nullptr, *w2a = nullptr, *w2b = nullptr, *w3a = nullptr, *w3b = nullptr, *cond_v = nullptr,
                *cond_u = nullptr;
};

struct N3Site {
    const uint8_t* tables = nullptr;
    int table_rows = 0, table_cols = 0, table_bits = 0;
    nhip_weights *key = nullptr, *value = nullptr;
    nhip_weights* key_value = nullptr;  // Key and Value stacked by rows (the context's own)
    const float* taps = nullptr;
};

}  // namespace

struct nhip_ctx {
    const nhip_model* model = nullptr;
    // geometry (Model.cs:65-121)
    int vocab = 0, dim = 0, heads = 0, kv = 0, layers = 0, qk = 0, vd = 0, hada_rows = 0, hada_cols = 0, window = 0;
    int engram_slots = 0, engram_sub = 0, engram_tables = 0, dilation = 0, order_count = 0, orders[4] = {};
    int site_count = 0, sites[16] = {};
    uint64_t global_mask = 0;
    int slots = 0, capacity = 0, max_rows = 0, max_chunks = 0;
    // weights
    nhip_weights* embedding = nullptr;
    const uint8_t* embedding_raw = nullptr;
    int embedding_bits = 4;
    Book book2{}, book4{};
    std::vector<N3Layer> layer;
    const float *a_pre = nullptr, *a_post = nullptr, *a_res = nullptr, *b_pre = nullptr, *b_post = nullptr,
                *b_res = nullptr;
    nhip_weights *phi_pre = nullptr, *phi_post = nullptr, *phi_res = nullptr;
    const uint8_t* phi_raw[3] = {nullptr, nullptr, nullptr};  // their archive bytes on the device
    int32_t *perm_a = nullptr, *perm_b = nullptr;
    std::vector<N3Site> site;
    const float* final_norm = nullptr;
    // per-slot state
    int8_t *keys = nullptr, *values = nullptr;
    float *key_scales = nullptr, *value_scales = nullptr;
    float *qkv_hist = nullptr, *engram_hist = nullptr, *snap_qkv = nullptr, *snap_engram = nullptr;
    std::vector<int32_t> len, marked, prev, snap_prev;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    // scratch for max_rows rows (stream_a holds the embedding, the layers
    // alternate between the two stream buffers)
    float *stream_a = nullptr, *stream_b = nullptr, *normed = nullptr, *input = nullptr, *residual = nullptr,
          *raw = nullptr, *gate = nullptr, *att = nullptr, *proj = nullptr, *key = nullptr, *stage = nullptr,
          *ein = nullptr, *post_gate = nullptr, *mix = nullptr, *qs = nullptr, *logits = nullptr, *act_s = nullptr,
          *act_o = nullptr, *act4_s = nullptr, *act4_o = nullptr;
    int8_t *act_v = nullptr, *act4_v = nullptr, *q8 = nullptr;  // act4: the stream's 4-bit Prepare (phi input)
    int32_t* d_in = nullptr;  // the per-row inputs of a step, kInSections x max_rows, then the engram rows
    int32_t* h_in = nullptr;  // their pinned host staging
    void* attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    void* topk_ws = nullptr;
    size_t topk_ws_bytes = 0;
    int32_t *d_topk_idx = nullptr, *d_argmax = nullptr;
    float* d_topk_lp = nullptr;
    size_t tail_lds = 0;
    size_t tail_hyper_lds = 0;  // 0: the fused tail + next-layer mix does not fit
    hipStream_t stream_h = nullptr;
    struct Graph {
        int rows, heads, k;
        bool argmax, single_runs;
        hipGraphExec_t exec;
    };
    std::vector<Graph> graphs;  // captured steps, by their shape
    std::vector<void*> allocations;
    std::vector<nhip_weights*> stacked;  // the stacked matrices above
};

namespace {

// per-row step inputs: token, slot, position, attention span of the global
// layers (first, count) and of the sliding-window layers, the row's index
// among the head rows (-1: none), the first row of the row's run, whether
// the row ends its run
enum {
    kInTokens, kInSlots, kInPos, kInFirst, kInCount, kInFirstW, kInCountW, kInHeadOf, kInRunStart, kInRunEnd,
    kInSections
};

int32_t* in(nhip_ctx* c, int32_t* base, int section) { return base + (size_t)section * c->max_rows; }
int32_t* in_erows(nhip_ctx* c, int32_t* base) { return base + (size_t)kInSections * c->max_rows; }

template <typename T>
int32_t ctx_alloc(nhip_ctx* c, T** p, size_t count)
{
    void* v = nullptr;
    NHIP_CHECK_HIP(hipMalloc(&v, std::max<size_t>(count * sizeof(T), 256)));
    NHIP_CHECK_HIP(hipMemset(v, 0, std::max<size_t>(count * sizeof(T), 256)));
    c->allocations.push_back(v);
    *p = static_cast<T*>(v);
    return NHIP_OK;
}

// Codebook records of one format and K stacked by rows into one matrix the
// context owns (Q, K, V and Gate; an engram site's Key and Value): they
// share their activations, and each output row keeps its own chain, so one
// decode launch with split outputs computes what MatMulBatch's jobs do.
int32_t stack_rows(nhip_ctx* c, const int* records, int parts, nhip_weights** out)
{
    nhip_codebook book2{}, book4{};
    int32_t rc = nhip_model_codebooks(c->model, &book2, &book4);
    if (rc) return rc;
    int rows = 0, cols = 0, bits = 0;
    for (int k = 0; k < parts; k++) {
        nhip_record_info ri{};
        if ((rc = nhip_model_record(c->model, records[k], &ri))) return rc;
        NHIP_REQUIRE(k == 0 || ((int)ri.shape[1] == cols && (int)ri.bits == bits), "stacked records differ in K or "
                     "format");
        rows += (int)ri.shape[0];
        cols = (int)ri.shape[1];
        bits = (int)ri.bits;
    }
    const size_t row_bytes = (size_t)cols * bits / 8, groups = (size_t)cols / 128;
    std::vector<uint8_t> codes((size_t)rows * row_bytes);
    std::vector<uint16_t> norms((size_t)rows * groups);
    size_t r0 = 0;
    for (int k = 0; k < parts; k++) {
        nhip_record_info ri{};
        nhip_model_record(c->model, records[k], &ri);
        const size_t n = ri.shape[0];
        const uint8_t* raw = nhip_model_raw(c->model, records[k]);  // the indices, then the fp16 norms
        NHIP_REQUIRE(raw, "record %d has no raw copy", records[k]);
        NHIP_CHECK_HIP(hipMemcpy(codes.data() + r0 * row_bytes, raw, n * row_bytes, hipMemcpyDeviceToHost));
        NHIP_CHECK_HIP(hipMemcpy(norms.data() + r0 * groups, raw + n * row_bytes, n * groups * 2,
                                 hipMemcpyDeviceToHost));
        r0 += n;
    }
    const nhip_cq cq{codes.data(), norms.data(), bits == 2 ? &book2 : &book4, rows, cols, bits};
    if ((rc = weights_cq_create_internal(&cq, out))) return rc;
    c->stacked.push_back(*out);
    return NHIP_OK;
}

// Model.Open's reader over the archive's records, in order (Model.cs:307-371).
struct RecordCursor {
    const nhip_model* m;
    int next = 0, count = 0;
    int last = -1;  // the record quant() took last
    int32_t status = NHIP_OK;
    nhip_record_info info(int i)
    {
        nhip_record_info r{};
        nhip_model_record(m, i, &r);
        return r;
    }
    int take(int dtype_a, int dtype_b, const char* what)
    {
        if (status) return -1;
        if (next >= count) {
            set_error("archive ends before its %s", what);
            status = NHIP_ERR_FORMAT;
            return -1;
        }
        const nhip_record_info r = info(next);
        if (r.dtype != dtype_a && r.dtype != dtype_b) {
            set_error("record %d: %s expected (dtype %d)", next, what, r.dtype);
            status = NHIP_ERR_FORMAT;
            return -1;
        }
        return next++;
    }
    nhip_weights* quant(int bits, int rows, int cols, const char* what)
    {
        const int i = take(NHIP_CACT_CQ, NHIP_CACT_CQ, what);
        if (i < 0) return nullptr;
        const nhip_record_info r = info(i);
        if ((bits && (int)r.bits != bits) || (rows && (int)r.shape[0] != rows) || (cols && (int)r.shape[1] != cols)) {
            set_error("record %d (%s): %ux%u %u-bit, expected %dx%d %d-bit", i, what, r.shape[0], r.shape[1], r.bits, rows,
                      cols, bits);
            status = NHIP_ERR_FORMAT;
            return nullptr;
        }
        last = i;
        return nhip_model_weights(m, i);
    }
    const float* dense(size_t elements, const char* what)
    {
        const int i = take(NHIP_CACT_FP16, NHIP_CACT_FP32, what);
        if (i < 0) return nullptr;
        const nhip_record_info r = info(i);
        size_t n = 1;
        for (int d = 0; d < r.ndim; d++) n *= r.shape[d];
        if (elements && n != elements) {
            set_error("record %d (%s): %zu elements, expected %zu", i, what, n, elements);
            status = NHIP_ERR_FORMAT;
            return nullptr;
        }
        return nhip_model_dense(m, i);
    }

    // A dense record of `first` or `second` elements, of which the engine
    // reads the first `first` (D1 and D4 are stored MLP-width in Needle 3
    // archives, tools/golden.py:186-195, and read over the hidden width,
    // Blocks.cs:1135 ScaleInput and :1216 AccumulateOutput).
    const float* dense_either(size_t first, size_t second, const char* what)
    {
        const int i = take(NHIP_CACT_FP16, NHIP_CACT_FP32, what);
        if (i < 0) return nullptr;
        const nhip_record_info r = info(i);
        size_t n = 1;
        for (int d = 0; d < r.ndim; d++) n *= r.shape[d];
        if (n != first && n != second) {
            set_error("record %d (%s): %zu elements, expected %zu or %zu", i, what, n, first, second);
            status = NHIP_ERR_FORMAT;
            return nullptr;
        }
        return nhip_model_dense(m, i);
    }
};

int32_t load_model(nhip_ctx* c)
{
    uint32_t h[48];
    float theta = 0.0f;
    int32_t records = 0;
    int32_t rc = nhip_model_info(c->model, h, &theta, &records);
    if (rc) return rc;
    c->vocab = (int)h[5];
    c->dim = (int)h[7];
    c->heads = (int)h[8];
    c->kv = (int)h[9];
    c->layers = (int)h[10];
    c->qk = (int)h[11];
    c->vd = (int)h[12];
    const int hada_n = (int)h[14];
    int bl = 0;
    for (uint32_t v = (uint32_t)(hada_n - 1); v; v >>= 1) bl++;
    c->hada_rows = hada_n > 0 ? 1 << (bl / 2) : 0;
    c->hada_cols = c->hada_rows ? hada_n / c->hada_rows : 0;
    c->window = (int)h[16];
    c->global_mask = (uint64_t)h[17] | ((uint64_t)h[18] << 32);
    c->engram_slots = (int)h[20];
    c->engram_sub = (int)h[21];
    c->engram_tables = (int)h[22];
    c->dilation = (int)h[24];
    c->order_count = (int)h[26];
    for (int i = 0; i < 4; i++) c->orders[i] = (int)h[27 + i];
    c->site_count = (int)h[31];
    for (int i = 0; i < 16; i++) c->sites[i] = (int)h[32 + i];
    // Model.Open's geometry requirements (Model.cs:326-331), plus this
    // engine's limits
    NHIP_REQUIRE(c->qk == 48 && c->vd == 64 && h[15] == 4, "head geometry qk %d v %d lanes %u; needs 48 / 64 / 4", c->qk,
                 c->vd, h[15]);
    NHIP_REQUIRE(h[19] == 3 && (c->site_count == 0 || h[23] == 4) && c->dim % 128 == 0 && c->dim <= 1024,
                 "conv taps %u, engram taps %u, dim %d (a multiple of 128 up to 1024)", h[19], h[23], c->dim);
    NHIP_REQUIRE(c->hada_cols % 8 == 0 && 64 % (c->hada_cols / 4) == 0 && c->hada_rows % 8 == 0 &&
                     c->hada_rows * c->hada_cols == hada_n && hada_n >= c->dim,
                 "MLP size %d must split into rows x cols (cols divisible by 8) covering dim %d", hada_n, c->dim);
    NHIP_REQUIRE(c->heads * c->qk + c->kv * (c->qk + c->vd) <= kHistPer * kThreads, "Q/K/V width %d above %d",
                 c->heads * c->qk + c->kv * (c->qk + c->vd), kHistPer * kThreads);
    NHIP_REQUIRE(c->heads > 0 && c->kv > 0 && c->heads % c->kv == 0 && c->heads * c->vd <= 1024 &&
                     (c->heads * c->vd) % 128 == 0,
                 "heads %d / kv %d (heads * 64 a multiple of 128 up to 1024)", c->heads, c->kv);
    NHIP_REQUIRE(c->site_count >= 0 && c->site_count <= 16 && c->order_count >= 0 && c->order_count <= 4,
                 "engram sites %d, orders %d", c->site_count, c->order_count);
    // EngramHashRowsBatch reads an n-gram's tokens from the run and the slot's
    // two carried tokens, so orders run 1..3; every site needs an order.
    NHIP_REQUIRE(c->site_count == 0 || c->order_count >= 1, "engram sites %d with no n-gram orders", c->site_count);
    for (int o = 0; o < c->order_count; o++)
        NHIP_REQUIRE(c->orders[o] >= 1 && c->orders[o] <= 3, "engram order %d is %d (1..3)", o, c->orders[o]);
    NHIP_REQUIRE(c->site_count == 0 || (c->engram_tables % std::max(c->order_count, 1) == 0 &&
                                       c->engram_tables * c->engram_sub == c->dim && c->engram_sub % 128 == 0 &&
                                       c->engram_slots > 0 && c->dilation >= 1 && 3 * c->dilation <= kEngramHistory),
                 "engram geometry: %d tables x %d columns, %d slots, dilation %d", c->engram_tables, c->engram_sub,
                 c->engram_slots, c->dilation);
    nhip_codebook b2, b4;
    nhip_model_codebooks(c->model, &b2, &b4);
    std::memcpy(c->book2.levels, b2.levels, sizeof(b2.levels));
    std::memcpy(c->book4.levels, b4.levels, sizeof(b4.levels));
    const int d = c->dim, qw = c->heads * c->qk, kw = c->kv * c->qk, vw = c->kv * c->vd, ow = c->heads * c->vd;
    const size_t width = (size_t)c->hada_rows * c->hada_cols;
    RecordCursor r{c->model, 0, records};
    {
        const int i = r.take(NHIP_CACT_CQ, NHIP_CACT_CQ, "embedding");
        if (i >= 0) {
            nhip_record_info ri = r.info(i);
            NHIP_REQUIRE(ri.bits == 4 && (int)ri.shape[1] == d && (int)ri.shape[0] == c->vocab,
                         "embedding %ux%u %u-bit, expected %dx%d 4-bit", ri.shape[0], ri.shape[1], ri.bits, c->vocab, d);
            c->embedding = nhip_model_weights(c->model, i);
            c->embedding_raw = nhip_model_raw(c->model, i);
        }
    }
    c->layer.resize(c->layers);
    for (int l = 0; l < c->layers && !r.status; l++) {
        N3Layer& w = c->layer[l];
        w.norm_in = r.dense(d, "NormIn");
        int qkvg_records[4];
        w.q = r.quant(2, qw, d, "Q");
        qkvg_records[0] = r.last;
        w.k = r.quant(2, kw, d, "K");
        qkvg_records[1] = r.last;
        w.v = r.quant(2, vw, d, "V");
        qkvg_records[2] = r.last;
        w.q_taps = r.dense((size_t)3 * qw, "QTaps");
        w.k_taps = r.dense((size_t)3 * kw, "KTaps");
        w.v_taps = r.dense((size_t)3 * vw, "VTaps");
        w.q_norm = r.dense(c->qk, "QNorm");
        w.k_norm = r.dense(c->qk, "KNorm");
        w.gate = r.quant(2, ow, d, "Gate");
        qkvg_records[3] = r.last;
        if (!r.status && (rc = stack_rows(c, qkvg_records, 4, &w.qkvg))) return rc;
        for (int m = 0; m < 4 && !r.status; m++) w.qkvg_raw[m] = nhip_model_raw(c->model, qkvg_records[m]);
        w.out = r.quant(2, d, ow, "Out");
        w.out_raw = r.status ? nullptr : nhip_model_raw(c->model, r.last);
        w.post_norm = r.dense(d, "PostNorm");
        const float* g = r.dense(1, "AttnGate");
        if (g) {  // LayerWeights: AttnGate = 1 / (1 + MathF.Exp(-x)), once, with the host libm
            float x = 0.0f;
            NHIP_CHECK_HIP(hipMemcpy(&x, g, sizeof(float), hipMemcpyDeviceToHost));
            w.attn_gate = 1.0f / (1.0f + std::exp(-x));
        }
        w.pre_hada = r.dense(d, "PreHada");
        w.d1 = r.dense_either(d, width, "D1");
        w.d2 = r.dense(width, "D2");
        w.b2 = r.dense(width, "B2");
        w.d3 = r.dense(width, "D3");
        w.d4 = r.dense_either(d, width, "D4");
        w.w1a = r.dense((size_t)c->hada_rows * c->hada_rows, "W1A");
        w.w1b = r.dense((size_t)c->hada_cols * c->hada_cols, "W1B");
        w.w2a = r.dense((size_t)c->hada_rows * c->hada_rows, "W2A");
        w.w2b = r.dense((size_t)c->hada_cols * c->hada_cols, "W2B");
        w.w3a = r.dense((size_t)c->hada_rows * c->hada_rows, "W3A");
        w.w3b = r.dense((size_t)c->hada_cols * c->hada_cols, "W3B");
        w.cond_v = r.dense((size_t)d * 8, "CondV");
        w.cond_u = r.dense(8 * width, "CondU");
    }
    c->a_pre = r.dense(c->layers, "APre");
    c->a_post = r.dense(c->layers, "APost");
    c->a_res = r.dense(c->layers, "ARes");
    c->b_pre = r.dense((size_t)c->layers * 4, "BPre");
    c->b_post = r.dense((size_t)c->layers * 4, "BPost");
    c->b_res = r.dense((size_t)c->layers * 16, "BRes");
    c->phi_pre = r.quant(4, c->layers * 4, 4 * d, "PhiPre");
    c->phi_raw[0] = r.status ? nullptr : nhip_model_raw(c->model, r.next - 1);
    c->phi_post = r.quant(4, c->layers * 4, 4 * d, "PhiPost");
    c->phi_raw[1] = r.status ? nullptr : nhip_model_raw(c->model, r.next - 1);
    c->phi_res = r.quant(4, c->layers * 16, 4 * d, "PhiRes");
    c->phi_raw[2] = r.status ? nullptr : nhip_model_raw(c->model, r.next - 1);
    const float* pa = r.dense(width, "PermA");
    const float* pb = r.dense(width, "PermB");
    c->site.resize(c->site_count);
    for (int s = 0; s < c->site_count && !r.status; s++) {
        N3Site& st = c->site[s];
        const int i = r.take(NHIP_CACT_CQ, NHIP_CACT_CQ, "engram tables");
        if (i >= 0) {
            const nhip_record_info ri = r.info(i);
            st.tables = nhip_model_raw(c->model, i);
            st.table_rows = (int)ri.shape[0];
            st.table_cols = (int)ri.shape[1];
            st.table_bits = (int)ri.bits;
            NHIP_REQUIRE(st.table_cols == c->engram_sub && st.table_rows >= c->engram_tables * c->engram_slots,
                         "engram tables %ux%u for %d tables of %d slots x %d", ri.shape[0], ri.shape[1], c->engram_tables,
                         c->engram_slots, c->engram_sub);
        }
        int kv_records[2];
        st.key = r.quant(2, d, d, "engram Key");
        kv_records[0] = r.last;
        st.value = r.quant(2, d, d, "engram Value");
        kv_records[1] = r.last;
        if (!r.status && (rc = stack_rows(c, kv_records, 2, &st.key_value))) return rc;
        st.taps = r.dense((size_t)kEngramTaps * d, "engram Taps");
    }
    c->final_norm = r.dense(d, "FinalNorm");
    if (r.status) return r.status;
    int32_t rc2;
    if ((rc2 = ctx_alloc(c, &c->perm_a, width)) || (rc2 = ctx_alloc(c, &c->perm_b, width))) return rc2;
    // HyperConnections' permutations (stored as floats, Model.cs:168-169):
    // every index must address the MLP's width
    std::vector<float> pf(width);
    std::vector<int32_t> pi(width);
    for (int k = 0; k < 2; k++) {
        NHIP_CHECK_HIP(hipMemcpy(pf.data(), k ? pb : pa, width * sizeof(float), hipMemcpyDeviceToHost));
        for (size_t i = 0; i < width; i++) {
            NHIP_REQUIRE(pf[i] >= 0.0f && pf[i] < (float)width && pf[i] == (float)(int32_t)pf[i],
                         "permutation %c entry %zu (%g) outside [0, %zu)", k ? 'B' : 'A', i, (double)pf[i], width);
            pi[i] = (int32_t)pf[i];
        }
        NHIP_CHECK_HIP(hipMemcpy(k ? c->perm_b : c->perm_a, pi.data(), width * sizeof(int32_t), hipMemcpyHostToDevice));
    }
    return NHIP_OK;
}

int32_t alloc_state(nhip_ctx* c)
{
    const int d = c->dim, R = c->max_rows, qw = c->heads * c->qk, kw = c->kv * c->qk, vw = c->kv * c->vd,
              ow = c->heads * c->vd, all = qw + kw + vw, sw = kLanes * d;
    const size_t cells = (size_t)c->layers * c->slots * c->capacity;
    const size_t hist = (size_t)c->layers * c->slots * 2 * all;
    const size_t ehist = (size_t)std::max(c->site_count, 1) * c->slots * kEngramHistory * d;
    const int stride4 = (sw / 128 + 7) / 8 * 8;
    int32_t rc;
    if ((rc = ctx_alloc(c, &c->keys, cells * kw)) || (rc = ctx_alloc(c, &c->values, cells * vw)) ||
        (rc = ctx_alloc(c, &c->key_scales, cells * c->kv)) || (rc = ctx_alloc(c, &c->value_scales, cells * c->kv)) ||
        (rc = ctx_alloc(c, &c->qkv_hist, hist)) || (rc = ctx_alloc(c, &c->snap_qkv, hist)) ||
        (rc = ctx_alloc(c, &c->engram_hist, ehist)) || (rc = ctx_alloc(c, &c->snap_engram, ehist)) ||
        (rc = ctx_alloc(c, &c->rope_cos, (size_t)c->capacity * c->qk / 2)) ||
        (rc = ctx_alloc(c, &c->rope_sin, (size_t)c->capacity * c->qk / 2)) ||
        (rc = ctx_alloc(c, &c->stream_a, (size_t)R * sw)) || (rc = ctx_alloc(c, &c->stream_b, (size_t)R * sw)) ||
        (rc = ctx_alloc(c, &c->normed, (size_t)R * sw)) || (rc = ctx_alloc(c, &c->input, (size_t)R * d)) ||
        (rc = ctx_alloc(c, &c->residual, (size_t)R * d)) || (rc = ctx_alloc(c, &c->raw, (size_t)R * all)) ||
        (rc = ctx_alloc(c, &c->gate, (size_t)R * ow)) || (rc = ctx_alloc(c, &c->att, (size_t)R * ow)) ||
        (rc = ctx_alloc(c, &c->proj, (size_t)R * d)) || (rc = ctx_alloc(c, &c->key, (size_t)R * d)) ||
        (rc = ctx_alloc(c, &c->stage, (size_t)R * (kEngramHistory + 1) * d)) ||
        (rc = ctx_alloc(c, &c->ein, (size_t)R * d)) || (rc = ctx_alloc(c, &c->act4_v, (size_t)R * sw)) ||
        (rc = ctx_alloc(c, &c->act4_s, (size_t)R * stride4)) || (rc = ctx_alloc(c, &c->act4_o, (size_t)R * stride4)) ||
        (rc = ctx_alloc(c, &c->post_gate, (size_t)R * 4)) || (rc = ctx_alloc(c, &c->mix, (size_t)R * 16)) ||
        (rc = ctx_alloc(c, &c->q8, (size_t)R * qw)) || (rc = ctx_alloc(c, &c->qs, (size_t)R * c->heads)) ||
        (rc = ctx_alloc(c, &c->logits, (size_t)R * c->vocab)) || (rc = ctx_alloc(c, &c->act_v, (size_t)R * sw)) ||
        (rc = ctx_alloc(c, &c->d_topk_idx, (size_t)R * 8)) || (rc = ctx_alloc(c, &c->d_topk_lp, (size_t)R * 8)) ||
        (rc = ctx_alloc(c, &c->d_argmax, (size_t)R)) ||
        (rc = ctx_alloc(c, &c->act_s, (size_t)R * stride4)) || (rc = ctx_alloc(c, &c->act_o, (size_t)R * stride4)) ||
        (rc = ctx_alloc(c, &c->d_in, (size_t)R * (kInSections + std::max(c->engram_tables, 1)))))
        return rc;
    NHIP_CHECK_HIP(hipHostMalloc(reinterpret_cast<void**>(&c->h_in),
                                 sizeof(int32_t) * (size_t)R * (kInSections + std::max(c->engram_tables, 1)),
                                 hipHostMallocDefault));
    c->attn_ws_bytes = nhip_attention_decode_workspace(R, c->heads, c->max_chunks);
    NHIP_CHECK_HIP(hipMalloc(&c->attn_ws, c->attn_ws_bytes));
    c->allocations.push_back(c->attn_ws);
    c->topk_ws_bytes = nhip_topk_lse_workspace(R, c->vocab);
    NHIP_CHECK_HIP(hipMalloc(&c->topk_ws, c->topk_ws_bytes));
    c->allocations.push_back(c->topk_ws);
    // EngineCore.RopeFrequencies + BuildRopeTables (Engine.cs:336-356):
    // float powf / cosf / sinf on the host, as MathF on Linux
    const int half = c->qk / 2;
    uint32_t hdr[48];
    float theta = 0.0f;
    nhip_model_info(c->model, hdr, &theta, nullptr);
    std::vector<float> freq(half), cs((size_t)c->capacity * half), sn((size_t)c->capacity * half);
    for (int i = 0; i < half; i++) freq[i] = 1.0f / std::pow(theta, 2.0f * (float)i / (float)c->qk);
    for (int p = 0; p < c->capacity; p++)
        for (int i = 0; i < half; i++) {
            const float angle = (float)p * freq[i];
            cs[(size_t)p * half + i] = std::cos(angle);
            sn[(size_t)p * half + i] = std::sin(angle);
        }
    NHIP_CHECK_HIP(hipMemcpy(c->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    NHIP_CHECK_HIP(hipMemcpy(c->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    c->len.assign(c->slots, 0);
    c->marked.assign(c->slots, 0);
    c->prev.assign(2 * c->slots, 0);
    c->snap_prev.assign(2 * c->slots, 0);
    const size_t width = (size_t)c->hada_rows * c->hada_cols;
    NHIP_REQUIRE(width <= (size_t)kPer * kThreads, "MLP size %zu above %d", width, kPer * kThreads);
    c->tail_lds = tail_lds_bytes(d, c->hada_rows, c->hada_cols);
    NHIP_REQUIRE(c->tail_lds <= 160 * 1024, "the layer tail's %zu bytes of LDS exceed the CU's", c->tail_lds);
    if (c->tail_lds > 64 * 1024)
        NHIP_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(n3_tail_kernel<false>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)c->tail_lds));
    // the fused tail + next-layer mix, where its LDS fits the CU
    c->tail_hyper_lds = c->tail_lds + tail_hyper_lds_bytes(d);
    if (c->tail_hyper_lds > 160 * 1024) {
        c->tail_hyper_lds = 0;
    } else if (c->tail_hyper_lds > 64 * 1024) {
        NHIP_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(n3_tail_kernel<true>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)c->tail_hyper_lds));
    }
    return NHIP_OK;
}

int stride_of(int cols) { return (cols / 128 + 7) / 8 * 8; }

// Rows [row0, row0 + count) of w over the prepared activations of `rows`
// rows: y[t * ldy + n] for those n.
int32_t matmul(nhip_ctx* c, const nhip_weights* w, int rows, int cols, int row0, int count, float* y, int ldy)
{
    return nhip_matmul_cq_dev(w, c->act_v, c->act_s, c->act_o, stride_of(cols), rows, y, ldy, row0, row0 + count,
                              c->stream_h);
}

// EngineCore.EngramHashRowsBatch (Engine.cs:2631-2656) on the host.
void engram_rows(const nhip_ctx* c, const int32_t* tokens, const int32_t* row_slots, int rows, int32_t* out)
{
    const int heads = c->engram_tables / c->order_count;
    int run_start = 0;
    for (int t = 0; t < rows; t++) {
        if (t == 0 || row_slots[t] != row_slots[t - 1]) run_start = t;
        const int slot = row_slots[t], position = c->len[slot] + t - run_start;
        const int32_t* pv = &c->prev[2 * slot];
        for (int o = 0; o < c->order_count; o++)
            for (int h = 0; h < heads; h++) {
                const int table = o * heads + h, order = c->orders[o];
                if (position < order - 1) {
                    out[t * c->engram_tables + table] = -1;
                    continue;
                }
                uint32_t acc = 0x9E3779B9u * (uint32_t)(table + 1);
                for (int j = 0; j < order; j++) {
                    const int back = t - run_start - j;
                    const int token = back >= 0 ? tokens[run_start + back] : pv[back + 2];
                    acc = (acc ^ (uint32_t)token) * 0x01000193u;
                }
                acc ^= acc >> 15;
                out[t * c->engram_tables + table] = table * c->engram_slots + (int)(acc % (uint32_t)c->engram_slots);
            }
    }
}


// One step over `rows` rows whose inputs are on the device; `heads` distinct
// head rows.  Per layer: the phi matmuls (one launch), the hyper-connection
// mix with the attention norm (or the engram input) and its Prepare, on
// engram layers the key / value matmuls and the engram blend with the
// attention norm, the Q/K/V/Gate matmuls, the attention inputs, attention,
// the gate with the output matmul's Prepare, the output matmul, and the
// layer tail (PostNormAdd, MLP, CombineDiff4x4, the next layer's norm and
// Prepare -- or the head rows' after the last layer).
int32_t enqueue_step(nhip_ctx* c, int rows, int heads, int k, bool argmax, bool single_runs)
{
    hipStream_t s = c->stream_h;
    const int d = c->dim, sw = kLanes * d, L = c->layers, H = c->heads, KV = c->kv, qw = H * c->qk,
              kw = KV * c->qk, vw = KV * c->vd, ow = H * c->vd, all = qw + kw + vw;
    const int stride4 = stride_of(sw), stride_d = stride_of(d), stride_o = stride_of(ow);
    const Act act{c->act_v, c->act_s, c->act_o};
    const Act act4{c->act4_v, c->act4_s, c->act4_o};
    int32_t rc;
    float* cur = c->stream_a;
    float* nxt = c->stream_b;
    // EngineCore's embeddingScale = sqrt(dim) (Engine.cs:123), host sqrtf
    const float emb_scale_m1 = std::sqrt((float)d) - 1.0f;
    // steps whose rows are one per slot run the attention in one launch
    // (attention_decode_needle3_impl), which then also forms Sinkhorn4x4 of
    // the mix kernel's residual-mix logits
    const bool sink_in_attention = single_runs && attention_needle3_fused(c->capacity, c->vd);
    auto site_of = [&](int l) -> const N3Site* {
        for (int k2 = 0; k2 < c->site_count; k2++)
            if (c->sites[k2] == l) return &c->site[k2];
        return nullptr;
    };
    // layer l's mix kernel arguments, with the hyper-connection phi
    // (RunLayerBatch, Engine.cs:2356-2364): the layer's 4 + 4 + 16 rows,
    // formed by the mix kernel itself
    auto hyper_args = [&](int l, const float* stream) {
        PhiRows phi{};
        const int per[3] = {4, 4, 16}, totals[3] = {4 * L, 4 * L, 16 * L};
        for (int m = 0; m < 3; m++) {
            phi.codes[m] = c->phi_raw[m] + (size_t)l * per[m] * (sw / 2);
            phi.norms[m] = reinterpret_cast<const uint16_t*>(c->phi_raw[m] + (size_t)totals[m] * (sw / 2)) +
                           (size_t)l * per[m] * (sw / 128);
        }
        std::memcpy(phi.split, c->phi_pre->split_table, sizeof(phi.split));
        phi.byte_scale = c->phi_pre->byte_scale;
        phi.in = act4;
        phi.stride = stride4;
        const N3Site* st = site_of(l);
        return HyperArgs{stream, phi, c->a_pre + l, c->a_post + l, c->a_res + l, c->b_pre + 4 * l,
                         c->b_post + 4 * l, c->b_res + 16 * l, l % kLanes, d, c->input, c->residual, c->post_gate,
                         c->mix, c->layer[l].norm_in, st ? st->tables : nullptr, st ? st->table_rows : 0,
                         st ? st->table_cols : 0, st ? st->table_bits : 0, c->engram_tables,
                         st && st->table_bits == 2 ? c->book2 : c->book4, in_erows(c, c->d_in), act, stride_d, rows};
    };
    // for those steps each layer's tail launch also runs the next layer's
    // mix (n3_tail_kernel<true>); NHIP_N3_TAIL_MIX=0 keeps the mix launches
    // (for A/B timing)
    static const bool tail_mix_enabled = [] {
        const char* e = getenv("NHIP_N3_TAIL_MIX");
        return !(e && e[0] == '0');
    }();
    const bool fuse_tail = tail_mix_enabled && sink_in_attention && c->tail_hyper_lds > 0;
    if (fuse_tail)  // the embedding launch also runs layer 0's mix
        hipLaunchKernelGGL(n3_embed_kernel<true>, dim3(rows), dim3(kThreads), 0, s, c->embedding_raw, c->vocab, d,
                           c->embedding_bits, c->book4, in(c, c->d_in, kInTokens), emb_scale_m1, cur, act4, stride4,
                           hyper_args(0, cur));
    else
        hipLaunchKernelGGL(n3_embed_kernel<false>, dim3(rows), dim3(kThreads), 0, s, c->embedding_raw, c->vocab, d,
                           c->embedding_bits, c->book4, in(c, c->d_in, kInTokens), emb_scale_m1, cur, act4, stride4,
                           HyperArgs{});
    NHIP_CHECK_HIP(hipGetLastError());
    for (int l = 0; l < L; l++) {
        const N3Layer& w = c->layer[l];
        const N3Site* st = site_of(l);
        if (!fuse_tail) {  // otherwise the embedding's or layer l - 1's tail launch ran the mix
            const HyperArgs ha = hyper_args(l, cur);
            // the attention launch forms the residual-mix rows' Sinkhorn for
            // steps whose rows are one per slot; the mix launch otherwise
            hipLaunchKernelGGL(n3_hyper_kernel, dim3(sink_in_attention ? rows : 2 * rows), dim3(kThreads), 0, s, ha);
            NHIP_CHECK_HIP(hipGetLastError());
        }
        EngramArgs ea{};
        if (st) {  // engram (ApplyEngramBatch, Engine.cs:2399-2463)
            const nhip_weights* jw[2] = {st->key, st->value};
            float* jy[2] = {c->key, c->stage + (size_t)kEngramHistory * d};
            const int32_t jl[2] = {d, (kEngramHistory + 1) * d};
            const int32_t jf[2] = {0, d};
            rc = matmul_cq_split_internal(st->key_value, c->act_v, c->act_s, c->act_o, stride_d, rows, jy, jl, jf, 2, s);
            if (rc < 0) return rc;
            if (rc && (rc = nhip_matmul_batch_dev(jw, 2, c->act_v, c->act_s, c->act_o, stride_d, rows, jy, jl, s)))
                return rc;
            ea = EngramArgs{c->stage,
                            c->engram_hist + (size_t)(st - c->site.data()) * c->slots * kEngramHistory * d,
                            in(c, c->d_in, kInSlots),
                            in(c, c->d_in, kInRunStart),
                            in(c, c->d_in, kInRunEnd),
                            st->taps,
                            c->dilation,
                            d,
                            c->input,
                            c->key,
                            c->residual,
                            1.0f / std::sqrt((float)d),
                            w.norm_in,
                            act,
                            stride_d};
            hipLaunchKernelGGL(n3_engram_mix_kernel, dim3(rows), dim3(kThreads), 0, s, ea);
            NHIP_CHECK_HIP(hipGetLastError());
        }
        // attention (RunAttentionBatch, Engine.cs:2480-2596).  For steps of 5
        // to 16 rows whose attention launch forms Sinkhorn (rows one per
        // slot), it forms the Q/K/V/Gate projections too (each workgroup its
        // heads' rows, more workgroups the Gate's; Needle3Proj): that costs
        // the attention about as much as the 1-4-row matmul launch but less
        // than MatMulBatch.  NHIP_N3_ATTN_PROJ=0 keeps the matmul launch (for
        // A/B timing)
        static const bool attn_proj_enabled = [] {
            const char* e = getenv("NHIP_N3_ATTN_PROJ");
            return !(e && e[0] == '0');
        }();
        const bool proj_in_attention = attn_proj_enabled && sink_in_attention && rows > 4 && rows <= 16 &&
                                       w.qkvg_raw[0] && w.qkvg_raw[1] && w.qkvg_raw[2] && w.qkvg_raw[3] &&
                                       (2 * c->qk + 64) * (d / 128) <= 3 * 512;
        if (!proj_in_attention) {
            const nhip_weights* pw[4] = {w.q, w.k, w.v, w.gate};
            float* py[4] = {c->raw, c->raw + qw, c->raw + qw + kw, c->gate};
            const int32_t pl[4] = {all, all, all, ow};
            const int32_t pf[4] = {0, qw, qw + kw, qw + kw + vw};
            // one launch over the stacked matrix up to 4 rows; MatMulBatch beyond
            rc = matmul_cq_split_internal(w.qkvg, c->act_v, c->act_s, c->act_o, stride_d, rows, py, pl, pf, 4, s);
            if (rc < 0) return rc;
            if (rc && (rc = nhip_matmul_batch_dev(pw, 4, c->act_v, c->act_s, c->act_o, stride_d, rows, py, pl, s)))
                return rc;
        }
        const size_t lcell = (size_t)l * c->slots * c->capacity;
        int8_t* keys = c->keys + lcell * kw;
        int8_t* values = c->values + lcell * vw;
        float* kscale = c->key_scales + lcell * KV;
        float* vscale = c->value_scales + lcell * KV;
        float* qkv_hist = c->qkv_hist + (size_t)l * c->slots * 2 * all;
        // the layer's span (Blocks.cs:973-978): global layers from 0, the
        // others over the window ending at the row
        const bool global = ((c->global_mask >> l) & 1) || c->window == 0;
        const int32_t* first = in(c, c->d_in, global ? kInFirst : kInFirstW);
        const int32_t* count = in(c, c->d_in, global ? kInCount : kInCountW);
        // steps whose rows are one per slot: the attention inputs inside the
        // attention launch; otherwise (runs of rows, long caches) two launches
        int32_t fused = 1;
        if (single_runs) {
            // with the Sinkhorn: the layer's residual-mix phi rows over the
            // stream's 4-bit prepared rows
            const HyperArgs hl = hyper_args(l, cur);
            Needle3AttnInputs n3in{c->raw,
                                         {w.q_taps, w.k_taps, w.v_taps},
                                         w.q_norm,
                                         w.k_norm,
                                         c->rope_cos,
                                         c->rope_sin,
                                         qkv_hist,
                                         sink_in_attention ? c->mix : nullptr,
                                         hl.phi,
                                         sw,
                                         hl.a_res,
                                         hl.b_res};
            if (proj_in_attention) {
                const int prow[4] = {qw, kw, vw, ow};
                Needle3Proj& pj = n3in.proj;
                for (int m = 0; m < 4; m++) {
                    pj.codes[m] = w.qkvg_raw[m];
                    pj.norms[m] = reinterpret_cast<const uint16_t*>(w.qkvg_raw[m] + (size_t)prow[m] * (d / 4));
                }
                pj.table = w.q->table[0];
                pj.byte_scale = w.q->byte_scale;
                pj.act = c->act_v;
                pj.scales = c->act_s;
                pj.offsets = c->act_o;
                pj.stride = stride_d;
                pj.k = d;
                pj.raw = c->raw;
                pj.gate = c->gate;
                pj.gate_rows = ow;
            }
            fused = attention_decode_needle3_impl(n3in, rows, H, KV, c->qk, c->vd, keys, kscale, values, vscale,
                                                  c->slots, c->capacity, in(c, c->d_in, kInSlots),
                                                  in(c, c->d_in, kInPos), first, count, c->max_chunks, c->att, s);
            if (fused < 0) return fused;
            NHIP_REQUIRE(fused == 0 || !sink_in_attention, "attention launch refused a step it takes");
        }
        if (fused == 1) {
            if ((rc = needle3_attention_inputs_impl(c->raw, rows, H, KV, c->qk, c->vd, w.q_taps, w.k_taps, w.v_taps,
                                                    w.q_norm, w.k_norm, c->rope_cos, c->rope_sin, qkv_hist,
                                                    in(c, c->d_in, kInSlots), in(c, c->d_in, kInPos), c->slots,
                                                    c->capacity, c->q8, c->qs, keys, kscale, values, vscale, false,
                                                    s)))
                return rc;
            if ((rc = attention_decode_impl(c->q8, c->qs, rows, H, KV, c->qk, keys, kscale, values, vscale, c->slots,
                                            c->capacity, in(c, c->d_in, kInSlots), first, count, c->max_chunks,
                                            c->attn_ws, c->attn_ws_bytes, c->att, nullptr, nullptr, s)))
                return rc;
        }
        // the gate also moves the slots' Q/K/V frames on, after attention's
        // inputs have read them
        const QkvHistArgs qh{qkv_hist, c->raw, in(c, c->d_in, kInSlots), in(c, c->d_in, kInRunStart),
                             in(c, c->d_in, kInRunEnd), qw, kw, vw};
        // NHIP_N3_GATE_OUT=0 keeps the two launches for every step (for A/B timing)
        static const bool gate_out_enabled = [] {
            const char* e = getenv("NHIP_N3_GATE_OUT");
            return !(e && e[0] == '0');
        }();
        // d and ow are multiples of 128 up to 1024 (load_model), so the d / 16
        // workgroups cover the columns; each takes at most kThreads of the
        // rows' Q/K/V history elements
        if (gate_out_enabled && rows <= kGateOutRows && w.out_raw && rows * (qw + kw + vw) <= kThreads * (d / 16)) {
            const GateOutArgs ga{reinterpret_cast<const uint16_t*>(w.out_raw + (size_t)d * (ow / 4)), c->proj, d,
                                 w.out->table[0], w.out->byte_scale, ea, qh};
            hipLaunchKernelGGL(n3_gate_out_kernel, dim3(d / 16), dim3(kThreads), 0, s, w.out_raw, c->att, c->gate,
                               (uint64_t)(uint32_t)rows | ((uint64_t)(uint32_t)ow << 32), ga);
            NHIP_CHECK_HIP(hipGetLastError());
        } else {
            hipLaunchKernelGGL(n3_gate_kernel, dim3(rows), dim3(kThreads), 0, s, c->att, c->gate, ow, act, stride_o, ea,
                               qh);
            NHIP_CHECK_HIP(hipGetLastError());
            if ((rc = matmul(c, w.out, rows, ow, 0, d, c->proj, d))) return rc;
        }
        const bool last = l == L - 1;
        TailArgs ta{c->residual, c->proj, w.post_norm, w.attn_gate, w.pre_hada, c->perm_a, c->perm_b, w.d1, w.d2,
                    w.b2, w.d3, w.d4, w.w1a, w.w1b, w.w2a, w.w2b, w.w3a, w.w3b, w.cond_v, w.cond_u, d, c->hada_rows,
                    c->hada_cols, cur, c->mix, c->input, c->post_gate, nxt,
                    last ? in(c, c->d_in, kInHeadOf) : nullptr, c->final_norm, last ? act : act4,
                    last ? stride_d : stride4};
        if (fuse_tail && !last)
            hipLaunchKernelGGL(n3_tail_kernel<true>, dim3(rows), dim3(kThreads), c->tail_hyper_lds, s, ta.proj,
                               ta.residual, ta.post_norm, ta.pre_norm, ta.mix, ta.post_gate, ta, hyper_args(l + 1, nxt));
        else
            hipLaunchKernelGGL(n3_tail_kernel<false>, dim3(rows), dim3(kThreads), c->tail_lds, s, ta.proj,
                               ta.residual, ta.post_norm, ta.pre_norm, ta.mix, ta.post_gate, ta, HyperArgs{});
        NHIP_CHECK_HIP(hipGetLastError());
        std::swap(cur, nxt);
    }
    if (heads == 0) return NHIP_OK;
    // the head rows' logits: the tied 4-bit embedding (PrepareHead,
    // Engine.cs:2188-2189)
    if ((rc = matmul(c, c->embedding, heads, d, 0, c->vocab, c->logits, c->vocab))) return rc;
    if (k > 0 && (rc = nhip_topk_lse_dev(c->logits, heads, c->vocab, k, c->topk_ws, c->topk_ws_bytes, c->d_topk_idx,
                                         c->d_topk_lp, s)))
        return rc;
    if (argmax && (rc = nhip_argmax_dev(c->logits, c->vocab, c->vocab, heads, c->d_argmax, nullptr, s))) return rc;
    return NHIP_OK;
}

// Steps of up to kMaxGraphRows rows replay a graph captured on first use for
// their (rows, heads, k, argmax): every per-step input lives in device
// arrays uploaded before the launch, so the captured kernels and arguments
// stay valid.  NHIP_ENGINE_GRAPHS=0 launches every step eagerly (for kernel
// tracers).
constexpr int kMaxGraphRows = 16;
constexpr size_t kMaxGraphs = 64;

int32_t run_step(nhip_ctx* c, int rows, int heads, int k, bool argmax, bool single_runs)
{
    static const bool graphs_enabled = [] {
        const char* e = getenv("NHIP_ENGINE_GRAPHS");
        return !(e && e[0] == '0');
    }();
    if (!graphs_enabled || rows > kMaxGraphRows) return enqueue_step(c, rows, heads, k, argmax, single_runs);
    hipGraphExec_t exec = nullptr;
    for (const nhip_ctx::Graph& g : c->graphs)
        if (g.rows == rows && g.heads == heads && g.k == k && g.argmax == argmax && g.single_runs == single_runs)
            exec = g.exec;
    if (!exec) {
        if (c->graphs.size() >= kMaxGraphs) {  // drop the oldest
            NHIP_CHECK_HIP(hipStreamSynchronize(c->stream_h));
            (void)hipGraphExecDestroy(c->graphs.front().exec);
            c->graphs.erase(c->graphs.begin());
        }
        hipGraph_t g;
        NHIP_CHECK_HIP(hipStreamBeginCapture(c->stream_h, hipStreamCaptureModeThreadLocal));
        const int32_t rc = enqueue_step(c, rows, heads, k, argmax, single_runs);
        hipError_t e = hipStreamEndCapture(c->stream_h, &g);
        if (rc) {
            if (e == hipSuccess) (void)hipGraphDestroy(g);
            return rc;
        }
        NHIP_CHECK_HIP(e);
        e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        NHIP_CHECK_HIP(e);
        c->graphs.push_back(nhip_ctx::Graph{rows, heads, k, argmax, single_runs, exec});
    }
    NHIP_CHECK_HIP(hipGraphLaunch(exec, c->stream_h));
    return NHIP_OK;
}

// The live histories of a slot (convolution frames of every layer, engram
// frames of every site) to or from its snapshot; MarkView / RewindView
// (Engine.cs:2235-2255) with the rewind restoring eagerly.
int32_t snapshot_slot(nhip_ctx* c, int slot, bool to_snapshot)
{
    const size_t all = (size_t)c->heads * c->qk + (size_t)c->kv * c->qk + (size_t)c->kv * c->vd;
    int32_t rc;
    for (int l = 0; l < c->layers; l++) {
        const size_t o = ((size_t)l * c->slots + slot) * 2 * all;
        float* live = c->qkv_hist + o;
        float* snap = c->snap_qkv + o;
        if ((rc = nhip_copy_dev(to_snapshot ? snap : live, to_snapshot ? live : snap, sizeof(float) * 2 * all,
                                c->stream_h)))
            return rc;
    }
    const size_t eh = (size_t)kEngramHistory * c->dim;
    for (int k = 0; k < c->site_count; k++) {
        const size_t o = ((size_t)k * c->slots + slot) * eh;
        float* live = c->engram_hist + o;
        float* snap = c->snap_engram + o;
        if ((rc = nhip_copy_dev(to_snapshot ? snap : live, to_snapshot ? live : snap, sizeof(float) * eh, c->stream_h)))
            return rc;
    }
    for (int i = 0; i < 2; i++) {
        if (to_snapshot) c->snap_prev[2 * slot + i] = c->prev[2 * slot + i];
        else c->prev[2 * slot + i] = c->snap_prev[2 * slot + i];
    }
    NHIP_CHECK_HIP(hipStreamSynchronize(c->stream_h));
    return NHIP_OK;
}

}  // namespace

extern "C" {

int32_t nhip_ctx_destroy(nhip_ctx* c)
{
    clear_error();
    if (!c) return NHIP_OK;
    if (c->stream_h) (void)hipStreamSynchronize(c->stream_h);
    for (nhip_ctx::Graph& g : c->graphs) (void)hipGraphExecDestroy(g.exec);
    for (void* p : c->allocations) (void)hipFree(p);
    for (nhip_weights* w : c->stacked) (void)nhip_weights_destroy(w);
    if (c->h_in) (void)hipHostFree(c->h_in);
    if (c->stream_h) (void)hipStreamDestroy(c->stream_h);
    delete c;
    return NHIP_OK;
}

int32_t nhip_ctx_create(const nhip_model* model, int32_t capacity, int32_t slots, int32_t chunk, int32_t max_chunks,
                        nhip_ctx** out)
{
    clear_error();
    NHIP_REQUIRE(model && out, "null argument");
    *out = nullptr;
    if (chunk <= 0) chunk = 64;
    if (max_chunks <= 0) max_chunks = 8;
    // BatchedEngine's limits (BatchEngine.cs:11-12): 1..16 slots
    NHIP_REQUIRE(capacity > 0 && slots >= 1 && slots <= 16 && chunk <= 4096 && max_chunks <= 256,
                 "capacity %d, slots %d (1..16), chunk %d (<= 4096), max_chunks %d (<= 256)", capacity, slots, chunk,
                 max_chunks);
    int32_t rc = ensure_device();
    if (rc) return rc;
    nhip_ctx* c = new nhip_ctx();
    c->model = model;
    c->slots = slots;
    c->capacity = capacity;
    c->max_rows = chunk;
    c->max_chunks = max_chunks;
    if (hipStreamCreateWithFlags(&c->stream_h, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        set_error("hipStreamCreateWithFlags failed");
        return NHIP_ERR_HIP;
    }
    if ((rc = load_model(c)) || (rc = alloc_state(c))) {
        const std::string why = nhip_last_error();
        nhip_ctx_destroy(c);
        set_error("%s", why.c_str());
        return rc;
    }
    if (hipStreamSynchronize(c->stream_h) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        nhip_ctx_destroy(c);
        set_error("context set-up failed");
        return NHIP_ERR_HIP;
    }
    *out = c;
    return NHIP_OK;
}

int32_t nhip_ctx_info(const nhip_ctx* c, int32_t* vocab, int32_t* slots, int32_t* capacity, int32_t* chunk)
{
    clear_error();
    NHIP_REQUIRE(c, "null context");
    if (vocab) *vocab = c->vocab;
    if (slots) *slots = c->slots;
    if (capacity) *capacity = c->capacity;
    if (chunk) *chunk = c->max_rows;
    return NHIP_OK;
}

int32_t nhip_step(nhip_ctx* c, const int32_t* tokens, const int32_t* row_slots, int32_t rows, const int32_t* head_rows,
                  int32_t heads, float* logits, int32_t k, int32_t* topk_idx, float* topk_lp, int32_t* argmax)
{
    clear_error();
    NHIP_REQUIRE(c && tokens && row_slots, "null argument");
    // ForwardBatch's checks (Engine.cs:2305-2307)
    NHIP_REQUIRE(rows >= 1 && rows <= c->max_rows, "rows %d outside [1, %d]", rows, c->max_rows);
    NHIP_REQUIRE(heads >= 0 && heads <= rows && (heads == 0 || head_rows), "heads %d outside [0, %d]", heads, rows);
    NHIP_REQUIRE(k >= 0 && k <= 8 && (k == 0 || (topk_idx && topk_lp)), "k %d outside [0, 8] or null top-k output", k);
    const int R = c->max_rows;
    int32_t* h = c->h_in;
    std::vector<char> seen(c->slots, 0);
    bool single_runs = true;  // every row the only row of its slot
    for (int rs = 0; rs < rows;) {
        const int slot = row_slots[rs];
        NHIP_REQUIRE(slot >= 0 && slot < c->slots, "row %d: slot %d outside [0, %d)", rs, slot, c->slots);
        NHIP_REQUIRE(!seen[slot], "the rows of slot %d must form one contiguous run", slot);
        seen[slot] = 1;
        int rk = rs;
        while (rk + 1 < rows && row_slots[rk + 1] == slot) rk++;
        single_runs = single_runs && rk == rs;
        NHIP_REQUIRE(c->len[slot] + (rk - rs + 1) <= c->capacity, "slot %d: context capacity %d exceeded", slot,
                     c->capacity);
        for (int t = rs; t <= rk; t++) {
            NHIP_REQUIRE(tokens[t] >= 0 && tokens[t] < c->vocab, "row %d: token %d outside [0, %d)", t, tokens[t],
                         c->vocab);
            const int pos = c->len[slot] + t - rs;
            const int first_w = c->window > 0 ? std::max(pos - c->window + 1, 0) : 0;
            h[kInTokens * R + t] = tokens[t];
            h[kInSlots * R + t] = slot;
            h[kInPos * R + t] = pos;
            h[kInFirst * R + t] = 0;
            h[kInCount * R + t] = pos + 1;
            h[kInFirstW * R + t] = first_w;
            h[kInCountW * R + t] = pos - first_w + 1;
            h[kInRunStart * R + t] = rs;
            h[kInRunEnd * R + t] = t == rk ? 1 : 0;
        }
        rs = rk + 1;
    }
    // the head runs once per distinct head row, in order of first mention;
    // repeated rows are copied out again
    for (int t = 0; t < rows; t++) h[kInHeadOf * R + t] = -1;
    std::vector<int> head_map(heads);
    int distinct = 0;
    for (int i = 0; i < heads; i++) {
        const int t = head_rows[i];
        NHIP_REQUIRE(t >= 0 && t < rows, "head row %d outside [0, %d)", t, rows);
        if (h[kInHeadOf * R + t] < 0) h[kInHeadOf * R + t] = distinct++;
        head_map[i] = h[kInHeadOf * R + t];
    }
    if (c->site_count > 0) engram_rows(c, tokens, row_slots, rows, in_erows(c, h));
    const size_t words = (size_t)R * (kInSections + std::max(c->engram_tables, 1));
    hipStream_t s = c->stream_h;
    int32_t rc = NHIP_OK;
    if (hipMemcpyAsync(c->d_in, h, words * sizeof(int32_t), hipMemcpyHostToDevice, s) != hipSuccess) {
        set_error("step input upload failed");
        rc = NHIP_ERR_HIP;
    }
    if (rc == NHIP_OK) rc = run_step(c, rows, distinct, k, argmax != nullptr, single_runs);
    const bool repeats = distinct < heads;
    std::vector<float> lg_h, lp_h;
    std::vector<int32_t> idx_h, am_h;
    if (rc == NHIP_OK && heads > 0) {
        const size_t hv = (size_t)distinct, V = (size_t)c->vocab;
        float* lg_dst = logits;
        float* lp_dst = topk_lp;
        int32_t* idx_dst = topk_idx;
        int32_t* am_dst = argmax;
        if (repeats) {  // download the distinct rows, expand below
            lg_h.resize(hv * V);
            lp_h.resize(hv * 8);
            idx_h.resize(hv * 8);
            am_h.resize(hv);
            lg_dst = lg_h.data();
            lp_dst = lp_h.data();
            idx_dst = idx_h.data();
            am_dst = am_h.data();
        }
        hipError_t e = hipSuccess;
        if (logits) e = hipMemcpyAsync(lg_dst, c->logits, hv * V * sizeof(float), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess && k > 0) {
            // the device lists are [heads][k] with stride k
            e = hipMemcpyAsync(idx_dst, c->d_topk_idx, hv * k * sizeof(int32_t), hipMemcpyDeviceToHost, s);
            if (e == hipSuccess)
                e = hipMemcpyAsync(lp_dst, c->d_topk_lp, hv * k * sizeof(float), hipMemcpyDeviceToHost, s);
        }
        if (e == hipSuccess && argmax)
            e = hipMemcpyAsync(am_dst, c->d_argmax, hv * sizeof(int32_t), hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) {
            set_error("step output download failed: %s", hipGetErrorString(e));
            rc = NHIP_ERR_HIP;
        }
    }
    // the staging buffer is reused by the next call: drain the stream first
    const hipError_t done = hipStreamSynchronize(s);
    if (rc != NHIP_OK) return rc;
    if (done != hipSuccess) {
        set_error("step failed: %s", hipGetErrorString(done));
        return NHIP_ERR_HIP;
    }
    if (repeats)
        for (int i = 0; i < heads; i++) {
            const size_t u = (size_t)head_map[i], V = (size_t)c->vocab;
            if (logits) std::memcpy(logits + i * V, lg_h.data() + u * V, V * sizeof(float));
            if (k > 0) {
                std::memcpy(topk_idx + (size_t)i * k, idx_h.data() + u * k, k * sizeof(int32_t));
                std::memcpy(topk_lp + (size_t)i * k, lp_h.data() + u * k, k * sizeof(float));
            }
            if (argmax) argmax[i] = am_h[u];
        }
    // the slots' lengths and previous tokens (ForwardBatch, Engine.cs:2326-2340)
    for (int rs = 0; rs < rows;) {
        const int slot = row_slots[rs];
        int rk = rs;
        while (rk + 1 < rows && row_slots[rk + 1] == slot) rk++;
        int32_t* pv = &c->prev[2 * slot];
        pv[0] = rk > rs ? tokens[rk - 1] : pv[1];
        pv[1] = tokens[rk];
        c->len[slot] += rk - rs + 1;
        rs = rk + 1;
    }
    return NHIP_OK;
}

int32_t nhip_slot_feed(nhip_ctx* c, int32_t slot, const int32_t* tokens, int32_t count, float* logits)
{
    clear_error();
    NHIP_REQUIRE(c && (tokens || count == 0), "null argument");
    NHIP_REQUIRE(slot >= 0 && slot < c->slots, "slot %d outside [0, %d)", slot, c->slots);
    NHIP_REQUIRE(count >= 0, "count %d", count);
    // FeedSlot (Engine.cs:2285-2301): the capacity is checked before any work
    NHIP_REQUIRE(c->len[slot] + count <= c->capacity, "slot %d: context capacity %d exceeded", slot, c->capacity);
    std::vector<int32_t> row_slots(c->max_rows, slot);
    for (int start = 0; start < count; start += c->max_rows) {
        const int n = std::min(c->max_rows, count - start);
        const bool last = start + n == count;
        const int32_t head = n - 1;
        const int heads = last && logits ? 1 : 0;
        const int32_t rc = nhip_step(c, tokens + start, row_slots.data(), n, heads ? &head : nullptr, heads,
                                     heads ? logits : nullptr, 0, nullptr, nullptr, nullptr);
        if (rc) return rc;
    }
    return NHIP_OK;
}

int32_t nhip_slot_reset(nhip_ctx* c, int32_t slot)
{
    clear_error();
    NHIP_REQUIRE(c && slot >= 0 && slot < c->slots, "slot %d outside the context's slots", slot);
    const size_t all = (size_t)c->heads * c->qk + (size_t)c->kv * c->qk + (size_t)c->kv * c->vd;
    for (int l = 0; l < c->layers; l++)
        NHIP_CHECK_HIP(hipMemsetAsync(c->qkv_hist + ((size_t)l * c->slots + slot) * 2 * all, 0, sizeof(float) * 2 * all,
                                      c->stream_h));
    const size_t eh = (size_t)kEngramHistory * c->dim;
    for (int k = 0; k < c->site_count; k++)
        NHIP_CHECK_HIP(
            hipMemsetAsync(c->engram_hist + ((size_t)k * c->slots + slot) * eh, 0, sizeof(float) * eh, c->stream_h));
    NHIP_CHECK_HIP(hipStreamSynchronize(c->stream_h));
    c->prev[2 * slot] = c->prev[2 * slot + 1] = 0;
    c->len[slot] = 0;
    c->marked[slot] = 0;
    return NHIP_OK;
}

int32_t nhip_slot_mark(nhip_ctx* c, int32_t slot)
{
    clear_error();
    NHIP_REQUIRE(c && slot >= 0 && slot < c->slots, "slot %d outside the context's slots", slot);
    const int32_t rc = snapshot_slot(c, slot, true);
    if (rc) return rc;
    c->marked[slot] = c->len[slot];
    return NHIP_OK;
}

int32_t nhip_slot_rewind(nhip_ctx* c, int32_t slot)
{
    clear_error();
    NHIP_REQUIRE(c && slot >= 0 && slot < c->slots, "slot %d outside the context's slots", slot);
    const int32_t rc = snapshot_slot(c, slot, false);
    if (rc) return rc;
    c->len[slot] = c->marked[slot];
    return NHIP_OK;
}

int32_t nhip_slot_length(const nhip_ctx* c, int32_t slot, int32_t* length)
{
    clear_error();
    NHIP_REQUIRE(c && length && slot >= 0 && slot < c->slots, "slot %d outside the context's slots", slot);
    *length = c->len[slot];
    return NHIP_OK;
}

int32_t nhip_slot_copy(nhip_ctx* c, int32_t dst, int32_t src)
{
    clear_error();
    NHIP_REQUIRE(c && dst >= 0 && dst < c->slots && src >= 0 && src < c->slots, "slots %d <- %d outside [0, %d)", dst,
                 src, c ? c->slots : 0);
    if (dst == src) return NHIP_OK;
    const size_t qw = (size_t)c->heads * c->qk, kw = (size_t)c->kv * c->qk, vw = (size_t)c->kv * c->vd,
                 all = qw + kw + vw, n = (size_t)c->len[src], KV = c->kv;
    hipStream_t s = c->stream_h;
    int32_t rc;
    for (int l = 0; l < c->layers; l++) {
        const size_t cs = ((size_t)l * c->slots + src) * c->capacity, cd = ((size_t)l * c->slots + dst) * c->capacity;
        const size_t hs = ((size_t)l * c->slots + src) * 2 * all, hd = ((size_t)l * c->slots + dst) * 2 * all;
        if ((rc = nhip_copy_dev(c->keys + cd * kw, c->keys + cs * kw, n * kw, s)) ||
            (rc = nhip_copy_dev(c->values + cd * vw, c->values + cs * vw, n * vw, s)) ||
            (rc = nhip_copy_dev(c->key_scales + cd * KV, c->key_scales + cs * KV, n * KV * sizeof(float), s)) ||
            (rc = nhip_copy_dev(c->value_scales + cd * KV, c->value_scales + cs * KV, n * KV * sizeof(float), s)) ||
            (rc = nhip_copy_dev(c->qkv_hist + hd, c->qkv_hist + hs, 2 * all * sizeof(float), s)) ||
            (rc = nhip_copy_dev(c->snap_qkv + hd, c->snap_qkv + hs, 2 * all * sizeof(float), s)))
            return rc;
    }
    const size_t eh = (size_t)kEngramHistory * c->dim;
    for (int k = 0; k < c->site_count; k++) {
        const size_t os = ((size_t)k * c->slots + src) * eh, od = ((size_t)k * c->slots + dst) * eh;
        if ((rc = nhip_copy_dev(c->engram_hist + od, c->engram_hist + os, eh * sizeof(float), s)) ||
            (rc = nhip_copy_dev(c->snap_engram + od, c->snap_engram + os, eh * sizeof(float), s)))
            return rc;
    }
    NHIP_CHECK_HIP(hipStreamSynchronize(s));
    for (int i = 0; i < 2; i++) {
        c->prev[2 * dst + i] = c->prev[2 * src + i];
        c->snap_prev[2 * dst + i] = c->snap_prev[2 * src + i];
    }
    c->len[dst] = c->len[src];
    c->marked[dst] = c->marked[src];
    return NHIP_OK;
}

}  // extern "C"

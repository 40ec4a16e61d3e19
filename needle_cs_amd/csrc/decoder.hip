// decoder.hip -- the beam/ragged-batched decode step of an int8 decoder on
// gfx950, and the beam-search driver around it.
//
// One forward runs `rows` packed rows (tokens of independent sequences or
// beams), each in its own KV-cache slot at its own position: embedding ->
// per layer [RMSNorm+quantize -> QKV matmul -> RoPE + per-head quantize +
// KV write -> ragged attention -> quantize -> output matmul -> residual +
// RMSNorm + quantize -> gate/up matmul -> SwiGLU + quantize -> down matmul]
// -> residual + final RMSNorm + quantize -> LM head -> top-k log-softmax.
// This is EngineCore.ForwardBatch's packing (src/Needle/Engine.cs:2303-2350,
// 2480-2596: rows from several slots in one pass, each attending its own
// cache) applied to the benchmark's plain pre-norm decoder; the matmuls are
// the literal int8 kernels (Scalar.MatMulRows' order), the attention is the
// AttentionBatch + MergePartials order, and the element-wise kernels below
// follow one canonical operation order (written out at each kernel) that
// the CPU path repeats exactly, so token streams are bit-identical.
// Beam search follows Whistle.BeamSearch (src/Needle/Whistle.Decode.cs:
// 226-350) with the beams batched into one forward per step instead of one
// Engine.Feed per beam; the last child of a parent keeps the parent's cache
// slot, other children get a copy (Engine.CopyFrom, Engine.cs:367-379).
// Decode steps replay a HIP graph per row count.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "common.hpp"

namespace nhip {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxPerThread = 16;  // d and ffn up to 4096 elements per row
constexpr int kMaxTopK = 8;
constexpr int kMaxMaskedRows = 16;  // rows of a masked (sparse-head) forward

constexpr int kGroups4 = 4;        // float4 groups per thread: rows up to 4096 elements

// Maximum over the block (4 waves, order-free) through wmax[4].
__device__ __forceinline__ float block_max(float v, float* wmax)
{
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
}

// The canonical row sum (common.hpp) of the partials p[t] held by the 256
// threads, broadcast to every thread through red[256] (red holds 257 floats;
// other reductions of the same kernel must not reuse red[256]).
__device__ __forceinline__ float block_canonical_sum(float p, float* red)
{
    red[threadIdx.x] = p;
    __syncthreads();
    if (threadIdx.x < 64) {
        const float total = canonical_finish(red, threadIdx.x);
        if (threadIdx.x == 0) red[kThreads] = total;
    }
    __syncthreads();
    return red[kThreads];
}

__device__ __forceinline__ uint32_t pack_q4(float4 h, float inverse)
{
    const uint32_t a = (uint32_t)(ref_quantize_one(h.x, inverse) & 0xFF);
    const uint32_t b = (uint32_t)(ref_quantize_one(h.y, inverse) & 0xFF);
    const uint32_t c = (uint32_t)(ref_quantize_one(h.z, inverse) & 0xFF);
    const uint32_t d = (uint32_t)(ref_quantize_one(h.w, inverse) & 0xFF);
    return a | (b << 8) | (c << 16) | (d << 24);
}

__device__ __forceinline__ float max_abs4(float m, float4 v)
{
    return fmaxf(fmaxf(m, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// Natural log for normal x > 0: x = m 2^e, m in [sqrt(1/2), sqrt(2)),
// log m = 2 atanh(s), s = (m-1)/(m+1), odd series to s^9; e*ln2 split as in
// Ops.Exp.
__device__ __forceinline__ float log_poly(float x)
{
    const uint32_t u = __float_as_uint(x);
    int e = (int)(u >> 23) - 127;
    float m = __uint_as_float((u & 0x7FFFFFu) | 0x3F800000u);
    if (m > 1.41421356f) {
        m = m * 0.5f;
        e = e + 1;
    }
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float z = s * s;
    float p = 0.11111111f;
    p = __builtin_fmaf(p, z, 0.14285715f);
    p = __builtin_fmaf(p, z, 0.2f);
    p = __builtin_fmaf(p, z, 0.33333334f);
    p = __builtin_fmaf(p, z, 1.0f);
    const float r = (2.0f * s) * p;
    const float fe = (float)e;
    return __builtin_fmaf(fe, 0.693359375f, __builtin_fmaf(fe, -2.12194440e-4f, r));
}

__global__ __launch_bounds__(kThreads) void embed_kernel(const int32_t* tokens, const float* emb, int d, float* x)
{
    asm volatile("" ::"s"(tokens), "s"(emb), "s"(d), "s"(x));  // one round trip to the arguments
    const float* src = emb + (size_t)tokens[blockIdx.x] * d;
    float* dst = x + (size_t)blockIdx.x * d;
    for (int i = threadIdx.x; i < d; i += kThreads) dst[i] = src[i];
}

// x += delta (when given); ss = sum x^2 (canonical sum); inv = 1 / sqrt(ss /
// d + eps); h = (x * inv) * gain; QuantizeInt8(h) -> q, scale.  Thread t
// holds the float4 groups at 4t + 1024j (d a multiple of 4, at most 4096).
// Block b reads row row_map[b] of x and delta (row b without a map) and
// writes row b of q and qscale: the LM head's rows of a forward.
template <bool DELTA>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_quant_kernel(float* x, const float* delta, const float* gain,
                                                                     int d, float eps, int8_t* q, float* qscale,
                                                                     const int32_t* row_map)
{
    __shared__ __align__(16) float red[kThreads + 8];  // partials, the broadcast sum, 4 wave maxima
    const int t = threadIdx.x;
    const int src = row_map ? row_map[blockIdx.x] : (int)blockIdx.x;
    float* xr = x + (size_t)src * d;
    const float* dr = DELTA ? delta + (size_t)src * d : nullptr;
    float4 v[kGroups4], gv[kGroups4];
#pragma unroll
    for (int j = 0; j < kGroups4; j++) {  // every load first
        const int i = min(4 * t + 1024 * j, d - 4);
        v[j] = *reinterpret_cast<const float4*>(xr + i);
        gv[j] = *reinterpret_cast<const float4*>(gain + i);
        if constexpr (DELTA) {
            const float4 e = *reinterpret_cast<const float4*>(dr + i);
            v[j] = make_float4(v[j].x + e.x, v[j].y + e.y, v[j].z + e.z, v[j].w + e.w);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kGroups4; j++) {
        const int i = 4 * t + 1024 * j;
        if (i < d) {
            if constexpr (DELTA) *reinterpret_cast<float4*>(xr + i) = v[j];
            s = s + v[j].x * v[j].x;
            s = s + v[j].y * v[j].y;
            s = s + v[j].z * v[j].z;
            s = s + v[j].w * v[j].w;
        }
    }
    const float ss = block_canonical_sum(s, red);
    const float inv = 1.0f / sqrtf(ss / (float)d + eps);
    float peak = 0.0f;
#pragma unroll
    for (int j = 0; j < kGroups4; j++) {
        if (4 * t + 1024 * j < d) {
            v[j] = make_float4((v[j].x * inv) * gv[j].x, (v[j].y * inv) * gv[j].y, (v[j].z * inv) * gv[j].z,
                               (v[j].w * inv) * gv[j].w);
            peak = max_abs4(peak, v[j]);
        }
    }
    peak = block_max(peak, red + kThreads + 4);
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    const float inverse = 1.0f / scale;
    int8_t* qr = q + (size_t)blockIdx.x * d;
#pragma unroll
    for (int j = 0; j < kGroups4; j++) {
        const int i = 4 * t + 1024 * j;
        if (i < d) *reinterpret_cast<uint32_t*>(qr + i) = pack_q4(v[j], inverse);
    }
    if (t == 0) qscale[blockIdx.x] = scale;
}

struct PostParams {
    const float* qkv;  // [rows][(H + 2 KV) * 64]
    const int32_t* slots;
    const int32_t* positions;
    const float* rope_cos;  // [capacity][32]
    const float* rope_sin;
    int8_t* q8;  // [rows][H][64]
    float* qs;   // [rows][H]
    int8_t* keys;
    float* key_scales;
    int8_t* values;
    float* value_scales;  // this layer's pools: [slots][capacity][KV(*64)]
    int heads, kv_heads, capacity;
};

// One wave per (row, head unit): query heads get RoPE and QuantizeInt8;
// key heads RoPE, QuantizeInt8 and the cache write at the row's position;
// value heads QuantizeInt8 and the cache write.  RoPE (rotate-half): x_i' =
// x_i c_i - x_{i+32} s_i, x_{i+32}' = x_{i+32} c_i + x_i s_i.
__global__ __launch_bounds__(64) void qkv_post_kernel(PostParams p)
{
    const int row = blockIdx.x;
    const int u = blockIdx.y;
    const int e = threadIdx.x;
    const int units = p.heads + 2 * p.kv_heads;
    const int pos = p.positions[row];
    float v = p.qkv[((size_t)row * units + u) * 64 + e];
    if (u < p.heads + p.kv_heads) {
        const int i = e & 31;
        const float c = p.rope_cos[(size_t)pos * 32 + i];
        const float s = p.rope_sin[(size_t)pos * 32 + i];
        const float other = __shfl_xor(v, 32);
        v = e < 32 ? v * c - other * s : v * c + other * s;
    }
    float peak = fabsf(v);
    for (int off = 32; off > 0; off >>= 1) peak = fmaxf(peak, __shfl_xor(peak, off));
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    const float inverse = 1.0f / scale;
    const int8_t qv = static_cast<int8_t>(ref_quantize_one(v, inverse));
    if (u < p.heads) {
        p.q8[((size_t)row * p.heads + u) * 64 + e] = qv;
        if (e == 0) p.qs[(size_t)row * p.heads + u] = scale;
        return;
    }
    const bool key = u < p.heads + p.kv_heads;
    const int kv = key ? u - p.heads : u - p.heads - p.kv_heads;
    const size_t cell = ((size_t)p.slots[row] * p.capacity + pos) * p.kv_heads + kv;
    (key ? p.keys : p.values)[cell * 64 + e] = qv;
    if (e == 0) (key ? p.key_scales : p.value_scales)[cell] = scale;
}

// a = (g / (1 + Exp(-g))) * u, then QuantizeInt8(a).  The gate/up outputs
// are tile-interleaved (gate j at 16*(j/8) + j%8, up j eight further on).
// Thread t holds the float4 groups at 4t + 1024j (ffn a multiple of 8, at
// most 4096).
__global__ __launch_bounds__(kThreads) void swiglu_quant_kernel(const float* gu, int ffn, int8_t* q, float* qscale)
{
    __shared__ float wmax[4];
    const int t = threadIdx.x;
    const float* row = gu + (size_t)blockIdx.x * 2 * ffn;
    float4 v[kGroups4], uv[kGroups4];
#pragma unroll
    for (int j = 0; j < kGroups4; j++) {  // every load first
        const int i = min(4 * t + 1024 * j, ffn - 4);
        const int gi = 16 * (i >> 3) + (i & 7);
        v[j] = *reinterpret_cast<const float4*>(row + gi);
        uv[j] = *reinterpret_cast<const float4*>(row + gi + 8);
    }
    float peak = 0.0f;
#pragma unroll
    for (int j = 0; j < kGroups4; j++) {
        if (4 * t + 1024 * j < ffn) {
            const float4 gi = v[j];
            v[j] = make_float4((gi.x / (1.0f + exp_poly(-gi.x))) * uv[j].x, (gi.y / (1.0f + exp_poly(-gi.y))) * uv[j].y,
                               (gi.z / (1.0f + exp_poly(-gi.z))) * uv[j].z, (gi.w / (1.0f + exp_poly(-gi.w))) * uv[j].w);
            peak = max_abs4(peak, v[j]);
        }
    }
    peak = block_max(peak, wmax);
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    const float inverse = 1.0f / scale;
    int8_t* qr = q + (size_t)blockIdx.x * ffn;
#pragma unroll
    for (int j = 0; j < kGroups4; j++) {
        const int i = 4 * t + 1024 * j;
        if (i < ffn) *reinterpret_cast<uint32_t*>(qr + i) = pack_q4(v[j], inverse);
    }
    if (t == 0) qscale[blockIdx.x] = scale;
}

// (value, id) order of TopKLogSoftmax: larger value first, equal values by
// the lower id.
__device__ __forceinline__ bool before(float va, int ia, float vb, int ib)
{
    return va > vb || (va == vb && ia < ib);
}

__device__ __forceinline__ bool masked(int i) { return i == 0 || i == 2 || i == 3; }

// TopKLogSoftmax (src/Needle/Ops.cs:1092-1221) in the canonical float form.
// The ids are the reference's selection (Ops.cs:1094-1166) for NaN-free
// rows: id 1 (always) and every id from 4 on holding a value above -inf are
// candidates, the top K of them under the order above fill the slots (the
// set is unique under that order, so merging per-thread and per-block lists
// equals the sequential insertion), slots left over hold (-inf, -1), and when
// no id from 4 on is above -inf while x[4] is -inf, the last slot, if left
// over, holds (-inf, 4): the reference's scan admits its first value even at
// -inf and drops it at the next entry.  log_shift = peak + log(S), masked v_i = -1e30, with
// S over blocks of kTopkBlock ids: S_b = sum Exp(v_i - m_b) (m_b the block
// maximum, the canonical row reduction over the block's ids) and S = sum_b
// Exp(m_b - peak) * S_b in ascending b; lp = v - log_shift.  One workgroup
// per (block, row) computes the block's top K, m_b and S_b; a second kernel
// merges a row's blocks.  K is a template parameter so that the per-thread
// lists stay in registers.
constexpr int kTopkBlock = 2048;
constexpr int kTopkMaxBlocks = 256;                           // vocab <= 524288
constexpr int kTopkMaxCandidates = kTopkMaxBlocks * kMaxTopK;  // the final merge's LDS

template <int K>
__global__ __launch_bounds__(kThreads) void topk_block_kernel(const float* logits, int n, int blocks, float* bvals,
                                                             int32_t* bids, float* bmax, float* bsum)
{
    __shared__ float tv[K][kThreads];
    __shared__ int ti[K][kThreads];
    __shared__ __align__(16) float red[kThreads + 8];  // partials, the broadcast sum, 4 wave maxima
    const int t = threadIdx.x;
    const int b = blockIdx.x;
    const int row = blockIdx.y;
    const float* x = logits + (size_t)row * n;
    const int b0 = b * kTopkBlock;
    // ids b0 + 4t + 1024h + e (h < 2): the block's canonical lane t
    float xv[8];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int g = b0 + 4 * t + 1024 * h;
        if ((n & 3) == 0) {
            const float4 v = *reinterpret_cast<const float4*>(x + min(g, n - 4));
            xv[4 * h] = v.x;
            xv[4 * h + 1] = v.y;
            xv[4 * h + 2] = v.z;
            xv[4 * h + 3] = v.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) xv[4 * h + e] = x[min(g + e, n - 1)];
        }
    }
    float bv[K];
    int bi[K];
#pragma unroll
    for (int m = 0; m < K; m++) {
        bv[m] = -INFINITY;
        bi[m] = 0x7FFFFFFF;
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int i = b0 + 4 * t + 1024 * (j >> 2) + (j & 3);
        if (i >= n) continue;
        xv[j] = masked(i) ? -1e30f : xv[j];
        mloc = fmaxf(mloc, xv[j]);
        // the reference's scan admits a value only above -inf (its first
        // scanned id aside, which the final merge restores), except id 1,
        // which it places first whatever its value
        if (masked(i) || (!(xv[j] > -INFINITY) && i != 1) || !before(xv[j], i, bv[K - 1], bi[K - 1])) continue;
        bv[K - 1] = xv[j];
        bi[K - 1] = i;
#pragma unroll
        for (int m = K - 1; m > 0; m--) {
            if (before(bv[m], bi[m], bv[m - 1], bi[m - 1])) {
                const float fv = bv[m];
                const int fi = bi[m];
                bv[m] = bv[m - 1];
                bi[m] = bi[m - 1];
                bv[m - 1] = fv;
                bi[m - 1] = fi;
            }
        }
    }
    const float mb = block_max(mloc, red + kThreads + 4);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int i = b0 + 4 * t + 1024 * (j >> 2) + (j & 3);
        if (i < n) s = s + exp_poly(xv[j] - mb);
    }
    const float sb = block_canonical_sum(s, red);
#pragma unroll
    for (int m = 0; m < K; m++) {
        tv[m][t] = bv[m];
        ti[m][t] = bi[m];
    }
    __syncthreads();
    for (int stride = 128; stride > 0; stride >>= 1) {
        if (t < stride) {
            float av[K], cv[K];
            int ai[K], ci[K];
#pragma unroll
            for (int m = 0; m < K; m++) {
                av[m] = tv[m][t];
                ai[m] = ti[m][t];
                cv[m] = tv[m][t + stride];
                ci[m] = ti[m][t + stride];
            }
            // merge two sorted lists, keeping the first K (compile-time indices)
#pragma unroll
            for (int m = 0; m < K; m++) {
                const bool take_a = before(av[0], ai[0], cv[0], ci[0]);
                tv[m][t] = take_a ? av[0] : cv[0];
                ti[m][t] = take_a ? ai[0] : ci[0];
#pragma unroll
                for (int q = 0; q < K - 1; q++) {
                    av[q] = take_a ? av[q + 1] : av[q];
                    ai[q] = take_a ? ai[q + 1] : ai[q];
                    cv[q] = take_a ? cv[q] : cv[q + 1];
                    ci[q] = take_a ? ci[q] : ci[q + 1];
                }
                av[K - 1] = take_a ? -INFINITY : av[K - 1];
                ai[K - 1] = take_a ? 0x7FFFFFFF : ai[K - 1];
                cv[K - 1] = take_a ? cv[K - 1] : -INFINITY;
                ci[K - 1] = take_a ? ci[K - 1] : 0x7FFFFFFF;
            }
        }
        __syncthreads();
    }
    const size_t slot = (size_t)row * blocks + b;
    if (t < K) {
        bvals[slot * K + t] = tv[t][0];
        bids[slot * K + t] = ti[t][0];
    }
    if (t == 0) {
        bmax[slot] = mb;
        bsum[slot] = sb;
    }
}

// Merge of a row's block lists (sequential insertion in the (value, id)
// order) and S = sum_b Exp(m_b - peak) * S_b in ascending b.
template <int K>
__global__ __launch_bounds__(64) void topk_final_kernel(const float* logits, int width, const float* bvals,
                                                         const int32_t* bids, const float* bmax, const float* bsum,
                                                         int blocks, int32_t* idx, float* lp)
{
    // The row's top K of the blocks' candidates under `before` (value, then
    // the lower id).  That order is total on the candidates (never NaN; the
    // blocks' (-inf, INT_MAX) placeholders are identical to each other), so
    // the result is the K first candidates in that order, whatever the
    // sequence of comparisons: every thread ranks its candidates against all
    // others in parallel (equal candidates by their index) and rank m goes to
    // slot m.
    __shared__ float sv[kTopkMaxCandidates];
    __shared__ int si[kTopkMaxCandidates];
    __shared__ float best_v[K];
    __shared__ int best_i[K];
    __shared__ float prod[kTopkMaxBlocks];
    const int tid = threadIdx.x;
    const int row = blockIdx.x;
    const size_t base = (size_t)row * blocks;
    const int n = blocks * K;
    // the log-sum-exp's block maxima and sums, and the special case's logit,
    // load with the candidates: nothing between depends on them
    constexpr int kPerThread = kTopkMaxBlocks / 64;
    float bm[kPerThread], bs[kPerThread];
#pragma unroll
    for (int q = 0; q < kPerThread; q++) {
        const int b = tid + 64 * q;
        if (b < blocks) {
            bm[q] = bmax[base + b];
            bs[q] = bsum[base + b];
        }
    }
    const float logit4 = tid == 0 && width > 4 ? logits[(size_t)row * width + 4] : 0.0f;
    for (int j = tid; j < n; j += 64) {
        sv[j] = bvals[base * K + j];
        si[j] = bids[base * K + j];
    }
    if (tid < K) {
        best_v[tid] = -INFINITY;
        best_i[tid] = 0x7FFFFFFF;
    }
    __syncthreads();
    for (int c = tid; c < n; c += 64) {
        const float v = sv[c];
        const int i = si[c];
        int rank = 0;
#pragma unroll 8
        for (int o = 0; o < n; o++) {  // unrolled: the LDS reads of 8 candidates issue together
            const float ov = sv[o];
            const int oi = si[o];
            rank += (before(ov, oi, v, i) || (ov == v && oi == i && o < c)) ? 1 : 0;
        }
        if (rank < K && v == v) {
            best_v[rank] = v;
            best_i[rank] = i;
        }
    }
    __syncthreads();
    if (tid == 0 && best_i[K - 1] == 0x7FFFFFFF && width > 4) {
        // fewer than K candidates: the reference keeps its first scanned id
        // (4) in the last slot when it was -inf and no later id entered
        bool later = false;
#pragma unroll
        for (int m = 0; m < K; m++) later = later || (best_i[m] != 1 && best_i[m] != 0x7FFFFFFF);
        if (!later && logit4 == -INFINITY) best_i[K - 1] = 4;
    }
    __syncthreads();
    // log-sum-exp over the blocks in ascending order: the terms
    // Exp(max_b - peak) * sum_b in parallel, then their sum in order
    const float peak = best_v[0];
#pragma unroll
    for (int q = 0; q < kPerThread; q++) {
        const int b = tid + 64 * q;
        if (b < blocks) prod[b] = exp_poly(bm[q] - peak) * bs[q];
    }
    __syncthreads();
    if (tid != 0) return;
    float total = 0.0f;
#pragma unroll 8
    for (int b = 0; b < blocks; b++) total = total + prod[b];
    const float log_shift = peak + log_poly(total);
#pragma unroll
    for (int m = 0; m < K; m++) {
        idx[(size_t)row * K + m] = best_i[m] == 0x7FFFFFFF ? -1 : best_i[m];
        lp[(size_t)row * K + m] = best_v[m] - log_shift;
    }
}

// Scratch of the top-k: per (row, block) K values and ids, the block maximum
// and sum.
struct TopkScratch {
    float* vals;
    int32_t* ids;
    float* bmax;
    float* bsum;
};

int32_t launch_topk(const float* logits, int rows, int n, int k, const TopkScratch& ts, int32_t* idx, float* lp,
                    hipStream_t s)
{
    const int blocks = (n + kTopkBlock - 1) / kTopkBlock;
    NHIP_REQUIRE(blocks <= kTopkMaxBlocks, "top-k: at most %d ids per row (got %d)", kTopkMaxBlocks * kTopkBlock, n);
    switch (k) {
#define NHIP_TOPK_CASE(K)                                                                                        \
    case K:                                                                                                      \
        hipLaunchKernelGGL(topk_block_kernel<K>, dim3(blocks, rows), dim3(kThreads), 0, s, logits, n, blocks,    \
                           ts.vals, ts.ids, ts.bmax, ts.bsum);                                                   \
        hipLaunchKernelGGL(topk_final_kernel<K>, dim3(rows), dim3(64), 0, s, logits, n, ts.vals, ts.ids, ts.bmax, \
                           ts.bsum, blocks, idx, lp);                                                            \
        break;
        NHIP_TOPK_CASE(1)
        NHIP_TOPK_CASE(2)
        NHIP_TOPK_CASE(3)
        NHIP_TOPK_CASE(4)
        NHIP_TOPK_CASE(5)
        NHIP_TOPK_CASE(6)
        NHIP_TOPK_CASE(7)
        NHIP_TOPK_CASE(8)
#undef NHIP_TOPK_CASE
        default:
            set_error("top-k %d outside [1, 8]", k);
            return NHIP_ERR_ARG;
    }
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

// Ops.ArgMaxMasked per row (src/Needle/Ops.cs:1223-1266): the scalar form
// scans the allowed ids in ascending order and takes a value only when it is
// strictly above the best so far (from -inf), so the result is the lowest id
// holding the largest allowed value above -inf (NaN never is), or -1.  Here
// each of 1024 threads keeps the best (value, id) of the ids tid, tid + 1024,
// ... (ascending, strict >; eight ids' mask words and values loaded
// together), and the block reduces the pairs with "larger value, then lower
// id", which gives the same id.  Values of ids that are not allowed are
// loaded but never compared.
constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxBatch = 8;

__global__ __launch_bounds__(kArgmaxThreads) void argmax_masked_kernel(const float* x, int ldx, const uint32_t* mask,
                                                                       int mask_ld, int words, int length,
                                                                       int32_t* index, float* value)
{
    __shared__ float sv[kArgmaxThreads / 64];
    __shared__ int si[kArgmaxThreads / 64];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* xr = x + (size_t)row * ldx;
    const uint32_t* mr = mask + (size_t)row * mask_ld;
    const int n = min(length, words * 32);
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int base = tid; base < n; base += kArgmaxThreads * kArgmaxBatch) {
        uint32_t mw[kArgmaxBatch];
        float v[kArgmaxBatch];
#pragma unroll
        for (int j = 0; j < kArgmaxBatch; j++) {
            const int i = min(base + j * kArgmaxThreads, n - 1);
            mw[j] = mr[i >> 5];
            v[j] = xr[i];
        }
#pragma unroll
        for (int j = 0; j < kArgmaxBatch; j++) {
            const int i = base + j * kArgmaxThreads;
            if (i < n && ((mw[j] >> (i & 31)) & 1u) && v[j] > bv) {
                bv = v[j];
                bi = i;
            }
        }
    }
    auto better = [](float v, int i, float bv2, int bi2) { return v > bv2 || (v == bv2 && i < bi2); };
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((tid & 63) == 0) {
        sv[tid >> 6] = bv;
        si[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; w++)
            if (better(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
        const bool found = bi != 0x7FFFFFFF;
        index[row] = found ? bi : -1;
        if (value) value[row] = found ? bv : -INFINITY;
    }
}

int32_t launch_argmax_masked(const float* x, int ldx, const uint32_t* mask, int mask_ld, int words, int length,
                             int rows, int32_t* index, float* value, hipStream_t s)
{
    hipLaunchKernelGGL(argmax_masked_kernel, dim3(rows), dim3(kArgmaxThreads), 0, s, x, ldx, mask, mask_ld, words,
                       length, index, value);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

// Ops.ArgMax per row (src/Needle/Ops.cs:1052-1090).  The scalar loop starts
// at id 0 and moves to id i only when x[i] > x[best], so: 0 when x[0] is
// NaN, otherwise the lowest id holding the largest non-NaN value (+0 and -0
// are equal, every -inf row gives 0).  The AVX path (first id equal to the
// maximum) gives the same id on every NaN-free row.  Each of 1024 threads
// keeps the best (value, id) of ids tid, tid + 1024, ... ("larger value,
// then lower id", NaN never taken) and the block reduces the pairs in the
// same order.
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* x, int ldx, int n, int32_t* index,
                                                                float* value)
{
    __shared__ float sv[kArgmaxThreads / 64];
    __shared__ int si[kArgmaxThreads / 64];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* xr = x + (size_t)row * ldx;
    auto better = [](float v, int i, float bv2, int bi2) { return v > bv2 || (v == bv2 && i < bi2); };
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int base = tid; base < n; base += kArgmaxThreads * kArgmaxBatch) {
        float v[kArgmaxBatch];
#pragma unroll
        for (int j = 0; j < kArgmaxBatch; j++) v[j] = xr[min(base + j * kArgmaxThreads, n - 1)];
#pragma unroll
        for (int j = 0; j < kArgmaxBatch; j++) {
            const int i = base + j * kArgmaxThreads;
            if (i < n && better(v[j], i, bv, bi)) {
                bv = v[j];
                bi = i;
            }
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((tid & 63) == 0) {
        sv[tid >> 6] = bv;
        si[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; w++)
            if (better(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
        const float x0 = xr[0];
        if (x0 != x0 || bi == 0x7FFFFFFF) {  // NaN at id 0 (or every value NaN with it)
            bi = 0;
            bv = x0;
        }
        index[row] = bi;
        if (value) value[row] = bv;
    }
}

int32_t launch_argmax(const float* x, int ldx, int n, int rows, int32_t* index, float* value, hipStream_t s)
{
    hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(kArgmaxThreads), 0, s, x, ldx, n, index, value);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

// Copies positions [0, length) of slot src to slot dst in every layer's
// four cache pools (Engine.CopyFrom).
__global__ void kv_copy_kernel(int8_t* keys, int8_t* values, float* key_scales, float* value_scales, int slots,
                               int capacity, int kv_heads, int dst, int src, int length)
{
    const int layer = blockIdx.y;
    const size_t base = (size_t)layer * slots * capacity;
    const size_t a = (base + (size_t)dst * capacity) * kv_heads;
    const size_t b = (base + (size_t)src * capacity) * kv_heads;
    const size_t cells = (size_t)length * kv_heads;
    const size_t n16 = cells * 64 / 16;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint4* ks = reinterpret_cast<const uint4*>(keys + b * 64);
    const uint4* vs = reinterpret_cast<const uint4*>(values + b * 64);
    uint4* kd = reinterpret_cast<uint4*>(keys + a * 64);
    uint4* vd = reinterpret_cast<uint4*>(values + a * 64);
    for (size_t i = tid; i < n16; i += stride) {
        kd[i] = ks[i];
        vd[i] = vs[i];
    }
    for (size_t i = tid; i < cells; i += stride) {
        key_scales[a + i] = key_scales[b + i];
        value_scales[a + i] = value_scales[b + i];
    }
}

}  // namespace
}  // namespace nhip

using namespace nhip;

// What a forward computes after its layers: the LM head over `heads` of its
// rows (all of them, in order, when `all_rows`), then the top-k (k > 0) or
// Ops.ArgMax (`argmax`) of each head row.
struct HeadPlan {
    int heads = 0;
    bool all_rows = true;
    int k = 0;
    bool argmax = false;
    bool operator==(const HeadPlan& o) const
    {
        return heads == o.heads && all_rows == o.all_rows && k == o.k && argmax == o.argmax;
    }
};

// A decode step captured as a graph: its row count and head plan.  Replays
// read the step's inputs (tokens, slots, positions, spans, head rows) from
// device memory the host refreshes before each launch.
struct StepGraph {
    int rows;
    HeadPlan head;
    hipGraphExec_t exec;
};

struct nhip_decoder {
    nhip_decoder_dims dims{};
    int qkv_n = 0;
    std::vector<nhip_weights*> wqkv, wo, wgu, wd;
    nhip_weights* wlm = nullptr;
    std::vector<float*> attn_norm, ffn_norm;
    float* final_norm = nullptr;
    float* emb = nullptr;
    float* rope_cos = nullptr;
    float* rope_sin = nullptr;
    std::vector<float> rope_cos_h, rope_sin_h;  // host copies of the tables
    int8_t* keys = nullptr;
    int8_t* values = nullptr;
    float* key_scales = nullptr;
    float* value_scales = nullptr;
    // activations for up to max_rows rows
    float* x = nullptr;
    float* x2 = nullptr;  // the other residual buffer of the fused forward
    float* delta = nullptr;
    int8_t* q8 = nullptr;
    float* qs = nullptr;
    float* qkv = nullptr;
    int8_t* qh = nullptr;
    float* qhs = nullptr;
    float* att = nullptr;
    float* gu = nullptr;
    float* act = nullptr;  // SwiGLU activations [rows][ffn] of the fused gate/up matmul
    float* logits = nullptr;
    int32_t* d_in = nullptr;  // tokens, slots, positions, first (0), count, head rows: 6 x max_rows
    // masked (grammar) head: id bitsets [rows][mask_words] and the chosen ids
    int32_t mask_words = 0;
    uint32_t* d_mask = nullptr;
    int32_t best_rows = 0;  // rows of d_best / d_best_val: max(max_rows, kMaxMaskedRows)
    int32_t* d_best = nullptr;
    float* d_best_val = nullptr;
    uint32_t* h_mask = nullptr;
    int32_t* h_best = nullptr;
    float* h_best_val = nullptr;
    int32_t* d_topk_idx = nullptr;
    TopkScratch topk{};  // per (row, block) partial top-k lists, maxima and sums
    float* d_topk_lp = nullptr;
    int32_t* h_in = nullptr;  // pinned host mirror of d_in
    int32_t* h_topk_idx = nullptr;
    float* h_topk_lp = nullptr;
    void* attn_ws = nullptr;
    size_t attn_ws_bytes = 0;
    hipStream_t stream = nullptr;
    std::vector<StepGraph> graphs;  // captured decode steps, by their shape
    std::vector<int32_t> slot_len, slot_mark;  // the step API's slot lengths and marks
    std::vector<void*> allocations;
};

namespace {

template <typename T>
int32_t dalloc(nhip_decoder* m, T** p, size_t count)
{
    void* v = nullptr;
    NHIP_CHECK_HIP(hipMalloc(&v, std::max<size_t>(count * sizeof(T), 256)));
    m->allocations.push_back(v);
    *p = static_cast<T*>(v);
    return NHIP_OK;
}

int32_t* in_tokens(nhip_decoder* m, int32_t* base) { return base; }
int32_t* in_slots(nhip_decoder* m, int32_t* base) { return base + m->dims.max_rows; }
int32_t* in_positions(nhip_decoder* m, int32_t* base) { return base + 2 * m->dims.max_rows; }
int32_t* in_first(nhip_decoder* m, int32_t* base) { return base + 3 * m->dims.max_rows; }
int32_t* in_count(nhip_decoder* m, int32_t* base) { return base + 4 * m->dims.max_rows; }
int32_t* in_heads(nhip_decoder* m, int32_t* base) { return base + 5 * m->dims.max_rows; }
// [max_rows][64]: the RoPE table's cos then sin row (32 each) of each row's
// position, staged with the step so that the attention reads them without a
// load that depends on the position
float* in_rope(nhip_decoder* m, int32_t* base) { return reinterpret_cast<float*>(base + 6 * m->dims.max_rows); }

// Residual + RMSNorm + quantize feeding a matmul.  For up to four rows and
// at most kFusedPrologueMaxTiles row tiles one fused launch computes the
// normalised rows in the matmul's prologue, reading *x and the pending delta
// and writing their sum to the other residual buffer (which then becomes
// *x); otherwise the element-wise kernel updates *x in place and the plain
// matmul follows.  Either way the residual ends in *x with the delta added.
// With `act` (the gate/up matmul) and up to four rows the matmul's chain
// applies SwiGLU to the tile-interleaved rows and writes the activations to
// act[rows][ffn], setting *fused; otherwise the interleaved rows go to y.
int32_t norm_matmul(nhip_decoder* m, int rows, float** x, bool pending, const float* gain, nhip_weights* w,
                    float* y, int ldy, bool fuse, float* act = nullptr, bool* fused = nullptr)
{
    const nhip_decoder_dims& D = m->dims;
    hipStream_t s = m->stream;
    if (fused) *fused = false;
    if (fuse && w->tiles_n <= kFusedPrologueMaxTiles) {
        float* other = *x == m->x ? m->x2 : m->x;
        DecodePrologue f{kProNorm, *x, pending ? m->delta : nullptr, pending ? other : nullptr, gain, D.eps,
                         act ? 1 : 0};
        const int32_t rc = act ? launch_decode_fused(w, f, rows, act, D.ffn, s) : launch_decode_fused(w, f, rows, y, ldy, s);
        if (rc <= 0) {
            if (rc == 0 && pending) *x = other;
            if (rc == 0 && fused) *fused = true;
            return rc;
        }
    }
    if (pending)
        hipLaunchKernelGGL(add_rmsnorm_quant_kernel<true>, dim3(rows), dim3(kThreads), 0, s, *x, m->delta, gain, D.d,
                           D.eps, m->q8, m->qs, nullptr);
    else
        hipLaunchKernelGGL(add_rmsnorm_quant_kernel<false>, dim3(rows), dim3(kThreads), 0, s, *x, nullptr, gain, D.d,
                           D.eps, m->q8, m->qs, nullptr);
    NHIP_CHECK_HIP(hipGetLastError());
    if (act && fuse) {
        const int32_t rc = launch_decode_swiglu(w, m->q8, m->qs, rows, act, D.ffn, s);
        if (rc <= 0) {
            if (rc == 0) *fused = true;
            return rc;
        }
    }
    return nhip_matmul_i8_dev(w, m->q8, m->qs, rows, y, ldy, 0, w->rows, s);
}

// Enqueues the forward of `rows` rows whose inputs are already in d_in,
// with the head of `hp` (ignored by the masked head).
int32_t enqueue_forward(nhip_decoder* m, int rows, const HeadPlan& hp, bool masked = false)
{
    // NHIP_DECODER_FUSED=0 keeps the element-wise kernels separate (for A/B timing)
    static const bool fused_enabled = [] {
        const char* e = getenv("NHIP_DECODER_FUSED");
        return !(e && e[0] == '0');
    }();
    const bool fuse = fused_enabled && rows <= 4;
    const nhip_decoder_dims& D = m->dims;
    const int d = D.d, H = D.heads, KV = D.kv_heads, F = D.ffn;
    hipStream_t s = m->stream;
    int32_t rc;
    float* x = m->x;
    // pending: m->delta holds an output not yet added to the residual x (the
    // fused output and down matmuls add it in their own chain instead and
    // write the new residual to the other buffer)
    bool pending = false;
    auto other_of = [m](const float* cur) { return cur == m->x ? m->x2 : m->x; };
    hipLaunchKernelGGL(embed_kernel, dim3(rows), dim3(kThreads), 0, s, in_tokens(m, m->d_in), m->emb, d, x);
    NHIP_CHECK_HIP(hipGetLastError());
    const size_t layer_cells = (size_t)D.slots * D.capacity * KV;
    for (int l = 0; l < D.layers; l++) {
        rc = norm_matmul(m, rows, &x, pending, m->attn_norm[l], m->wqkv[l], m->qkv, m->qkv_n, fuse);
        pending = false;
        if (rc) return rc;
        PostParams pp{};
        pp.qkv = m->qkv;
        pp.slots = in_slots(m, m->d_in);
        pp.positions = in_positions(m, m->d_in);
        pp.rope_cos = m->rope_cos;
        pp.rope_sin = m->rope_sin;
        pp.q8 = m->qh;
        pp.qs = m->qhs;
        pp.keys = m->keys + (size_t)l * layer_cells * 64;
        pp.values = m->values + (size_t)l * layer_cells * 64;
        pp.key_scales = m->key_scales + (size_t)l * layer_cells;
        pp.value_scales = m->value_scales + (size_t)l * layer_cells;
        pp.heads = H;
        pp.kv_heads = KV;
        pp.capacity = D.capacity;
        // single-chunk attention with every head in one workgroup also
        // quantizes its output rows
        const bool attn_quant =
            D.max_chunks == 1 &&
            decode_attention_kv_per_block(H / KV, KV, decode_attention_lmax(D.capacity, D.max_chunks)) >= KV;
        rc = 1;
        if (fuse && !attn_quant) {  // RoPE, quantize and the KV write inside the attention launch
            const AttnPostInputs in{m->qkv, pp.positions, in_rope(m, m->d_in)};
            rc = attention_decode_post_impl(in, rows, H, KV, pp.keys, pp.key_scales, pp.values, pp.value_scales,
                                            D.slots, D.capacity, pp.slots, in_first(m, m->d_in),
                                            in_count(m, m->d_in), D.max_chunks, m->att, s);
            if (rc < 0) return rc;
        }
        if (rc) {
            hipLaunchKernelGGL(qkv_post_kernel, dim3(rows, H + 2 * KV), dim3(64), 0, s, pp);
            NHIP_CHECK_HIP(hipGetLastError());
            rc = attention_decode_impl(m->qh, m->qhs, rows, H, KV, 64, pp.keys, pp.key_scales, pp.values,
                                       pp.value_scales, D.slots, D.capacity, pp.slots, in_first(m, m->d_in),
                                       in_count(m, m->d_in), D.max_chunks, m->attn_ws, m->attn_ws_bytes, m->att,
                                       attn_quant ? m->q8 : nullptr, attn_quant ? m->qs : nullptr, s);
            if (rc) return rc;
        }
        rc = 1;
        if (!attn_quant && fuse) {
            DecodePrologue f{kProQuant, m->att, nullptr, nullptr, nullptr, 0.0f, 0, x};
            rc = launch_decode_fused(m->wo[l], f, rows, other_of(x), d, s);
            if (rc < 0) return rc;
            if (rc == 0) x = other_of(x);
        }
        if (rc) {
            pending = true;
            if (!attn_quant) {
                rc = nhip_quantize_rows_dev(m->att, rows, H * 64, m->q8, m->qs, s);
                if (rc) return rc;
            }
            rc = nhip_matmul_i8_dev(m->wo[l], m->q8, m->qs, rows, m->delta, d, 0, d, s);
            if (rc) return rc;
        }
        bool act_ready = false;  // SwiGLU applied by the gate/up matmul (into m->act)
        rc = norm_matmul(m, rows, &x, pending, m->ffn_norm[l], m->wgu[l], m->gu, 2 * F, fuse, m->act, &act_ready);
        if (rc) return rc;
        pending = true;
        if (act_ready) {  // quantize the activations in the down matmul's prologue
            DecodePrologue f{kProQuant, m->act, nullptr, nullptr, nullptr, 0.0f, 0, x};
            rc = launch_decode_fused(m->wd[l], f, rows, other_of(x), d, s);
            if (rc < 0) return rc;
            if (rc == 0) {
                x = other_of(x);
                pending = false;
            } else {
                rc = nhip_quantize_rows_dev(m->act, rows, F, m->q8, m->qs, s);
                if (rc) return rc;
                rc = nhip_matmul_i8_dev(m->wd[l], m->q8, m->qs, rows, m->delta, d, 0, d, s);
                if (rc) return rc;
            }
        } else {  // interleaved gate/up rows -> SwiGLU + quantize -> down matmul
            hipLaunchKernelGGL(swiglu_quant_kernel, dim3(rows), dim3(kThreads), 0, s, m->gu, F, m->q8, m->qs);
            NHIP_CHECK_HIP(hipGetLastError());
            rc = nhip_matmul_i8_dev(m->wd[l], m->q8, m->qs, rows, m->delta, d, 0, d, s);
            if (rc) return rc;
        }
    }
    if (masked) {
        // the sparse head: the final norm, the LM head over the vocab tiles
        // that hold an allowed id of some row, and ArgMaxMasked per row
        if (pending)
            hipLaunchKernelGGL(add_rmsnorm_quant_kernel<true>, dim3(rows), dim3(kThreads), 0, s, x, m->delta,
                               m->final_norm, d, D.eps, m->q8, m->qs, nullptr);
        else
            hipLaunchKernelGGL(add_rmsnorm_quant_kernel<false>, dim3(rows), dim3(kThreads), 0, s, x, nullptr,
                               m->final_norm, d, D.eps, m->q8, m->qs, nullptr);
        NHIP_CHECK_HIP(hipGetLastError());
        rc = launch_decode_masked(m->wlm, m->q8, m->qs, rows, m->logits, D.vocab, m->d_mask, m->mask_words, s);
        if (rc) return rc;
        return launch_argmax_masked(m->logits, D.vocab, m->d_mask, m->mask_words, m->mask_words, D.vocab, rows,
                                    m->d_best, m->d_best_val, s);
    }
    // the final residual is not needed again: no x_out.  The head runs over
    // the plan's rows only (EngineCore.ForwardBatch's headRows,
    // src/Needle/Engine.cs:2341-2348): row i of the logits is row
    // head_rows[i] of the forward.
    const int heads = hp.all_rows ? rows : hp.heads;
    if (heads == 0) return NHIP_OK;
    rc = 1;
    if (hp.all_rows && fuse && m->wlm->tiles_n <= kFusedPrologueMaxTiles) {
        DecodePrologue f{kProNorm, x, pending ? m->delta : nullptr, nullptr, m->final_norm, D.eps, 0};
        rc = launch_decode_fused(m->wlm, f, rows, m->logits, D.vocab, s);
        if (rc < 0) return rc;
    }
    if (rc) {
        if (pending)
            hipLaunchKernelGGL(add_rmsnorm_quant_kernel<true>, dim3(heads), dim3(kThreads), 0, s, x, m->delta,
                               m->final_norm, d, D.eps, m->q8, m->qs, hp.all_rows ? nullptr : in_heads(m, m->d_in));
        else
            hipLaunchKernelGGL(add_rmsnorm_quant_kernel<false>, dim3(heads), dim3(kThreads), 0, s, x, nullptr,
                               m->final_norm, d, D.eps, m->q8, m->qs, hp.all_rows ? nullptr : in_heads(m, m->d_in));
        NHIP_CHECK_HIP(hipGetLastError());
        rc = nhip_matmul_i8_dev(m->wlm, m->q8, m->qs, heads, m->logits, D.vocab, 0, D.vocab, s);
        if (rc) return rc;
    }
    if (hp.k > 0) {
        rc = launch_topk(m->logits, heads, D.vocab, hp.k, m->topk, m->d_topk_idx, m->d_topk_lp, s);
        if (rc) return rc;
    }
    if (hp.argmax) return launch_argmax(m->logits, D.vocab, D.vocab, heads, m->d_best, m->d_best_val, s);
    return NHIP_OK;
}

int32_t stage_inputs(nhip_decoder* m, const int32_t* tokens, const int32_t* slots, const int32_t* positions,
                     int rows, const int32_t* head_rows = nullptr, int heads = 0)
{
    const nhip_decoder_dims& D = m->dims;
    for (int r = 0; r < rows; r++) {
        NHIP_REQUIRE(tokens[r] >= 0 && tokens[r] < D.vocab, "token %d out of range", tokens[r]);
        NHIP_REQUIRE(slots[r] >= 0 && slots[r] < D.slots, "slot %d out of range", slots[r]);
        NHIP_REQUIRE(positions[r] >= 0 && positions[r] < D.capacity, "position %d outside the cache capacity %d",
                     positions[r], D.capacity);
        in_tokens(m, m->h_in)[r] = tokens[r];
        in_slots(m, m->h_in)[r] = slots[r];
        in_positions(m, m->h_in)[r] = positions[r];
        in_first(m, m->h_in)[r] = 0;
        in_count(m, m->h_in)[r] = positions[r] + 1;
        float* rope = in_rope(m, m->h_in) + (size_t)r * 64;
        std::memcpy(rope, m->rope_cos_h.data() + (size_t)positions[r] * 32, 32 * sizeof(float));
        std::memcpy(rope + 32, m->rope_sin_h.data() + (size_t)positions[r] * 32, 32 * sizeof(float));
    }
    for (int i = 0; i < heads; i++) {
        NHIP_REQUIRE(head_rows[i] >= 0 && head_rows[i] < rows, "head row %d outside [0, %d)", head_rows[i], rows);
        in_heads(m, m->h_in)[i] = head_rows[i];
    }
    // the id arrays and the RoPE rows of the staged rows, in one copy
    NHIP_CHECK_HIP(hipMemcpyAsync(m->d_in, m->h_in, sizeof(int32_t) * 6 * D.max_rows + sizeof(float) * 64 * rows,
                                  hipMemcpyHostToDevice, m->stream));
    return NHIP_OK;
}

// Forward of staged inputs with the results of the top-k / argmax copied
// to the pinned mirrors; steps of up to kMaxGraphRows rows replay a graph
// captured on first use for their (rows, head plan).
constexpr int kMaxGraphRows = 16;
constexpr size_t kMaxGraphs = 64;

int32_t run_staged(nhip_decoder* m, int rows, const HeadPlan& hp, bool use_graph)
{
    // NHIP_DECODER_GRAPHS=0 launches decode steps eagerly (for kernel tracers)
    static const bool graphs_enabled = [] {
        const char* e = getenv("NHIP_DECODER_GRAPHS");
        return !(e && e[0] == '0');
    }();
    int32_t rc;
    use_graph = use_graph && graphs_enabled && rows <= kMaxGraphRows;
    if (use_graph) {
        hipGraphExec_t exec = nullptr;
        for (const StepGraph& g : m->graphs)
            if (g.rows == rows && g.head == hp) exec = g.exec;
        if (!exec) {
            if (m->graphs.size() >= kMaxGraphs) {  // drop the oldest
                NHIP_CHECK_HIP(hipStreamSynchronize(m->stream));
                (void)hipGraphExecDestroy(m->graphs.front().exec);
                m->graphs.erase(m->graphs.begin());
            }
            hipGraph_t g;
            NHIP_CHECK_HIP(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
            rc = enqueue_forward(m, rows, hp);
            hipError_t e = hipStreamEndCapture(m->stream, &g);
            if (rc) {
                if (e == hipSuccess) (void)hipGraphDestroy(g);
                return rc;
            }
            NHIP_CHECK_HIP(e);
            e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            NHIP_CHECK_HIP(e);
            m->graphs.push_back(StepGraph{rows, hp, exec});
        }
        NHIP_CHECK_HIP(hipGraphLaunch(exec, m->stream));
    } else {
        rc = enqueue_forward(m, rows, hp);
        if (rc) return rc;
    }
    const int heads = hp.all_rows ? rows : hp.heads;
    if (hp.k > 0 && heads > 0) {
        // ids and log-probabilities in one copy (the log-probabilities follow
        // the ids' region of max_rows * kMaxTopK entries)
        const size_t span = reinterpret_cast<const char*>(m->d_topk_lp + (size_t)heads * hp.k) -
                            reinterpret_cast<const char*>(m->d_topk_idx);
        NHIP_CHECK_HIP(hipMemcpyAsync(m->h_topk_idx, m->d_topk_idx, span, hipMemcpyDeviceToHost, m->stream));
    }
    if (hp.argmax && heads > 0) {
        NHIP_CHECK_HIP(hipMemcpyAsync(m->h_best, m->d_best, sizeof(int32_t) * 2 * m->best_rows, hipMemcpyDeviceToHost,
                                      m->stream));
    }
    NHIP_CHECK_HIP(hipStreamSynchronize(m->stream));
    return NHIP_OK;
}

int32_t forward_step(nhip_decoder* m, const int32_t* tokens, const int32_t* slots, const int32_t* positions,
                     int rows, int k, bool use_graph)
{
    int32_t rc = stage_inputs(m, tokens, slots, positions, rows);
    if (rc) return rc;
    HeadPlan hp;
    hp.k = k;
    return run_staged(m, rows, hp, use_graph);
}

int32_t copy_slot(nhip_decoder* m, int dst, int src, int length)
{
    const nhip_decoder_dims& D = m->dims;
    NHIP_REQUIRE(dst >= 0 && dst < D.slots && src >= 0 && src < D.slots, "slot out of range");
    NHIP_REQUIRE(length >= 0 && length <= D.capacity, "length %d outside [0, %d]", length, D.capacity);
    if (length == 0 || dst == src) return NHIP_OK;
    const size_t cells = (size_t)length * D.kv_heads;
    const int grid = (int)std::min<size_t>((cells * 4 + 255) / 256, 1024);
    hipLaunchKernelGGL(kv_copy_kernel, dim3(std::max(grid, 1), D.layers), dim3(256), 0, m->stream, m->keys, m->values,
                       m->key_scales, m->value_scales, D.slots, D.capacity, D.kv_heads, dst, src, length);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

// Captured decode graphs hold the weights' device pointers: weights that
// change (set_layer / set_head) drop them, and the next decode step
// captures again.  The stream is drained first so that no replay is running.
void drop_graphs(nhip_decoder* m)
{
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    for (StepGraph& g : m->graphs) (void)hipGraphExecDestroy(g.exec);
    m->graphs.clear();
}

int32_t upload(nhip_decoder* m, float** dst, const float* src, size_t count)
{
    int32_t rc = dalloc(m, dst, count);
    if (rc) return rc;
    NHIP_CHECK_HIP(hipMemcpy(*dst, src, count * sizeof(float), hipMemcpyHostToDevice));
    return NHIP_OK;
}

}  // namespace

extern "C" {

int32_t nhip_decoder_create(const nhip_decoder_dims* dims, nhip_decoder** out)
{
    clear_error();
    NHIP_REQUIRE(dims && out, "null argument");
    const nhip_decoder_dims& D = *dims;
    NHIP_REQUIRE(D.layers > 0 && D.d > 0 && D.d % 32 == 0 && D.d <= kMaxPerThread * kThreads,
                 "d_model %d must be a positive multiple of 32 up to %d", D.d, kMaxPerThread * kThreads);
    NHIP_REQUIRE(D.head_dim == 64, "head_dim must be 64");
    NHIP_REQUIRE(D.heads > 0 && D.kv_heads > 0 && D.heads % D.kv_heads == 0 && D.heads / D.kv_heads <= 16,
                 "heads/kv_heads");
    NHIP_REQUIRE(D.heads * 64 % 32 == 0 && D.ffn > 0 && D.ffn % 32 == 0 && D.ffn <= kMaxPerThread * kThreads,
                 "ffn %d must be a positive multiple of 32 up to %d", D.ffn, kMaxPerThread * kThreads);
    NHIP_REQUIRE(D.vocab > 4 && D.capacity > 0 && D.slots > 0 && D.max_rows > 0 && D.max_chunks > 0,
                 "vocab, capacity, slots, max_rows, max_chunks");
    NHIP_REQUIRE(D.vocab <= kTopkMaxBlocks * kTopkBlock, "vocab %d above the top-k's %d", D.vocab,
                 kTopkMaxBlocks * kTopkBlock);
    int32_t rc = ensure_device();
    if (rc) return rc;
    nhip_decoder* m = new nhip_decoder();
    m->dims = D;
    m->qkv_n = (D.heads + 2 * D.kv_heads) * 64;
    m->wqkv.assign(D.layers, nullptr);
    m->wo.assign(D.layers, nullptr);
    m->wgu.assign(D.layers, nullptr);
    m->wd.assign(D.layers, nullptr);
    m->attn_norm.assign(D.layers, nullptr);
    m->ffn_norm.assign(D.layers, nullptr);
    const size_t cells = (size_t)D.layers * D.slots * D.capacity * D.kv_heads;
    const int R = D.max_rows;
    m->best_rows = std::max(R, kMaxMaskedRows);
    m->slot_len.assign(D.slots, 0);
    m->slot_mark.assign(D.slots, 0);
    auto fail = [&](int32_t code) {
        nhip_decoder_destroy(m);
        return code;
    };
    if ((rc = dalloc(m, &m->keys, cells * 64)) || (rc = dalloc(m, &m->values, cells * 64)) ||
        (rc = dalloc(m, &m->key_scales, cells)) || (rc = dalloc(m, &m->value_scales, cells)) ||
        (rc = dalloc(m, &m->x, (size_t)R * D.d)) || (rc = dalloc(m, &m->x2, (size_t)R * D.d)) ||
        (rc = dalloc(m, &m->delta, (size_t)R * D.d)) ||
        (rc = dalloc(m, &m->q8, (size_t)R * std::max({D.d, D.ffn, D.heads * 64}))) || (rc = dalloc(m, &m->qs, (size_t)R)) ||
        (rc = dalloc(m, &m->qkv, (size_t)R * m->qkv_n)) || (rc = dalloc(m, &m->qh, (size_t)R * D.heads * 64)) ||
        (rc = dalloc(m, &m->qhs, (size_t)R * D.heads)) || (rc = dalloc(m, &m->att, (size_t)R * D.heads * 64)) ||
        (rc = dalloc(m, &m->gu, (size_t)R * 2 * D.ffn)) || (rc = dalloc(m, &m->act, (size_t)R * D.ffn)) || (rc = dalloc(m, &m->logits, (size_t)R * D.vocab)) ||
        (rc = dalloc(m, &m->d_in, (size_t)(6 + 64) * R)) || (rc = dalloc(m, &m->d_topk_idx, (size_t)2 * R * kMaxTopK)) ||
        (rc = dalloc(m, &m->d_mask, (size_t)kMaxMaskedRows * ((D.vocab + 31) / 32))) ||
        (rc = dalloc(m, &m->d_best, (size_t)2 * m->best_rows)) ||
        (rc = dalloc(m, &m->topk.vals, (size_t)R * ((D.vocab + kTopkBlock - 1) / kTopkBlock) * kMaxTopK)) ||
        (rc = dalloc(m, &m->topk.ids, (size_t)R * ((D.vocab + kTopkBlock - 1) / kTopkBlock) * kMaxTopK)) ||
        (rc = dalloc(m, &m->topk.bmax, (size_t)R * ((D.vocab + kTopkBlock - 1) / kTopkBlock))) ||
        (rc = dalloc(m, &m->topk.bsum, (size_t)R * ((D.vocab + kTopkBlock - 1) / kTopkBlock))))
        return fail(rc);
    m->attn_ws_bytes = nhip_attention_decode_workspace(R, D.heads, D.max_chunks);
    void* ws = nullptr;
    if (hipMalloc(&ws, m->attn_ws_bytes) != hipSuccess) {
        set_error("hipMalloc of %zu bytes for the attention workspace failed", m->attn_ws_bytes);
        return fail(NHIP_ERR_HIP);
    }
    m->allocations.push_back(ws);
    m->attn_ws = ws;
    m->mask_words = (D.vocab + 31) / 32;
    m->d_best_val = reinterpret_cast<float*>(m->d_best + m->best_rows);  // one copy returns both
    // the top-k ids, then their log-probabilities: one copy returns both
    m->d_topk_lp = reinterpret_cast<float*>(m->d_topk_idx + (size_t)R * kMaxTopK);
    if (hipHostMalloc(reinterpret_cast<void**>(&m->h_in), sizeof(int32_t) * (6 + 64) * R, hipHostMallocDefault) !=
            hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&m->h_topk_idx), sizeof(int32_t) * 2 * R * kMaxTopK,
                      hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&m->h_mask), sizeof(uint32_t) * kMaxMaskedRows * ((D.vocab + 31) / 32),
                      hipHostMallocDefault) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&m->h_best), sizeof(int32_t) * 2 * m->best_rows,
                      hipHostMallocDefault) != hipSuccess) {
        set_error("hipHostMalloc failed");
        return fail(NHIP_ERR_HIP);
    }
    m->h_best_val = reinterpret_cast<float*>(m->h_best + m->best_rows);
    m->h_topk_lp = reinterpret_cast<float*>(m->h_topk_idx + (size_t)R * kMaxTopK);
    if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess) {
        set_error("hipStreamCreate failed");
        return fail(NHIP_ERR_HIP);
    }
    // RoPE table: cos/sin of p * theta^(-2i/64) in double, rounded to float
    std::vector<float> c((size_t)D.capacity * 32), sn((size_t)D.capacity * 32);
    for (int p = 0; p < D.capacity; p++)
        for (int i = 0; i < 32; i++) {
            const double angle = (double)p * std::pow(D.theta, -2.0 * i / 64);
            c[(size_t)p * 32 + i] = (float)std::cos(angle);
            sn[(size_t)p * 32 + i] = (float)std::sin(angle);
        }
    if ((rc = upload(m, &m->rope_cos, c.data(), c.size())) || (rc = upload(m, &m->rope_sin, sn.data(), sn.size())))
        return fail(rc);
    m->rope_cos_h = std::move(c);
    m->rope_sin_h = std::move(sn);
    if (hipMemset(m->keys, 0, cells * 64) != hipSuccess || hipMemset(m->values, 0, cells * 64) != hipSuccess ||
        hipMemset(m->key_scales, 0, cells * 4) != hipSuccess || hipMemset(m->value_scales, 0, cells * 4) != hipSuccess) {
        set_error("hipMemset failed");
        return fail(NHIP_ERR_HIP);
    }
    *out = m;
    return NHIP_OK;
}

int32_t nhip_decoder_set_layer(nhip_decoder* m, int32_t layer, const int8_t* wqkv, const uint16_t* sqkv,
                               const int8_t* wo, const uint16_t* so, const int8_t* wgu, const uint16_t* sgu,
                               const int8_t* wd, const uint16_t* sd, const float* attn_norm, const float* ffn_norm)
{
    clear_error();
    NHIP_REQUIRE(m && layer >= 0 && layer < m->dims.layers, "bad decoder or layer %d", layer);
    NHIP_REQUIRE(wqkv && sqkv && wo && so && wgu && sgu && wd && sd && attn_norm && ffn_norm, "null weights");
    const nhip_decoder_dims& D = m->dims;
    int32_t rc;
    drop_graphs(m);
    nhip_weights** slots[4] = {&m->wqkv[layer], &m->wo[layer], &m->wgu[layer], &m->wd[layer]};
    // the gate/up rows are uploaded tile-interleaved: rows 16b..16b+7 are
    // gate rows 8b..8b+7, rows 16b+8..16b+15 the matching up rows
    const int F = D.ffn, G = D.d / 32;
    std::vector<int8_t> wgu_i((size_t)2 * F * D.d);
    std::vector<uint16_t> sgu_i((size_t)2 * F * G);
    for (int n = 0; n < 2 * F; n++) {
        const int b = n >> 4, e = n & 15;
        const int src = e < 8 ? 8 * b + e : F + 8 * b + (e - 8);
        std::memcpy(&wgu_i[(size_t)n * D.d], wgu + (size_t)src * D.d, D.d);
        std::memcpy(&sgu_i[(size_t)n * G], sgu + (size_t)src * G, sizeof(uint16_t) * G);
    }
    const int8_t* ws[4] = {wqkv, wo, wgu_i.data(), wd};
    const uint16_t* ss[4] = {sqkv, so, sgu_i.data(), sd};
    const int rows[4] = {m->qkv_n, D.d, 2 * D.ffn, D.d};
    const int cols[4] = {D.d, D.heads * 64, D.d, D.ffn};
    for (int i = 0; i < 4; i++) {
        if (*slots[i]) nhip_weights_destroy(*slots[i]);
        *slots[i] = nullptr;
        if ((rc = nhip_weights_i8_create(ws[i], ss[i], rows[i], cols[i], slots[i]))) return rc;
    }
    if (!m->attn_norm[layer] && (rc = dalloc(m, &m->attn_norm[layer], D.d))) return rc;
    if (!m->ffn_norm[layer] && (rc = dalloc(m, &m->ffn_norm[layer], D.d))) return rc;
    NHIP_CHECK_HIP(hipMemcpy(m->attn_norm[layer], attn_norm, sizeof(float) * D.d, hipMemcpyHostToDevice));
    NHIP_CHECK_HIP(hipMemcpy(m->ffn_norm[layer], ffn_norm, sizeof(float) * D.d, hipMemcpyHostToDevice));
    return NHIP_OK;
}

int32_t nhip_decoder_set_head(nhip_decoder* m, const float* embedding, const float* final_norm, const int8_t* wlm,
                              const uint16_t* slm)
{
    clear_error();
    NHIP_REQUIRE(m && embedding && final_norm && wlm && slm, "null argument");
    const nhip_decoder_dims& D = m->dims;
    int32_t rc;
    drop_graphs(m);
    if (!m->emb && (rc = dalloc(m, &m->emb, (size_t)D.vocab * D.d))) return rc;
    if (!m->final_norm && (rc = dalloc(m, &m->final_norm, D.d))) return rc;
    NHIP_CHECK_HIP(hipMemcpy(m->emb, embedding, sizeof(float) * D.vocab * D.d, hipMemcpyHostToDevice));
    NHIP_CHECK_HIP(hipMemcpy(m->final_norm, final_norm, sizeof(float) * D.d, hipMemcpyHostToDevice));
    if (m->wlm) nhip_weights_destroy(m->wlm);
    m->wlm = nullptr;
    return nhip_weights_i8_create(wlm, slm, D.vocab, D.d, &m->wlm);
}

static int32_t ready(const nhip_decoder* m)
{
    NHIP_REQUIRE(m, "null decoder");
    NHIP_REQUIRE(m->wlm && m->emb, "decoder head not set");
    for (int l = 0; l < m->dims.layers; l++) NHIP_REQUIRE(m->wqkv[l], "decoder layer %d not set", l);
    return NHIP_OK;
}

int32_t nhip_decoder_forward(nhip_decoder* m, const int32_t* tokens, const int32_t* slots, const int32_t* positions,
                             int32_t rows, float* logits, int32_t k, int32_t* topk_idx, float* topk_lp)
{
    clear_error();
    int32_t rc = ready(m);
    if (rc) return rc;
    NHIP_REQUIRE(rows > 0 && rows <= m->dims.max_rows, "rows %d outside [1, %d]", rows, m->dims.max_rows);
    NHIP_REQUIRE(k >= 0 && k <= kMaxTopK && (k == 0 || (topk_idx && topk_lp)), "k %d outside [0, %d]", k, kMaxTopK);
    NHIP_REQUIRE(tokens && slots && positions, "null inputs");
    rc = forward_step(m, tokens, slots, positions, rows, k, false);
    if (rc) return rc;
    if (k > 0) {
        std::memcpy(topk_idx, m->h_topk_idx, sizeof(int32_t) * rows * k);
        std::memcpy(topk_lp, m->h_topk_lp, sizeof(float) * rows * k);
    }
    if (logits)
        NHIP_CHECK_HIP(hipMemcpy(logits, m->logits, sizeof(float) * rows * m->dims.vocab, hipMemcpyDeviceToHost));
    return NHIP_OK;
}

int32_t nhip_decoder_forward_masked(nhip_decoder* m, const int32_t* tokens, const int32_t* slots,
                                    const int32_t* positions, int32_t rows, const uint32_t* masks, int32_t words,
                                    int32_t* best, float* best_logit)
{
    clear_error();
    int32_t rc = ready(m);
    if (rc) return rc;
    NHIP_REQUIRE(rows > 0 && rows <= std::min(m->dims.max_rows, kMaxMaskedRows), "rows %d outside [1, %d]", rows,
                 std::min(m->dims.max_rows, kMaxMaskedRows));
    NHIP_REQUIRE(tokens && slots && positions && masks && best && words > 0, "null inputs or words %d <= 0", words);
    rc = stage_inputs(m, tokens, slots, positions, rows);
    if (rc) return rc;
    // ids from vocab on (and words past the caller's) are not allowed
    const int MW = m->mask_words;
    const int keep = std::min(words, MW);
    for (int r = 0; r < rows; r++) {
        uint32_t* dst = m->h_mask + (size_t)r * MW;
        std::memcpy(dst, masks + (size_t)r * words, sizeof(uint32_t) * keep);
        for (int w = keep; w < MW; w++) dst[w] = 0u;
        const int tail = m->dims.vocab - 32 * (MW - 1);  // valid bits of the last word
        if (keep == MW && tail < 32) dst[MW - 1] &= (1u << tail) - 1u;
    }
    NHIP_CHECK_HIP(hipMemcpyAsync(m->d_mask, m->h_mask, sizeof(uint32_t) * rows * MW, hipMemcpyHostToDevice,
                                  m->stream));
    rc = enqueue_forward(m, rows, HeadPlan{}, true);
    if (rc) return rc;
    NHIP_CHECK_HIP(hipMemcpyAsync(m->h_best, m->d_best, sizeof(int32_t) * 2 * m->best_rows, hipMemcpyDeviceToHost,
                                  m->stream));
    NHIP_CHECK_HIP(hipStreamSynchronize(m->stream));
    std::memcpy(best, m->h_best, sizeof(int32_t) * rows);
    if (best_logit) std::memcpy(best_logit, m->h_best_val, sizeof(float) * rows);
    return NHIP_OK;
}

int32_t nhip_argmax_masked_dev(const float* d_x, int32_t ldx, const uint32_t* d_mask, int32_t mask_ld, int32_t words,
                               int32_t length, int32_t rows, int32_t* d_index, float* d_value, void* stream)
{
    clear_error();
    NHIP_REQUIRE(rows >= 0 && words >= 0 && length >= 0 && ldx >= 0 && mask_ld >= 0, "negative size");
    if (rows == 0) return NHIP_OK;
    NHIP_REQUIRE(d_x && d_mask && d_index, "null pointer");
    NHIP_REQUIRE(rows == 1 || (ldx >= length && mask_ld >= words),
                 "row strides (%d floats, %d words) shorter than a row (%d, %d)", ldx, mask_ld, length, words);
    int32_t rc = ensure_device();
    if (rc) return rc;
    return launch_argmax_masked(d_x, ldx, d_mask, mask_ld, words, length, rows, d_index, d_value, as_stream(stream));
}

// Workspace of nhip_topk_lse_dev: the decoder's TopkScratch arrays, each
// 256-byte aligned.
static size_t topk_ws_layout(int32_t rows, int32_t n, TopkScratch* ts, uint8_t* base)
{
    const size_t blocks = ((size_t)n + kTopkBlock - 1) / kTopkBlock;
    const size_t lists = (size_t)rows * blocks * kMaxTopK, per = (size_t)rows * blocks;
    auto a256 = [](size_t x) { return (x + 255) & ~size_t(255); };
    const size_t o_ids = a256(lists * sizeof(float));
    const size_t o_max = o_ids + a256(lists * sizeof(int32_t));
    const size_t o_sum = o_max + a256(per * sizeof(float));
    if (ts) {
        ts->vals = reinterpret_cast<float*>(base);
        ts->ids = reinterpret_cast<int32_t*>(base + o_ids);
        ts->bmax = reinterpret_cast<float*>(base + o_max);
        ts->bsum = reinterpret_cast<float*>(base + o_sum);
    }
    return o_sum + a256(per * sizeof(float));
}

size_t nhip_topk_lse_workspace(int32_t rows, int32_t n)
{
    if (rows <= 0 || n <= 0) return 0;
    return topk_ws_layout(rows, n, nullptr, nullptr);
}

int32_t nhip_topk_lse_dev(const float* d_logits, int32_t rows, int32_t n, int32_t k, void* d_workspace,
                          size_t workspace_bytes, int32_t* d_idx, float* d_lp, void* stream)
{
    clear_error();
    NHIP_REQUIRE(rows >= 0 && n >= 1 && k >= 1 && k <= kMaxTopK, "rows %d, n %d, k %d (1..%d)", rows, n, k, kMaxTopK);
    NHIP_REQUIRE(n <= kTopkMaxBlocks * kTopkBlock, "at most %d logits per row", kTopkMaxBlocks * kTopkBlock);
    if (rows == 0) return NHIP_OK;
    NHIP_REQUIRE(d_logits && d_workspace && d_idx && d_lp, "null pointer");
    NHIP_REQUIRE((reinterpret_cast<uintptr_t>(d_logits) & 15) == 0 && (reinterpret_cast<uintptr_t>(d_workspace) & 255) == 0,
                 "logits must be 16-byte aligned and the workspace 256-byte aligned");
    TopkScratch ts{};
    const size_t need = topk_ws_layout(rows, n, &ts, static_cast<uint8_t*>(d_workspace));
    NHIP_REQUIRE(workspace_bytes >= need, "workspace of %zu bytes, need %zu", workspace_bytes, need);
    int32_t rc = ensure_device();
    if (rc) return rc;
    return launch_topk(d_logits, rows, n, k, ts, d_idx, d_lp, as_stream(stream));
}

int32_t nhip_decoder_copy_slot(nhip_decoder* m, int32_t dst, int32_t src, int32_t length)
{
    clear_error();
    NHIP_REQUIRE(m, "null decoder");
    int32_t rc = copy_slot(m, dst, src, length);
    if (rc) return rc;
    m->slot_len[dst] = length;  // Engine.CopyFrom takes the source's length
    NHIP_CHECK_HIP(hipStreamSynchronize(m->stream));
    return NHIP_OK;
}

// EngineCore.ForwardBatch (src/Needle/Engine.cs:2303-2350): positions from
// the slots' lengths (row t of a run of slot s sits at len[s] + t - run
// start, Engine.cs:2655-2661), lengths advanced by the runs afterwards.
int32_t nhip_decoder_step(nhip_decoder* m, const int32_t* tokens, const int32_t* row_slots, int32_t rows,
                          const int32_t* head_rows, int32_t heads, float* logits, int32_t k, int32_t* topk_idx,
                          float* topk_lp, int32_t* argmax)
{
    clear_error();
    int32_t rc = ready(m);
    if (rc) return rc;
    const nhip_decoder_dims& D = m->dims;
    NHIP_REQUIRE(rows > 0 && rows <= D.max_rows, "rows %d outside [1, %d]", rows, D.max_rows);
    NHIP_REQUIRE(heads >= 0 && heads <= rows, "heads %d outside [0, %d]", heads, rows);
    NHIP_REQUIRE(tokens && row_slots && (heads == 0 || head_rows), "null inputs");
    NHIP_REQUIRE(k >= 0 && k <= kMaxTopK && (k == 0 || (topk_idx && topk_lp)), "k %d outside [0, %d]", k, kMaxTopK);
    std::vector<int32_t> pos(rows);
    std::vector<char> seen(D.slots, 0);
    for (int rs = 0; rs < rows;) {
        const int slot = row_slots[rs];
        NHIP_REQUIRE(slot >= 0 && slot < D.slots, "slot %d out of range", slot);
        NHIP_REQUIRE(!seen[slot], "the rows of slot %d must be one contiguous run", slot);
        seen[slot] = 1;
        int rk = rs;
        while (rk + 1 < rows && row_slots[rk + 1] == slot) rk++;
        NHIP_REQUIRE(m->slot_len[slot] + (rk - rs + 1) <= D.capacity, "slot %d: context capacity %d exceeded", slot,
                     D.capacity);
        for (int t = rs; t <= rk; t++) pos[t] = m->slot_len[slot] + t - rs;
        rs = rk + 1;
    }
    rc = stage_inputs(m, tokens, row_slots, pos.data(), rows, head_rows, heads);
    if (rc) return rc;
    HeadPlan hp;
    hp.heads = heads;
    hp.all_rows = false;
    hp.k = heads > 0 ? k : 0;
    hp.argmax = heads > 0 && argmax != nullptr;
    rc = run_staged(m, rows, hp, true);
    if (rc) return rc;
    for (int t = 0; t < rows; t++) m->slot_len[row_slots[t]] = std::max(m->slot_len[row_slots[t]], pos[t] + 1);
    if (heads > 0 && k > 0) {
        std::memcpy(topk_idx, m->h_topk_idx, sizeof(int32_t) * heads * k);
        std::memcpy(topk_lp, m->h_topk_lp, sizeof(float) * heads * k);
    }
    if (hp.argmax) std::memcpy(argmax, m->h_best, sizeof(int32_t) * heads);
    if (logits && heads > 0)
        NHIP_CHECK_HIP(hipMemcpy(logits, m->logits, sizeof(float) * heads * D.vocab, hipMemcpyDeviceToHost));
    return NHIP_OK;
}

// BatchedEngine.ResetSlot / MarkSlot / RewindSlot / SlotLength
// (src/Needle/BatchEngine.cs:25-30; Engine.cs:2227-2276).  The cache rows
// past a slot's length are never read, so a reset or a rewind only moves the
// length; a mark records it.
int32_t nhip_decoder_slot_reset(nhip_decoder* m, int32_t slot)
{
    clear_error();
    NHIP_REQUIRE(m && slot >= 0 && slot < m->dims.slots, "slot %d out of range", slot);
    m->slot_len[slot] = 0;
    m->slot_mark[slot] = 0;
    return NHIP_OK;
}

int32_t nhip_decoder_slot_mark(nhip_decoder* m, int32_t slot)
{
    clear_error();
    NHIP_REQUIRE(m && slot >= 0 && slot < m->dims.slots, "slot %d out of range", slot);
    m->slot_mark[slot] = m->slot_len[slot];
    return NHIP_OK;
}

int32_t nhip_decoder_slot_rewind(nhip_decoder* m, int32_t slot)
{
    clear_error();
    NHIP_REQUIRE(m && slot >= 0 && slot < m->dims.slots, "slot %d out of range", slot);
    m->slot_len[slot] = m->slot_mark[slot];
    return NHIP_OK;
}

int32_t nhip_decoder_slot_length(const nhip_decoder* m, int32_t slot, int32_t* length)
{
    clear_error();
    NHIP_REQUIRE(m && slot >= 0 && slot < m->dims.slots && length, "slot %d out of range", slot);
    *length = m->slot_len[slot];
    return NHIP_OK;
}

// ToolCaller.Complete's loop (src/Needle/ToolCaller.cs:59-77) on slot 0:
// reset, feed the prompt in chunks of max_rows rows with the head on its
// last row only (BatchedEngine.FeedSlot, Engine.cs:2286-2301), then per
// step Ops.ArgMax of the head row (Engine.Greedy, Engine.cs:103) on the
// device; stop before a token equal to `stop` (-1: none), otherwise record
// it and feed it as a one-row step (a replayed graph).
int32_t nhip_decoder_greedy(nhip_decoder* m, const int32_t* prompt, int32_t prompt_len, int32_t max_new,
                            int32_t stop, int32_t* out_tokens, int32_t* out_len, nhip_decode_stats* stats)
{
    clear_error();
    int32_t rc = ready(m);
    if (rc) return rc;
    const nhip_decoder_dims& D = m->dims;
    NHIP_REQUIRE(prompt && prompt_len > 0 && max_new >= 0 && out_len && (max_new == 0 || out_tokens),
                 "prompt length %d, max_new %d", prompt_len, max_new);
    NHIP_REQUIRE(prompt_len + max_new <= D.capacity, "prompt + new tokens exceed the capacity %d", D.capacity);
    using clock = std::chrono::steady_clock;
    const auto t0 = clock::now();
    m->slot_len[0] = 0;  // slot 0 starts over, as nhip_decoder_slot_reset leaves it
    m->slot_mark[0] = 0;
    std::vector<int32_t> sl(std::min(prompt_len, D.max_rows), 0);
    int32_t next = 0;
    for (int start = 0; start < prompt_len; start += D.max_rows) {
        const int count = std::min(D.max_rows, prompt_len - start);
        const bool last = start + count == prompt_len;
        const int32_t head = count - 1;
        rc = nhip_decoder_step(m, prompt + start, sl.data(), count, &head, last ? 1 : 0, nullptr, 0, nullptr, nullptr,
                               last ? &next : nullptr);
        if (rc) return rc;
    }
    const auto t1 = clock::now();
    int n = 0;
    const int32_t zero = 0;
    for (int step = 0; step < max_new; step++) {
        if (next == stop) break;
        out_tokens[n++] = next;
        rc = nhip_decoder_step(m, &next, &zero, 1, &zero, 1, nullptr, 0, nullptr, nullptr, &next);
        if (rc) return rc;
    }
    const auto t2 = clock::now();
    *out_len = n;
    if (stats) {
        stats->prefill_seconds = std::chrono::duration<double>(t1 - t0).count();
        stats->decode_seconds = std::chrono::duration<double>(t2 - t1).count();
        stats->fed_rows = n;
        stats->steps = n;
    }
    return NHIP_OK;
}

int32_t nhip_argmax_dev(const float* d_x, int32_t ldx, int32_t n, int32_t rows, int32_t* d_index, float* d_value,
                        void* stream)
{
    clear_error();
    NHIP_REQUIRE(rows >= 0 && n >= 1 && ldx >= 0, "rows %d, n %d", rows, n);
    if (rows == 0) return NHIP_OK;
    NHIP_REQUIRE(d_x && d_index, "null pointer");
    NHIP_REQUIRE(rows == 1 || ldx >= n, "row stride %d shorter than a row (%d)", ldx, n);
    int32_t rc = ensure_device();
    if (rc) return rc;
    return launch_argmax(d_x, ldx, n, rows, d_index, d_value, as_stream(stream));
}

int32_t nhip_decoder_beam_search(nhip_decoder* m, const int32_t* prompt, int32_t prompt_len, int32_t width,
                                 int32_t max_new, int32_t eos, int32_t* out_tokens, int32_t* out_len, float* out_score,
                                 nhip_decode_stats* stats)
{
    clear_error();
    int32_t rc = ready(m);
    if (rc) return rc;
    const nhip_decoder_dims& D = m->dims;
    NHIP_REQUIRE(prompt && prompt_len > 0 && prompt_len <= D.max_rows, "prompt length %d outside [1, %d]", prompt_len,
                 D.max_rows);
    NHIP_REQUIRE(width >= 1 && width <= kMaxTopK && width <= D.slots && width <= D.max_rows,
                 "beam width %d needs width <= %d, slots and max_rows", width, kMaxTopK);
    NHIP_REQUIRE(max_new >= 0 && prompt_len + max_new <= D.capacity, "prompt + new tokens exceed the capacity %d",
                 D.capacity);
    NHIP_REQUIRE(out_tokens && out_len && out_score, "null outputs");
    const int W = width;
    using clock = std::chrono::steady_clock;
    const auto t0 = clock::now();
    // prefill the prompt into slot 0; the top-k of its last row (the only
    // head row) starts the search
    std::vector<int32_t> pos(prompt_len), sl(prompt_len, 0);
    for (int i = 0; i < prompt_len; i++) pos[i] = i;
    const int32_t last = prompt_len - 1;
    rc = stage_inputs(m, prompt, sl.data(), pos.data(), prompt_len, &last, 1);
    if (rc) return rc;
    HeadPlan prefill_head;
    prefill_head.heads = 1;
    prefill_head.all_rows = false;
    prefill_head.k = W;
    rc = run_staged(m, prompt_len, prefill_head, false);
    if (rc) return rc;
    std::vector<int32_t> top_idx(m->h_topk_idx, m->h_topk_idx + W);
    std::vector<float> top_lp(m->h_topk_lp, m->h_topk_lp + W);
    const auto t1 = clock::now();

    struct Cand {
        float score;
        int parent, token;
    };
    struct Fin {
        float score;
        std::vector<int32_t> tokens;
    };
    std::vector<std::vector<int32_t>> live_tok(1), next_tok;
    std::vector<float> live_score(1, 0.0f);
    std::vector<int> live_slot(1, 0);
    std::vector<Fin> finished;
    int live_count = 1;
    long fed = 0;
    int steps = 0;
    for (int step = 0; step < max_new; step++) {
        std::vector<Cand> cand;
        for (int i = 0; i < live_count; i++)
            for (int k = 0; k < W; k++) cand.push_back({live_score[i] + top_lp[(size_t)i * W + k], i, top_idx[(size_t)i * W + k]});
        std::stable_sort(cand.begin(), cand.end(), [](const Cand& a, const Cand& b) { return a.score > b.score; });
        std::vector<int> parents, picks;
        std::vector<float> pick_scores;
        for (const Cand& c : cand) {
            if (c.token == eos)
                finished.push_back({c.score, live_tok[c.parent]});
            else {
                parents.push_back(c.parent);
                picks.push_back(c.token);
                pick_scores.push_back(c.score);
            }
            if ((int)parents.size() >= W) break;
        }
        const int kept = (int)parents.size();
        if (kept == 0) break;
        if ((int)finished.size() >= W) {
            float best_fin = -INFINITY, best_live = -INFINITY;
            for (const Fin& f : finished) best_fin = std::max(best_fin, f.score / (float)(f.tokens.size() + 1));
            for (int j = 0; j < kept; j++)
                best_live = std::max(best_live, pick_scores[j] / (float)(live_tok[parents[j]].size() + 1));
            if (best_fin >= best_live) break;
        }
        std::vector<int> last_child(live_count, -1), next_slot(kept);
        for (int j = 0; j < kept; j++) last_child[parents[j]] = j;
        std::vector<char> used(D.slots, 0);
        for (int j = 0; j < kept; j++)
            if (j == last_child[parents[j]]) used[live_slot[parents[j]]] = 1;
        next_tok.assign(kept, {});
        std::vector<int32_t> feed_tok(kept), feed_slot(kept), feed_pos(kept);
        for (int j = 0; j < kept; j++) {
            const int p = parents[j];
            if (j == last_child[p]) {
                next_slot[j] = live_slot[p];
            } else {
                int f = 0;
                while (used[f]) f++;
                used[f] = 1;
                rc = copy_slot(m, f, live_slot[p], prompt_len + (int)live_tok[p].size());
                if (rc) return rc;
                next_slot[j] = f;
            }
            next_tok[j] = live_tok[p];
            next_tok[j].push_back(picks[j]);
            feed_tok[j] = picks[j];
            feed_slot[j] = next_slot[j];
            feed_pos[j] = prompt_len + (int)live_tok[p].size();
        }
        rc = forward_step(m, feed_tok.data(), feed_slot.data(), feed_pos.data(), kept, W, true);
        if (rc) return rc;
        fed += kept;
        steps++;
        top_idx.assign(m->h_topk_idx, m->h_topk_idx + (size_t)kept * W);
        top_lp.assign(m->h_topk_lp, m->h_topk_lp + (size_t)kept * W);
        live_tok.swap(next_tok);
        live_slot = next_slot;
        live_score = pick_scores;
        live_count = kept;
    }
    const auto t2 = clock::now();
    const std::vector<int32_t>* winner = nullptr;
    float winner_score = -INFINITY;
    for (const Fin& f : finished) {
        const float sc = f.score / (float)(f.tokens.size() + 1);
        if (sc > winner_score) {
            winner_score = sc;
            winner = &f.tokens;
        }
    }
    if (!winner)
        for (int j = 0; j < live_count; j++) {
            const float sc = live_score[j] / (float)live_tok[j].size();
            if (sc > winner_score) {
                winner_score = sc;
                winner = &live_tok[j];
            }
        }
    *out_len = winner ? (int32_t)winner->size() : 0;
    if (winner) std::copy(winner->begin(), winner->end(), out_tokens);
    *out_score = winner_score;
    if (stats) {
        stats->prefill_seconds = std::chrono::duration<double>(t1 - t0).count();
        stats->decode_seconds = std::chrono::duration<double>(t2 - t1).count();
        stats->fed_rows = fed;
        stats->steps = steps;
    }
    return NHIP_OK;
}

int32_t nhip_decoder_destroy(nhip_decoder* m)
{
    if (!m) return NHIP_OK;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    for (StepGraph& g : m->graphs) (void)hipGraphExecDestroy(g.exec);
    for (auto* w : m->wqkv) nhip_weights_destroy(w);
    for (auto* w : m->wo) nhip_weights_destroy(w);
    for (auto* w : m->wgu) nhip_weights_destroy(w);
    for (auto* w : m->wd) nhip_weights_destroy(w);
    nhip_weights_destroy(m->wlm);
    for (void* p : m->allocations) (void)hipFree(p);
    if (m->h_in) (void)hipHostFree(m->h_in);
    if (m->h_topk_idx) (void)hipHostFree(m->h_topk_idx);
    if (m->h_mask) (void)hipHostFree(m->h_mask);
    if (m->h_best) (void)hipHostFree(m->h_best);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
    return NHIP_OK;
}

}  // extern "C"

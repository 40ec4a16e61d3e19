// attention.hip -- attention over the int8 KV cache on gfx950: the
// reference's AttentionTile / MergePartials kernel-table entries.
//
// Scores, softmax and value accumulation follow Scalar.AttentionHead
// (src/Needle/Scalar.cs:290-312): score_s = (float(dot_s) * keyScale_s) *
// (queryScale * 1/sqrt(qkDim)); the exponential is the reference's
// polynomial Ops.Exp (src/Needle/Ops.cs:16-31, shared bit-for-bit with the
// CPU restatement via exp_poly below); normalisation multiplies the
// accumulated sum_s (e_s * valueScale_s) * v_s by 1/sum_s e_s as the SIMD
// tile does (Blocks.cs:188-199, 415-435).  Position sums run in a fixed tree
// order, so results match the scalar reference to the reference's own
// conformance bound (5e-5 of the output peak), not bit for bit.
#include "common.hpp"

namespace nhip {

namespace {

constexpr int kMaxTileHeads = 6;
constexpr int kPartialFloats = kMaxTileHeads * 64 + 16;  // Blocks.cs:42-43
constexpr int kTileThreads = 256;

__device__ __forceinline__ float block_reduce_max(float v, float* red)
{
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ __forceinline__ float block_reduce_sum(float v, float* red)
{
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// One block per head.  keys/values/scales point at position `first`.
__global__ __launch_bounds__(kTileThreads) void tile_kernel(
    const int8_t* __restrict__ queries, const float* __restrict__ query_scales, const int8_t* __restrict__ keys,
    const float* __restrict__ key_scales, const int8_t* __restrict__ values, const float* __restrict__ value_scales,
    int key_stride, int value_stride, int scale_stride, int count, int qk_dim, float inv_sqrt,
    float* __restrict__ output, float* __restrict__ probabilities, int prob_stride, float* __restrict__ peaks,
    float* __restrict__ sums)
{
    extern __shared__ float scores[];
    __shared__ float red[4];
    __shared__ float part[4][64];
    const int h = blockIdx.x;
    const int8_t* q = queries + h * qk_dim;
    const float scale = query_scales[h] * inv_sqrt;
    float local_peak = -INFINITY;
    for (int s = threadIdx.x; s < count; s += kTileThreads) {
        const int8_t* k = keys + (size_t)s * key_stride;
        int dot = 0;
        for (int d = 0; d < qk_dim; d++) dot += (int)q[d] * (int)k[d];
        const float sc = ((float)dot * key_scales[(size_t)s * scale_stride]) * scale;
        scores[s] = sc;
        local_peak = fmaxf(local_peak, sc);
    }
    const float peak = block_reduce_max(local_peak, red);
    float local_sum = 0.0f;
    for (int s = threadIdx.x; s < count; s += kTileThreads) {
        const float e = exp_poly(scores[s] - peak);
        scores[s] = e;
        local_sum += e;
    }
    const float sum = block_reduce_sum(local_sum, red);
    const float inverse = peaks ? 1.0f : 1.0f / sum;
    if (probabilities)
        for (int s = threadIdx.x; s < count; s += kTileThreads)
            probabilities[h * prob_stride + s] = scores[s] * inverse;
    const int d = threadIdx.x & 63;
    const int quarter = threadIdx.x >> 6;
    float acc = 0.0f;
    for (int s = quarter; s < count; s += 4) {
        const float w = scores[s] * value_scales[(size_t)s * scale_stride];
        acc = __builtin_fmaf(w, (float)values[(size_t)s * value_stride + d], acc);
    }
    part[quarter][d] = acc;
    __syncthreads();
    if (threadIdx.x < 64) {
        const float total = (part[0][d] + part[1][d]) + (part[2][d] + part[3][d]);
        output[h * 64 + d] = total * inverse;
        if (peaks && d == 0) {
            peaks[h] = peak;
            sums[h] = sum;
        }
    }
}

// Blocks.cs:750-817: one thread per (head, dim).
__global__ void merge_kernel(const float* __restrict__ partials, int count, int heads, float* __restrict__ output)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= heads * 64) return;
    const int h = i >> 6;
    const int d = i & 63;
    float peak = -INFINITY;
    for (int c = 0; c < count; c++) peak = fmaxf(peak, partials[c * kPartialFloats + kMaxTileHeads * 64 + h]);
    float total = 0.0f;
    float sum = 0.0f;
    for (int c = 0; c < count; c++) {
        const float w = exp_poly(partials[c * kPartialFloats + kMaxTileHeads * 64 + h] - peak);
        total += w * partials[c * kPartialFloats + kMaxTileHeads * 64 + 8 + h];
        sum = __builtin_fmaf(w, partials[c * kPartialFloats + h * 64 + d], sum);
    }
    output[h * 64 + d] = sum * (1.0f / total);
}

int32_t staging_alloc(size_t bytes, uint8_t** buf)
{
    thread_local uint8_t* t_buf = nullptr;
    thread_local size_t t_cap = 0;
    if (bytes > t_cap) {
        if (t_buf) NHIP_CHECK_HIP(hipFree(t_buf));
        t_buf = nullptr;
        t_cap = 0;
        const size_t cap = (bytes + (1u << 20) - 1) & ~size_t((1u << 20) - 1);
        NHIP_CHECK_HIP(hipMalloc(&t_buf, cap));
        t_cap = cap;
    }
    *buf = t_buf;
    return NHIP_OK;
}

inline size_t a256(size_t x) { return (x + 255) & ~size_t(255); }

int32_t attention_tile_impl(const nhip_attn_tile* t)
{
    NHIP_REQUIRE(t, "tile is NULL");
    NHIP_REQUIRE(t->heads >= 1 && t->heads <= kMaxTileHeads, "tile heads %d outside [1,%d]", t->heads, kMaxTileHeads);
    NHIP_REQUIRE(t->count >= 1 && t->count <= 32768 && t->first >= 0, "tile span first %d count %d", t->first,
                 t->count);
    NHIP_REQUIRE(t->queries && t->query_scales && t->keys && t->key_scales && t->values && t->value_scales &&
                     t->output,
                 "null tile pointer");
    NHIP_REQUIRE((t->peaks == nullptr) == (t->sums == nullptr), "peaks and sums must be set together");
    int32_t rc = ensure_device();
    if (rc) return rc;
    const int heads = t->heads, count = t->count, first = t->first;
    // Device copies of the spans the tile reads (positions first..first+count-1).
    const size_t kspan = (size_t)(count - 1) * t->key_stride + 48;
    const size_t vspan = (size_t)(count - 1) * t->value_stride + 64;
    const size_t sspan = ((size_t)(count - 1) * t->scale_stride + 1) * sizeof(float);
    const size_t qbytes = (size_t)heads * 48, qsbytes = heads * sizeof(float);
    const size_t obytes = (size_t)heads * 64 * sizeof(float);
    const size_t pbytes = t->probabilities ? (size_t)heads * count * sizeof(float) : 0;
    const size_t total = a256(kspan) + a256(vspan) + 2 * a256(sspan) + a256(qbytes) + a256(qsbytes) + a256(obytes) +
                         a256(pbytes) + 2 * 256;
    uint8_t* buf = nullptr;
    rc = staging_alloc(total, &buf);
    if (rc) return rc;
    uint8_t* p = buf;
    auto take = [&](size_t n) { uint8_t* r = p; p += a256(n); return r; };
    int8_t* d_k = reinterpret_cast<int8_t*>(take(kspan));
    int8_t* d_v = reinterpret_cast<int8_t*>(take(vspan));
    float* d_ks = reinterpret_cast<float*>(take(sspan));
    float* d_vs = reinterpret_cast<float*>(take(sspan));
    int8_t* d_q = reinterpret_cast<int8_t*>(take(qbytes));
    float* d_qs = reinterpret_cast<float*>(take(qsbytes));
    float* d_out = reinterpret_cast<float*>(take(obytes));
    float* d_prob = pbytes ? reinterpret_cast<float*>(take(pbytes)) : nullptr;
    float* d_peaks = t->peaks ? reinterpret_cast<float*>(take(256)) : nullptr;
    float* d_sums = t->peaks ? reinterpret_cast<float*>(take(256)) : nullptr;
    hipStream_t s = default_stream();
    NHIP_CHECK_HIP(hipMemcpyAsync(d_k, t->keys + (size_t)first * t->key_stride, kspan, hipMemcpyHostToDevice, s));
    NHIP_CHECK_HIP(hipMemcpyAsync(d_v, t->values + (size_t)first * t->value_stride, vspan, hipMemcpyHostToDevice, s));
    NHIP_CHECK_HIP(hipMemcpyAsync(d_ks, t->key_scales + (size_t)first * t->scale_stride, sspan, hipMemcpyHostToDevice, s));
    NHIP_CHECK_HIP(
        hipMemcpyAsync(d_vs, t->value_scales + (size_t)first * t->scale_stride, sspan, hipMemcpyHostToDevice, s));
    NHIP_CHECK_HIP(hipMemcpyAsync(d_q, t->queries, qbytes, hipMemcpyHostToDevice, s));
    NHIP_CHECK_HIP(hipMemcpyAsync(d_qs, t->query_scales, qsbytes, hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(tile_kernel, dim3(heads), dim3(kTileThreads), (size_t)count * sizeof(float), s, d_q, d_qs, d_k,
                       d_ks, d_v, d_vs, t->key_stride, t->value_stride, t->scale_stride, count, 48,
                       0.14433756729740643f, d_out, d_prob, count, d_peaks, d_sums);
    NHIP_CHECK_HIP(hipGetLastError());
    NHIP_CHECK_HIP(hipMemcpyAsync(t->output, d_out, obytes, hipMemcpyDeviceToHost, s));
    if (d_prob)
        NHIP_CHECK_HIP(hipMemcpy2DAsync(t->probabilities + first, (size_t)t->probability_stride * sizeof(float), d_prob,
                                        (size_t)count * sizeof(float), (size_t)count * sizeof(float), heads,
                                        hipMemcpyDeviceToHost, s));
    if (d_peaks) {
        NHIP_CHECK_HIP(hipMemcpyAsync(t->peaks, d_peaks, heads * sizeof(float), hipMemcpyDeviceToHost, s));
        NHIP_CHECK_HIP(hipMemcpyAsync(t->sums, d_sums, heads * sizeof(float), hipMemcpyDeviceToHost, s));
    }
    NHIP_CHECK_HIP(hipStreamSynchronize(s));
    return NHIP_OK;
}

int32_t merge_partials_impl(const float* partials, int32_t count, int32_t heads, float* output)
{
    NHIP_REQUIRE(partials && output, "null pointer");
    NHIP_REQUIRE(count >= 1 && count <= 8 && heads >= 1 && heads <= kMaxTileHeads, "count %d heads %d", count, heads);
    int32_t rc = ensure_device();
    if (rc) return rc;
    const size_t pbytes = (size_t)count * kPartialFloats * sizeof(float);
    const size_t obytes = (size_t)heads * 64 * sizeof(float);
    uint8_t* buf = nullptr;
    rc = staging_alloc(a256(pbytes) + obytes, &buf);
    if (rc) return rc;
    float* d_p = reinterpret_cast<float*>(buf);
    float* d_o = reinterpret_cast<float*>(buf + a256(pbytes));
    hipStream_t s = default_stream();
    NHIP_CHECK_HIP(hipMemcpyAsync(d_p, partials, pbytes, hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(merge_kernel, dim3((heads * 64 + 63) / 64), dim3(64), 0, s, d_p, count, heads, d_o);
    NHIP_CHECK_HIP(hipGetLastError());
    NHIP_CHECK_HIP(hipMemcpyAsync(output, d_o, obytes, hipMemcpyDeviceToHost, s));
    NHIP_CHECK_HIP(hipStreamSynchronize(s));
    return NHIP_OK;
}

}  // namespace
}  // namespace nhip

using namespace nhip;

extern "C" {

void nhip_attention_tile(const nhip_attn_tile* tile)
{
    clear_error();
    attention_tile_impl(tile);
}

void nhip_merge_partials(const float* partials, int32_t count, int32_t heads, float* output)
{
    clear_error();
    merge_partials_impl(partials, count, heads, output);
}

}  // extern "C"

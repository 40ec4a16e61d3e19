// attention_decode.hip -- ragged decode attention over a pooled int8 KV
// cache on gfx950 (one launch for every row of a ragged batch).
//
// Semantics: AttentionBatch.ExecuteChunk + Attention.MergePartials
// (src/Needle/Blocks.cs:927-966, 750-817) for every (row, head):
//   * the row's positions first .. first+count-1 are split into chunks by the
//     reference's plan (Blocks.cs:934-938; chunk cap a parameter, 8 in the
//     reference);
//   * every chunk is the scalar tile in partial form: score_s =
//     (float(q.k_s) * keyScale_s) * (queryScale * 1/sqrt(qk)), peak = max,
//     e_s = Exp(score_s - peak), sum = sum_s e_s and out_d = sum_s
//     (e_s * valueScale_s) * v_{s,d}, both sums in ascending s;
//   * the chunks are merged in MergePartials' non-SIMD order.
// Exp is the reference polynomial Ops.Exp (exp_poly, common.hpp).  With
// these orders fixed the results are bit-identical to the CPU restatement.
//
// Mapping: one workgroup of 256 threads per (chunk, row, head block); a head
// block is whole kv groups, at most 16 query heads.  Phase 1 gives one
// thread per (kv head, position): it loads the key row once (16-byte loads)
// and forms the int32 dots of every query head of the group with v_dot4.
// Phase 4 gives one thread per (head, 4 value dims), which walks the chunk's
// positions in order, reading one value dword per position (a wave covers 4
// heads x 64 dims = 256 contiguous bytes of a cache row).  The last
// workgroup of a (row, head block) to finish merges the partials; its
// arrival counter is reset to zero by the merger, so the workspace needs
// zeroing only once.
#include <algorithm>

#include "common.hpp"

namespace nhip {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxHeadsPerBlock = 16;

struct DecodeAttnParams {
    const int8_t* q;        // [rows][heads][qk]
    const float* qscale;    // [rows][heads]
    const int8_t* keys;     // [slots][capacity][kv_heads*qk]
    const float* kscale;    // [slots][capacity][kv_heads]
    const int8_t* values;   // [slots][capacity][kv_heads*64]
    const float* vscale;    // [slots][capacity][kv_heads]
    const int32_t* row_slot;
    const int32_t* row_first;
    const int32_t* row_count;
    int32_t* arrivals;      // [rows][head_blocks]
    float* peaks;           // [rows][max_chunks][heads]
    float* sums;            // [rows][max_chunks][heads]
    float* partials;        // [rows][max_chunks][heads][64]
    float* out;             // [rows][heads][64]
    int32_t rows, heads, kv_heads, qk, slots, capacity, max_chunks, lmax, kv_per_block;
    float inv_sqrt;
};

// The reference's chunk plan (Blocks.cs:934-938).
__device__ __forceinline__ int plan(int count, int max_chunks, int* length)
{
    int needed = min(max(count / 16, 1), max_chunks);
    const int len = ((count + needed - 1) / needed + 3) & ~3;
    *length = len;
    return (count + len - 1) / len;
}

__device__ __forceinline__ float sx8(uint32_t v, int b)
{
    return static_cast<float>(static_cast<int32_t>(v << (24 - 8 * b)) >> 24);
}

__global__ __launch_bounds__(kThreads) void decode_attention_kernel(DecodeAttnParams p)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int hb = blockIdx.z;
    const int row = blockIdx.y;
    const int chunk = blockIdx.x;
    const int tid = threadIdx.x;
    const int group = p.heads / p.kv_heads;
    const int kv0 = hb * p.kv_per_block;
    const int nkv = min(p.kv_per_block, p.kv_heads - kv0);
    const int h0 = kv0 * group;
    const int nh = nkv * group;  // <= 16
    const int lmax = p.lmax;

    int8_t* q_lds = reinterpret_cast<int8_t*>(lds);                        // [16][64]
    float* score = reinterpret_cast<float*>(lds + kMaxHeadsPerBlock * 64);  // [16][lmax]
    float* ew = score + kMaxHeadsPerBlock * lmax;                           // [16][lmax]
    float* ww = ew + kMaxHeadsPerBlock * lmax;                              // [16][lmax]
    float* peak_lds = ww + kMaxHeadsPerBlock * lmax;                        // [16]
    __shared__ int last_flag;

    const int slot = p.row_slot[row];
    const int first = p.row_first[row];
    int count = p.row_count[row];
    // rows with an invalid slot or span produce zeros (no out-of-range reads)
    const bool valid = slot >= 0 && slot < p.slots && first >= 0 && count >= 1 && count <= p.capacity - first;
    if (!valid) {
        if (chunk == 0 && tid < nh * 16) {
            const int h = h0 + tid / 16;
            float4* o = reinterpret_cast<float4*>(p.out + ((size_t)row * p.heads + h) * 64 + 4 * (tid % 16));
            *o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        return;
    }
    int length;
    const int needed = plan(count, p.max_chunks, &length);
    if (chunk >= needed) return;
    const int begin = first + chunk * length;
    const int L = min(length, count - chunk * length);
    const size_t pos0 = (size_t)slot * p.capacity + begin;
    const int qk = p.qk;
    const int q4 = qk / 4;

    // stage the query heads of this block (nh * qk bytes, dword-granular)
    {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(p.q + ((size_t)row * p.heads + h0) * qk);
        uint32_t* dst = reinterpret_cast<uint32_t*>(q_lds);
        for (int i = tid; i < nh * q4; i += kThreads) dst[(i / q4) * 16 + (i % q4)] = src[i];
    }
    __syncthreads();

    // phase 1: scores, one thread per (kv head, position)
    for (int it = tid; it < nkv * L; it += kThreads) {
        const int kvl = it / L;
        const int s = it - kvl * L;
        const int kv = kv0 + kvl;
        const uint4* krow = reinterpret_cast<const uint4*>(p.keys + ((pos0 + s) * p.kv_heads + kv) * qk);
        uint4 kr[4];
        kr[0] = krow[0];
        kr[1] = krow[1];
        kr[2] = krow[2];
        kr[3] = qk == 64 ? krow[3] : make_uint4(0, 0, 0, 0);
        const float ks = p.kscale[(pos0 + s) * p.kv_heads + kv];
        for (int g = 0; g < group; g++) {
            const int hl = kvl * group + g;
            const uint4* qv = reinterpret_cast<const uint4*>(q_lds + hl * 64);
            int dot = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint4 a = j < 3 || qk == 64 ? qv[j] : make_uint4(0, 0, 0, 0);
                dot = __builtin_amdgcn_sdot4((int)a.x, (int)kr[j].x, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.y, (int)kr[j].y, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.z, (int)kr[j].z, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.w, (int)kr[j].w, dot, false);
            }
            const float scale = p.qscale[(size_t)row * p.heads + h0 + hl] * p.inv_sqrt;
            score[hl * lmax + s] = (static_cast<float>(dot) * ks) * scale;
        }
    }
    __syncthreads();

    // phase 2: per-head peak (max is order-independent; +0 preferred over -0)
    {
        const int wave = tid >> 6, lane = tid & 63;
        for (int hl = wave; hl < nh; hl += kThreads / 64) {
            float m = -INFINITY;
            for (int s = lane; s < L; s += 64) m = ref_max(m, score[hl * lmax + s]);
            for (int off = 32; off > 0; off >>= 1) m = ref_max(m, __shfl_xor(m, off));
            if (lane == 0) peak_lds[hl] = m;
        }
    }
    __syncthreads();

    // phase 3: e_s and e_s * valueScale_s
    for (int it = tid; it < nh * L; it += kThreads) {
        const int hl = it / L;
        const int s = it - hl * L;
        const int kv = kv0 + hl / group;
        const float e = exp_poly(score[hl * lmax + s] - peak_lds[hl]);
        ew[hl * lmax + s] = e;
        ww[hl * lmax + s] = e * p.vscale[(pos0 + s) * p.kv_heads + kv];
    }
    __syncthreads();

    // phase 4: one thread per (head, 4 dims), positions in ascending order
    const size_t pbase = ((size_t)row * p.max_chunks + chunk) * p.heads;
    if (tid < nh * 16) {
        const int hl = tid >> 4;
        const int qd = tid & 15;
        const int kv = kv0 + hl / group;
        const size_t vstride = (size_t)p.kv_heads * 64;
        const uint32_t* vp = reinterpret_cast<const uint32_t*>(p.values + (pos0 * p.kv_heads + kv) * 64 + 4 * qd);
        float o0 = 0.0f, o1 = 0.0f, o2 = 0.0f, o3 = 0.0f, total = 0.0f;
        int s = 0;
        for (; s + 8 <= L; s += 8) {
            uint32_t v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = vp[(size_t)(s + j) * (vstride / 4)];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float w = ww[hl * lmax + s + j];
                total = total + ew[hl * lmax + s + j];
                o0 = o0 + w * sx8(v[j], 0);
                o1 = o1 + w * sx8(v[j], 1);
                o2 = o2 + w * sx8(v[j], 2);
                o3 = o3 + w * sx8(v[j], 3);
            }
        }
        for (; s < L; s++) {
            const uint32_t v = vp[(size_t)s * (vstride / 4)];
            const float w = ww[hl * lmax + s];
            total = total + ew[hl * lmax + s];
            o0 = o0 + w * sx8(v, 0);
            o1 = o1 + w * sx8(v, 1);
            o2 = o2 + w * sx8(v, 2);
            o3 = o3 + w * sx8(v, 3);
        }
        const int h = h0 + hl;
        *reinterpret_cast<float4*>(p.partials + (pbase + h) * 64 + 4 * qd) = make_float4(o0, o1, o2, o3);
        if (qd == 0) {
            p.peaks[pbase + h] = peak_lds[hl];
            p.sums[pbase + h] = total;
        }
    }

    // arrival: the last workgroup of this (row, head block) merges
    __threadfence();
    __syncthreads();
    int32_t* counter = p.arrivals + (size_t)row * gridDim.z + hb;
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last_flag = old == needed - 1;
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    if (tid < nh * 16) {
        const int hl = tid >> 4;
        const int qd = tid & 15;
        const int h = h0 + hl;
        const size_t rb = (size_t)row * p.max_chunks * p.heads + h;  // + c * heads
        const size_t hs = p.heads;
        float r0, r1, r2, r3;
        if (needed == 2) {
            const float peak0 = p.peaks[rb], peak1 = p.peaks[rb + hs];
            const float pk = ref_max(peak0, peak1);
            const float w0 = exp_poly(peak0 - pk);
            const float w1 = exp_poly(peak1 - pk);
            float tot = 0.0f;
            tot = tot + w0 * p.sums[rb];
            tot = tot + w1 * p.sums[rb + hs];
            const float inv = 1.0f / tot;
            const float4 a = *reinterpret_cast<const float4*>(p.partials + rb * 64 + 4 * qd);
            const float4 b = *reinterpret_cast<const float4*>(p.partials + (rb + hs) * 64 + 4 * qd);
            r0 = (w0 * a.x + w1 * b.x) * inv;
            r1 = (w0 * a.y + w1 * b.y) * inv;
            r2 = (w0 * a.z + w1 * b.z) * inv;
            r3 = (w0 * a.w + w1 * b.w) * inv;
        } else {
            float peak = -INFINITY;
            for (int c = 0; c < needed; c++) peak = ref_max(peak, p.peaks[rb + c * hs]);
            float total = 0.0f;
            for (int c = 0; c < needed; c++) total = total + exp_poly(p.peaks[rb + c * hs] - peak) * p.sums[rb + c * hs];
            const float inverse = 1.0f / total;
            float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
            for (int c = 0; c < needed; c++) {
                const float w = exp_poly(p.peaks[rb + c * hs] - peak);
                const float4 a = *reinterpret_cast<const float4*>(p.partials + (rb + c * hs) * 64 + 4 * qd);
                s0 = s0 + w * a.x;
                s1 = s1 + w * a.y;
                s2 = s2 + w * a.z;
                s3 = s3 + w * a.w;
            }
            r0 = s0 * inverse;
            r1 = s1 * inverse;
            r2 = s2 * inverse;
            r3 = s3 * inverse;
        }
        *reinterpret_cast<float4*>(p.out + ((size_t)row * p.heads + h) * 64 + 4 * qd) = make_float4(r0, r1, r2, r3);
    }
    if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void zero_kernel(uint32_t* p, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

inline size_t a256(size_t x) { return (x + 255) & ~size_t(255); }

struct WorkspaceLayout {
    size_t arrivals, peaks, sums, partials, total;
};

WorkspaceLayout layout(int rows, int heads, int max_chunks)
{
    const int head_blocks = heads;  // upper bound on head blocks per row
    WorkspaceLayout w{};
    const size_t pc = (size_t)rows * max_chunks * heads;
    w.arrivals = 0;
    w.peaks = a256((size_t)rows * head_blocks * sizeof(int32_t));
    w.sums = w.peaks + a256(pc * sizeof(float));
    w.partials = w.sums + a256(pc * sizeof(float));
    w.total = w.partials + a256(pc * 64 * sizeof(float));
    return w;
}

}  // namespace
}  // namespace nhip

using namespace nhip;

extern "C" {

size_t nhip_attention_decode_workspace(int32_t rows, int32_t heads, int32_t max_chunks)
{
    if (rows <= 0 || heads <= 0 || max_chunks <= 0) return 0;
    return layout(rows, heads, max_chunks).total;
}

int32_t nhip_attention_decode_workspace_init(void* d_workspace, size_t bytes, void* stream)
{
    NHIP_REQUIRE(d_workspace && bytes % 4 == 0, "attention workspace: null or size not a multiple of 4");
    int32_t rc = ensure_device();
    if (rc) return rc;
    const size_t n = bytes / 4;
    const int grid = (int)std::min<size_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(zero_kernel, dim3(std::max(grid, 1)), dim3(256), 0, as_stream(stream),
                       static_cast<uint32_t*>(d_workspace), n);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

int32_t nhip_attention_decode_dev(const int8_t* d_q, const float* d_qscale, int32_t rows, int32_t heads,
                                  int32_t kv_heads, int32_t qk_dim, const int8_t* d_keys,
                                  const float* d_key_scales, const int8_t* d_values,
                                  const float* d_value_scales, int32_t slots, int32_t capacity,
                                  const int32_t* d_row_slot, const int32_t* d_row_first,
                                  const int32_t* d_row_count, int32_t max_chunks, void* d_workspace,
                                  size_t workspace_bytes, float* d_out, void* stream)
{
    clear_error();
    if (rows == 0) return NHIP_OK;
    NHIP_REQUIRE(rows > 0 && heads > 0 && kv_heads > 0 && heads % kv_heads == 0,
                 "attention: heads (%d) must be a positive multiple of kv_heads (%d)", heads, kv_heads);
    const int group = heads / kv_heads;
    NHIP_REQUIRE(group <= kMaxHeadsPerBlock, "attention: at most %d query heads per kv head (got %d)",
                 kMaxHeadsPerBlock, group);
    NHIP_REQUIRE(qk_dim == 48 || qk_dim == 64, "attention: qk_dim must be 48 or 64 (got %d)", qk_dim);
    NHIP_REQUIRE(slots > 0 && capacity > 0, "attention: slots and capacity must be positive");
    NHIP_REQUIRE(max_chunks >= 1 && max_chunks <= 256, "attention: max_chunks must be in [1, 256]");
    NHIP_REQUIRE(d_q && d_qscale && d_keys && d_key_scales && d_values && d_value_scales && d_row_slot &&
                     d_row_first && d_row_count && d_workspace && d_out,
                 "attention: null pointer");
    NHIP_REQUIRE(((reinterpret_cast<uintptr_t>(d_q) | reinterpret_cast<uintptr_t>(d_keys) |
                   reinterpret_cast<uintptr_t>(d_values) | reinterpret_cast<uintptr_t>(d_out)) & 15) == 0,
                 "attention: q, keys, values and out must be 16-byte aligned");
    const WorkspaceLayout wl = layout(rows, heads, max_chunks);
    NHIP_REQUIRE(workspace_bytes >= wl.total, "attention: workspace of %zu bytes, need %zu", workspace_bytes,
                 wl.total);
    // longest chunk: <= 32 below 16*max_chunks positions, else ceil(capacity/max_chunks) rounded up to 4
    const int lmax = std::max(32, ((capacity + max_chunks - 1) / max_chunks + 3) & ~3);
    const size_t lds = kMaxHeadsPerBlock * 64 + (size_t)3 * kMaxHeadsPerBlock * lmax * sizeof(float) +
                       kMaxHeadsPerBlock * sizeof(float);
    NHIP_REQUIRE(lds <= 64 * 1024, "attention: chunks of up to %d positions need %zu bytes of LDS; raise "
                 "max_chunks", lmax, lds);
    int32_t rc = ensure_device();
    if (rc) return rc;
    DecodeAttnParams p{};
    p.q = d_q;
    p.qscale = d_qscale;
    p.keys = d_keys;
    p.kscale = d_key_scales;
    p.values = d_values;
    p.vscale = d_value_scales;
    p.row_slot = d_row_slot;
    p.row_first = d_row_first;
    p.row_count = d_row_count;
    uint8_t* ws = static_cast<uint8_t*>(d_workspace);
    p.arrivals = reinterpret_cast<int32_t*>(ws + wl.arrivals);
    p.peaks = reinterpret_cast<float*>(ws + wl.peaks);
    p.sums = reinterpret_cast<float*>(ws + wl.sums);
    p.partials = reinterpret_cast<float*>(ws + wl.partials);
    p.out = d_out;
    p.rows = rows;
    p.heads = heads;
    p.kv_heads = kv_heads;
    p.qk = qk_dim;
    p.slots = slots;
    p.capacity = capacity;
    p.max_chunks = max_chunks;
    p.lmax = lmax;
    p.kv_per_block = std::max(1, kMaxHeadsPerBlock / group);
    p.inv_sqrt = static_cast<float>(1.0 / std::sqrt(static_cast<double>(qk_dim)));
    const int head_blocks = (kv_heads + p.kv_per_block - 1) / p.kv_per_block;
    hipLaunchKernelGGL(decode_attention_kernel, dim3(max_chunks, rows, head_blocks), dim3(kThreads), lds,
                       as_stream(stream), p);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

}  // extern "C"

// needle3.hip -- Needle 3's attention inputs on gfx950: the three-tap
// convolution over time, zero-centred RMS norm, rotary positions and
// QuantizeInt8 that turn a row's raw Q/K/V projections into the int8 query
// heads and the KV-cache row (EngineCore.TapsAndAttentionHeadsSingle,
// src/Needle/Engine.cs:1302-1387; Scalar.Taps3, src/Needle/Scalar.cs:285-288).
//
// One wave per (row, head), one lane per element of the head (qk <= 64,
// vd <= 64): the lane forms its convolution term, the wave's sum of squares
// runs in the AVX2 tier's Vector256 order (wave_v256_sum), the rotation pairs lanes
// i and i + qk/2, and the int8 row is quantized with the head's absolute
// maximum.  Rows of one slot with consecutive positions form a run: a row
// takes its previous frames from the rows before it in the run and, for the
// run's first rows, from the slot's history; a second launch then moves each
// slot's history to the run's last two frames.  Precondition (as in
// EngineCore.ForwardBatch's rows): the rows of a slot are one contiguous run
// of consecutive positions.  Apart from the sum of squares the arithmetic is
// the reference's scalar order (no contraction), so the outputs are
// bit-identical with the oracle's row-by-row step in the AVX2 row tier.
#include "common.hpp"

namespace nhip {
namespace {

struct Needle3Params {
    const float* raw;  // [rows][qw + kw + vw]
    const float* taps[3];
    const float* q_norm;
    const float* k_norm;
    const float* rope_cos;
    const float* rope_sin;
    float* history;  // [slots][2][qw], [2][kw], [2][vw]
    const int32_t* row_slot;
    const int32_t* row_pos;
    int8_t* q;
    float* q_scales;
    int8_t* keys;
    float* key_scales;
    int8_t* values;
    float* value_scales;
    int32_t rows, heads, kv_heads, qk, vd, slots, capacity;
};

// Row r's run flags from the (slot, position) of rows r - 2 .. r + 1, all
// loaded up front (clamped indexes) so they take one round trip: what
// row_valid and continues compute, without their chain of dependent loads.
struct RunFlags {
    bool valid, run1, run2, next_continues;
    int slot, pos;
};
// A uniform load through the scalar cache (the kernels store to global
// memory, so the compiler would otherwise use vector loads for these
// arrays, which no kernel of the launch writes).
__device__ __forceinline__ int32_t uniform_load(const int32_t* a, int i)
{
    return ((const __attribute__((address_space(4))) int32_t*)a)[i];
}

__device__ __forceinline__ RunFlags run_flags(const Needle3Params& p, int r)
{
    const int ra = max(r - 2, 0), rb = max(r - 1, 0), rc = min(r + 1, p.rows - 1);
    const int s2 = uniform_load(p.row_slot, ra), q2 = uniform_load(p.row_pos, ra);
    const int s1 = uniform_load(p.row_slot, rb), q1 = uniform_load(p.row_pos, rb);
    const int s0 = uniform_load(p.row_slot, r), q0 = uniform_load(p.row_pos, r);
    const int sn = uniform_load(p.row_slot, rc), qn = uniform_load(p.row_pos, rc);
    auto ok = [&](int s, int q) { return (s >= 0) & (s < p.slots) & (q >= 0) & (q < p.capacity); };
    RunFlags f;
    f.valid = ok(s0, q0);
    f.run1 = f.valid & (r >= 1) & ok(s1, q1) & (s1 == s0) & (q1 == q0 - 1);
    f.run2 = f.run1 & (r >= 2) & ok(s2, q2) & (s2 == s0) & (q2 == q0 - 2);
    f.next_continues = (r + 1 < p.rows) & ok(sn, qn) & f.valid & (sn == s0) & (qn == q0 + 1);
    f.slot = s0;
    f.pos = q0;
    return f;
}

__global__ __launch_bounds__(64) void needle3_inputs_kernel(Needle3Params p)
{
    __shared__ float val[64];
    __shared__ float red[64];
    const int r = blockIdx.x;
    const int unit = blockIdx.y;  // query heads, then key heads, then value heads
    const int c = threadIdx.x;
    const int qw = p.heads * p.qk, kw = p.kv_heads * p.qk, vw = p.kv_heads * p.vd;
    const int all = qw + kw + vw;
    const int part = unit < p.heads ? 0 : (unit < p.heads + p.kv_heads ? 1 : 2);
    const int head = part == 0 ? unit : (part == 1 ? unit - p.heads : unit - p.heads - p.kv_heads);
    const int n = part == 2 ? p.vd : p.qk;
    const int W = part == 0 ? qw : (part == 1 ? kw : vw);
    const int base = part == 0 ? 0 : (part == 1 ? qw : qw + kw);
    const int off = head * n;
    const RunFlags rf = run_flags(p, r);
    if (!rf.valid) {  // q = 0 with scale 1; nothing else is touched
        if (part == 0) {
            if (c < n) p.q[(size_t)r * qw + off + c] = 0;
            if (c == 0) p.q_scales[(size_t)r * p.heads + head] = 1.0f;
        }
        return;
    }
    const int slot = rf.slot, pos = rf.pos;
    const bool run1 = rf.run1;
    const bool run2 = rf.run2;
    const float* hist = p.history + (size_t)slot * 2 * all + 2 * base;  // frame 0, then frame 1 (latest)
    const float* taps = p.taps[part] + off;
    float x = 0.0f;
    if (c < n) {
        const int e = base + off + c;
        const float x2 = p.raw[(size_t)r * all + e];
        const float x1 = run1 ? p.raw[(size_t)(r - 1) * all + e] : hist[W + off + c];
        const float x0 = run2 ? p.raw[(size_t)(r - 2) * all + e] : (run1 ? hist[W + off + c] : hist[off + c]);
        x = taps[c] * x2 + taps[W + c] * x1 + taps[2 * W + c] * x0;
    }
    if (part < 2) {
        // ZeroCenteredRms, its sum of squares in the AVX2 tier's order
        red[c] = x;
        __syncthreads();
        const float sum = wave_v256_sum(red, red, n);
        const float inverse = 1.0f / sqrtf(sum / (float)n + 1e-6f);
        const float* scale = part == 0 ? p.q_norm : p.k_norm;
        x = c < n ? (1.0f + scale[c]) * x * inverse : 0.0f;
        // Rope: lanes i and i + n/2
        val[c] = x;
        __syncthreads();
        const int half = n / 2;
        if (c < n) {
            const int i = c < half ? c : c - half;
            const float cs = p.rope_cos[(size_t)pos * half + i];
            const float sn = p.rope_sin[(size_t)pos * half + i];
            const float a = val[i], b = val[half + i];
            x = c < half ? a * cs - b * sn : b * cs + a * sn;
        }
    }
    // QuantizeInt8 over the head (the maximum is order-free)
    const float m = wave_max(c < n ? fabsf(x) : 0.0f);
    const float scale = m > 0.0f ? m / 127.0f : 1.0f;
    const float inverse = 1.0f / scale;
    const int8_t qv = (int8_t)ref_quantize_one(x, inverse);
    const size_t cell = (size_t)slot * p.capacity + pos;
    if (part == 0) {
        if (c < n) p.q[(size_t)r * qw + off + c] = qv;
        if (c == 0) p.q_scales[(size_t)r * p.heads + head] = scale;
    } else if (part == 1) {
        if (c < n) p.keys[cell * kw + off + c] = qv;
        if (c == 0) p.key_scales[cell * p.kv_heads + head] = scale;
    } else {
        if (c < n) p.values[cell * vw + off + c] = qv;
        if (c == 0) p.value_scales[cell * p.kv_heads + head] = scale;
    }
}

// The last row of each run moves its slot's history to the run's last two
// frames: frame 0 <- the row before (or the old frame 1), frame 1 <- the row.
__global__ __launch_bounds__(256) void needle3_history_kernel(Needle3Params p)
{
    const int r = blockIdx.x;
    const RunFlags rf = run_flags(p, r);
    if (!rf.valid) return;
    if (rf.next_continues) return;  // not the run's last row
    const int qw = p.heads * p.qk, kw = p.kv_heads * p.qk, vw = p.kv_heads * p.vd;
    const int all = qw + kw + vw;
    const bool run1 = rf.run1;
    float* hist = p.history + (size_t)rf.slot * 2 * all;
    for (int e = threadIdx.x; e < all; e += blockDim.x) {
        const int part = e < qw ? 0 : (e < qw + kw ? 1 : 2);
        const int base = part == 0 ? 0 : (part == 1 ? qw : qw + kw);
        const int W = part == 0 ? qw : (part == 1 ? kw : vw);
        float* f0 = hist + 2 * base + (e - base);
        float* f1 = f0 + W;
        const float old1 = *f1;
        *f0 = run1 ? p.raw[(size_t)(r - 1) * all + e] : old1;
        *f1 = p.raw[(size_t)r * all + e];
    }
}

}  // namespace

// The attention inputs; with_history false leaves the slots' frames to the
// caller, which must move them on (as needle3_history_kernel does) after
// every row of the step has read them.
int32_t needle3_attention_inputs_impl(const float* d_raw, int32_t rows, int32_t heads, int32_t kv_heads,
                                      int32_t qk_dim, int32_t v_dim, const float* d_q_taps, const float* d_k_taps,
                                      const float* d_v_taps, const float* d_q_norm, const float* d_k_norm,
                                      const float* d_rope_cos, const float* d_rope_sin, float* d_history,
                                      const int32_t* d_row_slot, const int32_t* d_row_pos, int32_t slots,
                                      int32_t capacity, int8_t* d_q, float* d_q_scales, int8_t* d_keys,
                                      float* d_key_scales, int8_t* d_values, float* d_value_scales, bool with_history,
                                      hipStream_t s)
{
    NHIP_REQUIRE(rows >= 0, "rows %d < 0", rows);
    if (rows == 0) return NHIP_OK;
    NHIP_REQUIRE(heads > 0 && kv_heads > 0 && slots > 0 && capacity > 0, "heads, kv_heads, slots and capacity must be "
                 "positive");
    NHIP_REQUIRE(qk_dim >= 2 && qk_dim <= 64 && qk_dim % 2 == 0 && v_dim >= 1 && v_dim <= 64,
                 "qk_dim (%d) must be even and <= 64, v_dim (%d) <= 64", qk_dim, v_dim);
    NHIP_REQUIRE(d_raw && d_q_taps && d_k_taps && d_v_taps && d_q_norm && d_k_norm && d_rope_cos && d_rope_sin &&
                     d_history && d_row_slot && d_row_pos && d_q && d_q_scales && d_keys && d_key_scales &&
                     d_values && d_value_scales,
                 "null pointer");
    int32_t rc = ensure_device();
    if (rc) return rc;
    Needle3Params p{};
    p.raw = d_raw;
    p.taps[0] = d_q_taps;
    p.taps[1] = d_k_taps;
    p.taps[2] = d_v_taps;
    p.q_norm = d_q_norm;
    p.k_norm = d_k_norm;
    p.rope_cos = d_rope_cos;
    p.rope_sin = d_rope_sin;
    p.history = d_history;
    p.row_slot = d_row_slot;
    p.row_pos = d_row_pos;
    p.q = d_q;
    p.q_scales = d_q_scales;
    p.keys = d_keys;
    p.key_scales = d_key_scales;
    p.values = d_values;
    p.value_scales = d_value_scales;
    p.rows = rows;
    p.heads = heads;
    p.kv_heads = kv_heads;
    p.qk = qk_dim;
    p.vd = v_dim;
    p.slots = slots;
    p.capacity = capacity;
    hipLaunchKernelGGL(needle3_inputs_kernel, dim3(rows, heads + 2 * kv_heads), dim3(64), 0, s, p);
    NHIP_CHECK_HIP(hipGetLastError());
    if (with_history) {
        hipLaunchKernelGGL(needle3_history_kernel, dim3(rows), dim3(256), 0, s, p);
        NHIP_CHECK_HIP(hipGetLastError());
    }
    return NHIP_OK;
}

}  // namespace nhip

extern "C" int32_t nhip_needle3_attention_inputs_dev(
    const float* d_raw, int32_t rows, int32_t heads, int32_t kv_heads, int32_t qk_dim, int32_t v_dim,
    const float* d_q_taps, const float* d_k_taps, const float* d_v_taps, const float* d_q_norm,
    const float* d_k_norm, const float* d_rope_cos, const float* d_rope_sin, float* d_history,
    const int32_t* d_row_slot, const int32_t* d_row_pos, int32_t slots, int32_t capacity, int8_t* d_q,
    float* d_q_scales, int8_t* d_keys, float* d_key_scales, int8_t* d_values, float* d_value_scales, void* stream)
{
    nhip::clear_error();
    return nhip::needle3_attention_inputs_impl(d_raw, rows, heads, kv_heads, qk_dim, v_dim, d_q_taps, d_k_taps,
                                               d_v_taps, d_q_norm, d_k_norm, d_rope_cos, d_rope_sin, d_history,
                                               d_row_slot, d_row_pos, slots, capacity, d_q, d_q_scales, d_keys,
                                               d_key_scales, d_values, d_value_scales, true, nhip::as_stream(stream));
}

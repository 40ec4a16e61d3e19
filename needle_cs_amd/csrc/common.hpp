// common.hpp -- shared runtime helpers and exact device arithmetic for
// libneedle_hip.so (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/needle_hip.h"

namespace nhip {

// ---------------------------------------------------------------- errors --

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define NHIP_CHECK_HIP(expr)                                                        \
    do {                                                                            \
        hipError_t nhip_e_ = (expr);                                                \
        if (nhip_e_ != hipSuccess) {                                                \
            ::nhip::set_error("%s failed: %s (%s:%d)", #expr,                       \
                              hipGetErrorString(nhip_e_), __FILE__, __LINE__);      \
            return NHIP_ERR_HIP;                                                    \
        }                                                                           \
    } while (0)

#define NHIP_REQUIRE(cond, ...)                                                     \
    do {                                                                            \
        if (!(cond)) {                                                              \
            ::nhip::set_error(__VA_ARGS__);                                         \
            return NHIP_ERR_ARG;                                                    \
        }                                                                           \
    } while (0)

// Initialises the device on first use (device 0 unless nhip_init chose one).
int32_t ensure_device();
// True once a device has been initialised (by nhip_init or a first use).
bool device_ready();
// Compute units of the initialised device.
int device_cus();
// Looks up, once per device and with that device current, the address of
// the no-allocation attention entry's scratch array (attention_decode.hip);
// called by the device initialisation.
int32_t attention_scratch_setup();
hipStream_t default_stream();
inline hipStream_t as_stream(void* s) { return s ? static_cast<hipStream_t>(s) : default_stream(); }

// ------------------------------------------------ preloaded arguments --

// gfx950 loads a kernel's leading scalar arguments into SGPRs before its
// first instruction (kernarg preload, built with
// -amdgpu-kernarg-preload-count; 14 SGPRs at most), while a struct argument
// is read from the argument segment with a scalar memory round trip.  A
// kernel whose first loads need fields of its parameter struct takes those
// fields again as leading pointer and 64-bit arguments (a "head", at most
// seven 8-byte words) and overwrites the struct's copies with them: its
// first loads then issue without waiting for the argument segment (about
// 0.25 us per launch).  Pointers travel as pointers, so that the compiler
// still knows them to be global memory; 32-bit fields travel in pairs.
inline uint64_t head_pair(int32_t lo, int32_t hi) { return (uint64_t)(uint32_t)lo | ((uint64_t)(uint32_t)hi << 32); }
__device__ __forceinline__ int32_t head_lo(uint64_t v) { return (int32_t)(uint32_t)v; }
__device__ __forceinline__ int32_t head_hi(uint64_t v) { return (int32_t)(uint32_t)(v >> 32); }

// ------------------------------------------------------- device weights --

enum class WeightFormat : int32_t { Int8G32 = 8, Cq2 = 2, Cq4 = 4 };

// HBM-resident weight matrix.  `tiles` holds the weights re-tiled for the
// matmul kernels: 16-row tiles, each a sequence of 1 KB blocks in which lane
// l of a wave finds its 16 bytes at l*16 (see gemv.hip for the block map);
// `norms` holds fp16 scales [rows_pad][groups_pad8].
struct DeviceWeights {
    WeightFormat format;
    int32_t rows, cols, groups;
    int32_t tiles_n;      // ceil(rows / 16)
    int32_t blocks;       // 1 KB blocks per tile
    int32_t groups_pad8;  // scale row stride (halves)
    uint32_t table[4];    // codebook bytes 0..15 (Cq formats)
    uint32_t split_table[4];  // the same bytes as the decode kernel's split lookup tables
    float byte_scale;     // codebook ByteScale (1 for the literal format)
    uint8_t* tiles;
    uint16_t* norms;
    // literal int8 matrices of at most kNarrowMaxRows rows: the weights again
    // in their row-major [rows][cols] order, for the narrow decode kernel
    // (narrow.hip), which gives a workgroup 4 or 8 whole rows
    uint8_t* rowmajor;
    size_t device_bytes;
    int32_t special_scales;  // some scale has binary16 exponent 31 (inf/NaN patterns)
};

constexpr int kNarrowMaxRows = 4096;

}  // namespace nhip

struct nhip_weights : nhip::DeviceWeights {};

namespace nhip {
// Prefill matmul of the literal int8 format (gemm.hip): exact = Scalar
// order (bit-identical with the decode kernels), else the fused epilogue.
int32_t launch_gemm_i8(const DeviceWeights* w, const int8_t* q, const float* qscale, int32_t tokens, float* y,
                       int32_t ldy, int32_t row_start, int32_t row_end, bool exact, hipStream_t stream);
// Ragged decode attention (attention_decode.hip); with d_q_out the output
// rows are also quantized (QuantizeInt8 per row), which needs max_chunks 1
// and every head in one block.
int32_t attention_decode_impl(const int8_t* d_q, const float* d_qscale, int32_t rows, int32_t heads,
                              int32_t kv_heads, int32_t qk_dim, const int8_t* d_keys, const float* d_key_scales,
                              const int8_t* d_values, const float* d_value_scales, int32_t slots,
                              int32_t capacity, const int32_t* d_row_slot, const int32_t* d_row_first,
                              const int32_t* d_row_count, int32_t max_chunks, void* d_workspace,
                              size_t workspace_bytes, float* d_out, int8_t* d_q_out, float* d_qs_out,
                              hipStream_t stream);
// Decode matmul (1..4 tokens, literal int8 format, all rows) whose int8
// activation rows are computed in the kernel's prologue from fp32 inputs
// (gemv.hip): kProNorm = x (+ delta) -> RMSNorm * gain -> QuantizeInt8,
// workgroup 0 writing x + delta to x_out when both are given; kProQuant =
// QuantizeInt8(x).  Returns 1 (nothing launched) when the shape does not
// fit the kernel; the caller then runs the element-wise kernel and the
// plain matmul.
enum : int32_t { kProNorm = 1, kProQuant = 2 };
struct DecodePrologue {
    int32_t kind;
    const float* x;
    const float* delta;
    float* x_out;
    const float* gain;
    float eps;
    // nonzero: the weight rows are (8 gate rows, the 8 matching up rows) per
    // 16-row tile and the kernel stores a = (g / (1 + Exp(-g))) * u at
    // y[t][8*tile + r] (rows/2 outputs per token) instead of the rows
    int32_t swiglu;
    // set: the kernel stores residual[t][n] + the row's sum at y[t][n]
    // (residual laid out like y): the residual stream's update in the
    // producing matmul
    const float* residual;
};
int32_t launch_decode_fused(const DeviceWeights* w, const DecodePrologue& f, int32_t tokens, float* y, int32_t ldy,
                            hipStream_t stream);
// The narrow decode matmul (narrow.hip) over rows [row_start, row_end):
// kind 0 takes int8 rows `in` [tokens][cols] with scales qscale, kProNorm /
// kProQuant compute them from fp32 rows as launch_decode_fused does (gain,
// eps as in DecodePrologue); with `residual` it stores residual + y.
// Returns 1 (nothing launched) for weights or shapes it does not take: no
// row-major copy, exponent-31 scales, more than 4 tokens, K other than
// 1024, 2048 or 4096, a pending delta.
int32_t launch_i8_narrow(const DeviceWeights* w, int32_t kind, const void* in, const float* delta,
                         const float* gain, const float* qscale, float eps, const float* residual, int32_t tokens,
                         float* y, int32_t ldy, int32_t row_start, int32_t row_end, hipStream_t stream);
// The decode matmul of int8 rows q restricted to the 16-row tiles holding a
// row set in some token's mask ([tokens][mask_words] bitsets, bit id%32 of
// word id/32); the other outputs are left untouched (Engine.LogitsForRows'
// sparse head, src/Needle/Engine.cs:2683-2700).
int32_t launch_decode_masked(const DeviceWeights* w, const int8_t* q, const float* qscale, int32_t tokens, float* y,
                             int32_t ldy, const uint32_t* mask, int32_t mask_words, hipStream_t stream);
// The decode matmul of int8 rows q (scales qscale) over tile-interleaved
// gate/up weights, storing the SwiGLU activations at act[t][0 .. rows/2);
// returns 1 when the decode kernel does not take the shape.
int32_t launch_decode_swiglu(const DeviceWeights* w, const int8_t* q, const float* qscale, int32_t tokens,
                             float* act, int32_t ldy, hipStream_t stream);
// Fused prologues pay for their input rows in every workgroup; beyond this
// many 16-row tiles a separate element-wise launch and the plain matmul are
// faster (at 512 tiles of K = 1024 and 3 rows the fused launch still wins
// by about 0.4 us; an LM head of 2,000 tiles gains nothing either way).
constexpr int kFusedPrologueMaxTiles = 512;
// The decoder's step attention with its input post-processing folded in:
// RoPE on the query and key heads of the fp32 QKV rows, per-head
// QuantizeInt8, and each row's key and value write to the cache at its
// position (qk 64).  Rows of the batch that write positions of another row's
// span are read from the launch's own results.  Returns 1 without launching
// when it does not apply: more than 4 rows or caches over 512 positions.
struct AttnPostInputs {
    const float* qkv;          // [rows][(heads + 2 kv_heads) * 64]
    const int32_t* positions;  // [rows]
    const float* rope_rows;    // [rows][64]: cos then sin (32 each) of each row's position
};
int32_t attention_decode_post_impl(const AttnPostInputs& in, int32_t rows, int32_t heads, int32_t kv_heads,
                                   int8_t* d_keys, float* d_key_scales, int8_t* d_values, float* d_value_scales,
                                   int32_t slots, int32_t capacity, const int32_t* d_row_slot,
                                   const int32_t* d_row_first, const int32_t* d_row_count, int32_t max_chunks,
                                   float* d_out, hipStream_t stream);
// Needle 3's attention inputs and decode attention in one launch (the
// whole-row kernel's Needle 3 form), for steps whose rows are one per slot
// and caches of at most 512 positions: each (row, query head) workgroup forms
// its query head, and the row's key and value heads, from the raw Q/K/V
// projections as needle3_attention_inputs_impl does (three-tap convolution
// over the slot's two previous frames, ZeroCenteredRms and RoPE of the query
// and key heads, QuantizeInt8), attends over its span with its own key and
// value in place of the cache at the row's position, and the group's first
// query head writes that key and value to the cache.  The slots' frames are
// left for the caller to move on.  Returns 1 without launching when it does
// not apply (caches over 512 positions, value heads other than 64).
// Prepared activations (Quant.Activations): row t's values at values + t * cols,
// its group scales and offsets at scales / offsets + t * stride.
struct Act {
    int8_t* values;
    float* scales;
    float* offsets;
};

// The layer's hyper-connection phi rows (RunLayerBatch, Engine.cs:2356-2364):
// 4 pre, 4 post and 16 residual-mix outputs of three Cq4 matrices over the
// stream's 4-bit prepared activations.  codes[m] points at the layer's first
// row of matrix m ([rows][K / 2] codes, the archive's row-major bytes),
// norms[m] at its fp16 group norms ([rows][K / 128]).
constexpr int kPhiMaxGroups = 32;  // phi rows of K up to 4096
struct PhiRows {
    const uint8_t* codes[3];
    const uint16_t* norms[3];
    uint32_t split[4];  // the 4-bit codebook's split lookup tables (lut4x)
    float byte_scale;   // its ByteScale
    Act in;             // the stream's Quant.Prepare rows, K = kLanes * dim
    int stride;
};

// Thread u's (output, group) unit of `outputs` phi rows (u < outputs * K /
// 128, at most one unit a thread): its 64 code bytes and fp16 norm, loaded
// ahead of the activations they meet (phi_load).
struct PhiUnit {
    uint4 w[4];
    uint32_t norm;
};

// The step's Q/K/V/Gate projections formed inside the attention launch (when
// codes[0] is set), instead of read from a matmul's output: each (row, query
// head) workgroup forms its query head and its kv head's key and value heads
// (Scalar.MatMulRows over the row's 2-bit prepared activations and the
// records' row-major codes and fp16 norms) and stores them into raw (the key
// and value heads once per kv head, for the Q/K/V history move); gate_rows /
// 16 more workgroups form 16 Gate outputs each for every row.
struct Needle3Proj {
    const uint8_t* codes[4];   // Q, K, V, Gate records: [rows_m][k / 4] 2-bit codes
    const uint16_t* norms[4];  // [rows_m][k / 128]
    uint32_t table;            // the 2-bit codebook's four level bytes
    float byte_scale;
    const int8_t* act;         // [rows][k] prepared activations (Quant.Prepare, 2-bit planes)
    const float* scales;       // [rows][stride]
    const float* offsets;
    int stride, k;
    float* raw;                // [rows][qw + kw + vw]
    float* gate;               // [rows][gate_rows]
    int gate_rows;
};

struct Needle3AttnInputs {
    const float* raw;       // [rows][qw + kw + vw]
    const float* taps[3];   // query, key, value taps: [3][width] each
    const float* q_norm;    // [qk]
    const float* k_norm;    // [qk]
    const float* rope_cos;  // [capacity][qk / 2]
    const float* rope_sin;
    const float* history;   // [slots][2][qw], [2][kw], [2][vw]: frame 0, then frame 1
    // when set, one more workgroup per row forms the row's 16 residual-mix
    // logits, its phi outputs a_res * y + b_res[o] (res_phi's matrix 2 over
    // the K = res_k prepared stream row), and their Sinkhorn4x4 into mix
    // [rows][16] beside the attention (only the layer's tail reads it)
    float* mix;
    PhiRows res_phi;
    int res_k;
    const float* a_res;  // [1]
    const float* b_res;  // [16]
    Needle3Proj proj;
};
// Whether attention_decode_needle3_impl takes a step (caches of at most 512
// positions, value heads of 64).
bool attention_needle3_fused(int32_t capacity, int32_t v_dim);
int32_t attention_decode_needle3_impl(const Needle3AttnInputs& in, int32_t rows, int32_t heads, int32_t kv_heads,
                                      int32_t qk_dim, int32_t v_dim, int8_t* d_keys, float* d_key_scales,
                                      int8_t* d_values, float* d_value_scales, int32_t slots, int32_t capacity,
                                      const int32_t* d_row_slot, const int32_t* d_row_pos,
                                      const int32_t* d_row_first, const int32_t* d_row_count, int32_t max_chunks,
                                      float* d_out, hipStream_t stream);
// nhip_needle3_attention_inputs_dev; with_history false leaves the slots'
// Q/K/V frames to the caller, which moves them on after every row of the
// step has read them.
int32_t needle3_attention_inputs_impl(const float* d_raw, int32_t rows, int32_t heads, int32_t kv_heads,
                                      int32_t qk_dim, int32_t v_dim, const float* d_q_taps, const float* d_k_taps,
                                      const float* d_v_taps, const float* d_q_norm, const float* d_k_norm,
                                      const float* d_rope_cos, const float* d_rope_sin, float* d_history,
                                      const int32_t* d_row_slot, const int32_t* d_row_pos, int32_t slots,
                                      int32_t capacity, int8_t* d_q, float* d_q_scales, int8_t* d_keys,
                                      float* d_key_scales, int8_t* d_values, float* d_value_scales, bool with_history,
                                      hipStream_t s);
// Chunk-kernel geometry of attention_decode_impl: the longest chunk of the
// plan, and the kv heads per workgroup (0 when a chunk does not fit in LDS);
// a quantized output needs every head in one workgroup.
int decode_attention_lmax(int capacity, int max_chunks);
int decode_attention_kv_per_block(int group, int kv_heads, int lmax);
// Token count from which literal int8 matmuls use the prefill kernel.
constexpr int32_t kGemmMinTokens = 32;
}  // namespace nhip

namespace nhip {

// ------------------------------------------------ exact device arithmetic --

// Scalar.HalfToSingle (src/Needle/Scalar.cs:121-128): exact binary16 decode,
// +0 for both zeros, and the reference's integer formula for exponent 31.
__device__ __forceinline__ float ref_half_to_single(uint32_t half)
{
    const uint32_t mag = half & 0x7FFFu;
    const uint32_t bits = ((mag << 13) + 0x38000000u) | ((half & 0x8000u) << 16);
    float sub = static_cast<float>(static_cast<int32_t>(mag)) * 5.9604645e-8f;
    sub = (half & 0x8000u) ? -sub : sub;
    const float v = mag < 0x0400u ? sub : __uint_as_float(bits);
    return mag == 0 ? 0.0f : v;
}

// Scalar.RoundEven (src/Needle/Scalar.cs:51-53): (x + 1.5 * 2^23) - 1.5 * 2^23
// there, which rounds half to even for |x| < 2^22 -- rint (v_rndne_f32), one
// instruction.  Every caller clamps to [-128, 127], where the two agree for
// all x (past 2^22 both keep the sign and clamp to the same end).
__device__ __forceinline__ float ref_round_even(float x) { return __builtin_rintf(x); }

// One element of Scalar.QuantizeInt8 (Scalar.cs:67-74): clamp(RoundEven(x * inverse)).
__device__ __forceinline__ int ref_quantize_one(float x, float inverse)
{
    const float r = ref_round_even(x * inverse);
    return static_cast<int>(fminf(fmaxf(r, -128.0f), 127.0f));
}

// Four elements of QuantizeInt8 packed little-endian into a dword: the low
// bytes of the four ints gathered by three v_perm_b32.
__device__ __forceinline__ uint32_t ref_quantize4(float4 h, float inverse)
{
    const uint32_t b0 = (uint32_t)ref_quantize_one(h.x, inverse);
    const uint32_t b1 = (uint32_t)ref_quantize_one(h.y, inverse);
    const uint32_t b2 = (uint32_t)ref_quantize_one(h.z, inverse);
    const uint32_t b3 = (uint32_t)ref_quantize_one(h.w, inverse);
    const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);  // [b0, b1, 0, 0]
    const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x0c0c0400u);  // [b2, b3, 0, 0]
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);               // [b0, b1, b2, b3]
}

// MathF.Max for the non-NaN operands used here (+0 preferred over -0).
__device__ __forceinline__ float ref_max(float a, float b)
{
    return a > b ? a : (b > a ? b : (__float_as_uint(a) == 0x80000000u ? b : a));
}

// ------------------------------------------- canonical row reductions --
// The decoder's element-wise kernels reduce a row of n terms (squares for
// RMSNorm, exponentials for the top-k log-sum-exp) in one canonical order
// that the CPU path repeats:
//   p[t], t < 256: the terms of elements i with (i / 4) % 256 == t, added
//                  in ascending i starting from +0 (lane t loads the float4
//                  groups at 4t, 4t + 1024, ...);
//   q[m], m < 16:  p[16m] + p[16m+1] + ... + p[16m+15], left to right;
//   total:         q folded with strides 8, 4, 2, 1 (q[m] = q[m] + q[m+s]).
// The last two levels run in the 16 lanes of one DPP row.
__device__ __forceinline__ float dpp_row_shl(float v, int n)
{
    // lane l of a 16-lane row receives lane l + n (row_shl:n; invalid lanes get 0)
    switch (n) {
        case 8: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x108, 0xF, 0xF, false));
        case 4: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x104, 0xF, 0xF, false));
        case 2: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x102, 0xF, 0xF, false));
        default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x101, 0xF, 0xF, false));
    }
}

// Levels 2 and 3 of the canonical sum for the 256 partials p[] of one row in
// LDS; called by a whole wave, the total lands in lane 0 (lanes 16, 32 and 48
// hold the same value).
__device__ __forceinline__ float canonical_finish(const float* p, int lane)
{
    const float4* p4 = reinterpret_cast<const float4*>(p + 16 * (lane & 15));
    const float4 a = p4[0], b = p4[1], c = p4[2], d = p4[3];
    float q = a.x;
    q = q + a.y;
    q = q + a.z;
    q = q + a.w;
    q = q + b.x;
    q = q + b.y;
    q = q + b.z;
    q = q + b.w;
    q = q + c.x;
    q = q + c.y;
    q = q + c.z;
    q = q + c.w;
    q = q + d.x;
    q = q + d.y;
    q = q + d.z;
    q = q + d.w;
    q = q + dpp_row_shl(q, 8);
    q = q + dpp_row_shl(q, 4);
    q = q + dpp_row_shl(q, 2);
    q = q + dpp_row_shl(q, 1);
    return q;
}

// The value lane (lane ^ S) of the wave holds, S = 1..32, without an LDS
// round trip: DPP quad permutations [1,0,3,2] (1) and [2,3,0,1] (2), a row
// half-mirror then the quad reversal [3,2,1,0] (4: 7 - l, then 3 - that
// within the quad, is l ^ 4), a row rotation by 8 (8), and gfx950's
// permlane16 / permlane32 swaps of a register with itself (16, 32: the swap
// returns the lower rows' values in its first result and the upper rows' in
// its second).
template <int S>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v)
{
    if constexpr (S == 1) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
    } else if constexpr (S == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
    } else if constexpr (S == 4) {
        const int m = __builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false);
        return (uint32_t)__builtin_amdgcn_update_dpp(0, m, 0x1B, 0xF, 0xF, false);
    } else if constexpr (S == 8) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);
    } else if constexpr (S == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (threadIdx.x & 16) ? r[0] : r[1];
    } else {
        static_assert(S == 32, "lane_xor: S is a power of two below 64");
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (threadIdx.x & 32) ? r[0] : r[1];
    }
}
template <int S>
__device__ __forceinline__ float lane_xor(float v)
{
    return __uint_as_float(lane_xor<S>(__float_as_uint(v)));
}

// The end of a Vector256 sum: lane 8k + j holds lane j of accumulator s_k
// (k < 4); returns Vector256.Sum((s0 + s1) + (s2 + s3)), with Vector256.Sum(v)
// = ((v0 + v1) + (v2 + v3)) + ((v4 + v5) + (v6 + v7)), in every lane.  Lanes
// 0-7 form the vector from their xor-partners 8, 16 and 24 (lanes j + 8,
// j + 16, j + 24), the tree runs on xor-partners 1, 2, 4, and lane 0's total
// is read out.
__device__ __forceinline__ float v256_tree(float acc)
{
    const float a16 = lane_xor<16>(acc);
    const float v = (acc + lane_xor<8>(acc)) + (a16 + lane_xor<8>(a16));
    const float p2 = v + lane_xor<1>(v);
    const float p4 = p2 + lane_xor<2>(p2);
    const float p8 = p4 + lane_xor<4>(p4);
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(p8)));
}

// Ops.SumOfSquares / Ops.Dot in the AVX2 tier's Vector256 order (Ops.cs:
// 123-205; RmsStats / CenteredRmsStats, :513-630, sum the same way), by one
// whole wave over LDS rows a and b (b = a for the squares): lane 8k + j
// (k < 4, j < 8) is lane j of accumulator s_k and takes
// fma(a[i], b[i], acc) for i = 32m + 8k + j, m ascending, over n & ~31; a
// remaining 16-block goes to s0 and s1 (lanes 0-15) and an 8-block to s2
// (lanes 16-23); the rest is a sequential FMA tail.  The total is
// Vector256.Sum((s0 + s1) + (s2 + s3)) + tail with Vector256.Sum(v) =
// ((v0 + v1) + (v2 + v3)) + ((v4 + v5) + (v6 + v7)) (.NET's Sum(lower) +
// Sum(upper)).  Returns the total in every lane; call from wave-uniform code.
__device__ __forceinline__ float wave_v256_sum(const float* a, const float* b, int n)
{
    const int lane = threadIdx.x & 63;
    const int bulk = n & ~31;
    float acc = 0.0f;
    if (lane < 32) {
        int i = lane;
        for (; i + 7 * 32 < bulk; i += 8 * 32) {
            float x[8], y[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                x[u] = a[i + 32 * u];
                y[u] = b[i + 32 * u];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) acc = fmaf(x[u], y[u], acc);
        }
        for (; i < bulk; i += 32) acc = fmaf(a[i], b[i], acc);
    }
    int i = bulk;
    if (i + 16 <= n) {
        if (lane < 16) acc = fmaf(a[i + lane], b[i + lane], acc);
        i += 16;
    }
    if (i + 8 <= n) {
        if (lane >= 16 && lane < 24) acc = fmaf(a[i + lane - 16], b[i + lane - 16], acc);
        i += 8;
    }
    float tail = 0.0f;
    for (; i < n; i++) tail = fmaf(a[i], b[i], tail);
    // lane j < 8: v_j = (s0_j + s1_j) + (s2_j + s3_j), then the pairwise tree
    return v256_tree(acc) + tail;
}

// acc = fma(a[m], b[m], acc) for m = 0 .. count-1 in ascending order, over
// two 16-byte aligned LDS rows (count % 16 == 0).  The batches of 16 steps
// alternate between two register sets: each batch is read (four 16-byte
// reads per row) before the previous one is summed, and scheduling barriers
// keep the compiler from sinking those reads below the sums, so the chain
// runs behind its reads (at most 8 reads outstanding, within the LDS
// counter's range; LDS reads return in order).
template <bool kSquares>
__device__ __forceinline__ void lds_chain_load(const float4* a4, const float4* b4, int m4, float4 (&x)[4],
                                               float4 (&y)[4])
{
#pragma unroll
    for (int u = 0; u < 4; u++) {
        x[u] = a4[m4 + u];
        if constexpr (!kSquares) y[u] = b4[m4 + u];
    }
}

template <bool kSquares>
__device__ __forceinline__ float lds_chain_sum(const float4 (&x)[4], const float4 (&y)[4], float acc)
{
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const float4 v = kSquares ? x[u] : y[u];
        acc = fmaf(x[u].x, v.x, acc);
        acc = fmaf(x[u].y, v.y, acc);
        acc = fmaf(x[u].z, v.z, acc);
        acc = fmaf(x[u].w, v.w, acc);
    }
    return acc;
}

template <bool kSquares>
__device__ __forceinline__ float lds_chain(const float* a, const float* b, int count, float acc)
{
    const float4* a4 = reinterpret_cast<const float4*>(a);
    const float4* b4 = reinterpret_cast<const float4*>(b);
    const int batches = count / 16;
    float4 xa[4], xb[4], ya[4], yb[4];
    lds_chain_load<kSquares>(a4, b4, 0, xa, xb);
    int k = 0;
    for (; k + 2 < batches; k += 2) {
        lds_chain_load<kSquares>(a4, b4, 4 * (k + 1), ya, yb);
        __builtin_amdgcn_sched_barrier(0);
        acc = lds_chain_sum<kSquares>(xa, xb, acc);
        __builtin_amdgcn_sched_barrier(0);
        lds_chain_load<kSquares>(a4, b4, 4 * (k + 2), xa, xb);
        __builtin_amdgcn_sched_barrier(0);
        acc = lds_chain_sum<kSquares>(ya, yb, acc);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (k + 1 < batches) {
        lds_chain_load<kSquares>(a4, b4, 4 * (k + 1), ya, yb);
        __builtin_amdgcn_sched_barrier(0);
        acc = lds_chain_sum<kSquares>(xa, xb, acc);
        __builtin_amdgcn_sched_barrier(0);
        acc = lds_chain_sum<kSquares>(ya, yb, acc);
    } else {
        acc = lds_chain_sum<kSquares>(xa, xb, acc);
    }
    return acc;
}

__device__ __forceinline__ float lds_fma_chain(const float* a, const float* b, int count, float acc)
{
    return lds_chain<false>(a, b, count, acc);
}

// lds_fma_chain of a row with itself (a sum of squares from +0), one read per step.
__device__ __forceinline__ float lds_square_chain(const float* a, int count)
{
    return lds_chain<true>(a, a, count, 0.0f);
}

// The padded row stride of a lane-major copy of an n-element LDS row for
// wave_v256_squares (n % 512 == 0): element i sits at (i % 32) * stride +
// i / 32, so lane L's chain is one contiguous row; the pad of 4 keeps rows
// 16-byte aligned and spreads the copy's stores over the banks.
__host__ __device__ constexpr int v256_stride(int n) { return n / 32 + 4; }

// wave_v256_sum's sum of squares (every element i < n in lane i % 32's chain
// at step i / 32, then the same tree) from the lane-major copy t of the row.
__device__ __forceinline__ float wave_v256_squares(const float* t, int n)
{
    const int lane = threadIdx.x & 63;
    float acc = 0.0f;
    if (lane < 32) acc = lds_square_chain(t + lane * v256_stride(n), n / 32);
    return v256_tree(acc);
}

// Maximum over the 64 lanes of a wave (order-free), in every lane.
__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Ops.Exp (src/Needle/Ops.cs:16-31), one lane: the reference's polynomial
// exponential, shared bit-for-bit with the CPU restatement.
__device__ __forceinline__ float exp_poly(float x)
{
    x = fminf(fmaxf(x, -87.3f), 88.7f);
    const float n = __builtin_rintf(x * 1.44269504f);
    float r = __builtin_fmaf(-n, 0.693359375f, x);
    r = __builtin_fmaf(-n, -2.12194440e-4f, r);
    float p = 1.9875691500e-4f;
    p = __builtin_fmaf(p, r, 1.3981999507e-3f);
    p = __builtin_fmaf(p, r, 8.3334519073e-3f);
    p = __builtin_fmaf(p, r, 4.1665795894e-2f);
    p = __builtin_fmaf(p, r, 1.6666665459e-1f);
    p = __builtin_fmaf(p, r, 5.0000001201e-1f);
    const float y = __builtin_fmaf(p, r * r, r + 1.0f);
    const float scale = __uint_as_float((uint32_t)((int)n + 127) << 23);
    return y * scale;
}

// Lane l of a 16-lane row receives lane l + n (n > 0) or l - n (n < 0) of
// its row, written only into the lanes of bank `bank` (lanes 4 * bank ..
// 4 * bank + 3 of each row); the other lanes keep `old`.
template <int n, int bank>
__device__ __forceinline__ float dpp_bank_shift(float old, float v)
{
    constexpr int ctrl = n > 0 ? 0x100 + n : 0x110 - n;
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), ctrl, 0xF, 1 << bank, false));
}

// The entry of column (lane & 3) in row p of the 4 x 4 matrix held by lanes
// e = 4a + c of each 16-lane row: lane 4p + c, reached from bank a by a row
// shift of 4 (p - a).
template <int p>
__device__ __forceinline__ float column_entry(float r)
{
    float v = r;  // bank p holds it itself
    if constexpr (p != 0) v = dpp_bank_shift<4 * p, 0>(v, r);
    if constexpr (p != 1) v = dpp_bank_shift<4 * (p - 1), 1>(v, r);
    if constexpr (p != 2) v = dpp_bank_shift<4 * (p - 2), 2>(v, r);
    if constexpr (p != 3) v = dpp_bank_shift<4 * (p - 3), 3>(v, r);
    return v;
}

// Lane q of the quad of 4 lanes (quad_perm [q, q, q, q]).
template <int q>
__device__ __forceinline__ float quad_entry(float r)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(r), q * 0x55, 0xF, 0xF, false));
}

// Scalar.Sinkhorn4x4 of a 4 x 4 logit matrix (row-major, 16 floats) into
// `mix` by one wave, one lane per matrix entry (lane e = 4a + c of each
// 16-lane row, the four rows alike): a matrix row is a quad of lanes and a
// column the lanes c, 4 + c, 8 + c, 12 + c, reached through DPP.  Every lane
// of a row or column forms the same left-to-right sum of its four entries,
// so each normalisation is Scalar.Sinkhorn4x4's.
__device__ __forceinline__ void sinkhorn4x4_wave(const float* logits, float* mix)
{
    const int lane = threadIdx.x & 63;
    const int e = lane & 15;
    const float lg = logits[e];
    const float peak = fmaxf(fmaxf(quad_entry<0>(lg), quad_entry<1>(lg)), fmaxf(quad_entry<2>(lg), quad_entry<3>(lg)));
    float r = exp_poly(lg - peak);
    for (int it = 0; it < 20; it++) {
        const float rs = ((quad_entry<0>(r) + quad_entry<1>(r)) + quad_entry<2>(r)) + quad_entry<3>(r);
        r = r / rs;
        const float cs = ((column_entry<0>(r) + column_entry<1>(r)) + column_entry<2>(r)) + column_entry<3>(r);
        if (cs > 0.0f) r = r / cs;
    }
    if (lane < 16) mix[e] = r;
}

// A 16-entry byte table lookup of four 4-bit codes in three operations, for
// tables whose 16 bytes are all below 128 (codebook bytes are in [0, 126]).  v_perm_b32's selector byte s
// picks byte s of its 8-byte source for s < 8, the sign of source byte 1, 3,
// 5 or 7 (0x00 or 0xFF) for s = 8..11, 0x00 for 12 and 0xFF for 13..15.
// With
//   A = perm(TA, c),  B = perm(TB, c ^ 8),
//   TA = table bytes 0..7, TB = bytes 8..15, every byte but byte 4 of each
//        stored complemented,
// one of A, B is the stored byte (TA[c] for c < 8, TB[c - 8] for c >= 8)
// and the other is 0x00 for c = 4, 12 (selector 12; stored plain) and 0xFF
// for every other c (selectors 8..11 read the complemented, sign-set bytes
// 1, 3, 5, 7, and 13..15 give 0xFF), so A ^ B is the table byte.
// c: four codes 0..15, one per byte.
__device__ __forceinline__ uint32_t lut4x(uint32_t c, uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1)
{
    const uint32_t a = __builtin_amdgcn_perm(a1, a0, c);
    const uint32_t b = __builtin_amdgcn_perm(b1, b0, c ^ 0x08080808u);
    return a ^ b;
}

// Sum of an int over the 64 lanes of a wave (exact), in every lane.
__device__ __forceinline__ int wave_sum_i32(int v)
{
    v += (int)lane_xor<32>((uint32_t)v);
    v += (int)lane_xor<16>((uint32_t)v);
    v += (int)lane_xor<8>((uint32_t)v);
    v += (int)lane_xor<4>((uint32_t)v);
    v += (int)lane_xor<2>((uint32_t)v);
    v += (int)lane_xor<1>((uint32_t)v);
    return v;
}

// Bytes idx[0..3] (each 0..3) of the four-byte table t0: the 2-bit
// codebook's levels of four indices.
__device__ __forceinline__ uint32_t lut2(uint32_t idx, uint32_t t0)
{
    return __builtin_amdgcn_perm(t0, t0, idx);
}

// One butterfly stage of hadamard_wave: lanes e and e ^ S pair up; the lower
// lane takes a + b, the upper a - b, both as p + (+-v) (p the partner's value;
// IEEE addition commutes and p - v is p + (-v)), one add per value into
// which the compiler folds the DPP move.
template <int S>
__device__ __forceinline__ void hadamard_stage(float& v0, float& v1)
{
    const uint32_t neg = ((uint32_t)threadIdx.x & S) ? 0x80000000u : 0u;
    const float n0 = __uint_as_float(__float_as_uint(v0) ^ neg);
    const float n1 = __uint_as_float(__float_as_uint(v1) ^ neg);
    v0 = lane_xor<S>(v0) + n0;
    v1 = lane_xor<S>(v1) + n1;
}

// Scalar.Hadamard (Scalar.cs:76-89) of one 128-element group held by a wave:
// lane e holds elements e (v0) and e + 64 (v1).  Butterfly stage s < 64
// pairs lanes e and e ^ s, stage 64 pairs v0 with v1; the lower element of a
// pair becomes a + b, the upper a - b, exactly as the scalar loop computes
// them (the pairs of a stage are independent), then the 1/sqrt(128) scale.
__device__ __forceinline__ void hadamard_wave(float& v0, float& v1)
{
    hadamard_stage<1>(v0, v1);
    hadamard_stage<2>(v0, v1);
    hadamard_stage<4>(v0, v1);
    hadamard_stage<8>(v0, v1);
    hadamard_stage<16>(v0, v1);
    hadamard_stage<32>(v0, v1);
    const float a = v0, b = v1;
    v0 = (a + b) * 0.08838834764831845f;
    v1 = (a - b) * 0.08838834764831845f;
}

// The rest of Quant.Prepare's scalar branch (Quant.cs:473-488) for one
// Hadamard-rotated group held by a wave (as hadamard_wave leaves it):
// QuantizeInt8 (absmax / 127), the Planes permutation (Scalar.cs:91-111:
// destination d takes quantized[src(d)]) into dst[128], and lane 0 writes the
// group's scale and offset 63 * sum(q).  WORDS (2-bit only): dst takes the
// planes positions word-interleaved instead, position 32p + j at byte
// 16 * (j / 4) + 4p + j % 4, so that one 16-byte read finds the four planes'
// words that pair with index word j / 4 of the group.
template <bool WORDS = false>
__device__ __forceinline__ void prepare_group_wave(float v0, float v1, int bits, int8_t* dst, float* scale_out,
                                                   float* offset_out)
{
    const int lane = threadIdx.x & 63;
    const float peak = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    const float inverse = 1.0f / scale;
    const int q0 = ref_quantize_one(v0, inverse);
    const int q1 = ref_quantize_one(v1, inverse);
    const int sum = wave_sum_i32(q0 + q1);
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int d = lane + 64 * k;
        int sidx;
        if (bits == 2) {
            sidx = 4 * (d & 31) + (d >> 5);              // p*32 + j <- 4j + p
        } else {
            const int half = d >> 6, r = d & 63;
            sidx = half * 64 + 2 * (r & 31) + (r >> 5);  // half*64 + p*32 + j <- half*64 + 2j + p
        }
        const int a = __shfl(q0, sidx & 63);
        const int b = __shfl(q1, sidx & 63);
        const int at = WORDS ? 16 * ((d & 31) >> 2) + 4 * (d >> 5) + (d & 3) : d;
        dst[at] = static_cast<int8_t>(sidx < 64 ? a : b);
    }
    if (lane == 0) {
        *scale_out = scale;
        *offset_out = 63.0f * (float)sum;
    }
}

// Scalar.MatMulRows' exact int32 dot (Scalar.cs:166-184) of one Cq4 row's
// group (64 code bytes) with a group of 4-bit prepared activations (128
// int8 in Planes order): code byte j of half h carries activation
// 2h * 32 + j in its low nibble and (2h + 1) * 32 + j in its high nibble.
// The codes go through lut4x to their codebook bytes (below 128, so the
// signed byte dot is exact).
__device__ __forceinline__ int cq4_group_dot(const uint4 (&w4)[4], const int8_t* x, const uint32_t (&split)[4])
{
    const uint4* x4 = reinterpret_cast<const uint4*>(x);
    int dot = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint4 wv[2] = {w4[2 * h], w4[2 * h + 1]};
        const uint4 lo[2] = {x4[4 * h], x4[4 * h + 1]};
        const uint4 hi[2] = {x4[4 * h + 2], x4[4 * h + 3]};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint4& w = wv[k >> 2];
            const uint32_t word = (k & 3) == 0 ? w.x : (k & 3) == 1 ? w.y : (k & 3) == 2 ? w.z : w.w;
            const uint4& l = lo[k >> 2];
            const uint4& u = hi[k >> 2];
            const uint32_t xl = (k & 3) == 0 ? l.x : (k & 3) == 1 ? l.y : (k & 3) == 2 ? l.z : l.w;
            const uint32_t xh = (k & 3) == 0 ? u.x : (k & 3) == 1 ? u.y : (k & 3) == 2 ? u.z : u.w;
            const uint32_t bl = lut4x(word & 0x0F0F0F0Fu, split[0], split[1], split[2], split[3]);
            const uint32_t bh = lut4x((word >> 4) & 0x0F0F0F0Fu, split[0], split[1], split[2], split[3]);
            dot = __builtin_amdgcn_sdot4((int)bl, (int)xl, dot, false);
            dot = __builtin_amdgcn_sdot4((int)bh, (int)xh, dot, false);
        }
    }
    return dot;
}

// A global-memory pointer argument held in scalar registers: selecting
// between such values per lane stays a select, where selecting struct fields
// per lane becomes a load of the chosen field through a vector address (and a
// vmcnt(0) wait that also waits for every global load issued before it).
template <typename T>
using global_ptr = const __attribute__((address_space(1))) T*;
template <typename T>
__device__ __forceinline__ global_ptr<T> scalar_ptr(const T* p)
{
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (global_ptr<T>)(((uint64_t)hi << 32) | lo);
}

// first[m] is the first output of matrix m (outputs first[m] .. first[m + 1]
// - 1 read its rows 0, 1, ...).
// base: thread base + u takes unit u (keeping the units' address work off
// waves that have other work first).
__device__ __forceinline__ PhiUnit phi_load(const PhiRows& p, int K, int m0, const int (&first)[4], int base = 0)
{
    PhiUnit r{};
    const int groups = K / 128, outputs = first[3] - first[0];
    const int u = (int)threadIdx.x - base;
    if (u >= 0 && u < outputs * groups) {
        const int o = u / groups, g = u - o * groups;
        const int m = m0 + (o >= first[1] - first[0]) + (o >= first[2] - first[0]);
        const int row = o + first[0] - first[m - m0];
        const global_ptr<uint8_t> c0 = scalar_ptr(p.codes[0]), c1 = scalar_ptr(p.codes[1]),
                                  c2 = scalar_ptr(p.codes[2]);
        const global_ptr<uint16_t> n0 = scalar_ptr(p.norms[0]), n1 = scalar_ptr(p.norms[1]),
                                   n2 = scalar_ptr(p.norms[2]);
        const global_ptr<uint8_t> codes = m == 0 ? c0 : (m == 1 ? c1 : c2);
        const global_ptr<uint16_t> norms = m == 0 ? n0 : (m == 1 ? n1 : n2);
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const global_ptr<u32x4> w4 = (global_ptr<u32x4>)(codes + (size_t)row * (K / 2) + g * 64);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const u32x4 v = w4[k];
            r.w[k] = make_uint4(v.x, v.y, v.z, v.w);
        }
        r.norm = norms[(size_t)row * groups + g];
    }
    return r;
}

// The phi outputs of one row, whose prepared activations are x [K] and its
// group scales / offsets: thread u forms its unit's group dot and the two
// products of Scalar.MatMulRows' chain (Scalar.cs:146-192): scaled =
// (HalfToSingle(norm) * ByteScale) * scale[g], scaled * dot and scaled *
// offset[g], into prod[2 * u + 0 / 1].  After a barrier, lane o < outputs
// adds them in ascending group order (accumulator += scaled * dot, bias +=
// scaled * offset) and returns accumulator - bias (other lanes return 0).
__device__ __forceinline__ float phi_outputs(const PhiRows& p, const PhiUnit& unit, const int8_t* x,
                                             const float* scales, const float* offsets, int K,
                                             const int (&first)[4], float* prod, int base = 0)
{
    const int groups = K / 128, outputs = first[3] - first[0];
    const int u = (int)threadIdx.x - base;  // phi_load's base
    if (u >= 0 && u < outputs * groups) {
        const int g = u % groups;
        const float scaled = ref_half_to_single(unit.norm) * p.byte_scale * scales[g];
        const int dot = cq4_group_dot(unit.w, x + g * 128, p.split);
        prod[2 * u] = scaled * (float)dot;
        prod[2 * u + 1] = scaled * offsets[g];
    }
    __syncthreads();
    float y = 0.0f;
    const int o = threadIdx.x;
    if (o < outputs) {
        // groups % 4 == 0 (K = 4 * dim, dim % 128 == 0): two groups a float4,
        // eight groups' reads ahead of their adds
        const float4* pr = reinterpret_cast<const float4*>(prod) + o * (groups / 2);
        float accumulator = 0.0f, bias = 0.0f;
        int g = 0;
        for (; g + 8 <= groups; g += 8) {
            const float4 v[4] = {pr[g / 2], pr[g / 2 + 1], pr[g / 2 + 2], pr[g / 2 + 3]};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                accumulator += v[j].x;
                bias += v[j].y;
                accumulator += v[j].z;
                bias += v[j].w;
            }
        }
        for (; g < groups; g += 2) {
            const float4 v = pr[g / 2];
            accumulator += v.x;
            bias += v.y;
            accumulator += v.z;
            bias += v.w;
        }
        y = accumulator - bias;
    }
    return y;
}

}  // namespace nhip

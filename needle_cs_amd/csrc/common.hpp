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
hipStream_t default_stream();
inline hipStream_t as_stream(void* s) { return s ? static_cast<hipStream_t>(s) : default_stream(); }

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
    float byte_scale;     // codebook ByteScale (1 for the literal format)
    uint8_t* tiles;
    uint16_t* norms;
    size_t device_bytes;
    int32_t special_scales;  // some scale has binary16 exponent 31 (inf/NaN patterns)
};

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

// Scalar.RoundEven (src/Needle/Scalar.cs:51-53).
__device__ __forceinline__ float ref_round_even(float x)
{
    return (x + 12582912.0f) - 12582912.0f;
}

// One element of Scalar.QuantizeInt8 (Scalar.cs:67-74): clamp(RoundEven(x * inverse)).
__device__ __forceinline__ int ref_quantize_one(float x, float inverse)
{
    const float r = ref_round_even(x * inverse);
    return static_cast<int>(fminf(fmaxf(r, -128.0f), 127.0f));
}

// MathF.Max for the non-NaN operands used here (+0 preferred over -0).
__device__ __forceinline__ float ref_max(float a, float b)
{
    return a > b ? a : (b > a ? b : (__float_as_uint(a) == 0x80000000u ? b : a));
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

}  // namespace nhip

// quant.hip -- activation quantization on gfx950.
//
// quantize_rows: Scalar.QuantizeInt8 (src/Needle/Scalar.cs:67-74) on every
//   row: peak = max|x| (a max is order-free, so the wave reduction is exact),
//   scale = peak > 0 ? peak/127 : 1, q = clamp(RoundEven(x * (1/scale))).
// prepare: Quant.Prepare's scalar branch (src/Needle/Quant.cs:473-488) per
//   128-element group: Walsh-Hadamard (Scalar.cs:76-89; every butterfly stage
//   is a pure function of the previous one, so running a stage's 64 pairs in
//   parallel reproduces the sequential loop bit for bit), QuantizeInt8,
//   Planes permutation (Scalar.cs:91-111) and offset 63*sum(q).
// Both are bit-exact with the reference's scalar code; IEEE division is the
// HIP default (correctly rounded fp32 divide).
#include "common.hpp"

namespace nhip {
namespace {

__device__ __forceinline__ float wave_max(float v)
{
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// One block of 256 threads per row.
__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ x, int cols,
                                                           int8_t* __restrict__ q, float* __restrict__ scales)
{
    __shared__ float peaks[4];
    const float* row = x + (size_t)blockIdx.x * cols;
    float peak = 0.0f;
    for (int i = threadIdx.x; i < cols; i += 256) peak = fmaxf(peak, fabsf(row[i]));
    peak = wave_max(peak);
    if ((threadIdx.x & 63) == 0) peaks[threadIdx.x >> 6] = peak;
    __syncthreads();
    peak = fmaxf(fmaxf(peaks[0], peaks[1]), fmaxf(peaks[2], peaks[3]));
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    const float inverse = 1.0f / scale;
    int8_t* out = q + (size_t)blockIdx.x * cols;
    for (int i = threadIdx.x; i < cols; i += 256) out[i] = static_cast<int8_t>(ref_quantize_one(row[i], inverse));
    if (threadIdx.x == 0) scales[blockIdx.x] = scale;
}

// One wave per (token, group): lane e holds elements e and e + 64
// (hadamard_wave, prepare_group_wave).
__global__ __launch_bounds__(256) void prepare_kernel(const float* __restrict__ x, int tokens, int cols, int bits,
                                                     int8_t* __restrict__ values, float* __restrict__ scales,
                                                     float* __restrict__ offsets, int stride)
{
    const int groups = cols / 128;
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= tokens * groups) return;
    const int t = item / groups;
    const int g = item - t * groups;
    const float* src = x + (size_t)t * cols + g * 128;
    float v0 = src[lane];
    float v1 = src[lane + 64];
    hadamard_wave(v0, v1);
    prepare_group_wave(v0, v1, bits, values + (size_t)t * cols + g * 128, scales + (size_t)t * stride + g,
                       offsets + (size_t)t * stride + g);
}

}  // namespace

int32_t quantize_rows_internal(const float* x, int32_t tokens, int32_t cols, int8_t* q, float* scales,
                               hipStream_t stream)
{
    NHIP_REQUIRE(tokens >= 0 && cols > 0, "bad shape %dx%d", tokens, cols);
    if (tokens == 0) return NHIP_OK;
    NHIP_REQUIRE(x && q && scales, "null pointer");
    hipLaunchKernelGGL(quantize_rows_kernel, dim3(tokens), dim3(256), 0, stream, x, cols, q, scales);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

int32_t prepare_internal(const float* x, int32_t tokens, int32_t cols, int32_t bits, int8_t* values, float* scales,
                         float* offsets, int32_t stride, hipStream_t stream)
{
    NHIP_REQUIRE(bits == 2 || bits == 4, "bits %d is not 2 or 4", bits);
    NHIP_REQUIRE(tokens >= 0 && cols > 0 && cols % 128 == 0, "bad shape %dx%d", tokens, cols);
    NHIP_REQUIRE(stride >= cols / 128, "stride %d < groups %d", stride, cols / 128);
    if (tokens == 0) return NHIP_OK;
    NHIP_REQUIRE(x && values && scales && offsets, "null pointer");
    const int items = tokens * (cols / 128);
    hipLaunchKernelGGL(prepare_kernel, dim3((items + 3) / 4), dim3(256), 0, stream, x, tokens, cols, bits, values,
                       scales, offsets, stride);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

}  // namespace nhip

using namespace nhip;

extern "C" {

int32_t nhip_quantize_rows_dev(const float* d_x, int32_t tokens, int32_t cols, int8_t* d_q, float* d_scales,
                               void* stream)
{
    int32_t rc = ensure_device();
    if (rc) return rc;
    return quantize_rows_internal(d_x, tokens, cols, d_q, d_scales, as_stream(stream));
}

int32_t nhip_prepare_dev(const float* d_x, int32_t tokens, int32_t cols, int32_t bits, int8_t* d_values,
                         float* d_scales, float* d_offsets, int32_t stride, void* stream)
{
    int32_t rc = ensure_device();
    if (rc) return rc;
    return prepare_internal(d_x, tokens, cols, bits, d_values, d_scales, d_offsets, stride, as_stream(stream));
}

}  // extern "C"

// gemv.hip -- quantized matmul for decode (tokens <= 16 per pass) on gfx950.
//
// Restates Scalar.MatMulRows (src/Needle/Scalar.cs:146-192) bit-exactly:
//   D_g       = sum over the group of weight_byte * activation   (int32, exact)
//   scaled    = (HalfToSingle(norm[n][g]) * ByteScale) * scale[t][g]
//   acc      += scaled * D_g ;  bias += scaled * offset[t][g]     (g ascending)
//   y[t][n]   = acc - bias
// for three weight formats: the reference's 2- and 4-bit codebook tensors
// (Cq, 128-element groups, LUT "Bytes" in [0,126], planes-ordered
// activations with per-group scales and 63*sum offsets) and the literal int8
// format (32-element groups, int8 weights, one activation scale per row, no
// offsets: ByteScale 1 and offset 0 leave the same order and bits).
//
// Mapping to CDNA4: a wave owns one 16-row tile and the whole K extent.  Per
// group one v_mfma_i32_16x16x32_i8 (int8, Cq2) or two v_mfma_i32_16x16x64_i8
// (Cq4) produce D_g for 16 tokens x 16 rows; lane l then holds D_g for rows
// l%16 and tokens 4*(l/16)..+3, so the fp32 epilogue above runs inside the
// lane in ascending g -- the reference order, no cross-lane traffic.  Weights
// are re-tiled at upload so that every lane's 16-byte load of one 1 KB block
// is exactly its MFMA B operand(s): one block = 16 rows x (2 groups of 32 B)
// for int8/Cq2, 16 rows x 1 group of 64 B for Cq4.  Activations are staged in
// LDS in per-lane operand order (conflict-free ds_read).  The dot is
// permutation-invariant in k, so the lane->k assignment only has to agree
// between A (activations) and B (weights), which it does by construction.
#include <algorithm>
#include <cstring>

#include "common.hpp"

namespace nhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));

constexpr int kWavesPerBlock = 2;
constexpr int kThreads = 64 * kWavesPerBlock;

enum Fmt { kI8 = 0, kCq2 = 1, kCq4 = 2 };

template <int F>
struct Traits;
template <>
struct Traits<kI8> {
    static constexpr int GS = 32;           // elements per group
    static constexpr int SLOTS = 1;         // MFMA A operands per group per lane
    static constexpr int SLOT_BYTES = 8;    // bytes per A operand
    static constexpr int GPB = 2;           // groups per 1 KB weight block
    static constexpr int GROUP_BYTES = 32;  // weight bytes per row per group
};
template <>
struct Traits<kCq2> {
    static constexpr int GS = 128;
    static constexpr int SLOTS = 4;
    static constexpr int SLOT_BYTES = 8;
    static constexpr int GPB = 2;
    static constexpr int GROUP_BYTES = 32;
};
template <>
struct Traits<kCq4> {
    static constexpr int GS = 128;
    static constexpr int SLOTS = 2;
    static constexpr int SLOT_BYTES = 16;
    static constexpr int GPB = 1;
    static constexpr int GROUP_BYTES = 64;
};

// Offset, inside one token's group of activations, of the bytes that lane
// quarter kq feeds as MFMA A operand `slot`.  Planes order (Scalar.cs:91-111):
// 2-bit: index byte j of a group carries the elements at planes positions
// 32p + j (p = 0..3); 4-bit: byte 32h + j carries 64h + j (low nibble) and
// 64h + 32 + j (high nibble).
template <int F>
__device__ __host__ __forceinline__ int act_pos(int slot, int kq)
{
    if (F == kI8) return 8 * kq;
    if (F == kCq2) return 32 * slot + 8 * kq;
    return (slot ? 32 : 0) + 64 * (kq >> 1) + 16 * (kq & 1);
}

struct MatmulParams {
    const uint8_t* tiles;
    const uint16_t* norms;
    const int8_t* q;          // [tokens][cols]
    const float* qscale;      // int8: [tokens]; Cq: [tokens][stride]
    const float* offsets;     // Cq: [tokens][stride]
    float* y;
    int32_t* dots;
    int32_t tokens, cols, groups, blocks, groups_pad8, stride, ldy;
    int32_t row_start, row_end, tile_begin, tile_end;
    uint32_t t0, t1, t2, t3;  // codebook bytes 0..15
    float byte_scale;
};

__device__ __forceinline__ uint32_t lut2(uint32_t idx, uint32_t t0)
{
    return __builtin_amdgcn_perm(t0, t0, idx);
}

__device__ __forceinline__ uint32_t lut4(uint32_t idx, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3)
{
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
    const uint32_t b3 = (idx >> 3) & 0x01010101u;
    const uint32_t mask = (b3 << 8) - b3;  // 0xFF in every byte whose index has bit 3 set
    return (hi & mask) | (lo & ~mask);
}

// D_g for the group `h` (0/1) of the loaded block `w`.
template <int F>
__device__ __forceinline__ v4i group_dot(const u4& w, int h, const uint8_t* lds, int g, int lane,
                                         const MatmulParams& p)
{
    v4i d = {0, 0, 0, 0};
    if constexpr (F == kI8) {
        const long a = reinterpret_cast<const long*>(lds)[g * 64 + lane];
        const long b = h ? (long)(((uint64_t)w.w << 32) | w.z) : (long)(((uint64_t)w.y << 32) | w.x);
        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, d, 0, 0, 0);
    } else if constexpr (F == kCq2) {
        const uint32_t x0 = h ? w.z : w.x;
        const uint32_t x1 = h ? w.w : w.y;
        const long* la = reinterpret_cast<const long*>(lds) + (size_t)g * 4 * 64 + lane;
#pragma unroll
        for (int pl = 0; pl < 4; pl++) {
            const uint32_t b0 = lut2((x0 >> (2 * pl)) & 0x03030303u, p.t0);
            const uint32_t b1 = lut2((x1 >> (2 * pl)) & 0x03030303u, p.t0);
            const long b = (long)(((uint64_t)b1 << 32) | b0);
            d = __builtin_amdgcn_mfma_i32_16x16x32_i8(la[pl * 64], b, d, 0, 0, 0);
        }
    } else {
        const v4i* la = reinterpret_cast<const v4i*>(lds) + (size_t)g * 2 * 64 + lane;
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int sh = 4 * s;
            v4i b;
            b.x = (int)lut4((w.x >> sh) & 0x0F0F0F0Fu, p.t0, p.t1, p.t2, p.t3);
            b.y = (int)lut4((w.y >> sh) & 0x0F0F0F0Fu, p.t0, p.t1, p.t2, p.t3);
            b.z = (int)lut4((w.z >> sh) & 0x0F0F0F0Fu, p.t0, p.t1, p.t2, p.t3);
            b.w = (int)lut4((w.w >> sh) & 0x0F0F0F0Fu, p.t0, p.t1, p.t2, p.t3);
            d = __builtin_amdgcn_mfma_i32_16x16x64_i8(la[s * 64], b, d, 0, 0, 0);
        }
    }
    return d;
}

// One wave per 16-row tile, 2 waves per block, blockIdx.y = 16-token block.
// TI = token slots per lane (min(4, tokens)); CB = 1 KB blocks loaded per
// chunk (all of a tile's blocks when K is small enough).
template <int F, int TI, int CB, bool DOTS>
__global__ __launch_bounds__(kThreads) void matmul_kernel(MatmulParams p)
{
    using T = Traits<F>;
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tile = p.tile_begin + blockIdx.x * kWavesPerBlock + wave;
    const int tb = blockIdx.y * 16;
    const int ntok = min(16, p.tokens - tb);
    const int G = p.groups;

    // Stage activations in per-lane operand order: entry e = (g, slot, lane).
    {
        const int entries = G * T::SLOTS * 64;
        for (int e = threadIdx.x; e < entries; e += kThreads) {
            const int g = e / (T::SLOTS * 64);
            const int r = e - g * (T::SLOTS * 64);
            const int slot = r >> 6;
            const int el = r & 63;
            const int t = el & 15;
            const int kq = el >> 4;
            const int8_t* src = p.q + (size_t)(tb + t) * p.cols + g * T::GS + act_pos<F>(slot, kq);
            if constexpr (T::SLOT_BYTES == 8) {
                uint2 v = make_uint2(0, 0);
                if (t < ntok) v = *reinterpret_cast<const uint2*>(src);
                reinterpret_cast<uint2*>(lds)[e] = v;
            } else {
                uint4 v = make_uint4(0, 0, 0, 0);
                if (t < ntok) v = *reinterpret_cast<const uint4*>(src);
                reinterpret_cast<uint4*>(lds)[e] = v;
            }
        }
    }
    float* sc_lds = reinterpret_cast<float*>(lds + (size_t)G * T::SLOTS * 64 * T::SLOT_BYTES);
    float* off_lds = sc_lds + 16 * G;
    if constexpr (F != kI8 && !DOTS) {
        for (int e = threadIdx.x; e < 16 * G; e += kThreads) {
            const int t = e / G;
            const int g = e - t * G;
            const bool ok = t < ntok;
            sc_lds[e] = ok ? p.qscale[(size_t)(tb + t) * p.stride + g] : 0.0f;
            off_lds[e] = ok ? p.offsets[(size_t)(tb + t) * p.stride + g] : 0.0f;
        }
    }
    __syncthreads();
    if (tile >= p.tile_end) return;

    const int r = lane & 15;
    const int kq = lane >> 4;
    const int n = tile * 16 + r;

    float qs[TI];
    float acc[TI];
    float bias[TI];
#pragma unroll
    for (int i = 0; i < TI; i++) {
        const int t = 4 * kq + i;
        if constexpr (F == kI8 && !DOTS) qs[i] = t < ntok ? p.qscale[tb + t] : 0.0f;
        acc[i] = 0.0f;
        bias[i] = 0.0f;
    }

    const u4* wbase = reinterpret_cast<const u4*>(p.tiles) + (size_t)tile * p.blocks * 64 + lane;
    const uint16_t* nrow = p.norms + (size_t)n * p.groups_pad8;
    constexpr int GPC = CB * T::GPB;  // groups per chunk (multiple of 8)

    for (int b0 = 0; b0 < p.blocks; b0 += CB) {
        u4 w[CB];
#pragma unroll
        for (int c = 0; c < CB; c++)
            if (b0 + c < p.blocks) w[c] = __builtin_nontemporal_load(wbase + (size_t)(b0 + c) * 64);
        const int g0 = b0 * T::GPB;
        uint4 sv[GPC / 8];
#pragma unroll
        for (int j = 0; j < GPC / 8; j++)
            if (g0 + 8 * j < p.groups_pad8) sv[j] = *reinterpret_cast<const uint4*>(nrow + g0 + 8 * j);
#pragma unroll
        for (int c = 0; c < CB; c++) {
#pragma unroll
            for (int h = 0; h < T::GPB; h++) {
                const int gl = c * T::GPB + h;  // group within chunk
                const int g = g0 + gl;
                if (g >= G) break;
                const v4i d = group_dot<F>(w[c], h, lds, g, lane, p);
                if constexpr (DOTS) {
#pragma unroll
                    for (int i = 0; i < TI; i++) {
                        const int t = 4 * kq + i;
                        if (t < ntok && n >= p.row_start && n < p.row_end)
                            p.dots[((size_t)(tb + t) * (p.row_end - p.row_start) + (n - p.row_start)) * G + g] = d[i];
                    }
                } else {
                    const uint4 s4 = sv[gl >> 3];
                    const uint32_t word = ((gl & 7) < 4) ? (((gl & 7) < 2) ? s4.x : s4.y) : (((gl & 7) < 6) ? s4.z : s4.w);
                    const float hs = ref_half_to_single((gl & 1) ? (word >> 16) : (word & 0xFFFFu));
#pragma unroll
                    for (int i = 0; i < TI; i++) {
                        if constexpr (F == kI8) {
                            const float scaled = hs * qs[i];
                            acc[i] = acc[i] + scaled * static_cast<float>(d[i]);
                        } else {
                            const int t = 4 * kq + i;
                            const float scaled = (hs * p.byte_scale) * sc_lds[t * G + g];
                            acc[i] = acc[i] + scaled * static_cast<float>(d[i]);
                            bias[i] = bias[i] + scaled * off_lds[t * G + g];
                        }
                    }
                }
            }
        }
    }
    if constexpr (!DOTS) {
        if (n >= p.row_start && n < p.row_end) {
#pragma unroll
            for (int i = 0; i < TI; i++) {
                const int t = 4 * kq + i;
                if (t < ntok) p.y[(size_t)(tb + t) * p.ldy + n] = acc[i] - bias[i];
            }
        }
    }
}

template <int F, int TI, int CB, bool DOTS>
int32_t launch_tpl(const MatmulParams& p, size_t lds_bytes, hipStream_t stream)
{
    auto kernel = matmul_kernel<F, TI, CB, DOTS>;
    static bool attr_set = false;
    if (!attr_set) {
        NHIP_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr_set = true;
    }
    const int tiles = p.tile_end - p.tile_begin;
    dim3 grid((tiles + kWavesPerBlock - 1) / kWavesPerBlock, (p.tokens + 15) / 16);
    hipLaunchKernelGGL(kernel, grid, dim3(kThreads), lds_bytes, stream, p);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

template <int F, int TI, bool DOTS>
int32_t launch_cb(const MatmulParams& p, size_t lds, hipStream_t s)
{
    if (p.blocks <= 8) return launch_tpl<F, TI, 8, DOTS>(p, lds, s);
    if (p.blocks <= 16) return launch_tpl<F, TI, 16, DOTS>(p, lds, s);
    return launch_tpl<F, TI, 32, DOTS>(p, lds, s);
}

template <int F, bool DOTS>
int32_t launch_fmt(const MatmulParams& p, size_t lds, hipStream_t s)
{
    switch (std::min(4, p.tokens)) {
        case 1: return launch_cb<F, 1, DOTS>(p, lds, s);
        case 2: return launch_cb<F, 2, DOTS>(p, lds, s);
        case 3: return launch_cb<F, 3, DOTS>(p, lds, s);
        default: return launch_cb<F, 4, DOTS>(p, lds, s);
    }
}

constexpr size_t kMaxLds = 160 * 1024;

int32_t run_matmul(const DeviceWeights* w, const int8_t* q, const float* scales, const float* offsets,
                   int32_t stride, int32_t tokens, float* y, int32_t ldy, int32_t row_start,
                   int32_t row_end, int32_t* dots, hipStream_t stream)
{
    NHIP_REQUIRE(w, "weights are NULL");
    NHIP_REQUIRE(tokens >= 0, "tokens %d < 0", tokens);
    NHIP_REQUIRE(row_start >= 0 && row_start <= row_end && row_end <= w->rows,
                 "row range [%d,%d) outside [0,%d)", row_start, row_end, w->rows);
    if (tokens == 0 || row_start == row_end) return NHIP_OK;
    NHIP_REQUIRE(q && (scales || dots), "activations are NULL");
    NHIP_REQUIRE(dots || (y && ldy > 0), "output NULL or ldy %d <= 0", ldy);
    const bool cq = w->format != WeightFormat::Int8G32;
    if (cq && !dots)
        NHIP_REQUIRE(offsets && stride >= w->groups, "offsets NULL or stride %d < groups %d", stride, w->groups);
    int32_t rc = ensure_device();
    if (rc) return rc;

    MatmulParams p{};
    p.tiles = w->tiles;
    p.norms = w->norms;
    p.q = q;
    p.qscale = scales;
    p.offsets = offsets;
    p.y = y;
    p.dots = dots;
    p.tokens = tokens;
    p.cols = w->cols;
    p.groups = w->groups;
    p.blocks = w->blocks;
    p.groups_pad8 = w->groups_pad8;
    p.stride = stride;
    p.ldy = ldy;
    p.row_start = row_start;
    p.row_end = row_end;
    p.tile_begin = row_start / 16;
    p.tile_end = (row_end + 15) / 16;
    p.t0 = w->table[0];
    p.t1 = w->table[1];
    p.t2 = w->table[2];
    p.t3 = w->table[3];
    p.byte_scale = w->byte_scale;

    size_t lds = (size_t)w->cols * 16;  // 16 tokens x cols bytes of staged operands
    if (cq) lds += (size_t)32 * w->groups * sizeof(float);
    if (lds > kMaxLds) {
        set_error("cols %d needs %zu bytes of LDS (max %zu)", w->cols, lds, kMaxLds);
        return NHIP_ERR_UNSUPPORTED;
    }
    switch (w->format) {
        case WeightFormat::Int8G32:
            return dots ? launch_fmt<kI8, true>(p, lds, stream) : launch_fmt<kI8, false>(p, lds, stream);
        case WeightFormat::Cq2:
            return dots ? launch_fmt<kCq2, true>(p, lds, stream) : launch_fmt<kCq2, false>(p, lds, stream);
        case WeightFormat::Cq4:
            return dots ? launch_fmt<kCq4, true>(p, lds, stream) : launch_fmt<kCq4, false>(p, lds, stream);
    }
    return NHIP_ERR_ARG;
}

// ------------------------------------------------------------ re-tiling --

// One thread per 16-byte unit of the tiled buffer.  Unit u: tile u/(blocks*64),
// block b, lane l; row n = 16*tile + l%16, quarter kq = l/16.
template <int F>
__global__ void retile_kernel(const uint8_t* __restrict__ src, int rows, int row_bytes, int groups,
                              int blocks, size_t units, uint4* __restrict__ dst)
{
    using T = Traits<F>;
    const size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units) return;
    const int lane = (int)(u & 63);
    const size_t tb = u >> 6;
    const int b = (int)(tb % blocks);
    const int tile = (int)(tb / blocks);
    const int n = tile * 16 + (lane & 15);
    const int kq = lane >> 4;
    uint4 out = make_uint4(0, 0, 0, 0);
    if (n < rows) {
        const uint8_t* row = src + (size_t)n * row_bytes;
        if constexpr (T::GPB == 2) {
            const int g0 = 2 * b;
            if (g0 < groups) {
                const uint2 lo = *reinterpret_cast<const uint2*>(row + g0 * T::GROUP_BYTES + 8 * kq);
                out.x = lo.x;
                out.y = lo.y;
            }
            if (g0 + 1 < groups) {
                const uint2 hi = *reinterpret_cast<const uint2*>(row + (g0 + 1) * T::GROUP_BYTES + 8 * kq);
                out.z = hi.x;
                out.w = hi.y;
            }
        } else {
            if (b < groups) out = *reinterpret_cast<const uint4*>(row + b * T::GROUP_BYTES + 16 * kq);
        }
    }
    dst[u] = out;
}

__global__ void pad_norms_kernel(const uint16_t* __restrict__ src, int rows, int groups, int rows_pad,
                                 int groups_pad8, uint16_t* __restrict__ dst)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows_pad * groups_pad8) return;
    const int n = (int)(i / groups_pad8);
    const int g = (int)(i % groups_pad8);
    dst[i] = (n < rows && g < groups) ? src[(size_t)n * groups + g] : (uint16_t)0;
}

int32_t create_weights(WeightFormat fmt, const uint8_t* d_src, const uint16_t* d_norms, int32_t rows,
                       int32_t cols, const nhip_codebook* book, nhip_weights** out)
{
    const int bits = static_cast<int>(fmt);
    const int gs = fmt == WeightFormat::Int8G32 ? 32 : 128;
    NHIP_REQUIRE(out, "out is NULL");
    NHIP_REQUIRE(rows > 0 && cols > 0 && cols % gs == 0, "bad shape %dx%d (cols must be a multiple of %d)", rows,
                 cols, gs);
    auto* w = new nhip_weights();
    w->format = fmt;
    w->rows = rows;
    w->cols = cols;
    w->groups = cols / gs;
    w->tiles_n = (rows + 15) / 16;
    w->blocks = fmt == WeightFormat::Cq4 ? w->groups : (w->groups + 1) / 2;
    w->groups_pad8 = (w->groups + 7) & ~7;
    w->byte_scale = 1.0f;
    w->table[0] = w->table[1] = w->table[2] = w->table[3] = 0;
    if (book) {
        std::memcpy(w->table, book->bytes, 16);
        w->byte_scale = book->byte_scale;
    }
    const size_t units = (size_t)w->tiles_n * w->blocks * 64;
    const size_t norm_elems = (size_t)w->tiles_n * 16 * w->groups_pad8;
    w->device_bytes = units * 16 + norm_elems * 2;
    hipError_t e = hipMalloc(&w->tiles, units * 16);
    if (e == hipSuccess) e = hipMalloc(&w->norms, norm_elems * 2);
    if (e != hipSuccess) {
        set_error("hipMalloc of %zu weight bytes failed: %s", w->device_bytes, hipGetErrorString(e));
        (void)hipFree(w->tiles);
        delete w;
        return NHIP_ERR_HIP;
    }
    const int row_bytes = cols * bits / 8;
    hipStream_t s = default_stream();
    const unsigned nb = (unsigned)((units + 255) / 256);
    switch (fmt) {
        case WeightFormat::Int8G32:
            hipLaunchKernelGGL(retile_kernel<kI8>, dim3(nb), dim3(256), 0, s, d_src, rows, row_bytes, w->groups,
                               w->blocks, units, reinterpret_cast<uint4*>(w->tiles));
            break;
        case WeightFormat::Cq2:
            hipLaunchKernelGGL(retile_kernel<kCq2>, dim3(nb), dim3(256), 0, s, d_src, rows, row_bytes, w->groups,
                               w->blocks, units, reinterpret_cast<uint4*>(w->tiles));
            break;
        case WeightFormat::Cq4:
            hipLaunchKernelGGL(retile_kernel<kCq4>, dim3(nb), dim3(256), 0, s, d_src, rows, row_bytes, w->groups,
                               w->blocks, units, reinterpret_cast<uint4*>(w->tiles));
            break;
    }
    hipLaunchKernelGGL(pad_norms_kernel, dim3((unsigned)((norm_elems + 255) / 256)), dim3(256), 0, s, d_norms,
                       rows, w->groups, w->tiles_n * 16, w->groups_pad8, w->norms);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        set_error("weight re-tiling failed: %s", hipGetErrorString(e));
        (void)hipFree(w->tiles);
        (void)hipFree(w->norms);
        delete w;
        return NHIP_ERR_HIP;
    }
    *out = w;
    return NHIP_OK;
}

int32_t create_from_host(WeightFormat fmt, const uint8_t* src, const uint16_t* norms, int32_t rows, int32_t cols,
                         const nhip_codebook* book, nhip_weights** out)
{
    NHIP_REQUIRE(src && norms, "weights are NULL");
    int32_t rc = ensure_device();
    if (rc) return rc;
    const int bits = static_cast<int>(fmt);
    const int gs = fmt == WeightFormat::Int8G32 ? 32 : 128;
    NHIP_REQUIRE(rows > 0 && cols > 0 && cols % gs == 0, "bad shape %dx%d", rows, cols);
    const size_t wbytes = (size_t)rows * cols * bits / 8;
    const size_t nbytes = (size_t)rows * (cols / gs) * 2;
    uint8_t* d_src = nullptr;
    uint16_t* d_norms = nullptr;
    NHIP_CHECK_HIP(hipMalloc(&d_src, wbytes));
    hipError_t e = hipMalloc(&d_norms, nbytes);
    if (e == hipSuccess) e = hipMemcpy(d_src, src, wbytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(d_norms, norms, nbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        set_error("weight upload failed: %s", hipGetErrorString(e));
        (void)hipFree(d_src);
        (void)hipFree(d_norms);
        return NHIP_ERR_HIP;
    }
    rc = create_weights(fmt, d_src, d_norms, rows, cols, book, out);
    (void)hipFree(d_src);
    (void)hipFree(d_norms);
    return rc;
}

}  // namespace

int32_t matmul_cq_internal(const DeviceWeights* w, const int8_t* values, const float* scales, const float* offsets,
                           int32_t stride, int32_t tokens, float* y, int32_t ldy, int32_t row_start,
                           int32_t row_end, hipStream_t stream)
{
    return run_matmul(w, values, scales, offsets, stride, tokens, y, ldy, row_start, row_end, nullptr, stream);
}

int32_t weights_cq_create_internal(const nhip_cq* cq, nhip_weights** out)
{
    NHIP_REQUIRE(cq && cq->indices && cq->norms && cq->book, "Cq view is incomplete");
    NHIP_REQUIRE(cq->bits == 2 || cq->bits == 4, "bits %d is not 2 or 4", cq->bits);
    return create_from_host(cq->bits == 2 ? WeightFormat::Cq2 : WeightFormat::Cq4, cq->indices, cq->norms, cq->rows,
                            cq->cols, cq->book, out);
}

}  // namespace nhip

using namespace nhip;

extern "C" {

int32_t nhip_weights_i8_create(const int8_t* w, const uint16_t* scales, int32_t rows, int32_t cols,
                               nhip_weights** out)
{
    return create_from_host(WeightFormat::Int8G32, reinterpret_cast<const uint8_t*>(w), scales, rows, cols,
                            nullptr, out);
}

int32_t nhip_weights_i8_create_dev(const int8_t* d_w, const uint16_t* d_scales, int32_t rows, int32_t cols,
                                   nhip_weights** out)
{
    NHIP_REQUIRE(d_w && d_scales, "weights are NULL");
    int32_t rc = ensure_device();
    if (rc) return rc;
    return create_weights(WeightFormat::Int8G32, reinterpret_cast<const uint8_t*>(d_w), d_scales, rows, cols,
                          nullptr, out);
}

int32_t nhip_weights_cq_create(const nhip_cq* w, nhip_weights** out)
{
    return weights_cq_create_internal(w, out);
}

int32_t nhip_weights_destroy(nhip_weights* w)
{
    if (!w) return NHIP_OK;
    (void)hipFree(w->tiles);
    (void)hipFree(w->norms);
    delete w;
    return NHIP_OK;
}

int32_t nhip_weights_info(const nhip_weights* w, int32_t* rows, int32_t* cols, int32_t* bits, size_t* device_bytes)
{
    NHIP_REQUIRE(w, "weights are NULL");
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    if (bits) *bits = static_cast<int32_t>(w->format);
    if (device_bytes) *device_bytes = w->device_bytes;
    return NHIP_OK;
}

int32_t nhip_matmul_i8_dev(const nhip_weights* w, const int8_t* d_q, const float* d_qscale, int32_t tokens,
                           float* d_y, int32_t ldy, int32_t row_start, int32_t row_end, void* stream)
{
    NHIP_REQUIRE(w && w->format == WeightFormat::Int8G32, "weights are not in the int8 format");
    NHIP_REQUIRE(ldy >= row_end, "ldy %d < row_end %d", ldy, row_end);
    return run_matmul(w, d_q, d_qscale, nullptr, 0, tokens, d_y, ldy, row_start, row_end, nullptr,
                      as_stream(stream));
}

int32_t nhip_matmul_cq_dev(const nhip_weights* w, const int8_t* d_values, const float* d_scales,
                           const float* d_offsets, int32_t stride, int32_t tokens, float* d_y, int32_t ldy,
                           int32_t row_start, int32_t row_end, void* stream)
{
    NHIP_REQUIRE(w && w->format != WeightFormat::Int8G32, "weights are not in a codebook format");
    NHIP_REQUIRE(ldy >= row_end, "ldy %d < row_end %d", ldy, row_end);
    return run_matmul(w, d_values, d_scales, d_offsets, stride, tokens, d_y, ldy, row_start, row_end, nullptr,
                      as_stream(stream));
}

int32_t nhip_group_dots_i8_dev(const nhip_weights* w, const int8_t* d_q, int32_t tokens, int32_t row_start,
                               int32_t row_end, int32_t* d_dots, void* stream)
{
    NHIP_REQUIRE(w && w->format == WeightFormat::Int8G32, "weights are not in the int8 format");
    NHIP_REQUIRE(d_dots, "dots is NULL");
    return run_matmul(w, d_q, nullptr, nullptr, 0, tokens, nullptr, 0, row_start, row_end, d_dots,
                      as_stream(stream));
}

int32_t nhip_group_dots_cq_dev(const nhip_weights* w, const int8_t* d_values, int32_t tokens, int32_t row_start,
                               int32_t row_end, int32_t* d_dots, void* stream)
{
    NHIP_REQUIRE(w && w->format != WeightFormat::Int8G32, "weights are not in a codebook format");
    NHIP_REQUIRE(d_dots, "dots is NULL");
    return run_matmul(w, d_values, nullptr, nullptr, 0, tokens, nullptr, 0, row_start, row_end, d_dots,
                      as_stream(stream));
}

}  // extern "C"

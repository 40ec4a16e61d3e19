// narrow.hip -- decode matmul of the literal int8 format for narrow
// matrices (at most kNarrowMaxRows rows) and at most 4 tokens, on gfx950.
//
// The decode kernels of gemv.hip give each workgroup one 16-row tile, so a
// matrix of N rows has N/16 workgroups: 64 for the decoder's output and down
// matmuls (N = 1024), a quarter of the 256 CUs, each pulling 64 KB of
// weights.  Here a workgroup takes RW = 4 or 8 rows over the whole K, so the
// same matrix spreads over N/RW workgroups; every row's chain still runs in
// one workgroup, so the arithmetic is the decode kernels' (Scalar.MatMulRows,
// src/Needle/Scalar.cs:146-192, literal format):
//   D_g = sum of the group's 32 int8 products (exact int32, any order);
//   p_g = (h(scale[n][g]) * qscale[t]) * D_g;
//   y[t][n] = (((0 + p_0) + p_1) + ... + p_{G-1}), one lane per (t, n).
// The weights are read from a row-major copy (DeviceWeights::rowmajor): wave
// w owns the K quarter [w*K/4, (w+1)*K/4); lane (r, c) of a wave load reads
// 16 bytes of row r at byte 16c of a SEG-byte segment (SEG = 16 * 64/RW), so
// a wave instruction reads RW contiguous segments of 256 or 128 bytes.  The
// 16 bytes are half of a group: four v_dot4 per token give the half's int32
// sum and the partner lane (c ^ 1, the other half) adds its own through DPP.
// The activations come either as int8 rows (KIND 0), or are computed from
// fp32 rows in the prologue exactly as gemv.hip's fused decode kernel does
// (kProNorm: x -> RMSNorm with the canonical row sum of squares * gain ->
// QuantizeInt8; kProQuant: QuantizeInt8 of x) into LDS, while the weight
// loads are in flight.
#include "common.hpp"

namespace nhip {
namespace {

typedef unsigned int u4 __attribute__((ext_vector_type(4)));

struct NarrowParams {
    float* y;
    const float* residual;  // set: y[t][n] = residual[t][n] + the row's sum (same ldy)
    const float* qscale;    // KIND 0: the int8 rows' scales [tokens]
    int32_t ldy, row_start, row_end, gs;
    float eps;
};

__device__ __forceinline__ float narrow_half(uint32_t h)
{
    // exact binary16 -> binary32; the launcher takes no weights with
    // exponent-31 scales (those keep the 16-row kernels' exact decode)
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// lane ^ 1's value (DPP quad_perm [1, 0, 3, 2])
__device__ __forceinline__ int pair_swap(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }

template <int RW, int NL, int WAVES, int TI, int KIND>
__global__ __launch_bounds__(64 * WAVES) void matmul_i8_narrow_kernel(const int8_t* h_w, const uint16_t* h_norms,
                                                                         const void* h_in, const float* h_gain,
                                                                         uint64_t h_k_gp8,
                                                                         uint64_t h_rows_blk0, NarrowParams p)
{
    constexpr int LPR = 64 / RW;          // lanes per row in a wave load
    constexpr int SEG = LPR * 16;         // bytes of a row per wave load
    constexpr int NT = 64 * WAVES;        // threads
    constexpr int G4 = NL * 4 / RW;       // prologue float4 of a row per thread (K = 4 * NT * G4)
    constexpr bool PRO = KIND != 0;
    constexpr bool NORM = KIND == kProNorm;
    // every address of the first loads comes from these leading (preloaded)
    // arguments: no wait on the argument segment before they issue
    const int K = head_lo(h_k_gp8);
    const int GP8 = head_hi(h_k_gp8);
    const int rows = head_lo(h_rows_blk0);
    const int G = K >> 5;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r = lane / LPR;
    const int c = lane % LPR;
    const int blk = head_hi(h_rows_blk0) + (int)blockIdx.x;
    const int nl = min(blk * RW + r, rows - 1);  // rows past the end load the last row and store nothing
    const int kw0 = wave * (K / WAVES) + c * 16;    // this lane's first weight byte in the row

    extern __shared__ __align__(16) uint8_t lds[];
    float* pl = reinterpret_cast<float*>(lds);                     // products [TI * RW][gs]
    int8_t* qa = reinterpret_cast<int8_t*>(pl + TI * RW * p.gs);   // PRO: quantized rows [TI][K]
    float* red = reinterpret_cast<float*>(qa + (PRO ? TI * K : 0));  // NORM: partial sums [TI][256]
    float* sums = red + (NORM ? TI * 256 : 0);                     // NORM: [TI]
    float* wmax = sums + TI;                                       // PRO: wave peaks [TI][WAVES]

    // 1. the activations: fp32 prologue rows, or the int8 rows' pieces
    float4 xv[PRO ? TI : 1][PRO ? G4 : 1];
    float4 gv[NORM ? G4 : 1];
    u4 av[TI][NL];  // the int8 rows' pieces (PRO: read from LDS after the prologue)
    float qs[TI];
    if constexpr (PRO) {
        const float* x = static_cast<const float*>(h_in);
#pragma unroll
        for (int j = 0; j < G4; j++) {
            const int i = 4 * (tid + NT * j);
            if constexpr (NORM) gv[j] = *reinterpret_cast<const float4*>(h_gain + i);
#pragma unroll
            for (int t = 0; t < TI; t++) xv[t][j] = *reinterpret_cast<const float4*>(x + (size_t)t * K + i);
        }
    } else {
        const int8_t* q = static_cast<const int8_t*>(h_in);
#pragma unroll
        for (int t = 0; t < TI; t++)
#pragma unroll
            for (int j = 0; j < NL; j++) av[t][j] = *reinterpret_cast<const u4*>(q + (size_t)t * K + kw0 + j * SEG);
    }
    // 2. the scales of this lane's groups, 3. its weights
    uint16_t hraw[NL];
#pragma unroll
    for (int j = 0; j < NL; j++) hraw[j] = h_norms[(size_t)nl * GP8 + ((kw0 + j * SEG) >> 5)];
    u4 w[NL];
#pragma unroll
    for (int j = 0; j < NL; j++)
        w[j] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(h_w + (size_t)nl * K + kw0 + j * SEG));
    // 4. the residual value of chain lane (t, rr) = (tid / RW, tid % RW)
    float res = 0.0f;
    if (p.residual && tid < TI * RW)
        res = p.residual[(size_t)(tid / RW) * p.ldy + min(blk * RW + tid % RW, rows - 1)];
    if constexpr (!PRO) {
#pragma unroll
        for (int t = 0; t < TI; t++) qs[t] = p.qscale[t];
    }
    __builtin_amdgcn_sched_barrier(0);

    // 5. the quantized rows (gemv.hip's fused prologue; the norm's canonical
    // sum takes 256 threads, so NORM runs with WAVES = 4)
    if constexpr (PRO) {
        float peak[TI];
#pragma unroll
        for (int t = 0; t < TI; t++) peak[t] = 0.0f;
        if constexpr (NORM) {
#pragma unroll
            for (int t = 0; t < TI; t++) {
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < G4; j++) {
                    const float4 v = xv[t][j];
                    s = s + v.x * v.x;
                    s = s + v.y * v.y;
                    s = s + v.z * v.z;
                    s = s + v.w * v.w;
                }
                red[t * 256 + tid] = s;
            }
            __syncthreads();
            if (wave < TI) {
                const float total = canonical_finish(red + wave * 256, lane);
                if (lane == 0) sums[wave] = total;
            }
            __syncthreads();
#pragma unroll
            for (int t = 0; t < TI; t++) {
                const float inv = 1.0f / sqrtf(sums[t] / (float)K + p.eps);
#pragma unroll
                for (int j = 0; j < G4; j++) {
                    const float4 v = xv[t][j];
                    xv[t][j] = make_float4((v.x * inv) * gv[j].x, (v.y * inv) * gv[j].y, (v.z * inv) * gv[j].z,
                                           (v.w * inv) * gv[j].w);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < TI; t++)
#pragma unroll
            for (int j = 0; j < G4; j++)
                peak[t] = fmaxf(fmaxf(peak[t], fmaxf(fabsf(xv[t][j].x), fabsf(xv[t][j].y))),
                                fmaxf(fabsf(xv[t][j].z), fabsf(xv[t][j].w)));
        // the row peaks over the block (order-free)
#pragma unroll
        for (int t = 0; t < TI; t++) {
            const float v = wave_max(peak[t]);
            if (lane == 0) wmax[t * WAVES + wave] = v;
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < TI; t++) {
            float pk = wmax[t * WAVES];
#pragma unroll
            for (int k = 1; k < WAVES; k++) pk = fmaxf(pk, wmax[t * WAVES + k]);
            const float scale = pk > 0.0f ? pk / 127.0f : 1.0f;
            const float inverse = 1.0f / scale;
            qs[t] = scale;
#pragma unroll
            for (int j = 0; j < G4; j++) {
                const int i = 4 * (tid + NT * j);
                *reinterpret_cast<uint32_t*>(qa + (size_t)t * K + i) = ref_quantize4(xv[t][j], inverse);
            }
        }
        __syncthreads();
    }

    // 6. the group sums and products: lane (r, c) holds half of group g of
    // row r; the even lane of each pair writes p_g
    float* prow = pl + (size_t)r * p.gs;
    if constexpr (PRO) {
        // every piece read before the first product is written: the reads
        // issue together instead of each waiting behind a write
#pragma unroll
        for (int j = 0; j < NL; j++)
#pragma unroll
            for (int t = 0; t < TI; t++) av[t][j] = *reinterpret_cast<const u4*>(qa + (size_t)t * K + kw0 + j * SEG);
    }
#pragma unroll
    for (int j = 0; j < NL; j++) {
        const int g = (kw0 + j * SEG) >> 5;
        const float hs = narrow_half(hraw[j]);
#pragma unroll
        for (int t = 0; t < TI; t++) {
            const u4 a = av[t][j];
            int d = __builtin_amdgcn_sdot4((int)a.x, (int)w[j].x, 0, false);
            d = __builtin_amdgcn_sdot4((int)a.y, (int)w[j].y, d, false);
            d = __builtin_amdgcn_sdot4((int)a.z, (int)w[j].z, d, false);
            d = __builtin_amdgcn_sdot4((int)a.w, (int)w[j].w, d, false);
            d = d + pair_swap(d);
            if ((c & 1) == 0) prow[(size_t)t * RW * p.gs + g] = (hs * qs[t]) * static_cast<float>(d);
        }
    }
    __syncthreads();

    // 7. lane (t, rr) adds its row's products in ascending group order
    if (tid < TI * RW) {
        const float4* row = reinterpret_cast<const float4*>(pl + (size_t)tid * p.gs);
        const int G4s = G >> 2;  // a multiple of 8
        float acc = 0.0f;
        int c4 = 0;
        for (; c4 + 16 <= G4s; c4 += 16) {
            float4 v[16];
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = row[c4 + k];
#pragma unroll
            for (int k = 0; k < 16; k++) {
                acc = acc + v[k].x;
                acc = acc + v[k].y;
                acc = acc + v[k].z;
                acc = acc + v[k].w;
            }
        }
        for (; c4 < G4s; c4 += 8) {
            float4 v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = row[c4 + k];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                acc = acc + v[k].x;
                acc = acc + v[k].y;
                acc = acc + v[k].z;
                acc = acc + v[k].w;
            }
        }
        const int n = blk * RW + tid % RW;
        if (n < rows && n >= p.row_start && n < p.row_end)
            p.y[(size_t)(tid / RW) * p.ldy + n] = p.residual ? res + acc : acc;
    }
}

template <int RW, int NL, int WAVES, int TI, int KIND>
int32_t launch_narrow_ti(const DeviceWeights* w, const void* in, const float* gain, const NarrowParams& p, int blocks,
                         size_t lds, hipStream_t s)
{
    static_assert(KIND != kProNorm || WAVES == 4, "the canonical sum of squares takes 256 threads");
    hipLaunchKernelGGL((matmul_i8_narrow_kernel<RW, NL, WAVES, TI, KIND>), dim3(blocks), dim3(64 * WAVES), lds, s,
                       reinterpret_cast<const int8_t*>(w->rowmajor), w->norms, in, gain,
                       head_pair(w->cols, w->groups_pad8), head_pair(w->rows, p.row_start / RW), p);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

template <int RW, int NL, int WAVES, int KIND>
int32_t launch_narrow_tokens(const DeviceWeights* w, int tokens, const void* in, const float* gain,
                             const NarrowParams& p, int blocks, size_t lds, hipStream_t s)
{
    switch (tokens) {
        case 1: return launch_narrow_ti<RW, NL, WAVES, 1, KIND>(w, in, gain, p, blocks, lds, s);
        case 2: return launch_narrow_ti<RW, NL, WAVES, 2, KIND>(w, in, gain, p, blocks, lds, s);
        case 3: return launch_narrow_ti<RW, NL, WAVES, 3, KIND>(w, in, gain, p, blocks, lds, s);
        default: return launch_narrow_ti<RW, NL, WAVES, 4, KIND>(w, in, gain, p, blocks, lds, s);
    }
}

// NL = K * RW / (1024 * WAVES) weight loads per lane, for K = 1024, 2048 or 4096
template <int RW, int WAVES, int KIND>
int32_t launch_narrow_nl(const DeviceWeights* w, int tokens, const void* in, const float* gain, const NarrowParams& p,
                         int blocks, size_t lds, hipStream_t s)
{
    constexpr int NL1 = RW / WAVES > 0 ? RW / WAVES : 1;  // NL at K = 1024 when RW >= WAVES
    const int nl = w->cols * RW / (1024 * WAVES);
    if constexpr (RW >= WAVES) {
        if (nl == NL1) return launch_narrow_tokens<RW, NL1, WAVES, KIND>(w, tokens, in, gain, p, blocks, lds, s);
        if (nl == 2 * NL1)
            return launch_narrow_tokens<RW, 2 * NL1, WAVES, KIND>(w, tokens, in, gain, p, blocks, lds, s);
        return launch_narrow_tokens<RW, 4 * NL1, WAVES, KIND>(w, tokens, in, gain, p, blocks, lds, s);
    } else {  // RW 4, 8 waves: NL 1 (K = 2048) or 2 (K = 4096)
        if (nl == 1) return launch_narrow_tokens<RW, 1, WAVES, KIND>(w, tokens, in, gain, p, blocks, lds, s);
        return launch_narrow_tokens<RW, 2, WAVES, KIND>(w, tokens, in, gain, p, blocks, lds, s);
    }
}

template <int RW, int WAVES>
int32_t launch_narrow_kind(const DeviceWeights* w, int kind, int tokens, const void* in, const float* gain,
                           const NarrowParams& p, int blocks, size_t lds, hipStream_t s)
{
    if constexpr (WAVES == 4) {
        if (kind == kProNorm) return launch_narrow_nl<RW, 4, kProNorm>(w, tokens, in, gain, p, blocks, lds, s);
    }
    if (kind == kProQuant) return launch_narrow_nl<RW, WAVES, kProQuant>(w, tokens, in, gain, p, blocks, lds, s);
    return launch_narrow_nl<RW, WAVES, 0>(w, tokens, in, gain, p, blocks, lds, s);
}

int env_int(const char* name, int fallback)
{
    const char* e = getenv(name);
    return e ? atoi(e) : fallback;
}

}  // namespace

// Which launches take the narrow kernel, and its shape.  Measured on the
// decoder's matmuls (12 layers, d 1024, M = 3; traced per launch against the
// 16-row fused kernel): down (N 1024, K 4096, quantize prologue) 7.17 ->
// 5.14 us with 4-row workgroups; output (N 1024, K 1024) 3.78 -> 3.22 us;
// the QKV matmul with its RMSNorm prologue (N 3072) 5.30 -> 5.01 us with
// 8-row workgroups (5.52 with 4-row ones).  NHIP_NARROW_RW (0 off, 4 or 8),
// NHIP_NARROW_WAVES (4 or 8) and NHIP_NARROW_NORM=0 (the norm prologue on
// the 16-row kernel) override the choices for timing.
int32_t launch_i8_narrow(const DeviceWeights* w, int32_t kind, const void* in, const float* delta,
                         const float* gain, const float* qscale, float eps, const float* residual,
                         int32_t tokens, float* y, int32_t ldy, int32_t row_start, int32_t row_end,
                         hipStream_t stream)
{
    static const int forced_rw = env_int("NHIP_NARROW_RW", -1);
    static const int forced_waves = env_int("NHIP_NARROW_WAVES", 0);
    static const bool norm_ok = env_int("NHIP_NARROW_NORM", 1) == 1;
    if (!w || !w->rowmajor || w->format != WeightFormat::Int8G32 || w->special_scales) return 1;
    // K = 1024, 2048 or 4096: each wave's K range is then a whole number of
    // NL row segments (NL = K * RW / (1024 * WAVES)) and the prologue's G4
    // float4 per thread cover K exactly; K = 3072 would leave a remainder
    if (tokens < 1 || tokens > 4 || (w->cols != 1024 && w->cols != 2048 && w->cols != 4096)) return 1;
    // a prologue with a pending delta (a decoder fallback path) keeps the
    // 16-row kernel, which also stores x + delta
    if (delta || (kind == kProNorm && !norm_ok)) return 1;
    const int rw = forced_rw >= 0 ? forced_rw : (w->rows <= 2048 ? 4 : 8);
    if (rw != 4 && rw != 8) return 1;
    int waves = forced_waves ? forced_waves : (w->cols >= 2048 ? 8 : 4);
    if (kind == kProNorm || (waves == 8 && w->cols < 2048)) waves = 4;
    NHIP_REQUIRE(in && y && ldy >= w->rows, "narrow matmul: null input/output or ldy %d below %d rows", ldy, w->rows);
    NHIP_REQUIRE(kind != 0 || qscale, "narrow matmul: int8 rows without scales");
    NHIP_REQUIRE(kind != kProNorm || gain, "narrow matmul: RMSNorm without a gain");
    const int K = w->cols;
    NarrowParams p{};
    p.y = y;
    p.residual = residual;
    p.qscale = qscale;
    p.ldy = ldy;
    p.row_start = row_start;
    p.row_end = row_end;
    p.gs = w->groups + 4;
    p.eps = eps;
    const int blocks = (row_end + rw - 1) / rw - row_start / rw;
    if (blocks <= 0) return NHIP_OK;
    const size_t lds = (size_t)tokens * rw * p.gs * 4 + (kind ? (size_t)tokens * K : 0) +
                       (kind == kProNorm ? (size_t)tokens * 256 * 4 : 0) + (size_t)tokens * (1 + waves) * 4;
    if (rw == 4)
        return waves == 8 ? launch_narrow_kind<4, 8>(w, kind, tokens, in, gain, p, blocks, lds, stream)
                          : launch_narrow_kind<4, 4>(w, kind, tokens, in, gain, p, blocks, lds, stream);
    return waves == 8 ? launch_narrow_kind<8, 8>(w, kind, tokens, in, gain, p, blocks, lds, stream)
                      : launch_narrow_kind<8, 4>(w, kind, tokens, in, gain, p, blocks, lds, stream);
}

}  // namespace nhip

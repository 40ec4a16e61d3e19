// gemm.hip -- prefill matmul of the literal int8 format (many tokens) on
// gfx950.
//
// y[t][n] for a block of 64 tokens x 128 weight rows per workgroup; each of
// the four waves owns 32 rows (two 16-row weight tiles) and all 64 tokens.
// Per 32-element group one v_mfma_i32_16x16x32_i8 per (16-token subtile,
// 16-row tile) gives the exact int32 group sums D_g (Scalar.cs:162-184);
// lane l then holds D_g for row l%16 and tokens 4*(l/16)..+3 of the
// subtile.  Two epilogues:
//   exact  acc = acc + (h(scale[n][g]) * qscale[t]) * D_g, g ascending --
//          Scalar.MatMulRows' order (Scalar.cs:185-186), bit-identical with
//          the decode kernels and the CPU restatement;
//   fused  acc = fma(h(scale[n][g]), D_g, acc), y = acc * qscale[t] -- two
//          VALU operations per (token, row, group) instead of four, within
//          1e-4 of RMS(y) of the exact result.
// The epilogue is VALU work on every (token, row, group) triple, which bounds
// this kernel below the MFMA peak: the int8 MFMAs need 2*M*N*K / 5 POPS,
// the epilogue M*N*K/32 triples x (2 or 4) operations at the VALU rate.
// Weights are the same re-tiled 1 KB blocks as the decode kernels (one
// dwordx4 per lane is the B operand of two groups), loaded by each wave for
// its own tiles.  Activations go through LDS: per stage of 4 blocks (256 K
// elements) the 256 threads load 64 tokens x 256 bytes with row-contiguous
// 16-byte loads (1 KB per wave instruction) and store them in MFMA fragment
// order, so every A operand is one conflict-free ds_read_b64 (8-byte A
// fragments loaded straight from rows 2 KB apart were the bottleneck).  The
// LDS stage is double-buffered: the next stage's activations, weights and
// scales are in flight while the current one is multiplied.
#include <algorithm>

#include "common.hpp"

namespace nhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));

constexpr int kTokensPerBlock = 64;
constexpr int kTilesPerBlock = 8;  // 16-row tiles per workgroup (2 per wave)
constexpr int kStage = 4;          // weight blocks (2 groups each) per pipeline stage
constexpr int kStageLds = kStage * 2 * 4 * 64 * 8;  // A fragments of one stage: 16 KB

struct GemmParams {
    const uint8_t* tiles;
    const uint16_t* norms;
    const int8_t* q;
    const float* qscale;
    float* y;
    int32_t tokens, cols, groups, blocks, groups_pad8, ldy;
    int32_t row_start, row_end, tile_begin, tile_end;
};

struct WStage {
    u4 w[kStage][2];  // weight blocks of the wave's two tiles
    uint4 s[2];       // fp16 scales of the stage's 8 groups, per tile row
};

template <bool EXACT, bool SPECIAL>
__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmParams p)
{
    __shared__ __align__(16) uint2 afrag[2][kStageLds / 8];  // [buf][block][h][subtile][lane]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r = lane & 15;
    const int kq = lane >> 4;
    const int t0 = blockIdx.y * kTokensPerBlock;
    const int tile0 = p.tile_begin + blockIdx.x * kTilesPerBlock + wave * 2;
    const int stages = (p.blocks + kStage - 1) / kStage;

    const u4* wbase[2];
    const uint16_t* nrow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int tj = min(tile0 + j, p.tile_end - 1);
        wbase[j] = reinterpret_cast<const u4*>(p.tiles) + (size_t)tj * p.blocks * 64 + lane;
        nrow[j] = p.norms + (size_t)(tj * 16 + r) * p.groups_pad8;
    }
    float qs[4][4];  // activation scale of token t0 + 16i + 4kq + e
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) qs[i][e] = p.qscale[min(t0 + 16 * i + 4 * kq + e, p.tokens - 1)];

    // activation staging: 16-byte unit u = j*256 + tid of a stage is token
    // u/16, bytes 16*(u%16) .. of the stage's 256-byte K slice
    auto load_a = [&](uint4 (&av)[4], int st) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int u = j * 256 + tid;
            const int t = min(t0 + (u >> 4), p.tokens - 1);
            const int kb = min(st * kStage * 64 + 16 * (u & 15), p.cols - 16);  // past K only in the padded group
            av[j] = *reinterpret_cast<const uint4*>(p.q + (size_t)t * p.cols + kb);
        }
    };
    auto store_a = [&](const uint4 (&av)[4], int buf) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int u = j * 256 + tid;
            const int tl = u >> 4;  // token within the block of 64
            const int c = u & 15;   // 16-byte chunk: block c/4, group (c%4)/2, kq 2*(c%2), +1
            const int base = (((c >> 2) * 2 + ((c & 3) >> 1)) * 4 + (tl >> 4)) * 64 + (tl & 15);
            const int k0 = 2 * (c & 1);
            afrag[buf][base + 16 * k0] = make_uint2(av[j].x, av[j].y);
            afrag[buf][base + 16 * (k0 + 1)] = make_uint2(av[j].z, av[j].w);
        }
    };
    auto load_w = [&](WStage& ws, int st) {
#pragma unroll
        for (int b = 0; b < kStage; b++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                ws.w[b][j] = wbase[j][(size_t)min(st * kStage + b, p.blocks - 1) * 64];  // cached: 8 token blocks share it
#pragma unroll
        for (int j = 0; j < 2; j++) ws.s[j] = *reinterpret_cast<const uint4*>(nrow[j] + st * kStage * 2);
    };

    float acc[2][4][4];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[j][i][e] = 0.0f;

    auto compute = [&](const WStage& ws, int buf, int st) {
#pragma unroll
        for (int b = 0; b < kStage; b++) {
            if (st * kStage + b >= p.blocks) break;  // uniform
#pragma unroll
            for (int h = 0; h < 2; h++) {
                long av[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint2 f = afrag[buf][((b * 2 + h) * 4 + i) * 64 + lane];
                    av[i] = (long)(((uint64_t)f.y << 32) | f.x);
                }
                const int g8 = b * 2 + h;  // group within the stage's 8
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const u4& wc = ws.w[b][j];
                    const long bop = h ? (long)(((uint64_t)wc.w << 32) | wc.z) : (long)(((uint64_t)wc.y << 32) | wc.x);
                    const uint4 s4 = ws.s[j];
                    const uint32_t word = g8 < 4 ? (g8 < 2 ? s4.x : s4.y) : (g8 < 6 ? s4.z : s4.w);
                    const uint32_t hbits = (g8 & 1) ? (word >> 16) : (word & 0xFFFFu);
                    float hs;
                    if constexpr (SPECIAL)
                        hs = ref_half_to_single(hbits);
                    else
                        hs = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(hbits)));
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const v4i zero = {0, 0, 0, 0};
                        const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[i], bop, zero, 0, 0, 0);
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const float df = static_cast<float>(d[e]);
                            if constexpr (EXACT)
                                acc[j][i][e] = acc[j][i][e] + (hs * qs[i][e]) * df;
                            else
                                acc[j][i][e] = __builtin_fmaf(hs, df, acc[j][i][e]);
                        }
                    }
                }
            }
        }
    };

    // pipeline: stage st+1's loads are in flight while stage st is multiplied
    uint4 areg[4];
    WStage wcur, wnext;
    load_a(areg, 0);
    load_w(wcur, 0);
    store_a(areg, 0);
    __syncthreads();
    for (int st = 0; st < stages; st++) {
        const int buf = st & 1;
        const bool more = st + 1 < stages;
        if (more) {
            load_a(areg, st + 1);
            load_w(wnext, st + 1);
        }
        compute(wcur, buf, st);
        if (more) {
            store_a(areg, buf ^ 1);  // that buffer was last read two stages ago
            wcur = wnext;
        }
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int n = (tile0 + j) * 16 + r;
        if (tile0 + j >= p.tile_end || n < p.row_start || n >= p.row_end) continue;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = t0 + 16 * i + 4 * kq + e;
                if (t < p.tokens) p.y[(size_t)t * p.ldy + n] = EXACT ? acc[j][i][e] : acc[j][i][e] * qs[i][e];
            }
    }
}

template <bool EXACT>
int32_t launch(const GemmParams& p, bool special, hipStream_t stream)
{
    const int tiles = p.tile_end - p.tile_begin;
    dim3 grid((tiles + kTilesPerBlock - 1) / kTilesPerBlock, (p.tokens + kTokensPerBlock - 1) / kTokensPerBlock);
    if (special)
        hipLaunchKernelGGL((gemm_i8_kernel<EXACT, true>), grid, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL((gemm_i8_kernel<EXACT, false>), grid, dim3(256), 0, stream, p);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

}  // namespace

int32_t launch_gemm_i8(const DeviceWeights* w, const int8_t* q, const float* qscale, int32_t tokens, float* y,
                       int32_t ldy, int32_t row_start, int32_t row_end, bool exact, hipStream_t stream)
{
    GemmParams p{};
    p.tiles = w->tiles;
    p.norms = w->norms;
    p.q = q;
    p.qscale = qscale;
    p.y = y;
    p.tokens = tokens;
    p.cols = w->cols;
    p.groups = w->groups;
    p.blocks = w->blocks;
    p.groups_pad8 = w->groups_pad8;
    p.ldy = ldy;
    p.row_start = row_start;
    p.row_end = row_end;
    p.tile_begin = row_start / 16;
    p.tile_end = (row_end + 15) / 16;
    return exact ? launch<true>(p, w->special_scales != 0, stream) : launch<false>(p, w->special_scales != 0, stream);
}

}  // namespace nhip

using namespace nhip;

extern "C" int32_t nhip_matmul_i8_fused_dev(const nhip_weights* w, const int8_t* d_q, const float* d_qscale,
                                            int32_t tokens, float* d_y, int32_t ldy, int32_t row_start,
                                            int32_t row_end, void* stream)
{
    clear_error();
    NHIP_REQUIRE(w && w->format == WeightFormat::Int8G32, "weights are not in the int8 format");
    NHIP_REQUIRE(tokens >= 0, "tokens %d < 0", tokens);
    NHIP_REQUIRE(row_start >= 0 && row_start <= row_end && row_end <= w->rows,
                 "row range [%d,%d) outside [0,%d)", row_start, row_end, w->rows);
    NHIP_REQUIRE(ldy >= row_end, "ldy %d < row_end %d", ldy, row_end);
    if (tokens == 0 || row_start == row_end) return NHIP_OK;
    NHIP_REQUIRE(d_q && d_qscale && d_y, "null pointer");
    int32_t rc = ensure_device();
    if (rc) return rc;
    return launch_gemm_i8(w, d_q, d_qscale, tokens, d_y, ldy, row_start, row_end, false, as_stream(stream));
}

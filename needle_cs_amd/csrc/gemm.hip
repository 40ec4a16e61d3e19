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
// Two format limits bound this kernel below the int8 MFMA peak: a group of
// 32 is one v_mfma_i32_16x16x32_i8 (16 cycles on gfx950, half the rate of
// the K=64 int8 instruction, whose sum would span two groups of different
// scales), and the epilogue is VALU work on every (token, row, group)
// triple, M*N*K/32 x (2 or 4) operations at the VALU rate.  Each stage is
// software-pipelined: group k+1's MFMAs and group k+2's LDS reads are in
// flight while group k's epilogue runs.
// Weights are the same re-tiled 1 KB blocks as the decode kernels (one
// dwordx4 per lane is the B operand of two groups), loaded by each wave for
// its own tiles.  Activations go through LDS: per stage of 4 blocks (256 K
// elements) the threads load 64 tokens x 256 bytes in 16-byte units and
// store each unit with one 16-byte write into an order in which every MFMA
// A operand is one conflict-free ds_read_b64 and every wave's writes are
// contiguous.  The LDS stage is double-buffered: the next stage's
// activations, weights and scales are in flight while the current one is
// multiplied.
#include <algorithm>

#include "common.hpp"

namespace nhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));

constexpr int kTokensPerBlock = 64;
constexpr int kTilesPerBlock = 8;  // 16-row tiles per workgroup (2 per wave)
constexpr int kStage = 4;          // weight blocks (2 groups each) per pipeline stage
constexpr int kSubtileSlots = 66;  // 8-byte slots per (group, subtile) block: 64 + 2 of padding
constexpr int kStageLds = kStage * 2 * 4 * kSubtileSlots * 8;  // A fragments of one stage (16.5 KB)

struct GemmParams {
    const uint8_t* tiles;
    const uint16_t* norms;
    const int8_t* q;
    const float* qscale;
    float* y;
    int32_t tokens, cols, groups, blocks, groups_pad8, ldy;
    int32_t row_start, row_end, tile_begin, tile_end;
};

template <int TPW>
struct WStage {
    u4 w[kStage][TPW];  // weight blocks of the wave's tiles
    uint4 s[TPW];       // fp16 scales of the stage's 8 groups, per tile row
};

// WAVES waves per workgroup, each owning TPW = 8 / WAVES 16-row tiles (four
// waves of two tiles measured fastest: eight waves of one tile read the
// A operands twice as often).
template <bool EXACT, bool SPECIAL, int WAVES>
__device__ __forceinline__ void gemm_i8_body(const GemmParams& p)
{
    constexpr int TPW = kTilesPerBlock / WAVES;
    constexpr int NT = 64 * WAVES;           // threads
    constexpr int AU = 1024 / NT;            // 16-byte activation units per thread and stage
    __shared__ __align__(16) uint2 afrag[2][kStageLds / 8];  // [buf][group][subtile][token][kq]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r = lane & 15;
    const int kq = lane >> 4;
    const int t0 = blockIdx.y * kTokensPerBlock;
    const int tile0 = p.tile_begin + blockIdx.x * kTilesPerBlock + wave * TPW;
    const int stages = (p.blocks + kStage - 1) / kStage;

    const u4* wbase[TPW];
    const uint16_t* nrow[TPW];
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        const int tj = min(tile0 + j, p.tile_end - 1);
        wbase[j] = reinterpret_cast<const u4*>(p.tiles) + (size_t)tj * p.blocks * 64 + lane;
        nrow[j] = p.norms + (size_t)(tj * 16 + r) * p.groups_pad8;
    }
    float qs[4][4];  // activation scale of token t0 + 16i + 4kq + e
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) qs[i][e] = p.qscale[min(t0 + 16 * i + 4 * kq + e, p.tokens - 1)];

    // activation staging: 16-byte unit u = j*NT + tid of a stage is token
    // 16*i + t16 (t16 = u%16, i = (u/32)%4), bytes 32*gs + 16*p (p = (u/16)%2,
    // gs = u/128: group within the stage) of the stage's 256-byte K slice.
    // LDS order [gs][i][t16][kq] (8 bytes each, each (gs, i) block padded to
    // 528 bytes so that the paired reads of subtiles i and i+1 fall on
    // different banks): the unit is k-slices 2p and 2p+1, one 16-byte write,
    // and lane (t16, kq) of an MFMA reads its A operand from 512 contiguous
    // bytes.
    auto load_a = [&](uint4 (&av)[AU], int st) {
#pragma unroll
        for (int j = 0; j < AU; j++) {
            const int u = j * NT + tid;
            const int t = min(t0 + ((u >> 5) & 3) * 16 + (u & 15), p.tokens - 1);
            const int kb = min(st * kStage * 64 + 32 * (u >> 7) + 16 * ((u >> 4) & 1), p.cols - 16);  // past K only in the padded group
            av[j] = *reinterpret_cast<const uint4*>(p.q + (size_t)t * p.cols + kb);
        }
    };
    auto store_a = [&](const uint4 (&av)[AU], int buf) {
#pragma unroll
        for (int j = 0; j < AU; j++) {
            const int u = j * NT + tid;
            const int slot = ((u >> 7) * 4 + ((u >> 5) & 3)) * kSubtileSlots + (u & 15) * 4 + 2 * ((u >> 4) & 1);
            *reinterpret_cast<uint4*>(&afrag[buf][slot]) = av[j];
        }
    };
    auto load_w = [&](WStage<TPW>& ws, int st) {
#pragma unroll
        for (int b = 0; b < kStage; b++)
#pragma unroll
            for (int j = 0; j < TPW; j++)
                ws.w[b][j] = wbase[j][(size_t)min(st * kStage + b, p.blocks - 1) * 64];  // cached: 8 token blocks share it
#pragma unroll
        for (int j = 0; j < TPW; j++) ws.s[j] = *reinterpret_cast<const uint4*>(nrow[j] + st * kStage * 2);
    };

    float acc[TPW][4][4];
#pragma unroll
    for (int j = 0; j < TPW; j++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[j][i][e] = 0.0f;

    // one stage: group k's A operands (four 16-token subtiles), its MFMAs
    // and its epilogue, software-pipelined so that group k+1's MFMAs and
    // group k+2's LDS reads are in flight during group k's epilogue
    auto read_a = [&](long (&av)[4], int buf, int k) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint2 f = afrag[buf][(k * 4 + i) * kSubtileSlots + r * 4 + kq];
            av[i] = (long)(((uint64_t)f.y << 32) | f.x);
        }
    };
    auto issue = [&](v4i (&d)[TPW][4], const long (&av)[4], const WStage<TPW>& ws, int k) {
        const v4i zero = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < TPW; j++) {
            const u4& wc = ws.w[k >> 1][j];
            const long bop = (k & 1) ? (long)(((uint64_t)wc.w << 32) | wc.z) : (long)(((uint64_t)wc.y << 32) | wc.x);
#pragma unroll
            for (int i = 0; i < 4; i++) d[j][i] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[i], bop, zero, 0, 0, 0);
        }
    };
    auto epilogue = [&](const v4i (&d)[TPW][4], const WStage<TPW>& ws, int k) {
#pragma unroll
        for (int j = 0; j < TPW; j++) {
            const uint4 s4 = ws.s[j];
            const uint32_t word = k < 4 ? (k < 2 ? s4.x : s4.y) : (k < 6 ? s4.z : s4.w);
            const uint32_t hbits = (k & 1) ? (word >> 16) : (word & 0xFFFFu);
            float hs;
            if constexpr (SPECIAL)
                hs = ref_half_to_single(hbits);
            else
                hs = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(hbits)));
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float df = static_cast<float>(d[j][i][e]);
                    if constexpr (EXACT)
                        acc[j][i][e] = acc[j][i][e] + (hs * qs[i][e]) * df;
                    else
                        acc[j][i][e] = __builtin_fmaf(hs, df, acc[j][i][e]);
                }
        }
    };
    constexpr int KG = 2 * kStage;  // groups per stage
    auto compute = [&](const WStage<TPW>& ws, int buf, int st) {
        long aa[2][4];
        v4i dd[2][TPW][4];
        read_a(aa[0], buf, 0);
        read_a(aa[1], buf, 1);
        issue(dd[0], aa[0], ws, 0);
#pragma unroll
        for (int k = 0; k < KG; k++) {
            if (k + 1 < KG) issue(dd[(k + 1) & 1], aa[(k + 1) & 1], ws, k + 1);
            if (k + 2 < KG) read_a(aa[k & 1], buf, k + 2);
            // groups past the last block (a partial last stage) are computed
            // on clamped operands and dropped here
            if (st * kStage + (k >> 1) < p.blocks) epilogue(dd[k & 1], ws, k);
        }
    };

    // pipeline: stage st+1's loads are in flight while stage st is
    // multiplied (the last iteration reloads the last stage, unused)
    uint4 areg[AU];
    WStage<TPW> wcur, wnext;
    load_a(areg, 0);
    load_w(wcur, 0);
    store_a(areg, 0);
    __syncthreads();
    for (int st = 0; st < stages; st++) {
        const int buf = st & 1;
        const int nst = min(st + 1, stages - 1);
        load_a(areg, nst);
        load_w(wnext, nst);
        compute(wcur, buf, st);
        store_a(areg, buf ^ 1);  // that buffer was last read two stages ago
        wcur = wnext;
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < TPW; j++) {
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

template <bool EXACT, bool SPECIAL>
__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmParams p)
{
    gemm_i8_body<EXACT, SPECIAL, 4>(p);
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

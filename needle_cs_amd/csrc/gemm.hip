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
// elements) 64 tokens x 256 bytes are copied straight from memory into LDS
// (global_load_lds, 16 bytes per lane, no registers) in an order in which
// every MFMA A operand is one conflict-free ds_read_b64.  The LDS stage is
// double-buffered: the next stage's activations, weights and scales are
// issued at the top of a stage and in flight while the current one is
// multiplied; one wait and one barrier end the stage.  (Staged through
// registers, the compiler sank the activation loads to the end of the stage
// to save registers and exposed their latency every stage.)
#include <algorithm>

#include "common.hpp"

namespace nhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));

constexpr int kTokensPerBlock = 64;
constexpr int kTilesPerBlock = 8;  // 16-row tiles per workgroup (2 per wave)
constexpr int kStage = 4;          // weight blocks (2 groups each) per pipeline stage
constexpr int kStageLds = kStage * 2 * 4 * 512;  // A fragments of one stage (16 KB)
// s_waitcnt immediate (gfx9 encoding): vmcnt 0, expcnt and lgkmcnt not waited on
constexpr int kWaitVmcnt0 = 0x0F70;

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
    __shared__ __align__(16) uint8_t afrag[2][kStageLds];  // [buf][group][subtile] blocks of 512 bytes
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

    // Activation staging, straight from memory into LDS (global_load_lds,
    // no registers): per stage 32 blocks (group gs of the stage, 16-token
    // subtile i) of 512 bytes, block b = 4*gs + i.  Position x (0..31) of a
    // block holds the 16 bytes of token 16i + x/2, k-slices 2p and 2p + 1 of
    // the group, with p = (x & 1) ^ bit 3 of the token ^ (i & 1): the MFMA
    // A reads (lane (t16, kq): 8 bytes at position 2*t16 + (kq/2 ^ ...),
    // half kq & 1) then cover all 64 banks in each half-wave, and the paired
    // reads of subtiles i and i + 1 fall on different banks.  Wave
    // instruction j of wave w fills blocks 2R and 2R + 1, R = AU*w + j, one
    // contiguous KB: lane l writes its 16 bytes at 16*l.
    auto load_a = [&](int buf, int st) {
#pragma unroll
        for (int j = 0; j < AU; j++) {
            const int R = AU * wave + j;
            const int b = 2 * R + (lane >> 5);
            const int gs = b >> 2;
            const int i = b & 3;
            const int x = lane & 31;
            const int rr = x >> 1;
            const int pp = (x & 1) ^ ((rr >> 3) & 1) ^ (i & 1);
            const int t = min(t0 + 16 * i + rr, p.tokens - 1);
            const int kb = min(st * kStage * 64 + 32 * gs + 16 * pp, p.cols - 16);  // past K only in padded groups
            __builtin_amdgcn_global_load_lds(p.q + (size_t)t * p.cols + kb, &afrag[buf][R * 1024], 16, 0, 0);
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
            const int x = 2 * r + ((kq >> 1) ^ ((r >> 3) & 1) ^ (i & 1));
            av[i] = *reinterpret_cast<const long*>(&afrag[buf][(k * 4 + i) * 512 + x * 16 + (kq & 1) * 8]);
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
            asm volatile("" : "+v"(hs));  // one conversion per scale, then full-rate v_fma_f32
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
            // groups past the last block (a partial last stage) run on
            // clamped operands with the zero scales of the padded scale rows
            epilogue(dd[k & 1], ws, k);
        }
    };

    // pipeline: stage st+1's loads are in flight while stage st is
    // multiplied (the last iteration reloads the last stage, unused)
    WStage<TPW> wcur, wnext;
    load_a(0, 0);
    load_w(wcur, 0);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    for (int st = 0; st < stages; st++) {
        const int buf = st & 1;
        const int nst = min(st + 1, stages - 1);
        load_a(buf ^ 1, nst);  // that buffer was last read in the previous stage, before the barrier
        load_w(wnext, nst);
        compute(wcur, buf, st);
        wcur = wnext;
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // this wave's LDS writes of the next stage have landed
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

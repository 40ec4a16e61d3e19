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
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "common.hpp"

namespace nhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));

constexpr size_t kMaxLds = 64 * 1024;  // dynamic LDS per block

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
    // tiles .. mask_rows: what the decode kernels' first loads need, also
    // passed as their preloaded leading arguments (MATMUL_HEAD_PARAMS)
    const uint8_t* tiles;
    const uint16_t* norms;
    const int8_t* q;          // [tokens][cols]
    const float* qscale;      // int8: [tokens]; Cq: [tokens][stride]
    int32_t tokens, cols, groups, blocks;
    int32_t tile_begin;
    int32_t mask_rows;        // > 0: tile_mask is set (see below)
    const float* offsets;     // Cq: [tokens][stride]
    float* y;
    int32_t* dots;
    int32_t groups_pad8, stride, ldy;  // groups_pad8 = (groups + 7) & ~7
    int32_t row_start, row_end, tile_end;
    int32_t gph;              // groups per phase (a multiple of Traits::GPB)
    int32_t d_bytes;          // LDS bytes of the D buffer of one phase
    int32_t ldd;              // LDS row stride (int32) of D and scales: roundup4(gph) + 4
    int32_t st_bytes;         // int8 path: LDS bytes of the staged activation operands
    int32_t swz;              // decode path, 5..16 tokens: float4-column swizzle mask of the products
    int32_t swiglu;           // fused decode path: rows are (8 gate, 8 up) pairs per tile, store SwiGLU
    const float* residual;    // fused decode path: y[t][n] = residual[t][n] + the row's sum (same ldy)
    const uint32_t* tile_mask;  // decode kernel: [mask_rows][mask_words] id bitsets; tiles with no set bit
    int32_t mask_words;         // in any row are skipped (their outputs are left untouched)
    uint32_t t0, t1, t2, t3;  // codebook bytes 0..15
    uint32_t x0, x1, x2, x3;  // the split tables of lut4x (TA, TB)
    float byte_scale;
    // codebook decode kernels: rows n >= split_row[k] (k < split_n, rows
    // ascending) are stored at row n - split_row[k] of split_y[k] (stride
    // split_ldy[k]) instead of y, so one launch over matrices stacked by rows
    // (sharing the activations and K) fills each one's own output
    int32_t split_n;
    int32_t split_row[3], split_ldy[3];
    float* split_y[3];
};

// Row nn of token t's output (the split outputs, and the row range).
__device__ __forceinline__ void store_row(const MatmulParams& p, int t, int nn, float v)
{
    if (nn < p.row_start || nn >= p.row_end) return;
    float* y = p.y;
    int ldy = p.ldy, n = nn;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        if (k < p.split_n && nn >= p.split_row[k]) {
            y = p.split_y[k];
            ldy = p.split_ldy[k];
            n = nn - p.split_row[k];
        }
    }
    y[(size_t)t * ldy + n] = v;
}

// The argument-segment fields the products and the chain use, read once the
// first loads are in flight: used only after a barrier, the compiler would
// load them there, one more round trip on the kernel's critical path.
#define MATMUL_TAIL_FIELDS(p)                                                                                   \
    asm volatile("" ::"s"((p).y), "s"((p).ldy), "s"((p).row_start), "s"((p).row_end), "s"((p).swiglu),          \
                 "s"((p).residual), "s"((p).ldd), "s"((p).swz), "s"(blockDim.x))

// The split outputs' fields (codebook decode kernels), read at the same time.
#define MATMUL_SPLIT_FIELDS(p)                                                                                   \
    asm volatile("" ::"s"((p).split_n), "s"((p).split_row[0]), "s"((p).split_row[1]), "s"((p).split_row[2]),   \
                 "s"((p).split_ldy[0]), "s"((p).split_ldy[1]), "s"((p).split_ldy[2]), "s"((p).split_y[0]),     \
                 "s"((p).split_y[1]), "s"((p).split_y[2]))

// The decode kernels' head (see head_pair): the fields of their first loads.
#define MATMUL_HEAD_PARAMS const uint8_t *h_tiles, const uint16_t *h_norms, const int8_t *h_q, const float *h_qscale, \
                           uint64_t h_tokens_cols, uint64_t h_groups_blocks, uint64_t h_begin_mask
#define MATMUL_HEAD_ARGS(p) (p).tiles, (p).norms, (p).q, (p).qscale, head_pair((p).tokens, (p).cols), \
                            head_pair((p).groups, (p).blocks), head_pair((p).tile_begin, (p).mask_rows)
#define MATMUL_TAKE_HEAD(p)                    \
    do {                                       \
        (p).tiles = h_tiles;                   \
        (p).norms = h_norms;                   \
        (p).q = h_q;                           \
        (p).qscale = h_qscale;                 \
        (p).tokens = head_lo(h_tokens_cols);   \
        (p).cols = head_hi(h_tokens_cols);     \
        (p).groups = head_lo(h_groups_blocks); \
        (p).blocks = head_hi(h_groups_blocks); \
        (p).tile_begin = head_lo(h_begin_mask); \
        (p).mask_rows = head_hi(h_begin_mask); \
    } while (0)

__device__ __forceinline__ uint32_t lut4(uint32_t idx, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3)
{
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
    const uint32_t b3 = (idx >> 3) & 0x01010101u;
    const uint32_t mask = (b3 << 8) - b3;  // 0xFF in every byte whose index has bit 3 set
    return (hi & mask) | (lo & ~mask);
}

// The MFMA A operand(s) one lane supplies for one group: activation bytes of
// token lane%16 at act_pos(slot, lane/16) inside the group.
template <int F>
struct Operand;
template <>
struct Operand<kI8> {
    long a;
};
template <>
struct Operand<kCq2> {
    long a[4];
};
template <>
struct Operand<kCq4> {
    v4i a[2];
};

template <int F>
__device__ __forceinline__ Operand<F> load_operand(const int8_t* qrow, bool valid, int g, int kq)
{
    using T = Traits<F>;
    Operand<F> o;
    const int8_t* base = qrow + (size_t)g * T::GS;
    if constexpr (F == kI8) {
        const long v = *reinterpret_cast<const long*>(base + act_pos<F>(0, kq));
        o.a = valid ? v : 0;
    } else if constexpr (F == kCq2) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const long v = *reinterpret_cast<const long*>(base + act_pos<F>(s, kq));
            o.a[s] = valid ? v : 0;
        }
    } else {
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const v4i v = *reinterpret_cast<const v4i*>(base + act_pos<F>(s, kq));
            const v4i zero = {0, 0, 0, 0};
            o.a[s] = valid ? v : zero;
        }
    }
    return o;
}

// d + the MFMA products of group `h` (0/1) of the loaded weight block `w`:
// D_g itself when d is zero.
// SPLIT: Cq4 codes go through lut4x and the split tables x0..x3.
template <int F, bool SPLIT = false>
__device__ __forceinline__ v4i group_dot(const u4& w, int h, const Operand<F>& a, const MatmulParams& p,
                                         v4i d = v4i{0, 0, 0, 0})
{
    if constexpr (F == kI8) {
        const long b = h ? (long)(((uint64_t)w.w << 32) | w.z) : (long)(((uint64_t)w.y << 32) | w.x);
        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a.a, b, d, 0, 0, 0);
    } else if constexpr (F == kCq2) {
        const uint32_t x0 = h ? w.z : w.x;
        const uint32_t x1 = h ? w.w : w.y;
#pragma unroll
        for (int pl = 0; pl < 4; pl++) {
            const uint32_t b0 = lut2((x0 >> (2 * pl)) & 0x03030303u, p.t0);
            const uint32_t b1 = lut2((x1 >> (2 * pl)) & 0x03030303u, p.t0);
            d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a.a[pl], (long)(((uint64_t)b1 << 32) | b0), d, 0, 0, 0);
        }
    } else {
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int sh = 4 * s;
            v4i b;
            if constexpr (SPLIT) {
                b.x = (int)lut4x((w.x >> sh) & 0x0F0F0F0Fu, p.x0, p.x1, p.x2, p.x3);
                b.y = (int)lut4x((w.y >> sh) & 0x0F0F0F0Fu, p.x0, p.x1, p.x2, p.x3);
                b.z = (int)lut4x((w.z >> sh) & 0x0F0F0F0Fu, p.x0, p.x1, p.x2, p.x3);
                b.w = (int)lut4x((w.w >> sh) & 0x0F0F0F0Fu, p.x0, p.x1, p.x2, p.x3);
            } else {
                b.x = (int)lut4((w.x >> sh) & 0x0F0F0F0Fu, p.t0, p.t1, p.t2, p.t3);
                b.y = (int)lut4((w.y >> sh) & 0x0F0F0F0Fu, p.t0, p.t1, p.t2, p.t3);
                b.z = (int)lut4((w.z >> sh) & 0x0F0F0F0Fu, p.t0, p.t1, p.t2, p.t3);
                b.w = (int)lut4((w.w >> sh) & 0x0F0F0F0Fu, p.t0, p.t1, p.t2, p.t3);
            }
            d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.a[s], b, d, 0, 0, 0);
        }
    }
    return d;
}

// The operand itself, or zeros (an A row block that must not contribute).
template <int F>
__device__ __forceinline__ Operand<F> operand_if(const Operand<F>& o, bool keep)
{
    Operand<F> z;
    if constexpr (F == kI8) {
        z.a = keep ? o.a : 0;
    } else if constexpr (F == kCq2) {
#pragma unroll
        for (int s = 0; s < 4; s++) z.a[s] = keep ? o.a[s] : 0;
    } else {
        const v4i zero = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < 2; s++) z.a[s] = keep ? o.a[s] : zero;
    }
    return z;
}

// One block per (16-row tile, 16-token block); S = blockDim.x/64 waves split
// the tile's weight blocks.  Per phase of `gph` groups:
//  1. group dots: every wave loads its share of activation operands (first)
//     and 1 KB weight blocks (all in flight together), runs one MFMA chain per
//     group and writes the int32 D_g of the valid tokens to LDS [g][t][row];
//     the fp16 scales of its groups are decoded (Scalar.HalfToSingle) to LDS;
//  2. epilogue: thread c owns the (token c/16, row c%16) accumulator and
//     walks the phase's groups in ascending order:
//         scaled = (hs * ByteScale) * scale[t][g]; acc += scaled * D_g;
//         bias += scaled * offset[t][g]           (Cq formats)
//         scaled = hs * scale[t];  acc += scaled * D_g          (int8)
//     which is Scalar.MatMulRows' exact operation order (Scalar.cs:185-189);
//     phases continue the same accumulators, so the order spans all of K.
template <int F, int CB, bool DOTS>
__device__ __forceinline__ void matmul_tile(const MatmulParams& p, const int tile)
{
    using T = Traits<F>;
    extern __shared__ __align__(16) uint8_t lds[];
    // D as [token][row][gph + 4] int32 and scales as [row][gph + 4] float: a
    // chain reads 4 consecutive groups per 16-byte load, and the 16-byte row
    // padding spreads the MFMA-side writes of 16 rows over distinct banks.
    const int ld = p.ldd;
    int32_t* dl = reinterpret_cast<int32_t*>(lds);
    float* hl = reinterpret_cast<float*>(lds + p.d_bytes);
    const int S = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tb = blockIdx.y * 16;
    const int M = min(16, p.tokens - tb);
    const int G = p.groups;
    const int r = lane & 15;
    const int kq = lane >> 4;
    const int n = tile * 16 + r;
    // A operand token = lane % 16; lanes past the last token load token
    // M-1's bytes (a valid address) and zero them.
    const bool tok_ok = r < M;
    const int8_t* qrow = p.q + (size_t)(tb + min(r, M - 1)) * p.cols;
    const u4* wbase = reinterpret_cast<const u4*>(p.tiles) + (size_t)tile * p.blocks * 64 + lane;
    const uint16_t* nrow = p.norms + (size_t)n * p.groups_pad8;
    int32_t* dummy = reinterpret_cast<int32_t*>(lds + p.d_bytes + 16 * p.ldd * 4);  // sink for masked stores

    // epilogue ownership: thread c accumulates (token c/16, row c%16)
    const int ct = threadIdx.x >> 4;
    const int cr = threadIdx.x & 15;
    const bool chain = !DOTS && ct < M;
    float acc = 0.0f, bias = 0.0f;

    for (int p0 = 0; p0 < G; p0 += p.gph) {
        const int gend = min(G, p0 + p.gph);
        const int b_begin = p0 / T::GPB;
        const int b_end = (gend + T::GPB - 1) / T::GPB;
        const int per = (b_end - b_begin + S - 1) / S;
        const int mb0 = b_begin + wave * per;
        const int mb1 = min(b_end, mb0 + per);
        const int g_first = mb0 * T::GPB;
        const int g_last = min(gend, mb1 * T::GPB);  // exclusive

        // Straight-line issue: operands, then every weight block, then the
        // raw scales, all in flight before the first MFMA waits.  Blocks and
        // groups past this wave's share are clamped to valid addresses and
        // their results discarded.
        Operand<F> ops[CB * T::GPB];
#pragma unroll
        for (int c = 0; c < CB; c++)
#pragma unroll
            for (int h = 0; h < T::GPB; h++) {
                const int g = min((mb0 + c) * T::GPB + h, G - 1);
                ops[c * T::GPB + h] = load_operand<F>(qrow, tok_ok, g, kq);
            }
        u4 w[CB];
#pragma unroll
        for (int c = 0; c < CB; c++) w[c] = __builtin_nontemporal_load(wbase + (size_t)min(mb0 + c, b_end - 1) * 64);
        constexpr int HJ = (CB * T::GPB + 3) / 4;
        uint16_t hraw[HJ];
        if constexpr (!DOTS) {
#pragma unroll
            for (int j = 0; j < HJ; j++) hraw[j] = nrow[min(g_first + 4 * j + kq, G - 1)];
        }
        // Keep every load above this point: the scheduler would otherwise sink
        // weight loads between MFMAs and serialise memory round trips.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < CB; c++) {
#pragma unroll
            for (int h = 0; h < T::GPB; h++) {
                const int g = (mb0 + c) * T::GPB + h;
                const bool g_ok = g < g_last;
                const v4i d = group_dot<F>(w[c], h, ops[c * T::GPB + h], p);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = 4 * kq + i;
                    if constexpr (DOTS) {
                        if (g_ok && t < M && n >= p.row_start && n < p.row_end)
                            p.dots[((size_t)(tb + t) * (p.row_end - p.row_start) + (n - p.row_start)) * G + g] = d[i];
                    } else {
                        int32_t* dst = (g_ok && t < M) ? dl + (t * 16 + r) * ld + (g - p0) : dummy + lane;
                        *dst = d[i];
                    }
                }
            }
        }
        if constexpr (DOTS) continue;
#pragma unroll
        for (int j = 0; j < HJ; j++) {
            const int g = g_first + 4 * j + kq;
            float* dst = g < g_last ? hl + r * ld + (g - p0) : reinterpret_cast<float*>(dummy) + lane;
            *dst = ref_half_to_single(hraw[j]);
        }
        __syncthreads();
        if (chain) {
            float qs = 0.0f;
            if constexpr (F == kI8) qs = p.qscale[tb + ct];
            const int32_t* drow = dl + (ct * 16 + cr) * ld;
            const float* hrow = hl + cr * ld;
            const float* sc_row = nullptr;
            const float* off_row = nullptr;
            if constexpr (F != kI8) {
                sc_row = p.qscale + (size_t)(tb + ct) * p.stride + p0;
                off_row = p.offsets + (size_t)(tb + ct) * p.stride + p0;
            }
            const int cnt = gend - p0;
            int g = 0;
            for (; g + 8 <= cnt; g += 8) {
                const v4i d0 = *reinterpret_cast<const v4i*>(drow + g);
                const v4i d1 = *reinterpret_cast<const v4i*>(drow + g + 4);
                const float4 h0 = *reinterpret_cast<const float4*>(hrow + g);
                const float4 h1 = *reinterpret_cast<const float4*>(hrow + g + 4);
                const float dv[8] = {(float)d0.x, (float)d0.y, (float)d0.z, (float)d0.w,
                                     (float)d1.x, (float)d1.y, (float)d1.z, (float)d1.w};
                const float hv[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
                if constexpr (F == kI8) {
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        const float scaled = hv[k] * qs;
                        acc = acc + scaled * dv[k];
                    }
                } else {
                    const float4 s0 = *reinterpret_cast<const float4*>(sc_row + g);
                    const float4 s1 = *reinterpret_cast<const float4*>(sc_row + g + 4);
                    const float4 o0 = *reinterpret_cast<const float4*>(off_row + g);
                    const float4 o1 = *reinterpret_cast<const float4*>(off_row + g + 4);
                    const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
                    const float ov[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        const float scaled = (hv[k] * p.byte_scale) * sv[k];
                        acc = acc + scaled * dv[k];
                        bias = bias + scaled * ov[k];
                    }
                }
            }
            for (; g < cnt; g++) {
                const float dv = static_cast<float>(drow[g]);
                if constexpr (F == kI8) {
                    const float scaled = hrow[g] * qs;
                    acc = acc + scaled * dv;
                } else {
                    const float scaled = (hrow[g] * p.byte_scale) * sc_row[g];
                    acc = acc + scaled * dv;
                    bias = bias + scaled * off_row[g];
                }
            }
        }
        __syncthreads();
    }
    if (chain) {
        const int nc = tile * 16 + cr;
        if (nc >= p.row_start && nc < p.row_end) p.y[(size_t)(tb + ct) * p.ldy + nc] = acc - bias;
    }
}

template <int F, int CB, bool DOTS>
__global__ __launch_bounds__(512) void matmul_kernel(MatmulParams p)
{
    matmul_tile<F, CB, DOTS>(p, p.tile_begin + blockIdx.x);
}

// Literal int8 path.  Same phases and epilogue as matmul_kernel, but the
// activation operands are staged once per block: the M token rows of the
// phase's K range are read with coalesced 16-byte loads (issued before the
// weight blocks) and written to LDS as [group][kq][token] 8-byte MFMA A
// operands, so each wave issues one weight load per 1 KB block and no
// scattered activation loads.
template <int CB, int NS, bool DOTS>
__global__ __launch_bounds__(512) void matmul_i8_kernel(MatmulParams p)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int ld = p.ldd;
    uint2* st = reinterpret_cast<uint2*>(lds);
    float* pl = reinterpret_cast<float*>(lds + p.st_bytes);  // products [token][row][ld]
    float* dummy = reinterpret_cast<float*>(lds + p.st_bytes + p.d_bytes);  // 256-float sink
    const int S = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tile = p.tile_begin + blockIdx.x;
    const int tb = blockIdx.y * 16;
    const int M = min(16, p.tokens - tb);
    const int G = p.groups;
    const int r = lane & 15;
    const int kq = lane >> 4;
    const int n = tile * 16 + r;
    const int ra = min(r, M - 1);  // A operand token (lanes past M read a valid row and zero it)
    const u4* wbase = reinterpret_cast<const u4*>(p.tiles) + (size_t)tile * p.blocks * 64 + lane;
    const uint16_t* nrow = p.norms + (size_t)n * p.groups_pad8;
    const int8_t* qblock = p.q + (size_t)tb * p.cols;

    const int ct = threadIdx.x >> 4;
    const int cr = threadIdx.x & 15;
    const bool chain = !DOTS && ct < M;
    float acc = 0.0f;

    for (int p0 = 0; p0 < G; p0 += p.gph) {
        const int gend = min(G, p0 + p.gph);
        const int gcnt = gend - p0;
        const int b_begin = p0 >> 1;
        const int b_end = (gend + 1) >> 1;
        const int per = (b_end - b_begin + S - 1) / S;
        const int mb0 = b_begin + wave * per;
        const int mb1 = min(b_end, mb0 + per);
        const int g_first = mb0 * 2;
        const int g_last = min(gend, mb1 * 2);

        // 1. activation rows of this phase: unit u = (token, 16-byte offset)
        const int units = M * gcnt * 2;
        uint4 sv[NS];
#pragma unroll
        for (int j = 0; j < NS; j++) {
            const int u = min((int)threadIdx.x + j * (int)blockDim.x, units - 1);
            const int t = u / (2 * gcnt);
            const int o = (u - t * 2 * gcnt) * 16;
            sv[j] = *reinterpret_cast<const uint4*>(qblock + (size_t)t * p.cols + p0 * 32 + o);
        }
        // 2. raw scales (lane kq holds groups g_first+4j+kq), 3. weight
        //    blocks -- scales first so that waiting for them does not wait
        //    for the weights (loads complete in issue order)
        constexpr int HJ = (CB * 2 + 3) / 4;
        uint16_t hraw[HJ];
        // activation scales of the four tokens this lane's MFMA results belong to
        float qraw[4];
        if constexpr (!DOTS) {
#pragma unroll
            for (int j = 0; j < HJ; j++) hraw[j] = nrow[min(g_first + 4 * j + kq, G - 1)];
#pragma unroll
            for (int i = 0; i < 4; i++) qraw[i] = p.qscale[tb + min(4 * kq + i, M - 1)];
        }
        u4 w[CB];
#pragma unroll
        for (int c = 0; c < CB; c++) w[c] = __builtin_nontemporal_load(wbase + (size_t)min(mb0 + c, b_end - 1) * 64);
        __builtin_amdgcn_sched_barrier(0);
        // 4. staged operands to LDS: bytes o..o+15 of a row are kq = (o%32)/8
        //    and kq+1 of group o/32
#pragma unroll
        for (int j = 0; j < NS; j++) {
            const int u = (int)threadIdx.x + j * (int)blockDim.x;
            const int uc = min(u, units - 1);
            const int t = uc / (2 * gcnt);
            const int o = (uc - t * 2 * gcnt) * 16;
            const int g = o >> 5;
            const int k0 = (o & 31) >> 3;
            uint2* d0 = u < units ? st + (g * 4 + k0) * M + t : reinterpret_cast<uint2*>(dummy) + lane;
            uint2* d1 = u < units ? st + (g * 4 + k0 + 1) * M + t : reinterpret_cast<uint2*>(dummy) + 64 + lane;
            *d0 = make_uint2(sv[j].x, sv[j].y);
            *d1 = make_uint2(sv[j].z, sv[j].w);
        }
        float hsv[HJ];
        if constexpr (!DOTS) {
#pragma unroll
            for (int j = 0; j < HJ; j++) hsv[j] = ref_half_to_single(hraw[j]);
        }
        __syncthreads();
        // 5. all A operands from LDS, then all MFMAs (each waits only for its
        //    own weight block), then the products of Scalar.cs:185-186
        //      scaled = HalfToSingle(norm[n][g]) * ByteScale(1) * scale[t]
        //      prod   = scaled * D_g      (rounded; added to acc in step 6)
        long av[2 * CB];
#pragma unroll
        for (int k = 0; k < 2 * CB; k++) {
            const int gl = min(g_first + k, gend - 1) - p0;
            const long araw = *reinterpret_cast<const long*>(st + (gl * 4 + kq) * M + ra);
            av[k] = r < M ? araw : 0;
        }
        v4i dv[2 * CB];
#pragma unroll
        for (int k = 0; k < 2 * CB; k++) {
            const u4& wc = w[k >> 1];
            const long b = (k & 1) ? (long)(((uint64_t)wc.w << 32) | wc.z) : (long)(((uint64_t)wc.y << 32) | wc.x);
            const v4i zero = {0, 0, 0, 0};
            dv[k] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[k], b, zero, 0, 0, 0);
        }
        if constexpr (DOTS) {
#pragma unroll
            for (int k = 0; k < 2 * CB; k++) {
                const int g = g_first + k;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = 4 * kq + i;
                    if (g < g_last && t < M && n >= p.row_start && n < p.row_end)
                        p.dots[((size_t)(tb + t) * (p.row_end - p.row_start) + (n - p.row_start)) * G + g] = dv[k][i];
                }
            }
        } else {
            float qs[4];
#pragma unroll
            for (int i = 0; i < 4; i++) qs[i] = 4 * kq + i < M ? qraw[i] : 0.0f;
            // scale of (row r, group g_first + k) sits in lane (k % 4) * 16 + r
            float hk[2 * CB];
#pragma unroll
            for (int k = 0; k < 2 * CB; k++) hk[k] = __shfl(hsv[k >> 2], (k & 3) * 16 + r);
#pragma unroll
            for (int k = 0; k < 2 * CB; k++) {
                const int g = g_first + k;
                const bool g_ok = g < g_last;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = 4 * kq + i;
                    const float scaled = hk[k] * qs[i];
                    const float prod = scaled * static_cast<float>(dv[k][i]);
                    float* dst = (g_ok && t < M) ? pl + (t * 16 + r) * ld + (g - p0) : dummy + 128 + lane;
                    *dst = prod;
                }
            }
        }
        __syncthreads();
        if constexpr (DOTS) continue;
        // 6. each (token, row) accumulator adds its products in ascending g
        if (chain) {
            const float* prow = pl + (ct * 16 + cr) * ld;
            int g = 0;
            for (; g + 8 <= gcnt; g += 8) {
                const float4 v0 = *reinterpret_cast<const float4*>(prow + g);
                const float4 v1 = *reinterpret_cast<const float4*>(prow + g + 4);
                acc = acc + v0.x;
                acc = acc + v0.y;
                acc = acc + v0.z;
                acc = acc + v0.w;
                acc = acc + v1.x;
                acc = acc + v1.y;
                acc = acc + v1.z;
                acc = acc + v1.w;
            }
            for (; g < gcnt; g++) acc = acc + prow[g];
        }
        __syncthreads();
    }
    if (chain) {
        const int nc = tile * 16 + cr;
        if (nc >= p.row_start && nc < p.row_end) p.y[(size_t)(tb + ct) * p.ldy + nc] = acc;
    }
}

__device__ __forceinline__ float decode_scale_fast(uint32_t h)
{
    // binary16 -> binary32 is exact; a -0 scale gives a +-0 product, which
    // cannot change an accumulator that starts at +0.
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// M <= 4 tokens: four groups g..g+3 share one D.  MFMA j of a set holds group
// g+j's activations in A rows 4j..4j+3 (zero elsewhere) and accumulates into
// the previous result; the row blocks are disjoint, so D rows 4j+i are
// exactly D_{g+j} of token i, and lane (r, kq) ends up holding the M tokens
// of group g+kq.  Each product (hs * scale[t]) * D_g goes to LDS at
// pl[(t*16 + r)*GS + g].  av[c]: this lane's A operand of set c (token r%4,
// group g + r/4, k-slice kq; zero for tokens >= M); hraw[c]: the scale of
// (row r, group g + kq).
template <int CB, int TI, bool EXACT>
__device__ __forceinline__ void narrow_products(const long (&av)[2 * CB / 4], const float (&qs)[TI],
                                                const uint16_t (&hraw)[2 * CB / 4], const u4 (&w)[CB], float* pl,
                                                int GS, int M, int g_first, int r, int kq)
{
    const v4i zero = {0, 0, 0, 0};
    float* prow = pl + (size_t)r * GS + g_first + kq;
#pragma unroll
    for (int c = 0; c < 2 * CB / 4; c++) {
        v4i d = zero;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const u4& wc = w[2 * c + (j >> 1)];
            const long b = (j & 1) ? (long)(((uint64_t)wc.w << 32) | wc.z) : (long)(((uint64_t)wc.y << 32) | wc.x);
            d = __builtin_amdgcn_mfma_i32_16x16x32_i8((r >> 2) == j ? av[c] : 0, b, d, 0, 0, 0);
        }
        const float hs = EXACT ? ref_half_to_single(hraw[c]) : decode_scale_fast(hraw[c]);
        // groups >= G are written (inside the row) but never read
#pragma unroll
        for (int i = 0; i < TI; i++)
            if (i < M) prow[(size_t)i * 16 * GS + 4 * c] = (hs * qs[i]) * static_cast<float>(d[i]);
    }
}

// The lanes (t, r) of the first M*16 threads add row (t, r)'s products in
// ascending group order and store y[t][n].  Float4 column c of product row
// x sits at column c ^ (x & swz).  With p.swiglu the tile's rows are gate
// rows j = 8*tile + r (r < 8) followed by the matching up rows: lane r < 8
// takes lane r + 8's sum (DPP row_shl:8 within the token's 16-lane row) and
// stores a = (g / (1 + Exp(-g))) * u at y[t][j].
// res: this lane's residual value when p.residual is set (the stored value
// is then res + acc)
__device__ __forceinline__ void store_chain(float acc, int t, int rr, int nn, int tile, const MatmulParams& p,
                                            float res = 0.0f)
{
    if (p.swiglu) {
        const float u = dpp_row_shl(acc, 8);
        if (rr < 8) p.y[(size_t)t * p.ldy + tile * 8 + rr] = (acc / (1.0f + exp_poly(-acc))) * u;
    } else if (nn >= p.row_start && nn < p.row_end) {
        p.y[(size_t)t * p.ldy + nn] = p.residual ? res + acc : acc;
    }
}

__device__ __forceinline__ void chain_products(const float* pl, int GS, int swz, int M, int G, int tile,
                                               const MatmulParams& p, float res = 0.0f)
{
    for (int x = threadIdx.x; x < M * 16; x += blockDim.x) {
        const int t = x >> 4;
        const int rr = x & 15;
        const int nn = tile * 16 + rr;
        const float4* row = reinterpret_cast<const float4*>(pl + (size_t)x * GS);
        const int sw = x & swz;
        float acc = 0.0f;
        // the float4 columns in batches of 16 (64 groups), then 4: every read
        // of a batch is issued before its first add, so the LDS latency is
        // exposed once per batch (a one-batch-ahead prefetch of 4 columns,
        // which the compiler served only after the current batch's wait,
        // exposed it every 16 groups)
        const int G4 = G >> 2;
        int c4 = 0;
        for (; c4 + 16 <= G4; c4 += 16) {
            float4 v[16];
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = row[(c4 + j) ^ sw];
#pragma unroll
            for (int j = 0; j < 16; j++) {
                acc = acc + v[j].x;
                acc = acc + v[j].y;
                acc = acc + v[j].z;
                acc = acc + v[j].w;
            }
        }
        for (; c4 + 4 <= G4; c4 += 4) {
            float4 v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = row[(c4 + j) ^ sw];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc = acc + v[j].x;
                acc = acc + v[j].y;
                acc = acc + v[j].z;
                acc = acc + v[j].w;
            }
        }
        const int full = c4 >> 2;  // chunks of 16 groups done
        const float* rowf = reinterpret_cast<const float*>(row);
        for (int c = full * 16; c < G; c++) acc = acc + rowf[(((c >> 2) ^ sw) << 2) | (c & 3)];
        store_chain(acc, t, rr, nn, tile, p, res);
    }
}

// Decode path of the literal int8 format for M <= 16 tokens (beam rows,
// packed sequences).  Each of the S waves of a 16-row tile owns CB weight
// blocks (2*CB groups) and loads its A operands (its K range of the M rows)
// straight from memory; it computes the products p_g = (hs * scale[t]) * D_g
// (Scalar.cs:185-186) and leaves them in LDS as [t][r][g]; after one barrier
// the lanes (t, r) add them in ascending group order, so each y[t][n] is
// exactly (((0 + p_0) + p_1) + ... + p_{G-1}).
//   TI <= 4: narrow_products (four groups per MFMA set, every lane's
//            products useful); product rows are padded (stride
//            GS = roundup4(2*blocks) + 4).
//   TI == 16: one group per MFMA; lane (r, kq) holds tokens 4kq..4kq+3 of
//            row r; the products are M*16 rows of GS = roundup4(2*blocks)
//            floats, the float4 column c of product row x stored at column
//            c ^ (x & swz), which keeps both the writes and the chain's
//            reads free of bank conflicts without padding.
// Preconditions (checked on the host): CB is 4 or 8 and every wave owns CB
// blocks (its scales are 16-byte aligned in the padded scale rows).
template <int CB, int TI, bool EXACT>
__device__ __forceinline__ void i8_decode_tile(const MatmulParams& p, const int tile)
{
    constexpr bool WIDE = TI > 4;
    constexpr int SETS = 2 * CB / 4;  // TI <= 4: sets of four groups per wave
    extern __shared__ __align__(16) uint8_t lds[];
    float* pl = reinterpret_cast<float*>(lds);  // products [t][r][GS]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int M = p.tokens;  // <= TI
    const int G = p.groups;
    const int GS = p.ldd;    // product row stride (floats), multiple of 4
    const int r = lane & 15;
    const int kq = lane >> 4;
    const int n = tile * 16 + r;
    const int mb0 = wave * CB;
    const int g_first = mb0 * 2;
    const u4* wbase = reinterpret_cast<const u4*>(p.tiles) + (size_t)tile * p.blocks * 64 + lane;
    const uint16_t* nrow = p.norms + (size_t)n * ((G + 7) & ~7) + g_first;
    if (p.mask_rows > 0) {
        // sparse rows: the tile's 16 ids are bits 16*(tile&1).. of word tile/2
        // (the mask and its word count are read from the argument segment
        // only on this path)
        uint32_t live = 0;
        for (int t = 0; t < p.mask_rows; t++)
            live |= (p.tile_mask[(size_t)t * p.mask_words + (tile >> 1)] >> (16 * (tile & 1))) & 0xFFFFu;
        if (!live) return;  // uniform over the workgroup
    }

    // 1. activation operands, 2. activation scales, 3. weight scales,
    // 4. weight blocks -- in this order, all in flight together
    constexpr int NA = WIDE ? 2 * CB : SETS;
    constexpr int TL = WIDE ? 4 : TI;  // tokens per lane
    long av[NA];
    float qraw[TL];
    if constexpr (WIDE) {
        // 8 bytes (k-slice kq) of token r per group
        const int8_t* qrow = p.q + (size_t)min(r, M - 1) * p.cols + kq * 8;
#pragma unroll
        for (int k = 0; k < NA; k++)
            av[k] = *reinterpret_cast<const long*>(qrow + (size_t)min(g_first + k, G - 1) * 32);
#pragma unroll
        for (int i = 0; i < 4; i++) qraw[i] = p.qscale[min(4 * kq + i, M - 1)];
    } else {
        // lane (r, kq) feeds A row r of MFMA r/4: token r%4, group
        // g + r/4, k-slice kq
        const int8_t* qrow = p.q + (size_t)min(r & 3, M - 1) * p.cols + kq * 8;
#pragma unroll
        for (int c = 0; c < NA; c++)
            av[c] = *reinterpret_cast<const long*>(qrow + (size_t)min(g_first + 4 * c + (r >> 2), G - 1) * 32);
#pragma unroll
        for (int i = 0; i < TI; i++) qraw[i] = p.qscale[min(i, M - 1)];
    }
    constexpr int SJ = WIDE ? CB / 4 : SETS;
    uint4 sraw[WIDE ? SJ : 1];
    uint16_t hraw[WIDE ? 1 : SJ];
    if constexpr (WIDE) {
        // 8 groups per 16-byte load
#pragma unroll
        for (int j = 0; j < SJ; j++) sraw[j] = *reinterpret_cast<const uint4*>(nrow + 8 * j);
    } else {
        // the scale of this lane's group g + kq in each set
#pragma unroll
        for (int c = 0; c < SJ; c++) hraw[c] = nrow[4 * c + kq];
    }
    u4 w[CB];
#pragma unroll
    for (int c = 0; c < CB; c++) w[c] = __builtin_nontemporal_load(wbase + (size_t)(mb0 + c) * 64);
    __builtin_amdgcn_sched_barrier(0);
    MATMUL_TAIL_FIELDS(p);

    if constexpr (WIDE) {
        const v4i zero = {0, 0, 0, 0};
        const int tq = 4 * kq;  // first token of this lane's MFMA results
        float qs[4];
#pragma unroll
        for (int i = 0; i < 4; i++) qs[i] = tq + i < M ? qraw[i] : 0.0f;
        float pr[2 * CB][4];
#pragma unroll
        for (int k = 0; k < 2 * CB; k++) {
            const u4& wc = w[k >> 1];
            const long b = (k & 1) ? (long)(((uint64_t)wc.w << 32) | wc.z) : (long)(((uint64_t)wc.y << 32) | wc.x);
            const long a = r < M ? av[k] : 0;
            const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, zero, 0, 0, 0);
            const uint4 s4 = sraw[k >> 3];
            const int kk = k & 7;
            const uint32_t word = kk < 4 ? (kk < 2 ? s4.x : s4.y) : (kk < 6 ? s4.z : s4.w);
            const uint32_t h = (kk & 1) ? (word >> 16) : (word & 0xFFFFu);
            const float hs = EXACT ? ref_half_to_single(h) : decode_scale_fast(h);
#pragma unroll
            for (int i = 0; i < 4; i++) pr[k][i] = (hs * qs[i]) * static_cast<float>(d[i]);
        }
        // groups >= G are written (inside the row) but never read
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int x = (tq + i) * 16 + r;  // product row
            if (tq + i < M) {
                float4* dst = reinterpret_cast<float4*>(pl + (size_t)x * GS);
#pragma unroll
                for (int k4 = 0; k4 < 2 * CB; k4 += 4)
                    dst[((g_first + k4) >> 2) ^ (x & p.swz)] =
                        make_float4(pr[k4][i], pr[k4 + 1][i], pr[k4 + 2][i], pr[k4 + 3][i]);
            }
        }
    } else {
        const bool feeds = (r & 3) < M;  // A rows of tokens >= M stay zero
#pragma unroll
        for (int c = 0; c < NA; c++) av[c] = feeds ? av[c] : 0;
        narrow_products<CB, TI, EXACT>(av, qraw, hraw, w, pl, GS, M, g_first, r, kq);
    }
    __syncthreads();
    chain_products(pl, GS, WIDE ? p.swz : 0, M, G, tile, p);
}

template <int CB, int TI, bool EXACT>
__global__ __launch_bounds__(512) void matmul_i8_decode_kernel(MATMUL_HEAD_PARAMS, MatmulParams p)
{
    MATMUL_TAKE_HEAD(p);
    i8_decode_tile<CB, TI, EXACT>(p, p.tile_begin + blockIdx.x);
}

// Quant.MatMulBatch (src/Needle/Quant.cs:679-816): up to four weight
// matrices with the same K that share one set of activations, in one launch.
// Job j owns the workgroups [first[j], first[j+1]), one per 16-row tile of
// its rows; every job has the same tile shape (blocks, waves, LDS), so one
// kernel instance serves them all.
constexpr int kMaxBatchJobs = 4;

struct MatmulBatch {
    MatmulParams job[kMaxBatchJobs];
    int32_t first[kMaxBatchJobs + 1];
    int32_t count;
};

__device__ __forceinline__ int batch_job(const MatmulBatch& b)
{
    int j = 0;
#pragma unroll
    for (int i = 1; i < kMaxBatchJobs; i++) j += (i < b.count && (int)blockIdx.x >= b.first[i]) ? 1 : 0;
    return j;
}

// MatMulBatch over more tokens than the decode kernels take: the general
// kernel's tiles of every job (same K, tokens and phase plan) in one launch.
template <int F, int CB>
__global__ __launch_bounds__(512) void matmul_batch_kernel(MatmulBatch b)
{
    const int j = batch_job(b);
    const MatmulParams& p = b.job[j];
    matmul_tile<F, CB, false>(p, p.tile_begin + (int)blockIdx.x - b.first[j]);
}

template <int CB, int TI, bool EXACT>
__global__ __launch_bounds__(512) void matmul_i8_decode_batch_kernel(MatmulBatch b)
{
    const int j = batch_job(b);
    const MatmulParams& p = b.job[j];
    i8_decode_tile<CB, TI, EXACT>(p, p.tile_begin + (int)blockIdx.x - b.first[j]);
}

// Codebook formats, M <= 4 tokens: the four-group MFMA sets of
// narrow_products with the codebook epilogue.  Wave w owns the GPW groups
// from g_first = GPW*w (groups past G run on clamped operands and are
// dropped).  Set c covers groups g_first + 4c + j, j < 4: group j's MFMAs
// take A rows 4j..4j+3 (tokens 0..3) and that group's weights, so lane
// (r, kq) ends up holding D_g of row r, g = g_first + 4c + kq, for tokens
// 0..3.  The lane leaves
//     scaled     = (HalfToSingle(norm[n][g]) * ByteScale) * scale[t][g]
//     pa[t][r][g] = scaled * D_g,   pb[t][r][g] = scaled * offset[t][g]
// in LDS; after one barrier lane (t, r) adds both rows in ascending g and
// stores acc - bias, Scalar.MatMulRows' operations in its order
// (Scalar.cs:185-189).
template <int F, int GPW, bool EXACT, bool SPLIT>
__device__ __forceinline__ void cq_decode_tile(const MatmulParams& p, const int tile)
{
    using T = Traits<F>;
    constexpr int SETS = GPW / 4;
    constexpr int CB = GPW / T::GPB;  // weight blocks per wave
    extern __shared__ __align__(16) uint8_t lds[];
    const int M = p.tokens;  // 1..4
    const int G = p.groups;
    const int GS = p.ldd;    // product row stride (floats), a multiple of 4
    float* pa = reinterpret_cast<float*>(lds);
    float* pb = pa + (size_t)M * 16 * GS;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;
    const int kq = lane >> 4;
    const int n = tile * 16 + r;
    const int g_first = wave * GPW;
    const u4* wbase = reinterpret_cast<const u4*>(p.tiles) + (size_t)tile * p.blocks * 64 + lane;
    const uint16_t* nrow = p.norms + (size_t)n * ((G + 7) & ~7);

    // 1. A operands: lane (r, kq) feeds A row r of every set, token r%4
    //    (rows of tokens >= M repeat token M-1; their D rows are never
    //    read) of group g_first + 4c + r/4; 2. weight scales of the lane's
    //    groups g_first + 4c + kq; 3. weight blocks; 4. the activation
    //    scales and offsets of those groups -- all in flight together (the
    //    first three from the preloaded arguments, the last after the
    //    argument segment's stride and offsets arrive)
    const int8_t* qrow = p.q + (size_t)min(r & 3, M - 1) * p.cols;
    Operand<F> av[SETS];
#pragma unroll
    for (int c = 0; c < SETS; c++) av[c] = load_operand<F>(qrow, true, min(g_first + 4 * c + (r >> 2), G - 1), kq);
    uint16_t hraw[SETS];
#pragma unroll
    for (int c = 0; c < SETS; c++) hraw[c] = nrow[min(g_first + 4 * c + kq, G - 1)];
    u4 w[CB];
#pragma unroll
    for (int c = 0; c < CB; c++)
        w[c] = __builtin_nontemporal_load(wbase + (size_t)min(wave * CB + c, p.blocks - 1) * 64);
    float sc[SETS][4], of[SETS][4];
#pragma unroll
    for (int c = 0; c < SETS; c++) {
        const int g = min(g_first + 4 * c + kq, G - 1);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const size_t at = (size_t)min(i, M - 1) * p.stride + g;
            sc[c][i] = p.qscale[at];
            of[c][i] = p.offsets[at];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    MATMUL_TAIL_FIELDS(p);
    if constexpr (SPLIT) MATMUL_SPLIT_FIELDS(p);

#pragma unroll
    for (int c = 0; c < SETS; c++) {
        v4i d = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int gl = 4 * c + j;  // group within the wave
            d = group_dot<F, true>(w[gl / T::GPB], gl % T::GPB, operand_if<F>(av[c], (r >> 2) == j), p, d);
        }
        const float hs = EXACT ? ref_half_to_single(hraw[c]) : decode_scale_fast(hraw[c]);
        const float hb = hs * p.byte_scale;
        // groups >= G are written (inside the row) but never read
        const size_t at = (size_t)r * GS + g_first + 4 * c + kq;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (i < M) {
                const float scaled = hb * sc[c][i];
                pa[at + (size_t)i * 16 * GS] = scaled * static_cast<float>(d[i]);
                pb[at + (size_t)i * 16 * GS] = scaled * of[c][i];
            }
        }
    }
    __syncthreads();
    for (int x = threadIdx.x; x < M * 16; x += blockDim.x) {
        const int nn = tile * 16 + (x & 15);
        const float* ra = pa + (size_t)x * GS;
        const float* rb = pb + (size_t)x * GS;
        float acc = 0.0f, bias = 0.0f;
        int g = 0;
        // 16 groups per batch, every read of a batch issued before its
        // first add (one exposed LDS latency per batch)
        for (; g + 16 <= G; g += 16) {
            float4 a[4], b[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                a[j] = *reinterpret_cast<const float4*>(ra + g + 4 * j);
                b[j] = *reinterpret_cast<const float4*>(rb + g + 4 * j);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc = acc + a[j].x;
                bias = bias + b[j].x;
                acc = acc + a[j].y;
                bias = bias + b[j].y;
                acc = acc + a[j].z;
                bias = bias + b[j].z;
                acc = acc + a[j].w;
                bias = bias + b[j].w;
            }
        }
        for (; g + 4 <= G; g += 4) {
            const float4 a = *reinterpret_cast<const float4*>(ra + g);
            const float4 b = *reinterpret_cast<const float4*>(rb + g);
            acc = acc + a.x;
            bias = bias + b.x;
            acc = acc + a.y;
            bias = bias + b.y;
            acc = acc + a.z;
            bias = bias + b.z;
            acc = acc + a.w;
            bias = bias + b.w;
        }
        for (; g < G; g++) {
            acc = acc + ra[g];
            bias = bias + rb[g];
        }
        if constexpr (SPLIT)
            store_row(p, x >> 4, nn, acc - bias);
        else if (nn >= p.row_start && nn < p.row_end)
            p.y[(size_t)(x >> 4) * p.ldy + nn] = acc - bias;
    }
}

// Codebook formats, 5..16 tokens: one group per MFMA set, whose A rows are
// the 16 tokens (rows of tokens >= M zero), so lane (r, kq) holds D_g of
// row r for tokens 4kq..4kq+3.  Wave w owns the GPW groups from
// g_first = GPW*w (groups past G run on clamped operands; their columns are
// never read).  The lane leaves, per group and token,
//     scaled = (HalfToSingle(norm[n][g]) * ByteScale) * scale[t][g]
//     pa[t][r][g] = scaled * D_g,   pb[t][r][g] = scaled * offset[t][g]
// in LDS as float4 columns of four groups, column c of product row x at
// c ^ (x & swz) (the int8 decode path's swizzle); after one barrier lane
// (t, r) adds both rows in ascending g and stores acc - bias, Scalar.MatMulRows'
// operations in its order (Scalar.cs:185-189), as cq_decode_tile does.
template <int F, int GPW, bool EXACT, bool SPLIT>
__device__ __forceinline__ void cq_decode_wide_tile(const MatmulParams& p, const int tile)
{
    using T = Traits<F>;
    static_assert(GPW % 4 == 0, "products are stored four groups at a time");
    constexpr int CB = GPW / T::GPB;  // weight blocks per wave
    extern __shared__ __align__(16) uint8_t lds[];
    const int M = p.tokens;  // 5..16
    const int G = p.groups;
    const int GS = p.ldd;    // product row stride (floats): every group a wave writes, a multiple of 4
    float4* pa = reinterpret_cast<float4*>(lds);
    float4* pb = pa + (size_t)M * 16 * (GS / 4);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;
    const int kq = lane >> 4;
    const int n = tile * 16 + r;
    const int g_first = wave * GPW;
    const u4* wbase = reinterpret_cast<const u4*>(p.tiles) + (size_t)tile * p.blocks * 64 + lane;
    const uint16_t* nrow = p.norms + (size_t)n * ((G + 7) & ~7);

    // 1. A operands of token r, 2. weight scales of row n, 3. weight blocks,
    // 4. activation scales and offsets of tokens 4kq..4kq+3 (their stride
    // and offsets come from the argument segment) -- all in flight together
    const int8_t* qrow = p.q + (size_t)min(r, M - 1) * p.cols;
    Operand<F> av[GPW];
#pragma unroll
    for (int c = 0; c < GPW; c++) av[c] = load_operand<F>(qrow, r < M, min(g_first + c, G - 1), kq);
    uint16_t hraw[GPW];
#pragma unroll
    for (int c = 0; c < GPW; c++) hraw[c] = nrow[min(g_first + c, G - 1)];
    u4 w[CB];
#pragma unroll
    for (int c = 0; c < CB; c++)
        w[c] = __builtin_nontemporal_load(wbase + (size_t)min(wave * CB + c, p.blocks - 1) * 64);
    float sc[GPW][4], of[GPW][4];
#pragma unroll
    for (int c = 0; c < GPW; c++) {
        const int g = min(g_first + c, G - 1);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const size_t at = (size_t)min(4 * kq + i, M - 1) * p.stride + g;
            sc[c][i] = p.qscale[at];
            of[c][i] = p.offsets[at];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    MATMUL_TAIL_FIELDS(p);

    const int tq = 4 * kq;  // first token of this lane's MFMA results
#pragma unroll
    for (int c4 = 0; c4 < GPW / 4; c4++) {
        float ra[4][4], rb[4][4];  // [token i][group j of the column]
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int gl = 4 * c4 + j;
            const v4i d = group_dot<F, true>(w[gl / T::GPB], gl % T::GPB, av[gl], p);
            const float hs = EXACT ? ref_half_to_single(hraw[gl]) : decode_scale_fast(hraw[gl]);
            const float hb = hs * p.byte_scale;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float scaled = hb * sc[gl][i];
                ra[i][j] = scaled * static_cast<float>(d[i]);
                rb[i][j] = scaled * of[gl][i];
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int x = (tq + i) * 16 + r;  // product row
            if (tq + i < M) {
                const int col = ((g_first >> 2) + c4) ^ (x & p.swz);
                pa[(size_t)x * (GS / 4) + col] = make_float4(ra[i][0], ra[i][1], ra[i][2], ra[i][3]);
                pb[(size_t)x * (GS / 4) + col] = make_float4(rb[i][0], rb[i][1], rb[i][2], rb[i][3]);
            }
        }
    }
    __syncthreads();
    for (int x = threadIdx.x; x < M * 16; x += blockDim.x) {
        const int nn = tile * 16 + (x & 15);
        const float4* row_a = pa + (size_t)x * (GS / 4);
        const float4* row_b = pb + (size_t)x * (GS / 4);
        const int sw = x & p.swz;
        float acc = 0.0f, bias = 0.0f;
        int c = 0;
        for (; c + 4 <= (G >> 2); c += 4) {  // 16 groups per batch, reads first
            float4 a[4], b[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                a[j] = row_a[(c + j) ^ sw];
                b[j] = row_b[(c + j) ^ sw];
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc = acc + a[j].x;
                bias = bias + b[j].x;
                acc = acc + a[j].y;
                bias = bias + b[j].y;
                acc = acc + a[j].z;
                bias = bias + b[j].z;
                acc = acc + a[j].w;
                bias = bias + b[j].w;
            }
        }
        for (; c < (G >> 2); c++) {
            const float4 a = row_a[c ^ sw];
            const float4 b = row_b[c ^ sw];
            acc = acc + a.x;
            bias = bias + b.x;
            acc = acc + a.y;
            bias = bias + b.y;
            acc = acc + a.z;
            bias = bias + b.z;
            acc = acc + a.w;
            bias = bias + b.w;
        }
        if (G & 3) {
            const float4 a = row_a[(G >> 2) ^ sw];
            const float4 b = row_b[(G >> 2) ^ sw];
            const float av4[4] = {a.x, a.y, a.z, a.w}, bv4[4] = {b.x, b.y, b.z, b.w};
            for (int j = 0; j < (G & 3); j++) {
                acc = acc + av4[j];
                bias = bias + bv4[j];
            }
        }
        if constexpr (SPLIT)
            store_row(p, x >> 4, nn, acc - bias);
        else if (nn >= p.row_start && nn < p.row_end)
            p.y[(size_t)(x >> 4) * p.ldy + nn] = acc - bias;
    }
}

// SPLIT: the split outputs (MatmulParams::split_n), for stacked matrices.
template <int F, int GPW, bool EXACT, bool WIDE, bool SPLIT = false>
__global__ __launch_bounds__(512) void matmul_cq_decode_kernel(MATMUL_HEAD_PARAMS, MatmulParams p)
{
    MATMUL_TAKE_HEAD(p);
    if constexpr (WIDE)
        cq_decode_wide_tile<F, GPW, EXACT, SPLIT>(p, p.tile_begin + blockIdx.x);
    else
        cq_decode_tile<F, GPW, EXACT, SPLIT>(p, p.tile_begin + blockIdx.x);
}

template <int F, int GPW, bool EXACT, bool WIDE>
__global__ __launch_bounds__(512) void matmul_cq_decode_batch_kernel(MatmulBatch b)
{
    const int j = batch_job(b);
    const MatmulParams& p = b.job[j];
    if constexpr (WIDE)
        cq_decode_wide_tile<F, GPW, EXACT, false>(p, p.tile_begin + (int)blockIdx.x - b.first[j]);
    else
        cq_decode_tile<F, GPW, EXACT, false>(p, p.tile_begin + (int)blockIdx.x - b.first[j]);
}

// The decode kernel for M <= 4 with its activation rows computed in the
// prologue from fp32 inputs instead of read as int8 (one launch instead of
// an element-wise kernel and a matmul).  Every workgroup loads the inputs
// first, then its scales and weight blocks, and computes the M = TI
// quantized rows (all K) into LDS while the weights are in flight; the rows
// are bit-identical with the element-wise kernels they replace:
//   kProNorm    x (+ delta) -> RMSNorm (canonical row sum of squares) *
//               gain -> QuantizeInt8; workgroup 0 also writes x + delta to
//               x_out;
//   kProQuant   QuantizeInt8 of x.
// With p.residual the chain stores residual + y (the residual stream's
// update, x + delta in Engine's order of operands: one IEEE addition, so the
// same bits) instead of y.
// Thread t of the prologue holds the float4 groups at 4t + 4*nt*j, j < G4
// (nt = 256 for the norm, whose lanes are the canonical sum's, else the
// whole block).  Every prologue load is unconditional, so the weight loads
// stay in flight across the prologue.  The first loads' arguments come
// preloaded (the head: x, delta, gain, tiles, norms, (waves, K), (G,
// blocks)); tile_begin is 0 (every row).
template <int CB, int KIND, bool DELTA, int G4, int TI>
__global__ __launch_bounds__(512) void matmul_i8_decode_fused_kernel(const float* h_x, const float* h_delta,
                                                                     const float* h_gain, const uint8_t* h_tiles,
                                                                     const uint16_t* h_norms, uint64_t h_waves_cols,
                                                                     uint64_t h_groups_blocks, MatmulParams p,
                                                                     DecodePrologue f)
{
    f.x = h_x;
    f.delta = h_delta;
    f.gain = h_gain;
    p.tiles = h_tiles;
    p.norms = h_norms;
    p.tokens = TI;
    p.cols = head_hi(h_waves_cols);
    p.groups = head_lo(h_groups_blocks);
    p.blocks = head_hi(h_groups_blocks);
    constexpr int SETS = 2 * CB / 4;
    extern __shared__ __align__(16) uint8_t lds[];
    float* pl = reinterpret_cast<float*>(lds);                            // products [t][r][GS]
    int8_t* qa = reinterpret_cast<int8_t*>(lds + p.d_bytes);              // quantized rows [TI][K]
    float* red = reinterpret_cast<float*>(lds + p.d_bytes + p.st_bytes);  // [TI][256] partial sums
    float* sums = red + TI * 256;                                         // [TI]
    float* wmax = sums + TI;                                              // [TI][8]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nwaves = head_lo(h_waves_cols);
    const int tile = blockIdx.x;
    constexpr int M = TI;
    const int K = p.cols;
    const int G = p.groups;
    const int GS = p.ldd;
    const int r = lane & 15;
    const int kq = lane >> 4;
    const int n = tile * 16 + r;
    const bool active = wave * CB < p.blocks;  // waves past the tile's blocks only run the prologue
    const int mb0 = active ? wave * CB : 0;
    const int g_first = mb0 * 2;
    const u4* wbase = reinterpret_cast<const u4*>(p.tiles) + (size_t)tile * p.blocks * 64 + lane;
    const uint16_t* nrow = p.norms + (size_t)n * ((G + 7) & ~7) + g_first;
    constexpr bool NORM = KIND == kProNorm;
    const int nt = NORM ? 256 : 64 * nwaves;

    // 1. prologue inputs
    float4 xv[TI][G4], dv[TI][G4], gv[G4];  // dv: the delta of the norm
#pragma unroll
    for (int j = 0; j < G4; j++) {
        const int i = min(4 * (tid + nt * j), K - 4);
        if constexpr (NORM) gv[j] = *reinterpret_cast<const float4*>(f.gain + i);
#pragma unroll
        for (int t = 0; t < TI; t++) {
            const size_t row = (size_t)min(t, M - 1);
            xv[t][j] = *reinterpret_cast<const float4*>(f.x + row * K + i);
            if constexpr (DELTA) dv[t][j] = *reinterpret_cast<const float4*>(f.delta + row * K + i);
        }
    }
    // 2. weight scales, 3. weight blocks
    uint16_t hraw[SETS];
#pragma unroll
    for (int c = 0; c < SETS; c++) hraw[c] = nrow[4 * c + kq];
    u4 w[CB];
#pragma unroll
    for (int c = 0; c < CB; c++) w[c] = __builtin_nontemporal_load(wbase + (size_t)(mb0 + c) * 64);
    // 4. the residual value of chain lane (t, r) = (tid / 16, tid % 16)
    float res = 0.0f;
    if (p.residual)
        res = p.residual[(size_t)min(tid >> 4, M - 1) * p.ldy + min(tile * 16 + (tid & 15), p.row_end - 1)];
    __builtin_amdgcn_sched_barrier(0);
    MATMUL_TAIL_FIELDS(p);
    asm volatile("" ::"s"(f.eps), "s"(f.x_out), "s"(p.d_bytes), "s"(p.st_bytes));

    // 5. the quantized rows, while the weights arrive
    float peak[TI];
#pragma unroll
    for (int t = 0; t < TI; t++) peak[t] = 0.0f;
    if constexpr (NORM) {
        const bool pt = tid < 256;
#pragma unroll
        for (int t = 0; t < TI; t++) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < G4; j++) {
                if (pt && 4 * (tid + 256 * j) < K) {
                    float4 v = xv[t][j];
                    if constexpr (DELTA) v = make_float4(v.x + dv[t][j].x, v.y + dv[t][j].y, v.z + dv[t][j].z, v.w + dv[t][j].w);
                    xv[t][j] = v;
                    s = s + v.x * v.x;
                    s = s + v.y * v.y;
                    s = s + v.z * v.z;
                    s = s + v.w * v.w;
                }
            }
            if (pt) red[t * 256 + tid] = s;
        }
        __syncthreads();
        if (wave < TI) {
            const float total = canonical_finish(red + wave * 256, lane);
            if (lane == 0) sums[wave] = total;
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < TI; t++) {
            const float inv = 1.0f / sqrtf(sums[t] / (float)K + f.eps);
#pragma unroll
            for (int j = 0; j < G4; j++) {
                const int i = 4 * (tid + 256 * j);
                if (pt && i < K) {
                    if (DELTA && f.x_out && blockIdx.x == 0 && t < M)
                        *reinterpret_cast<float4*>(f.x_out + (size_t)t * K + i) = xv[t][j];
                    const float4 v = xv[t][j];
                    xv[t][j] = make_float4((v.x * inv) * gv[j].x, (v.y * inv) * gv[j].y, (v.z * inv) * gv[j].z,
                                           (v.w * inv) * gv[j].w);
                    peak[t] = fmaxf(fmaxf(peak[t], fmaxf(fabsf(xv[t][j].x), fabsf(xv[t][j].y))),
                                    fmaxf(fabsf(xv[t][j].z), fabsf(xv[t][j].w)));
                }
            }
        }
    } else {
#pragma unroll
        for (int t = 0; t < TI; t++) {
#pragma unroll
            for (int j = 0; j < G4; j++) {
                if (4 * (tid + nt * j) < K) {
                    peak[t] = fmaxf(fmaxf(peak[t], fmaxf(fabsf(xv[t][j].x), fabsf(xv[t][j].y))),
                                    fmaxf(fabsf(xv[t][j].z), fabsf(xv[t][j].w)));
                }
            }
        }
    }
    // block max per row (order-free)
#pragma unroll
    for (int t = 0; t < TI; t++) {
        const float v = wave_max(peak[t]);
        if (lane == 0) wmax[t * 8 + wave] = v;
    }
    __syncthreads();
    float qs[TI];
#pragma unroll
    for (int t = 0; t < TI; t++) {
        float pk = wmax[t * 8];
        for (int wv = 1; wv < nwaves; wv++) pk = fmaxf(pk, wmax[t * 8 + wv]);
        const float scale = pk > 0.0f ? pk / 127.0f : 1.0f;
        const float inverse = 1.0f / scale;
        qs[t] = scale;
#pragma unroll
        for (int j = 0; j < G4; j++) {
            const int i = 4 * (tid + nt * j);
            if (tid < nt && i < K) {
                *reinterpret_cast<uint32_t*>(qa + (size_t)t * K + i) = ref_quantize4(xv[t][j], inverse);
            }
        }
    }
    __syncthreads();
    // 6. A operands from the quantized rows (token r%4, group g + r/4, k-slice kq)
    if (active) {
        long av[SETS];
        const bool feeds = (r & 3) < M;
#pragma unroll
        for (int c = 0; c < SETS; c++) {
            const int g = min(g_first + 4 * c + (r >> 2), G - 1);
            const long a = *reinterpret_cast<const long*>(qa + (size_t)min(r & 3, M - 1) * K + g * 32 + kq * 8);
            av[c] = feeds ? a : 0;
        }
        narrow_products<CB, TI, false>(av, qs, hraw, w, pl, GS, M, g_first, r, kq);
    }
    __syncthreads();
    chain_products(pl, GS, 0, M, G, tile, p, res);
}

template <int CB, int TI, bool EXACT>
int32_t launch_dec_tpl(const MatmulParams& p, int waves, size_t lds, hipStream_t stream)
{
    const int tiles = p.tile_end - p.tile_begin;
    hipLaunchKernelGGL((matmul_i8_decode_kernel<CB, TI, EXACT>), dim3(tiles), dim3(64 * waves), lds, stream,
                       MATMUL_HEAD_ARGS(p), p);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

template <int CB, bool EXACT>
int32_t launch_dec_ti(const MatmulParams& p, int waves, size_t lds, hipStream_t s)
{
    switch (p.tokens) {
        case 1: return launch_dec_tpl<CB, 1, EXACT>(p, waves, lds, s);
        case 2: return launch_dec_tpl<CB, 2, EXACT>(p, waves, lds, s);
        case 3: return launch_dec_tpl<CB, 3, EXACT>(p, waves, lds, s);
        case 4: return launch_dec_tpl<CB, 4, EXACT>(p, waves, lds, s);
        default: return launch_dec_tpl<CB, 16, EXACT>(p, waves, lds, s);
    }
}

// The int8 decode kernel's launch shape for these weights and p.tokens:
// sets p.ldd and p.swz, the waves per tile and the LDS bytes; false when the
// kernel does not apply (the caller falls back to the general kernel).
bool plan_i8_decode(const DeviceWeights* w, MatmulParams& p, int* waves_out, size_t* lds_out)
{
    if (p.tokens > 16 || p.dots) return false;
    static const int waves_override = [] {
        // tuning knob: 2, 4 or 8 waves per tile, or 1 to use the general kernel
        const char* e = getenv("NHIP_DECODE_WAVES");
        const int v = e ? atoi(e) : 0;
        return (v == 1 || v == 2 || v == 4 || v == 8) ? v : 0;
    }();
    if (waves_override == 1) return false;
    int waves = 0;
    // 5..16 tokens: more waves split the larger per-tile product work
    const int cands[3] = {p.tokens > 4 ? 8 : 4, p.tokens > 4 ? 4 : 8, 2};
    for (int c : cands) {
        if (waves_override && c != waves_override) continue;
        if (w->blocks % c == 0 && (w->blocks / c == 4 || w->blocks / c == 8)) {
            waves = c;
            break;
        }
    }
    if (!waves) return false;
    const int m = p.tokens;
    size_t lds;
    if (m <= 4) {
        p.ldd = ((2 * w->blocks + 3) & ~3) + 4;  // product row stride: every group a wave writes
        p.swz = 0;
    } else {
        // the swizzle mask is the largest power of two (<= 16) dividing the
        // float4 columns, less 1
        p.ldd = (2 * w->blocks + 3) & ~3;
        const int cols4 = p.ldd / 4;
        p.swz = std::min(cols4 & -cols4, 16) - 1;
    }
    lds = (size_t)m * 16 * p.ldd * sizeof(float);
    if (lds > kMaxLds) return false;
    *waves_out = waves;
    *lds_out = lds;
    return true;
}

// Runs the decode kernel when its preconditions hold; returns 1 when it did
// not apply (the caller falls back to the general kernel).
int32_t try_i8_decode(const DeviceWeights* w, MatmulParams& p, hipStream_t stream)
{
    int waves = 0;
    size_t lds = 0;
    if (!plan_i8_decode(w, p, &waves, &lds)) return 1;
    // the kernel's CB must equal the blocks per wave (4 or 8)
    if (w->blocks / waves == 4)
        return w->special_scales ? launch_dec_ti<4, true>(p, waves, lds, stream)
                                 : launch_dec_ti<4, false>(p, waves, lds, stream);
    return w->special_scales ? launch_dec_ti<8, true>(p, waves, lds, stream)
                             : launch_dec_ti<8, false>(p, waves, lds, stream);
}

template <int F, int GPW, bool WIDE>
void launch_cq_decode_w(const MatmulParams& p, bool exact, int waves, size_t lds, hipStream_t stream)
{
    const int tiles = p.tile_end - p.tile_begin;
    // split launches: 1..4 tokens, never exact (matmul_cq_split_internal)
    if constexpr (!WIDE) {
        if (p.split_n) {
            hipLaunchKernelGGL((matmul_cq_decode_kernel<F, GPW, false, false, true>), dim3(tiles), dim3(64 * waves),
                               lds, stream, MATMUL_HEAD_ARGS(p), p);
            return;
        }
    }
    if (exact)
        hipLaunchKernelGGL((matmul_cq_decode_kernel<F, GPW, true, WIDE>), dim3(tiles), dim3(64 * waves), lds, stream,
                           MATMUL_HEAD_ARGS(p), p);
    else
        hipLaunchKernelGGL((matmul_cq_decode_kernel<F, GPW, false, WIDE>), dim3(tiles), dim3(64 * waves), lds, stream,
                           MATMUL_HEAD_ARGS(p), p);
}

template <int F, int GPW>
int32_t launch_cq_decode_tpl(const MatmulParams& p, bool exact, int waves, size_t lds, hipStream_t stream)
{
    if constexpr (GPW <= 8) {  // the planner takes 5..16 tokens only up to 8 groups per wave
        if (p.tokens > 4) {
            launch_cq_decode_w<F, GPW, true>(p, exact, waves, lds, stream);
            NHIP_CHECK_HIP(hipGetLastError());
            return NHIP_OK;
        }
    }
    launch_cq_decode_w<F, GPW, false>(p, exact, waves, lds, stream);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

template <int F>
int32_t launch_cq_decode_gpw(const MatmulParams& p, int gpw, bool exact, int waves, size_t lds, hipStream_t s)
{
    switch (gpw) {
        case 4: return launch_cq_decode_tpl<F, 4>(p, exact, waves, lds, s);
        case 8: return launch_cq_decode_tpl<F, 8>(p, exact, waves, lds, s);
        default: return launch_cq_decode_tpl<F, 16>(p, exact, waves, lds, s);
    }
}

// Codebook formats, 1..16 tokens: runs matmul_cq_decode_kernel (the
// four-group sets for up to 4 tokens, one group per MFMA set for 5..16) with
// GPW groups per wave (4 by default, more when that would take over 8
// waves; NHIP_CQ_DECODE_GPW = 4, 8 or 16 overrides it for tuning) and one
// wave per GPW groups.  Returns false when it does not apply (more than 16
// tokens, group sums requested, K over 16*8 groups, products over 64 KB of
// LDS, or 5..16 tokens over more than 256 row tiles).
bool plan_cq_decode(const DeviceWeights* w, MatmulParams& p, int* gpw_out, int* waves_out, size_t* lds_out)
{
    if (p.tokens > 16 || p.dots) return false;
    static const int gpw_override = [] {
        const char* e = getenv("NHIP_CQ_DECODE_GPW");
        const int v = e ? atoi(e) : 0;
        return (v == 4 || v == 8 || v == 16) ? v : 0;
    }();
    int gpw = gpw_override ? gpw_override : 4;
    while (gpw < 16 && (w->groups + gpw - 1) / gpw > 8) gpw *= 2;
    const int waves = (w->groups + gpw - 1) / gpw;
    if (waves > 8 || (p.tokens > 4 && gpw > 8)) return false;
    // 5..16 tokens over more than 256 tiles measured faster on the general kernel
    // (Cq4 16 x 2048 x 8192: 6.46 against 5.71 us), fewer faster here (Cq2
    // 16 x 768 x 2560: 4.13 against 7.10 us)
    if (p.tokens > 4 && p.tile_end - p.tile_begin > 256) return false;
    if (p.tokens <= 4) {
        p.ldd = waves * gpw + 4;  // every group a wave writes, + 4: conflict-free product writes
        p.swz = 0;
    } else {
        // every group a wave writes, in float4 columns swizzled within the
        // largest power-of-two block (<= 16) that divides them
        p.ldd = waves * gpw;
        const int cols4 = p.ldd / 4;
        p.swz = std::min(cols4 & -cols4, 16) - 1;
    }
    const size_t lds = (size_t)2 * p.tokens * 16 * p.ldd * sizeof(float);
    if (lds > kMaxLds) return false;
    *gpw_out = gpw;
    *waves_out = waves;
    *lds_out = lds;
    return true;
}

int32_t try_cq_decode(const DeviceWeights* w, MatmulParams& p, hipStream_t stream)
{
    int gpw = 0, waves = 0;
    size_t lds = 0;
    if (!plan_cq_decode(w, p, &gpw, &waves, &lds)) return 1;
    const bool cq4 = w->format == WeightFormat::Cq4;
    const bool exact = w->special_scales != 0;
    return cq4 ? launch_cq_decode_gpw<kCq4>(p, gpw, exact, waves, lds, stream)
               : launch_cq_decode_gpw<kCq2>(p, gpw, exact, waves, lds, stream);
}

template <int CB, int KIND, bool DELTA, int G4, int TI>
int32_t launch_fused_ti(const MatmulParams& p, const DecodePrologue& f, int waves, size_t lds, hipStream_t stream)
{
    const int tiles = p.tile_end - p.tile_begin;
    hipLaunchKernelGGL((matmul_i8_decode_fused_kernel<CB, KIND, DELTA, G4, TI>), dim3(tiles), dim3(64 * waves), lds,
                       stream, f.x, f.delta, f.gain, p.tiles, p.norms, head_pair(waves, p.cols),
                       head_pair(p.groups, p.blocks), p, f);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

template <int CB, int KIND, bool DELTA, int G4>
int32_t launch_fused_tpl(const MatmulParams& p, const DecodePrologue& f, int waves, size_t lds, hipStream_t s)
{
    switch (p.tokens) {
        case 1: return launch_fused_ti<CB, KIND, DELTA, G4, 1>(p, f, waves, lds, s);
        case 2: return launch_fused_ti<CB, KIND, DELTA, G4, 2>(p, f, waves, lds, s);
        case 3: return launch_fused_ti<CB, KIND, DELTA, G4, 3>(p, f, waves, lds, s);
        default: return launch_fused_ti<CB, KIND, DELTA, G4, 4>(p, f, waves, lds, s);
    }
}

template <int CB, int G4>
int32_t launch_fused_kind(const MatmulParams& p, const DecodePrologue& f, int waves, size_t lds, hipStream_t s)
{
    switch (f.kind) {
        case kProNorm:
            return f.delta ? launch_fused_tpl<CB, kProNorm, true, G4>(p, f, waves, lds, s)
                           : launch_fused_tpl<CB, kProNorm, false, G4>(p, f, waves, lds, s);
        default: return launch_fused_tpl<CB, kProQuant, false, G4>(p, f, waves, lds, s);
    }
}

template <int CB>
int32_t launch_fused_g4(const MatmulParams& p, const DecodePrologue& f, int waves, int g4, size_t lds, hipStream_t s)
{
    return g4 == 1 ? launch_fused_kind<CB, 1>(p, f, waves, lds, s) : launch_fused_kind<CB, 2>(p, f, waves, lds, s);
}

template <int CB, int NS, bool DOTS>
int32_t launch_i8_tpl(const MatmulParams& p, int waves, size_t lds_bytes, hipStream_t stream)
{
    const int tiles = p.tile_end - p.tile_begin;
    dim3 grid(tiles, (p.tokens + 15) / 16);
    hipLaunchKernelGGL((matmul_i8_kernel<CB, NS, DOTS>), grid, dim3(64 * waves), lds_bytes, stream, p);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

template <int CB, bool DOTS>
int32_t launch_i8_ns(const MatmulParams& p, int waves, int ns, size_t lds, hipStream_t s)
{
    if (ns <= 1) return launch_i8_tpl<CB, 1, DOTS>(p, waves, lds, s);
    if (ns <= 2) return launch_i8_tpl<CB, 2, DOTS>(p, waves, lds, s);
    if (ns <= 4) return launch_i8_tpl<CB, 4, DOTS>(p, waves, lds, s);
    return launch_i8_tpl<CB, 8, DOTS>(p, waves, lds, s);
}

template <bool DOTS>
int32_t launch_i8(const MatmulParams& p, int waves, int ns, size_t lds, hipStream_t s)
{
    const int per = ((p.gph + 1) / 2 + waves - 1) / waves;
    if (per <= 2) return launch_i8_ns<2, DOTS>(p, waves, ns, lds, s);
    if (per <= 4) return launch_i8_ns<4, DOTS>(p, waves, ns, lds, s);
    return launch_i8_ns<8, DOTS>(p, waves, ns, lds, s);
}

template <int F, int CB, bool DOTS>
int32_t launch_tpl(const MatmulParams& p, int waves, size_t lds_bytes, hipStream_t stream)
{
    auto kernel = matmul_kernel<F, CB, DOTS>;
    const int tiles = p.tile_end - p.tile_begin;
    dim3 grid(tiles, (p.tokens + 15) / 16);
    hipLaunchKernelGGL(kernel, grid, dim3(64 * waves), lds_bytes, stream, p);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

template <int F, bool DOTS>
int32_t launch_fmt(const MatmulParams& p, int waves, size_t lds, hipStream_t s)
{
    using T = Traits<F>;
    const int per = ((p.gph + T::GPB - 1) / T::GPB + waves - 1) / waves;
    if (per <= 2) return launch_tpl<F, 2, DOTS>(p, waves, lds, s);
    if (per <= 4) return launch_tpl<F, 4, DOTS>(p, waves, lds, s);
    return launch_tpl<F, 8, DOTS>(p, waves, lds, s);
}


MatmulParams matmul_params(const DeviceWeights* w, const int8_t* q, const float* scales, const float* offsets,
                           int32_t stride, int32_t tokens, float* y, int32_t ldy, int32_t row_start, int32_t row_end,
                           int32_t* dots)
{
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
    p.x0 = w->split_table[0];
    p.x1 = w->split_table[1];
    p.x2 = w->split_table[2];
    p.x3 = w->split_table[3];
    p.byte_scale = w->byte_scale;
    return p;
}

// Waves per 16-row tile of the general kernels (each loads 1/waves of the
// tile's weight blocks) for `tiles` row tiles; NHIP_MATMUL_WAVES (4 or 8)
// overrides the default for tuning.
int general_waves(int tiles, int tokens)
{
    static const int waves_override = [] {
        const char* e = getenv("NHIP_MATMUL_WAVES");
        const int v = e ? atoi(e) : 0;
        return (v == 4 || v == 8) ? v : 0;
    }();
    return waves_override ? waves_override : (tiles * ((tokens + 15) / 16) >= 512 ? 4 : 8);
}

// Codebook formats, general kernel.  Groups per phase: the int32 D buffer
// [gph][M][16] plus the decoded scales [gph][16] stay within 64 KB of LDS,
// and no wave holds more than 8 weight blocks.  False (and the bytes needed
// in *lds) when it does not fit.
bool plan_general_cq(const DeviceWeights* w, MatmulParams& p, int waves, size_t* lds)
{
    const int m = std::min(16, p.tokens);
    const int gpb = w->format == WeightFormat::Cq4 ? 1 : 2;
    int gph = std::min(std::min(w->groups, 1024 / (m + 1) - 12), 8 * waves * gpb);
    gph -= gph % gpb;
    if (gph < gpb) gph = gpb;
    p.gph = gph;
    p.ldd = ((gph + 3) & ~3) + 4;
    p.d_bytes = m * 16 * p.ldd * 4;
    *lds = (size_t)p.d_bytes + (size_t)16 * p.ldd * 4 + 64 * 4;
    return *lds <= kMaxLds;
}

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

    MatmulParams p = matmul_params(w, q, scales, offsets, stride, tokens, y, ldy, row_start, row_end, dots);

    const int tiles = p.tile_end - p.tile_begin;
    const int waves = general_waves(tiles, tokens);
    const int m = std::min(16, tokens);
    if (w->format == WeightFormat::Int8G32) {
        if (!dots && tokens >= kGemmMinTokens)
            return launch_gemm_i8(w, q, scales, tokens, y, ldy, row_start, row_end, true, stream);
        if (!dots) {
            const int32_t nrc = launch_i8_narrow(w, 0, q, nullptr, nullptr, scales, 0.0f, nullptr, tokens, y, ldy,
                                                 row_start, row_end, stream);
            if (nrc <= 0) return nrc;
        }
        const int32_t drc = try_i8_decode(w, p, stream);
        if (drc <= 0) return drc;
        // LDS per phase: staged operands gph*32*m + products m*16*ldd*4 + a
        // 1 KB sink, within 64 KB; no wave holds more than 8 weight blocks.
        int gph = std::min(w->groups, 16 * waves);
        auto need = [&](int g) {
            const int ldd = ((g + 3) & ~3) + 4;
            return (size_t)g * 32 * m + (size_t)m * 16 * ldd * 4 + 1024;
        };
        while (gph > 2 && need(gph) > kMaxLds) gph -= 2;
        if (gph > 1 && gph % 2) gph -= 1;
        p.gph = gph;
        p.ldd = ((gph + 3) & ~3) + 4;
        p.st_bytes = (gph * 32 * m + 15) & ~15;
        p.d_bytes = m * 16 * p.ldd * 4;
        const size_t lds = need(gph);
        const int ns = (m * gph * 2 + 64 * waves - 1) / (64 * waves);
        if (lds > kMaxLds || ns > 8) {
            set_error("matmul needs %zu bytes of LDS (max %zu)", lds, kMaxLds);
            return NHIP_ERR_UNSUPPORTED;
        }
        return dots ? launch_i8<true>(p, waves, ns, lds, stream) : launch_i8<false>(p, waves, ns, lds, stream);
    }
    {
        const int32_t drc = try_cq_decode(w, p, stream);
        if (drc <= 0) return drc;
    }
    size_t lds = 0;
    if (!plan_general_cq(w, p, waves, &lds)) {
        set_error("matmul needs %zu bytes of LDS (max %zu)", lds, kMaxLds);
        return NHIP_ERR_UNSUPPORTED;
    }
    switch (w->format) {
        case WeightFormat::Int8G32:
            break;
        case WeightFormat::Cq2:
            return dots ? launch_fmt<kCq2, true>(p, waves, lds, stream) : launch_fmt<kCq2, false>(p, waves, lds, stream);
        case WeightFormat::Cq4:
            return dots ? launch_fmt<kCq4, true>(p, waves, lds, stream) : launch_fmt<kCq4, false>(p, waves, lds, stream);
    }
    return NHIP_ERR_ARG;
}

// ------------------------------------------------------ batched matmuls --

template <int CB, int TI, bool EXACT>
int32_t launch_dec_batch_tpl(const MatmulBatch& b, int waves, size_t lds, hipStream_t s)
{
    hipLaunchKernelGGL((matmul_i8_decode_batch_kernel<CB, TI, EXACT>), dim3(b.first[b.count]), dim3(64 * waves), lds,
                       s, b);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

template <int CB, bool EXACT>
int32_t launch_dec_batch_ti(const MatmulBatch& b, int waves, size_t lds, hipStream_t s)
{
    switch (b.job[0].tokens) {
        case 1: return launch_dec_batch_tpl<CB, 1, EXACT>(b, waves, lds, s);
        case 2: return launch_dec_batch_tpl<CB, 2, EXACT>(b, waves, lds, s);
        case 3: return launch_dec_batch_tpl<CB, 3, EXACT>(b, waves, lds, s);
        case 4: return launch_dec_batch_tpl<CB, 4, EXACT>(b, waves, lds, s);
        default: return launch_dec_batch_tpl<CB, 16, EXACT>(b, waves, lds, s);
    }
}

template <int F, int GPW, bool WIDE>
void launch_cq_batch_w(const MatmulBatch& b, bool exact, int waves, size_t lds, hipStream_t s)
{
    if (exact)
        hipLaunchKernelGGL((matmul_cq_decode_batch_kernel<F, GPW, true, WIDE>), dim3(b.first[b.count]),
                           dim3(64 * waves), lds, s, b);
    else
        hipLaunchKernelGGL((matmul_cq_decode_batch_kernel<F, GPW, false, WIDE>), dim3(b.first[b.count]),
                           dim3(64 * waves), lds, s, b);
}

template <int F, int GPW>
int32_t launch_cq_batch_tpl(const MatmulBatch& b, bool exact, int waves, size_t lds, hipStream_t s)
{
    if constexpr (GPW <= 8) {
        if (b.job[0].tokens > 4) {
            launch_cq_batch_w<F, GPW, true>(b, exact, waves, lds, s);
            NHIP_CHECK_HIP(hipGetLastError());
            return NHIP_OK;
        }
    }
    launch_cq_batch_w<F, GPW, false>(b, exact, waves, lds, s);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

template <int F>
int32_t launch_cq_batch_gpw(const MatmulBatch& b, int gpw, bool exact, int waves, size_t lds, hipStream_t s)
{
    switch (gpw) {
        case 4: return launch_cq_batch_tpl<F, 4>(b, exact, waves, lds, s);
        case 8: return launch_cq_batch_tpl<F, 8>(b, exact, waves, lds, s);
        default: return launch_cq_batch_tpl<F, 16>(b, exact, waves, lds, s);
    }
}

template <int F, int CB>
int32_t launch_gen_batch(const MatmulBatch& b, int waves, size_t lds, hipStream_t s)
{
    hipLaunchKernelGGL((matmul_batch_kernel<F, CB>), dim3(b.first[b.count], (b.job[0].tokens + 15) / 16),
                       dim3(64 * waves), lds, s, b);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

template <int F>
int32_t launch_gen_batch_fmt(const MatmulBatch& b, int per, int waves, size_t lds, hipStream_t s)
{
    if (per <= 2) return launch_gen_batch<F, 2>(b, waves, lds, s);
    if (per <= 4) return launch_gen_batch<F, 4>(b, waves, lds, s);
    return launch_gen_batch<F, 8>(b, waves, lds, s);
}

// Quant.MatMulBatch.Run (src/Needle/Quant.cs:697-706, 753-772): every job's
// MatMulRows over all its rows with the shared activations.  The decode
// sizes (up to 16 tokens), and the codebook formats at any token count (the
// general kernel), run as one launch over the row tiles of every job; the
// literal format past 16 tokens runs the jobs one after another (the same
// kernels as nhip_matmul_*_dev, so the same bits either way).
int32_t run_matmul_batch(const DeviceWeights* const* w, int32_t count, const int8_t* q, const float* scales,
                         const float* offsets, int32_t stride, int32_t tokens, float* const* y, const int32_t* ldy,
                         hipStream_t stream)
{
    NHIP_REQUIRE(w && y && ldy && count >= 1 && count <= kMaxBatchJobs, "batch of %d jobs outside [1, %d]", count,
                 kMaxBatchJobs);
    NHIP_REQUIRE(tokens >= 0, "tokens %d < 0", tokens);
    for (int j = 0; j < count; j++) {
        NHIP_REQUIRE(w[j] && y[j], "job %d: null weights or output", j);
        NHIP_REQUIRE(w[j]->format == w[0]->format && w[j]->cols == w[0]->cols,
                     "job %d: every job needs the format and K of job 0", j);
        NHIP_REQUIRE(ldy[j] >= w[j]->rows, "job %d: ldy %d below its %d rows", j, ldy[j], w[j]->rows);
    }
    if (tokens == 0) return NHIP_OK;
    NHIP_REQUIRE(q && scales, "activations are NULL");
    const bool cq = w[0]->format != WeightFormat::Int8G32;
    if (cq) NHIP_REQUIRE(offsets && stride >= w[0]->groups, "offsets NULL or stride %d < groups %d", stride, w[0]->groups);
    int32_t rc = ensure_device();
    if (rc) return rc;
    MatmulBatch b{};
    b.count = count;
    bool exact = false;
    for (int j = 0; j < count; j++) {
        b.job[j] = matmul_params(w[j], q, scales, offsets, stride, tokens, y[j], ldy[j], 0, w[j]->rows, nullptr);
        b.first[j + 1] = b.first[j] + (b.job[j].tile_end - b.job[j].tile_begin);
        exact = exact || w[j]->special_scales;
    }
    int waves = 0, gpw = 0;
    size_t lds = 0;
    bool planned = true;
    for (int j = 0; j < count && planned; j++)  // the same shape for every job (same K and tokens)
        planned = cq ? plan_cq_decode(w[j], b.job[j], &gpw, &waves, &lds) : plan_i8_decode(w[j], b.job[j], &waves, &lds);
    if (planned) {
        if (!cq)
            return w[0]->blocks / waves == 4 ? (exact ? launch_dec_batch_ti<4, true>(b, waves, lds, stream)
                                                      : launch_dec_batch_ti<4, false>(b, waves, lds, stream))
                                             : (exact ? launch_dec_batch_ti<8, true>(b, waves, lds, stream)
                                                      : launch_dec_batch_ti<8, false>(b, waves, lds, stream));
        return w[0]->format == WeightFormat::Cq4 ? launch_cq_batch_gpw<kCq4>(b, gpw, exact, waves, lds, stream)
                                                 : launch_cq_batch_gpw<kCq2>(b, gpw, exact, waves, lds, stream);
    }
    if (cq) {  // the general kernel over every job's tiles, one launch
        const int waves2 = general_waves(b.first[count], tokens);
        size_t lds2 = 0;
        bool fits = true;
        for (int j = 0; j < count && fits; j++) fits = plan_general_cq(w[j], b.job[j], waves2, &lds2);
        if (fits) {
            const int gpb = w[0]->format == WeightFormat::Cq4 ? 1 : 2;
            const int per = ((b.job[0].gph + gpb - 1) / gpb + waves2 - 1) / waves2;
            return w[0]->format == WeightFormat::Cq4 ? launch_gen_batch_fmt<kCq4>(b, per, waves2, lds2, stream)
                                                     : launch_gen_batch_fmt<kCq2>(b, per, waves2, lds2, stream);
        }
    }
    for (int j = 0; j < count; j++) {
        rc = run_matmul(w[j], q, scales, offsets, stride, tokens, y[j], ldy[j], 0, w[j]->rows, nullptr, stream);
        if (rc) return rc;
    }
    return NHIP_OK;
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
                                 int groups_pad8, uint16_t* __restrict__ dst, int* __restrict__ special)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows_pad * groups_pad8) return;
    const int n = (int)(i / groups_pad8);
    const int g = (int)(i % groups_pad8);
    const uint16_t h = (n < rows && g < groups) ? src[(size_t)n * groups + g] : (uint16_t)0;
    dst[i] = h;
    if ((h & 0x7C00u) == 0x7C00u) atomicOr(special, 1);
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
        // lut4x's split tables: bytes 0..7 and 8..15, every byte but the
        // fifth of each complemented (the codebook bytes are below 128)
        uint8_t split[16];
        for (int i = 0; i < 16; i++)
            split[i] = (i & 7) == 4 ? book->bytes[i] : static_cast<uint8_t>(~book->bytes[i]);
        std::memcpy(w->split_table, split, 16);
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
    int* d_special = nullptr;
    e = hipMalloc(&d_special, sizeof(int));
    if (e == hipSuccess) e = hipMemsetAsync(d_special, 0, sizeof(int), s);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(pad_norms_kernel, dim3((unsigned)((norm_elems + 255) / 256)), dim3(256), 0, s, d_norms,
                           rows, w->groups, w->tiles_n * 16, w->groups_pad8, w->norms, d_special);
        e = hipGetLastError();
    }
    int special = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&special, d_special, sizeof(int), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(d_special);
    if (e != hipSuccess) {
        set_error("weight re-tiling failed: %s", hipGetErrorString(e));
        (void)hipFree(w->tiles);
        (void)hipFree(w->norms);
        delete w;
        return NHIP_ERR_HIP;
    }
    w->special_scales = special;
    if (fmt == WeightFormat::Int8G32 && rows <= kNarrowMaxRows) {
        // the narrow decode kernel's row-major copy (narrow.hip)
        e = hipMalloc(&w->rowmajor, (size_t)rows * cols);
        if (e == hipSuccess) e = hipMemcpyAsync(w->rowmajor, d_src, (size_t)rows * cols, hipMemcpyDeviceToDevice, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) {
            set_error("row-major weight copy failed: %s", hipGetErrorString(e));
            (void)hipFree(w->rowmajor);
            (void)hipFree(w->tiles);
            (void)hipFree(w->norms);
            delete w;
            return NHIP_ERR_HIP;
        }
        w->device_bytes += (size_t)rows * cols;
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

// The codebook decode matmul of every row of w, rows [firsts[k], firsts[k+1])
// into ys[k] (stride ldys[k]) at their row - firsts[k] (firsts[0] == 0,
// ascending, parts <= 4): MatMulBatch's jobs as one matrix stacked by rows.
// Returns 1 (nothing launched) for what it does not take: more than 4
// tokens, exponent-31 norms, or a shape the decode kernel does not take.
int32_t matmul_cq_split_internal(const DeviceWeights* w, const int8_t* values, const float* scales,
                                 const float* offsets, int32_t stride, int32_t tokens, float* const* ys,
                                 const int32_t* ldys, const int32_t* firsts, int32_t parts, hipStream_t stream)
{
    NHIP_REQUIRE(w && w->format != WeightFormat::Int8G32, "weights are not in a codebook format");
    NHIP_REQUIRE(values && scales && offsets && stride >= w->groups, "null activations or stride %d < groups %d",
                 stride, w->groups);
    NHIP_REQUIRE(parts >= 1 && parts <= 4 && firsts[0] == 0, "split matmul: %d parts", parts);
    for (int k = 0; k < parts; k++) {
        const int end = k + 1 < parts ? firsts[k + 1] : w->rows;
        NHIP_REQUIRE(ys[k] && firsts[k] < end && ldys[k] >= end - firsts[k], "split matmul: part %d rows [%d, %d), "
                     "ldy %d", k, firsts[k], end, ldys[k]);
    }
    // 1..4 tokens (the four-group-set tile); with 5..16 the wide tile's
    // schedule put an argument wait ahead of its first loads
    if (tokens < 1 || tokens > 4 || w->special_scales) return 1;
    int32_t rc = ensure_device();
    if (rc) return rc;
    MatmulParams p = matmul_params(w, values, scales, offsets, stride, tokens, ys[0], ldys[0], 0, w->rows, nullptr);
    p.split_n = parts - 1;
    for (int k = 1; k < parts; k++) {
        p.split_row[k - 1] = firsts[k];
        p.split_ldy[k - 1] = ldys[k];
        p.split_y[k - 1] = ys[k];
    }
    return try_cq_decode(w, p, stream);
}

int32_t launch_decode_masked(const DeviceWeights* w, const int8_t* q, const float* qscale, int32_t tokens, float* y,
                             int32_t ldy, const uint32_t* mask, int32_t mask_words, hipStream_t stream)
{
    NHIP_REQUIRE(w && w->format == WeightFormat::Int8G32, "weights are not in the int8 format");
    NHIP_REQUIRE(q && qscale && y && mask && ldy >= w->rows, "masked matmul: null pointer or ldy %d too small", ldy);
    NHIP_REQUIRE(mask_words >= (w->rows + 31) / 32, "masked matmul: %d mask words for %d rows", mask_words, w->rows);
    int32_t rc = ensure_device();
    if (rc) return rc;
    if (tokens >= 1 && tokens <= 16) {
        MatmulParams p = matmul_params(w, q, qscale, nullptr, 0, tokens, y, ldy, 0, w->rows, nullptr);
        p.tile_mask = mask;
        p.mask_words = mask_words;
        p.mask_rows = tokens;
        rc = try_i8_decode(w, p, stream);
        if (rc <= 0) return rc;
    }
    // shapes the decode kernel does not take: every row (a superset)
    return run_matmul(w, q, qscale, nullptr, 0, tokens, y, ldy, 0, w->rows, nullptr, stream);
}

int32_t launch_decode_swiglu(const DeviceWeights* w, const int8_t* q, const float* qscale, int32_t tokens,
                             float* act, int32_t ldy, hipStream_t stream)
{
    NHIP_REQUIRE(w && w->format == WeightFormat::Int8G32, "weights are not in the int8 format");
    NHIP_REQUIRE(w->rows % 16 == 0, "SwiGLU pairs need whole 16-row tiles");
    NHIP_REQUIRE(q && qscale && act && ldy >= w->rows / 2, "SwiGLU matmul: null input/output or ldy %d too small",
                 ldy);
    if (tokens < 1 || tokens > 16) return 1;
    int32_t rc = ensure_device();
    if (rc) return rc;
    MatmulParams p = matmul_params(w, q, qscale, nullptr, 0, tokens, act, ldy, 0, w->rows, nullptr);
    p.swiglu = 1;
    return try_i8_decode(w, p, stream);
}

int32_t launch_decode_fused(const DeviceWeights* w, const DecodePrologue& f, int32_t tokens, float* y, int32_t ldy,
                            hipStream_t stream)
{
    NHIP_REQUIRE(w && w->format == WeightFormat::Int8G32, "weights are not in the int8 format");
    NHIP_REQUIRE(f.x && y && ldy >= (f.swiglu ? w->rows / 2 : w->rows), "fused matmul: null input/output or ldy %d "
                 "too small", ldy);
    NHIP_REQUIRE(!f.swiglu || w->rows % 16 == 0, "fused matmul: SwiGLU pairs need whole 16-row tiles");
    if (tokens < 1 || tokens > 4 || w->special_scales) return 1;
    if (!f.swiglu) {
        const int32_t nrc = launch_i8_narrow(w, f.kind, f.x, f.delta, f.gain, nullptr, f.eps, f.residual, tokens, y,
                                             ldy, 0, w->rows, stream);
        if (nrc <= 0) return nrc;
    }
    const int K = w->cols;
    // waves: 4, or 8 when the (non-norm) prologue needs more threads; CB in
    // {2, 4, 8} dividing the tile's blocks with at most `waves` waves busy
    int waves = 4;
    if (f.kind != kProNorm && K > 4 * 256 * 2) waves = 8;
    const int nt = f.kind == kProNorm ? 256 : 64 * waves;
    const int g4 = (K + 4 * nt - 1) / (4 * nt);
    if (g4 > 2) return 1;
    int cb = 0;
    for (int c : {2, 4, 8}) {
        if (w->blocks % c == 0 && w->blocks <= waves * c) {
            cb = c;
            break;
        }
    }
    if (!cb) return 1;
    MatmulParams p{};
    p.tiles = w->tiles;
    p.norms = w->norms;
    p.y = y;
    p.tokens = tokens;
    p.cols = K;
    p.groups = w->groups;
    p.blocks = w->blocks;
    p.groups_pad8 = w->groups_pad8;
    p.ldy = ldy;
    p.row_start = 0;
    p.row_end = w->rows;
    p.tile_begin = 0;  // the kernel runs every row from tile 0
    p.tile_end = w->tiles_n;
    p.swiglu = f.swiglu;
    p.residual = f.residual;
    p.ldd = ((2 * w->blocks + 3) & ~3) + 4;
    p.d_bytes = tokens * 16 * p.ldd * (int)sizeof(float);
    p.st_bytes = (4 * K + 15) & ~15;
    const size_t lds = (size_t)p.d_bytes + p.st_bytes + (4 * 256 + 4 + 4 * 8) * sizeof(float);
    if (lds > kMaxLds) return 1;
    int32_t rc = ensure_device();
    if (rc) return rc;
    if (cb == 2) return launch_fused_g4<2>(p, f, waves, g4, lds, stream);
    if (cb == 4) return launch_fused_g4<4>(p, f, waves, g4, lds, stream);
    return launch_fused_g4<8>(p, f, waves, g4, lds, stream);
}

int32_t weights_cq_create_internal(const nhip_cq* cq, nhip_weights** out)
{
    NHIP_REQUIRE(cq && cq->indices && cq->norms && cq->book, "Cq view is incomplete");
    NHIP_REQUIRE(cq->bits == 2 || cq->bits == 4, "bits %d is not 2 or 4", cq->bits);
    // the kernels multiply codebook bytes as signed int8 MFMA operands
    for (int i = 0; i < (1 << cq->bits); i++)
        NHIP_REQUIRE(cq->book->bytes[i] < 128, "codebook byte %d is %d: the matmul takes codebook bytes in [0, 127] "
                     "(Codebook.Fill makes [0, 126])", i, cq->book->bytes[i]);
    return create_from_host(cq->bits == 2 ? WeightFormat::Cq2 : WeightFormat::Cq4, cq->indices, cq->norms, cq->rows,
                            cq->cols, cq->book, out);
}

// A pure read with the decode GEMV's access pattern, the bandwidth ceiling
// one launch of that many bytes can reach: 256-thread workgroups over 32 KB,
// wave w over 8 KB of them, eight 16-byte non-temporal loads per lane, each
// wave instruction 1 KB contiguous.  The loaded words are folded by XOR and
// each workgroup stores its fold (so no load is dead).
constexpr int kReadChunk = 32 * 1024;

__global__ __launch_bounds__(256) void read_stream_kernel(const u4* src, size_t n16, uint32_t* sink)
{
    __shared__ uint32_t wf[4];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const size_t base = (size_t)blockIdx.x * (kReadChunk / 16) + (size_t)wave * 512 + lane;
    u4 v[8];
#pragma unroll
    for (int c = 0; c < 8; c++) {
        const size_t i = base + (size_t)c * 64;
        v[c] = i < n16 ? __builtin_nontemporal_load(src + i) : u4{0u, 0u, 0u, 0u};
    }
    uint32_t f = 0u;
#pragma unroll
    for (int c = 0; c < 8; c++) f ^= v[c].x ^ v[c].y ^ v[c].z ^ v[c].w;
    for (int off = 32; off > 0; off >>= 1) f ^= __shfl_xor(f, off);
    if (lane == 0) wf[wave] = f;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = wf[0] ^ wf[1] ^ wf[2] ^ wf[3];
}

}  // namespace nhip

using namespace nhip;

extern "C" {

int32_t nhip_read_stream_dev(const void* d_src, size_t bytes, uint32_t* d_sink, void* stream)
{
    clear_error();
    NHIP_REQUIRE(bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(d_src) & 15) == 0,
                 "read stream: 16-byte aligned source and a multiple of 16 bytes");
    if (bytes == 0) return NHIP_OK;
    NHIP_REQUIRE(d_src && d_sink, "read stream: null pointer");
    int32_t rc = ensure_device();
    if (rc) return rc;
    const size_t grid = (bytes + kReadChunk - 1) / kReadChunk;
    NHIP_REQUIRE(grid <= 0x7FFFFFFF, "read stream: too many bytes");
    hipLaunchKernelGGL(read_stream_kernel, dim3((unsigned)grid), dim3(256), 0, as_stream(stream),
                       static_cast<const u4*>(d_src), bytes / 16, d_sink);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

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
    (void)hipFree(w->rowmajor);
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

int32_t nhip_matmul_batch_dev(const nhip_weights* const* w, int32_t count, const int8_t* d_q, const float* d_scales,
                              const float* d_offsets, int32_t stride, int32_t tokens, float* const* d_y,
                              const int32_t* ldy, void* stream)
{
    clear_error();
    NHIP_REQUIRE(w && count >= 1 && count <= kMaxBatchJobs, "batch of %d jobs outside [1, %d]", count, kMaxBatchJobs);
    const DeviceWeights* dw[kMaxBatchJobs] = {};
    for (int j = 0; j < count; j++) dw[j] = w[j];
    return run_matmul_batch(dw, count, d_q, d_scales, d_offsets, stride, tokens, d_y, ldy, as_stream(stream));
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

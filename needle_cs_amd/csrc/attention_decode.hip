// attention_decode.hip -- ragged decode attention over a pooled int8 KV
// cache on gfx950 (one launch for every row of a ragged batch).
//
// Semantics: AttentionBatch.ExecuteChunk + Attention.MergePartials
// (src/Needle/Blocks.cs:927-966, 750-817) for every (row, head):
//   * the row's positions first .. first+count-1 are split into chunks by the
//     reference's plan (Blocks.cs:934-938; chunk cap a parameter, 8 in the
//     reference);
//   * every chunk is the scalar tile in partial form: score_s =
//     (float(q.k_s) * keyScale_s) * (queryScale * 1/sqrt(qk)), peak = max,
//     e_s = Exp(score_s - peak), sum = sum_s e_s and out_d = sum_s
//     (e_s * valueScale_s) * v_{s,d}, both sums in ascending s;
//   * the chunks are merged in MergePartials' non-SIMD order.
// Exp is the reference polynomial Ops.Exp (exp_poly, common.hpp).  With
// these orders fixed the results are bit-identical to the CPU restatement.
//
// Mapping: one workgroup of 256 threads per (chunk, row, head block); a head
// block is whole kv groups, at most 16 query heads.  Phase 1 gives one
// thread per (kv head, position): it loads the key row once (16-byte loads)
// and forms the int32 dots of every query head of the group with v_dot4.
// Phase 4 gives one thread per (head, 4 value dims), which walks the chunk's
// positions in order, reading one value dword per position (a wave covers 4
// heads x 64 dims = 256 contiguous bytes of a cache row).  A second kernel
// merges each (row, head block)'s partials with one thread per (head, dim);
// the kernel boundary makes the partials visible across XCDs (an in-kernel
// last-arrival merge would need an L2 writeback and invalidate per
// workgroup).
#include <algorithm>
#include <mutex>

#include "common.hpp"

// Scratch of nhip_attention_decode_noalloc_dev: room for the chunk partials
// (peaks, sums and per-chunk outputs) of one call, in a file-scope device
// array that every GPU the library runs on holds until the process ends.  In
// host code this name is only a stand-in for the symbol; host code uses the
// per-device address that attention_scratch_setup() looks up.
constexpr size_t kAttentionScratchBytes = size_t(8) << 20;
static __device__ __align__(256) uint8_t scratch[kAttentionScratchBytes];

namespace nhip {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxHeadsPerBlock = 16;

struct DecodeAttnParams {
    const int8_t* q;        // [rows][heads][qk]
    const float* qscale;    // [rows][heads]
    const int8_t* keys;     // [slots][capacity][kv_heads*qk]
    const float* kscale;    // [slots][capacity][kv_heads]
    const int8_t* values;   // [slots][capacity][kv_heads*64]
    const float* vscale;    // [slots][capacity][kv_heads]
    const int32_t* row_slot;
    const int32_t* row_first;
    const int32_t* row_count;
    float* peaks;           // [rows][max_chunks][heads]
    float* sums;            // [rows][max_chunks][heads]
    float* partials;        // [rows][max_chunks][heads][64]
    float* out;             // [rows][heads][64]
    int8_t* q_out;          // optional: QuantizeInt8 of each output row [rows][heads*64]
    float* qs_out;          //   and its scale [rows] (single-chunk plans, one head block)
    // the whole-row kernel's POST form: fp32 QKV rows [rows][(heads + 2 kv_heads) * 64],
    // each row's position, RoPE tables [capacity][32], and the cache it writes
    const float* qkv;
    const int32_t* positions;
    const float* rope_rows;  // [rows][64]: cos then sin of each row's position (32 each)
    int8_t* wkeys;
    float* wkscale;
    int8_t* wvalues;
    float* wvscale;
    // the whole-row kernel's Needle 3 form: the step's raw Q/K/V projections
    // and what turns them into the query and the cache row
    Needle3AttnInputs n3;
    int32_t rows, heads, kv_heads, qk, slots, capacity, max_chunks, lmax, kv_per_block;
    float inv_sqrt;
    int32_t cus;         // compute units of the device (the chunk kernel's placement period)
    uint32_t cus_magic;  // magic(cus) for fast_div
};

// The attention kernels' preloaded head (head_pair, common.hpp): the span
// arrays, the two pointers of the kernel's first other loads (A, B: the
// chunk and row kernels' q and qscale, the POST row kernel's qkv and
// positions, the merge kernel's peaks and sums), (heads, kv_heads) and
// (kv_per_block, rows).
#define ATTN_HEAD_PARAMS const int32_t *h_slot, const int32_t *h_first, const int32_t *h_count, const void *h_a, \
                         const void *h_b, uint64_t h_heads, uint64_t h_blocks_rows
#define ATTN_HEAD_ARGS(p, A, B) (p).row_slot, (p).row_first, (p).row_count, (const void*)(A), (const void*)(B), \
                                head_pair((p).heads, (p).kv_heads), head_pair((p).kv_per_block, (p).rows)
#define ATTN_TAKE_HEAD(p, A, B)                                              \
    do {                                                                     \
        (p).row_slot = h_slot;                                               \
        (p).row_first = h_first;                                             \
        (p).row_count = h_count;                                             \
        (p).A = (decltype((p).A))(h_a);                                      \
        (p).B = (decltype((p).B))(h_b);                                      \
        (p).heads = head_lo(h_heads);                                        \
        (p).kv_heads = head_hi(h_heads);                                     \
        (p).kv_per_block = head_lo(h_blocks_rows);                           \
        (p).rows = head_hi(h_blocks_rows);                                   \
    } while (0)

}  // namespace

// Longest chunk of the plan: at most 32 positions below 16*max_chunks
// positions, else ceil(capacity/max_chunks) rounded up to 4.
int decode_attention_lmax(int capacity, int max_chunks)
{
    return std::max(32, ((capacity + max_chunks - 1) / max_chunks + 3) & ~3);
}

// LDS of the chunk kernel: query heads, scores / weights / value scales per
// head and position of a block, its peaks and query scales.
size_t decode_attention_lds(int lmax, int kv_per_block, int group)
{
    return kMaxHeadsPerBlock * 64 + (size_t)3 * kv_per_block * group * lmax * sizeof(float) +
           2 * kMaxHeadsPerBlock * sizeof(float);
}

// KV heads per workgroup: whole groups of at most 16 query heads, fewer when
// a block's scores would not fit in 64 KB of LDS (0: none fit).
int decode_attention_kv_per_block(int group, int kv_heads, int lmax)
{
    int kv = std::min(std::max(1, kMaxHeadsPerBlock / group), kv_heads);
    while (kv > 0 && decode_attention_lds(lmax, kv, group) > 64 * 1024) kv--;
    return kv;
}

namespace {

// The reference's chunk plan (Blocks.cs:934-938).
__device__ __forceinline__ int plan(int count, int max_chunks, int* length)
{
    int needed = min(max(count / 16, 1), max_chunks);
    const int len = ((count + needed - 1) / needed + 3) & ~3;
    *length = len;
    return (count + len - 1) / len;
}

// n / d for d in [1, 256] and n < 2^24, with mag = magic(d): multiply-high
// by ceil(2^32 / d) (d == 1, whose multiplier does not fit, passes n through)
__device__ __forceinline__ uint32_t magic(uint32_t d) { return d == 1 ? 0u : 0xFFFFFFFFu / d + 1u; }
__device__ __forceinline__ int fast_div(int n, uint32_t mag) { return mag ? (int)__umulhi((uint32_t)n, mag) : n; }

// Unsigned keys in the order of the floats (-0 below +0, as MathF.Max
// prefers +0): max over keys is max over values, in any order.
__device__ __forceinline__ uint32_t order_key(float x)
{
    const uint32_t u = __float_as_uint(x);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float order_value(uint32_t k)
{
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__device__ __forceinline__ float sx8(uint32_t v, int b)
{
    return static_cast<float>(static_cast<int32_t>(v << (24 - 8 * b)) >> 24);
}

constexpr int kVBlock = 32;  // value dwords per thread loaded together

// A uniform load of data that no kernel of the launch writes, through the
// scalar cache.  Kernels that store to global memory would otherwise load
// such arrays with vector loads (the compiler cannot rule out aliasing),
// which costs a memory round trip of its own ahead of the dependent loads.
__device__ __forceinline__ int32_t uniform_load(const int32_t* a, int i)
{
    return ((const __attribute__((address_space(4))) int32_t*)a)[i];
}

// Placement of the chunk kernel's (row, chunk) units on compute units, for
// batches of up to kPlacedRows rows.  A launch's workgroups are dealt to the
// CUs in turn (workgroup g to CU g mod P, P CUs, all resident at once), and a
// CU's time grows with the positions of its units, so the units are ordered
// by chunk length, longest first (ties: lower row first), and unit j goes to
// workgroup g whose round g / P runs forward on even rounds and backward on
// odd ones: each CU's long and short units pair up.  Every lane of a wave
// takes one row (span, plan); lane r's units are j in [before_r, before_r +
// needed_r), before_r summing the units of the rows ordered ahead of it, a
// quarter of the rows per wave, combined through LDS.  Rows with an invalid
// span count as one unit of length 0 (its workgroup writes the zeros).
// Returns false, uniformly over the workgroup, when workgroup g has no unit.
constexpr int kPlacedRows = 64;

struct PlacedUnit {
    int row, chunk, slot, first, count, needed, length;
    bool valid;
};

__device__ __forceinline__ bool place_unit(const DecodeAttnParams& p, int g, PlacedUnit& u)
{
    __shared__ int quarter_sums[4][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform, so the loop below is
    const bool live = lane < p.rows;
    int s = 0, f = 0, c = 0;
    if (live) {
        s = p.row_slot[lane];
        f = p.row_first[lane];
        c = p.row_count[lane];
    }
    // the cache pointers and sizes in the same round trip (left to itself the
    // compiler loads them from the argument segment after the placement)
    asm volatile("" ::"s"(p.keys), "s"(p.kscale), "s"(p.values), "s"(p.vscale), "s"(p.lmax), "s"(p.qk),
                 "s"(p.inv_sqrt), "s"(p.slots), "s"(p.capacity), "s"(p.max_chunks), "s"(p.cus), "s"(p.cus_magic),
                 "s"(p.out), "s"(p.partials), "s"(p.q_out));
    const bool ok = live & (s >= 0) & (s < p.slots) & (f >= 0) & (c >= 1) & (c <= p.capacity - f);
    // the reference's plan (as plan()) in unsigned arithmetic, count >= 1
    const uint32_t cu = ok ? (uint32_t)c : 16u;
    const uint32_t want = min(max(cu >> 4, 1u), (uint32_t)p.max_chunks);
    const uint32_t len = (((cu + want - 1) / want) + 3) & ~3u;
    const int need = ok ? (int)((cu + len - 1) / len) : (live ? 1 : 0);
    const int key = live ? (ok ? (int)len : 0) * 64 + (63 - lane) : -1;
    const int per = (p.rows + 3) >> 2;
    const int r_end = min(p.rows, (wave + 1) * per);
    int before = 0;
    for (int r = wave * per; r < r_end; r++) {  // uniform bounds
        const int kr = __builtin_amdgcn_readlane(key, r);
        const int nr = __builtin_amdgcn_readlane(need, r);
        before += kr > key ? nr : 0;
    }
    quarter_sums[wave][lane] = before;
    __syncthreads();
    before = quarter_sums[0][lane] + quarter_sums[1][lane] + quarter_sums[2][lane] + quarter_sums[3][lane];
    const int P = p.cus;
    const int round = fast_div(g, p.cus_magic);
    const int at = g - round * P;
    const int j = round * P + ((round & 1) ? P - 1 - at : at);
    const uint64_t hit = __ballot(live && before <= j && j < before + need);
    if (hit == 0) return false;
    const int r = __builtin_ctzll(hit);
    u.row = r;
    u.chunk = j - __builtin_amdgcn_readlane(before, r);
    u.slot = __builtin_amdgcn_readlane(s, r);
    u.first = __builtin_amdgcn_readlane(f, r);
    u.count = __builtin_amdgcn_readlane(c, r);
    u.needed = __builtin_amdgcn_readlane(need, r);
    u.length = __builtin_amdgcn_readlane((int)len, r);
    u.valid = __builtin_amdgcn_readlane((int)ok, r) != 0;
    return true;
}

__global__ __launch_bounds__(kThreads) void decode_attention_kernel(ATTN_HEAD_PARAMS, DecodeAttnParams p)
{
    ATTN_TAKE_HEAD(p, q, qscale);
    extern __shared__ __align__(16) uint8_t lds[];
    const int hb = blockIdx.z;
    const int tid = threadIdx.x;
    const int group = p.heads / p.kv_heads;
    const int kv0 = hb * p.kv_per_block;
    const int nkv = min(p.kv_per_block, p.kv_heads - kv0);
    const int h0 = kv0 * group;
    const int nh = nkv * group;  // <= 16
    const int lmax = p.lmax;

    const int hmax = p.kv_per_block * group;                                // heads of a full block
    int8_t* q_lds = reinterpret_cast<int8_t*>(lds);                        // [16][64]
    float* score = reinterpret_cast<float*>(lds + kMaxHeadsPerBlock * 64);  // [hmax][lmax], then e_s
    float* vsc = score + hmax * lmax;                                       // [kv][lmax]
    float* wl = vsc + hmax * lmax;                                          // [hmax][lmax] e_s * valueScale_s
    float* qs_lds = wl + hmax * lmax;                                       // [16]
    uint32_t* peak_key = reinterpret_cast<uint32_t*>(qs_lds + kMaxHeadsPerBlock);  // [16]

    // the unit, its row's span and plan in one round trip
    PlacedUnit u;
    if (p.rows <= kPlacedRows) {
        if (!place_unit(p, blockIdx.x, u)) return;
    } else {  // one workgroup per (chunk, row): scalar loads, no branch between them
        u.row = blockIdx.y;
        u.chunk = blockIdx.x;
        u.slot = uniform_load(p.row_slot, u.row);
        u.first = uniform_load(p.row_first, u.row);
        u.count = uniform_load(p.row_count, u.row);
        // the cache pointers and sizes in the same round trip: left to itself
        // the compiler loads them from the argument segment only after the
        // plan, a second round trip ahead of the first cache load
        asm volatile("" ::"s"(p.keys), "s"(p.kscale), "s"(p.values), "s"(p.vscale), "s"(p.lmax), "s"(p.qk),
                     "s"(p.inv_sqrt));
        // rows with an invalid slot or span produce zeros (no out-of-range reads)
        u.valid = (u.slot >= 0) & (u.slot < p.slots) & (u.first >= 0) & (u.count >= 1) &
                  (u.count <= p.capacity - u.first);
        u.needed = u.valid ? plan(u.count, p.max_chunks, &u.length) : 1;
    }
    const int row = u.row, chunk = u.chunk, slot = u.slot, first = u.first, count = u.count;
    if (!u.valid) {
        if (chunk == 0 && tid < nh * 16) {
            *reinterpret_cast<float4*>(p.out + ((size_t)row * p.heads + h0 + (tid >> 4)) * 64 + 4 * (tid & 15)) =
                make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (p.q_out) *reinterpret_cast<uint32_t*>(p.q_out + (size_t)row * p.heads * 64 + 4 * tid) = 0u;
        }
        if (chunk == 0 && tid == 0 && p.q_out) p.qs_out[row] = 1.0f;
        return;
    }
    const int needed = u.needed, length = u.length;
    if (chunk >= needed) return;
    const int begin = first + chunk * length;
    const int L = min(length, count - chunk * length);
    const size_t pos0 = (size_t)slot * p.capacity + begin;
    const int qk = p.qk;
    const int q4 = qk / 4;

    // Loads are issued oldest-first in the order they are consumed (the
    // vector memory counter retires in order): the query heads and scales,
    // the first pass of key rows and scales (phase 1), then this thread's
    // value dwords of the first kVBlock positions (phase 4), which arrive
    // while the scores are formed.
    const uint32_t qword = tid < nh * q4
        ? reinterpret_cast<const uint32_t*>(p.q + ((size_t)row * p.heads + h0) * qk)[tid] : 0u;
    const float qsc = tid < nh ? p.qscale[(size_t)row * p.heads + h0 + tid] : 0.0f;

    // Cache addresses: a uniform base at the chunk's first (position, kv
    // head) cell plus a 32-bit lane offset (one add per load; the launch
    // checks that a chunk's cells span less than 2 GB)
    const size_t cell0 = pos0 * p.kv_heads + kv0;
    const bool vthread = tid < nh * 16;
    const int vhl = vthread ? tid >> 4 : 0;
    const int vqd = tid & 15;
    const uint32_t vrow = (uint32_t)p.kv_heads * 64u;  // value bytes per cache position
    const uint8_t* vbase = reinterpret_cast<const uint8_t*>(p.values) + cell0 * 64;
    const uint32_t voff = (uint32_t)(vhl / group) * 64u + 4u * (uint32_t)vqd;
    auto vload = [&](int s) {
        return *reinterpret_cast<const uint32_t*>(vbase + (voff + (uint32_t)min(s, L - 1) * vrow));
    };
    uint32_t vreg[kVBlock];

    // phase 1: scores.  The chunk's key rows for this head block are read as
    // 16-byte units, four consecutive lanes per (position, kv head) -- a wave
    // instruction covers 1 KB of consecutive cache rows (768 B for qk 48,
    // whose fourth lane idles).  Each lane dots its 16 bytes with the query
    // heads of the group (v_dot4) and the four partial int32 sums are added
    // across the lanes (exact).
    const int units = L * nkv * 4;
    const int pieces = qk / 16;
    const int lslot = tid & 3;
    const int qslot = min(lslot, pieces - 1);
    const uint32_t mag_kv = magic((uint32_t)nkv);
    const uint32_t mag_l = magic((uint32_t)L);
    // slot 0 the key scale, slot 1 the value scale
    const float* sbase = ((lslot & 1) ? p.vscale : p.kscale) + cell0;
    const int8_t* kbase = p.keys + cell0 * qk;
    const uint32_t kgap = (uint32_t)(p.kv_heads - nkv);  // cells of other blocks per position
    constexpr int KU = 8;  // units per thread per pass, loads issued together
    auto pass = [&](int base) {
        uint4 kw[KU];
        float sv[KU];
#pragma unroll
        for (int k = 0; k < KU; k++) {
            if (base + k * kThreads >= units) break;  // uniform: no duplicate loads
            const uint32_t w = (uint32_t)min(base + k * kThreads + tid, units - 1) >> 2;
            // cell offset (s * kv_heads + kvl) of unit w = s * nkv + kvl
            const uint32_t cw = kgap ? w + (uint32_t)fast_div((int)w, mag_kv) * kgap : w;
            kw[k] = *reinterpret_cast<const uint4*>(kbase + (cw * (uint32_t)qk + 16u * (uint32_t)qslot));
            sv[k] = sbase[cw];
        }
        if (base == 0) {  // the value loads, then stage the query heads and scales
#pragma unroll
            for (int j = 0; j < kVBlock; j++) vreg[j] = vload(j);
            if (tid < nh * q4) reinterpret_cast<uint32_t*>(q_lds)[(tid / q4) * 16 + (tid % q4)] = qword;
            if (tid < nh) {
                qs_lds[tid] = qsc * p.inv_sqrt;
                peak_key[tid] = order_key(-INFINITY);
            }
            __syncthreads();
        }
#pragma unroll
        for (int k = 0; k < KU; k++) {
            const int u = base + k * kThreads + tid;
            if (base + k * kThreads >= units) break;  // uniform
            const bool ok = u < units;  // whole aligned 4-lane groups
            const int w = min(u, units - 1) >> 2;
            const int s = fast_div(w, mag_kv);
            const int kvl = w - s * nkv;
            for (int g = 0; g < group; g++) {
                const int hl = kvl * group + g;
                const uint4 qv = *reinterpret_cast<const uint4*>(q_lds + hl * 64 + 16 * qslot);
                int part = 0;
                part = __builtin_amdgcn_sdot4((int)qv.x, (int)kw[k].x, part, false);
                part = __builtin_amdgcn_sdot4((int)qv.y, (int)kw[k].y, part, false);
                part = __builtin_amdgcn_sdot4((int)qv.z, (int)kw[k].z, part, false);
                part = __builtin_amdgcn_sdot4((int)qv.w, (int)kw[k].w, part, false);
                part = lslot < pieces ? part : 0;
                // sum over the aligned 4-lane group: quad permutations [1,0,3,2]
                // and [2,3,0,1] (DPP, no LDS round trip)
                part += __builtin_amdgcn_mov_dpp(part, 0xB1, 0xF, 0xF, false);
                part += __builtin_amdgcn_mov_dpp(part, 0x4E, 0xF, 0xF, false);
                if (ok && lslot == 0) {
                    const float sc = (static_cast<float>(part) * sv[k]) * qs_lds[hl];
                    score[hl * lmax + s] = sc;
                    atomicMax(&peak_key[hl], order_key(sc));  // the chunk peak (max is order-free)
                }
            }
            if (ok && lslot == 1) vsc[kvl * lmax + s] = sv[k];
        }
    };
    pass(0);  // peeled: the common case (units <= KU * 256) is straight-line code
    for (int base = KU * kThreads; base < units; base += KU * kThreads) pass(base);
    __syncthreads();

    // phase 3: e_s = Exp(score_s - peak) and e_s * valueScale_s
    for (int it = tid; it < nh * L; it += kThreads) {
        const int hl = fast_div(it, mag_l);
        const int s = it - hl * L;
        const float e = exp_poly(score[hl * lmax + s] - order_value(peak_key[hl]));
        score[hl * lmax + s] = e;
        wl[hl * lmax + s] = e * vsc[(hl / group) * lmax + s];
    }
    __syncthreads();

    // phase 4: one thread per (head, 4 dims), positions in ascending order
    const size_t pbase = ((size_t)row * p.max_chunks + chunk) * p.heads;
    float vout[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (vthread) {
        const int hl = vhl;
        float o0 = 0.0f, o1 = 0.0f, o2 = 0.0f, o3 = 0.0f, total = 0.0f;
        auto step = [&](float e, float w, uint32_t v) {
            total = total + e;
            o0 = o0 + w * sx8(v, 0);
            o1 = o1 + w * sx8(v, 1);
            o2 = o2 + w * sx8(v, 2);
            o3 = o3 + w * sx8(v, 3);
        };
        for (int s0 = 0; s0 < L; s0 += kVBlock) {
            if (s0 > 0) {
#pragma unroll
                for (int j = 0; j < kVBlock; j++) vreg[j] = vload(s0 + j);
            }
#pragma unroll
            for (int j4 = 0; j4 < kVBlock; j4 += 4) {
                if (s0 + j4 >= L) break;  // uniform
                const float4 e4 = *reinterpret_cast<const float4*>(score + hl * lmax + s0 + j4);
                const float4 w4 = *reinterpret_cast<const float4*>(wl + hl * lmax + s0 + j4);
                const int rem = L - (s0 + j4);
                step(e4.x, w4.x, vreg[j4]);
                if (rem > 1) step(e4.y, w4.y, vreg[j4 + 1]);
                if (rem > 2) step(e4.z, w4.z, vreg[j4 + 2]);
                if (rem > 3) step(e4.w, w4.w, vreg[j4 + 3]);
            }
        }
        const int h = h0 + hl;
        if (needed == 1) {
            // the merge of a single partial, in MergePartials' order with
            // w = Exp(peak - peak)
            const float pk = order_value(peak_key[hl]);
            const float w = exp_poly(pk - pk);
            float tot = 0.0f;
            tot = tot + w * total;
            const float inverse = 1.0f / tot;
            o0 = (0.0f + w * o0) * inverse;
            o1 = (0.0f + w * o1) * inverse;
            o2 = (0.0f + w * o2) * inverse;
            o3 = (0.0f + w * o3) * inverse;
            *reinterpret_cast<float4*>(p.out + ((size_t)row * p.heads + h) * 64 + 4 * vqd) =
                make_float4(o0, o1, o2, o3);
        } else {
            *reinterpret_cast<float4*>(p.partials + (pbase + h) * 64 + 4 * vqd) = make_float4(o0, o1, o2, o3);
            if (vqd == 0) {
                p.peaks[pbase + h] = order_value(peak_key[hl]);
                p.sums[pbase + h] = total;
            }
        }
        vout[0] = o0;
        vout[1] = o1;
        vout[2] = o2;
        vout[3] = o3;
    }
    if (needed == 1 && p.q_out) {
        __shared__ float qred[kThreads / 64];
        float m = vthread ? fmaxf(fmaxf(fabsf(vout[0]), fabsf(vout[1])), fmaxf(fabsf(vout[2]), fabsf(vout[3]))) : 0.0f;
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        if ((tid & 63) == 0) qred[tid >> 6] = m;
        __syncthreads();
        const float peak = fmaxf(fmaxf(qred[0], qred[1]), fmaxf(qred[2], qred[3]));
        const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
        const float inverse = 1.0f / scale;
        if (vthread) {
            *reinterpret_cast<uint32_t*>(p.q_out + (size_t)row * p.heads * 64 + (h0 + vhl) * 64 + 4 * vqd) =
                ref_quantize4(make_float4(vout[0], vout[1], vout[2], vout[3]), inverse);
        }
        if (tid == 0) p.qs_out[row] = scale;
    }
}

// Merge of a (row, head)'s chunk partials, one workgroup of 64 threads
// (one per dim): MergePartials' non-SIMD order (Blocks.cs:760-815).  Every
// load is issued first; thread c (< needed) holds chunk c's peak and sum;
// after one barrier every thread walks the chunks in ascending order with
// two independent chains, the total (the same in every thread) and its own
// dim's weighted sum.
constexpr int kMergeBatch = 64;

__global__ __launch_bounds__(64) void decode_merge_kernel(ATTN_HEAD_PARAMS, DecodeAttnParams p)
{
    ATTN_TAKE_HEAD(p, peaks, sums);
    __shared__ __align__(16) float msm[256];
    __shared__ __align__(16) float wts[256];
    const int row = blockIdx.x;
    const int h = blockIdx.y;
    const int d = threadIdx.x;
    const int slot = uniform_load(p.row_slot, row);
    const int first = uniform_load(p.row_first, row);
    const int count = uniform_load(p.row_count, row);
    // the argument-segment fields of the partial loads, read in the same
    // round trip as the span
    asm volatile("" ::"s"(p.partials), "s"(p.out), "s"(p.max_chunks), "s"(p.capacity), "s"(p.slots));
    const bool valid = (slot >= 0) & (slot < p.slots) & (first >= 0) & (count >= 1) & (count <= p.capacity - first);
    float* dst = p.out + ((size_t)row * p.heads + h) * 64 + d;
    if (!valid) return;  // uniform over the block; the chunk kernel wrote zeros
    int length;
    const int needed = plan(count, p.max_chunks, &length);
    if (needed == 1) return;  // the chunk kernel finished the row
    // uniform bases at the (row, head)'s first chunk, 32-bit lane offsets
    // (chunk c at + c * heads for the peaks and sums, + c * heads * 64 for
    // the partials; the workspace layout keeps them below 4 GB)
    const size_t rbase = (size_t)row * p.max_chunks * p.heads + h;
    const float* kbase = p.peaks + rbase;
    const float* sbase = p.sums + rbase;
    const float* pbase = p.partials + rbase * 64;
    const uint32_t heads = (uint32_t)p.heads;
    const uint32_t cstride = heads * 64u;
    // this thread's chunks' peaks and sums (c = d, d + 64, ...; needed <= 256)
    float pk[4], sm[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t c = (uint32_t)min(d + 64 * j, needed - 1);
        pk[j] = kbase[c * heads];
        sm[j] = sbase[c * heads];
    }
    float a[kMergeBatch];
#pragma unroll
    for (int j = 0; j < kMergeBatch; j++) a[j] = pbase[(uint32_t)d + (uint32_t)min(j, needed - 1) * cstride];
    if (needed == 2) {  // uniform over the block: MergePartials' two-chunk branch
        const float peak0 = __shfl(pk[0], 0), peak1 = __shfl(pk[0], 1);
        const float sum0 = __shfl(sm[0], 0), sum1 = __shfl(sm[0], 1);
        const float peak = ref_max(peak0, peak1);
        const float w0 = exp_poly(peak0 - peak);
        const float w1 = exp_poly(peak1 - peak);
        float tot = 0.0f;
        tot = tot + w0 * sum0;
        tot = tot + w1 * sum1;
        const float inv = 1.0f / tot;
        *dst = (w0 * a[0] + w1 * a[1]) * inv;
        return;
    }
    // peak = the largest chunk peak (order-free)
    float peak = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (d + 64 * j < needed) peak = ref_max(peak, pk[j]);
    peak = wave_max(peak);
    // chunk weights and sums, zero from `needed` to the end of its batch of
    // kMergeBatch: the walk below then runs whole batches without branches,
    // and its extra steps add +0 to sums that start at +0 (never -0 under
    // round-to-nearest), which leaves them unchanged
    const int padded = (needed + kMergeBatch - 1) / kMergeBatch * kMergeBatch;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int c = d + 64 * j;
        if (c < padded) {
            wts[c] = c < needed ? exp_poly(pk[j] - peak) : 0.0f;
            msm[c] = c < needed ? sm[j] : 0.0f;
        }
    }
    __syncthreads();
    float total = 0.0f, sum = 0.0f;
    for (int c0 = 0; c0 < needed; c0 += kMergeBatch) {
        if (c0 > 0) {
#pragma unroll
            for (int j = 0; j < kMergeBatch; j++)
                a[j] = pbase[(uint32_t)d + (uint32_t)min(c0 + j, needed - 1) * cstride];
        }
        float4 w4[kMergeBatch / 4], s4[kMergeBatch / 4];
#pragma unroll
        for (int i = 0; i < kMergeBatch / 4; i++) {
            w4[i] = *reinterpret_cast<const float4*>(wts + c0 + 4 * i);
            s4[i] = *reinterpret_cast<const float4*>(msm + c0 + 4 * i);
        }
        const int rem = needed - c0;
        auto step = [&](float w, float sv, float av, int j) {
            total = total + w * sv;
            sum = sum + w * (j < rem ? av : 0.0f);
        };
#pragma unroll
        for (int i = 0; i < kMergeBatch / 4; i++) {
            step(w4[i].x, s4[i].x, a[4 * i], 4 * i);
            step(w4[i].y, s4[i].y, a[4 * i + 1], 4 * i + 1);
            step(w4[i].z, s4[i].z, a[4 * i + 2], 4 * i + 2);
            step(w4[i].w, s4[i].w, a[4 * i + 3], 4 * i + 3);
        }
    }
    *dst = sum * (1.0f / total);
}

// Whole-row attention for caches of at most kRowMaxCapacity positions: one
// workgroup per (row, query head) runs every chunk of the row's plan and then
// merges them itself, with the chunk kernel's per-chunk arithmetic and
// decode_merge_kernel's merge, so the results are the same bits.  For short
// contexts the chunk kernel's grid is small (a few chunks per row, all heads
// in one workgroup) and the merge is a second launch; here the (row, head)
// grid is wider and there is one launch.
//   phase 1: thread per (position, 16-byte key piece), v_dot4 + quad DPP sum;
//            chunk peaks by LDS atomicMax on order keys
//   phase 3: e_s and e_s * valueScale_s
//   phase 4: thread per (chunk, 4 value dims) walks the chunk's positions
//   merge:   wave 0, one lane per dim, chunks in ascending order
//
// POST (the decoder's step, at most kPostRows rows, qk 64): the workgroup
// first builds its inputs from the fp32 QKV rows, as qkv_post_kernel in
// decoder.hip does: RoPE (rotate-half) on its query head and QuantizeInt8
// into the query; RoPE and QuantizeInt8 of the key head and QuantizeInt8 of
// the value head of every row of the batch that writes a position of this
// row's span (same slot) -- those positions are taken from the workgroup's
// own results, not from the cache, since other workgroups of the launch
// write them.  The workgroups of the group's first query head write their
// row's key and value heads and scales to the cache.
constexpr int kRowMaxCapacity = 512;
constexpr int kRowMaxChunks = kRowMaxCapacity / 16;  // the plan makes at most count/16 chunks
constexpr int kPostRows = 4;
// the row kernel's forms: q given, the decoder's step (POST), Needle 3's step (N3)
constexpr int kRowPlain = 0, kRowPost = 1, kRowNeedle3 = 2;
// Threads of a (row, head) workgroup.  The decode forms have a few rows, so
// a workgroup per (row, head) leaves most of the chip idle and 8 waves finish
// each row sooner; the plain form also runs prefill chunks of up to 128 rows
// (thousands of workgroups), where 4 waves keep twice the workgroups resident.
constexpr int row_threads(int mode) { return mode == kRowPlain ? 256 : 512; }

// Needle3Proj's Gate outputs 16 j .. 16 j + 15 of every row t < rows (at
// most 16): wave g < k / 128 takes group g through four i8 MFMAs, one per
// plane (A the rows' prepared activations, B the 2-bit codes through the
// codebook bytes; the codebook decode kernels' operands), then one lane per
// (row, output) runs Scalar.MatMulRows' chain (Scalar.cs:146-192):
//   scaled = (HalfToSingle(norm[n][g]) * ByteScale) * scale[t][g]
//   acc += scaled * D_g;  bias += scaled * offset[t][g]  (g ascending);  y = acc - bias
// lds: 2 * 16 * 16 * 8 floats.
typedef int n3_v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void n3_gate_tile(const Needle3Proj& q, int rows, int j, float* lds)
{
    const int groups = q.k >> 7;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nr = lane & 15, kq = lane >> 4;
    float* pa = lds;  // [t][n][8]
    float* pb = lds + 16 * 16 * 8;
    if (wave < groups) {
        const size_t n = (size_t)j * 16 + nr;
        const uint2 code = *reinterpret_cast<const uint2*>(q.codes[3] + n * (q.k >> 2) + wave * 32 + kq * 8);
        const uint32_t norm = q.norms[3][n * groups + wave];
        n3_v4i d = {0, 0, 0, 0};
#pragma unroll
        for (int pl = 0; pl < 4; pl++) {
            long av = 0;
            if (nr < rows) av = *reinterpret_cast<const long*>(q.act + (size_t)nr * q.k + wave * 128 + 32 * pl + 8 * kq);
            const uint32_t b0 = lut2((code.x >> (2 * pl)) & 0x03030303u, q.table);
            const uint32_t b1 = lut2((code.y >> (2 * pl)) & 0x03030303u, q.table);
            d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, (long)(((uint64_t)b1 << 32) | b0), d, 0, 0, 0);
        }
        // lane l holds D[t = 4 (l / 16) + i][output l % 16] in d[i]
        const float hb = ref_half_to_single(norm) * q.byte_scale;
        const int dv[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 4 * kq + i;
            if (t < rows) {
                const float scaled = hb * q.scales[(size_t)t * q.stride + wave];
                pa[(t * 16 + nr) * 8 + wave] = scaled * static_cast<float>(dv[i]);
                pb[(t * 16 + nr) * 8 + wave] = scaled * q.offsets[(size_t)t * q.stride + wave];
            }
        }
    }
    __syncthreads();
    const int x = threadIdx.x;
    if (x < rows * 16) {
        const float4* ra = reinterpret_cast<const float4*>(pa + x * 8);
        const float4* rb = reinterpret_cast<const float4*>(pb + x * 8);
        const float4 a0 = ra[0], a1 = ra[1], b0 = rb[0], b1 = rb[1];
        const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const float bv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
        float acc = 0.0f, bias = 0.0f;
#pragma unroll
        for (int g = 0; g < 8; g++) {
            if (g < groups) {
                acc = acc + av[g];
                bias = bias + bv[g];
            }
        }
        q.gate[(size_t)(x >> 4) * q.gate_rows + j * 16 + (x & 15)] = acc - bias;
    }
}

template <int MODE>
__global__ __launch_bounds__(row_threads(MODE)) void decode_attention_row_kernel(ATTN_HEAD_PARAMS, DecodeAttnParams p)
{
    constexpr int kRowThreads = row_threads(MODE);
    constexpr int kRowUnits = kRowMaxCapacity * 4 / kRowThreads;  // key pieces per thread
    constexpr int kPostIters = (2 * kPostRows + 1 + kRowThreads / 64 - 1) / (kRowThreads / 64);  // POST units per wave
    constexpr bool POST = MODE == kRowPost;
    constexpr bool N3 = MODE == kRowNeedle3;
    constexpr bool SUB = POST || N3;                 // positions written in this launch come from LDS
    constexpr int kSub = POST ? kPostRows : 1;       // N3: only the row's own position
    if constexpr (POST)
        ATTN_TAKE_HEAD(p, qkv, positions);
    else if constexpr (N3)
        ATTN_TAKE_HEAD(p, n3.raw, positions);
    else
        ATTN_TAKE_HEAD(p, q, qscale);
    if constexpr (N3) {
        // the extra column of workgroups (launched with n3.mix): the row's
        // residual-mix logits (RunLayerBatch, Engine.cs:2364-2378: the phi
        // outputs' Scalar.MatMulRows chains, then a_res * y + b_res[o]) and
        // their Sinkhorn4x4 by wave 0, beside the attention
        if (p.n3.mix && (int)blockIdx.y == p.heads) {
            __shared__ __align__(16) float phi_prod[2 * 16 * kPhiMaxGroups];
            __shared__ __align__(16) int8_t phi_x[128 * kPhiMaxGroups];  // the prepared stream row
            __shared__ float phi_so[2 * kPhiMaxGroups];                   // its group scales, offsets
            __shared__ float logits[16];
            const PhiRows& ph = p.n3.res_phi;
            const int t = blockIdx.x, K = p.n3.res_k, groups = K / 128;
            const int first[4] = {0, 16, 16, 16};
            const PhiUnit unit = phi_load(ph, K, 2, first);
            const float ga = p.n3.a_res[0], gb = p.n3.b_res[threadIdx.x & 15];
            // the row once into LDS (each unit reads a group of it)
            for (int e = threadIdx.x; e < K / 16; e += blockDim.x)
                reinterpret_cast<uint4*>(phi_x)[e] = reinterpret_cast<const uint4*>(ph.in.values + (size_t)t * K)[e];
            if ((int)threadIdx.x < 2 * groups) {
                const float* src = (int)threadIdx.x < groups ? ph.in.scales : ph.in.offsets;
                phi_so[threadIdx.x] = src[(size_t)t * ph.stride + (int)threadIdx.x % groups];
            }
            __syncthreads();
            const float y = phi_outputs(ph, unit, phi_x, phi_so, phi_so + groups, K, first, phi_prod);
            if (threadIdx.x < 16) logits[threadIdx.x] = ga * y + gb;
            __syncthreads();
            if (threadIdx.x < 64) sinkhorn4x4_wave(logits, p.n3.mix + t * 16);
            return;
        }
        // the Gate columns of workgroups (launched with n3.proj): 16 Gate
        // outputs of every row each
        const int gate_col0 = p.heads + (p.n3.mix ? 1 : 0);
        if ((int)blockIdx.y >= gate_col0) {
            __shared__ __align__(16) float gate_lds[2 * 16 * 16 * 8];
            const int j = ((int)blockIdx.y - gate_col0) * p.rows + (int)blockIdx.x;
            if (j < p.n3.proj.gate_rows / 16) n3_gate_tile(p.n3.proj, p.rows, j, gate_lds);
            return;
        }
    }
    // scores, then e_s; e_s * valueScale_s (each padded by kVBlock floats:
    // phase 4 reads the last chunk's rows up to the chunk length)
    __shared__ __align__(16) float score[kRowMaxCapacity + kVBlock];
    __shared__ __align__(16) float wl[kRowMaxCapacity + kVBlock];
    __shared__ float vsc[kRowMaxCapacity];
    __shared__ __align__(16) float part[kRowMaxChunks * 64];
    __shared__ uint32_t peak_key[kRowMaxChunks];
    __shared__ float csum[kRowMaxChunks];
    __shared__ float cwt[kRowMaxChunks];
    __shared__ __align__(16) uint32_t q_lds[16];
    __shared__ __align__(16) uint32_t sub_k[kSub][16];  // POST, N3: key / value heads of the
    __shared__ __align__(16) uint32_t sub_v[kSub][16];  // positions written in this launch
    __shared__ float sub_ks[kSub], sub_vs[kSub], q_scale[1];
    __shared__ float n3_red[N3 ? 3 : 1][64], n3_val[N3 ? 3 : 1][64];  // N3: per-unit norm and RoPE rows
    // N3 with proj: the Q/K/V products [192][8] twice, the heads [192], the
    // row's group scales and offsets [8 + 8] and its activations [1024 B]
    __shared__ __align__(16) float n3_proj_lds[N3 ? 2 * 192 * 8 + 192 + 16 + 256 : 1];

    const int row = blockIdx.x;
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const int group = p.heads / p.kv_heads;
    const int kv = h / group;
    // The first round trip: this row's span (scalar loads), and for POST the
    // fp32 QKV heads of the workgroup's units (they depend on nothing) and
    // every row's position and slot, one per lane (vector loads, read back
    // with v_readlane).  Nothing branches on them, so the loads issue
    // together.  A row with an invalid slot or span runs on the span (slot
    // 0, first 0, count 1), writes zeros and no cache row.
    const int slot_in = uniform_load(p.row_slot, row);
    const int first_in = uniform_load(p.row_first, row);
    const int count_in = uniform_load(p.row_count, row);
    const int e = tid & 63;
    const int units_all = p.heads + 2 * p.kv_heads;
    // POST units: unit 0 is the query head, unit 1 + 2r (+1) row r's key
    // (value) head; of W waves, wave w takes units w, w + W, ... (clamped
    // rows: the loads are unconditional, so no wait gathers them at a join)
    float post_x[kPostIters], post_c[kPostIters], post_sn[kPostIters];
    int rpos[kPostRows], rslot[kPostRows];
    if constexpr (POST) {
#pragma unroll
        for (int k = 0; k < kPostIters; k++) {
            const int u = (tid >> 6) + (kRowThreads / 64) * k;
            const int r = u == 0 ? row : min((u - 1) >> 1, p.rows - 1);
            const bool value = u > 0 && ((u - 1) & 1);
            const int col = u == 0 ? h : (value ? p.heads + p.kv_heads + kv : p.heads + kv);
            post_x[k] = p.qkv[((size_t)r * units_all + col) * 64 + e];
            // the RoPE factors of the unit's row (the query's row, or the
            // row whose key this is), staged per row: no dependence on the
            // position, so they arrive with this first round trip
            const float* rope = p.rope_rows + (size_t)r * 64 + (e & 31);
            post_c[k] = rope[0];
            post_sn[k] = rope[32];
        }
        const int lr = min(e, p.rows - 1);
        const int mpos = p.positions[lr];
        const int mslot = p.row_slot[lr];
#pragma unroll
        for (int r = 0; r < kPostRows; r++) {
            rpos[r] = __builtin_amdgcn_readlane(mpos, r);
            rslot[r] = __builtin_amdgcn_readlane(mslot, r);
        }
    }
    // N3 units: wave 0 the query head h, wave 1 the key head and wave 2 the
    // value head of the row (the step's rows are one per slot): the row's
    // projection, the taps and the norm scales load now, the slot's two
    // previous frames and the RoPE factors once the slot and position are in
    const int n3_part = tid >> 6;  // 0 query, 1 key, 2 value, 3 none
    const int n3_n = n3_part == 2 ? 64 : p.qk;
    const int n3_qw = p.heads * p.qk, n3_kw = p.kv_heads * p.qk;
    const int n3_all = n3_qw + n3_kw + p.kv_heads * 64;
    const int n3_W = n3_part == 0 ? n3_qw : (n3_part == 1 ? n3_kw : p.kv_heads * 64);
    const int n3_base = n3_part == 0 ? 0 : (n3_part == 1 ? n3_qw : n3_qw + n3_kw);
    const int n3_off = (n3_part == 0 ? h : kv) * n3_n;
    const bool n3_lane = n3_part < 3 && e < n3_n;
    const bool n3_proj = N3 && p.n3.proj.codes[0] != nullptr;  // the projections formed here
    // N3 with proj: the loads of this thread's (output, group) units of the
    // row's Q/K/V heads, its piece of the row's activations and its group
    // scale or offset, issued before every other vector load of the
    // workgroup (the memory counter waits in order: loaded after the cache
    // rows, the products would wait for those too)
    constexpr int kProjUnits = 3;  // units <= 3 * kRowThreads (host check)
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 pj_cw[kProjUnits][2];
    uint32_t pj_cn[kProjUnits];
    uint4 pj_x = make_uint4(0u, 0u, 0u, 0u);
    float pj_so = 0.0f;
    if constexpr (N3) {
        if (n3_proj) {
            const Needle3Proj& q = p.n3.proj;
            const int groups = q.k >> 7, nq = p.qk, units_n = (2 * nq + 64) * groups;
            if (tid < q.k / 16) pj_x = reinterpret_cast<const uint4*>(q.act + (size_t)row * q.k)[tid];
            const global_ptr<float> gs = scalar_ptr(q.scales), go = scalar_ptr(q.offsets);
            if (tid < 2 * groups) pj_so = (tid < groups ? gs : go)[(size_t)row * q.stride + tid % groups];
            const global_ptr<uint8_t> c0 = scalar_ptr(q.codes[0]), c1 = scalar_ptr(q.codes[1]),
                                      c2 = scalar_ptr(q.codes[2]);
            const global_ptr<uint16_t> m0 = scalar_ptr(q.norms[0]), m1 = scalar_ptr(q.norms[1]),
                                       m2 = scalar_ptr(q.norms[2]);
#pragma unroll
            for (int k = 0; k < kProjUnits; k++) {
                const int u = tid + k * kRowThreads;
                if (u < units_n) {
                    const int o = u / groups, g = u - o * groups;
                    const int m = o < nq ? 0 : (o < 2 * nq ? 1 : 2);
                    const int r = m == 0 ? h * nq + o : (m == 1 ? kv * nq + o - nq : kv * 64 + o - 2 * nq);
                    const global_ptr<uint8_t> cb = m == 0 ? c0 : (m == 1 ? c1 : c2);
                    const global_ptr<uint16_t> nb = m == 0 ? m0 : (m == 1 ? m1 : m2);
                    const global_ptr<u32x4> w4 = (global_ptr<u32x4>)(cb + (size_t)r * (q.k >> 2) + g * 32);
                    pj_cw[k][0] = w4[0];
                    pj_cw[k][1] = w4[1];
                    pj_cn[k] = nb[(size_t)r * groups + g];
                }
            }
        }
    }
    float n3_x2 = 0.0f, n3_x1 = 0.0f, n3_x0 = 0.0f, n3_t0 = 0.0f, n3_t1 = 0.0f, n3_t2 = 0.0f, n3_sc = 0.0f;
    float n3_cs = 0.0f, n3_sn = 0.0f;
    int n3_pos = 0;
    if constexpr (N3) {
        n3_pos = uniform_load(p.positions, row);
        if (n3_lane) {
            if (!n3_proj) n3_x2 = p.n3.raw[(size_t)row * n3_all + n3_base + n3_off + e];
            // (selected, not indexed: a runtime index into the argument's
            // array would copy it to scratch)
            const float* taps = (n3_part == 0 ? p.n3.taps[0] : (n3_part == 1 ? p.n3.taps[1] : p.n3.taps[2])) + n3_off + e;
            n3_t0 = taps[0];
            n3_t1 = taps[n3_W];
            n3_t2 = taps[2 * n3_W];
            if (n3_part < 2) n3_sc = (n3_part == 0 ? p.n3.q_norm : p.n3.k_norm)[e];
        }
    }
    float* dst = p.out + ((size_t)row * p.heads + h) * 64;
    const bool valid = (slot_in >= 0) & (slot_in < p.slots) & (first_in >= 0) & (count_in >= 1) &
                       (count_in <= p.capacity - first_in);
    const int slot = valid ? slot_in : 0;
    const int first = valid ? first_in : 0;
    const int count = valid ? count_in : 1;
    const bool n3_row_ok = (slot_in >= 0) & (slot_in < p.slots) & (n3_pos >= 0) & (n3_pos < p.capacity);
    if constexpr (N3) {
        if (n3_lane) {
            // frame 0, then frame 1 (the latest) of the slot's Q/K/V history
            const float* hist = p.n3.history + (size_t)slot * 2 * n3_all + 2 * n3_base;
            n3_x1 = hist[n3_W + n3_off + e];
            n3_x0 = hist[n3_off + e];
            if (n3_part < 2) {
                const int half = n3_n / 2;
                const size_t rp = (size_t)(n3_row_ok ? n3_pos : 0) * half + (e < half ? e : e - half);
                n3_cs = p.n3.rope_cos[rp];
                n3_sn = p.n3.rope_sin[rp];
            }
        }
    }
    int length;
    const int needed = plan(count, p.max_chunks, &length);  // count <= capacity <= 512: needed <= 32
    const uint32_t mag_len = magic((uint32_t)length);       // s < 512: s / length is exact
    const size_t pos0 = (size_t)slot * p.capacity + first;
    const int qk = p.qk;
    const int pieces = qk / 16;

    // POST: the rows r of the batch that write a position of this row's span
    // (bit r of `subs`, at span position rel[r]); the same in every thread.
    // Then the RoPE factors of the query and key units.
    uint32_t subs = 0u;
    int rel[kSub];
    int pos_row = 0;
    if constexpr (N3) {
        rel[0] = n3_pos - first;
        subs = (uint32_t)(n3_row_ok & (slot_in == slot) & (rel[0] >= 0) & (rel[0] < count));
        pos_row = n3_pos;
    }
    if constexpr (POST) {
#pragma unroll
        for (int r = 0; r < kPostRows; r++) {
            rel[r] = rpos[r] - first;
            subs |= (uint32_t)((r < p.rows) & (rslot[r] == slot) & (rel[r] >= 0) & (rel[r] < count)) << r;
            pos_row = r == row ? rpos[r] : pos_row;
        }
    }

    uint32_t qword = 0u;
    float qsc = 0.0f;
    if constexpr (!SUB) {
        qword = tid < qk / 4 ? reinterpret_cast<const uint32_t*>(p.q + ((size_t)row * p.heads + h) * qk)[tid] : 0u;
        qsc = p.qscale[(size_t)row * p.heads + h] * p.inv_sqrt;
    }

    // phase 4's value dwords of the first kVBlock positions of this thread's
    // chunk, issued ahead of the key rows
    const int vj = tid & 15;
    const size_t vstride4 = (size_t)p.kv_heads * 16;  // dwords per cache position
    auto vbase = [&](int c) {
        return reinterpret_cast<const uint32_t*>(p.values) + ((pos0 + (size_t)c * length) * p.kv_heads + kv) * 16 + vj;
    };
    uint32_t vreg[kVBlock];
    {
        const int c = tid >> 4;
        if (c < needed) {
            const int L = min(length, count - c * length);
            const uint32_t* vp = vbase(c);
#pragma unroll
            for (int j = 0; j < kVBlock; j++) vreg[j] = vp[(size_t)min(j, L - 1) * vstride4];
        }
    }

    // phase 1: scores
    const int units = count * 4;
    const int lslot = tid & 3;
    const int qslot = min(lslot, pieces - 1);
    const float* sbase = (lslot & 1) ? p.vscale : p.kscale;  // slot 0 the key scale, slot 1 the value scale
    uint4 kw[kRowUnits];
    float sv[kRowUnits];
#pragma unroll
    for (int k = 0; k < kRowUnits; k++) {
        if (k * kRowThreads >= units) break;  // uniform
        const int u = min(k * kRowThreads + tid, units - 1);
        const size_t cell = (pos0 + (u >> 2)) * p.kv_heads + kv;
        kw[k] = *reinterpret_cast<const uint4*>(p.keys + cell * qk + 16 * qslot);
        sv[k] = sbase[cell];
    }
    if constexpr (N3) {
        if (n3_proj) {
            // the row's query head h and its kv head's key and value heads
            // (Scalar.MatMulRows, Scalar.cs:146-192): thread per (output,
            // group), the group's exact int32 dot of the 2-bit codes (through
            // the codebook bytes) with the prepared activations, and
            //   scaled = (HalfToSingle(norm) * ByteScale) * scale[g]
            //   acc += scaled * D_g;  bias += scaled * offset[g]  (g ascending)
            // then one lane per output: y = acc - bias
            const Needle3Proj& q = p.n3.proj;
            const int groups = q.k >> 7, nq = p.qk, outs = 2 * nq + 64, units_n = outs * groups;
            float* ppa = n3_proj_lds;  // [outs][8]
            float* ppb = ppa + 192 * 8;
            float* praw = ppb + 192 * 8;  // [outs]
            float* pso = praw + 192;      // scales [8], offsets [8]
            int8_t* px = reinterpret_cast<int8_t*>(pso + 16);
            if (tid < q.k / 16) reinterpret_cast<uint4*>(px)[tid] = pj_x;
            if (tid < 2 * groups) pso[(tid < groups ? 0 : 8) + tid % groups] = pj_so;
            __syncthreads();
#pragma unroll
            for (int k = 0; k < kProjUnits; k++) {
                const int u = tid + k * kRowThreads;
                if (u < units_n) {
                    const int o = u / groups, g = u - o * groups;
                    // code word w (bytes 4w..4w+3: elements 4j + plane) meets
                    // activation word plane * 8 + w (planes order)
                    const uint4* xa = reinterpret_cast<const uint4*>(px + g * 128);
                    int dot = 0;
#pragma unroll
                    for (int pl = 0; pl < 4; pl++) {
                        const uint4 xv[2] = {xa[2 * pl], xa[2 * pl + 1]};
#pragma unroll
                        for (int w = 0; w < 8; w++) {
                            const uint32_t cword = w < 4 ? pj_cw[k][0][w] : pj_cw[k][1][w - 4];
                            const uint4& xq = xv[w >> 2];
                            const uint32_t xword = (w & 3) == 0 ? xq.x : (w & 3) == 1 ? xq.y : (w & 3) == 2 ? xq.z : xq.w;
                            dot = __builtin_amdgcn_sdot4((int)lut2((cword >> (2 * pl)) & 0x03030303u, q.table),
                                                         (int)xword, dot, false);
                        }
                    }
                    const float scaled = (ref_half_to_single(pj_cn[k]) * q.byte_scale) * pso[g];
                    ppa[o * 8 + g] = scaled * static_cast<float>(dot);
                    ppb[o * 8 + g] = scaled * pso[8 + g];
                }
            }
            __syncthreads();
            if (tid < outs) {
                float acc = 0.0f, bias = 0.0f;
#pragma unroll
                for (int g = 0; g < 8; g++) {
                    if (g < groups) {
                        acc = acc + ppa[tid * 8 + g];
                        bias = bias + ppb[tid * 8 + g];
                    }
                }
                const float v = acc - bias;
                praw[tid] = v;
                float* rrow = q.raw + (size_t)row * n3_all;
                if (tid < nq)
                    rrow[h * nq + tid] = v;
                else if (h % group == 0)  // once per kv head
                    rrow[tid < 2 * nq ? n3_qw + kv * nq + tid - nq : n3_qw + n3_kw + kv * 64 + tid - 2 * nq] = v;
            }
            __syncthreads();
            if (n3_lane) n3_x2 = praw[(n3_part == 0 ? 0 : (n3_part == 1 ? nq : 2 * nq)) + e];
        }
    }
    if constexpr (POST) {
        // RoPE, then QuantizeInt8 per head, in qkv_post_kernel's arithmetic
#pragma unroll
        for (int k = 0; k < kPostIters; k++) {
            const int u = (tid >> 6) + (kRowThreads / 64) * k;
            const int r = u == 0 ? row : (u - 1) >> 1;
            if (u > 2 * kPostRows || (u > 0 && !((subs >> r) & 1u))) continue;  // uniform per wave
            const bool value = u > 0 && ((u - 1) & 1);
            float v = post_x[k];
            const float other = __shfl_xor(v, 32);
            if (!value) v = e < 32 ? v * post_c[k] - other * post_sn[k] : v * post_c[k] + other * post_sn[k];
            // max |v| over the head (order-free: any reduction order gives
            // the same maximum)
            const float peak = wave_max(fabsf(v));
            const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
            const float inverse = 1.0f / scale;
            const int8_t qv = static_cast<int8_t>(ref_quantize_one(v, inverse));
            if (u == 0) {
                reinterpret_cast<int8_t*>(q_lds)[e] = qv;
                if (e == 0) q_scale[0] = scale;
                continue;
            }
            reinterpret_cast<int8_t*>(value ? sub_v[r] : sub_k[r])[e] = qv;
            if (e == 0) (value ? sub_vs : sub_ks)[r] = scale;
            if (valid && r == row && h % group == 0) {  // this row's cache write, once per kv head
                const size_t cell = ((size_t)slot * p.capacity + pos_row) * p.kv_heads + kv;
                (value ? p.wvalues : p.wkeys)[cell * 64 + e] = qv;
                if (e == 0) (value ? p.wvscale : p.wkscale)[cell] = scale;
            }
        }
    } else if constexpr (N3) {
        // EngineCore.TapsAndAttentionHeadsSingle (Engine.cs:1302-1387) for
        // the row's own units, with needle3_inputs_kernel's arithmetic: the
        // three-tap convolution (Scalar.Taps3), ZeroCenteredRms of query and
        // key heads (sum of squares in the AVX2 tier's order) and RoPE on
        // lanes i and i + n/2, then QuantizeInt8 over the head
        if (n3_part < 3) {  // uniform per wave
            float x = n3_lane ? n3_t0 * n3_x2 + n3_t1 * n3_x1 + n3_t2 * n3_x0 : 0.0f;
            if (n3_part < 2) {
                n3_red[n3_part][e] = x;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const float sum = wave_v256_sum(n3_red[n3_part], n3_red[n3_part], n3_n);
                const float inverse = 1.0f / sqrtf(sum / (float)n3_n + 1e-6f);
                x = n3_lane ? (1.0f + n3_sc) * x * inverse : 0.0f;
                n3_val[n3_part][e] = x;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const int half = n3_n / 2;
                if (n3_lane) {
                    const int i = e < half ? e : e - half;
                    const float a = n3_val[n3_part][i], b = n3_val[n3_part][half + i];
                    x = e < half ? a * n3_cs - b * n3_sn : b * n3_cs + a * n3_sn;
                }
            }
            const float m = wave_max(n3_lane ? fabsf(x) : 0.0f);
            const float scale = m > 0.0f ? m / 127.0f : 1.0f;
            const float inverse = 1.0f / scale;
            const int8_t qv = static_cast<int8_t>(ref_quantize_one(x, inverse));
            if (n3_part == 0) {
                reinterpret_cast<int8_t*>(q_lds)[e] = n3_lane ? qv : static_cast<int8_t>(0);
                if (e == 0) q_scale[0] = scale;
            } else {
                const bool value = n3_part == 2;
                if (n3_lane) reinterpret_cast<int8_t*>(value ? sub_v[0] : sub_k[0])[e] = qv;
                if (e == 0) (value ? sub_vs : sub_ks)[0] = scale;
                if (n3_row_ok && h % group == 0) {  // the row's cache row, once per kv head
                    const size_t cell = ((size_t)slot_in * p.capacity + n3_pos) * p.kv_heads + kv;
                    if (n3_lane) (value ? p.wvalues : p.wkeys)[cell * n3_n + e] = qv;
                    if (e == 0) (value ? p.wvscale : p.wkscale)[cell] = scale;
                }
            }
        }
    } else {
        if (tid < 16) q_lds[tid] = qword;
    }
    if (tid < kRowMaxChunks) peak_key[tid] = order_key(-INFINITY);
    __syncthreads();
    if constexpr (SUB) qsc = q_scale[0] * p.inv_sqrt;
    const uint4 qv = *reinterpret_cast<const uint4*>(q_lds + 4 * qslot);
#pragma unroll
    for (int k = 0; k < kRowUnits; k++) {
        if (k * kRowThreads >= units) break;  // uniform
        const int u = k * kRowThreads + tid;
        const bool ok = u < units;  // whole aligned 4-lane groups
        const int s = min(u, units - 1) >> 2;
        if constexpr (SUB) {
#pragma unroll
            for (int r = 0; r < kSub; r++) {
                if (((subs >> r) & 1u) && s == rel[r]) {
                    kw[k] = *reinterpret_cast<const uint4*>(&sub_k[r][4 * qslot]);
                    sv[k] = (lslot & 1) ? sub_vs[r] : sub_ks[r];
                }
            }
        }
        int d4 = 0;
        d4 = __builtin_amdgcn_sdot4((int)qv.x, (int)kw[k].x, d4, false);
        d4 = __builtin_amdgcn_sdot4((int)qv.y, (int)kw[k].y, d4, false);
        d4 = __builtin_amdgcn_sdot4((int)qv.z, (int)kw[k].z, d4, false);
        d4 = __builtin_amdgcn_sdot4((int)qv.w, (int)kw[k].w, d4, false);
        d4 = lslot < pieces ? d4 : 0;
        d4 += __builtin_amdgcn_mov_dpp(d4, 0xB1, 0xF, 0xF, false);
        d4 += __builtin_amdgcn_mov_dpp(d4, 0x4E, 0xF, 0xF, false);
        if (ok && lslot == 0) {
            const float sc = (static_cast<float>(d4) * sv[k]) * qsc;
            score[s] = sc;
            atomicMax(&peak_key[fast_div(s, mag_len)], order_key(sc));
        }
        if (ok && lslot == 1) vsc[s] = sv[k];
    }
    __syncthreads();

    // phase 3
    for (int s = tid; s < count; s += kRowThreads) {
        const float e = exp_poly(score[s] - order_value(peak_key[fast_div(s, mag_len)]));
        score[s] = e;
        wl[s] = e * vsc[s];
    }
    __syncthreads();

    // phase 4: chunk c's sums in ascending positions
    for (int c0 = 0; c0 < needed; c0 += kRowThreads / 16) {
        const int c = c0 + (tid >> 4);
        if (c >= needed) break;
        const int b = c * length;
        const int L = min(length, count - b);
        const uint32_t* vp = vbase(c);
        float o0 = 0.0f, o1 = 0.0f, o2 = 0.0f, o3 = 0.0f, total = 0.0f;
        auto step = [&](float e, float w, uint32_t v) {
            total = total + e;
            o0 = o0 + w * sx8(v, 0);
            o1 = o1 + w * sx8(v, 1);
            o2 = o2 + w * sx8(v, 2);
            o3 = o3 + w * sx8(v, 3);
        };
        // POST: the positions this launch writes come from the workgroup's
        // own rows, not from the cache
        auto substitute = [&](int s0) {
            if constexpr (SUB) {
#pragma unroll
                for (int r = 0; r < kSub; r++) {
                    const int jj = rel[r] - (b + s0);
                    if (((subs >> r) & 1u) && jj >= 0 && jj < kVBlock) {
                        const uint32_t w = sub_v[r][vj];
#pragma unroll
                        for (int j = 0; j < kVBlock; j++) vreg[j] = j == jj ? w : vreg[j];
                    }
                }
            }
        };
        if (length <= kVBlock) {  // uniform: every chunk in one pass
            if (c0 > 0) {
#pragma unroll
                for (int j = 0; j < kVBlock; j++) vreg[j] = vp[(size_t)min(j, L - 1) * vstride4];
            }
            substitute(0);
            // Positions past L (the last chunk's tail, up to `length`) run as
            // steps of weight 0, so that every thread of the pass runs the
            // same instructions: total + 0 and o + 0 * v leave the sums
            // unchanged, since no partial sum is -0 (they start at +0, and a
            // rounded sum is -0 only when both operands are).  The LDS rows
            // are padded for the reads past the last position.
#pragma unroll
            for (int j4 = 0; j4 < kVBlock; j4 += 4) {
                if (j4 >= length) break;  // uniform
                const float4 e4 = *reinterpret_cast<const float4*>(score + b + j4);
                const float4 w4 = *reinterpret_cast<const float4*>(wl + b + j4);
                step(j4 < L ? e4.x : 0.0f, j4 < L ? w4.x : 0.0f, vreg[j4]);
                step(j4 + 1 < L ? e4.y : 0.0f, j4 + 1 < L ? w4.y : 0.0f, vreg[j4 + 1]);
                step(j4 + 2 < L ? e4.z : 0.0f, j4 + 2 < L ? w4.z : 0.0f, vreg[j4 + 2]);
                step(j4 + 3 < L ? e4.w : 0.0f, j4 + 3 < L ? w4.w : 0.0f, vreg[j4 + 3]);
            }
        } else {
            for (int s0 = 0; s0 < L; s0 += kVBlock) {
                if (s0 > 0 || c0 > 0) {
#pragma unroll
                    for (int j = 0; j < kVBlock; j++) vreg[j] = vp[(size_t)min(s0 + j, L - 1) * vstride4];
                }
                substitute(s0);
#pragma unroll
                for (int j4 = 0; j4 < kVBlock; j4 += 4) {
                    if (s0 + j4 >= L) break;
                    const float4 e4 = *reinterpret_cast<const float4*>(score + b + s0 + j4);
                    const float4 w4 = *reinterpret_cast<const float4*>(wl + b + s0 + j4);
                    const int rem = L - (s0 + j4);
                    step(e4.x, w4.x, vreg[j4]);
                    if (rem > 1) step(e4.y, w4.y, vreg[j4 + 1]);
                    if (rem > 2) step(e4.z, w4.z, vreg[j4 + 2]);
                    if (rem > 3) step(e4.w, w4.w, vreg[j4 + 3]);
                }
            }
        }
        if (needed == 1) {
            // the merge of a single partial, as in the chunk kernel
            const float pk = order_value(peak_key[0]);
            const float w = exp_poly(pk - pk);
            float tot = 0.0f;
            tot = tot + w * total;
            const float inverse = 1.0f / tot;
            *reinterpret_cast<float4*>(dst + 4 * vj) =
                valid ? make_float4((0.0f + w * o0) * inverse, (0.0f + w * o1) * inverse, (0.0f + w * o2) * inverse,
                                    (0.0f + w * o3) * inverse)
                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        } else {
            *reinterpret_cast<float4*>(part + c * 64 + 4 * vj) = make_float4(o0, o1, o2, o3);
            if (vj == 0) csum[c] = total;
        }
    }
    if (needed == 1) return;  // uniform
    __syncthreads();

    // merge: decode_merge_kernel's arithmetic.  Every wave finds the same
    // peak; thread c < needed writes chunk c's weight.
    const int d = tid & 63;
    const float pkd = d < needed ? order_value(peak_key[d]) : -INFINITY;
    float peak = -INFINITY;
    if (d < needed) peak = ref_max(peak, pkd);
    peak = wave_max(peak);
    if (tid < needed) cwt[tid] = exp_poly(pkd - peak);
    __syncthreads();
    if (tid >= 64) return;
    if (needed == 2) {  // MergePartials' two-chunk branch
        const float peak0 = __shfl(pkd, 0), peak1 = __shfl(pkd, 1);
        const float pk2 = ref_max(peak0, peak1);
        const float w0 = exp_poly(peak0 - pk2);
        const float w1 = exp_poly(peak1 - pk2);
        float tot = 0.0f;
        tot = tot + w0 * csum[0];
        tot = tot + w1 * csum[1];
        const float inv = 1.0f / tot;
        dst[d] = (w0 * part[d] + w1 * part[64 + d]) * inv;
        return;
    }
    float total = 0.0f, sum = 0.0f;
    for (int c = 0; c < needed; c++) {
        const float w = cwt[c];
        total = total + w * csum[c];
        sum = sum + w * part[c * 64 + d];
    }
    dst[d] = sum * (1.0f / total);
}

__global__ void zero_kernel(uint32_t* p, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

inline size_t a256(size_t x) { return (x + 255) & ~size_t(255); }

struct WorkspaceLayout {
    size_t peaks, sums, partials, total;
};

WorkspaceLayout layout(int rows, int heads, int max_chunks)
{
    WorkspaceLayout w{};
    const size_t pc = (size_t)rows * max_chunks * heads;
    w.peaks = 0;
    w.sums = w.peaks + a256(pc * sizeof(float));
    w.partials = w.sums + a256(pc * sizeof(float));
    w.total = w.partials + a256(pc * 64 * sizeof(float));
    return w;
}

}  // namespace
}  // namespace nhip

using namespace nhip;

namespace nhip {

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxScratchDevices] = {};  // the scratch array's address on each device
}  // namespace

int32_t attention_scratch_setup()
{
    int dev = -1;
    NHIP_CHECK_HIP(hipGetDevice(&dev));
    NHIP_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, "device %d above %d", dev, kMaxScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch[dev]) return NHIP_OK;
    void* p = nullptr;
    NHIP_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    NHIP_REQUIRE(p != nullptr, "no device address for the attention scratch on device %d", dev);
    g_scratch[dev] = p;
    return NHIP_OK;
}

// The scratch address on the current device (looked up there if this
// device was not the one initialised).
int32_t attention_scratch_address(void** out)
{
    int dev = -1;
    NHIP_CHECK_HIP(hipGetDevice(&dev));
    NHIP_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, "device %d above %d", dev, kMaxScratchDevices);
    {
        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        if (g_scratch[dev]) {
            *out = g_scratch[dev];
            return NHIP_OK;
        }
    }
    int32_t rc = attention_scratch_setup();  // takes the mutex itself
    if (rc) return rc;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    *out = g_scratch[dev];
    return NHIP_OK;
}

int32_t attention_decode_post_impl(const AttnPostInputs& in, int32_t rows, int32_t heads, int32_t kv_heads,
                                   int8_t* d_keys, float* d_key_scales, int8_t* d_values, float* d_value_scales,
                                   int32_t slots, int32_t capacity, const int32_t* d_row_slot,
                                   const int32_t* d_row_first, const int32_t* d_row_count, int32_t max_chunks,
                                   float* d_out, hipStream_t stream)
{
    if (rows < 1 || rows > kPostRows || capacity > kRowMaxCapacity) return 1;
    NHIP_REQUIRE(heads > 0 && kv_heads > 0 && heads % kv_heads == 0 && slots > 0 && capacity > 0 && max_chunks >= 1,
                 "attention: bad shape");
    NHIP_REQUIRE(in.qkv && in.positions && in.rope_rows && d_keys && d_key_scales && d_values &&
                     d_value_scales && d_row_slot && d_row_first && d_row_count && d_out,
                 "attention: null pointer");
    DecodeAttnParams p{};
    p.keys = d_keys;
    p.kscale = d_key_scales;
    p.values = d_values;
    p.vscale = d_value_scales;
    p.wkeys = d_keys;
    p.wkscale = d_key_scales;
    p.wvalues = d_values;
    p.wvscale = d_value_scales;
    p.row_slot = d_row_slot;
    p.row_first = d_row_first;
    p.row_count = d_row_count;
    p.qkv = in.qkv;
    p.positions = in.positions;
    p.rope_rows = in.rope_rows;
    p.out = d_out;
    p.rows = rows;
    p.heads = heads;
    p.kv_heads = kv_heads;
    p.qk = 64;
    p.slots = slots;
    p.capacity = capacity;
    p.max_chunks = max_chunks;
    p.inv_sqrt = static_cast<float>(1.0 / std::sqrt(64.0));
    hipLaunchKernelGGL(decode_attention_row_kernel<kRowPost>, dim3(rows, heads), dim3(row_threads(kRowPost)), 0, stream,
                       ATTN_HEAD_ARGS(p, p.qkv, p.positions), p);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

bool attention_needle3_fused(int32_t capacity, int32_t v_dim) { return capacity <= kRowMaxCapacity && v_dim == 64; }

int32_t attention_decode_needle3_impl(const Needle3AttnInputs& in, int32_t rows, int32_t heads, int32_t kv_heads,
                                      int32_t qk_dim, int32_t v_dim, int8_t* d_keys, float* d_key_scales,
                                      int8_t* d_values, float* d_value_scales, int32_t slots, int32_t capacity,
                                      const int32_t* d_row_slot, const int32_t* d_row_pos,
                                      const int32_t* d_row_first, const int32_t* d_row_count, int32_t max_chunks,
                                      float* d_out, hipStream_t stream)
{
    if (rows < 1 || !attention_needle3_fused(capacity, v_dim)) return 1;
    NHIP_REQUIRE(heads > 0 && kv_heads > 0 && heads % kv_heads == 0 && slots > 0 && capacity > 0 && max_chunks >= 1,
                 "attention: bad shape");
    NHIP_REQUIRE(qk_dim == 48 || qk_dim == 64, "attention: qk_dim must be 48 or 64 (got %d)", qk_dim);
    NHIP_REQUIRE(in.raw && in.taps[0] && in.taps[1] && in.taps[2] && in.q_norm && in.k_norm && in.rope_cos &&
                     in.rope_sin && in.history && d_keys && d_key_scales && d_values && d_value_scales &&
                     d_row_slot && d_row_pos && d_row_first && d_row_count && d_out,
                 "attention: null pointer");
    DecodeAttnParams p{};
    p.keys = d_keys;
    p.kscale = d_key_scales;
    p.values = d_values;
    p.vscale = d_value_scales;
    p.wkeys = d_keys;
    p.wkscale = d_key_scales;
    p.wvalues = d_values;
    p.wvscale = d_value_scales;
    p.row_slot = d_row_slot;
    p.row_first = d_row_first;
    p.row_count = d_row_count;
    p.positions = d_row_pos;
    p.n3 = in;
    p.out = d_out;
    p.rows = rows;
    p.heads = heads;
    p.kv_heads = kv_heads;
    p.qk = qk_dim;
    p.slots = slots;
    p.capacity = capacity;
    p.max_chunks = max_chunks;
    p.inv_sqrt = static_cast<float>(1.0 / std::sqrt(static_cast<double>(qk_dim)));
    NHIP_REQUIRE(!in.mix || (in.res_phi.codes[2] && in.res_phi.norms[2] && in.a_res && in.b_res && in.res_k > 0 &&
                             in.res_k % 128 == 0 && in.res_k / 128 <= kPhiMaxGroups),
                 "attention: the Sinkhorn workgroups need the residual-mix phi rows (K %d)", in.res_k);
    int gate_cols = 0;
    if (in.proj.codes[0]) {
        const Needle3Proj& q = in.proj;
        NHIP_REQUIRE(q.codes[1] && q.codes[2] && q.codes[3] && q.norms[0] && q.norms[1] && q.norms[2] && q.norms[3] &&
                         q.act && q.scales && q.offsets && q.raw && q.gate,
                     "attention: null projection pointer");
        NHIP_REQUIRE(rows <= 16 && q.k > 0 && q.k % 128 == 0 && q.k <= 1024 && q.gate_rows > 0 &&
                         q.gate_rows % 16 == 0 && (2 * qk_dim + 64) * (q.k / 128) <= 3 * row_threads(kRowNeedle3),
                     "attention: projections of %d rows, K %d, %d gate rows", rows, q.k, q.gate_rows);
        gate_cols = (q.gate_rows / 16 + rows - 1) / rows;
    }
    hipLaunchKernelGGL(decode_attention_row_kernel<kRowNeedle3>, dim3(rows, heads + (in.mix ? 1 : 0) + gate_cols),
                       dim3(row_threads(kRowNeedle3)), 0, stream, ATTN_HEAD_ARGS(p, p.n3.raw, p.positions), p);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

int32_t attention_decode_impl(const int8_t* d_q, const float* d_qscale, int32_t rows, int32_t heads,
                              int32_t kv_heads, int32_t qk_dim, const int8_t* d_keys, const float* d_key_scales,
                              const int8_t* d_values, const float* d_value_scales, int32_t slots,
                              int32_t capacity, const int32_t* d_row_slot, const int32_t* d_row_first,
                              const int32_t* d_row_count, int32_t max_chunks, void* d_workspace,
                              size_t workspace_bytes, float* d_out, int8_t* d_q_out, float* d_qs_out,
                              hipStream_t stream)
{
    clear_error();
    if (rows == 0) return NHIP_OK;
    NHIP_REQUIRE(rows > 0 && heads > 0 && kv_heads > 0 && heads % kv_heads == 0,
                 "attention: heads (%d) must be a positive multiple of kv_heads (%d)", heads, kv_heads);
    const int group = heads / kv_heads;
    NHIP_REQUIRE(group <= kMaxHeadsPerBlock, "attention: at most %d query heads per kv head (got %d)",
                 kMaxHeadsPerBlock, group);
    NHIP_REQUIRE(qk_dim == 48 || qk_dim == 64, "attention: qk_dim must be 48 or 64 (got %d)", qk_dim);
    NHIP_REQUIRE(slots > 0 && capacity > 0, "attention: slots and capacity must be positive");
    NHIP_REQUIRE(max_chunks >= 1 && max_chunks <= 256, "attention: max_chunks must be in [1, 256]");
    NHIP_REQUIRE(d_q && d_qscale && d_keys && d_key_scales && d_values && d_value_scales && d_row_slot &&
                     d_row_first && d_row_count && d_workspace && d_out,
                 "attention: null pointer");
    NHIP_REQUIRE(((reinterpret_cast<uintptr_t>(d_q) | reinterpret_cast<uintptr_t>(d_keys) |
                   reinterpret_cast<uintptr_t>(d_values) | reinterpret_cast<uintptr_t>(d_out)) & 15) == 0,
                 "attention: q, keys, values and out must be 16-byte aligned");
    const WorkspaceLayout wl = layout(rows, heads, max_chunks);
    NHIP_REQUIRE(workspace_bytes >= wl.total, "attention: workspace of %zu bytes, need %zu", workspace_bytes,
                 wl.total);
    const int lmax = decode_attention_lmax(capacity, max_chunks);
    const int kv_per_block = decode_attention_kv_per_block(group, kv_heads, lmax);
    NHIP_REQUIRE(kv_per_block > 0, "attention: chunks of up to %d positions do not fit in LDS; raise max_chunks",
                 lmax);
    NHIP_REQUIRE((int64_t)lmax * kv_heads * 64 < (int64_t(1) << 31),
                 "attention: a chunk of %d positions x %d kv heads spans 2 GB of the cache or more", lmax, kv_heads);
    const size_t lds = decode_attention_lds(lmax, kv_per_block, group);
    int32_t rc = ensure_device();
    if (rc) return rc;
    DecodeAttnParams p{};
    p.q = d_q;
    p.qscale = d_qscale;
    p.keys = d_keys;
    p.kscale = d_key_scales;
    p.values = d_values;
    p.vscale = d_value_scales;
    p.row_slot = d_row_slot;
    p.row_first = d_row_first;
    p.row_count = d_row_count;
    uint8_t* ws = static_cast<uint8_t*>(d_workspace);
    p.peaks = reinterpret_cast<float*>(ws + wl.peaks);
    p.sums = reinterpret_cast<float*>(ws + wl.sums);
    p.partials = reinterpret_cast<float*>(ws + wl.partials);
    p.out = d_out;
    p.q_out = d_q_out;
    p.qs_out = d_qs_out;
    p.rows = rows;
    p.heads = heads;
    p.kv_heads = kv_heads;
    p.qk = qk_dim;
    p.slots = slots;
    p.capacity = capacity;
    p.max_chunks = max_chunks;
    p.lmax = lmax;
    p.kv_per_block = kv_per_block;
    p.inv_sqrt = static_cast<float>(1.0 / std::sqrt(static_cast<double>(qk_dim)));
    const int head_blocks = (kv_heads + p.kv_per_block - 1) / p.kv_per_block;
    NHIP_REQUIRE(!d_q_out || (d_qs_out && max_chunks == 1 && head_blocks == 1),
                 "attention: a quantized output needs max_chunks 1 and all heads in one block");
    if (!d_q_out && capacity <= kRowMaxCapacity) {  // every count <= capacity: one workgroup per (row, head)
        hipLaunchKernelGGL(decode_attention_row_kernel<kRowPlain>, dim3(rows, heads), dim3(row_threads(kRowPlain)), 0, stream,
                           ATTN_HEAD_ARGS(p, p.q, p.qscale), p);
        NHIP_CHECK_HIP(hipGetLastError());
        return NHIP_OK;
    }
    p.cus = std::max(device_cus(), 1);
    p.cus_magic = p.cus == 1 ? 0u : 0xFFFFFFFFu / (uint32_t)p.cus + 1u;  // as magic(): exact for g < 2^16
    dim3 grid(max_chunks, rows, head_blocks);
    if (rows <= kPlacedRows) {  // placed units: whole rounds of p.cus workgroups
        grid.x = rows * max_chunks;
        if ((int)grid.x > p.cus) grid.x = (grid.x + p.cus - 1) / p.cus * p.cus;
        grid.y = 1;
    }
    hipLaunchKernelGGL(decode_attention_kernel, grid, dim3(kThreads), lds, stream, ATTN_HEAD_ARGS(p, p.q, p.qscale),
                       p);
    NHIP_CHECK_HIP(hipGetLastError());
    if (max_chunks > 1) {  // single-chunk plans are finished by the chunk kernel
        hipLaunchKernelGGL(decode_merge_kernel, dim3(rows, heads), dim3(64), 0, stream,
                           ATTN_HEAD_ARGS(p, p.peaks, p.sums), p);
        NHIP_CHECK_HIP(hipGetLastError());
    }
    return NHIP_OK;
}

}  // namespace nhip

extern "C" {

size_t nhip_attention_decode_workspace(int32_t rows, int32_t heads, int32_t max_chunks)
{
    if (rows <= 0 || heads <= 0 || max_chunks <= 0) return 0;
    return layout(rows, heads, max_chunks).total;
}

int32_t nhip_attention_decode_workspace_init(void* d_workspace, size_t bytes, void* stream)
{
    NHIP_REQUIRE(d_workspace && bytes % 4 == 0, "attention workspace: null or size not a multiple of 4");
    int32_t rc = ensure_device();
    if (rc) return rc;
    const size_t n = bytes / 4;
    const int grid = (int)std::min<size_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(zero_kernel, dim3(std::max(grid, 1)), dim3(256), 0, as_stream(stream),
                       static_cast<uint32_t*>(d_workspace), n);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

int32_t nhip_attention_decode_dev(const int8_t* d_q, const float* d_qscale, int32_t rows, int32_t heads,
                                  int32_t kv_heads, int32_t qk_dim, const int8_t* d_keys,
                                  const float* d_key_scales, const int8_t* d_values,
                                  const float* d_value_scales, int32_t slots, int32_t capacity,
                                  const int32_t* d_row_slot, const int32_t* d_row_first,
                                  const int32_t* d_row_count, int32_t max_chunks, void* d_workspace,
                                  size_t workspace_bytes, float* d_out, void* stream)
{
    return attention_decode_impl(d_q, d_qscale, rows, heads, kv_heads, qk_dim, d_keys, d_key_scales, d_values,
                                 d_value_scales, slots, capacity, d_row_slot, d_row_first, d_row_count, max_chunks,
                                 d_workspace, workspace_bytes, d_out, nullptr, nullptr, as_stream(stream));
}

int32_t nhip_attention_decode_noalloc_dev(const int8_t* d_q, const float* d_qscale, int32_t rows, int32_t heads,
                                          int32_t kv_heads, int32_t qk_dim, const int8_t* d_keys,
                                          const float* d_key_scales, const int8_t* d_values,
                                          const float* d_value_scales, int32_t slots, int32_t capacity,
                                          const int32_t* d_row_slot, const int32_t* d_row_first,
                                          const int32_t* d_row_count, int32_t max_chunks, float* d_out, void* stream)
{
    clear_error();
    NHIP_REQUIRE(device_ready(), "attention (no allocation): call nhip_init first");
    int32_t rc = ensure_device();
    if (rc) return rc;
    if (rows == 0) return NHIP_OK;
    NHIP_REQUIRE(rows > 0 && heads > 0 && max_chunks >= 1 && max_chunks <= 256,
                 "attention (no allocation): rows %d, heads %d, max_chunks %d", rows, heads, max_chunks);
    const size_t need = layout(rows, heads, max_chunks).total;
    NHIP_REQUIRE(need <= kAttentionScratchBytes,
                 "attention (no allocation): %d rows x %d heads x %d chunks need %zu bytes of partials, above the "
                 "%zu-byte scratch; use nhip_attention_decode_dev with a workspace",
                 rows, heads, max_chunks, need, kAttentionScratchBytes);
    void* ws = nullptr;
    rc = attention_scratch_address(&ws);
    if (rc) return rc;
    return attention_decode_impl(d_q, d_qscale, rows, heads, kv_heads, qk_dim, d_keys, d_key_scales, d_values,
                                 d_value_scales, slots, capacity, d_row_slot, d_row_first, d_row_count, max_chunks, ws,
                                 kAttentionScratchBytes, d_out, nullptr, nullptr, as_stream(stream));
}

}  // extern "C"

// model.hip -- the .cact archive reader of Model.Open on gfx950: the
// archive is parsed in place (the caller's bytes, e.g. a memory map) and
// every tensor is uploaded to HBM once.
//
// Layout (src/Needle/Model.cs:190-276, 307-389; src/Needle/ModelInfo.cs:7-8):
//   header   48 uint32 + 1 float (196 bytes): [0] magic 0x05E12A84, [1]
//            tensor count, [2] codebook floats, [3..47] geometry, float
//            [48] RoPE theta;
//   codebook header[2] floats; the 2-bit book is Codebook.Fill(levels 0..3,
//            4), the 4-bit book Codebook.Fill(levels 12..27, 16);
//   records  header[1] x 44 bytes (packed) {u8 dtype, u8 ndim, u16 pad, u32
//            shape[4], u64 offset, u64 bytes, u32 group, u32 bits}; dtype 1
//            fp16, 2 fp32, 3 codebook-quantized (CQ), 4 raw bytes;
//   CQ data  rows x cols*bits/8 index bytes, then fp16 norms [rows][cols/128].
// The well-formedness checks are Model.RequireWellFormed's, done on the host
// before any device work.  CQ tensors become device weights (the matmul
// kernels' re-tiled layout) and also keep their raw bytes on the device (for
// row gathers: Quant.GatherRow of the embedding and the engram tables);
// fp16 / fp32 tensors become fp32 device arrays.  fp16 records decode with
// Scalar.HalfToSingle, except in archives that carry audio weights (a
// 13-element fp32 record, Model.cs:343, 391-397): there the records before
// the audio block decode with HalfToSingleUpstream, as Model.Open's reader
// does (ExactHalves = !HasAudioWeights, Model.cs:334, 346).  Raw tensors
// (the tokenizer blob) stay in the caller's bytes.
#include <cstring>
#include <vector>

#include "common.hpp"

namespace nhip {

int32_t weights_cq_create_internal(const nhip_cq* cq, nhip_weights** out);

namespace {

constexpr uint32_t kMagic = 0x05E12A84u;
constexpr size_t kHeaderBytes = 196;
constexpr size_t kRecordBytes = 44;  // packed: 1+1+2 + 4*4 + 8+8 + 4+4
constexpr int kGroup = 128;

// Scalar.HalfToSingle (src/Needle/Scalar.cs:121-128) on the host.
float half_to_single(uint16_t half)
{
    const uint32_t mag = half & 0x7FFFu;
    if (mag == 0) return 0.0f;
    if (mag < 0x0400u) {
        const float sub = static_cast<float>(mag) * 5.9604645e-8f;
        return (half & 0x8000u) ? -sub : sub;
    }
    const uint32_t bits = ((mag << 13) + 0x38000000u) | ((half & 0x8000u) << 16);
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Scalar.HalfToSingleUpstream (src/Needle/Scalar.cs:113-119): the exponent
// rebias without the subnormal case.
float half_to_single_upstream(uint16_t half)
{
    const uint32_t mag = half & 0x7FFFu;
    if (mag == 0) return 0.0f;
    const uint32_t bits = ((mag << 13) + 0x38000000u) | ((uint32_t)(half & 0x8000u) << 16);
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Codebook.Fill (src/Needle/Model.cs:44-52): MathF.Round is round-half-even.
void codebook_fill(nhip_codebook* book, const float* levels, int count)
{
    float peak = 0.0f;
    for (int i = 0; i < count; i++) {
        const float a = std::fabs(levels[i]);
        peak = a > peak ? a : peak;
    }
    book->byte_scale = peak / 63.0f;
    for (int i = 0; i < 16; i++) book->levels[i] = levels[i % count];
    for (int i = 0; i < 32; i++)
        book->bytes[i] = i % 16 < count ? static_cast<uint8_t>(std::nearbyint(levels[i % 16] / book->byte_scale) + 63.0f)
                                        : static_cast<uint8_t>(0);
}

// Element count of a dense record, in 128 bits so that untrusted shapes
// cannot wrap around the bounds checks.
unsigned __int128 elements(const nhip_record_info& r)
{
    unsigned __int128 n = 1;
    for (int i = 0; i < r.ndim && i < 4; i++) n *= r.shape[i];
    return n;
}

}  // namespace
}  // namespace nhip

using namespace nhip;

struct nhip_model {
    uint32_t header[48] = {};
    float rope_theta = 0.0f;
    nhip_codebook book2{}, book4{};
    std::vector<nhip_record_info> info;
    std::vector<nhip_weights*> weights;  // CQ records
    std::vector<uint8_t*> raw;           // CQ records: their bytes (indices, then norms) on the device
    std::vector<float*> dense;           // fp16 / fp32 records, fp32 on the device
};

namespace {

#define NHIP_FORMAT(cond, ...)              \
    do {                                    \
        if (!(cond)) {                      \
            ::nhip::set_error(__VA_ARGS__); \
            return NHIP_ERR_FORMAT;         \
        }                                   \
    } while (0)

// Model.RequireWellFormed (src/Needle/Model.cs:372-389) plus the per-record
// checks of Reader.Dense / Reader.Quantized (Model.cs:236-267): everything a
// reader must know before it touches the data.
int32_t check_archive(const uint8_t* data, size_t length, uint32_t* header, std::vector<nhip_record_info>& info)
{
    NHIP_FORMAT(length >= kHeaderBytes, "not a .cact archive: %zu bytes, shorter than the %zu-byte header", length,
                kHeaderBytes);
    std::memcpy(header, data, 48 * sizeof(uint32_t));
    NHIP_FORMAT(header[0] == kMagic, "not a supported .cact archive: magic 0x%08X, expected 0x%08X", header[0], kMagic);
    const uint64_t count = header[1];
    const uint64_t table_end = kHeaderBytes + (uint64_t)header[2] * 4 + count * kRecordBytes;
    NHIP_FORMAT(count != 0 && table_end <= length,
                "truncated .cact archive: %llu tensors and %u codebook floats need %llu bytes of tables, the archive "
                "has %zu", (unsigned long long)count, header[2], (unsigned long long)table_end, length);
    NHIP_FORMAT(header[2] >= 28, "the codebook holds %u floats; the 4-bit levels need 28", header[2]);
    NHIP_FORMAT(header[26] <= 4 && header[31] <= 16, "unsupported engram layout: %u orders, %u sites", header[26],
                header[31]);
    const uint8_t* rec = data + kHeaderBytes + (size_t)header[2] * 4;
    info.resize(count);
    for (uint64_t i = 0; i < count; i++) {
        const uint8_t* r = rec + i * kRecordBytes;
        nhip_record_info& ri = info[i];
        ri.dtype = r[0];
        ri.ndim = r[1];
        uint32_t shape[4];
        std::memcpy(shape, r + 4, 16);
        for (int d = 0; d < 4; d++) ri.shape[d] = shape[d];
        std::memcpy(&ri.offset, r + 20, 8);
        std::memcpy(&ri.bytes, r + 28, 8);
        uint32_t gb[2];
        std::memcpy(gb, r + 36, 8);
        ri.group = gb[0];
        ri.bits = gb[1];
        NHIP_FORMAT(ri.offset <= length && ri.bytes <= length - ri.offset,
                    "truncated .cact archive: tensor %llu ends at byte %llu of %zu", (unsigned long long)i,
                    (unsigned long long)(ri.offset + ri.bytes), length);
        NHIP_FORMAT(ri.ndim <= 4, "tensor %llu has %d dimensions", (unsigned long long)i, ri.ndim);
        if (ri.dtype == NHIP_CACT_CQ) {
            NHIP_FORMAT(ri.bits == 2 || ri.bits == 4, "tensor %llu: 2- or 4-bit CQ tensor expected, %u bits",
                        (unsigned long long)i, ri.bits);
            NHIP_FORMAT(ri.group == kGroup && ri.shape[1] % kGroup == 0 && ri.shape[0] > 0,
                        "tensor %llu: CQ group of 128 expected (group %u, %u x %u)", (unsigned long long)i, ri.group,
                        ri.shape[0], ri.shape[1]);
            const unsigned __int128 need = (unsigned __int128)ri.shape[0] * ri.shape[1] * ri.bits / 8 +
                                           (unsigned __int128)ri.shape[0] * (ri.shape[1] / kGroup) * 2;
            NHIP_FORMAT(need <= length - ri.offset, "tensor %llu: its indices and norms end past the archive",
                        (unsigned long long)i);
            NHIP_FORMAT(ri.shape[0] < (1u << 31) && ri.shape[1] < (1u << 31), "tensor %llu: %u x %u is too large",
                        (unsigned long long)i, ri.shape[0], ri.shape[1]);
        } else if (ri.dtype == NHIP_CACT_FP16 || ri.dtype == NHIP_CACT_FP32) {
            const unsigned __int128 need = elements(ri) * (ri.dtype == NHIP_CACT_FP16 ? 2u : 4u);
            NHIP_FORMAT(need <= length - ri.offset, "tensor %llu: its elements end past the archive",
                        (unsigned long long)i);
        } else {
            NHIP_FORMAT(ri.dtype == NHIP_CACT_RAW, "tensor %llu: unknown dtype %d", (unsigned long long)i, ri.dtype);
        }
    }
    return NHIP_OK;
}

}  // namespace

extern "C" {

int32_t nhip_open(const uint8_t* cact, size_t length, nhip_model** out)
{
    clear_error();
    NHIP_REQUIRE(cact && out, "nhip_open: null pointer");
    *out = nullptr;
    auto* m = new nhip_model();
    int32_t rc = check_archive(cact, length, m->header, m->info);
    if (rc) {
        delete m;
        return rc;
    }
    std::memcpy(&m->rope_theta, cact + 48 * sizeof(uint32_t), sizeof(float));
    const float* levels = reinterpret_cast<const float*>(cact + kHeaderBytes);
    float lv[28];
    std::memcpy(lv, levels, sizeof(lv));  // the map need not be 4-byte aligned
    codebook_fill(&m->book2, lv, 4);
    codebook_fill(&m->book4, lv + 12, 16);
    if ((rc = ensure_device())) {
        delete m;
        return rc;
    }
    const size_t count = m->info.size();
    m->weights.assign(count, nullptr);
    m->raw.assign(count, nullptr);
    m->dense.assign(count, nullptr);
    // HasAudioWeights: the audio block starts at a 13-element fp32 record
    size_t audio_at = count;
    for (size_t i = 0; i < count && audio_at == count; i++)
        if (m->info[i].dtype == NHIP_CACT_FP32 && m->info[i].ndim == 1 && m->info[i].shape[0] == 13) audio_at = i;
    std::vector<float> host;
    for (size_t i = 0; i < count && rc == NHIP_OK; i++) {
        const nhip_record_info& ri = m->info[i];
        const uint8_t* src = cact + ri.offset;
        if (ri.dtype == NHIP_CACT_CQ) {
            const size_t index_bytes = (size_t)ri.shape[0] * ri.shape[1] * ri.bits / 8;
            // the norms follow the indices; copy them if they are not 2-byte aligned
            std::vector<uint16_t> norms((size_t)ri.shape[0] * (ri.shape[1] / kGroup));
            std::memcpy(norms.data(), src + index_bytes, norms.size() * 2);
            nhip_cq cq{src, norms.data(), ri.bits == 2 ? &m->book2 : &m->book4, (int32_t)ri.shape[0],
                       (int32_t)ri.shape[1], (int32_t)ri.bits};
            rc = weights_cq_create_internal(&cq, &m->weights[i]);
            if (rc == NHIP_OK) {
                void* d = nullptr;
                hipError_t e = hipMalloc(&d, std::max<size_t>(ri.bytes, 1));
                if (e == hipSuccess) e = hipMemcpy(d, src, ri.bytes, hipMemcpyHostToDevice);
                if (e != hipSuccess) {
                    set_error("codebook tensor %zu raw upload failed: %s", i, hipGetErrorString(e));
                    rc = NHIP_ERR_HIP;
                }
                m->raw[i] = static_cast<uint8_t*>(d);
            }
        } else if (ri.dtype == NHIP_CACT_FP16 || ri.dtype == NHIP_CACT_FP32) {
            const size_t n = (size_t)elements(ri);
            host.resize(std::max<size_t>(n, 1));
            if (ri.dtype == NHIP_CACT_FP16) {
                for (size_t e = 0; e < n; e++) {
                    uint16_t h;
                    std::memcpy(&h, src + 2 * e, 2);
                    host[e] = audio_at < count && i < audio_at ? half_to_single_upstream(h) : half_to_single(h);
                }
            } else {
                std::memcpy(host.data(), src, n * 4);
            }
            void* d = nullptr;
            hipError_t e = hipMalloc(&d, std::max<size_t>(n, 1) * 4);
            if (e == hipSuccess) e = hipMemcpy(d, host.data(), n * 4, hipMemcpyHostToDevice);
            if (e != hipSuccess) {
                set_error("dense tensor %zu upload failed: %s", i, hipGetErrorString(e));
                rc = NHIP_ERR_HIP;
            }
            m->dense[i] = static_cast<float*>(d);
        }
    }
    if (rc) {
        nhip_model_close(m);
        return rc;
    }
    *out = m;
    return NHIP_OK;
}

int32_t nhip_model_info(const nhip_model* m, uint32_t* header48, float* rope_theta, int32_t* records)
{
    clear_error();
    NHIP_REQUIRE(m, "model is NULL");
    if (header48) std::memcpy(header48, m->header, sizeof(m->header));
    if (rope_theta) *rope_theta = m->rope_theta;
    if (records) *records = (int32_t)m->info.size();
    return NHIP_OK;
}

int32_t nhip_model_record(const nhip_model* m, int32_t index, nhip_record_info* info)
{
    clear_error();
    NHIP_REQUIRE(m && info, "null argument");
    NHIP_REQUIRE(index >= 0 && (size_t)index < m->info.size(), "record %d outside [0, %zu)", index, m->info.size());
    *info = m->info[index];
    return NHIP_OK;
}

const uint8_t* nhip_model_raw(const nhip_model* m, int32_t index)
{
    if (!m || index < 0 || (size_t)index >= m->raw.size()) return nullptr;
    return m->raw[index];
}

int32_t nhip_model_codebooks(const nhip_model* m, nhip_codebook* book2, nhip_codebook* book4)
{
    clear_error();
    NHIP_REQUIRE(m, "model is NULL");
    if (book2) *book2 = m->book2;
    if (book4) *book4 = m->book4;
    return NHIP_OK;
}

nhip_weights* nhip_model_weights(const nhip_model* m, int32_t index)
{
    if (!m || index < 0 || (size_t)index >= m->weights.size()) return nullptr;
    return m->weights[index];
}

const float* nhip_model_dense(const nhip_model* m, int32_t index)
{
    if (!m || index < 0 || (size_t)index >= m->dense.size()) return nullptr;
    return m->dense[index];
}

int32_t nhip_model_close(nhip_model* m)
{
    if (!m) return NHIP_OK;
    for (nhip_weights* w : m->weights)
        if (w) nhip_weights_destroy(w);
    for (float* d : m->dense)
        if (d) (void)hipFree(d);
    for (uint8_t* d : m->raw)
        if (d) (void)hipFree(d);
    delete m;
    return NHIP_OK;
}

}  // extern "C"

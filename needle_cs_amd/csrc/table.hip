// table.hip -- the reference's KernelTable entries (host pointers,
// synchronous) backed by the device kernels.
//
// The reference calls these from its thread pool concurrently on disjoint
// row ranges (src/Needle/Quant.cs:725-771), so every entry is re-entrant:
// per-thread staging buffers and stream, and a mutex-guarded cache mapping a
// weight view's host pointers to its HBM copy (uploaded on first use, kept
// until nhip_table_release drops the entries of a model's host range, which
// the host calls when it disposes of the model: a later model mapped at the
// same addresses must not find the old weights).
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

#include "common.hpp"

namespace nhip {

int32_t matmul_cq_internal(const DeviceWeights* w, const int8_t* values, const float* scales, const float* offsets,
                           int32_t stride, int32_t tokens, float* y, int32_t ldy, int32_t row_start,
                           int32_t row_end, hipStream_t stream);
int32_t weights_cq_create_internal(const nhip_cq* cq, nhip_weights** out);
int32_t quantize_rows_internal(const float* x, int32_t tokens, int32_t cols, int8_t* q, float* scales,
                               hipStream_t stream);
int32_t prepare_internal(const float* x, int32_t tokens, int32_t cols, int32_t bits, int8_t* values, float* scales,
                         float* offsets, int32_t stride, hipStream_t stream);

namespace {

using WeightKey = std::tuple<const void*, const void*, const void*, int32_t, int32_t, int32_t>;
std::mutex g_cache_mutex;
std::map<WeightKey, nhip_weights*> g_cache;

// Per-thread device staging: one growable buffer and one stream.
struct Staging {
    hipStream_t stream = nullptr;
    uint8_t* buf = nullptr;
    size_t cap = 0;
    ~Staging()
    {
        if (buf) hipFree(buf);
        if (stream) hipStreamDestroy(stream);
    }
};
thread_local Staging t_staging;

int32_t staging(size_t bytes, uint8_t** out, hipStream_t* stream)
{
    Staging& s = t_staging;
    if (!s.stream) NHIP_CHECK_HIP(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking));
    if (bytes > s.cap) {
        if (s.buf) NHIP_CHECK_HIP(hipFree(s.buf));
        s.buf = nullptr;
        s.cap = 0;
        const size_t cap = (bytes + (1u << 20) - 1) & ~size_t((1u << 20) - 1);
        NHIP_CHECK_HIP(hipMalloc(&s.buf, cap));
        s.cap = cap;
    }
    *out = s.buf;
    *stream = s.stream;
    return NHIP_OK;
}

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int32_t cached_weights(const nhip_cq* w, nhip_weights** out)
{
    const WeightKey key{w->indices, w->norms, w->book, w->rows, w->cols, w->bits};
    std::lock_guard<std::mutex> lock(g_cache_mutex);
    auto it = g_cache.find(key);
    if (it != g_cache.end()) {
        *out = it->second;
        return NHIP_OK;
    }
    nhip_weights* dw = nullptr;
    int32_t rc = weights_cq_create_internal(w, &dw);
    if (rc) return rc;
    g_cache.emplace(key, dw);
    *out = dw;
    return NHIP_OK;
}

int32_t matmul_rows_impl(const nhip_cq* w, const nhip_activations* a, int32_t tokens, float* y, int32_t ldy,
                         int32_t row_start, int32_t row_end)
{
    NHIP_REQUIRE(w && a, "null weight or activation view");
    NHIP_REQUIRE(tokens >= 0 && row_start >= 0 && row_start <= row_end && row_end <= w->rows,
                 "bad tokens %d or row range [%d,%d) of %d rows", tokens, row_start, row_end, w->rows);
    if (tokens == 0 || row_start == row_end) return NHIP_OK;
    NHIP_REQUIRE(y && ldy >= row_end, "y NULL or ldy %d < row_end %d", ldy, row_end);
    NHIP_REQUIRE(a->cols == w->cols && a->stride >= w->cols / 128, "activation cols %d / stride %d do not fit", a->cols,
                 a->stride);
    int32_t rc = ensure_device();
    if (rc) return rc;
    nhip_weights* dw = nullptr;
    rc = cached_weights(w, &dw);
    if (rc) return rc;
    const int32_t rows = row_end - row_start;
    const size_t vbytes = (size_t)tokens * a->cols;
    const size_t sbytes = (size_t)tokens * a->stride * sizeof(float);
    const size_t ybytes = (size_t)tokens * rows * sizeof(float);
    uint8_t* buf = nullptr;
    hipStream_t s = nullptr;
    rc = staging(align256(vbytes) + 2 * align256(sbytes) + ybytes, &buf, &s);
    if (rc) return rc;
    int8_t* d_values = reinterpret_cast<int8_t*>(buf);
    float* d_scales = reinterpret_cast<float*>(buf + align256(vbytes));
    float* d_offsets = reinterpret_cast<float*>(buf + align256(vbytes) + align256(sbytes));
    float* d_y = reinterpret_cast<float*>(buf + align256(vbytes) + 2 * align256(sbytes));
    NHIP_CHECK_HIP(hipMemcpyAsync(d_values, a->values, vbytes, hipMemcpyHostToDevice, s));
    NHIP_CHECK_HIP(hipMemcpyAsync(d_scales, a->scales, sbytes, hipMemcpyHostToDevice, s));
    NHIP_CHECK_HIP(hipMemcpyAsync(d_offsets, a->offsets, sbytes, hipMemcpyHostToDevice, s));
    // Compute rows [row_start,row_end) into a compact [tokens][rows] buffer:
    // with base d_y - row_start and ldy = rows, row n of token t lands at
    // d_y[t*rows + n - row_start].
    rc = matmul_cq_internal(dw, d_values, d_scales, d_offsets, a->stride, tokens, d_y - row_start, rows, row_start,
                            row_end, s);
    if (rc) return rc;
    NHIP_CHECK_HIP(hipMemcpy2DAsync(y + row_start, (size_t)ldy * sizeof(float), d_y, (size_t)rows * sizeof(float),
                                    (size_t)rows * sizeof(float), tokens, hipMemcpyDeviceToHost, s));
    NHIP_CHECK_HIP(hipStreamSynchronize(s));
    return NHIP_OK;
}

int32_t prepare_impl(const float* x, int32_t tokens, int32_t cols, int32_t bits, const nhip_activations* a)
{
    NHIP_REQUIRE(a, "activation view is NULL");
    NHIP_REQUIRE(tokens >= 0 && cols > 0 && cols % 128 == 0 && (bits == 2 || bits == 4), "bad prepare %dx%d %d-bit",
                 tokens, cols, bits);
    if (tokens <= 0 || a->groups <= 0) return NHIP_OK;
    NHIP_REQUIRE(x && a->values && a->scales && a->offsets, "null pointer");
    int32_t rc = ensure_device();
    if (rc) return rc;
    const size_t xbytes = (size_t)tokens * cols * sizeof(float);
    const size_t vbytes = (size_t)tokens * cols;
    const size_t sbytes = (size_t)tokens * a->stride * sizeof(float);
    uint8_t* buf = nullptr;
    hipStream_t s = nullptr;
    rc = staging(align256(xbytes) + align256(vbytes) + 2 * align256(sbytes), &buf, &s);
    if (rc) return rc;
    float* d_x = reinterpret_cast<float*>(buf);
    int8_t* d_values = reinterpret_cast<int8_t*>(buf + align256(xbytes));
    float* d_scales = reinterpret_cast<float*>(buf + align256(xbytes) + align256(vbytes));
    float* d_offsets = reinterpret_cast<float*>(buf + align256(xbytes) + align256(vbytes) + align256(sbytes));
    NHIP_CHECK_HIP(hipMemcpyAsync(d_x, x, xbytes, hipMemcpyHostToDevice, s));
    // Slots the kernel does not write (padding of the stride) keep the
    // caller's values, as the reference leaves them.
    NHIP_CHECK_HIP(hipMemcpyAsync(d_scales, a->scales, sbytes, hipMemcpyHostToDevice, s));
    NHIP_CHECK_HIP(hipMemcpyAsync(d_offsets, a->offsets, sbytes, hipMemcpyHostToDevice, s));
    rc = prepare_internal(d_x, tokens, cols, bits, d_values, d_scales, d_offsets, a->stride, s);
    if (rc) return rc;
    NHIP_CHECK_HIP(hipMemcpyAsync(a->values, d_values, vbytes, hipMemcpyDeviceToHost, s));
    NHIP_CHECK_HIP(hipMemcpyAsync(a->scales, d_scales, sbytes, hipMemcpyDeviceToHost, s));
    NHIP_CHECK_HIP(hipMemcpyAsync(a->offsets, d_offsets, sbytes, hipMemcpyDeviceToHost, s));
    NHIP_CHECK_HIP(hipStreamSynchronize(s));
    return NHIP_OK;
}

int32_t quantize_impl(const float* x, int32_t n, int8_t* destination, float* scale)
{
    NHIP_REQUIRE(n > 0 && x && destination, "bad quantize arguments");
    int32_t rc = ensure_device();
    if (rc) return rc;
    const size_t xbytes = (size_t)n * sizeof(float);
    uint8_t* buf = nullptr;
    hipStream_t s = nullptr;
    rc = staging(align256(xbytes) + align256((size_t)n) + 256, &buf, &s);
    if (rc) return rc;
    float* d_x = reinterpret_cast<float*>(buf);
    int8_t* d_q = reinterpret_cast<int8_t*>(buf + align256(xbytes));
    float* d_s = reinterpret_cast<float*>(buf + align256(xbytes) + align256((size_t)n));
    NHIP_CHECK_HIP(hipMemcpyAsync(d_x, x, xbytes, hipMemcpyHostToDevice, s));
    rc = quantize_rows_internal(d_x, 1, n, d_q, d_s, s);
    if (rc) return rc;
    NHIP_CHECK_HIP(hipMemcpyAsync(destination, d_q, (size_t)n, hipMemcpyDeviceToHost, s));
    NHIP_CHECK_HIP(hipMemcpyAsync(scale, d_s, sizeof(float), hipMemcpyDeviceToHost, s));
    NHIP_CHECK_HIP(hipStreamSynchronize(s));
    return NHIP_OK;
}

}  // namespace
}  // namespace nhip

using namespace nhip;

extern "C" {

void nhip_matmul_rows(const nhip_cq* w, const nhip_activations* a, int32_t tokens, float* y, int32_t ldy,
                      int32_t row_start, int32_t row_end)
{
    clear_error();
    matmul_rows_impl(w, a, tokens, y, ldy, row_start, row_end);
}

void nhip_prepare(float* x, int32_t tokens, int32_t cols, int32_t bits, const nhip_activations* a)
{
    clear_error();
    prepare_impl(x, tokens, cols, bits, a);
}

float nhip_quantize_int8(const float* x, int32_t n, int8_t* destination)
{
    clear_error();
    float scale = 1.0f;
    if (n <= 0) return scale;
    if (quantize_impl(x, n, destination, &scale) != NHIP_OK) return 1.0f;
    return scale;
}

int32_t nhip_table_release(const void* base, size_t bytes, int32_t* released)
{
    clear_error();
    int32_t n = 0;
    {
        std::lock_guard<std::mutex> lock(g_cache_mutex);
        const uintptr_t lo = reinterpret_cast<uintptr_t>(base);
        for (auto it = g_cache.begin(); it != g_cache.end();) {
            const uintptr_t idx = reinterpret_cast<uintptr_t>(std::get<0>(it->first));
            if (!base || (idx >= lo && idx - lo < bytes)) {
                if (device_ready()) (void)hipDeviceSynchronize();  // no kernel still reads them
                nhip_weights_destroy(it->second);
                it = g_cache.erase(it);
                n++;
            } else {
                ++it;
            }
        }
    }
    if (released) *released = n;
    return NHIP_OK;
}

int32_t nhip_table_cached(int32_t* entries, size_t* device_bytes)
{
    clear_error();
    std::lock_guard<std::mutex> lock(g_cache_mutex);
    size_t total = 0;
    for (const auto& kv : g_cache) {
        size_t b = 0;
        (void)nhip_weights_info(kv.second, nullptr, nullptr, nullptr, &b);
        total += b;
    }
    if (entries) *entries = (int32_t)g_cache.size();
    if (device_bytes) *device_bytes = total;
    return NHIP_OK;
}

int32_t nhip_fill_kernel_table(void** table, int32_t count)
{
    NHIP_REQUIRE(table && count >= 27, "a KernelTable has 27 slots (got %d)", count);
    for (int i = 0; i < count; i++) table[i] = nullptr;
    table[0] = reinterpret_cast<void*>(&nhip_matmul_rows);
    table[1] = reinterpret_cast<void*>(&nhip_prepare);
    table[3] = reinterpret_cast<void*>(&nhip_attention_tile);
    table[4] = reinterpret_cast<void*>(&nhip_merge_partials);
    table[22] = reinterpret_cast<void*>(&nhip_quantize_int8);
    return NHIP_OK;
}

}  // extern "C"

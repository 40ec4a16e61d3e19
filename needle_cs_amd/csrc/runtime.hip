// runtime.hip -- error channel, device selection, memory/stream/event
// plumbing and the synthetic workload generators of libneedle_hip.so.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstring>
#include <mutex>

#include "common.hpp"

namespace nhip {

namespace {
thread_local char g_error[1024] = "";
std::mutex g_init_mutex;
int g_device = -1;
int g_cus = 0;
hipStream_t g_stream = nullptr;
char g_describe[256] = "";
}  // namespace

void set_error(const char* fmt, ...)
{
    va_list args;
    va_start(args, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, args);
    va_end(args);
}

void clear_error() { g_error[0] = '\0'; }

static int32_t init_locked(int32_t device)
{
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) {
        set_error("no HIP device: %s", e == hipSuccess ? "device count is 0" : hipGetErrorString(e));
        return NHIP_ERR_NODEV;
    }
    if (device < 0 || device >= count) {
        set_error("device %d out of range (count %d)", device, count);
        return NHIP_ERR_ARG;
    }
    hipDeviceProp_t prop;
    NHIP_CHECK_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error("device %d is %s; this build targets gfx950 only", device, prop.gcnArchName);
        return NHIP_ERR_NODEV;
    }
    NHIP_CHECK_HIP(hipSetDevice(device));
    int32_t rc = attention_scratch_setup();
    if (rc) return rc;
    if (g_stream == nullptr) NHIP_CHECK_HIP(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    g_device = device;
    g_cus = prop.multiProcessorCount;
    snprintf(g_describe, sizeof(g_describe), "needle_hip 0.1 %s (%d CUs, %.0f GiB HBM)", prop.gcnArchName,
             prop.multiProcessorCount, prop.totalGlobalMem / 1073741824.0);
    return NHIP_OK;
}

int32_t ensure_device()
{
    if (g_device >= 0) {
        // Threads other than the initialising one start on device 0.
        int current = -1;
        if (hipGetDevice(&current) == hipSuccess && current != g_device) NHIP_CHECK_HIP(hipSetDevice(g_device));
        return NHIP_OK;
    }
    std::lock_guard<std::mutex> lock(g_init_mutex);
    if (g_device >= 0) return NHIP_OK;
    return init_locked(0);
}

bool device_ready() { return g_device >= 0; }

int device_cus() { return g_cus; }

hipStream_t default_stream() { return g_stream; }

// XorShift64 (tests/Needle.Tests/Conformance/Conformance.cs:19-27).
static inline uint64_t xs_next(uint64_t* s)
{
    uint64_t x = *s;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *s = x;
    return x;
}

static inline double u53(uint64_t* s) { return (double)(xs_next(s) >> 11) * (1.0 / 9007199254740992.0); }

static uint16_t single_to_half_rne(float f)
{
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t)(sign | (a > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (a >= 0x38800000u) {
        const uint32_t mant = a & 0x7FFFFFu;
        uint32_t h = (((a >> 23) - 112u) << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (a <= 0x33000000u) return (uint16_t)sign;
    const uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
    const int shift = 126 - (int)(a >> 23);
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

}  // namespace nhip

using namespace nhip;

namespace {

__global__ void copy_kernel(uint8_t* dst, const uint8_t* src, size_t n16, size_t tail)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint4* d4 = reinterpret_cast<uint4*>(dst);
    const uint4* s4 = reinterpret_cast<const uint4*>(src);
    for (size_t i = tid; i < n16; i += stride) d4[i] = s4[i];
    const size_t base = n16 * 16;
    for (size_t i = tid; i < tail; i += stride) dst[base + i] = src[base + i];
}

}  // namespace

extern "C" {

const char* nhip_last_error(void) { return g_error; }

const char* nhip_describe(void)
{
    if (ensure_device() != NHIP_OK) return "needle_hip 0.1 (no gfx950 device)";
    return g_describe;
}

int32_t nhip_init(int32_t device)
{
    std::lock_guard<std::mutex> lock(g_init_mutex);
    if (g_device == device) return NHIP_OK;
    if (g_device >= 0) {
        set_error("already initialised on device %d", g_device);
        return NHIP_ERR_ARG;
    }
    return init_locked(device);
}

int32_t nhip_device_count(int32_t* count)
{
    NHIP_REQUIRE(count, "count is NULL");
    int c = 0;
    hipError_t e = hipGetDeviceCount(&c);
    *count = e == hipSuccess ? c : 0;
    return NHIP_OK;
}

int32_t nhip_malloc(void** ptr, size_t bytes)
{
    NHIP_REQUIRE(ptr, "ptr is NULL");
    int32_t rc = ensure_device();
    if (rc) return rc;
    *ptr = nullptr;
    if (bytes == 0) return NHIP_OK;
    NHIP_CHECK_HIP(hipMalloc(ptr, bytes));
    return NHIP_OK;
}

int32_t nhip_free(void* ptr)
{
    if (!ptr) return NHIP_OK;
    NHIP_CHECK_HIP(hipFree(ptr));
    return NHIP_OK;
}

int32_t nhip_memcpy_htod(void* dst, const void* src, size_t bytes)
{
    if (bytes == 0) return NHIP_OK;
    int32_t rc = ensure_device();
    if (rc) return rc;
    // Ordered after the work already queued on the library stream.
    NHIP_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
    NHIP_CHECK_HIP(hipStreamSynchronize(g_stream));
    return NHIP_OK;
}

int32_t nhip_memcpy_dtoh(void* dst, const void* src, size_t bytes)
{
    if (bytes == 0) return NHIP_OK;
    int32_t rc = ensure_device();
    if (rc) return rc;
    NHIP_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
    NHIP_CHECK_HIP(hipStreamSynchronize(g_stream));
    return NHIP_OK;
}

int32_t nhip_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream)
{
    if (bytes == 0) return NHIP_OK;
    int32_t rc = ensure_device();
    if (rc) return rc;
    NHIP_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
    return NHIP_OK;
}

// Plain device copy as a kernel on the given stream (capturable in a graph,
// unlike a DMA copy); 16-byte vectors where both pointers allow, bytes else.
int32_t nhip_copy_dev(void* dst, const void* src, size_t bytes, void* stream)
{
    if (bytes == 0) return NHIP_OK;
    NHIP_REQUIRE(dst && src, "copy: null pointer");
    int32_t rc = ensure_device();
    if (rc) return rc;
    const bool vec = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15) == 0;
    const size_t n16 = vec ? bytes / 16 : 0;
    const size_t tail = bytes - n16 * 16;
    const size_t work = std::max(n16, tail);
    const int block = 256;
    const size_t want = (work + block - 1) / block;
    const int grid = (int)std::min<size_t>(std::max<size_t>(want, 1), 4096);
    hipLaunchKernelGGL(copy_kernel, dim3(grid), dim3(block), 0, as_stream(stream), static_cast<uint8_t*>(dst),
                       static_cast<const uint8_t*>(src), n16, tail);
    NHIP_CHECK_HIP(hipGetLastError());
    return NHIP_OK;
}

int32_t nhip_memset(void* dst, int32_t value, size_t bytes)
{
    if (bytes == 0) return NHIP_OK;
    int32_t rc = ensure_device();
    if (rc) return rc;
    NHIP_CHECK_HIP(hipMemsetAsync(dst, value, bytes, g_stream));
    NHIP_CHECK_HIP(hipStreamSynchronize(g_stream));
    return NHIP_OK;
}

int32_t nhip_stream_create(void** stream)
{
    NHIP_REQUIRE(stream, "stream is NULL");
    int32_t rc = ensure_device();
    if (rc) return rc;
    hipStream_t s;
    NHIP_CHECK_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return NHIP_OK;
}

int32_t nhip_stream_destroy(void* stream)
{
    if (!stream) return NHIP_OK;
    NHIP_CHECK_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)));
    return NHIP_OK;
}

int32_t nhip_stream_sync(void* stream)
{
    int32_t rc = ensure_device();
    if (rc) return rc;
    NHIP_CHECK_HIP(hipStreamSynchronize(as_stream(stream)));
    return NHIP_OK;
}

int32_t nhip_device_sync(void)
{
    int32_t rc = ensure_device();
    if (rc) return rc;
    NHIP_CHECK_HIP(hipDeviceSynchronize());
    return NHIP_OK;
}

int32_t nhip_event_create(void** event)
{
    NHIP_REQUIRE(event, "event is NULL");
    int32_t rc = ensure_device();
    if (rc) return rc;
    hipEvent_t e;
    NHIP_CHECK_HIP(hipEventCreate(&e));
    *event = e;
    return NHIP_OK;
}

int32_t nhip_event_destroy(void* event)
{
    if (!event) return NHIP_OK;
    NHIP_CHECK_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)));
    return NHIP_OK;
}

int32_t nhip_event_record(void* event, void* stream)
{
    NHIP_REQUIRE(event, "event is NULL");
    NHIP_CHECK_HIP(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)));
    return NHIP_OK;
}

int32_t nhip_event_elapsed_ms(void* start, void* stop, float* ms)
{
    NHIP_REQUIRE(start && stop && ms, "null argument");
    NHIP_CHECK_HIP(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
    NHIP_CHECK_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
    return NHIP_OK;
}

int32_t nhip_graph_begin(void* stream)
{
    int32_t rc = ensure_device();
    if (rc) return rc;
    NHIP_CHECK_HIP(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal));
    return NHIP_OK;
}

int32_t nhip_graph_end(void* stream, void** graph_exec)
{
    NHIP_REQUIRE(graph_exec, "graph_exec is NULL");
    hipGraph_t graph = nullptr;
    NHIP_CHECK_HIP(hipStreamEndCapture(as_stream(stream), &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) {
        set_error("hipGraphInstantiate failed: %s", hipGetErrorString(e));
        return NHIP_ERR_HIP;
    }
    *graph_exec = exec;
    return NHIP_OK;
}

int32_t nhip_graph_launch(void* graph_exec, void* stream)
{
    NHIP_REQUIRE(graph_exec, "graph_exec is NULL");
    NHIP_CHECK_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), as_stream(stream)));
    return NHIP_OK;
}

int32_t nhip_graph_destroy(void* graph_exec)
{
    if (!graph_exec) return NHIP_OK;
    NHIP_CHECK_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)));
    return NHIP_OK;
}

void nhip_synth_normal(uint64_t* state, float* x, size_t n)
{
    for (size_t i = 0; i < n; i++) {
        const double u1 = 1.0 - u53(state);
        const double u2 = u53(state);
        x[i] = (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
}

void nhip_synth_uniform(uint64_t* state, float* x, size_t n, float lo, float hi)
{
    for (size_t i = 0; i < n; i++) x[i] = (float)((double)lo + ((double)hi - (double)lo) * u53(state));
}

void nhip_synth_int8(uint64_t* state, int8_t* x, size_t n)
{
    for (size_t i = 0; i < n; i++) x[i] = (int8_t)(-127 + (int)(xs_next(state) % 255u));
}

void nhip_synth_half_uniform(uint64_t* state, uint16_t* x, size_t n, float lo, float hi)
{
    for (size_t i = 0; i < n; i++) {
        const float v = (float)((double)lo + ((double)hi - (double)lo) * u53(state));
        x[i] = single_to_half_rne(v);
    }
}

}  // extern "C"

// Runtime part of the C ABI: device selection, the library stream, memory, events, errors.
#include "fmlh_internal.h"

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace fmlh {

namespace {
thread_local std::string g_error;
std::mutex g_init_mu;
bool g_ready = false;
bool g_shut = false;  // fmlh_shutdown ran; only fmlh_init starts the library again
int g_device = 0;
int g_cus = 0;
hipStream_t g_stream = nullptr;
char g_arch[64] = {0};
// Countdowns of the failure hook (0: off): the event that takes a counter from 1 to 0 fails.
std::atomic<long> g_fault[2] = {{0}, {0}};

void arm_faults() {
    g_fault[kFaultAlloc] = 0;
    g_fault[kFaultLaunch] = 0;
    const char* e = std::getenv("FMLH_FAULT");
    if (!e) return;
    long n = 0;
    if (std::sscanf(e, "alloc:%ld", &n) == 1 && n > 0) g_fault[kFaultAlloc] = n;
    else if (std::sscanf(e, "launch:%ld", &n) == 1 && n > 0) g_fault[kFaultLaunch] = n;
}
}  // namespace

bool inject_fault(FaultKind kind) {
    std::atomic<long>& c = g_fault[kind];
    if (c.load(std::memory_order_relaxed) <= 0) return false;
    return c.fetch_sub(1) == 1;
}

int device_malloc(void** p, size_t bytes) {
    *p = nullptr;
    if (inject_fault(kFaultAlloc))
        return set_error(FMLH_E_HIP, "hipMalloc of %zu bytes failed: out of memory (injected by FMLH_FAULT)", bytes);
    FMLH_HIP(hipMalloc(p, bytes));
    return FMLH_OK;
}

int set_error(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

void clear_error() { g_error.clear(); }

static int init_locked(int device) {
    if (g_ready) {
        if (device != g_device)
            return set_error(FMLH_E_STATE, "already initialised on device %d", g_device);
        return FMLH_OK;
    }
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
        return set_error(FMLH_E_NODEVICE, "no HIP device (%s)", hipGetErrorString(e));
    if (device < 0 || device >= n)
        return set_error(FMLH_E_INVALID, "device %d out of range (%d devices)", device, n);
    FMLH_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    FMLH_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return set_error(FMLH_E_NODEVICE, "device %d is %s; this library is built for gfx950",
                         device, prop.gcnArchName);
    std::snprintf(g_arch, sizeof(g_arch), "%s", prop.gcnArchName);
    g_cus = prop.multiProcessorCount;
    // Default priority on purpose: no stream of this library is created with another one.
    FMLH_HIP(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    g_device = device;
    g_ready = true;
    return setup_noalloc_scratch(device);
}

int ensure_init() {
    std::lock_guard<std::mutex> lock(g_init_mu);
    if (g_shut) return set_error(FMLH_E_STATE, "library shut down (fmlh_shutdown); fmlh_init starts it again");
    if (g_ready) return FMLH_OK;
    arm_faults();
    return init_locked(0);
}

hipStream_t stream() { return g_stream; }
int cu_count() { return g_cus; }

}  // namespace fmlh

using namespace fmlh;

extern "C" {

int fmlh_init(int device) {
    std::lock_guard<std::mutex> lock(g_init_mu);
    g_shut = false;
    arm_faults();
    return init_locked(device);
}

int fmlh_shutdown(void) {
    {
        std::lock_guard<std::mutex> lock(g_init_mu);
        if (!g_ready) {
            g_shut = true;
            return FMLH_OK;
        }
    }
    int rc = FMLH_OK;
    if (hipStreamSynchronize(g_stream) != hipSuccess) rc = set_error(FMLH_E_HIP, "fmlh_shutdown: stream sync failed");
    destroy_all_engines();
    release_global_workspace();
    std::lock_guard<std::mutex> lock(g_init_mu);
    if (g_stream && hipStreamDestroy(g_stream) != hipSuccess && rc == FMLH_OK)
        rc = set_error(FMLH_E_HIP, "fmlh_shutdown: stream destroy failed");
    g_stream = nullptr;
    g_ready = false;
    g_shut = true;
    return rc;
}

int fmlh_device_info(char* arch, size_t arch_len, int* cus) {
    FMLH_TRY(ensure_init());
    if (arch && arch_len) std::snprintf(arch, arch_len, "%s", g_arch);
    if (cus) *cus = g_cus;
    return FMLH_OK;
}

const char* fmlh_last_error(void) { return g_error.c_str(); }

void* fmlh_get_stream(void) {
    if (ensure_init() != FMLH_OK) return nullptr;
    return reinterpret_cast<void*>(g_stream);
}

int fmlh_malloc(void** dptr, size_t bytes) {
    FMLH_REQUIRE(dptr != nullptr, "fmlh_malloc: null output pointer");
    FMLH_TRY(ensure_init());
    *dptr = nullptr;
    if (bytes == 0) bytes = 4;
    return device_malloc(dptr, bytes);
}

int fmlh_free(void* dptr) {
    if (!dptr) return FMLH_OK;
    FMLH_TRY(ensure_init());
    // Work already enqueued may still read the buffer.
    FMLH_HIP(hipStreamSynchronize(g_stream));
    FMLH_HIP(hipFree(dptr));
    return FMLH_OK;
}

int fmlh_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    FMLH_TRY(ensure_init());
    if (!bytes) return FMLH_OK;
    FMLH_REQUIRE(dst && src, "fmlh_memcpy_h2d: null pointer");
    FMLH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
    // Pageable source: the caller may reuse it as soon as we return.
    FMLH_HIP(hipStreamSynchronize(g_stream));
    return FMLH_OK;
}

int fmlh_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    FMLH_TRY(ensure_init());
    if (!bytes) return FMLH_OK;
    FMLH_REQUIRE(dst && src, "fmlh_memcpy_d2h: null pointer");
    FMLH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
    FMLH_HIP(hipStreamSynchronize(g_stream));
    return FMLH_OK;
}

int fmlh_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    FMLH_TRY(ensure_init());
    if (!bytes) return FMLH_OK;
    FMLH_REQUIRE(dst && src, "fmlh_memcpy_d2d: null pointer");
    FMLH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
    return FMLH_OK;
}

int fmlh_synchronize(void) {
    FMLH_TRY(ensure_init());
    FMLH_HIP(hipStreamSynchronize(g_stream));
    return FMLH_OK;
}

int fmlh_event_create(void** ev) {
    FMLH_REQUIRE(ev != nullptr, "fmlh_event_create: null output pointer");
    FMLH_TRY(ensure_init());
    hipEvent_t e;
    FMLH_HIP(hipEventCreate(&e));
    *ev = reinterpret_cast<void*>(e);
    return FMLH_OK;
}

int fmlh_event_destroy(void* ev) {
    if (!ev) return FMLH_OK;
    FMLH_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)));
    return FMLH_OK;
}

int fmlh_event_record(void* ev) {
    FMLH_REQUIRE(ev != nullptr, "fmlh_event_record: null event");
    FMLH_TRY(ensure_init());
    FMLH_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), g_stream));
    return FMLH_OK;
}

int fmlh_event_elapsed_ms(void* start, void* stop, float* ms) {
    FMLH_REQUIRE(start && stop && ms, "fmlh_event_elapsed_ms: null argument");
    FMLH_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)));
    FMLH_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                 reinterpret_cast<hipEvent_t>(stop)));
    return FMLH_OK;
}

}  // extern "C"

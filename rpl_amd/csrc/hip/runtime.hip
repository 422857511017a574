// Device bring-up, error reporting, memory, streams and events of the C ABI.
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.h"

namespace rplhip {

static thread_local char g_err[512] = "";
static pthread_once_t g_once = PTHREAD_ONCE_INIT;
static int g_init_status = RPLHIP_ERR_NO_DEVICE;
static char g_init_err[512] = "device not initialised";
static int g_cu_count = 0;
static int g_clock_khz = 0;
static char g_arch[64] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

static void init_once() {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        snprintf(g_init_err, sizeof(g_init_err), "no HIP device visible (%s)",
                 e != hipSuccess ? hipGetErrorString(e) : "count = 0");
        g_init_status = RPLHIP_ERR_NO_DEVICE;
        return;
    }
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, 0)) != hipSuccess) {
        snprintf(g_init_err, sizeof(g_init_err), "hipGetDeviceProperties: %s",
                 hipGetErrorString(e));
        g_init_status = RPLHIP_ERR_HIP;
        return;
    }
    snprintf(g_arch, sizeof(g_arch), "%s", prop.gcnArchName);
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        snprintf(g_init_err, sizeof(g_init_err),
                 "device 0 is %s; this build only carries gfx950 code", prop.gcnArchName);
        g_init_status = RPLHIP_ERR_NO_DEVICE;
        return;
    }
    if ((e = hipSetDevice(0)) != hipSuccess) {
        snprintf(g_init_err, sizeof(g_init_err), "hipSetDevice: %s", hipGetErrorString(e));
        g_init_status = RPLHIP_ERR_HIP;
        return;
    }
    g_cu_count = prop.multiProcessorCount;
    g_clock_khz = prop.clockRate;
    g_init_status = RPLHIP_OK;
}

int ensure_device() {
    pthread_once(&g_once, init_once);
    if (g_init_status != RPLHIP_OK) return fail(g_init_status, "%s", g_init_err);
    // hipSetDevice is per host thread.
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != 0) {
        hipError_t e = hipSetDevice(0);
        if (e != hipSuccess) return fail(RPLHIP_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(e));
    }
    return RPLHIP_OK;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(RPLHIP_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
    return RPLHIP_OK;
}

int ws_alloc(void** p, size_t bytes, hipStream_t stream) {
    *p = nullptr;
    if (bytes == 0) return RPLHIP_OK;
    hipError_t e = hipMallocAsync(p, bytes, stream);
    if (e != hipSuccess) {
        *p = nullptr;
        return fail(RPLHIP_ERR_NOMEM, "workspace of %zu bytes: %s", bytes, hipGetErrorString(e));
    }
    return RPLHIP_OK;
}

void ws_free(void* p, hipStream_t stream) {
    if (p) (void)hipFreeAsync(p, stream);
}

int cu_count() { return g_cu_count > 0 ? g_cu_count : 256; }

}  // namespace rplhip

using namespace rplhip;

extern "C" {

int rplhip_init(void) { return ensure_device(); }

const char* rplhip_last_error(void) { return g_err; }

int rplhip_device_info(char* arch, size_t arch_len, int* cus, int* clock_khz) {
    RPLHIP_REQUIRE_DEVICE();
    if (arch && arch_len) snprintf(arch, arch_len, "%s", g_arch);
    if (cus) *cus = g_cu_count;
    if (clock_khz) *clock_khz = g_clock_khz;
    return RPLHIP_OK;
}

int rplhip_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(RPLHIP_ERR_INVALID, "rplhip_malloc: ptr is NULL");
    *ptr = nullptr;
    RPLHIP_REQUIRE_DEVICE();
    if (bytes == 0) return RPLHIP_OK;
    hipError_t e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) {
        *ptr = nullptr;
        return fail(RPLHIP_ERR_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    return RPLHIP_OK;
}

int rplhip_free(void* ptr) {
    if (!ptr) return RPLHIP_OK;
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipFree(ptr));
    return RPLHIP_OK;
}

int rplhip_memcpy_htod(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return RPLHIP_OK;
    if (!dst || !src) return fail(RPLHIP_ERR_INVALID, "rplhip_memcpy_htod: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return RPLHIP_OK;
}

int rplhip_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return RPLHIP_OK;
    if (!dst || !src) return fail(RPLHIP_ERR_INVALID, "rplhip_memcpy_dtoh: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return RPLHIP_OK;
}

int rplhip_memcpy_dtod(void* dst, const void* src, size_t bytes, rplhip_stream_t s) {
    if (bytes == 0) return RPLHIP_OK;
    if (!dst || !src) return fail(RPLHIP_ERR_INVALID, "rplhip_memcpy_dtod: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(s)));
    return RPLHIP_OK;
}

int rplhip_memset(void* ptr, int value, size_t bytes, rplhip_stream_t s) {
    if (bytes == 0) return RPLHIP_OK;
    if (!ptr) return fail(RPLHIP_ERR_INVALID, "rplhip_memset: NULL pointer");
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipMemsetAsync(ptr, value, bytes, as_stream(s)));
    return RPLHIP_OK;
}

int rplhip_synchronize(void) {
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipDeviceSynchronize());
    return RPLHIP_OK;
}

int rplhip_stream_create(rplhip_stream_t* s) {
    if (!s) return fail(RPLHIP_ERR_INVALID, "rplhip_stream_create: NULL");
    RPLHIP_REQUIRE_DEVICE();
    hipStream_t h;
    RPLHIP_CHECK(hipStreamCreateWithFlags(&h, hipStreamNonBlocking));
    *s = h;
    return RPLHIP_OK;
}

int rplhip_stream_destroy(rplhip_stream_t s) {
    if (!s) return RPLHIP_OK;
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipStreamDestroy(as_stream(s)));
    return RPLHIP_OK;
}

int rplhip_stream_synchronize(rplhip_stream_t s) {
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipStreamSynchronize(as_stream(s)));
    return RPLHIP_OK;
}

int rplhip_event_create(rplhip_event_t* ev) {
    if (!ev) return fail(RPLHIP_ERR_INVALID, "rplhip_event_create: NULL");
    RPLHIP_REQUIRE_DEVICE();
    hipEvent_t h;
    RPLHIP_CHECK(hipEventCreate(&h));
    *ev = h;
    return RPLHIP_OK;
}

int rplhip_event_destroy(rplhip_event_t ev) {
    if (!ev) return RPLHIP_OK;
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)));
    return RPLHIP_OK;
}

int rplhip_event_record(rplhip_event_t ev, rplhip_stream_t s) {
    if (!ev) return fail(RPLHIP_ERR_INVALID, "rplhip_event_record: NULL event");
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), as_stream(s)));
    return RPLHIP_OK;
}

int rplhip_event_synchronize(rplhip_event_t ev) {
    if (!ev) return fail(RPLHIP_ERR_INVALID, "rplhip_event_synchronize: NULL event");
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipEventSynchronize(reinterpret_cast<hipEvent_t>(ev)));
    return RPLHIP_OK;
}

int rplhip_event_elapsed_ms(float* ms, rplhip_event_t a, rplhip_event_t b) {
    if (!ms || !a || !b) return fail(RPLHIP_ERR_INVALID, "rplhip_event_elapsed_ms: NULL");
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(a),
                                     reinterpret_cast<hipEvent_t>(b)));
    return RPLHIP_OK;
}

}  // extern "C"

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

// ---------------------------------------------------------------- workspaces
//
// Temporary device memory of one call (split-K partials, reduction partials,
// the transposed B of gemm_int8).  hipMallocAsync/hipFreeAsync cost 10-25 us
// each on the host, which dominated small training steps, so blocks are
// cached instead.  A block released on stream S is handed out again only to
// a later request on S: stream order then runs the new user's kernels after
// the old user's.  Blocks are given back to HIP only after a device-wide
// synchronisation (trim), so no kernel can still be using them.
struct WsBlock {
    void* p;
    size_t bytes;        // size class (see ws_class)
    hipStream_t stream;  // stream of the last user
    bool idle;           // true: no queued work uses it; any stream may take it
    bool in_use;
};
static pthread_mutex_t g_ws_mu = PTHREAD_MUTEX_INITIALIZER;
static WsBlock* g_ws;
static size_t g_ws_len, g_ws_cap, g_ws_cached;
// Cached bytes above which unused blocks are returned before a new one is made.
constexpr size_t kWsRetainBytes = size_t(4) << 30;

// Four size classes per power of two (<= 25% slack), at least 256 B.
static size_t ws_class(size_t b) {
    if (b <= 256) return 256;
    int lg = 63 - __builtin_clzll((unsigned long long)(b - 1));
    size_t step = size_t(1) << (lg - 2);
    return (b + step - 1) / step * step;
}

// Free every unused block; the caller holds g_ws_mu.  Synchronises the device.
static void ws_trim_locked() {
    bool any = false;
    for (size_t i = 0; i < g_ws_len; i++) any |= !g_ws[i].in_use;
    if (!any) return;
    if (hipDeviceSynchronize() != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    size_t j = 0;
    for (size_t i = 0; i < g_ws_len; i++) {
        if (g_ws[i].in_use) {
            g_ws[j++] = g_ws[i];
        } else {
            (void)hipFree(g_ws[i].p);
            g_ws_cached -= g_ws[i].bytes;
        }
    }
    g_ws_len = j;
}

static void ws_trim() {
    pthread_mutex_lock(&g_ws_mu);
    ws_trim_locked();
    pthread_mutex_unlock(&g_ws_mu);
}

int ws_alloc(void** p, size_t bytes, hipStream_t stream) {
    *p = nullptr;
    if (bytes == 0) return RPLHIP_OK;
    const size_t cls = ws_class(bytes);
    pthread_mutex_lock(&g_ws_mu);
    for (size_t i = 0; i < g_ws_len; i++) {
        WsBlock& b = g_ws[i];
        if (!b.in_use && b.bytes == cls && (b.idle || b.stream == stream)) {
            b.in_use = true;
            b.idle = false;
            b.stream = stream;
            *p = b.p;
            pthread_mutex_unlock(&g_ws_mu);
            return RPLHIP_OK;
        }
    }
    if (g_ws_cached + cls > kWsRetainBytes) ws_trim_locked();
    if (g_ws_len == g_ws_cap) {
        size_t nc = g_ws_cap ? 2 * g_ws_cap : 32;
        WsBlock* nb = (WsBlock*)realloc(g_ws, nc * sizeof(WsBlock));
        if (!nb) {
            pthread_mutex_unlock(&g_ws_mu);
            return fail(RPLHIP_ERR_NOMEM, "workspace table of %zu entries", nc);
        }
        g_ws = nb;
        g_ws_cap = nc;
    }
    void* q = nullptr;
    hipError_t e = hipMalloc(&q, cls);
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();
        ws_trim_locked();
        e = hipMalloc(&q, cls);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        pthread_mutex_unlock(&g_ws_mu);
        return fail(RPLHIP_ERR_NOMEM, "workspace of %zu bytes: %s", bytes, hipGetErrorString(e));
    }
    g_ws[g_ws_len++] = WsBlock{q, cls, stream, false, true};
    g_ws_cached += cls;
    *p = q;
    pthread_mutex_unlock(&g_ws_mu);
    return RPLHIP_OK;
}

void ws_free(void* p, hipStream_t stream) {
    if (!p) return;
    pthread_mutex_lock(&g_ws_mu);
    for (size_t i = 0; i < g_ws_len; i++) {
        if (g_ws[i].p == p) {
            g_ws[i].in_use = false;
            g_ws[i].stream = stream;
            break;
        }
    }
    pthread_mutex_unlock(&g_ws_mu);
}

// `s` has no queued work left (all = every stream): its unused blocks may go
// to any stream.
static void ws_stream_idle(hipStream_t s, bool all = false) {
    pthread_mutex_lock(&g_ws_mu);
    for (size_t i = 0; i < g_ws_len; i++)
        if (!g_ws[i].in_use && (all || g_ws[i].stream == s)) g_ws[i].idle = true;
    pthread_mutex_unlock(&g_ws_mu);
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
    if (e == hipErrorOutOfMemory) {
        // Give the cached workspaces back first.
        (void)hipGetLastError();
        ws_trim();
        e = hipMalloc(ptr, bytes);
    }
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
    ws_stream_idle(nullptr, true);
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
    // Drain it first so the workspaces it used are free for other streams
    // (a later stream may be given the same handle).
    RPLHIP_CHECK(hipStreamSynchronize(as_stream(s)));
    ws_stream_idle(as_stream(s));
    RPLHIP_CHECK(hipStreamDestroy(as_stream(s)));
    return RPLHIP_OK;
}

int rplhip_stream_synchronize(rplhip_stream_t s) {
    RPLHIP_REQUIRE_DEVICE();
    RPLHIP_CHECK(hipStreamSynchronize(as_stream(s)));
    ws_stream_idle(as_stream(s));
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

/*
 * Host-only stress test of the device-buffer registry and pool
 * (rpl_amd/csrc/host/rpl_runtime.c) under ThreadSanitizer or
 * AddressSanitizer + UBSan, built by tests/test_host_sanitizers.py with gcc.
 *
 * The rplhip_* device calls the runtime makes are replaced by host stand-ins
 * (malloc, memcpy, memset), so the registry's locking, handle reuse, chunk
 * growth and gradient attachment run exactly as in the library, with no GPU.
 * Eight threads each keep up to kLive tensors resident at once (together
 * more than one 1024-entry chunk of handles), and create, upload, read,
 * attach gradients to, fill, download and free them in a pseudo-random
 * order; every downloaded value is checked.  Exit status 0 = all checks
 * passed; the sanitizers report data races or memory errors on stderr and
 * make the exit status non-zero.
 */
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "rpl_host.h"

/* ------------------------------------------------ host stand-ins for rplhip */

int rplhip_init(void) { return RPLHIP_OK; }
const char* rplhip_last_error(void) { return "stand-in"; }
int rplhip_malloc(void** ptr, size_t bytes) {
    *ptr = malloc(bytes ? bytes : 1);
    return *ptr ? RPLHIP_OK : RPLHIP_ERR_NOMEM;
}
int rplhip_free(void* ptr) {
    free(ptr);
    return RPLHIP_OK;
}
int rplhip_memcpy_htod(void* dst, const void* src, size_t bytes) {
    memcpy(dst, src, bytes);
    return RPLHIP_OK;
}
int rplhip_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    memcpy(dst, src, bytes);
    return RPLHIP_OK;
}
int rplhip_memset(void* ptr, int value, size_t bytes, rplhip_stream_t stream) {
    (void)stream;
    memset(ptr, value, bytes);
    return RPLHIP_OK;
}
int rplhip_fill(float* x, uint64_t n, float value, rplhip_stream_t stream) {
    (void)stream;
    for (uint64_t i = 0; i < n; i++) x[i] = value;
    return RPLHIP_OK;
}
int rplhip_synchronize(void) { return RPLHIP_OK; }

/* ------------------------------------------------------------------ driver */

enum { kThreads = 8, kLive = 256, kIters = 6000 };

static int g_failures;
static pthread_mutex_t g_fail_mu = PTHREAD_MUTEX_INITIALIZER;

static void failure(const char* what, int tid, int it) {
    pthread_mutex_lock(&g_fail_mu);
    if (g_failures++ < 10) fprintf(stderr, "thread %d iteration %d: %s\n", tid, it, what);
    pthread_mutex_unlock(&g_fail_mu);
}

static uint64_t next(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static void* worker(void* arg) {
    const int tid = (int)(intptr_t)arg;
    Tensor* live[kLive] = {0};
    float tag[kLive] = {0};
    uint64_t rng = 0x52504C00u + (uint64_t)tid;
    for (int it = 0; it < kIters; it++) {
        const int i = (int)(next(&rng) % kLive);
        if (!live[i]) {
            uint32_t shape[2] = {1 + (uint32_t)(next(&rng) % 7), 1 + (uint32_t)(next(&rng) % 9)};
            Tensor* t = tensor_create(2, shape, (next(&rng) & 1) != 0);
            if (!t) {
                failure("tensor_create", tid, it);
                continue;
            }
            tag[i] = (float)(tid * 100000 + it);
            for (uint32_t k = 0; k < t->size; k++) t->data[k] = tag[i] + (float)k;
            tensor_to_gpu(t);
            if (!rpl__is_gpu(t)) failure("tensor_to_gpu", tid, it);
            live[i] = t;
            continue;
        }
        Tensor* t = live[i];
        switch (next(&rng) % 4) {
            case 0: { /* download and check the uploaded values */
                memset(t->data, 0, (size_t)t->size * sizeof(float));
                tensor_from_gpu(t);
                for (uint32_t k = 0; k < t->size; k++)
                    if (t->data[k] != tag[i] + (float)k) {
                        failure("downloaded value", tid, it);
                        break;
                    }
                break;
            }
            case 1: { /* a device gradient, attached once, zero until filled */
                if (!t->grad) t->grad = (float*)rpitorch_aligned_alloc(64, (size_t)t->size * sizeof(float));
                if (!rpl__attach_grad(t) || !rpl__dev_grad(t)) failure("attach_grad", tid, it);
                if (!rpl__attach_grad(t)) failure("attach_grad again", tid, it);
                break;
            }
            case 2: { /* fill host and device copies */
                tag[i] = (float)(-tid * 1000 - it % 1000);
                tensor_fill(t, tag[i]);
                float* d = rpl__dev_data(t);
                if (!d) failure("dev_data", tid, it);
                else
                    for (uint32_t k = 0; k < t->size; k++) d[k] = tag[i] + (float)k;
                break;
            }
            default: /* release */
                tensor_free(t);
                live[i] = NULL;
        }
    }
    for (int i = 0; i < kLive; i++) tensor_free(live[i]);
    return NULL;
}

int main(void) {
    pthread_t th[kThreads];
    for (int t = 0; t < kThreads; t++) pthread_create(&th[t], NULL, worker, (void*)(intptr_t)t);
    for (int t = 0; t < kThreads; t++) pthread_join(th[t], NULL);
    rpl__pool_release_all();
    if (g_failures) {
        fprintf(stderr, "%d failures\n", g_failures);
        return 1;
    }
    printf("registry stress: %d threads x %d iterations OK\n", kThreads, kIters);
    return 0;
}

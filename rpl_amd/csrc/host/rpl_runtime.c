/*
 * Tensor memory, the device-buffer registry behind Tensor.gpu_buffer, the
 * staging of host tensors, and the device seam of include/rpl.h
 * (rpl_gpu_init / tensor_to_gpu / tensor_from_gpu, src/rpl_gpu.c:88-230).
 */
#define _GNU_SOURCE
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "rpl_host.h"

/* ------------------------------------------------------------ errors */

static __thread char g_last_error[512];

const char* rpl_last_error(void) { return g_last_error; }
void rpl_clear_last_error(void) { g_last_error[0] = '\0'; }

int rpl__ok(int st, const char* what) {
    if (st == RPLHIP_OK) return 1;
    snprintf(g_last_error, sizeof(g_last_error), "%s: %s", what, rplhip_last_error());
    fprintf(stderr, "rpl: %s\n", g_last_error);
    return 0;
}

int rpl__bad(const char* what, const char* fmt, ...) {
    char msg[400];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof(msg), fmt, ap);
    va_end(ap);
    snprintf(g_last_error, sizeof(g_last_error), "%s: %s", what, msg);
    fprintf(stderr, "rpl: %s\n", g_last_error);
    return 0;
}

/* ------------------------------------------------------- device pool */

typedef struct {
    void* p;
    size_t bytes;
} PoolBlock;

static pthread_mutex_t g_pool_mu = PTHREAD_MUTEX_INITIALIZER;
static PoolBlock* g_pool;
static size_t g_pool_len, g_pool_cap;

static size_t pool_round(size_t b) { return (b + 255) & ~(size_t)255; }

void* rpl__pool_alloc(size_t bytes) {
    if (bytes == 0) bytes = 1;
    bytes = pool_round(bytes);
    pthread_mutex_lock(&g_pool_mu);
    for (size_t i = 0; i < g_pool_len; i++) {
        if (g_pool[i].bytes == bytes) {
            void* p = g_pool[i].p;
            g_pool[i] = g_pool[--g_pool_len];
            pthread_mutex_unlock(&g_pool_mu);
            return p;
        }
    }
    pthread_mutex_unlock(&g_pool_mu);
    void* p = NULL;
    if (rplhip_malloc(&p, bytes) != RPLHIP_OK) {
        /* Release cached blocks and retry once. */
        rplhip_synchronize();
        rpl__pool_release_all();
        if (!rpl__ok(rplhip_malloc(&p, bytes), "device allocation")) return NULL;
    }
    return p;
}

void rpl__pool_free(void* p, size_t bytes) {
    if (!p) return;
    bytes = pool_round(bytes ? bytes : 1);
    pthread_mutex_lock(&g_pool_mu);
    if (g_pool_len == g_pool_cap) {
        size_t nc = g_pool_cap ? 2 * g_pool_cap : 64;
        PoolBlock* nb = (PoolBlock*)realloc(g_pool, nc * sizeof(PoolBlock));
        if (!nb) {
            pthread_mutex_unlock(&g_pool_mu);
            rplhip_free(p);
            return;
        }
        g_pool = nb;
        g_pool_cap = nc;
    }
    g_pool[g_pool_len].p = p;
    g_pool[g_pool_len].bytes = bytes;
    g_pool_len++;
    pthread_mutex_unlock(&g_pool_mu);
}

void rpl__pool_release_all(void) {
    pthread_mutex_lock(&g_pool_mu);
    for (size_t i = 0; i < g_pool_len; i++) rplhip_free(g_pool[i].p);
    g_pool_len = 0;
    pthread_mutex_unlock(&g_pool_mu);
}

/* ------------------------------------------------ device-buffer registry */

/* Handles index entries held in fixed chunks of kRegChunk that are allocated
 * once and never move or shrink, so a handle always names the same slot.
 * Every field is read and written under g_reg_mu, and readers get copies:
 * no pointer into the table escapes the lock, so a concurrent
 * tensor_to_gpu (which may add a chunk) or tensor_free cannot leave another
 * thread with a dangling entry. */
typedef struct {
    float* data;
    float* grad;
    size_t bytes;
    int used;
    int grad_lazy;  /* the device gradient holds grad_val everywhere, not yet written (contents undefined) */
    float grad_val;
} RegEntry;

enum { kRegChunkBits = 10, kRegChunk = 1 << kRegChunkBits, kRegMaxChunks = 4096 };

static pthread_mutex_t g_reg_mu = PTHREAD_MUTEX_INITIALIZER;
static RegEntry* g_reg_chunks[kRegMaxChunks];
static uint32_t g_reg_len; /* slots handed out so far (handles 1..g_reg_len) */

/* Slot of handle h (caller holds g_reg_mu), or NULL for an invalid handle. */
static RegEntry* reg_slot(uint32_t h) {
    if (h < 1 || h > g_reg_len) return NULL;
    RegEntry* e = &g_reg_chunks[(h - 1) >> kRegChunkBits][(h - 1) & (kRegChunk - 1)];
    return e->used ? e : NULL;
}

/* Copy of handle h's entry; returns 0 (and a zeroed *out) if it is not live. */
static int reg_read(uint32_t h, RegEntry* out) {
    pthread_mutex_lock(&g_reg_mu);
    const RegEntry* e = reg_slot(h);
    if (e) *out = *e;
    pthread_mutex_unlock(&g_reg_mu);
    if (!e) memset(out, 0, sizeof(*out));
    return e != NULL;
}

static uint32_t reg_new(float* data, float* grad, size_t bytes, int grad_zero) {
    pthread_mutex_lock(&g_reg_mu);
    uint32_t h = 0;
    for (uint32_t i = 0; i < g_reg_len; i++)
        if (!g_reg_chunks[i >> kRegChunkBits][i & (kRegChunk - 1)].used) {
            h = i + 1;
            break;
        }
    if (!h) {
        const uint32_t c = g_reg_len >> kRegChunkBits;
        if (c == kRegMaxChunks) {
            pthread_mutex_unlock(&g_reg_mu);
            return 0;
        }
        if (!g_reg_chunks[c]) {
            g_reg_chunks[c] = (RegEntry*)calloc(kRegChunk, sizeof(RegEntry));
            if (!g_reg_chunks[c]) {
                pthread_mutex_unlock(&g_reg_mu);
                return 0;
            }
        }
        h = ++g_reg_len;
    }
    RegEntry* e = &g_reg_chunks[(h - 1) >> kRegChunkBits][(h - 1) & (kRegChunk - 1)];
    e->data = data;
    e->grad = grad;
    e->bytes = bytes;
    e->used = 1;
    e->grad_lazy = grad_zero;
    e->grad_val = 0.0f;
    pthread_mutex_unlock(&g_reg_mu);
    return h;
}

/* Retire handle h and return its buffers to the pool.  The entry is taken
 * out of the table under the lock, so exactly one caller frees them. */
static void reg_release(uint32_t h) {
    RegEntry copy = {0};
    pthread_mutex_lock(&g_reg_mu);
    RegEntry* e = reg_slot(h);
    if (e) {
        copy = *e;
        e->used = 0;
        e->data = e->grad = NULL;
    }
    pthread_mutex_unlock(&g_reg_mu);
    if (!copy.used) return;
    rpl__pool_free(copy.data, copy.bytes);
    if (copy.grad) rpl__pool_free(copy.grad, copy.bytes);
}

static int reg_read_tensor(const Tensor* t, RegEntry* out) {
    if (!t || t->device != DEVICE_GPU) {
        memset(out, 0, sizeof(*out));
        return 0;
    }
    return reg_read(t->gpu_buffer, out);
}

int rpl__is_gpu(const Tensor* t) {
    RegEntry e;
    return reg_read_tensor(t, &e);
}

float* rpl__dev_data(const Tensor* t) {
    RegEntry e;
    reg_read_tensor(t, &e);
    return e.data;
}

float* rpl__dev_grad(const Tensor* t) {
    RegEntry e;
    reg_read_tensor(t, &e);
    return e.grad;
}

int rpl__attach(Tensor* t, int upload) {
    if (rpl__is_gpu(t)) return 1;
    size_t bytes = (size_t)t->size * sizeof(float);
    float* d = (float*)rpl__pool_alloc(bytes);
    if (!d) return 0;
    float* g = NULL;
    if (t->grad) {
        /* A new output's gradient starts as zero: recorded, not written. */
        g = (float*)rpl__pool_alloc(bytes);
        if (!g || (upload && !rpl__ok(rplhip_memcpy_htod(g, t->grad, bytes), "tensor grad to device"))) {
            rpl__pool_free(d, bytes);
            if (g) rpl__pool_free(g, bytes);
            return 0;
        }
    }
    if (upload && !rpl__ok(rplhip_memcpy_htod(d, t->data, bytes), "tensor to device")) {
        rpl__pool_free(d, bytes);
        if (g) rpl__pool_free(g, bytes);
        return 0;
    }
    uint32_t h = reg_new(d, g, bytes, g && !upload);
    if (!h) {
        rpl__pool_free(d, bytes);
        if (g) rpl__pool_free(g, bytes);
        return rpl__bad("tensor_to_gpu", "registry allocation failed");
    }
    t->gpu_buffer = h;
    t->device = DEVICE_GPU;
    return 1;
}

int rpl__attach_grad(Tensor* t) {
    RegEntry e;
    if (!reg_read_tensor(t, &e)) return 0;
    if (e.grad) return 1;
    float* g = (float*)rpl__pool_alloc(e.bytes);
    if (!g) return 0;
    /* Install by handle under the lock (as zero, not yet written); if another
     * thread installed one (or released the tensor) meanwhile, keep the
     * table as it is. */
    int installed = 0, live = 0;
    pthread_mutex_lock(&g_reg_mu);
    RegEntry* s = reg_slot(t->gpu_buffer);
    if (s) {
        live = 1;
        if (!s->grad) {
            s->grad = g;
            s->grad_lazy = 1;
            s->grad_val = 0.0f;
            installed = 1;
        }
    }
    pthread_mutex_unlock(&g_reg_mu);
    if (!installed) rpl__pool_free(g, e.bytes);
    return live;
}

/* Test and clear the zero mark of t's device gradient: 1 if it was +0.0
 * only logically -- the caller then writes every element (as 0 + x).  A
 * gradient marked with another value keeps its mark (0 returned). */
int rpl__grad_take_zero(const Tensor* t) {
    if (!t || t->device != DEVICE_GPU) return 0;
    int was = 0;
    pthread_mutex_lock(&g_reg_mu);
    RegEntry* e = reg_slot(t->gpu_buffer);
    if (e && e->grad && e->grad_lazy) {
        uint32_t bits;
        memcpy(&bits, &e->grad_val, 4);
        if (bits == 0) {
            was = 1;
            e->grad_lazy = 0;
        }
    }
    pthread_mutex_unlock(&g_reg_mu);
    return was;
}

/* Mark t's device gradient as holding v everywhere, without writing it
 * (tensor_zero_grad: 0; tensor_backward's root: 1). */
void rpl__grad_set_value(const Tensor* t, float v) {
    if (!t || t->device != DEVICE_GPU) return;
    pthread_mutex_lock(&g_reg_mu);
    RegEntry* e = reg_slot(t->gpu_buffer);
    if (e && e->grad) {
        e->grad_lazy = 1;
        e->grad_val = v;
    }
    pthread_mutex_unlock(&g_reg_mu);
}

void rpl__grad_set_zero(const Tensor* t) { rpl__grad_set_value(t, 0.0f); }

/* 1 (and *v) when t's device gradient holds one value only logically; the
 * mark is kept. */
int rpl__grad_lazy_value(const Tensor* t, float* v) {
    if (!t || t->device != DEVICE_GPU) return 0;
    int lazy = 0;
    pthread_mutex_lock(&g_reg_mu);
    RegEntry* e = reg_slot(t->gpu_buffer);
    if (e && e->grad && e->grad_lazy) {
        lazy = 1;
        *v = e->grad_val;
    }
    pthread_mutex_unlock(&g_reg_mu);
    return lazy;
}

/* Write a marked gradient's value into every element and clear the mark.
 * 0 on a failed fill. */
static int grad_materialize(const Tensor* t, float* g) {
    float v;
    if (!rpl__grad_lazy_value(t, &v)) return 1;
    if (!rpl__ok(rplhip_fill(g, t->size, v, NULL), "device gradient")) return 0;
    pthread_mutex_lock(&g_reg_mu);
    RegEntry* e = reg_slot(t->gpu_buffer);
    if (e) e->grad_lazy = 0;
    pthread_mutex_unlock(&g_reg_mu);
    return 1;
}

/* t's device gradient with its values in memory: a marked gradient is
 * filled first.  NULL if t has none. */
float* rpl__dev_grad_ready(const Tensor* t) {
    float* g = rpl__dev_grad(t);
    if (g && !grad_materialize(t, g)) return NULL;
    return g;
}

/* ---------------------------------------------------------------- staging */

void* rpl__stage_host(RplStage* s, void* host, size_t bytes, int upload, int writeback) {
    if (s->err) return NULL;
    if (s->n == RPL_STAGE_MAX) {
        s->err = 1;
        rpl__bad("staging", "too many staged buffers");
        return NULL;
    }
    void* d = rpl__pool_alloc(bytes);
    if (!d) {
        s->err = 1;
        return NULL;
    }
    if (upload && bytes && !rpl__ok(rplhip_memcpy_htod(d, host, bytes), "host to device copy")) {
        rpl__pool_free(d, bytes);
        s->err = 1;
        return NULL;
    }
    s->e[s->n].dev = d;
    s->e[s->n].host = host;
    s->e[s->n].bytes = bytes;
    s->e[s->n].writeback = writeback;
    s->n++;
    return d;
}

float* rpl__view_data(RplStage* s, const Tensor* t, int upload, int writeback) {
    if (s->err) return NULL;
    float* d = rpl__dev_data(t);
    if (d) return d;
    return (float*)rpl__stage_host(s, t->data, (size_t)t->size * sizeof(float), upload, writeback);
}

float* rpl__view_grad(RplStage* s, const Tensor* t, int upload, int writeback) {
    if (s->err) return NULL;
    if (rpl__is_gpu(t)) {
        float* g = rpl__dev_grad_ready(t);
        if (!g) {
            s->err = 1;
            rpl__bad("autograd", "GPU tensor has no device gradient");
        }
        return g;
    }
    return (float*)rpl__stage_host(s, t->grad, (size_t)t->size * sizeof(float), upload, writeback);
}

float* rpl__view_grad_acc(RplStage* s, const Tensor* t, int* overwrite) {
    *overwrite = 0;
    if (s->err) return NULL;
    if (rpl__is_gpu(t)) {
        float* g = rpl__dev_grad(t);
        if (!g) {
            s->err = 1;
            rpl__bad("autograd", "GPU tensor has no device gradient");
            return NULL;
        }
        /* A zero mark becomes an overwrite; another value is written out
         * first and then accumulated into. */
        *overwrite = rpl__grad_take_zero(t);
        if (!*overwrite && !grad_materialize(t, g)) {
            s->err = 1;
            return NULL;
        }
        return g;
    }
    return (float*)rpl__stage_host(s, t->grad, (size_t)t->size * sizeof(float), 1, 1);
}

int rpl__stage_finish(RplStage* s) {
    int ok = !s->err;
    int any_wb = 0;
    for (int i = 0; i < s->n; i++) any_wb |= s->e[i].writeback;
    if (ok && any_wb) {
        for (int i = 0; i < s->n && ok; i++)
            if (s->e[i].writeback && s->e[i].bytes)
                ok = rpl__ok(rplhip_memcpy_dtoh(s->e[i].host, s->e[i].dev, s->e[i].bytes), "device to host copy");
    }
    for (int i = 0; i < s->n; i++) rpl__pool_free(s->e[i].dev, s->e[i].bytes);
    s->n = 0;
    return ok;
}

/* ----------------------------------------------------------- Tensor memory */

/* src/rpl_core.c:33-41 */
void* rpitorch_aligned_alloc(size_t alignment, size_t size) {
    void* p = NULL;
    if (posix_memalign(&p, alignment, size ? size : 1) != 0) return NULL;
    return p;
}

void rpitorch_aligned_free(void* ptr) { free(ptr); }

static Tensor* tensor_create_impl(uint32_t dims, const uint32_t* shape, bool requires_grad, int zero_grad);

/* src/rpl_core.c:43-70 */
Tensor* tensor_create(uint32_t dims, const uint32_t* shape, bool requires_grad) {
    return tensor_create_impl(dims, shape, requires_grad, 1);
}

/* An op's output that is about to become GPU-resident: the host buffers are
 * allocated (tensor_from_gpu fills them) but the host gradient is not
 * zeroed -- while a tensor is GPU-resident its host copies are stale by
 * definition, and its device gradient is zeroed by rpl__attach. */
Tensor* rpl__tensor_create_gpu(uint32_t dims, const uint32_t* shape, bool requires_grad) {
    return tensor_create_impl(dims, shape, requires_grad, 0);
}

static Tensor* tensor_create_impl(uint32_t dims, const uint32_t* shape, bool requires_grad, int zero_grad) {
    Tensor* t = (Tensor*)calloc(1, sizeof(Tensor));
    if (!t) return NULL;
    if (dims > MAX_DIMS) {
        free(t);
        rpl__bad("tensor_create", "dims %u > MAX_DIMS", dims);
        return NULL;
    }
    t->dims = dims;
    t->size = 1;
    for (uint32_t i = 0; i < dims; i++) {
        t->shape[i] = shape[i];
        t->size *= shape[i];
    }
    if (dims) {
        t->strides[dims - 1] = 1;
        for (int i = (int)dims - 2; i >= 0; i--) t->strides[i] = t->strides[i + 1] * t->shape[i + 1];
    }
    size_t bytes = (size_t)t->size * sizeof(float);
    t->_allocation = rpitorch_aligned_alloc(64, bytes);
    t->_alloc_size = bytes;
    t->data = (float*)t->_allocation;
    if (requires_grad) {
        t->grad = (float*)rpitorch_aligned_alloc(64, bytes);
        if (t->grad && zero_grad) memset(t->grad, 0, bytes);
    }
    t->requires_grad = requires_grad;
    t->is_leaf = true;
    return t;
}

/* ------------------------------------------- internal graph tensors */

/* linear_forward's intermediate GEMM output is never freed by the reference
 * (src/rpl_nn.c:73-74): only the returned tensor points at it.  Its host
 * memory leaks as there; its device buffers are released when the tensor
 * that owns it is freed, so a training loop does not grow device memory. */
typedef struct {
    const Tensor* owner;
    Tensor* internal;
} Adopted;

static pthread_mutex_t g_adopt_mu = PTHREAD_MUTEX_INITIALIZER;
static Adopted* g_adopt;
static size_t g_adopt_len, g_adopt_cap;

void rpl__adopt(const Tensor* owner, Tensor* internal) {
    if (!owner || !internal || !rpl__is_gpu(internal)) return;
    pthread_mutex_lock(&g_adopt_mu);
    if (g_adopt_len == g_adopt_cap) {
        size_t nc = g_adopt_cap ? 2 * g_adopt_cap : 64;
        Adopted* na = (Adopted*)realloc(g_adopt, nc * sizeof(Adopted));
        if (!na) {
            pthread_mutex_unlock(&g_adopt_mu);
            return; /* keeps the device buffers, like the host ones */
        }
        g_adopt = na;
        g_adopt_cap = nc;
    }
    g_adopt[g_adopt_len].owner = owner;
    g_adopt[g_adopt_len].internal = internal;
    g_adopt_len++;
    pthread_mutex_unlock(&g_adopt_mu);
}

static void release_adopted(const Tensor* owner) {
    pthread_mutex_lock(&g_adopt_mu);
    for (size_t i = 0; i < g_adopt_len;) {
        if (g_adopt[i].owner == owner) {
            Tensor* in = g_adopt[i].internal;
            g_adopt[i] = g_adopt[--g_adopt_len];
            pthread_mutex_unlock(&g_adopt_mu);
            if (in->device == DEVICE_GPU && in->gpu_buffer) reg_release(in->gpu_buffer);
            in->device = DEVICE_CPU;
            in->gpu_buffer = 0;
            pthread_mutex_lock(&g_adopt_mu);
        } else {
            i++;
        }
    }
    pthread_mutex_unlock(&g_adopt_mu);
}

/* src/rpl_core.c:72-77, plus the device buffers */
void tensor_free(Tensor* t) {
    if (!t) return;
    if (t->device == DEVICE_GPU && t->gpu_buffer) reg_release(t->gpu_buffer);
    release_adopted(t);
    free(t->_allocation);
    free(t->grad);
    free(t);
}

/* src/rpl_core.c:83-86 (the device copy too when GPU-resident) */
void tensor_fill(Tensor* t, float value) {
    if (!t) return;
    for (uint32_t i = 0; i < t->size; i++) t->data[i] = value;
    float* d = rpl__dev_data(t);
    if (d) rpl__ok(rplhip_fill(d, t->size, value, NULL), "tensor_fill");
}

/* ------------------------------------------------------------ device seam */

bool rpl_gpu_init(void) { return rpl__ok(rplhip_init(), "rpl_gpu_init"); }

void rpl_gpu_shutdown(void) {
    if (rplhip_init() != RPLHIP_OK) return;
    rplhip_synchronize();
    rpl__pool_release_all();
}

void rpl_gpu_synchronize(void) { rpl__ok(rplhip_synchronize(), "rpl_gpu_synchronize"); }

void* rpl_gpu_stream(void) { return NULL; }

float* rpl_tensor_device_data(const Tensor* t) { return rpl__dev_data(t); }
float* rpl_tensor_device_grad(const Tensor* t) { return rpl__dev_grad_ready(t); }

/* src/rpl_gpu.c:201-214: upload and mark GPU-resident (no-op if already). */
void tensor_to_gpu(Tensor* t) {
    if (!t || rpl__is_gpu(t)) return;
    if (!rpl_gpu_init()) return;
    rpl__attach(t, 1);
}

/* src/rpl_gpu.c:217-230: copy the device values back into t->data (and the
 * gradient into t->grad); the tensor stays GPU-resident, as in the reference. */
void tensor_from_gpu(Tensor* t) {
    if (!t || t->device == DEVICE_CPU) return;
    float* d = rpl__dev_data(t);
    if (!d) return;
    size_t bytes = (size_t)t->size * sizeof(float);
    if (!rpl__ok(rplhip_memcpy_dtoh(t->data, d, bytes), "tensor_from_gpu")) return;
    float* g = rpl__dev_grad(t);
    if (!g || !t->grad) return;
    float v;
    if (rpl__grad_lazy_value(t, &v)) {
        /* one value only logically: the host copy gets it, the device
         * gradient keeps its mark */
        for (uint32_t i = 0; i < t->size; i++) t->grad[i] = v;
        return;
    }
    rpl__ok(rplhip_memcpy_dtoh(t->grad, g, bytes), "tensor_from_gpu (grad)");
}

/* Internal helpers of the C host layer (not installed). */
#ifndef RPL_HOST_H
#define RPL_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "rpl.h"
#include "rplhip.h"
#include "rplhip_internal.h"

/* Record a failure of `what` (prints it, sets rpl_last_error) when st != 0.
 * Returns 1 on success, 0 on failure. */
int rpl__ok(int st, const char* what);
/* Record a caller error (bad shape etc.); always returns 0. */
int rpl__bad(const char* what, const char* fmt, ...);

/* Device memory pool: exact-size reuse of freed device buffers.  All library
 * work runs on one stream, so a buffer freed after queuing kernels that use
 * it can be handed to later work on the same stream. */
void* rpl__pool_alloc(size_t bytes);
void rpl__pool_free(void* p, size_t bytes);
void rpl__pool_release_all(void);

/* Device buffers of a GPU-resident tensor (NULL if not resident / no grad). */
float* rpl__dev_data(const Tensor* t);
float* rpl__dev_grad(const Tensor* t);
/* Make `t` GPU-resident: allocate device data (and a zeroed device grad when
 * t->grad is set); copy the host values up when `upload`.  Returns 1 on
 * success. */
int rpl__attach(Tensor* t, int upload);
/* tensor_create for an output that becomes GPU-resident at once (host
 * gradient left unzeroed: stale while resident). */
Tensor* rpl__tensor_create_gpu(uint32_t dims, const uint32_t* shape, bool requires_grad);
/* Release internal's device buffers when owner is freed (internal is a
 * graph tensor nothing else references, e.g. linear_forward's GEMM output). */
void rpl__adopt(const Tensor* owner, Tensor* internal);
int rpl__is_gpu(const Tensor* t);
/* Give a GPU-resident tensor a zeroed device gradient if it has none (a
 * root whose host gradient was created after it went to the device). */
int rpl__attach_grad(Tensor* t);

/* Device gradients are filled lazily: a new output's gradient, one attached
 * by rpl__attach_grad and one cleared by tensor_zero_grad are only marked
 * zero, tensor_backward's root is marked 1.  The first accumulation into a
 * zero-marked gradient overwrites it (0 + x, the same bits as accumulating
 * into zeros); readers, and accumulations into another value, get it
 * filled.  rpl__grad_take_zero tests and clears a zero mark,
 * rpl__grad_set_value / rpl__grad_set_zero set the mark,
 * rpl__grad_lazy_value reads it, rpl__dev_grad_ready fills a marked
 * gradient and returns it. */
int rpl__grad_take_zero(const Tensor* t);
void rpl__grad_set_zero(const Tensor* t);
void rpl__grad_set_value(const Tensor* t, float v);
int rpl__grad_lazy_value(const Tensor* t, float* v);
float* rpl__dev_grad_ready(const Tensor* t);

/* Staging of host tensors through device memory for one call. */
#define RPL_STAGE_MAX 12
typedef struct {
    int n;
    int err;
    struct {
        void* dev;
        void* host;
        size_t bytes;
        int writeback;
    } e[RPL_STAGE_MAX];
} RplStage;

/* Device view of a host or device buffer.  For host memory: a pool buffer,
 * filled from `host` when `upload`, copied back at rpl__stage_finish when
 * `writeback`.  For GPU-resident tensors the registry pointer is returned. */
void* rpl__stage_host(RplStage* s, void* host, size_t bytes, int upload, int writeback);
float* rpl__view_data(RplStage* s, const Tensor* t, int upload, int writeback);
float* rpl__view_grad(RplStage* s, const Tensor* t, int upload, int writeback);
/* The gradient of t as the target of an accumulation (grad += x): staged
 * with write-back for host tensors; for GPU-resident ones the device
 * gradient, with *overwrite = 1 when it was zero only logically (the caller
 * must then write every element, as 0 + x). */
float* rpl__view_grad_acc(RplStage* s, const Tensor* t, int* overwrite);
/* Copies write-backs to the host (synchronizing if there are any), releases
 * the staging buffers.  Returns 1 if the call succeeded. */
int rpl__stage_finish(RplStage* s);

#endif

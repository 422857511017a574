/*
 * Device entry points used only by the host layer (not installed, not part of
 * include/).  Each is the include/rplhip.h function of the same name without
 * the leading underscore plus an `overwrite` flag: when it is set, the
 * accumulation target is taken to hold zeros and is written, not read --
 * every element becomes 0.0f + x (or the fused form the public function
 * applies to a target of +0.0), the same bits as accumulating into a
 * zero-filled buffer.  The autograd layer uses them for gradients that are
 * zero only logically (never materialized).
 */
#ifndef RPLHIP_INTERNAL_H
#define RPLHIP_INTERNAL_H

#include "rplhip.h"

#ifdef __cplusplus
extern "C" {
#endif

int rplhip__accumulate(const float* dy, float* dx, uint64_t n, int overwrite, rplhip_stream_t stream);
int rplhip__relu_backward(const float* x, const float* dy, float* dx, uint64_t n, int overwrite,
                          rplhip_stream_t stream);
/* g0 NULL: the root gradient's value is g0_value. */
int rplhip__mse_backward(const float* pred, const float* target, uint64_t n, const float* g0, float g0_value,
                         float* dpred, int overwrite, rplhip_stream_t stream);
int rplhip__bias_grad(const float* dy, uint64_t n, float* db, uint64_t nb, int overwrite, rplhip_stream_t stream);

/* backward_add (src/rpl_core.c:319-337) of out = x + b[i % nb] in two
 * steps that keep the reference's order -- x's gradient, x's subgraph,
 * then b's gradient: _begin reads dy once, writing dx += dy (dx = 0 + dy
 * with dx_overwrite) and the column partial sums of the bias gradient into
 * a workspace held in *cs; _finish adds them into db (db = 0 + sum with
 * db_overwrite; db NULL: just release) and releases the workspace.  The
 * bits are those of rplhip__accumulate followed by rplhip__bias_grad. */
typedef struct {
    void* ws;
    uint64_t splits, nb;
} RplColsum;
/* Where _begin's dy comes from when it is not simply read (src NULL, or
 * kind 0): the add output's gradient g right after the ReLU (kind 1: x = the
 * add output's values, y = the ReLU output's gradient) or MSE (kind 2: x =
 * predictions, y = targets, root gradient *g0p, or g0v when g0p is NULL)
 * backward that consumes the add accumulated into it.  _begin computes that
 * accumulation element by element with the same arithmetic, writes g, and
 * uses the result as dy: the bits of rplhip__relu_backward /
 * rplhip__mse_backward followed by _begin on g. */
typedef struct {
    int kind;
    const float* x;
    const float* y;
    float* g;
    int g_overwrite;
    const float* g0p;
    float g0v;
} RplGradSrc;
int rplhip__add_backward_begin(const float* dy, uint64_t n, float* dx, int dx_overwrite, uint64_t nb,
                               const RplGradSrc* src, RplColsum* cs, rplhip_stream_t stream);
int rplhip__add_backward_finish(RplColsum* cs, float* db, int db_overwrite, rplhip_stream_t stream);

/* rplhip_sgd_step for up to RPL_SGD_MULTI parameter tensors in one launch
 * (optimizer_sgd_step's parameters are independent; the same bits as one
 * launch each).  `first` is filled in by the call. */
#define RPL_SGD_MULTI 8
typedef struct {
    float* p[RPL_SGD_MULTI];
    float* g[RPL_SGD_MULTI];
    float* v[RPL_SGD_MULTI];
    uint64_t n[RPL_SGD_MULTI];
    uint32_t first[RPL_SGD_MULTI + 1];
    int count;
} RplSgdTensors;
int rplhip__sgd_step_multi(RplSgdTensors* ts, float lr, float momentum, float dampening, float weight_decay,
                           int nesterov, rplhip_stream_t stream);

/* linear_forward (src/rpl_nn.c:55-77) in one call: mm = X W^T (X [M,K],
 * W [N,K]; C written without being read, i.e. 1.0f * sum + 0.0f as
 * tensor_gemm over a zeroed C) and out = mm + b[n] (tensor_add_out's
 * broadcast, src/rpl_core.c:112-120), the bias add fused into the GEMM's
 * last pass where the GEMM path allows it.  mm may be NULL. */
int rplhip__linear_forward(const float* X, const float* W, const float* b, float* mm, float* out, uint32_t M,
                           uint32_t N, uint32_t K, rplhip_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif

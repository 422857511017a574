/*
 * The Linear layer and the autograd pieces it uses (src/rpl_nn.c:16-83,
 * src/rpl_core.c:95-135,274-300,319-480) on the gfx950 backend.  The graph
 * walk is the reference's: each backward_fn accumulates into its parents'
 * gradients and recurses, depth first.  The arithmetic runs on the device:
 * dX / dW are f32-MFMA GEMMs with beta = 1 (accumulate), the bias gradient
 * is a column reduction.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "rpl_host.h"

static int any_gpu(const Tensor* a, const Tensor* b) { return rpl__is_gpu(a) || (b && rpl__is_gpu(b)); }

/* src/rpl_core.c:95-129 */
void tensor_add_out(Tensor* out, const Tensor* a, const Tensor* b) {
    if (!out || !a || !b || b->size == 0) {
        rpl__bad("tensor_add_out", "bad arguments");
        return;
    }
    /* The reference reads a[i] for every output element and b[i % b->size]
     * and overruns when the sizes disagree; here that is an error. */
    if (a->size != out->size || out->size % b->size) {
        rpl__bad("tensor_add_out", "sizes %u + %u -> %u do not broadcast", a->size, b->size, out->size);
        return;
    }
    if (!rpl_gpu_init()) return;
    RplStage s = {0};
    const float* da = rpl__view_data(&s, a, 1, 0);
    const float* db = rpl__view_data(&s, b, 1, 0);
    float* dout = rpl__view_data(&s, out, 0, 1);
    if (!s.err) s.err = !rpl__ok(rplhip_add_broadcast(da, db, dout, out->size, b->size, NULL), "tensor_add_out");
    rpl__stage_finish(&s);
    if (out->requires_grad) {
        out->parent1 = (Tensor*)a;
        out->parent2 = (Tensor*)b;
        out->backward_fn = backward_add;
        out->is_leaf = false;
    }
}

/* src/rpl_core.c:131-135 */
Tensor* tensor_add(const Tensor* a, const Tensor* b) {
    const int gpu = any_gpu(a, b);
    Tensor* out = (gpu ? rpl__tensor_create_gpu : tensor_create)(a->dims, a->shape,
                                                                 a->requires_grad || b->requires_grad);
    if (!out) return NULL;
    if (gpu && !rpl__attach(out, 0)) return out;
    tensor_add_out(out, a, b);
    return out;
}

void tensor_add_gpu(Tensor* out, const Tensor* a, const Tensor* b) {
    tensor_to_gpu((Tensor*)a);
    tensor_to_gpu((Tensor*)b);
    if (!rpl__is_gpu(out) && !rpl__attach(out, 0)) return;
    tensor_add_out(out, a, b);
}

/* src/rpl_core.c:274-300 */
Tensor* tensor_relu(const Tensor* t) {
    const int gpu = rpl__is_gpu(t);
    Tensor* out = (gpu ? rpl__tensor_create_gpu : tensor_create)(t->dims, t->shape, t->requires_grad);
    if (!out) return NULL;
    if (gpu && !rpl__attach(out, 0)) return out;
    if (!rpl_gpu_init()) return out;
    RplStage s = {0};
    const float* dx = rpl__view_data(&s, t, 1, 0);
    float* dy = rpl__view_data(&s, out, 0, 1);
    if (!s.err) s.err = !rpl__ok(rplhip_relu(dx, dy, t->size, NULL), "tensor_relu");
    rpl__stage_finish(&s);
    if (out->requires_grad) {
        out->parent1 = (Tensor*)t;
        out->backward_fn = backward_relu;
        out->is_leaf = false;
    }
    return out;
}

/* The device seam's elementwise ops (src/rpl_gpu.c:437-522, dispatch_unary_op):
 * `in` moves to the device; an output that is not resident takes in's
 * shape and becomes resident, as the reference does -- provided its host
 * buffer holds that many elements (the reference would overrun it).  A
 * resident output must already have in's size. */
static void unary_gpu(Tensor* out, const Tensor* in, int (*fn)(const float*, float*, uint64_t, rplhip_stream_t),
                      const char* what) {
    if (!out || !in) {
        rpl__bad(what, "NULL tensor");
        return;
    }
    if (!rpl_gpu_init()) return;
    tensor_to_gpu((Tensor*)in);
    if (!rpl__is_gpu(in)) return;
    if (!rpl__is_gpu(out)) {
        if (out->size < in->size) {
            rpl__bad(what, "output holds %u elements, input has %u", out->size, in->size);
            return;
        }
        out->dims = in->dims;
        memcpy(out->shape, in->shape, sizeof(in->shape));
        out->size = in->size;
        if (!rpl__attach(out, 0)) return;
    } else if (out->size != in->size) {
        rpl__bad(what, "output has %u elements, input has %u", out->size, in->size);
        return;
    }
    RplStage s = {0};
    const float* dx = rpl__view_data(&s, in, 1, 0);
    float* dy = rpl__view_data(&s, out, 0, 1);
    if (!s.err) s.err = !rpl__ok(fn(dx, dy, in->size, NULL), what);
    rpl__stage_finish(&s);
}

/* src/rpl_gpu.c:475-477 */
void tensor_relu_gpu(Tensor* out, const Tensor* in) { unary_gpu(out, in, rplhip_relu, "tensor_relu_gpu"); }
/* src/rpl_gpu.c:479-481 (CPU formula: tensor_sigmoid, src/rpl_core.c:302-304) */
void tensor_sigmoid_gpu(Tensor* out, const Tensor* in) { unary_gpu(out, in, rplhip_sigmoid, "tensor_sigmoid_gpu"); }
/* src/rpl_gpu.c:515-517 (CPU formula: tensor_tanh_inplace, src/rpl_core.c:490-491) */
void tensor_tanh_gpu(Tensor* out, const Tensor* in) { unary_gpu(out, in, rplhip_tanh, "tensor_tanh_gpu"); }
/* src/rpl_gpu.c:519-521 (CPU formula: tensor_gelu_inplace, src/rpl_core.c:493-497) */
void tensor_gelu_gpu(Tensor* out, const Tensor* in) { unary_gpu(out, in, rplhip_gelu, "tensor_gelu_gpu"); }

/* src/rpl_core.c:449-465 */
Tensor* tensor_mse_loss(const Tensor* pred, const Tensor* target) {
    uint32_t shape[1] = {1};
    Tensor* out = tensor_create(1, shape, pred->requires_grad);
    if (!out) return NULL;
    if (any_gpu(pred, target) && !rpl__attach(out, 0)) return out;
    if (!rpl_gpu_init()) return out;
    RplStage s = {0};
    const float* dp = rpl__view_data(&s, pred, 1, 0);
    const float* dt = rpl__view_data(&s, target, 1, 0);
    float* dl = rpl__view_data(&s, out, 0, 1);
    if (!s.err) s.err = !rpl__ok(rplhip_mse_loss(dp, dt, pred->size, dl, NULL), "tensor_mse_loss");
    rpl__stage_finish(&s);
    if (out->requires_grad) {
        out->parent1 = (Tensor*)pred;
        out->parent2 = (Tensor*)target;
        out->backward_fn = backward_mse;
        out->is_leaf = false;
    }
    return out;
}

/* src/rpl_core.c:319-337.  Gradients are accumulated; a device gradient
 * that is still zero only logically is overwritten instead (the same bits). */
/* backward_add's path with t, both parents and their gradients on the
 * device: one pass over dy writes a's gradient and the bias gradient's
 * column partial sums, which are added into b's gradient after a's
 * subgraph, in the reference's order.  src (may be NULL): dy is t's
 * gradient right after the ReLU / MSE backward that consumes t
 * accumulated into it, computed within the same pass (see RplGradSrc). */
static int add_backward_device_ok(const Tensor* t) {
    const Tensor* a = t->parent1;
    const Tensor* b = t->parent2;
    return t->backward_fn == backward_add && t->grad && a && a->grad && b && b->grad && b->size > 0 &&
           rpl__is_gpu(t) && rpl__is_gpu(a) && rpl__is_gpu(b);
}
static void add_backward_device(Tensor* t, const RplGradSrc* src) {
    Tensor* a = t->parent1;
    Tensor* b = t->parent2;
    RplStage s = {0};
    int ow_a = 0, ow_b = 0;
    RplColsum cs = {0};
    const float* dy = src ? NULL : rpl__view_grad(&s, t, 1, 0);
    float* da = rpl__view_grad_acc(&s, a, &ow_a);
    if (!s.err)
        s.err = !rpl__ok(rplhip__add_backward_begin(dy, t->size, da, ow_a, b->size, src, &cs, NULL), "backward_add");
    rpl__stage_finish(&s);
    if (a->backward_fn) a->backward_fn(a);
    RplStage s2 = {0};
    float* db = s.err ? NULL : rpl__view_grad_acc(&s2, b, &ow_b);
    if (!rpl__ok(rplhip__add_backward_finish(&cs, s2.err ? NULL : db, ow_b, NULL), "backward_add (bias)")) s2.err = 1;
    rpl__stage_finish(&s2);
    if (b->backward_fn) b->backward_fn(b);
}

void backward_add(Tensor* t) {
    Tensor* a = t->parent1;
    Tensor* b = t->parent2;
    if (a && a->grad && b && b->grad && rpl__is_gpu(t) && rpl__is_gpu(a) && rpl__is_gpu(b)) {
        add_backward_device(t, NULL);
        return;
    }
    if (a && a->grad) {
        RplStage s = {0};
        int ow = 0;
        const float* dy = rpl__view_grad(&s, t, 1, 0);
        float* da = rpl__view_grad_acc(&s, a, &ow);
        if (!s.err) s.err = !rpl__ok(rplhip__accumulate(dy, da, t->size, ow, NULL), "backward_add");
        rpl__stage_finish(&s);
        if (a->backward_fn) a->backward_fn(a);
    }
    if (b && b->grad) {
        RplStage s = {0};
        int ow = 0;
        const float* dy = rpl__view_grad(&s, t, 1, 0);
        float* db = rpl__view_grad_acc(&s, b, &ow);
        if (!s.err) s.err = !rpl__ok(rplhip__bias_grad(dy, t->size, db, b->size, ow, NULL), "backward_add (bias)");
        rpl__stage_finish(&s);
        if (b->backward_fn) b->backward_fn(b);
    }
}

/* C += op(A) op(B) (beta = 1), or C = op(A) op(B) + 0.0f when C's values
 * are zero only logically (overwrite): the same bits, C not read. */
static int sgemm_acc(int ta, int tb, uint32_t M, uint32_t N, uint32_t K, const float* A, uint32_t lda,
                     const float* B, uint32_t ldb, float* C, uint32_t ldc, int overwrite) {
    return rplhip_sgemm_batched(ta, tb, M, N, K, 1.0f, A, lda, 0, B, ldb, 0, 1.0f, C, ldc, 0, 1, overwrite ? 0 : 1,
                                NULL);
}

/* src/rpl_core.c:363-416, including its layout guess for B (b is taken as
 * [N,K] -- the Linear weight layout -- when its shape says so). */
void backward_matmul(Tensor* t) {
    Tensor* a = t->parent1;
    Tensor* b = t->parent2;
    uint32_t M = t->shape[0], N = t->shape[1], K = a->shape[1];
    bool b_trans = (b->shape[0] == N && b->shape[1] == K);
    if (a->grad) {
        /* dA[M,K] += dt[M,N] * (b_trans ? B[N,K] : B[K,N]^T) */
        RplStage s = {0};
        int ow = 0;
        const float* dt = rpl__view_grad(&s, t, 1, 0);
        const float* db = rpl__view_data(&s, b, 1, 0);
        float* da = rpl__view_grad_acc(&s, a, &ow);
        if (!s.err)
            s.err = !rpl__ok(sgemm_acc(0, !b_trans, M, K, N, dt, N, db, b_trans ? K : N, da, K, ow),
                             "backward_matmul (dA)");
        rpl__stage_finish(&s);
        if (a->backward_fn) a->backward_fn(a);
    }
    if (b->grad) {
        RplStage s = {0};
        int ow = 0;
        const float* dt = rpl__view_grad(&s, t, 1, 0);
        const float* da = rpl__view_data(&s, a, 1, 0);
        float* dbg = rpl__view_grad_acc(&s, b, &ow);
        int st = RPLHIP_OK;
        if (!s.err) {
            if (b_trans) /* dB[N,K] += dt^T[N,M] * A[M,K] */
                st = sgemm_acc(1, 0, N, K, M, dt, N, da, K, dbg, K, ow);
            else /* dB[K,N] += A^T[K,M] * dt[M,N] */
                st = sgemm_acc(1, 0, K, N, M, da, K, dt, N, dbg, N, ow);
            s.err = !rpl__ok(st, "backward_matmul (dB)");
        }
        rpl__stage_finish(&s);
        if (b->backward_fn) b->backward_fn(b);
    }
}

/* src/rpl_core.c:418-424 */
void backward_relu(Tensor* t) {
    Tensor* a = t->parent1;
    if (a && a->grad && rpl__is_gpu(t) && t->grad && add_backward_device_ok(a)) {
        /* a = x + bias on the device: the ReLU backward's accumulation into
         * a's gradient runs inside a's add backward pass (same bits). */
        RplStage s = {0};
        RplGradSrc src = {1, NULL, NULL, NULL, 0, NULL, 0.0f};
        src.x = rpl__view_data(&s, a, 1, 0);
        src.y = rpl__view_grad(&s, t, 1, 0);
        src.g = rpl__view_grad_acc(&s, a, &src.g_overwrite);
        rpl__stage_finish(&s);
        if (!s.err) add_backward_device(a, &src);
        return;
    }
    if (a && a->grad) {
        RplStage s = {0};
        int ow = 0;
        const float* dx = rpl__view_data(&s, a, 1, 0);
        const float* dy = rpl__view_grad(&s, t, 1, 0);
        float* dg = rpl__view_grad_acc(&s, a, &ow);
        if (!s.err) s.err = !rpl__ok(rplhip__relu_backward(dx, dy, dg, t->size, ow, NULL), "backward_relu");
        rpl__stage_finish(&s);
        if (a->backward_fn) a->backward_fn(a);
    }
}

/* src/rpl_core.c:437-447 */
void backward_mse(Tensor* t) {
    Tensor* pred = t->parent1;
    Tensor* target = t->parent2;
    if (pred && pred->grad && rpl__is_gpu(t) && rpl__is_gpu(pred) && rpl__is_gpu(target) &&
        add_backward_device_ok(pred)) {
        /* pred = x + bias on the device: the MSE backward's accumulation
         * into pred's gradient runs inside pred's add backward pass (same
         * bits). */
        RplStage s = {0};
        RplGradSrc src = {2, NULL, NULL, NULL, 0, NULL, 0.0f};
        src.x = rpl__view_data(&s, pred, 1, 0);
        src.y = rpl__view_data(&s, target, 1, 0);
        src.g0p = t->size == 1 && rpl__grad_lazy_value(t, &src.g0v) ? NULL : rpl__view_grad(&s, t, 1, 0);
        src.g = rpl__view_grad_acc(&s, pred, &src.g_overwrite);
        rpl__stage_finish(&s);
        if (!s.err) add_backward_device(pred, &src);
        return;
    }
    if (pred && pred->grad) {
        RplStage s = {0};
        int ow = 0;
        const float* dp = rpl__view_data(&s, pred, 1, 0);
        const float* dtg = rpl__view_data(&s, target, 1, 0);
        /* The root gradient tensor_backward marks 1 goes in as a value. */
        float g0v = 0.0f;
        const float* g0 = t->size == 1 && rpl__grad_lazy_value(t, &g0v) ? NULL : rpl__view_grad(&s, t, 1, 0);
        float* dg = rpl__view_grad_acc(&s, pred, &ow);
        if (!s.err)
            s.err = !rpl__ok(rplhip__mse_backward(dp, dtg, pred->size, g0, g0v, dg, ow, NULL), "backward_mse");
        rpl__stage_finish(&s);
        if (pred->backward_fn) pred->backward_fn(pred);
    }
}

/* src/rpl_core.c:467-476 */
void tensor_backward(Tensor* t) {
    if (!t->requires_grad) return;
    if (!t->grad) {
        t->grad = (float*)rpitorch_aligned_alloc(64, (size_t)t->size * sizeof(float));
        if (!t->grad) return;
    }
    for (uint32_t i = 0; i < t->size; i++) t->grad[i] = 1.0f;
    if (rpl__is_gpu(t)) {
        /* marked 1 everywhere, written only when read as an array */
        if (!rpl__attach_grad(t)) return;
        rpl__grad_set_value(t, 1.0f);
    }
    if (t->backward_fn) t->backward_fn(t);
}

/* src/rpl_core.c:478-480 (the device gradient is marked zero, not written) */
void tensor_zero_grad(Tensor* t) {
    if (!t || !t->grad) return;
    memset(t->grad, 0, (size_t)t->size * sizeof(float));
    rpl__grad_set_zero(t);
}

/* src/rpl_nn.c:23-43: same Xavier-style init from rand(), so a given
 * srand() seed yields the reference's weights. */
Linear* linear_create(uint32_t in_features, uint32_t out_features) {
    Linear* layer = (Linear*)calloc(1, sizeof(Linear));
    if (!layer) return NULL;
    layer->in_features = in_features;
    layer->out_features = out_features;
    uint32_t weight_shape[2] = {out_features, in_features};
    layer->weight = tensor_create(2, weight_shape, true);
    uint32_t bias_shape[1] = {out_features};
    layer->bias = tensor_create(1, bias_shape, true);
    float std = sqrtf(2.0f / (in_features + out_features));
    for (uint32_t i = 0; i < layer->weight->size; i++)
        layer->weight->data[i] = ((float)rand() / RAND_MAX - 0.5f) * 2.0f * std;
    for (uint32_t i = 0; i < layer->bias->size; i++) layer->bias->data[i] = 0.0f;
    return layer;
}

/* src/rpl_nn.c:55-77: NT GEMM x * W^T into a zeroed buffer, then the
 * broadcast bias add; matmul_out stays alive as part of the graph. */
Tensor* linear_forward(Linear* layer, const Tensor* input) {
    uint32_t output_shape[2] = {input->shape[0], layer->out_features};
    const int gpu = any_gpu(input, layer->weight) || rpl__is_gpu(layer->bias);
    Tensor* (*create)(uint32_t, const uint32_t*, bool) = gpu ? rpl__tensor_create_gpu : tensor_create;
    Tensor* matmul_out = create(2, output_shape, input->requires_grad || layer->weight->requires_grad);
    if (!matmul_out) return NULL;
    if (gpu && !rpl__attach(matmul_out, 0)) return NULL;
    /* The reference zeroes the buffer and runs tensor_gemm (beta = 0, which
     * still reads C).  With input and weight resident, one GEMM that writes
     * C without reading it gives the same bits (alpha*x + 0.0f) and skips
     * the fill; otherwise zero the buffer (on the device when resident: its
     * host copy is stale by definition) and go through tensor_gemm. */
    const uint32_t M = input->shape[0], K = input->shape[1], N = layer->out_features;
    const int fused = gpu && rpl__is_gpu(input) && rpl__is_gpu(layer->weight) && rpl__is_gpu(layer->bias) &&
                      input->dims == 2 && K == layer->in_features && layer->bias->size == N;
    if (fused) {
        /* GEMM and bias add in one call (the add fused into the GEMM's last
         * pass where its path allows); out's graph links are set below. */
    } else if (gpu && rpl__is_gpu(input) && rpl__is_gpu(layer->weight) && input->dims == 2 && K == layer->in_features) {
        rpl__ok(rplhip_sgemm_batched(0, 1, M, N, K, 1.0f, rpl__dev_data(input), K, 0, rpl__dev_data(layer->weight),
                                     K, 0, 0.0f, rpl__dev_data(matmul_out), N, 0, 1, 0, NULL),
                "linear_forward");
    } else {
        if (gpu)
            rpl__ok(rplhip_fill(rpl__dev_data(matmul_out), matmul_out->size, 0.0f, NULL), "linear_forward");
        else
            tensor_fill(matmul_out, 0.0f);
        tensor_gemm(matmul_out, input, layer->weight, 1.0f, 0.0f, false, true);
    }
    if (matmul_out->requires_grad) {
        matmul_out->parent1 = (Tensor*)input;
        matmul_out->parent2 = layer->weight;
        matmul_out->backward_fn = backward_matmul;
        matmul_out->is_leaf = false;
    }
    Tensor* out = create(2, output_shape, matmul_out->requires_grad || layer->bias->requires_grad);
    if (!out) return NULL;
    if (gpu && !rpl__attach(out, 0)) return NULL;
    if (fused) {
        rpl__ok(rplhip__linear_forward(rpl__dev_data(input), rpl__dev_data(layer->weight), rpl__dev_data(layer->bias),
                                       rpl__dev_data(matmul_out), rpl__dev_data(out), M, N, K, NULL),
                "linear_forward");
        if (out->requires_grad) { /* tensor_add_out's graph links (src/rpl_core.c:122-128) */
            out->parent1 = matmul_out;
            out->parent2 = layer->bias;
            out->backward_fn = backward_add;
            out->is_leaf = false;
        }
    } else {
        tensor_add_out(out, matmul_out, layer->bias);
    }
    if (gpu) rpl__adopt(out, matmul_out);
    return out;
}

/* src/rpl_nn.c:79-83 */
void linear_free(Linear* layer) {
    if (!layer) return;
    tensor_free(layer->weight);
    tensor_free(layer->bias);
    free(layer);
}

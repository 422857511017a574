/*
 * QAT fake quantization (src/rpl_quantization.c:170-258) and the FP16 codec
 * (src/rpl_half.c:77-113) on the device.
 *
 * FakeQuantize is file-local in the reference; its layout is kept so the
 * reference's own functions and these interoperate.  The scale / zero-point
 * moving averages are host scalars computed with the fused forms GCC makes
 * of the reference's expressions (fmaf((1-m), s, m * s_new)), so the state
 * matches the reference bit for bit; the min/max of a training step is a
 * device reduction with the reference's OpenMP semantics (NaN never
 * selected).
 */
#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "rpl_host.h"

struct FakeQuantize {
    Tensor* scale;
    Tensor* zero_point;
    bool training;
    uint32_t num_batches_tracked;
};

/* src/rpl_quantization.c:181-193 */
FakeQuantize* fake_quantize_create(void) {
    FakeQuantize* fq = (FakeQuantize*)calloc(1, sizeof(FakeQuantize));
    if (!fq) return NULL;
    uint32_t shape[1] = {1};
    fq->scale = tensor_create(1, shape, true);
    fq->zero_point = tensor_create(1, shape, true);
    if (!fq->scale || !fq->zero_point) {
        tensor_free(fq->scale);
        tensor_free(fq->zero_point);
        free(fq);
        return NULL;
    }
    fq->scale->data[0] = 1.0f;
    fq->zero_point->data[0] = 0.0f;
    fq->training = true;
    return fq;
}

/* src/rpl_quantization.c:246-253: straight-through (identity) gradient. */
void backward_fake_quant(Tensor* t) {
    Tensor* input = t->parent1;
    if (input && input->grad) {
        RplStage s = {0};
        int ow = 0;
        const float* dy = rpl__view_grad(&s, t, 1, 0);
        float* dx = rpl__view_grad_acc(&s, input, &ow);
        if (!s.err) s.err = !rpl__ok(rplhip__accumulate(dy, dx, t->size, ow, NULL), "backward_fake_quant");
        rpl__stage_finish(&s);
        if (input->backward_fn) input->backward_fn(input);
    }
}

/* src/rpl_quantization.c:195-244 */
Tensor* fake_quantize_forward(FakeQuantize* fq, const Tensor* input) {
    if (!fq || !input) {
        rpl__bad("fake_quantize_forward", "NULL argument");
        return NULL;
    }
    const int gpu = rpl__is_gpu(input);
    Tensor* out = (gpu ? rpl__tensor_create_gpu : tensor_create)(input->dims, input->shape, input->requires_grad);
    if (!out) return NULL;
    if (gpu && !rpl__attach(out, 0)) return out;
    if (!rpl_gpu_init()) return out;
    float scale = fq->scale->data[0];
    float zp = fq->zero_point->data[0];
    RplStage s = {0};
    const float* dx = rpl__view_data(&s, input, 1, 0);
    float* dy = rpl__view_data(&s, out, 0, 1);
    if (!s.err && fq->training) {
        float mm[2] = {FLT_MAX, -FLT_MAX};
        if (input->size) {
            float* dmm = (float*)rpl__stage_host(&s, mm, sizeof(mm), 0, 0);
            if (!s.err) s.err = !rpl__ok(rplhip_min_max(dx, input->size, dmm, NULL), "fake_quantize_forward");
            if (!s.err)
                s.err = !rpl__ok(rplhip_memcpy_dtoh(mm, dmm, sizeof(mm)), "fake_quantize_forward (min/max)");
        }
        if (!s.err) {
            const float min_val = mm[0], max_val = mm[1];
            const float new_scale = (max_val - min_val) / 255.0f;
            const float new_zp = -min_val / new_scale;
            const float momentum = 0.1f;
            scale = fmaf(1.0f - momentum, scale, momentum * new_scale);
            zp = fmaf(1.0f - momentum, zp, momentum * new_zp);
            fq->scale->data[0] = scale;
            fq->zero_point->data[0] = zp;
            fq->num_batches_tracked++;
        }
    }
    if (!s.err) s.err = !rpl__ok(rplhip_fake_quant(dx, dy, input->size, scale, zp, NULL), "fake_quantize_forward");
    rpl__stage_finish(&s);
    if (out->requires_grad) {
        out->parent1 = (Tensor*)input;
        out->backward_fn = backward_fake_quant;
        out->is_leaf = false;
    }
    return out;
}

/* src/rpl_quantization.c:255-260 */
void fake_quantize_free(FakeQuantize* fq) {
    if (!fq) return;
    tensor_free(fq->scale);
    tensor_free(fq->zero_point);
    free(fq);
}

/* src/rpl_half.c:77-96.  The result always holds its values in host memory
 * (device = CPU): the reference leaves `data` unfilled for a GPU-resident
 * input; here the conversion runs on the device either way. */
HalfTensor* tensor_to_half(const Tensor* t) {
    if (!t) return NULL;
    HalfTensor* ht = (HalfTensor*)calloc(1, sizeof(HalfTensor));
    if (!ht) return NULL;
    ht->dims = t->dims;
    ht->size = t->size;
    memcpy(ht->shape, t->shape, sizeof(t->shape));
    memcpy(ht->strides, t->strides, sizeof(t->strides));
    ht->device = DEVICE_CPU;
    ht->_allocation = rpitorch_aligned_alloc(64, (size_t)ht->size * sizeof(rpl_half));
    ht->data = (rpl_half*)ht->_allocation;
    if (!ht->data) {
        free(ht);
        return NULL;
    }
    if (!t->size || !rpl_gpu_init()) return ht;
    RplStage s = {0};
    const float* dx = rpl__view_data(&s, t, 1, 0);
    uint16_t* dh = (uint16_t*)rpl__stage_host(&s, ht->data, (size_t)ht->size * sizeof(rpl_half), 0, 1);
    if (!s.err) s.err = !rpl__ok(rplhip_float_to_half(dx, dh, t->size, NULL), "tensor_to_half");
    rpl__stage_finish(&s);
    return ht;
}

/* src/rpl_half.c:98-110 (a host tensor, like the reference's for CPU input) */
Tensor* tensor_from_half(const HalfTensor* ht) {
    if (!ht) return NULL;
    Tensor* t = tensor_create(ht->dims, ht->shape, false);
    if (!t || !t->size || !rpl_gpu_init()) return t;
    RplStage s = {0};
    const uint16_t* dh =
        (const uint16_t*)rpl__stage_host(&s, ht->data, (size_t)ht->size * sizeof(rpl_half), 1, 0);
    float* dx = rpl__view_data(&s, t, 0, 1);
    if (!s.err) s.err = !rpl__ok(rplhip_half_to_float(dh, dx, t->size, NULL), "tensor_from_half");
    rpl__stage_finish(&s);
    return t;
}

/* src/rpl_half.c:109-113 */
void half_tensor_free(HalfTensor* t) {
    if (!t) return;
    if (t->_allocation) rpitorch_aligned_free(t->_allocation);
    free(t);
}

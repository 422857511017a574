/*
 * Quantization entry points of the reference (src/rpl_core.c:511-530,
 * src/ops_extended.c:52-80, src/rpl_quantization.c:18-168) on the gfx950
 * kernels.  The quantized outputs are host structures, as in the reference.
 */
#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "rpl_host.h"

static QuantizedTensor* qt_alloc(const Tensor* input) {
    QuantizedTensor* qt = (QuantizedTensor*)calloc(1, sizeof(QuantizedTensor));
    if (!qt) return NULL;
    qt->size = input->size;
    qt->dims = input->dims;
    memcpy(qt->shape, input->shape, input->dims * sizeof(uint32_t));
    qt->data = (int8_t*)rpitorch_aligned_alloc(64, qt->size);
    if (!qt->data) {
        free(qt);
        return NULL;
    }
    return qt;
}

/* Quantize `input` on the device.  mode 0: given scale/zp; 1: symmetric;
 * 2: asymmetric (scale/zp computed on the device and copied back). */
static QuantizedTensor* quantize(const Tensor* input, int mode, float scale, int32_t zp, const char* what) {
    if (!input) {
        rpl__bad(what, "NULL tensor");
        return NULL;
    }
    if (!rpl_gpu_init()) return NULL;
    QuantizedTensor* qt = qt_alloc(input);
    if (!qt) return NULL;
    qt->scale = scale;
    qt->zero_point = zp;
    RplStage s = {0};
    const float* dx = rpl__view_data(&s, input, 1, 0);
    int8_t* dq = rpl__stage_host(&s, qt->data, qt->size, 0, 1);
    float* dscale = mode ? rpl__stage_host(&s, &qt->scale, sizeof(float), 0, 1) : NULL;
    int32_t* dzp = mode == 2 ? rpl__stage_host(&s, &qt->zero_point, sizeof(int32_t), 0, 1) : NULL;
    if (!s.err) {
        int st = mode == 0   ? rplhip_quantize_int8(dx, input->size, scale, zp, dq, NULL)
                 : mode == 1 ? rplhip_quantize_symmetric(dx, input->size, dq, dscale, NULL)
                             : rplhip_quantize_asymmetric(dx, input->size, dq, dscale, dzp, NULL);
        s.err = !rpl__ok(st, what);
    }
    if (!rpl__stage_finish(&s)) {
        quantized_tensor_free(qt);
        return NULL;
    }
    if (mode == 1) qt->zero_point = 0;
    return qt;
}

/* src/rpl_core.c:511-530 */
QuantizedTensor* tensor_quantize_int8(const Tensor* input, float scale, int32_t zero_point) {
    return quantize(input, 0, scale, zero_point, "tensor_quantize_int8");
}

/* src/rpl_quantization.c:77-91 */
QuantizedTensor* tensor_quantize_int8_symmetric(const Tensor* input) {
    return quantize(input, 1, 0.0f, 0, "tensor_quantize_int8_symmetric");
}

/* src/rpl_quantization.c:93-107 */
QuantizedTensor* tensor_quantize_int8_asymmetric(const Tensor* input) {
    return quantize(input, 2, 0.0f, 0, "tensor_quantize_int8_asymmetric");
}

/* src/rpl_quantization.c:120-160: leading-axis slices of size/num_channels
 * elements, num_channels = shape[channel_axis] (the reference indexes
 * c*channel_size + i whatever the axis). */
PerChannelQuantizedTensor* tensor_quantize_per_channel(const Tensor* input, uint32_t channel_axis) {
    if (!input || channel_axis >= input->dims || input->shape[channel_axis] == 0) {
        rpl__bad("tensor_quantize_per_channel", "bad tensor or channel axis");
        return NULL;
    }
    if (!rpl_gpu_init()) return NULL;
    PerChannelQuantizedTensor* qt = (PerChannelQuantizedTensor*)calloc(1, sizeof(PerChannelQuantizedTensor));
    if (!qt) return NULL;
    qt->num_channels = input->shape[channel_axis];
    qt->channel_size = input->size / qt->num_channels;
    qt->dims = input->dims;
    memcpy(qt->shape, input->shape, input->dims * sizeof(uint32_t));
    qt->data = (int8_t*)rpitorch_aligned_alloc(RPITORCH_CACHE_LINE, input->size);
    qt->scales = (float*)malloc(qt->num_channels * sizeof(float));
    qt->zero_points = (int32_t*)calloc(qt->num_channels, sizeof(int32_t));
    if (!qt->data || !qt->scales || !qt->zero_points) {
        per_channel_quantized_tensor_free(qt);
        return NULL;
    }
    RplStage s = {0};
    const float* dx = rpl__view_data(&s, input, 1, 0);
    int8_t* dq = rpl__stage_host(&s, qt->data, (size_t)qt->num_channels * qt->channel_size, 0, 1);
    float* ds = rpl__stage_host(&s, qt->scales, qt->num_channels * sizeof(float), 0, 1);
    if (!s.err)
        s.err = !rpl__ok(rplhip_quantize_per_channel(dx, qt->num_channels, qt->channel_size, dq, ds, NULL),
                         "tensor_quantize_per_channel");
    if (!rpl__stage_finish(&s)) {
        per_channel_quantized_tensor_free(qt);
        return NULL;
    }
    return qt;
}

/* src/rpl_quantization.c:162-168 */
void per_channel_quantized_tensor_free(PerChannelQuantizedTensor* qt) {
    if (!qt) return;
    rpitorch_aligned_free(qt->data);
    free(qt->scales);
    free(qt->zero_points);
    free(qt);
}

/* src/ops_extended.c:75-80 */
void quantized_tensor_free(QuantizedTensor* qt) {
    if (!qt) return;
    if (qt->data) rpitorch_aligned_free(qt->data);
    free(qt);
}

/* src/ops_extended.c:64-73 */
Tensor* tensor_dequantize_int8(QuantizedTensor* input) {
    if (!input) return NULL;
    if (!rpl_gpu_init()) return NULL;
    Tensor* out = tensor_create(input->dims, input->shape, false);
    if (!out) return NULL;
    RplStage s = {0};
    const int8_t* dq = rpl__stage_host(&s, input->data, input->size, 1, 0);
    float* dy = rpl__view_data(&s, out, 0, 1);
    if (!s.err)
        s.err = !rpl__ok(rplhip_dequantize_int8(dq, input->size, input->scale, input->zero_point, dy, NULL),
                         "tensor_dequantize_int8");
    rpl__stage_finish(&s);
    return out;
}

/* src/ops_extended.c:52-61 (sequential-scan semantics on the device) */
void tensor_get_min_max(const Tensor* t, float* min_val, float* max_val) {
    if (!t || t->size == 0) return;
    if (!rpl_gpu_init()) return;
    float mm[2] = {*min_val, *max_val};
    RplStage s = {0};
    const float* dx = rpl__view_data(&s, t, 1, 0);
    float* d2 = rpl__stage_host(&s, mm, sizeof(mm), 0, 1);
    if (!s.err) s.err = !rpl__ok(rplhip_get_min_max(dx, t->size, d2, NULL), "tensor_get_min_max");
    if (rpl__stage_finish(&s)) {
        *min_val = mm[0];
        *max_val = mm[1];
    }
}

/* src/rpl_quantization.c:26-31 */
QuantizationCalibrator* calibrator_create(void) {
    QuantizationCalibrator* cal = (QuantizationCalibrator*)calloc(1, sizeof(QuantizationCalibrator));
    if (!cal) return NULL;
    cal->min_val = FLT_MAX;
    cal->max_val = -FLT_MAX;
    return cal;
}

/* src/rpl_quantization.c:33-54: the tensor's min/max on the device, merged
 * into the running range exactly as the critical section does. */
void calibrator_update(QuantizationCalibrator* cal, const Tensor* t) {
    if (!cal || !t) return;
    if (!rpl_gpu_init()) return;
    float mm[2] = {FLT_MAX, -FLT_MAX};
    RplStage s = {0};
    const float* dx = rpl__view_data(&s, t, 1, 0);
    float* d2 = rpl__stage_host(&s, mm, sizeof(mm), 0, 1);
    if (!s.err) s.err = !rpl__ok(rplhip_min_max(dx, t->size, d2, NULL), "calibrator_update");
    if (!rpl__stage_finish(&s)) return;
    if (mm[0] < cal->min_val) cal->min_val = mm[0];
    if (mm[1] > cal->max_val) cal->max_val = mm[1];
    cal->num_samples++;
}

/* src/rpl_quantization.c:56-67 (host scalar arithmetic, as in the reference) */
void calibrator_compute_params(QuantizationCalibrator* cal, bool symmetric) {
    if (!cal) return;
    if (symmetric) {
        float abs_max = fmaxf(fabsf(cal->min_val), fabsf(cal->max_val));
        cal->scale = abs_max / 127.0f;
        cal->zero_point = 0;
    } else {
        float range = cal->max_val - cal->min_val;
        cal->scale = range / 255.0f;
        cal->zero_point = (int32_t)roundf(-cal->min_val / cal->scale);
    }
}

void calibrator_free(QuantizationCalibrator* cal) { free(cal); }

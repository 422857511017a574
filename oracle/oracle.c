/*
 * CPU oracle for RPL's GEMM hot path -- TEST INFRASTRUCTURE ONLY.
 * Used as the checker by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg; never linked into or called by the product library.
 *
 * Each function restates the reference algorithm cited above it, with the
 * same loop order and the same expression shapes, so that GCC (-O3
 * -std=gnu11, -ffp-contract=fast by default) forms the same FMAs.  The float
 * -> int32 conversions are written as plain C casts, exactly like the
 * reference: on x86-64 they compile to cvttss2si, which yields INT_MIN for
 * NaN and out-of-range values.  That hardware result is part of the contract
 * (an all-zero tensor quantizes to -128), and the device code emulates it.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* rpl_core.c:199-217 */
void orc_sgemm_rows(const float* A, const float* B, float* C, uint32_t M, uint32_t N,
                    uint32_t K, float alpha, float beta, bool ta, bool tb, uint32_t row0,
                    uint32_t row1) {
    if (row1 > M) row1 = M;
#pragma omp parallel for collapse(2)
    for (uint32_t i = row0; i < row1; i++) {
        for (uint32_t j = 0; j < N; j++) {
            float sum = 0;
            for (uint32_t k = 0; k < K; k++) {
                float va = ta ? A[k * M + i] : A[i * K + k];
                float vb = tb ? B[j * K + k] : B[k * N + j];
                sum += va * vb;
            }
            C[i * N + j] = alpha * sum + beta * C[i * N + j];
        }
    }
}

void orc_sgemm(const float* A, const float* B, float* C, uint32_t M, uint32_t N, uint32_t K,
               float alpha, float beta, bool ta, bool tb) {
    orc_sgemm_rows(A, B, C, M, N, K, alpha, beta, ta, tb, 0, M);
}

/* ops_extended.c:83-123 (the non-NEON branch, :113-117, then :119-120) */
void orc_gemm_int8_rows(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M,
                        uint32_t N, uint32_t K, float sa, float sb, float sc, int32_t za,
                        int32_t zb, uint32_t row0, uint32_t row1) {
    if (row1 > M) row1 = M;
#pragma omp parallel for collapse(2)
    for (uint32_t i = row0; i < row1; i++) {
        for (uint32_t j = 0; j < N; j++) {
            int32_t sum = 0;
            for (uint32_t k = 0; k < K; k++) {
                sum += (int32_t)(A[i * K + k] - za) * (int32_t)(B[k * N + j] - zb);
            }
            float result = sum * sa * sb / sc;
            C[i * N + j] = (int32_t)roundf(result);
        }
    }
}

void orc_gemm_int8(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N,
                   uint32_t K, float sa, float sb, float sc, int32_t za, int32_t zb) {
    orc_gemm_int8_rows(A, B, C, M, N, K, sa, sb, sc, za, zb, 0, M);
}

/* rpl_core.c:521-527.  The reference's `(int32_t)roundf(..) + zero_point`
 * overflows for a NaN / out-of-range value (INT32_MIN) with a negative zero
 * point; its x86 build wraps (a plain `add`), which is restated here as an
 * unsigned add so that the oracle itself has no undefined behaviour. */
void orc_quantize_int8(const float* x, uint32_t n, float scale, int32_t zp, int8_t* q) {
#pragma omp parallel for
    for (uint32_t i = 0; i < n; i++) {
        int32_t quantized = (int32_t)((uint32_t)(int32_t)roundf(x[i] / scale) + (uint32_t)zp);
        if (quantized < -128) quantized = -128;
        if (quantized > 127) quantized = 127;
        q[i] = (int8_t)quantized;
    }
}

/* rpl_quantization.c:79-85 (OpenMP min/max reduction; NaN never selected) */
static void omp_min_max(const float* x, uint32_t n, float* mn, float* mx) {
    float min_val = FLT_MAX, max_val = -FLT_MAX;
#pragma omp parallel for reduction(min : min_val) reduction(max : max_val)
    for (uint32_t i = 0; i < n; i++) {
        if (x[i] < min_val) min_val = x[i];
        if (x[i] > max_val) max_val = x[i];
    }
    *mn = min_val;
    *mx = max_val;
}

/* rpl_quantization.c:77-91 */
float orc_quantize_symmetric(const float* x, uint32_t n, int8_t* q) {
    float min_val, max_val;
    omp_min_max(x, n, &min_val, &max_val);
    float abs_max = fmaxf(fabsf(min_val), fabsf(max_val));
    float scale = abs_max / 127.0f;
    orc_quantize_int8(x, n, scale, 0, q);
    return scale;
}

/* rpl_quantization.c:93-107 */
void orc_quantize_asymmetric(const float* x, uint32_t n, int8_t* q, float* scale_out,
                             int32_t* zp_out) {
    float min_val, max_val;
    omp_min_max(x, n, &min_val, &max_val);
    float range = max_val - min_val;
    float scale = range / 255.0f;
    int32_t zero_point = (int32_t)roundf(-min_val / scale);
    orc_quantize_int8(x, n, scale, zero_point, q);
    *scale_out = scale;
    *zp_out = zero_point;
}

/* rpl_quantization.c:120-160 */
void orc_quantize_per_channel(const float* x, uint32_t num_channels, uint32_t channel_size,
                              int8_t* q, float* scales, int32_t* zero_points) {
#pragma omp parallel for
    for (uint32_t c = 0; c < num_channels; c++) {
        float min_val = FLT_MAX, max_val = -FLT_MAX;
        for (uint32_t i = 0; i < channel_size; i++) {
            uint32_t idx = c * channel_size + i;
            if (x[idx] < min_val) min_val = x[idx];
            if (x[idx] > max_val) max_val = x[idx];
        }
        float abs_max = fmaxf(fabsf(min_val), fabsf(max_val));
        scales[c] = abs_max / 127.0f;
        if (zero_points) zero_points[c] = 0;
        for (uint32_t i = 0; i < channel_size; i++) {
            uint32_t idx = c * channel_size + i;
            int32_t v = (int32_t)roundf(x[idx] / scales[c]);
            v = (v < -128) ? -128 : (v > 127 ? 127 : v);
            q[idx] = (int8_t)v;
        }
    }
}

/* ops_extended.c:64-73 */
void orc_dequantize_int8(const int8_t* q, uint32_t n, float scale, int32_t zp, float* y) {
#pragma omp parallel for
    for (uint32_t i = 0; i < n; i++) y[i] = (q[i] - zp) * scale;
}

/* ops_extended.c:52-61 */
void orc_get_min_max(const float* x, uint32_t n, float* mn, float* mx) {
    if (n == 0) return;
    *mn = x[0];
    *mx = x[0];
    for (uint32_t i = 1; i < n; i++) {
        if (x[i] < *mn) *mn = x[i];
        if (x[i] > *mx) *mx = x[i];
    }
}

/* rpl_quantization.c:33-54 (the per-thread/critical merge is an exact min/max) */
void orc_calibrator_update(const float* x, uint32_t n, float* mn, float* mx) {
    float lo, hi;
    omp_min_max(x, n, &lo, &hi);
    if (lo < *mn) *mn = lo;
    if (hi > *mx) *mx = hi;
}

/* rpl_quantization.c:56-67 */
void orc_calibrator_params(float mn, float mx, bool symmetric, float* scale, int32_t* zp) {
    if (symmetric) {
        float abs_max = fmaxf(fabsf(mn), fabsf(mx));
        *scale = abs_max / 127.0f;
        *zp = 0;
    } else {
        float range = mx - mn;
        *scale = range / 255.0f;
        *zp = (int32_t)roundf(-mn / *scale);
    }
}

/* rpl_quantization.c:314-353 (non-dotprod branch :340-343, bias :346-348) */
void orc_linear_int8(const int8_t* x, const int8_t* w, const int8_t* bias, int32_t* out,
                     uint32_t M, uint32_t K, uint32_t N) {
#pragma omp parallel for
    for (uint32_t b = 0; b < M; b++) {
        for (uint32_t o = 0; o < N; o++) {
            int32_t sum = 0;
            for (uint32_t i = 0; i < K; i++) sum += x[b * K + i] * w[o * K + i];
            if (bias) sum += bias[o];
            out[b * N + o] = sum;
        }
    }
}

/* No reference function: the dequant order of ops_extended.c:119 with sc = 1. */
void orc_dequant_acc(const int32_t* acc, uint32_t M, uint32_t N, const float* sx,
                     bool sx_per_row, const float* sw, bool sw_per_col, float* y) {
#pragma omp parallel for
    for (uint32_t m = 0; m < M; m++) {
        float a = sx[sx_per_row ? m : 0];
        for (uint32_t n = 0; n < N; n++) {
            float v = (float)acc[(size_t)m * N + n] * a;
            y[(size_t)m * N + n] = v * sw[sw_per_col ? n : 0];
        }
    }
}

/* rpl_core.c:95-121 (both branches compute a[i] + b[i % nb]) */
void orc_add_broadcast(const float* a, const float* b, float* out, uint32_t n, uint32_t nb) {
    if (nb == n) {
#pragma omp parallel for
        for (uint32_t i = 0; i < n; i++) out[i] = a[i] + b[i];
    } else {
#pragma omp parallel for
        for (uint32_t i = 0; i < n; i++) {
            float val_b = b[i % nb];
            out[i] = a[i] + val_b;
        }
    }
}

/* rpl_core.c:289-291 */
void orc_relu(const float* x, float* y, uint32_t n) {
#pragma omp parallel for
    for (uint32_t i = 0; i < n; i++) y[i] = (x[i] > 0) ? x[i] : 0;
}

/* rpl_core.c:418-424 */
void orc_relu_backward(const float* x, const float* dy, float* dx, uint32_t n) {
    for (uint32_t i = 0; i < n; i++)
        if (x[i] > 0) dx[i] += dy[i];
}

/* rpl_core.c:319-337 */
void orc_add_backward(const float* dy, uint32_t n, float* da, float* db, uint32_t nb) {
    if (da) {
#pragma omp parallel for
        for (uint32_t i = 0; i < n; i++) da[i] += dy[i];
    }
    if (db) {
#pragma omp parallel for
        for (uint32_t i = 0; i < nb; i++) {
            float g = 0;
            for (uint32_t j = i; j < n; j += nb) g += dy[j];
            db[i] += g;
        }
    }
}

/* rpl_core.c:363-416 */
void orc_matmul_backward(const float* dt, const float* a, const float* b, uint32_t M,
                         uint32_t N, uint32_t K, uint32_t b_rows, uint32_t b_cols, float* da,
                         float* db) {
    bool b_trans = (b_rows == N && b_cols == K);
    if (da) {
#pragma omp parallel for collapse(2)
        for (uint32_t i = 0; i < M; i++) {
            for (uint32_t k = 0; k < K; k++) {
                float sum = 0;
                for (uint32_t j = 0; j < N; j++) {
                    float val_b = b_trans ? b[j * K + k] : b[k * N + j];
                    sum += dt[i * N + j] * val_b;
                }
                da[i * K + k] += sum;
            }
        }
    }
    if (db) {
        if (b_trans) {
#pragma omp parallel for collapse(2)
            for (uint32_t j = 0; j < N; j++) {
                for (uint32_t k = 0; k < K; k++) {
                    float sum = 0;
                    for (uint32_t i = 0; i < M; i++) sum += dt[i * N + j] * a[i * K + k];
                    db[j * K + k] += sum;
                }
            }
        } else {
#pragma omp parallel for collapse(2)
            for (uint32_t k = 0; k < K; k++) {
                for (uint32_t j = 0; j < N; j++) {
                    float sum = 0;
                    for (uint32_t i = 0; i < M; i++) sum += a[i * K + k] * dt[i * N + j];
                    db[k * N + j] += sum;
                }
            }
        }
    }
}

/* rpl_core.c:449-465 */
float orc_mse_loss(const float* pred, const float* target, uint32_t n) {
    float loss = 0;
    for (uint32_t i = 0; i < n; i++) {
        float d = pred[i] - target[i];
        loss += d * d;
    }
    return loss / n;
}

/* rpl_core.c:437-447 */
void orc_mse_backward(const float* pred, const float* target, uint32_t n, float g0,
                      float* dpred) {
    float factor = 2.0f / n;
    for (uint32_t i = 0; i < n; i++) dpred[i] += g0 * factor * (pred[i] - target[i]);
}

/* The reference MLP step: linear_forward (rpl_nn.c:55-77) twice around
 * tensor_relu, tensor_mse_loss, then tensor_backward's DFS (rpl_core.c:467)
 * which visits backward_mse -> backward_add(out2) -> backward_matmul(mm2)
 * [dA first, recursing into backward_relu -> backward_add(out1) ->
 * backward_matmul(mm1) (dW1 only) -> db1, then dW2] -> db2. */
float orc_mlp_step(const float* X, const float* Y, const float* W1, const float* b1,
                   const float* W2, const float* b2, uint32_t B, uint32_t IN, uint32_t H,
                   uint32_t O, float* h, float* a, float* o, float* dW1, float* db1,
                   float* dW2, float* db2) {
    size_t nh = (size_t)B * H, no = (size_t)B * O;
    float* mm1 = (float*)calloc(nh, sizeof(float));
    float* mm2 = (float*)calloc(no, sizeof(float));
    float* g_out2 = (float*)calloc(no, sizeof(float));
    float* g_mm2 = (float*)calloc(no, sizeof(float));
    float* g_a = (float*)calloc(nh, sizeof(float));
    float* g_out1 = (float*)calloc(nh, sizeof(float));
    float* g_mm1 = (float*)calloc(nh, sizeof(float));

    orc_sgemm(X, W1, mm1, B, H, IN, 1.0f, 0.0f, false, true);
    orc_add_broadcast(mm1, b1, h, (uint32_t)nh, H);
    orc_relu(h, a, (uint32_t)nh);
    orc_sgemm(a, W2, mm2, B, O, H, 1.0f, 0.0f, false, true);
    orc_add_broadcast(mm2, b2, o, (uint32_t)no, O);
    float loss = orc_mse_loss(o, Y, (uint32_t)no);

    orc_mse_backward(o, Y, (uint32_t)no, 1.0f, g_out2);
    /* backward_add(out2): a-branch first (recursing fully), then the bias */
    orc_add_backward(g_out2, (uint32_t)no, g_mm2, NULL, O);
    /* backward_matmul(mm2): dA, recurse through relu / layer 1, then dB */
    orc_matmul_backward(g_mm2, a, W2, B, O, H, O, H, g_a, NULL);
    orc_relu_backward(h, g_a, g_out1, (uint32_t)nh);
    orc_add_backward(g_out1, (uint32_t)nh, g_mm1, NULL, H);
    orc_matmul_backward(g_mm1, X, W1, B, H, IN, H, IN, NULL, dW1);
    orc_add_backward(g_out1, (uint32_t)nh, NULL, db1, H);
    orc_matmul_backward(g_mm2, a, W2, B, O, H, O, H, NULL, dW2);
    orc_add_backward(g_out2, (uint32_t)no, NULL, db2, O);

    free(mm1); free(mm2); free(g_out2); free(g_mm2); free(g_a); free(g_out1); free(g_mm1);
    return loss;
}

/* rpl_training.c:70-114 (optimizer_sgd_step) for one parameter tensor: the
 * same loops and expression shapes, so GCC forms the same FMAs.  grad is
 * updated in place (weight decay, Nesterov), as in the reference. */
void orc_sgd_step(float* param, float* grad, float* velocity, uint32_t n, float lr, float momentum,
                  float dampening, float weight_decay, bool nesterov) {
    float* d_p = grad;
    if (weight_decay != 0.0f) {
#pragma omp simd
        for (uint32_t i = 0; i < n; i++) d_p[i] += weight_decay * param[i];
    }
    if (momentum != 0.0f) {
#pragma omp simd
        for (uint32_t i = 0; i < n; i++) velocity[i] = momentum * velocity[i] + (1.0f - dampening) * d_p[i];
        if (nesterov) {
#pragma omp simd
            for (uint32_t i = 0; i < n; i++) d_p[i] += momentum * velocity[i];
        } else {
            d_p = velocity;
        }
    }
#pragma omp simd
    for (uint32_t i = 0; i < n; i++) param[i] -= lr * d_p[i];
}

/* tensor_sigmoid (rpl_core.c:302-304) */
void orc_sigmoid(const float* x, float* y, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) y[i] = 1.0f / (1.0f + expf(-x[i]));
}

/* tensor_tanh_inplace (rpl_core.c:490-491), out of place */
void orc_tanh(const float* x, float* y, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) y[i] = tanhf(x[i]);
}

/* tensor_gelu_inplace (rpl_core.c:493-497), out of place */
void orc_gelu(const float* x, float* y, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) {
        float v = x[i];
        y[i] = 0.5f * v * (1.0f + tanhf(sqrtf(2.0f / M_PI) * (v + 0.044715f * powf(v, 3))));
    }
}

/* scaled_dot_product_attention (rpl_attention.c:16-111) on raw arrays:
 * Q [B,Sq,dk], K [B,Sk,dk], V [B,Sk,dv], mask [B,Sq,Sk] or NULL (0 ->
 * -1e9 before the softmax), out [B,Sq,dv].  Dropout is the reference's
 * no-op stub (rpl_core.c:533), so it does not appear. */
void orc_sdpa(const float* Q, const float* K, const float* V, const float* mask, float* out, uint32_t B,
              uint32_t Sq, uint32_t Sk, uint32_t dk, uint32_t dv) {
    float* scores = (float*)malloc((size_t)B * Sq * Sk * sizeof(float));
    if (!scores) return;
    float scale = 1.0f / sqrtf((float)dk);
#pragma omp parallel for collapse(2)
    for (uint32_t b = 0; b < B; b++) {
        for (uint32_t i = 0; i < Sq; i++) {
            for (uint32_t j = 0; j < Sk; j++) {
                float sum = 0.0f;
                for (uint32_t k = 0; k < dk; k++) sum += Q[b * Sq * dk + i * dk + k] * K[b * Sk * dk + j * dk + k];
                scores[b * Sq * Sk + i * Sk + j] = sum * scale;
            }
        }
    }
    if (mask) {
#pragma omp parallel for
        for (uint32_t i = 0; i < B * Sq * Sk; i++)
            if (mask[i] == 0.0f) scores[i] = -1e9f;
    }
#pragma omp parallel for collapse(2)
    for (uint32_t b = 0; b < B; b++) {
        for (uint32_t i = 0; i < Sq; i++) {
            float* row = &scores[b * Sq * Sk + i * Sk];
            float max_val = -FLT_MAX;
            for (uint32_t j = 0; j < Sk; j++)
                if (row[j] > max_val) max_val = row[j];
            float sum_exp = 0.0f;
            for (uint32_t j = 0; j < Sk; j++) {
                row[j] = expf(row[j] - max_val);
                sum_exp += row[j];
            }
            for (uint32_t j = 0; j < Sk; j++) row[j] /= sum_exp;
        }
    }
#pragma omp parallel for collapse(2)
    for (uint32_t b = 0; b < B; b++) {
        for (uint32_t i = 0; i < Sq; i++) {
            for (uint32_t k = 0; k < dv; k++) {
                float sum = 0.0f;
                for (uint32_t j = 0; j < Sk; j++) sum += scores[b * Sq * Sk + i * Sk + j] * V[b * Sk * dv + j * dv + k];
                out[b * Sq * dv + i * dv + k] = sum;
            }
        }
    }
    free(scores);
}

/* float_to_half_impl (rpl_half.c:10-42): truncating, subnormal results and
 * inputs flush to zero, overflow to infinity, NaN -> 0x7e00 | sign. */
void orc_float_to_half(const float* x, uint16_t* h, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) {
        uint32_t f;
        memcpy(&f, &x[i], 4);
        uint32_t sign = (f >> 31) & 0x01, exp = (f >> 23) & 0xFF, mant = f & 0x7FFFFF;
        uint16_t h_sign = (uint16_t)(sign << 15), h_exp = 0, h_mant = 0;
        if (exp == 255) {
            h_exp = 31;
            h_mant = mant ? 0x200 : 0;
        } else if (exp != 0) {
            int new_exp = (int)exp - 127 + 15;
            if (new_exp >= 31) {
                h_exp = 31;
            } else if (new_exp > 0) {
                h_exp = (uint16_t)new_exp;
                h_mant = (uint16_t)(mant >> 13);
            }
        }
        h[i] = (uint16_t)(h_sign | (h_exp << 10) | h_mant);
    }
}

/* half_to_float_impl (rpl_half.c:44-75): subnormal halves -> 0. */
void orc_half_to_float(const uint16_t* h, float* x, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) {
        uint32_t sign = (h[i] >> 15) & 0x01, exp = (h[i] >> 10) & 0x1F, mant = h[i] & 0x3FF;
        uint32_t f_exp, f_mant;
        if (exp == 31) {
            f_exp = 255;
            f_mant = mant ? 0x7FFFFF : 0;
        } else if (exp == 0) {
            f_exp = 0;
            f_mant = 0;
        } else {
            f_exp = exp + 127 - 15;
            f_mant = mant << 13;
        }
        uint32_t f = (sign << 31) | (f_exp << 23) | f_mant;
        memcpy(&x[i], &f, 4);
    }
}

/* fake_quantize_forward (rpl_quantization.c:195-237) on raw arrays, with the
 * FakeQuantize state as scale / zp in-out: the same expression shapes. */
void orc_fake_quant(const float* x, float* y, uint32_t n, float* scale_io, float* zp_io, bool training) {
    float scale = *scale_io, zp = *zp_io;
    if (training) {
        float min_val = FLT_MAX, max_val = -FLT_MAX;
        for (uint32_t i = 0; i < n; i++) {
            if (x[i] < min_val) min_val = x[i];
            if (x[i] > max_val) max_val = x[i];
        }
        float new_scale = (max_val - min_val) / 255.0f;
        float new_zp = -min_val / new_scale;
        float momentum = 0.1f;
        scale = (1.0f - momentum) * scale + momentum * new_scale;
        zp = (1.0f - momentum) * zp + momentum * new_zp;
        *scale_io = scale;
        *zp_io = zp;
    }
    float inv_scale = 1.0f / scale;
    for (uint32_t i = 0; i < n; i++) {
        int32_t q = (int32_t)roundf(x[i] * inv_scale + zp);
        q = (q < -128) ? -128 : (q > 127 ? 127 : q);
        y[i] = (q - zp) * scale;
    }
}

/*
 * CPU oracle for RPL's GEMM hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference algorithms, used as the checker by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.  Nothing in
 * the product library links, loads or calls this code.  Every function cites
 * the reference file:line it restates (paths relative to the reference repo).
 *
 * Build flags must match the reference's CMakeLists.txt:5 (-O3 -fopenmp
 * -std=gnu11, an FMA-capable -march) so that GCC's default
 * -ffp-contract=fast contracts the same multiply-adds into FMAs and the fp32
 * results are bit-identical to the reference's own build.
 *
 * Parity pins (each function is checked by tests/test_oracle_*.py):
 *   - bit-exact against oracle/_ref (the reference sources compiled as-is),
 *   - against committed golden vectors generated from oracle/_ref,
 *   - against closed forms / brute force (int64 sums, float64 GEMM bounds,
 *     identity products, roundf tie cases, x86 cast edge cases).
 * No function is "parity unpinned".
 */
#ifndef RPL_ORACLE_H
#define RPL_ORACLE_H

#include <stdint.h>
#include <stddef.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

/* rpl_core.c:199-217 tensor_gemm: C = alpha*op(A)*op(B) + beta*C, row-major.
 * A is [M,K] (or [K,M] when ta), B is [K,N] (or [N,K] when tb). */
void orc_sgemm(const float* A, const float* B, float* C, uint32_t M, uint32_t N,
               uint32_t K, float alpha, float beta, bool ta, bool tb);

/* Same as orc_sgemm but only rows [row0,row1) of C: used for the bounded
 * CPU-baseline sample (each row of C costs the same). */
void orc_sgemm_rows(const float* A, const float* B, float* C, uint32_t M, uint32_t N,
                    uint32_t K, float alpha, float beta, bool ta, bool tb,
                    uint32_t row0, uint32_t row1);

/* ops_extended.c:83-123 gemm_int8_fallback (x86 scalar branch :113-117) */
void orc_gemm_int8(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N,
                   uint32_t K, float sa, float sb, float sc, int32_t za, int32_t zb);
void orc_gemm_int8_rows(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M,
                        uint32_t N, uint32_t K, float sa, float sb, float sc, int32_t za,
                        int32_t zb, uint32_t row0, uint32_t row1);

/* rpl_core.c:511-530 tensor_quantize_int8 (element loop only) */
void orc_quantize_int8(const float* x, uint32_t n, float scale, int32_t zp, int8_t* q);

/* rpl_quantization.c:77-91 tensor_quantize_int8_symmetric; returns scale */
float orc_quantize_symmetric(const float* x, uint32_t n, int8_t* q);

/* rpl_quantization.c:93-107 tensor_quantize_int8_asymmetric */
void orc_quantize_asymmetric(const float* x, uint32_t n, int8_t* q, float* scale,
                             int32_t* zp);

/* rpl_quantization.c:120-160 tensor_quantize_per_channel (leading-axis slices
 * of length size/num_channels, whatever channel_axis names) */
void orc_quantize_per_channel(const float* x, uint32_t num_channels, uint32_t channel_size,
                              int8_t* q, float* scales, int32_t* zero_points);

/* ops_extended.c:64-73 tensor_dequantize_int8 */
void orc_dequantize_int8(const int8_t* q, uint32_t n, float scale, int32_t zp, float* y);

/* ops_extended.c:52-61 tensor_get_min_max (sequential; n==0 leaves outputs) */
void orc_get_min_max(const float* x, uint32_t n, float* mn, float* mx);

/* rpl_quantization.c:18-67 QuantizationCalibrator update + compute_params */
void orc_calibrator_update(const float* x, uint32_t n, float* mn, float* mx);
void orc_calibrator_params(float mn, float mx, bool symmetric, float* scale, int32_t* zp);

/* rpl_quantization.c:314-353 linear_int8 (x86 branch :340-343; bias may be NULL) */
void orc_linear_int8(const int8_t* x, const int8_t* w, const int8_t* bias, int32_t* out,
                     uint32_t M, uint32_t K, uint32_t N);

/* Fused dequant epilogue (no reference function; follows the float op order
 * of ops_extended.c:119 with scale_c == 1 and without the roundf):
 * y[m,n] = ((float)acc[m,n] * sx[m or 0]) * sw[n or 0]. */
void orc_dequant_acc(const int32_t* acc, uint32_t M, uint32_t N, const float* sx,
                     bool sx_per_row, const float* sw, bool sw_per_col, float* y);

/* rpl_core.c:95-129 tensor_add_out: out[i] = a[i] + b[i % nb] */
void orc_add_broadcast(const float* a, const float* b, float* out, uint32_t n, uint32_t nb);

/* rpl_core.c:274-300 tensor_relu */
void orc_relu(const float* x, float* y, uint32_t n);

/* rpl_core.c:418-424 backward_relu: dx[i] += dy[i] where x[i] > 0 */
void orc_relu_backward(const float* x, const float* dy, float* dx, uint32_t n);

/* rpl_core.c:319-337 backward_add: da[i] += dy[i]; db[i] += sum_{j = i mod nb} dy[j] */
void orc_add_backward(const float* dy, uint32_t n, float* da, float* db, uint32_t nb);

/* rpl_core.c:363-416 backward_matmul with t=[M,N], a=[M,K], b given by shape
 * (b_rows,b_cols).  da or db may be NULL (no grad). */
void orc_matmul_backward(const float* dt, const float* a, const float* b, uint32_t M,
                         uint32_t N, uint32_t K, uint32_t b_rows, uint32_t b_cols,
                         float* da, float* db);

/* rpl_core.c:449-465 tensor_mse_loss */
float orc_mse_loss(const float* pred, const float* target, uint32_t n);

/* rpl_core.c:437-447 backward_mse */
void orc_mse_backward(const float* pred, const float* target, uint32_t n, float g0,
                      float* dpred);

/* One MLP training step (forward + backward through the reference's
 * autograd order, rpl_core.c:467-476 driving :437, :319, :363, :418) for
 * X[B,IN] -> Linear(IN,H) -> ReLU -> Linear(H,O) -> MSE(Y).
 * Gradients accumulate into dW1, db1, dW2, db2 (caller zeroes them);
 * returns the loss.  h, a, o are [B,H],[B,H],[B,O] forward buffers. */
float orc_mlp_step(const float* X, const float* Y, const float* W1, const float* b1,
                   const float* W2, const float* b2, uint32_t B, uint32_t IN, uint32_t H,
                   uint32_t O, float* h, float* a, float* o, float* dW1, float* db1,
                   float* dW2, float* db2);

/* rpl_training.c:70-114 */
void orc_sgd_step(float* param, float* grad, float* velocity, uint32_t n, float lr, float momentum,
                  float dampening, float weight_decay, bool nesterov);

/* rpl_core.c:302-304, 490-497 */
void orc_sigmoid(const float* x, float* y, uint32_t n);
void orc_tanh(const float* x, float* y, uint32_t n);
void orc_gelu(const float* x, float* y, uint32_t n);

/* rpl_attention.c:16-111 */
void orc_sdpa(const float* Q, const float* K, const float* V, const float* mask, float* out, uint32_t B,
              uint32_t Sq, uint32_t Sk, uint32_t dk, uint32_t dv);

/* rpl_half.c:10-75 */
void orc_float_to_half(const float* x, uint16_t* h, uint32_t n);
void orc_half_to_float(const uint16_t* h, float* x, uint32_t n);
/* rpl_quantization.c:195-237 */
void orc_fake_quant(const float* x, float* y, uint32_t n, float* scale_io, float* zp_io, bool training);

#ifdef __cplusplus
}
#endif
#endif

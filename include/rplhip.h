/*
 * rplhip.h -- the device-side C ABI of the MI355X (gfx950) backend for RPL's
 * GEMM hot path.
 *
 * Plain pointers and sizes only.  All tensor pointers are DEVICE pointers
 * (from rplhip_malloc or any other HIP allocation) in RPL's row-major
 * layouts; every call is asynchronous on `stream` (NULL = the null stream)
 * and returns an rplhip_status.  The reference's synchronous host entry
 * points (include/rpl.h) are implemented on top of this layer.
 *
 * Each compute entry point names the reference function whose semantics it
 * reproduces (paths relative to the reference repo).  There is no CPU
 * fallback: without a usable gfx950 device every call returns
 * RPLHIP_ERR_NO_DEVICE and rplhip_last_error() says why.
 */
#ifndef RPLHIP_H
#define RPLHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    RPLHIP_OK = 0,
    RPLHIP_ERR_INVALID = 1,     /* bad argument: NULL pointer, shape, size */
    RPLHIP_ERR_NO_DEVICE = 2,   /* no usable gfx950 device */
    RPLHIP_ERR_HIP = 3,         /* a HIP runtime call or kernel launch failed */
    RPLHIP_ERR_NOMEM = 4,       /* device allocation failed */
    RPLHIP_ERR_UNSUPPORTED = 5  /* valid request this build does not serve */
} rplhip_status;

typedef void* rplhip_stream_t; /* a hipStream_t */
typedef void* rplhip_event_t;  /* a hipEvent_t */

/* ---------------------------------------------------------------- runtime */

/* Select device 0 and check it is gfx950.  Idempotent and thread-safe; every
 * other entry point calls it implicitly.  Replaces the EGL bring-up of
 * rpl_gpu_init (src/rpl_gpu.c:88-189). */
int rplhip_init(void);
/* Human-readable reason for the last non-OK status on this thread. */
const char* rplhip_last_error(void);
/* Device name (gcnArchName), compute-unit count and peak clock in kHz. */
int rplhip_device_info(char* arch, size_t arch_len, int* cu_count, int* clock_khz);

int rplhip_malloc(void** ptr, size_t bytes);
int rplhip_free(void* ptr);
int rplhip_memcpy_htod(void* dst, const void* src, size_t bytes);
int rplhip_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int rplhip_memcpy_dtod(void* dst, const void* src, size_t bytes, rplhip_stream_t stream);
int rplhip_memset(void* ptr, int value, size_t bytes, rplhip_stream_t stream);
int rplhip_synchronize(void);
int rplhip_stream_create(rplhip_stream_t* stream);
int rplhip_stream_destroy(rplhip_stream_t stream);
int rplhip_stream_synchronize(rplhip_stream_t stream);
int rplhip_event_create(rplhip_event_t* event);
int rplhip_event_destroy(rplhip_event_t event);
int rplhip_event_record(rplhip_event_t event, rplhip_stream_t stream);
int rplhip_event_synchronize(rplhip_event_t event);
int rplhip_event_elapsed_ms(float* ms, rplhip_event_t start, rplhip_event_t stop);

/* ------------------------------------------------------------- FP32 GEMM */

/* C = alpha * op(A) * op(B) + beta * C on f32 MFMA.
 * op(A) is [M,K]: A is [M,K] (lda >= K) or, when trans_a, [K,M] (lda >= M).
 * op(B) is [K,N]: B is [K,N] (ldb >= N) or, when trans_b, [N,K] (ldb >= K).
 * C is [M,N] with ldc >= N.  C is always read (as rpl_core.c:214 does), so a
 * NaN in C propagates even when beta == 0.
 * Replaces tensor_gemm (src/rpl_core.c:199-217) and, with alpha = beta = 1,
 * gemm_optimized_cortex_a72 / parallel_gemm_optimized
 * (src/gemm_optimized.c:127-186, intended C += A*B). */
int rplhip_sgemm(int trans_a, int trans_b, uint32_t M, uint32_t N, uint32_t K, float alpha,
                 const float* A, uint32_t lda, const float* B, uint32_t ldb, float beta,
                 float* C, uint32_t ldc, rplhip_stream_t stream);

/* `batch` GEMMs of one shape in one launch: C_z = alpha * op(A_z) * op(B_z)
 * (+ beta * C_z when read_c), with X_z = X + z * stride_x (elements).
 * read_c = 0 writes C without reading it (beta ignored).  No reference
 * counterpart: it serves scaled_dot_product_attention
 * (src/rpl_attention.c:30-107), whose per-batch tensor_gemm calls it
 * replaces. */
int rplhip_sgemm_batched(int trans_a, int trans_b, uint32_t M, uint32_t N, uint32_t K, float alpha,
                         const float* A, uint32_t lda, uint64_t stride_a, const float* B, uint32_t ldb,
                         uint64_t stride_b, float beta, float* C, uint32_t ldc, uint64_t stride_c,
                         uint32_t batch, int read_c, rplhip_stream_t stream);

/* ------------------------------------------------------------- INT8 GEMM */

/* gemm_int8 (src/ops_extended.c:83-129): A [M,K] int8, B [K,N] int8,
 * acc = sum_k (A - za)(B - zb) in wrapping int32 (i8 MFMA), then
 * C = (int32)roundf(((float)acc * sa) * sb / sc) with the x86 conversion
 * (NaN / out of range -> INT32_MIN).  Uses a device workspace of K*N bytes
 * (plus 4*(M+N) when a zero point is non-zero) from the stream-ordered pool. */
int rplhip_gemm_int8(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N,
                     uint32_t K, float sa, float sb, float sc, int32_t za, int32_t zb,
                     rplhip_stream_t stream);

/* No counterpart in the reference: rplhip_gemm_int8 (same arguments, same
 * results bit for bit) for callers that cannot allocate device memory --
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  It calls no hipMalloc, hipFree or allocating library routine:
 * its scratch (B transposed, K*N bytes, when B cannot be read in place, plus
 * 4*(M+N) bytes of zero-point sums) is a static 16 MiB device array per GPU,
 * held until the process ends.  Calls needing more than 16 MiB of scratch
 * fail with RPLHIP_ERR_UNSUPPORTED.  All calls on one GPU share the array:
 * calls on one stream are ordered and safe, calls that overlap on one GPU
 * (different streams) race. */
int rplhip_gemm_int8_noalloc(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N,
                             uint32_t K, float sa, float sb, float sc, int32_t za, int32_t zb,
                             rplhip_stream_t stream);

/* linear_int8 (src/rpl_quantization.c:314-353): X [M,K] int8, W [N,K] int8
 * (Linear layout), out[m,n] = sum_k X[m,k] W[n,k] (+ bias[n] if bias != NULL),
 * int32.  Zero points are ignored, as in the reference.  M <= 16 runs the
 * bandwidth-bound skinny kernel. */
int rplhip_linear_int8(const int8_t* X, const int8_t* W, const int8_t* bias, int32_t* out,
                       uint32_t M, uint32_t K, uint32_t N, rplhip_stream_t stream);

/* Fused-dequant INT8 linear (no reference function: the int32 result of
 * linear_int8 followed by the float order of src/ops_extended.c:119 with
 * scale_c == 1 and no rounding):
 *   Y[m,n] = ((float)sum_k X[m,k] W[n,k] * x_scale[x_per_row ? m : 0])
 *            * w_scale[w_per_row ? n : 0]
 * x_scale / w_scale are DEVICE pointers (e.g. written by the quantizers
 * below), so a quantize -> GEMM chain never syncs.  M <= 16 runs the skinny
 * kernel. */
int rplhip_linear_int8_dequant(const int8_t* X, const float* x_scale, int x_per_row,
                               const int8_t* W, const float* w_scale, int w_per_row, float* Y,
                               uint32_t M, uint32_t K, uint32_t N, rplhip_stream_t stream);

/* Same epilogue for the gemm_int8 layout (B [K,N], per-tensor or per-column
 * B scales): Y[m,n] = ((float)sum_k A[m,k] B[k,n] * a_scale[..]) * b_scale[..]. */
int rplhip_gemm_int8_dequant(const int8_t* A, const float* a_scale, int a_per_row,
                             const int8_t* B, const float* b_scale, int b_per_col, float* Y,
                             uint32_t M, uint32_t N, uint32_t K, rplhip_stream_t stream);

/* ---------------------------------------------------------- quantization */

/* tensor_quantize_int8 element loop (src/rpl_core.c:521-527):
 * q = clamp((int32)roundf(x / scale) + zp, -128, 127), IEEE division,
 * ties away from zero, x86 conversion. */
int rplhip_quantize_int8(const float* x, uint64_t n, float scale, int32_t zp, int8_t* q,
                         rplhip_stream_t stream);

/* tensor_quantize_int8_symmetric (src/rpl_quantization.c:77-91): min/max
 * reduction (NaN never selected), scale = fmaxf(|min|,|max|) / 127, zp = 0.
 * The scale is written to the DEVICE float *scale_out. */
int rplhip_quantize_symmetric(const float* x, uint64_t n, int8_t* q, float* scale_out,
                              rplhip_stream_t stream);

/* tensor_quantize_int8_asymmetric (src/rpl_quantization.c:93-107):
 * scale = (max - min) / 255, zp = (int32)roundf(-min / scale).
 * scale_out / zp_out are DEVICE pointers. */
int rplhip_quantize_asymmetric(const float* x, uint64_t n, int8_t* q, float* scale_out,
                               int32_t* zp_out, rplhip_stream_t stream);

/* tensor_quantize_per_channel (src/rpl_quantization.c:120-160): the input is
 * num_channels contiguous slices of channel_size elements (leading-axis
 * slicing, as the reference indexes); per slice scale = absmax / 127 and
 * q = clamp((int32)roundf(x / scale)).  Used per output channel for W [N,K]
 * and per token for X [M,K].  scales is a DEVICE float[num_channels]. */
int rplhip_quantize_per_channel(const float* x, uint32_t num_channels, uint32_t channel_size,
                                int8_t* q, float* scales, rplhip_stream_t stream);

/* tensor_dequantize_int8 (src/ops_extended.c:64-73): y = (float)(q - zp) * scale */
int rplhip_dequantize_int8(const int8_t* q, uint64_t n, float scale, int32_t zp, float* y,
                           rplhip_stream_t stream);

/* Min and max as the OpenMP reductions of src/rpl_quantization.c:81-85 and
 * :33-54 compute them (start at +/-FLT_MAX, NaN never selected).
 * out2 is a DEVICE float[2] = {min, max}. */
int rplhip_min_max(const float* x, uint64_t n, float* out2, rplhip_stream_t stream);

/* tensor_get_min_max (src/ops_extended.c:52-61): sequential-scan semantics,
 * i.e. the first element attaining the extreme wins (signed zeros, a NaN in
 * x[0] is returned for both).  n == 0 leaves out2 untouched. */
int rplhip_get_min_max(const float* x, uint64_t n, float* out2, rplhip_stream_t stream);

/* --------------------------------------------- Linear forward / backward */

/* tensor_add_out (src/rpl_core.c:95-129): out[i] = a[i] + b[i % nb]. */
int rplhip_add_broadcast(const float* a, const float* b, float* out, uint64_t n, uint64_t nb,
                         rplhip_stream_t stream);
/* tensor_relu (src/rpl_core.c:274-300): y = x > 0 ? x : 0. */
int rplhip_relu(const float* x, float* y, uint64_t n, rplhip_stream_t stream);
/* Fused Linear epilogue: out = mm + b[i % nb]; act = relu(out) (act may be
 * NULL).  Same values as tensor_add_out followed by tensor_relu. */
int rplhip_bias_add_relu(const float* mm, const float* b, float* out, float* act, uint64_t n,
                         uint64_t nb, rplhip_stream_t stream);
/* backward_relu (src/rpl_core.c:418-424): dx[i] += dy[i] where x[i] > 0. */
int rplhip_relu_backward(const float* x, const float* dy, float* dx, uint64_t n,
                         rplhip_stream_t stream);
/* backward_add's first branch (src/rpl_core.c:322-326): dx[i] += dy[i]. */
int rplhip_accumulate(const float* dy, float* dx, uint64_t n, rplhip_stream_t stream);
/* backward_add's broadcast branch (src/rpl_core.c:327-336), the bias-gradient
 * column reduction: db[i] += sum_{j = i mod nb} dy[j] (rows of dy [n/nb, nb]). */
int rplhip_bias_grad(const float* dy, uint64_t n, float* db, uint64_t nb,
                     rplhip_stream_t stream);
/* tensor_mse_loss (src/rpl_core.c:449-465): *loss = sum (p - t)^2 / n, DEVICE
 * float* loss. */
int rplhip_mse_loss(const float* pred, const float* target, uint64_t n, float* loss,
                    rplhip_stream_t stream);
/* backward_mse (src/rpl_core.c:437-447): dp[i] += g0 * (2/n) * (p[i] - t[i]),
 * g0 read from the DEVICE float *g0. */
int rplhip_mse_backward(const float* pred, const float* target, uint64_t n, const float* g0,
                        float* dpred, rplhip_stream_t stream);
/* y = activation(x) elementwise, DEVICE pointers (the device seam's
 * tensor_sigmoid_gpu / tensor_tanh_gpu / tensor_gelu_gpu, src/rpl_gpu.c:
 * 437-522, with the CPU formulas of src/rpl_core.c:302-304 and 490-497):
 * sigmoid 1/(1+exp(-x)); tanh; gelu 0.5x(1+tanh(sqrt(2/pi)(x+0.044715x^3))).
 * Within a few float32 ulp of glibc (the device's exp/tanh/pow differ). */
int rplhip_sigmoid(const float* x, float* y, uint64_t n, rplhip_stream_t stream);
int rplhip_tanh(const float* x, float* y, uint64_t n, rplhip_stream_t stream);
int rplhip_gelu(const float* x, float* y, uint64_t n, rplhip_stream_t stream);
/* scaled_dot_product_attention (src/rpl_attention.c:16-111), DEVICE pointers:
 * Q [B,Sq,dk], K [B,Sk,dk], V [B,Sk,dv], mask [B,Sq,Sk] or NULL (entries
 * == 0 become -1e9 before the softmax), out [B,Sq,dv].  scores =
 * (Q K^T) * (1/sqrtf(dk)) on the FP32 GEMM, row softmax, out = P V.  Uses a
 * B*Sq*Sk-float workspace. */
int rplhip_attention(const float* Q, const float* K, const float* V, const float* mask, float* out,
                     uint32_t B, uint32_t Sq, uint32_t Sk, uint32_t dk, uint32_t dv, rplhip_stream_t stream);
/* fake_quantize_forward's elementwise step (src/rpl_quantization.c:226-233),
 * DEVICE pointers: y = (clamp(roundf(x * (1/scale) + zp), -128, 127) - zp)
 * * scale, bit-exact with the reference (its fused multiply-add included). */
int rplhip_fake_quant(const float* x, float* y, uint64_t n, float scale, float zero_point, rplhip_stream_t stream);
/* The FP16 codec of src/rpl_half.c:10-75, DEVICE pointers, bit-exact:
 * float -> half truncates, flushes subnormals to zero and overflows to inf;
 * half -> float flushes subnormal halves to zero. */
int rplhip_float_to_half(const float* x, uint16_t* h, uint64_t n, rplhip_stream_t stream);
int rplhip_half_to_float(const uint16_t* h, float* x, uint64_t n, rplhip_stream_t stream);
/* optimizer_sgd_step (src/rpl_training.c:70-114) on one parameter tensor of
 * n floats, all DEVICE pointers: weight decay and Nesterov update grad in
 * place as the reference does; velocity (the momentum buffer) may be NULL
 * when momentum == 0. */
int rplhip_sgd_step(float* param, float* grad, float* velocity, uint64_t n, float lr, float momentum,
                    float dampening, float weight_decay, int nesterov, rplhip_stream_t stream);
/* Fill a DEVICE float buffer with a value (tensor_fill, src/rpl_core.c:83-86). */
int rplhip_fill(float* x, uint64_t n, float value, rplhip_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* RPLHIP_H */

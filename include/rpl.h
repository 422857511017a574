/*
 * rpl.h -- RPL's public C API for the GEMM hot path, served by the MI355X
 * (gfx950) backend.
 *
 * Every type keeps the reference's field order and sizes, and every function
 * keeps the reference's name, signature, ownership rule and accumulate-into
 * semantics, so existing callers (C code, the ctypes bindings) relink
 * unchanged.  Citations are path:line in the reference repository.
 *
 * Residency: a Tensor whose `device` is DEVICE_GPU keeps its authoritative
 * values in device memory; `gpu_buffer` is a handle into this library's
 * device-buffer registry (the reference stored a GL buffer name there, which
 * is why the field is 32 bits).  Operations whose inputs are all
 * GPU-resident run with no host copies and without synchronizing; results
 * are GPU-resident.  Operations on host tensors stage them through device
 * memory, compute on the GPU and copy the result back before returning.
 * There is no CPU compute path: without a gfx950 device the calls print the
 * reason, set rpl_last_error() and leave their outputs untouched.
 */
#ifndef RPL_H
#define RPL_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* include/rpl.h:23-26 */
typedef enum { DEVICE_CPU, DEVICE_GPU } DeviceType;

/* include/rpl.h:32-35 */
#define MAX_DIMS 8
#define RPL_MAX_DIMS MAX_DIMS
#define RPITORCH_MAX_DIMS MAX_DIMS
#define RPITORCH_CACHE_LINE 64

/* include/rpl.h:57-78 -- same field order and types */
typedef struct Tensor {
    float* data;
    float* grad;
    uint32_t dims;
    uint32_t shape[MAX_DIMS];
    uint32_t strides[MAX_DIMS];
    uint32_t size;
    bool requires_grad;
    void* _allocation;
    size_t _alloc_size;
    DeviceType device;
    uint32_t gpu_buffer; /* device-buffer registry handle (0 = none) */
    bool is_leaf;
    struct Tensor* parent1;
    struct Tensor* parent2;
    void (*backward_fn)(struct Tensor*);
} Tensor;

/* include/rpl.h:80-92 */
typedef uint16_t rpl_half;
typedef struct HalfTensor {
    rpl_half* data;
    uint32_t dims;
    uint32_t shape[MAX_DIMS];
    uint32_t strides[MAX_DIMS];
    uint32_t size;
    void* _allocation;
    DeviceType device;
    uint32_t gpu_buffer;
} HalfTensor;

/* include/rpl.h:167-174 */
typedef struct {
    int8_t* data;
    float scale;
    int32_t zero_point;
    uint32_t size;
    uint32_t dims;
    uint32_t shape[MAX_DIMS];
} QuantizedTensor;

/* src/rpl_quantization.c:110-118 (defined in the .c there; exposed here) */
typedef struct {
    int8_t* data;
    float* scales;
    int32_t* zero_points;
    uint32_t num_channels;
    uint32_t channel_size;
    uint32_t dims;
    uint32_t shape[RPITORCH_MAX_DIMS];
} PerChannelQuantizedTensor;

/* src/rpl_quantization.c:18-24 (defined in the .c there; exposed here) */
typedef struct {
    float min_val;
    float max_val;
    float scale;
    int32_t zero_point;
    uint32_t num_samples;
} QuantizationCalibrator;

/* src/rpl_nn.c:16-21 (opaque in the reference header; layout kept) */
typedef struct Linear Linear;
struct Linear {
    Tensor* weight; /* [out_features, in_features] */
    Tensor* bias;   /* [out_features] */
    uint32_t in_features;
    uint32_t out_features;
};

/* ---- memory (include/rpl.h:99-102, src/rpl_core.c:33-77) ---- */
Tensor* tensor_create(uint32_t dims, const uint32_t* shape, bool requires_grad);
void tensor_free(Tensor* t); /* also releases the device buffers */
void* rpitorch_aligned_alloc(size_t alignment, size_t size);
void rpitorch_aligned_free(void* ptr);
void tensor_fill(Tensor* t, float value); /* include/rpl.h:122 */

/* ---- device seam (include/rpl.h:105-111, src/rpl_gpu.c) ---- */
bool rpl_gpu_init(void);
void rpl_gpu_shutdown(void);
void tensor_to_gpu(Tensor* t);   /* upload data (and grad), device = GPU */
void tensor_from_gpu(Tensor* t); /* download data (and grad); stays GPU-resident */
void tensor_add_gpu(Tensor* out, const Tensor* a, const Tensor* b);
void tensor_matmul_gpu(Tensor* C, const Tensor* A, const Tensor* B);
void tensor_relu_gpu(Tensor* out, const Tensor* in);
/* include/rpl.h:112-114: elementwise on the device; an output that is not
 * resident takes in's shape (its host buffer must hold in->size floats). */
void tensor_sigmoid_gpu(Tensor* out, const Tensor* in);
void tensor_tanh_gpu(Tensor* out, const Tensor* in);
void tensor_gelu_gpu(Tensor* out, const Tensor* in);

/* ---- FP32 GEMM ---- */
/* include/rpl.h:130, src/rpl_core.c:199-217 */
void tensor_gemm(Tensor* C, const Tensor* A, const Tensor* B, float alpha, float beta, bool trans_a,
                 bool trans_b);
/* include/rpl.h:131, src/rpl_core.c:177-193 */
Tensor* tensor_matmul(const Tensor* a, const Tensor* b);
/* src/gemm_optimized.c:127-186: C += A*B (the intended semantics) */
void gemm_optimized_cortex_a72(const float* A, const float* B, float* C, int M, int N, int K, int lda,
                               int ldb, int ldc);
void parallel_gemm_optimized(const float* A, const float* B, float* C, uint32_t M, uint32_t N,
                             uint32_t K);
void gemm_init_buffers(void);
void gemm_free_buffers(void);

/* ---- INT8 (include/rpl.h:176-187, src/rpl_quantization.c) ---- */
QuantizedTensor* tensor_quantize_int8(const Tensor* input, float scale, int32_t zero_point);
QuantizedTensor* tensor_quantize_int8_symmetric(const Tensor* input);
QuantizedTensor* tensor_quantize_int8_asymmetric(const Tensor* input);
PerChannelQuantizedTensor* tensor_quantize_per_channel(const Tensor* input, uint32_t channel_axis);
void per_channel_quantized_tensor_free(PerChannelQuantizedTensor* qt);
void quantized_tensor_free(QuantizedTensor* qt);
void tensor_get_min_max(const Tensor* t, float* min_val, float* max_val);
Tensor* tensor_dequantize_int8(QuantizedTensor* input);
void gemm_int8(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N, uint32_t K,
               float sa, float sb, float sc, int32_t za, int32_t zb);
void linear_int8(const QuantizedTensor* input, const QuantizedTensor* weight,
                 const QuantizedTensor* bias, int32_t* output, uint32_t batch_size,
                 uint32_t in_features, uint32_t out_features);
QuantizationCalibrator* calibrator_create(void);
void calibrator_update(QuantizationCalibrator* cal, const Tensor* t);
void calibrator_compute_params(QuantizationCalibrator* cal, bool symmetric);
void calibrator_free(QuantizationCalibrator* cal);

/* ---- Linear layer and its autograd (include/rpl.h:126-161,180,230-232) ---- */
Tensor* tensor_add(const Tensor* a, const Tensor* b);
void tensor_add_out(Tensor* out, const Tensor* a, const Tensor* b);
Tensor* tensor_relu(const Tensor* t);
Tensor* tensor_mse_loss(const Tensor* pred, const Tensor* target);
void tensor_backward(Tensor* t);
void tensor_zero_grad(Tensor* t);
void backward_add(Tensor* t);
void backward_matmul(Tensor* t);
void backward_relu(Tensor* t);
void backward_mse(Tensor* t);
Linear* linear_create(uint32_t in_features, uint32_t out_features);
Tensor* linear_forward(Linear* layer, const Tensor* input);
void linear_free(Linear* layer);

/* ---- FP16 codec (include/rpl.h:117-119, src/rpl_half.c), bit-exact with
 * the reference: float -> half truncates and flushes subnormals; the result
 * of tensor_to_half always holds its values in host memory. ---- */
HalfTensor* tensor_to_half(const Tensor* t);
Tensor* tensor_from_half(const HalfTensor* t);
void half_tensor_free(HalfTensor* t);

/* ---- QAT fake quantization (src/rpl_quantization.c:170-260; exported
 * there, not declared in the reference header).  Layout:
 * { Tensor* scale; Tensor* zero_point; bool training;
 *   uint32_t num_batches_tracked; } ---- */
typedef struct FakeQuantize FakeQuantize;
FakeQuantize* fake_quantize_create(void);
Tensor* fake_quantize_forward(FakeQuantize* fq, const Tensor* input);
void backward_fake_quant(Tensor* t);
void fake_quantize_free(FakeQuantize* fq);

/* ---- attention (src/rpl_attention.c:16-111; exported there, not declared
 * in the reference header): Q [B,Sq,dk], K [B,Sk,dk], V [B,Sk,dv], mask
 * with B*Sq*Sk elements or NULL; dropout is a no-op as in the reference. ---- */
Tensor* scaled_dot_product_attention(const Tensor* Q, const Tensor* K, const Tensor* V, const Tensor* mask,
                                     float dropout_p, bool training);

/* ---- SGD optimizer step on the device (include/rpl.h:306-316,
 * src/rpl_training.c:20-114).  Optimizer is opaque; its layout is the
 * reference's, so optimizers made by either library interoperate with the
 * reference's optimizer_step / optimizer_free / schedulers. ---- */
typedef enum {
    OPTIMIZER_SGD,
    OPTIMIZER_ADAM,
    OPTIMIZER_RMSPROP,
    OPTIMIZER_ADAGRAD,
    OPTIMIZER_ADAMW,
    OPTIMIZER_LAMB
} OptimizerType;
typedef struct Optimizer Optimizer;
Optimizer* optimizer_sgd_create(Tensor** parameters, uint32_t num_params, float lr, float momentum,
                                float dampening, float weight_decay, bool nesterov);
/* src/rpl_training.c:70-114 (exported there, called by optimizer_step). */
void optimizer_sgd_step(Optimizer* opt);

/* ---- additions of this backend (no reference counterpart) ---- */
/* Reason for the last failure on this thread ("" if none). */
const char* rpl_last_error(void);
/* Forget the recorded failure (rpl_last_error() returns "" again). */
void rpl_clear_last_error(void);
/* Wait for all queued device work of this library. */
void rpl_gpu_synchronize(void);
/* The library's HIP stream (a hipStream_t), for callers that mix in their
 * own rplhip_* calls on GPU-resident tensors. */
void* rpl_gpu_stream(void);
/* Device pointer behind a GPU-resident tensor's data / grad (NULL if none). */
float* rpl_tensor_device_data(const Tensor* t);
float* rpl_tensor_device_grad(const Tensor* t);
/* Seeded, platform-independent inputs: element i depends only on (seed, i).
 * splitmix64(seed + (i+1)*0x9E3779B97F4A7C15) -> top 24 bits -> [0,1);
 * uniform = lo + (hi-lo)*u; normal = Box-Muller in double from two draws
 * (2i, 2i+1), then mean + std*z rounded to float. */
void rpl_fill_uniform(float* out, uint64_t n, uint64_t seed, float lo, float hi);
void rpl_fill_normal(float* out, uint64_t n, uint64_t seed, float mean, float std);
/* labels[i] = top bits of the stream, modulo classes; one_hot (if not NULL)
 * is [n, classes] with 1.0 at the label. */
void rpl_fill_labels(uint32_t* labels, float* one_hot, uint64_t n, uint64_t seed, uint32_t classes);

#ifdef __cplusplus
}
#endif
#endif /* RPL_H */

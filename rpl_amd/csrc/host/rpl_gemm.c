/*
 * The reference's GEMM entry points (FP32 and INT8) on the gfx950 backend.
 * Host tensors are staged through device memory; GPU-resident tensors are
 * used in place (no copies, no synchronization).
 */
#include <stdio.h>
#include <string.h>

#include "rpl_host.h"

/* src/rpl_core.c:199-217.  M and K come from A's shape[0..1] and N from
 * B's, whatever the tensors' ranks, and B's own inner dimension is not
 * consulted -- exactly as in the reference: it reads A as a dense [M,K]
 * (or [K,M]) matrix, B as [K,N] (or [N,K]) and C as [M,N], each from its
 * first elements.  multi_head_attention_forward (src/rpl_attention.c:175-177,
 * 232) relies on this with 3-D [batch, seq, d_model] tensors (M = batch,
 * K = seq).  Where the reference stays inside its buffers (M*K, N*K and M*N
 * within the tensors' sizes) the result is the same; where it would read or
 * write past them, the call is refused. */
void tensor_gemm(Tensor* C, const Tensor* A, const Tensor* B, float alpha, float beta, bool trans_a,
                 bool trans_b) {
    if (!C || !A || !B) {
        rpl__bad("tensor_gemm", "NULL tensor");
        return;
    }
    uint32_t M = trans_a ? A->shape[1] : A->shape[0];
    uint32_t K = trans_a ? A->shape[0] : A->shape[1];
    uint32_t N = trans_b ? B->shape[0] : B->shape[1];
    if (A->dims < 2 || B->dims < 2 || (uint64_t)M * K > A->size || (uint64_t)N * K > B->size ||
        (uint64_t)M * N > C->size) {
        rpl__bad("tensor_gemm", "out of bounds: op(A) %ux%u of %u, op(B) %ux%u of %u, C %ux%u of %u elements", M, K,
                 A->size, K, N, B->size, M, N, C->size);
        return;
    }
    if (!rpl_gpu_init()) return;
    RplStage s = {0};
    const float* dA = rpl__view_data(&s, A, 1, 0);
    const float* dB = rpl__view_data(&s, B, 1, 0);
    float* dC = rpl__view_data(&s, C, 1, 1);
    if (!s.err)
        s.err = !rpl__ok(rplhip_sgemm(trans_a, trans_b, M, N, K, alpha, dA, trans_a ? M : K, dB,
                                      trans_b ? K : N, beta, dC, N, NULL),
                         "tensor_gemm");
    rpl__stage_finish(&s);
}

/* src/rpl_core.c:177-193 */
Tensor* tensor_matmul(const Tensor* a, const Tensor* b) {
    uint32_t M = a->shape[a->dims - 2];
    uint32_t N = b->shape[b->dims - 1];
    uint32_t shape[2] = {M, N};
    const int gpu = rpl__is_gpu(a) || rpl__is_gpu(b);
    Tensor* out = (gpu ? rpl__tensor_create_gpu : tensor_create)(2, shape, a->requires_grad || b->requires_grad);
    if (!out) return NULL;
    if (gpu && !rpl__attach(out, 0)) return out;
    /* Zero C (the GEMM reads it even with beta = 0): on the device only when
     * resident, the host copy being stale until tensor_from_gpu. */
    if (gpu)
        rpl__ok(rplhip_fill(rpl__dev_data(out), out->size, 0.0f, NULL), "tensor_matmul");
    else
        tensor_fill(out, 0.0f);
    tensor_gemm(out, a, b, 1.0f, 0.0f, false, false);
    if (out->requires_grad) {
        out->parent1 = (Tensor*)a;
        out->parent2 = (Tensor*)b;
        out->backward_fn = backward_matmul;
        out->is_leaf = false;
    }
    return out;
}

/* include/rpl.h:110, src/rpl_gpu.c:354-400: C = A * B with A [M,K], B [K,N]. */
void tensor_matmul_gpu(Tensor* C, const Tensor* A, const Tensor* B) {
    if (!rpl_gpu_init()) return;
    uint32_t M = A->shape[0], K = A->shape[1], N = B->shape[1];
    if (B->shape[0] != K) {
        rpl__bad("tensor_matmul_gpu", "GEMM shape mismatch: %ux%u vs %ux%u", M, K, B->shape[0], N);
        return;
    }
    tensor_to_gpu((Tensor*)A);
    tensor_to_gpu((Tensor*)B);
    if (!rpl__is_gpu(C)) {
        C->shape[0] = M;
        C->shape[1] = N;
        if (C->dims < 2) C->dims = 2;
        if ((uint64_t)M * N > C->size) {
            rpl__bad("tensor_matmul_gpu", "output holds %u elements, needs %u", C->size, M * N);
            return;
        }
        C->size = M * N;
        if (!rpl__attach(C, 0)) return;
    }
    tensor_gemm(C, A, B, 1.0f, 0.0f, false, false);
}

/* src/gemm_optimized.c:127-180 with the intended semantics C += A*B
 * (the reference kernel's packed-panel indexing is wrong for N != 4). */
void gemm_optimized_cortex_a72(const float* A, const float* B, float* C, int M, int N, int K, int lda,
                               int ldb, int ldc) {
    if (M <= 0 || N <= 0) return;
    if (K < 0 || lda < (K > 0 ? K : 0) || ldb < N || ldc < N || (K > 0 && (!A || !B)) || !C) {
        rpl__bad("gemm_optimized_cortex_a72", "bad arguments");
        return;
    }
    if (!rpl_gpu_init()) return;
    RplStage s = {0};
    size_t na = K ? (size_t)(M - 1) * lda + K : 0;
    size_t nb = K ? (size_t)(K - 1) * ldb + N : 0;
    size_t nc = (size_t)(M - 1) * ldc + N;
    const float* dA = K ? rpl__stage_host(&s, (void*)A, na * sizeof(float), 1, 0) : NULL;
    const float* dB = K ? rpl__stage_host(&s, (void*)B, nb * sizeof(float), 1, 0) : NULL;
    float* dC = rpl__stage_host(&s, C, nc * sizeof(float), 1, 1);
    if (!s.err)
        s.err = !rpl__ok(rplhip_sgemm(0, 0, (uint32_t)M, (uint32_t)N, (uint32_t)K, 1.0f, dA, (uint32_t)lda, dB,
                                      (uint32_t)ldb, 1.0f, dC, (uint32_t)ldc, NULL),
                         "gemm_optimized_cortex_a72");
    rpl__stage_finish(&s);
}

/* src/gemm_optimized.c:183-186 */
void parallel_gemm_optimized(const float* A, const float* B, float* C, uint32_t M, uint32_t N, uint32_t K) {
    gemm_optimized_cortex_a72(A, B, C, (int)M, (int)N, (int)K, (int)K, (int)N, (int)N);
}

/* src/gemm_optimized.c:23-33: the device kernel needs no packing buffers. */
void gemm_init_buffers(void) {}
void gemm_free_buffers(void) {}

/* include/rpl.h:187, src/ops_extended.c:83-129 */
void gemm_int8(const int8_t* A, const int8_t* B, int32_t* C, uint32_t M, uint32_t N, uint32_t K, float sa,
               float sb, float sc, int32_t za, int32_t zb) {
    if (M == 0 || N == 0) return;
    if (!C || (K && (!A || !B))) {
        rpl__bad("gemm_int8", "NULL pointer");
        return;
    }
    if (!rpl_gpu_init()) return;
    RplStage s = {0};
    const int8_t* dA = rpl__stage_host(&s, (void*)A, (size_t)M * K, 1, 0);
    const int8_t* dB = rpl__stage_host(&s, (void*)B, (size_t)K * N, 1, 0);
    int32_t* dC = rpl__stage_host(&s, C, (size_t)M * N * sizeof(int32_t), 0, 1);
    if (!s.err) s.err = !rpl__ok(rplhip_gemm_int8(dA, dB, dC, M, N, K, sa, sb, sc, za, zb, NULL), "gemm_int8");
    rpl__stage_finish(&s);
}

/* src/rpl_quantization.c:314-353 */
void linear_int8(const QuantizedTensor* input, const QuantizedTensor* weight, const QuantizedTensor* bias,
                 int32_t* output, uint32_t batch_size, uint32_t in_features, uint32_t out_features) {
    if (batch_size == 0 || out_features == 0) return;
    if (!input || !weight || !output) {
        rpl__bad("linear_int8", "NULL argument");
        return;
    }
    if (!rpl_gpu_init()) return;
    RplStage s = {0};
    const int8_t* dX = rpl__stage_host(&s, input->data, (size_t)batch_size * in_features, 1, 0);
    const int8_t* dW = rpl__stage_host(&s, weight->data, (size_t)out_features * in_features, 1, 0);
    const int8_t* dBias = bias ? rpl__stage_host(&s, bias->data, out_features, 1, 0) : NULL;
    int32_t* dO = rpl__stage_host(&s, output, (size_t)batch_size * out_features * sizeof(int32_t), 0, 1);
    if (!s.err)
        s.err = !rpl__ok(rplhip_linear_int8(dX, dW, dBias, dO, batch_size, in_features, out_features, NULL),
                         "linear_int8");
    rpl__stage_finish(&s);
}

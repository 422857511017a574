/*
 * scaled_dot_product_attention (src/rpl_attention.c:16-111) on the device.
 *
 * Q [B,Sq,dk], K [B,Sk,dk], V [B,Sk,dv] as 3-D tensors, mask (optional)
 * with B*Sq*Sk elements; returns out [B,Sq,dv] (GPU-resident when an input
 * is).  Dropout is the reference's no-op (tensor_dropout is an empty stub,
 * src/rpl_core.c:533), so dropout_p and training change nothing here
 * either.  Shapes are checked: the reference reads out of bounds when they
 * disagree.
 */
#include "rpl_host.h"

Tensor* scaled_dot_product_attention(const Tensor* Q, const Tensor* K, const Tensor* V, const Tensor* mask,
                                     float dropout_p, bool training) {
    (void)dropout_p;
    (void)training;
    if (!Q || !K || !V || Q->dims != 3 || K->dims != 3 || V->dims != 3) {
        rpl__bad("scaled_dot_product_attention", "Q, K, V must be 3-D tensors [batch, seq, dim]");
        return NULL;
    }
    const uint32_t B = Q->shape[0], Sq = Q->shape[1], dk = Q->shape[2];
    const uint32_t Sk = K->shape[1], dv = V->shape[2];
    if (K->shape[0] != B || K->shape[2] != dk || V->shape[0] != B || V->shape[1] != Sk) {
        rpl__bad("scaled_dot_product_attention", "shapes Q [%u,%u,%u], K [%u,%u,%u], V [%u,%u,%u] disagree", B, Sq,
                 dk, K->shape[0], Sk, K->shape[2], V->shape[0], V->shape[1], dv);
        return NULL;
    }
    if (mask && (uint64_t)mask->size != (uint64_t)B * Sq * Sk) {
        rpl__bad("scaled_dot_product_attention", "mask has %u elements, scores %llu", mask->size,
                 (unsigned long long)B * Sq * Sk);
        return NULL;
    }
    const int gpu = rpl__is_gpu(Q) || rpl__is_gpu(K) || rpl__is_gpu(V);
    const uint32_t shape[3] = {B, Sq, dv};
    Tensor* out = (gpu ? rpl__tensor_create_gpu : tensor_create)(3, shape, Q->requires_grad);
    if (!out) return NULL;
    if (gpu && !rpl__attach(out, 0)) return out;
    if (!rpl_gpu_init()) return out;
    RplStage s = {0};
    const float* dq = rpl__view_data(&s, Q, 1, 0);
    const float* dkp = rpl__view_data(&s, K, 1, 0);
    const float* dvp = rpl__view_data(&s, V, 1, 0);
    const float* dm = mask ? rpl__view_data(&s, mask, 1, 0) : NULL;
    float* dout = rpl__view_data(&s, out, 0, 1);
    if (!s.err)
        s.err = !rpl__ok(rplhip_attention(dq, dkp, dvp, dm, dout, B, Sq, Sk, dk, dv, NULL),
                         "scaled_dot_product_attention");
    rpl__stage_finish(&s);
    return out;
}

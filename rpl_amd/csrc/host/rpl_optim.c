/*
 * optimizer_sgd_create / optimizer_sgd_step (src/rpl_training.c:42-114)
 * with the update on the device.
 *
 * struct Optimizer and struct SGDState are opaque in rpl.h; the layouts
 * below are the reference's (src/rpl_training.c:20-39), so an optimizer made
 * by either library works with the other's optimizer_step, optimizer_free
 * and learning-rate schedulers, which read these fields directly.
 *
 * A GPU-resident parameter is updated in place with no copies; its momentum
 * buffer moves to the device at the first step and stays there (its host
 * copy is then stale, like any resident tensor's).  Host-resident
 * parameters are staged through device memory for the call.
 */
#include <stdlib.h>

#include "rpl_host.h"

struct Optimizer {
    OptimizerType type;
    float learning_rate;
    float weight_decay;
    uint32_t num_params;
    Tensor** parameters;
    void* state;
};

struct SGDState {
    float momentum;
    float dampening;
    bool nesterov;
    Tensor** velocity; /* momentum buffers, only when momentum > 0 */
};

/* src/rpl_training.c:42-68 */
Optimizer* optimizer_sgd_create(Tensor** parameters, uint32_t num_params, float lr, float momentum,
                                float dampening, float weight_decay, bool nesterov) {
    Optimizer* opt = (Optimizer*)calloc(1, sizeof(Optimizer));
    struct SGDState* state = (struct SGDState*)calloc(1, sizeof(struct SGDState));
    if (!opt || !state) {
        free(opt);
        free(state);
        rpl__bad("optimizer_sgd_create", "out of host memory");
        return NULL;
    }
    opt->type = OPTIMIZER_SGD;
    opt->learning_rate = lr;
    opt->weight_decay = weight_decay;
    opt->num_params = num_params;
    opt->parameters = parameters;
    state->momentum = momentum;
    state->dampening = dampening;
    state->nesterov = nesterov;
    if (momentum > 0.0f) {
        state->velocity = (Tensor**)calloc(num_params, sizeof(Tensor*));
        for (uint32_t i = 0; state->velocity && i < num_params; i++) {
            state->velocity[i] = tensor_create(parameters[i]->dims, parameters[i]->shape, false);
            if (state->velocity[i]) tensor_fill(state->velocity[i], 0.0f);
        }
    }
    opt->state = state;
    return opt;
}

/* src/rpl_training.c:70-114 */
void optimizer_sgd_step(Optimizer* opt) {
    if (!opt || !opt->state) return;
    struct SGDState* st = (struct SGDState*)opt->state;
    /* Device-resident parameters are updated RPL_SGD_MULTI per launch (the
     * parameters are independent, so the order of launches does not matter). */
    RplSgdTensors batch;
    batch.count = 0;
    for (uint32_t p = 0; p < opt->num_params; p++) {
        Tensor* param = opt->parameters[p];
        if (!param || !param->grad) continue;
        Tensor* v = NULL;
        if (st->momentum != 0.0f) {
            v = st->velocity ? st->velocity[p] : NULL;
            if (!v) {
                rpl__bad("optimizer_sgd_step", "momentum %g but no momentum buffer for parameter %u",
                         (double)st->momentum, p);
                return;
            }
            if (rpl__is_gpu(param) && !rpl__is_gpu(v) && !rpl__attach(v, 1)) return;
        }
        if (rpl__is_gpu(param) && (!v || rpl__is_gpu(v))) {
            float* dg = rpl__dev_grad_ready(param);
            if (!dg) {
                rpl__bad("optimizer_sgd_step", "GPU parameter %u has no device gradient", p);
                return;
            }
            const int k = batch.count++;
            batch.p[k] = rpl__dev_data(param);
            batch.g[k] = dg;
            batch.v[k] = v ? rpl__dev_data(v) : NULL;
            batch.n[k] = param->size;
            if (batch.count == RPL_SGD_MULTI) {
                if (!rpl__ok(rplhip__sgd_step_multi(&batch, opt->learning_rate, st->momentum, st->dampening,
                                                    opt->weight_decay, st->nesterov, NULL),
                             "optimizer_sgd_step"))
                    return;
                batch.count = 0;
            }
            continue;
        }
        RplStage s = {0};
        float* dp = rpl__view_data(&s, param, 1, 1);
        float* dg = rpl__view_grad(&s, param, 1, 1);
        float* dv = v ? rpl__view_data(&s, v, 1, 1) : NULL;
        if (!s.err)
            s.err = !rpl__ok(rplhip_sgd_step(dp, dg, dv, param->size, opt->learning_rate, st->momentum,
                                             st->dampening, opt->weight_decay, st->nesterov, NULL),
                             "optimizer_sgd_step");
        if (!rpl__stage_finish(&s)) return;
    }
    if (batch.count)
        rpl__ok(rplhip__sgd_step_multi(&batch, opt->learning_rate, st->momentum, st->dampening, opt->weight_decay,
                                       st->nesterov, NULL),
                "optimizer_sgd_step");
}

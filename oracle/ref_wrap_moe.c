/*
 * ref_wrap_moe.c -- exports the reference's header-only routing / f32 MoE code
 * (moe_route.h, moe_exec.h, compiled from /root/reference by build_ref.sh) as
 * plain functions so the tests can check the oracle against the reference's
 * own implementation.  TEST INFRASTRUCTURE ONLY; never linked by the product.
 */
#include <stdint.h>
#include <stdlib.h>

#include "moe_route.h"
#include "moe_exec.h"

float ref_sigmoid(float x) { return moe_sigmoid(x); }

int ref_route_select(const float *logits, const float *bias, int experts,
                     int top_k, int score_fn, int *indices, float *weights,
                     float *scores, float *selection_scores) {
    return moe_route_select(logits, bias, experts, top_k, (MoeScoreFn)score_fn,
                            indices, weights, scores, selection_scores);
}

int ref_route_fixed(const float *logits, int experts, const int *indices,
                    int count, int score_fn, float *weights, float *scores) {
    return moe_route_fixed(logits, experts, indices, count, (MoeScoreFn)score_fn,
                           weights, scores);
}

void ref_route_finalize(float *weights, int count, int normalize, float scale) {
    moe_route_finalize(weights, count, normalize, scale);
}

static int forward_flat(int hidden, int intermediate, int experts, int top_k,
                        int normalize, float route_scale, float swiglu_limit,
                        const float *router, const float *bias,
                        const float *gate, const float *up, const float *down,
                        int n_shared, const float *shared_gate,
                        const float *shared_up, const float *shared_down,
                        const float *input, int tokens, const int64_t *fixed,
                        float *output);

/* moe_f32_forward over flat arrays: gate/up [E][I][H], down [E][H][I];
 * shared experts likewise with n_shared entries of width I. */
int ref_moe_forward_flat(int hidden, int intermediate, int experts, int top_k,
                         int normalize, float route_scale, float swiglu_limit,
                         const float *router, const float *bias,
                         const float *gate, const float *up, const float *down,
                         int n_shared, const float *shared_gate,
                         const float *shared_up, const float *shared_down,
                         const float *input, int tokens, float *output) {
    return forward_flat(hidden, intermediate, experts, top_k, normalize, route_scale,
                        swiglu_limit, router, bias, gate, up, down, n_shared, shared_gate,
                        shared_up, shared_down, input, tokens, NULL, output);
}

/* The same with fixed experts per token row (moe_f32_forward's fixed_experts
 * path: token t uses fixed[t * top_k ...]). */
int ref_moe_forward_fixed_flat(int hidden, int intermediate, int experts, int top_k,
                               int normalize, float route_scale, const float *router,
                               const float *gate, const float *up, const float *down,
                               int n_shared, const float *shared_gate,
                               const float *shared_up, const float *shared_down,
                               const float *input, int tokens, const int64_t *fixed,
                               float *output) {
    return forward_flat(hidden, intermediate, experts, top_k, normalize, route_scale, 0.0f,
                        router, NULL, gate, up, down, n_shared, shared_gate, shared_up,
                        shared_down, input, tokens, fixed, output);
}

static int forward_flat(int hidden, int intermediate, int experts, int top_k,
                        int normalize, float route_scale, float swiglu_limit,
                        const float *router, const float *bias,
                        const float *gate, const float *up, const float *down,
                        int n_shared, const float *shared_gate,
                        const float *shared_up, const float *shared_down,
                        const float *input, int tokens, const int64_t *fixed,
                        float *output) {
    size_t mat = (size_t)intermediate * hidden;
    MoeExpertF32 *routed = calloc((size_t)experts, sizeof(*routed));
    MoeExpertF32 *shared = calloc((size_t)(n_shared > 0 ? n_shared : 1), sizeof(*shared));
    for (int e = 0; e < experts; ++e) {
        routed[e].w1 = gate + e * mat;
        routed[e].w3 = up + e * mat;
        routed[e].w2 = down + e * mat;
    }
    for (int e = 0; e < n_shared; ++e) {
        shared[e].w1 = shared_gate + e * mat;
        shared[e].w3 = shared_up + e * mat;
        shared[e].w2 = shared_down + e * mat;
    }
    MoeF32 model = {0};
    model.hidden = hidden;
    model.intermediate = intermediate;
    model.n_experts = experts;
    model.top_k = top_k;
    model.score_fn = MOE_SCORE_SIGMOID;
    model.normalize = normalize;
    model.route_scale = route_scale;
    model.swiglu_limit = swiglu_limit;
    model.router = router;
    model.selection_bias = bias;
    model.experts = routed;
    model.shared_experts = n_shared > 0 ? shared : NULL;
    model.n_shared_experts = n_shared;
    int *token_ids = NULL;
    if (fixed) {
        token_ids = malloc((size_t)tokens * sizeof(int));
        for (int t = 0; t < tokens; ++t) token_ids[t] = t;
        model.fixed_experts = fixed;
        model.vocab_size = tokens;
    }
    int ok = moe_f32_forward(&model, input, token_ids, tokens, output);
    free(token_ids);
    free(routed);
    free(shared);
    return ok;
}

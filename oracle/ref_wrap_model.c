/*
 * ref_wrap_model.c -- wraps the reference's container reader
 * (moonlight_model.c + st.h + json.h, compiled from /root/reference by
 * build_ref.sh) so tests can compare the product's config / tensor-table
 * parsing with it.  TEST INFRASTRUCTURE ONLY; never linked by the product.
 */
#include <string.h>

#include "moonlight_model.h"

/* Copies the parsed config (MoonlightConfig, moonlight_model.h:17-37) into
 * 19 ints/floats in declaration order; returns the tensor count or -1. */
int ref_model_probe(const char *path, int *ints16, float *floats3,
                    char *error, int error_size) {
    MoonlightModelData *data = NULL;
    if (!moonlight_model_data_open(&data, path, error, (size_t)error_size)) return -1;
    const MoonlightConfig *c = moonlight_model_data_config(data);
    int values[16] = {c->hidden_size, c->layer_count, c->head_count,
                      c->expert_count, c->experts_per_token,
                      c->dense_intermediate_size, c->moe_intermediate_size,
                      c->first_dense_layer_count, c->q_lora_rank,
                      c->kv_lora_rank, c->qk_nope_dim, c->qk_rope_dim,
                      c->value_dim, c->shared_expert_count, c->normalize_topk,
                      c->vocab_size};
    memcpy(ints16, values, sizeof(values));
    floats3[0] = c->rms_norm_epsilon;
    floats3[1] = c->rope_theta;
    floats3[2] = c->routed_scale;
    int count = moonlight_model_data_tensor_count(data);
    moonlight_model_data_close(data);
    return count;
}

/* Looks a tensor up by name: dtype, numel, nbytes; 0 when absent. */
int ref_model_tensor(const char *path, const char *name, int *dtype,
                     long long *numel, long long *nbytes) {
    MoonlightModelData *data = NULL;
    char error[256];
    if (!moonlight_model_data_open(&data, path, error, sizeof(error))) return 0;
    int index = moonlight_model_data_find(data, name);
    if (index >= 0) {
        MoonlightTensorInfo t = moonlight_model_data_tensor(data, index);
        *dtype = t.dtype;
        *numel = t.element_count;
        *nbytes = t.byte_count;
    }
    moonlight_model_data_close(data);
    return index >= 0;
}

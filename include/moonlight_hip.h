/*
 * moonlight_hip.h -- the Moonlight session C API on MI355X (HIP, gfx950).
 *
 * Drop-in for floyd's moonlight_metal.h:7-94: identical type layouts, function
 * names, argument meaning, return values (1 success / 0 failure, an English
 * message in `error` when it is non-NULL and non-empty) and preconditions, so
 * floyd.c, moonlight_chat.c and the reference's tests link against
 * libfloyd_amd.so in place of moonlight_metal.m.  Each declaration names the
 * reference definition it replaces (moonlight_metal.m line numbers).
 *
 * Differences a caller can observe:
 *   - moonlight_device_name reports the HIP device ("... [gfx950]"), not an
 *     Apple GPU name.
 *   - Kernel limits: head_count <= 16, kv_lora_rank a multiple of 64 and
 *     <= 512, qk_rope_dim even and <= 64, qk_nope_dim <= 256, expert_count
 *     <= 256, experts_per_token <= 16; session creation rejects other shapes
 *     with "unsupported Moonlight MLA dimensions" (the reference's own check,
 *     moonlight_metal.m:1041-1045, is a superset of these bounds).
 *   - MoonlightStats.command_buffers counts synchronising submissions to the
 *     device (one per forward, one per test primitive, two for
 *     moonlight_test_moe), keeping the reference tests' pins.
 */
#ifndef MOONLIGHT_HIP_H
#define MOONLIGHT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct MoonlightModel MoonlightModel;
typedef struct MoonlightSession MoonlightSession;

typedef struct {
    int context_size;
    int max_batch;
} MoonlightOptions;

typedef struct {
    int hidden_size;
    int layer_count;
    int vocab_size;
    int head_count;
    int kv_lora_rank;
    int qk_nope_dim;
    int qk_rope_dim;
    int value_dim;
    int expert_count;
    int experts_per_token;
    int moe_intermediate_size;
    int shared_expert_count;
    int first_dense_layer_count;
    float rms_norm_epsilon;
    float rope_theta;
    float routed_scale;
    uint64_t resident_bytes;
} MoonlightModelInfo;

typedef struct {
    uint64_t command_buffers;
    uint64_t prefill_tokens;
    uint64_t decode_tokens;
    uint64_t cpu_fallbacks;
    uint64_t buffer_allocations;
    uint64_t resident_bytes;
    double prefill_ms;
    double decode_ms;
} MoonlightStats;

/* moonlight_metal.m:757-874: reads config.json + every *.safetensors of the
 * container directory into HBM (one arena, double-buffered pinned staging). */
int moonlight_model_open(MoonlightModel **out, const char *path,
                         char *error, size_t error_size);
/* moonlight_metal.m:876-907 */
void moonlight_model_close(MoonlightModel *model);
/* moonlight_metal.m:909-911 */
const char *moonlight_device_name(const MoonlightModel *model);
/* moonlight_metal.m:913-936 */
MoonlightModelInfo moonlight_model_info(const MoonlightModel *model);

/* moonlight_metal.m:938-1125 */
int moonlight_session_create(MoonlightSession **out, MoonlightModel *model,
                             const MoonlightOptions *options,
                             char *error, size_t error_size);
/* moonlight_metal.m:1127-1161 */
void moonlight_session_destroy(MoonlightSession *session);
/* moonlight_metal.m:1163-1177: zeroes kv lengths, position and counters,
 * keeps allocations. */
void moonlight_session_reset(MoonlightSession *session);
/* moonlight_metal.m:1179-1181 */
int moonlight_session_position(const MoonlightSession *session);
/* moonlight_metal.m:1183-1186 */
MoonlightStats moonlight_session_stats(const MoonlightSession *session);
/* moonlight_metal.m:1988-2005: position must be 0, count <= max_batch. */
int moonlight_session_prefill(MoonlightSession *session, const int *ids,
                              int count, float *last_logits,
                              char *error, size_t error_size);
/* moonlight_metal.m:2007-2022: position > 0 and position + count <= context. */
int moonlight_session_append(MoonlightSession *session, const int *ids,
                             int count, float *last_logits,
                             char *error, size_t error_size);
/* moonlight_metal.m:2024-2037: position < context. */
int moonlight_session_decode(MoonlightSession *session, int token,
                             float *logits, char *error, size_t error_size);
/* moonlight_metal.m:2039-2053: full prefill that also returns every layer's
 * output [layers, count, hidden]. */
int moonlight_test_prefill_layers(MoonlightSession *session, const int *ids,
                                  int count, float *layer_outputs,
                                  float *last_logits,
                                  char *error, size_t error_size);

/* Test hooks, moonlight_metal.m:1188-1812 / 2055-2070 (0 on failure, no
 * message). */
int moonlight_test_embed(MoonlightSession *session, const int *ids,
                         int count, float *output);
int moonlight_test_rmsnorm(MoonlightSession *session, const float *input,
                           const char *weight_name, int rows, int width,
                           float *output);
int moonlight_test_matmul(MoonlightSession *session, const char *weight_name,
                          const float *input, int rows, int input_width,
                          int output_width, float *output);
int moonlight_test_attention(MoonlightSession *session, int layer,
                             const float *input, int rows, int position,
                             float *output);
int moonlight_test_kv_length(const MoonlightSession *session, int layer);
int moonlight_test_copy_kv(const MoonlightSession *session, int layer,
                           float *latent, float *rope, int capacity);
int moonlight_test_moe(MoonlightSession *session, int layer,
                       const float *input, int rows, int *route_ids,
                       float *route_weights, float *router_scores,
                       float *routed_output, float *shared_output,
                       float *output);
int moonlight_test_dense_mlp(MoonlightSession *session, int layer,
                             const float *input, int rows, float *output);
int moonlight_test_copy_routes(const MoonlightSession *session, int layer,
                               int *route_ids, int capacity);

#ifdef __cplusplus
}
#endif
#endif

/*
 * moonlight_hip_ext.h -- additions to the Moonlight session API that have no
 * counterpart in floyd's moonlight_metal.h.  They exist for callers that
 * build models in HBM without a container on disk (benchmarks, synthetic
 * parity runs) and for inspecting device state.
 */
#ifndef MOONLIGHT_HIP_EXT_H
#define MOONLIGHT_HIP_EXT_H

#include <stddef.h>
#include <stdint.h>

#include "moonlight_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Shape and packing of a synthetic Moonlight container generated directly in
 * HBM: every tensor a converted container holds (tools/convert_moonlight.py),
 * same names, dtypes and byte counts.  Matrices are drawn ~N(0, weight_std),
 * rounded to bf16 and packed per row at `expert_bits` (routed experts) or
 * `dense_bits` (attention, dense and shared FFNs), 8 or 4; embed, lm_head and
 * the router stay f32; norm weights are 1; e_score_correction_bias is
 * linspace(-0.1, 0.1, experts). */
typedef struct {
    int hidden_size, layer_count, head_count, expert_count, experts_per_token;
    int dense_intermediate_size, moe_intermediate_size, first_dense_layer_count;
    int kv_lora_rank, qk_nope_dim, qk_rope_dim, value_dim;
    int shared_expert_count, normalize_topk, vocab_size;
    float rms_norm_epsilon, rope_theta, routed_scale;
    int expert_bits, dense_bits;
    float weight_std;
    uint64_t seed;
} MoonlightSyntheticConfig;

/* Parses config.json and every safetensors header of a container directory
 * without touching the GPU (moonlight_model.c:41-190 semantics): fills
 * ints16 / floats3 in the field order of floyd's MoonlightConfig
 * (moonlight_model.h:17-37) and returns the tensor count, or -1 with a
 * message in `error`. */
int moonlight_container_probe(const char *path, int *ints16, float *floats3,
                              char *error, size_t error_size);
/* dtype code, element and byte count of one tensor of a container directory
 * (no GPU); 1 when found, 0 otherwise. */
int moonlight_container_tensor(const char *path, const char *name, int *dtype,
                               int64_t *numel, int64_t *nbytes);

/* Moonlight-16B-A3B dimensions (27 layers, hidden 2048, 16 heads, MLA 512+64,
 * 64 experts top-6 + 2 shared, vocab 163840), q8 packing, seed 1. */
MoonlightSyntheticConfig moonlight_synthetic_moonlight_config(void);

int moonlight_model_create_synthetic(MoonlightModel **out,
                                     const MoonlightSyntheticConfig *config,
                                     char *error, size_t error_size);

/* Copies tensor `name` of the model (its raw bytes as stored in HBM) into
 * host memory; returns the byte count, 0 if absent or capacity too small. */
size_t moonlight_model_read_tensor(const MoonlightModel *model,
                                   const char *name, void *dst,
                                   size_t capacity);
/* dtype code (0 bf16, 1 f16, 2 f32, 3 u8) and sizes of a tensor; 0 if absent. */
int moonlight_model_tensor_info(const MoonlightModel *model, const char *name,
                                int *dtype, int64_t *numel, int64_t *nbytes);

/* Overwrites the latent / rope cache of `layer` with `length` rows drawn
 * ~N(0, 1) from `seed` on the device, and sets that layer's kv length; when
 * `layer` < 0 every layer is filled (seed + layer) and the session position
 * becomes `length`.  Used to measure decode at a given context. */
int moonlight_session_fill_kv(MoonlightSession *session, int layer,
                              int length, uint64_t seed);

/* Times `iters` back-to-back device passes (after `warmup` untimed ones) of
 * one MoE layer exactly as a forward runs it (router GEMV with the fused
 * post-attention RMSNorm, top-k and route tables, grouped gate/up + down
 * expert launches, shared expert, combine into the residual) on `rows` token
 * rows drawn ~N(0, 1) and resident in HBM.  layer >= 0: that layer, one input
 * drawn from `seed`; layer < 0: the passes cycle through every MoE layer and
 * pass i reads its own input (seed + i), so the weights come from HBM rather
 * than the 256 MB last-level cache.  avg_us: HIP-event time per pass;
 * unique_experts: the distinct routed experts summed over the timed passes
 * (for the byte count).  rows is at most one routing call (16384 / top_k). */
int moonlight_session_time_moe(MoonlightSession *session, int layer, int rows,
                               uint64_t seed, int warmup, int iters,
                               double *avg_us, int *unique_experts);

/* Times `iters` back-to-back device passes (after `warmup` untimed ones) of
 * one attention block exactly as a decode runs it (the [q | kv_a] GEMV with
 * the input RMSNorm, cache append, query RoPE and absorb, split attention
 * over the `position` cached keys plus the new rows, merge, value and o_proj
 * with the residual) on `rows` token rows drawn ~N(0, 1), at cache position
 * `position` (0 <= position, position + rows <= context_size; the cache rows
 * at position .. position + rows - 1 are rewritten by every pass and the
 * session's cache lengths are left unchanged).  layer >= 0: that layer, one
 * input drawn from `seed`; layer < 0: the passes cycle through every layer
 * (fill every layer's cache first) and pass i reads its own input
 * (seed + i).  avg_us: HIP-event time per pass. */
int moonlight_session_time_attention(MoonlightSession *session, int layer, int rows,
                                     int position, uint64_t seed, int warmup, int iters,
                                     double *avg_us);

/* Fixes the routed experts of the next moonlight_test_moe /
 * moonlight_session_time_moe calls: token row r uses expert_ids[r * top_k ..]
 * (moe_route_fixed semantics, moe_route.h:76-87: weights are the router's
 * sigmoid scores of those ids, then finalised), for batches of at most `rows`
 * rows.  expert_ids == NULL restores top-k routing.  Forward passes always
 * route by top-k.  Returns 0 for ids out of range, an expert repeated within
 * a row, or rows > max_batch. */
int moonlight_session_fix_routes(MoonlightSession *session,
                                 const int *expert_ids, int rows);

/* Device time (milliseconds, HIP events around the launches) of the last
 * prefill / append / decode of the session. */
int moonlight_session_device_time(MoonlightSession *session, double *ms);

/* One-row decode steps run as one graph replay (captured on the session's
 * second decode; the attention kernels read the position from device memory
 * so the same launches serve every position).  enable = 0 turns this off for
 * the session (every decode launches its kernels in stream order, and a
 * captured graph is dropped), 1 turns it back on, < 0 only queries.  Returns
 * 1 when decode steps replay a captured graph, else 0.  No counterpart in
 * the reference (its decode encodes every layer each step). */
int moonlight_session_decode_graph(MoonlightSession *session, int enable);

/* Next token from the logits of the session's last prefill / append / decode,
 * chosen on the device as choose_token does on the host
 * (moonlight_chat.c:96-131, draw from random_unit at :89-94): temperature <= 0
 * takes the first index of the maximum; otherwise softmax at `temperature`,
 * candidates by descending probability (equal probabilities in token order),
 * the smallest prefix whose sum reaches top_p, one draw.  *rng_state is the
 * caller's xorshift64 state (the reference's chat->rng); it advances once when
 * temperature > 0 and a token is returned, and may be NULL otherwise.
 * Returns 1 and *token, or 0 with an error (no forward yet, non-finite
 * logits).  Replaces the host qsort of 163,840 candidates per token. */
int moonlight_session_sample(MoonlightSession *session, float temperature,
                             float top_p, uint64_t *rng_state, int *token,
                             char *error, size_t error_size);

/* moonlight_session_decode (moonlight_metal.h) followed by
 * moonlight_session_sample in the same device submission: the logits stay in
 * HBM and only the 4-byte token comes back.  Same preconditions and errors as
 * the two calls it combines. */
int moonlight_session_decode_sample(MoonlightSession *session, int token,
                                    float temperature, float top_p,
                                    uint64_t *rng_state, int *next_token,
                                    char *error, size_t error_size);

/* Device route tables of the session's last routing (moonlight_test_moe,
 * moonlight_session_time_moe or a forward's last MoE layer), for `rows`
 * token rows: the number of distinct experts, the experts in first-appearance
 * order over (row, slot) (unique, [expert_count], first *n_unique valid),
 * entries per expert (counts, [expert_count]), the start of each active
 * expert's compact list (offsets, [expert_count], valid where counts > 0),
 * and per list entry its token row and slot (list_rows / list_slots,
 * [rows * top_k]); list_pos[r * top_k + k] is the list entry of (r, k).
 * Expert e's j-th entry, list_rows[offsets[e] + j], is the reference's
 * rows[e * max_batch + j] of prepare_route_tables (moonlight_metal.m:525-559).
 * Any output may be NULL.  Returns 1, or 0 for rows outside [1, max_batch]. */
int moonlight_session_copy_route_tables(const MoonlightSession *session, int rows,
                                        int *n_unique, int *unique, int *counts,
                                        int *offsets, int *list_rows, int *list_slots,
                                        int *list_pos);

/* enable != 0: every later forward also keeps the router logits of each MoE
 * layer ([layer][row][expert_count], f32, before the sigmoid) in a session
 * buffer allocated here; 0 frees it.  A captured decode graph is dropped
 * either way (its launches differ).  Returns 1 on success. */
int moonlight_session_trace_router(MoonlightSession *session, int enable);

/* Copies the router logits of `layer` of the last forward ([rows]
 * [expert_count] floats; rows = that forward's row count) into `logits`.
 * Returns 1, or 0 without an enabled trace or for a dense layer. */
int moonlight_session_copy_router_trace(const MoonlightSession *session, int layer,
                                        float *logits, int capacity_rows);

#ifdef __cplusplus
}
#endif
#endif

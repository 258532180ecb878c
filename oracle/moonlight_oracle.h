/*
 * moonlight_oracle.h -- CPU restatement of floyd's quantized Moonlight arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP product
 * path is compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never links,
 * calls or falls back to it.
 *
 * Every function names the reference file:line whose semantics it restates
 * (paths relative to the c4pt0r/floyd tree).  Arithmetic is plain IEEE fp32,
 * compiled with -ffp-contract=off so each expression rounds exactly as written;
 * loops run in the reference's serial index order.
 *
 * Parity pinning (how each function is itself checked, see tests/):
 *   orc_quant_int8 / orc_quant_int4 : golden vectors written by importing
 *       tools/convert_moonlight.py:46-66 (tests/golden/make_golden.py) plus
 *       closed-form special cases (zero rows, amax element, odd width, ties).
 *   orc_matmul_*   : f64 brute force (tests/test_backend_metal.c:9-33 method),
 *                    closed forms (unit-vector input, constant input).
 *   orc_route_*    : moe_route.h compiled from the reference (oracle/_ref):
 *                    ids bit-exact, weights within 4 ulp (the reference twin's
 *                    glibc expf is not correctly rounded for ~0.06 % of inputs,
 *                    the oracle's score is); the closed-form cases of
 *                    tests/test_moe_route.c:16-112; the score itself against
 *                    numpy's f64 exp rounded to f32.
 *   orc_route_tables : brute force on tiny inputs (first-appearance order).
 *   orc_rmsnorm / orc_rope / orc_cache_append : closed forms (unit weight,
 *                    position 0 identity, rotation norm preservation).
 *   orc_mla_attention : explicit decompression K=W_UK lat, V=W_UV lat and
 *                    textbook softmax in f64 (algebraic identity), single-key
 *                    and shift-invariance cases.
 *   orc_route_fixed : moe_route_fixed + moe_route_finalize compiled from the
 *                    reference (oracle/_ref), weights within 4 ulp as above.
 *   orc_moe_layer / orc_dense_mlp : moe_exec.h compiled from the reference
 *                    (f32 SwiGLU MoE) on dequantised weights.
 *   orc_forward    : composition of the above; split prefill+append equals full
 *                    prefill; routing equals orc_route on the same logits.
 *   orc_random_unit / orc_choose_token : Marsaglia's xorshift64 (13, 7, 17)
 *                    restated independently in the test; greedy = numpy's
 *                    first-index argmax; sampling against closed forms
 *                    (top_p below the largest probability returns the argmax
 *                    for every draw, equal logits return floor(u * count) of
 *                    the nucleus in token order, draw 0 returns the argmax) and
 *                    against an independent numpy form (lexsort + cumsum).
 */
#ifndef MOONLIGHT_ORACLE_H
#define MOONLIGHT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- synthetic inputs -------------------------------------------------- */
/* Counter-based SplitMix64: value k of stream `seed` is mix(seed + (k+1)*G). */
uint64_t orc_splitmix64_at(uint64_t seed, uint64_t k);
/* out[i] = mean + std * N(0,1) from Box-Muller (cos branch) on the pair of
 * SplitMix64 draws (2i, 2i+1); rounded to bf16 (RNE) when bf16 != 0. */
void orc_fill_normal(float *out, int64_t n, uint64_t seed, double mean,
                     double std, int bf16);
float orc_bf16_round(float x);

/* ---- container packing (tools/convert_moonlight.py:46-66) -------------- */
void orc_quant_int8(const float *w, int rows, int cols, uint8_t *q, float *s);
void orc_quant_int4(const float *w, int rows, int cols, uint8_t *q, float *s);

/* ---- matmul (moonlight_kernels.metal:43-130) ---------------------------
 * y[r,o] = (sum_i x[r,i] * W[o,i]) (* s[o] for q8/q4).  fmt: 0 f32, 1 q8, 2 q4.
 * threads > 1 splits output rows over OpenMP threads (same per-row math). */
void orc_matmul(int fmt, const void *w, const float *s, const float *x,
                float *y, int out_width, int in_width, int rows, int threads);
/* Thread count used by the model-level functions below (default 1). */
void orc_set_threads(int threads);
/* Format detection of resolve_matrix (moonlight_metal.m:129-162): returns
 * 1 (q8) / 2 (q4) from the U8 byte count, -1 when neither matches. */
int orc_detect_format(int64_t byte_count, int out_width, int in_width);

/* ---- elementwise pieces ------------------------------------------------ */
void orc_rmsnorm(const float *x, const float *w, float *y, int rows, int width,
                 float eps);
/* RoPE of moonlight_kernels.metal:172-200 on one vector: reads pairs
 * (2p, 2p+1), writes half layout [p] and [half+p]. */
void orc_rope(const float *in, float *out, int width, int position,
              float theta);
float orc_rope_inv_freq(float theta, int pair, int width);
float orc_silu_mul(float gate, float up);

/* ---- routing (moonlight_kernels.metal:469-512, moe_route.h:47-99) ------ */
void orc_route_sigmoid_topk(const float *logits, const float *bias, int rows,
                            int experts, int top_k, int normalize,
                            float routed_scale, int *ids, float *weights);
/* prepare_route_tables (moonlight_metal.m:525-559).  Writes unique experts in
 * first-appearance order, per-expert counts, and rows/slots at
 * expert*max_batch + j.  Returns the unique count, -1 on a bad id. */
int orc_route_tables(const int *ids, int rows, int top_k, int experts,
                     int max_batch, int *unique, int *counts, int *expert_rows,
                     int *expert_slots);

/* ---- model-level pieces over a named-tensor table ---------------------- */
typedef struct OrcModel OrcModel;

typedef struct {
    int hidden_size, layer_count, head_count, expert_count, experts_per_token;
    int dense_intermediate_size, moe_intermediate_size, first_dense_layer_count;
    int q_lora_rank, kv_lora_rank, qk_nope_dim, qk_rope_dim, value_dim;
    int shared_expert_count, normalize_topk, vocab_size;
    float rms_norm_epsilon, rope_theta, routed_scale;
} OrcConfig;

/* dtype codes follow moonlight_model.h:10-15: 0 bf16, 1 f16, 2 f32, 3 u8. */
OrcModel *orc_model_create(const OrcConfig *config, int context_size);
void orc_model_destroy(OrcModel *model);
/* Registers a caller-owned tensor (pointer must outlive the model). */
int orc_model_add_tensor(OrcModel *model, const char *name, int dtype,
                         const void *data, int64_t numel, int64_t nbytes);
void orc_model_reset(OrcModel *model);
int orc_model_kv_length(const OrcModel *model, int layer);
/* Overwrites the KV cache of every layer with caller data and sets the
 * per-layer length and position (bench-only prefill of the latent cache). */
int orc_model_set_kv(OrcModel *model, int layer, const float *latent,
                     const float *rope, int length);
int orc_model_copy_kv(const OrcModel *model, int layer, float *latent,
                      float *rope, int capacity);

/* Quantized matmul by tensor name, format detected like resolve_matrix. */
int orc_named_matmul(const OrcModel *model, const char *name, const float *x,
                     int rows, int in_width, int out_width, float *y);
/* encode_attention_buffer (moonlight_metal.m:287-440): q/kv_a projections,
 * cache append at `position`, absorbed attention, o_proj.  Updates the KV
 * cache and kv length of `layer`. */
int orc_attention(OrcModel *model, int layer, const float *x, int rows,
                  int position, float *out);
/* moonlight_test_moe (moonlight_metal.m:1520-1733) semantics. */
int orc_route_fixed(const float *logits, int rows, int experts, int top_k,
                    int normalize, float routed_scale, const int *ids,
                    float *weights);
int orc_moe_layer_fixed(OrcModel *model, int layer, const float *x, int rows,
                        const int *fixed_ids, float *route_weights, float *out);
int orc_moe_layer(OrcModel *model, int layer, const float *x, int rows,
                  int *route_ids, float *route_weights, float *router_logits,
                  float *routed, float *shared, float *out);
int orc_dense_mlp(OrcModel *model, int layer, const float *x, int rows,
                  float *out);
/* run_tokens_fast (moonlight_metal.m:1892-1986).  layer_outputs optional
 * [layers, rows, hidden]; route_trace optional [layers, rows, top_k]. */
int orc_forward_routes(OrcModel *model, const int *ids, int rows,
                       int start_position, const int *fixed_trace,
                       float *layer_outputs, float *last_logits);
int orc_forward(OrcModel *model, const int *ids, int rows, int start_position,
                float *layer_outputs, int *route_trace, float *last_logits);

/* ---- next-token choice (caller-side sampler) ------------------------- */
/* random_unit (moonlight_chat.c:89-94): one xorshift64 step of *state, then
 * the top 53 bits as a double in [0, 1). */
double orc_random_unit(uint64_t *state);
/* choose_token (moonlight_chat.c:96-131).  temperature <= 0: the first index
 * of the maximum (strict > scan).  Otherwise p = expf((logit - max) / T),
 * normalised by their double sum, sorted by descending p with equal p in
 * ascending token order (what glibc 2.35's qsort, a stable merge sort at this
 * size, gives the reference), the smallest prefix whose double sum reaches
 * top_p kept, and one draw random_unit * kept located in the prefix sums.
 * *rng advances once when temperature > 0. */
int orc_choose_token(const float *logits, int vocab, float temperature, float top_p,
                     uint64_t *rng);

#ifdef __cplusplus
}
#endif
#endif

// mla.h -- compressed-MLA attention launches (internal; see mla.hip).
#pragma once

#include "mlh_host.h"

namespace mlh {

constexpr int kMlaMaxHeads = 16;        // Moonlight: 16 heads
constexpr int kMlaTileKeys = 16;        // keys per mla_attend tile
constexpr int kMlaAttendGroups = 256;   // mla_attend workgroups per launch group (all rows)
constexpr int kMlaMaxLatent = 512;      // kv_lora_rank limit (moonlight_metal.m:1041)
constexpr int kMlaDecodeRows = 16;      // token rows per decode-path launch group
constexpr int kMlaValueDims = 32;       // latent dims per merge + value workgroup
constexpr int kMlaCountStride = 32;     // ints between arrival counters (one per 128 bytes)

// A weight matrix in one of the container formats (f32 / int8 / packed int4)
// with its per-row scales.
struct MatrixRef {
    int fmt = kQ8;
    const uint8_t *w = nullptr;
    const float *s = nullptr;
};

// One attention call for `rows` token rows starting at `position`, for one
// layer: caches point at that layer's [context][latent] / [context][rope].
struct MlaParams {
    int rows = 0, position = 0, heads = 0;
    // When set, the kernels read the position from this device int instead
    // of `position` (a captured decode graph replays at every position), and
    // the attend grid is grid_splits workgroups per row whatever the position.
    const int *position_dev = nullptr;
    int grid_splits = 0;
    int splits = 0;  // attend workgroups per row of a launch group (set by mla_attention_core)
    int nope = 0, rope = 0, vdim = 0, latent = 0;
    float eps = 1e-5f, scale = 1.0f;
    const float *query = nullptr;       // [rows][heads * (nope + rope)] (q_proj output)
    long query_stride = 0;              // floats between token rows of query
    const float *compressed = nullptr;  // [rows][latent + rope] (kv_a output)
    long compressed_stride = 0;         // floats between token rows of compressed
    const float *kv_norm = nullptr;     // [latent] kv_a_layernorm weight
    const float *inv_freq = nullptr;    // [rope / 2] theta^(-2p/rope), host-computed
    MatrixRef kv_b;                     // [heads * (nope + vdim), latent]
    float *latent_cache = nullptr;      // this layer: [context, latent]
    // this layer: [context][2][latent] f16 bit patterns, the halves hi, lo of
    // every latent_cache value as the attention products split them
    // (split_f16), written with the cache; the prefill attention reads them
    uint16_t *latent_split = nullptr;
    float *rope_cache = nullptr;        // this layer: [context, rope]
    float *query_rope = nullptr;        // scratch [rows, heads, rope]
    float *query_absorbed = nullptr;    // scratch [rows, heads, latent]
    int max_splits = 0;                 // split capacity of the partial buffers
    float *part_max = nullptr;          // [rows, kMlaMaxHeads, max_splits]
    float *part_sum = nullptr;          // [rows, kMlaMaxHeads, max_splits]
    float *part_lc = nullptr;           // [rows, kMlaMaxHeads, latent / kMlaValueDims, max_splits, kMlaValueDims]
    float *latent_context = nullptr;    // scratch [rows, heads, latent] merged lc
    // prefill of at least kMlaExpandMinRows rows with position + rows <=
    // expand_keys: every key's per-head k_nope and value (kv_b . latent) as
    // f16 halves, laid out for mla_flash_kernel (mla_expand_kv_bytes per key)
    uint16_t *kv_expanded = nullptr;
    long expand_keys = 0;               // key capacity of kv_expanded (a multiple of 64)
    float *context = nullptr;           // out [rows, heads, vdim]
    // decode path (at most kMlaDecodeRows rows per launch group):
    float *value_part = nullptr;   // [rows][heads][latent / kMlaValueDims][vdim] value partials
    int *merge_count = nullptr;    // [rows][heads] x kMlaCountStride arrival counters, zero between launches
    // optional: set to range_code (if still 0) when a query or key value
    // written for the attention products is finite but outside the f16
    // range of their split-f16 operands (|v| >= 65504)
    int *range_error = nullptr;
    int range_code = 0;
};

// Prefill rows from which the attention runs on per-head keys and values
// (kv_b applied to every cached latent row once) instead of in the absorbed
// form, and the bytes of their expanded copy per key (0: the shape or the
// kv_b format (q8 / q4 only) has no expanded form).
constexpr int kMlaExpandMinRows = 64;
// Keys an expanded copy holds at most (a session's allocation: at Moonlight's
// shape 21,760 bytes a key, 713 MB at this limit).
constexpr long kMlaExpandMaxKeys = 32768;
size_t mla_expand_kv_bytes(int heads, int nope, int rope, int vdim, int latent, int kv_b_fmt);

// Prefill: cache append + query RoPE, then either the per-head expansion
// and a flash attention over it (kMlaExpandMinRows rows or more, keys
// within expand_keys), or the absorb GEMM, flash attention on the latent
// rows and the value GEMM.  Decode: cache append + query RoPE + absorb, split-K
// attention, merge + value projection (three launches per group of
// kMlaDecodeRows rows).  o_proj is a plain GEMV on `context`.
int mla_attention_core(const MlaParams &p, hipStream_t stream);

// The f16 halves of `rows` rows of a latent cache (latent values each) into
// its split copy, for caches filled by other means than the attention's own
// cache append.
int mla_split_cache(const float *latent, uint16_t *split, long rows, int width,
                    hipStream_t stream);

}  // namespace mlh

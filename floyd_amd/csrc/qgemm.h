// qgemm.h -- grouped int8-MFMA GEMM for prefill (many token rows per matrix).
//
// Y[m][n] = s_w[n] * sum_k W[n][k] * x[m][k] for the token rows m of a task,
// with W in the container's q8 (int8) or q4 (nibble) packing, used as exact
// int8 operands of v_mfma_i32_32x32x32_i8.  Activations are quantised per
// token row into three int8 limbs, x ~= s_x * (65536 * hi + 256 * mid + lo)
// with |65536 * hi + 256 * mid + lo| <= 2^22 (23 significant bits against the
// row's max, the precision of an fp32 operand), and every limb is multiplied
// by the same weight fragment; the int32 sums are combined in fp32 in the
// epilogue.  The per-element rounding of x is at most amax / 2^23, so a row
// whose max is 100x its rms still sees ~4e-6 relative error: outputs match the
// fp32 matmul of moonlight_kernels.metal:62-130 to fp32 rounding while every
// product and sum is exact.
//
// A launch covers a table of independent tasks (one per active routed expert
// plus the shared expert, or one dense matrix).  Tiles are 128 token rows x
// 256 weight rows (SwiGLU pairs: 128 gate + 128 matching up rows, 128
// outputs), or 32 token rows x 256 weight rows where a launch's tasks hold
// few rows each; the tile order groups 4 row tiles of a task so that consecutive
// workgroups on one XCD share weight tiles in that XCD's L2.
#pragma once

#include "gemv_impl.h"

namespace mlh {

constexpr int kQgBM = 128;  // token rows per tile
constexpr int kQgBMSmall = 32;  // token rows per tile of few-row launches
constexpr int kQgBW = 256;  // weight rows per tile
constexpr int kQgBK = 64;   // k per pipeline stage
constexpr int kQgGroup = 4; // row tiles per locality group
constexpr int kQgMaxTasks = 272;

// One independent product: rows x n_out outputs, reduction length k.
struct GemmTask {
    const uint8_t *w = nullptr, *w2 = nullptr;  // [n_out][k] packed (w2: up rows, SwiGLU)
    const float *s = nullptr, *s2 = nullptr;    // per weight row scales
    int rows = 0, n_out = 0, k = 0;
    int w_ld = 0;  // weight row length in elements (0: k); a k slice of longer rows
    // quantised activations: limb l (0 hi, 1 mid, 2 lo) of row r at
    // a + l * a_plane + r * a_stride
    const int8_t *a = nullptr;
    long a_plane = 0;
    const float *a_scale = nullptr;
    long a_stride = 0;
    const int *a_rows = nullptr;  // optional: activation row of token row m
    float *y = nullptr;           // output row m at y + m * y_stride
    long y_stride = 0;
    const float *resid = nullptr;  // optional residual (y = resid + product)
    long resid_stride = 0;
};

struct QGemmLaunch {
    const GemmTask *tasks = nullptr;  // device table (MoE); nullptr: `single`
    const int *tile_start = nullptr;  // device [tasks + 1] tile prefix sums
    const int *n_routed = nullptr;    // device: routed task count (shared tasks follow)
    int n_shared = 1;                 // shared-expert tasks after the routed ones
    int range = 0;                    // 0 all tasks, 1 routed only, 2 shared only
    GemmTask single;
};

// Per-row activation quantisation (optionally RMSNorm'ed first,
// moonlight_kernels.metal:23-41): rows of `x` (stride x_stride floats) ->
// limbs hi, mid, lo at q, q + plane, q + 2 plane (row stride `width` bytes)
// and scales.
int quantize_activations(const float *x, long x_stride, int rows, int width, const float *norm_w,
                         float eps, int8_t *q, long plane, float *scale, hipStream_t stream);

// One dense task, e.g. a prefill projection.  Epilogue: plain or residual
// (task.resid) or SwiGLU pair (dual, task.w2 = up).
int qgemm_single(int fmt, bool dual, const GemmTask &task, hipStream_t stream);

// MoE prefill: builds the per-expert task tables from the device route tables
// and runs both expert stages for all active experts plus the shared expert.
struct MoeGemmParams {
    int rows = 0, experts = 0, top_k = 0, hidden = 0, inter = 0, shared_width = 0;
    // with route_in_prep (rows <= kRouteOneGroupRows, experts <= 64 not
    // required): the routing of the batch from route.logits and its tables
    // run in the first launch (no routing launch before moe_gemm)
    int route_in_prep = 0;
    RouteParams route;
    int expert_fmt = kQ8, shared_fmt = kQ8, has_shared = 1;
    const ExpertWeights *expert_table = nullptr;
    const uint8_t *shared_gate = nullptr, *shared_up = nullptr, *shared_down = nullptr;
    const float *shared_gate_s = nullptr, *shared_up_s = nullptr, *shared_down_s = nullptr;
    const int *n_unique = nullptr, *unique = nullptr, *counts = nullptr, *offsets = nullptr;
    const int *list_rows = nullptr;
    const float *x = nullptr;  // residual stream [rows, hidden]
    const float *norm_w = nullptr;
    float eps = 1e-5f;
    // scratch
    // three limb planes each (limb l at base + l * plane)
    int8_t *xq = nullptr;  // [3][rows, hidden]
    long xq_plane = 0;
    float *xq_scale = nullptr;  // [rows]
    int8_t *hq = nullptr;  // [3][rows*top_k, inter]
    long hq_plane = 0;
    float *hq_scale = nullptr;  // [rows*top_k]
    int8_t *sq = nullptr;  // [3][rows, shared_width]
    long sq_plane = 0;
    float *sq_scale = nullptr;  // [rows]
    GemmTask *tasks = nullptr;                   // [2][kQgMaxTasks]
    int *tile_start = nullptr;                   // [2][kQgMaxTasks + 1]
    // outputs (same layouts as the GEMV expert path)
    float *expert_hidden = nullptr;  // [rows*top_k, inter]
    float *expert_out = nullptr;     // [rows*top_k, hidden]
    float *shared_hidden = nullptr;  // [rows, shared_width]
    float *shared_out = nullptr;     // [rows, hidden]
    // optional [rows, hidden]: the shared down projection runs as two k
    // halves (shared_out + shared_out2) when its width is twice inter
    float *shared_out2 = nullptr;
};
int moe_gemm(const MoeGemmParams &p, hipStream_t stream);

// Shapes the MFMA path takes (k a multiple of kQgBK, 16-byte aligned rows).
bool qgemm_shape_ok(int fmt, int k);

}  // namespace mlh

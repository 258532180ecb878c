// moe.h -- MoE routing / expert launches (internal; see moe.hip).
#pragma once

#include "gemv_impl.h"

namespace mlh {

// Sigmoid top-k + route tables for `rows` token rows (one workgroup); the
// RouteParams type is shared with the grouped expert launches (gemv_impl.h).
// A call routes at most kRouteMaxPositions (row, slot) positions.
constexpr int kRouteMaxPositions = 16384;
int route_topk(const RouteParams &p, hipStream_t stream);

// f32 router logits of many token rows, x RMSNorm'ed with norm_w when it is
// non-null: logits [rows, experts].
int router_logits(const float *x, const float *norm_w, float eps, const float *w, int rows,
                  int experts, int width, float *logits, hipStream_t stream);
// The same for fewer rows (one workgroup per expert and 16 rows; width a
// multiple of 8).
int router_logits_small(const float *x, const float *norm_w, float eps, const float *w, int rows,
                        int experts, int width, float *logits, hipStream_t stream);

struct CombineParams {
    int rows = 0, hidden = 0, top_k = 0;
    const float *weights = nullptr;     // [rows, top_k]
    const int *list_pos = nullptr;      // [rows, top_k]
    const float *expert_out = nullptr;  // [list, hidden]
    float *shared_out = nullptr;        // [rows, hidden]
    const float *shared_out2 = nullptr; // optional second part of the shared output
    const float *resid = nullptr;       // optional [rows, hidden]
    float *routed_copy = nullptr;       // optional [rows, hidden] (test hook: shared_out
                                        // then holds the summed shared output)
    float *out = nullptr;               // [rows, hidden]
};
int moe_combine(const CombineParams &p, hipStream_t stream);

struct ExpertFfnParams {
    int rows = 0, experts = 0, top_k = 0, hidden = 0, inter = 0, shared_width = 0;
    int expert_fmt = kQ8, shared_fmt = kQ8, has_shared = 1;
    // one token row, at most 64 experts: with route.logits set, stage 0
    // routes inline (see ExpertGemvParams::route) and no routing launch is
    // needed before expert_ffn
    RouteParams route;
    const ExpertWeights *expert_table = nullptr;  // device [experts]
    const uint8_t *shared_gate = nullptr, *shared_up = nullptr, *shared_down = nullptr;
    const float *shared_gate_s = nullptr, *shared_up_s = nullptr, *shared_down_s = nullptr;
    const int *n_unique = nullptr, *unique = nullptr, *counts = nullptr, *offsets = nullptr;
    const int *list_rows = nullptr;
    const ExpertTask *tasks = nullptr;  // optional per-task table from the routing
    const float *x = nullptr;       // residual stream [rows, hidden] (normalised on the fly)
    const float *norm_w = nullptr;  // post-attention RMSNorm weight
    float eps = 1e-5f;
    float *expert_hidden = nullptr;  // [rows*top_k, inter]
    float *expert_out = nullptr;     // [rows*top_k, hidden]
    float *shared_hidden = nullptr;  // [rows, shared_width]
    float *shared_out = nullptr;     // [rows, hidden]
    // optional pre-split inputs (limb_quantise_rows): when limb_x is set the
    // token rows are split once per stage instead of in every workgroup.
    // Row strides of all four are limb_stride_x / limb_stride_h / ...
    unsigned char *limb_x = nullptr, *limb_xs = nullptr;  // token rows (expert / shared fmt)
    unsigned char *limb_h = nullptr, *limb_sh = nullptr;  // list rows / shared rows
    long limb_x_stride = 0, limb_h_stride = 0, limb_sh_stride = 0;
    // one token row (down_combine_ok): with `combine_out` set, the down
    // projections and the combine run as one launch (moe_down_combine_kernel)
    // and write combine_out = combine_resid + (routed + shared); moe_combine
    // is then not needed.  route_weights / list_pos are the route tables.
    float *combine_out = nullptr;
    const float *combine_resid = nullptr;  // optional
    float *combine_routed = nullptr;       // optional copy of the routed sum
    float *combine_shared = nullptr;       // optional copy of the shared expert output
    const float *route_weights = nullptr;
    const int *list_pos = nullptr;
};

// Whether a one-row layer of this shape can take the fused down + combine
// launch: one format for routed and shared experts, shared width a multiple
// of the expert width, at most 16 units (top_k + shared_width / inter), an
// expert row of at most kDownCombineChunks 16-byte chunks per lane group.
bool down_combine_ok(const ExpertFfnParams &f);
int expert_ffn(const ExpertFfnParams &f, hipStream_t stream);

int rmsnorm_rows(const float *x, const float *w, float *y, int rows, int width, float eps,
                 long in_stride, long out_stride, hipStream_t stream);
// Embedding gather; also zeroes *clear_flag (the route error flag of the
// forward) when it is non-null.
int embed_rows(const float *table, const int *ids, float *out, int rows, int width, int vocab,
               int *clear_flag, hipStream_t stream);
int add_vectors(const float *a, const float *b, float *out, long n, hipStream_t stream);

// Planning helpers shared with gemv.hip.
GemvPlan plan_expert_gemv(int fmt, int O, int I, int rows, bool dual, int tasks, int max_I);
int gemv_rows_per_block(const GemvPlan &plan, bool dual);

}  // namespace mlh

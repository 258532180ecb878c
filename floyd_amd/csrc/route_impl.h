// route_impl.h -- device routing of one token row with at most 64 experts
// (internal), shared by the routing kernels and the grouped expert launches.
//
// References (c4pt0r/floyd): moe_route_select + moe_route_finalize
// (moe_route.h:47-99), moonlight_route_sigmoid_topk
// (moonlight_kernels.metal:469-512), prepare_route_tables
// (moonlight_metal.m:525-559).
//
// Included by gemv_impl.h after the expert types (ExpertWeights, ExpertTask,
// RouteParams) it uses.
#pragma once

namespace mlh {

// Router score 1 / (1 + e^-x) (moe_route.h:12-14) with e^-x correctly
// rounded to f32: exp is evaluated in double and rounded once.  Host glibc
// expf, which the reference's CPU twin calls, misrounds ~0.06 % of inputs by
// one ulp; a selection can only change where two selection scores tie within
// that ulp.
__device__ __forceinline__ float sigmoid_exact(float logit) {
    const float e = (float)exp(-(double)logit);
    return 1.0f / (1.0f + e);
}

// Field-wise store of a task entry (a struct copy would go through scratch).
__device__ __forceinline__ void store_task(ExpertTask *t, const ExpertWeights &w, int count,
                                           int offset) {
    t->w.gate = w.gate;
    t->w.up = w.up;
    t->w.down = w.down;
    t->w.gate_s = w.gate_s;
    t->w.up_s = w.up_s;
    t->w.down_s = w.down_s;
    t->count = count;
    t->offset = offset;
}

// Routing of token row r with at most 64 experts (one per lane) by one wave,
// with no serial arg-max chain.  The top-k selection is a rank: expert e is
// taken in slot rank(e) = #{o : sel_o > sel_e or (sel_o == sel_e and o < e)}
// when rank(e) < top_k, which is the order the repeated arg-max of
// moe_route.h:59-71 produces (larger first, lower index on ties).  Only
// experts with sel > -inf can be taken (NaN never compares greater), as in
// the arg-max.  With WRITE, writes ids / weights / trace (and lds_ids);
// returns the slot of this lane's expert (-1: not taken) and the mask of
// filled slots.
struct RowSelection {
    int slot;
    unsigned long long filled;  // bit k: slot k holds a valid expert
};

template <bool WRITE = true>
__device__ __forceinline__ RowSelection select_row_64(const RouteParams &p, int r, int lane,
                                                     int *lds_ids) {
    const int E = p.experts, K = p.top_k;
    const bool have = lane < E;
    const float logit = have ? p.logits[(long)r * E + lane] : 0.0f;
    const float bias = have ? p.bias[lane] : 0.0f;
    const float score = have ? sigmoid_exact(logit) : 0.0f;
    const float sel = have ? score + bias : -INFINITY;
    RowSelection rs{-1, 0ull};
    if (p.fixed_ids) {
        for (int k = 0; k < K; ++k)
            if (p.fixed_ids[(long)r * K + k] == lane) rs.slot = k;
    } else if (sel > -INFINITY) {
        const int sel_bits = __float_as_int(sel);
        int rank = 0;
#pragma unroll 8
        for (int o = 0; o < 64; ++o) {
            const float so = __int_as_float(__builtin_amdgcn_readlane(sel_bits, o));
            rank += (so > sel) || (so == sel && o < lane);
        }
        if (rank < K) rs.slot = rank;
    }
    // slot k -> expert; weights summed in slot order (moe_route_finalize)
    int my_id = -1;
    float my_w = 0.0f, wsum = 0.0f;
    for (int k = 0; k < K; ++k) {
        const unsigned long long m = __ballot(rs.slot == k);
        const int src = m ? __ffsll((long long)m) - 1 : -1;
        if (src >= 0) rs.filled |= 1ull << k;
        if constexpr (WRITE) {
            const float w =
                src >= 0 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(score), src))
                         : 0.0f;
            if (lane == k) {
                my_id = src;
                my_w = w;
            }
            wsum += w;
        }
    }
    if (!WRITE) return rs;
    if (p.normalize)
        wsum += 1e-20f;
    else
        wsum = 1.0f;
    if (lane < K) {
        p.ids[(long)r * K + lane] = my_id;
        if (lds_ids) lds_ids[r * K + lane] = my_id;
        p.weights[(long)r * K + lane] = my_w / wsum * p.routed_scale;
        if (p.trace) p.trace[(long)r * K + lane] = my_id;
    }
    return rs;
}

// One token row: routing and route tables by a single wave with no barrier.
// With one row and distinct experts the tables are direct: expert e in slot k
// is the u-th taken expert (u = k unless a fixed id was invalid), with one
// list entry at offset u.
__device__ __forceinline__ void route_single_64(const RouteParams &p, int lane) {
    const int E = p.experts, K = p.top_k;
    const bool have = lane < E;
    ExpertWeights ew{};
    if (p.tasks && have) ew = p.expert_table[lane];  // in flight with the logits
    const RowSelection rs = select_row_64(p, 0, lane, nullptr);
    const int slot = rs.slot;
    if (lane < K && !((rs.filled >> lane) & 1ull)) {
        p.list_pos[lane] = -1;
        *p.error = 1;  // prepare_route_tables rejects such ids (moonlight_metal.m:545)
    }
    const int n_unique = __popcll(rs.filled);
    if (lane == 0) *p.n_unique = n_unique;
    if (have) p.counts[lane] = slot >= 0 ? 1 : 0;
    if (slot >= 0) {
        const int u = __popcll(rs.filled & ((1ull << slot) - 1ull));
        p.offsets[lane] = u;
        p.unique[u] = lane;
        p.list_rows[u] = 0;
        p.list_slots[u] = slot;
        p.list_pos[slot] = u;
        if (p.tasks) store_task(p.tasks + u, ew, 1, u);
    }
    if (p.tasks && lane >= n_unique && lane < p.task_slots)
        store_task(p.tasks + lane, ExpertWeights{}, 0, 0);
}


// The expert of routed task `task` (the task-th taken expert in slot order)
// of a one-row batch, selected from the router logits exactly as
// route_single_64 selects it, and its weights; -1 when the task is empty.
// Every lane loads its expert's table entry alongside the logits, so the
// weights need no dependent load.  Called by whole waves.
__device__ __forceinline__ int inline_task_expert(const RouteParams &p, int task,
                                                  ExpertWeights *ew) {
    const int lane = threadIdx.x & 63;
    ExpertWeights mine{};
    if (lane < p.experts) mine = p.expert_table[lane];
    const RowSelection rs = select_row_64<false>(p, 0, lane, nullptr);
    const int u = rs.slot >= 0 ? __popcll(rs.filled & ((1ull << rs.slot) - 1ull)) : -1;
    const unsigned long long m = __ballot(u == task);
    if (!m) return -1;
    const int src = __ffsll((long long)m) - 1;
    auto pick = [src](const void *ptr) -> const void * {
        const unsigned long long v = reinterpret_cast<unsigned long long>(ptr);
        const unsigned lo = __builtin_amdgcn_readlane((unsigned)v, src);
        const unsigned hi = __builtin_amdgcn_readlane((unsigned)(v >> 32), src);
        return reinterpret_cast<const void *>(((unsigned long long)hi << 32) | lo);
    };
    ew->gate = static_cast<const uint8_t *>(pick(mine.gate));
    ew->up = static_cast<const uint8_t *>(pick(mine.up));
    ew->down = static_cast<const uint8_t *>(pick(mine.down));
    ew->gate_s = static_cast<const float *>(pick(mine.gate_s));
    ew->up_s = static_cast<const float *>(pick(mine.up_s));
    ew->down_s = static_cast<const float *>(pick(mine.down_s));
    return src;
}

}  // namespace mlh

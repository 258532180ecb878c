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

#include <climits>

namespace mlh {

// experts of a one-row batch whose logits come as GEMV partials
constexpr int kMaxRouteFused = 64;

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
// filled slots.  `keys` is the calling wave's own 64-entry LDS scratch
// (16-byte aligned).
struct RowSelection {
    int slot;
    unsigned long long filled;  // bit k: slot k holds a valid expert
};

// The rank above for every lane of a wave at once.  Each lane publishes a
// 64-bit key that is unique in the wave: the order-preserving bit pattern of
// its selection score (sign flipped for positive scores, all bits inverted
// for negative ones, so unsigned order is float order) above 63 - lane, so
// that of two equal scores the lower lane has the larger key.  rank(e) is
// then the number of keys above e's: 64 compares against keys read back as
// LDS broadcasts.  A lane that cannot be taken (score -inf or NaN) publishes
// 0, below every live key, so it outranks no lane.
__device__ __forceinline__ int wave_rank_desc(float sel, bool live, int lane,
                                              unsigned long long *keys) {
    const unsigned u = __float_as_uint(sel);
    const unsigned ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    const unsigned long long key =
        live ? ((unsigned long long)ord << 32) | (unsigned)(63 - lane) : 0ull;
    keys[lane] = key;
    // the wave's own LDS accesses complete in issue order: the loads below
    // see every lane's store
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    int ra = 0, rb = 0;
#pragma unroll
    for (int o = 0; o < 64; o += 4) {
        const ulonglong2 k0 = *reinterpret_cast<const ulonglong2 *>(keys + o);
        const ulonglong2 k1 = *reinterpret_cast<const ulonglong2 *>(keys + o + 2);
        ra += (k0.x > key) + (k0.y > key);
        rb += (k1.x > key) + (k1.y > key);
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    return ra + rb;
}

template <bool WRITE = true>
__device__ __forceinline__ RowSelection select_row_64_v(const RouteParams &p, int r, int lane,
                                                       int *lds_ids, float logit, float bias,
                                                       unsigned long long *keys);
template <bool WRITE = true>
__device__ __forceinline__ RowSelection select_row_64(const RouteParams &p, int r, int lane,
                                                     int *lds_ids, unsigned long long *keys) {
    const bool have = lane < p.experts;
    return select_row_64_v<WRITE>(p, r, lane, lds_ids, have ? p.logits[(long)r * p.experts + lane] : 0.0f,
                                  have ? p.bias[lane] : 0.0f, keys);
}
// The same with this lane's logit and bias already loaded.
template <bool WRITE>
__device__ __forceinline__ RowSelection select_row_64_v(const RouteParams &p, int r, int lane,
                                                       int *lds_ids, float logit, float bias,
                                                       unsigned long long *keys) {
    const int E = p.experts, K = p.top_k;
    const bool have = lane < E;
    const float score = have ? sigmoid_exact(logit) : 0.0f;
    const float sel = have ? score + bias : -INFINITY;
    RowSelection rs{-1, 0ull};
    if (p.fixed_ids) {
        for (int k = 0; k < K; ++k)
            if (p.fixed_ids[(long)r * K + k] == lane) rs.slot = k;
    } else {
        const bool live = sel > -INFINITY;
        const int rank = wave_rank_desc(sel, live, lane, keys);
        if (live && rank < K) rs.slot = rank;
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

// The router logits of one token row from the GEMV partials described at
// RouteParams::logit_parts, by the whole workgroup of 256 threads (one
// barrier; every thread must call it).  The experts + 1 rows (expert rows,
// then the sum-of-squares row) of NP floats are read coalesced: a row's
// NP / 4 lanes each take one 16-byte piece, a wave instruction covers
// 64 / (NP / 4) rows, and every load is unconditional (rows clamped, the
// count fixed at compile time), so the workgroup waits for one round of
// loads.  A row's lanes meet by an xor-shuffle tree, the same in every
// workgroup, so every workgroup gets the same bits.  lds [experts + 1]
// receives them scaled; workgroup 0 also stores the logits (logits_out).
template <int NP>
__device__ inline void logits_from_parts_np(const RouteParams &p, float *lds) {
    constexpr int kLpr = NP / 4;                        // lanes per row
    constexpr int kRpi = 64 / kLpr;                     // rows per wave instruction
    constexpr int kStride = 4 * kRpi;                   // rows per round of the 4 waves
    constexpr int kIter = (kMaxRouteFused + kStride) / kStride;  // covers 64 + 1 rows
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int E = p.experts;
    const int sub = lane / kLpr, piece = lane % kLpr;
    float sum[kIter];
#pragma unroll
    for (int i = 0; i < kIter; ++i) {
        const int row = wave * kRpi + i * kStride + sub;
        const int rc = row <= E ? row : E;  // clamped: loaded, unused
        const f32x4 v = load_f4(p.logit_parts + (long)rc * NP + 4 * piece);
        sum[i] = (v.x + v.y) + (v.z + v.w);
    }
    // the rows' trees step by step across all rows, so that the shuffles of
    // one step are independent and overlap
#pragma unroll
    for (int o = 1; o < kLpr; o <<= 1) {
#pragma unroll
        for (int i = 0; i < kIter; ++i) sum[i] += __shfl_xor(sum[i], o, 64);
    }
#pragma unroll
    for (int i = 0; i < kIter; ++i) {
        const int row = wave * kRpi + i * kStride + sub;
        if (piece == 0 && row <= E) lds[row] = sum[i];
    }
    __syncthreads();
    const float inv_rms = 1.0f / sqrtf(lds[E] / (float)p.width + p.eps);
    if (t < E) {
        const float lg = lds[t] * inv_rms;
        lds[t] = lg;
        if (blockIdx.x == 0 && blockIdx.y == 0 && p.logits_out) p.logits_out[t] = lg;
    }
    __syncthreads();
}
// n_parts: a power of two from 16 to 256; experts <= kMaxRouteFused.
__device__ inline void logits_from_parts(const RouteParams &p, float *lds) {
    switch (p.n_parts) {
    case 16: logits_from_parts_np<16>(p, lds); break;
    case 32: logits_from_parts_np<32>(p, lds); break;
    case 64: logits_from_parts_np<64>(p, lds); break;
    case 128: logits_from_parts_np<128>(p, lds); break;
    default: logits_from_parts_np<256>(p, lds); break;
    }
}

// One token row: routing and route tables by a single wave with no barrier.
// With one row and distinct experts the tables are direct: expert e in slot k
// is the u-th taken expert (u = k unless a fixed id was invalid), with one
// list entry at offset u.
// A lane's routing operands for a one-row batch (lane = expert): its router
// logit (LOGIT), its selection bias and its expert table entry (zero past
// the experts).  Loaded unconditionally (index clamped; p.logits and
// p.expert_table set), so the loads stay in flight together.
struct LaneRoute {
    float logit, bias;
    ExpertWeights w;
};
template <bool LOGIT>
__device__ __forceinline__ LaneRoute lane_route_load(const RouteParams &p, int lane) {
    const bool have = lane < p.experts;
    const int e = have ? lane : 0;
    LaneRoute r;
    r.w = p.expert_table[e];
    const float b = p.bias[e];
    r.bias = have ? b : 0.0f;
    r.logit = 0.0f;
    if constexpr (LOGIT) {
        const float lg = p.logits[e];
        r.logit = have ? lg : 0.0f;
    }
    return r;
}

__device__ __forceinline__ void route_single_64(const RouteParams &p, int lane,
                                                unsigned long long *keys, const LaneRoute &lr) {
    const int E = p.experts, K = p.top_k;
    const bool have = lane < E;
    const RowSelection rs = select_row_64_v<true>(p, 0, lane, nullptr, lr.logit, lr.bias, keys);
    const ExpertWeights &ew = lr.w;
    const int slot = rs.slot;
    if (lane < K && !((rs.filled >> lane) & 1ull)) {
        p.list_pos[lane] = -1;
        if (*p.error == 0) *p.error = p.error_code;  // prepare_route_tables rejects such ids (moonlight_metal.m:545)
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
// The same from memory (route_kernel; the expert table may be absent when
// no task table is written).
__device__ __forceinline__ void route_single_64(const RouteParams &p, int lane,
                                                unsigned long long *keys) {
    const bool have = lane < p.experts;
    LaneRoute lr{have ? p.logits[lane] : 0.0f, have ? p.bias[lane] : 0.0f, ExpertWeights{}};
    if (p.expert_table && have) lr.w = p.expert_table[lane];
    route_single_64(p, lane, keys, lr);
}


// The expert of routed task `task` (the task-th taken expert in slot order)
// of a one-row batch, selected from the router logits exactly as
// route_single_64 selects it, and its weights; -1 when the task is empty.
// Every lane holds its expert's table entry (LaneRoute), so the weights need
// no dependent load.  Called by whole waves.
__device__ __forceinline__ int inline_task_expert(const RouteParams &p, int task,
                                                  ExpertWeights *ew, unsigned long long *keys,
                                                  const LaneRoute &lr) {
    const int lane = threadIdx.x & 63;
    const ExpertWeights &mine = lr.w;
    const RowSelection rs = select_row_64_v<false>(p, 0, lane, nullptr, lr.logit, lr.bias, keys);
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

// ---------------------------------------------------------------------------
// Any expert count and small batches (one workgroup): the arg-max scan, the
// route tables.
// ---------------------------------------------------------------------------

constexpr int kMaxExperts = 256;
constexpr int kMaxTopK = 16;

// Routing of one token row by one wave: sigmoid scores, top-k selection (or
// the given expert ids, moe_route_fixed, moe_route.h:76-87), finalised
// weights (moe_route_finalize, moe_route.h:89-99).  Writes ids / weights /
// trace, and the ids into lds_ids when it is non-null.
__device__ inline void route_row(const RouteParams &p, int r, int lane, int *lds_ids) {
    const int E = p.experts, K = p.top_k;
    float score[kMaxExperts / 64];
    float sel[kMaxExperts / 64];
#pragma unroll
    for (int j = 0; j < kMaxExperts / 64; ++j) {
        const int e = lane + 64 * j;
        if (e < E) {
            score[j] = sigmoid_exact(p.logits[(long)r * E + e]);
            sel[j] = score[j] + p.bias[e];
        } else {
            score[j] = 0.0f;
            sel[j] = -INFINITY;
        }
    }
    // lane k keeps the k-th id and weight; the weight sum runs in slot order
    int my_id = -1;
    float my_w = 0.0f, wsum = 0.0f;
    if (p.fixed_ids) {
        for (int k = 0; k < K; ++k) {
            const int e = p.fixed_ids[(long)r * K + k];
            const bool valid = e >= 0 && e < E;
            const int owner = valid ? (e & 63) : 0, slot_j = valid ? e >> 6 : -1;
            float chosen = 0.0f;
#pragma unroll
            for (int j = 0; j < kMaxExperts / 64; ++j)
                if (lane == owner && j == slot_j) chosen = score[j];
            const float w = __shfl(chosen, owner, 64);
            if (lane == k) {
                my_id = valid ? e : -1;
                my_w = w;
            }
            wsum += w;
        }
    } else {
        unsigned taken = 0;  // bit j: lane's expert lane + 64 j already chosen
        for (int k = 0; k < K; ++k) {
            // lane-local scan in increasing expert order, strict '>' keeps the
            // lower index on ties (moe_route.h:59-71)
            float best_v = -INFINITY;
            int best_e = INT_MAX;
#pragma unroll
            for (int j = 0; j < kMaxExperts / 64; ++j) {
                const int e = lane + 64 * j;
                if (e < E && !(taken & (1u << j)) && sel[j] > best_v) {
                    best_v = sel[j];
                    best_e = e;
                }
            }
            // wave arg-max: larger value wins, equal values keep the lower id
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const float ov = __shfl_xor(best_v, o, 64);
                const int oe = __shfl_xor(best_e, o, 64);
                if (ov > best_v || (ov == best_v && oe < best_e)) {
                    best_v = ov;
                    best_e = oe;
                }
            }
            if (best_e == INT_MAX) best_e = -1;  // only NaN scores remain
            const int owner = best_e < 0 ? 0 : (best_e & 63), slot_j = best_e < 0 ? -1 : best_e >> 6;
            float chosen = 0.0f;
#pragma unroll
            for (int j = 0; j < kMaxExperts / 64; ++j)
                if (lane == owner && j == slot_j) {
                    taken |= 1u << j;
                    chosen = score[j];
                }
            const float w = __shfl(chosen, owner, 64);
            if (lane == k) {
                my_id = best_e;
                my_w = w;
            }
            wsum += w;
        }
    }
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
}

// Any expert count: the rank form for up to 64 experts, else the arg-max scan.
__device__ inline void route_any(const RouteParams &p, int r, int lane, int *lds_ids,
                                 unsigned long long *keys) {
    if (p.experts <= 64)
        (void)select_row_64(p, r, lane, lds_ids, keys);
    else
        route_row(p, r, lane, lds_ids);
}

// Rows routed inside one workgroup (2 rows per wave); larger batches select
// with one wave per row across many workgroups.
constexpr int kRouteOneGroupRows = 8;

// Route tables of a small batch (rows * top_k <= kRouteFusedMaxPositions,
// ids already in LDS), built by one workgroup of 4 waves.
constexpr int kRouteFusedMaxPositions = 1024;
struct RouteLds {
    int first_pos[kMaxExperts], counts[kMaxExperts], offsets[kMaxExperts];
    int unique[kMaxExperts];  // experts in first-appearance order
    int ids[kRouteFusedMaxPositions];
    unsigned long long first_mask[kRouteFusedMaxPositions / 64];
    int word_prefix[kRouteFusedMaxPositions / 64];
    int rank_of[kMaxExperts], count_by_rank[kMaxExperts], offset_by_rank[kMaxExperts];
    int unique_total;
};

// The per-task table of the grouped expert launches: entry u describes the
// u-th active expert (weights, rows, list offset); entries up to task_slots
// past the active experts get count 0.
__device__ inline void write_tasks(const RouteParams &p, const int *counts, const int *offsets,
                            const int *rank_of, int n_unique) {
    if (!p.tasks) return;
    for (int e = threadIdx.x; e < p.experts; e += blockDim.x) {
        const int rk = rank_of[e];
        if (rk >= 0 && rk < p.task_slots) store_task(p.tasks + rk, p.expert_table[e], counts[e], offsets[e]);
    }
    for (int u = n_unique + threadIdx.x; u < p.task_slots; u += blockDim.x)
        store_task(p.tasks + u, ExpertWeights{}, 0, 0);
}

// A barrier for LDS data: the wave's LDS accesses complete, then the
// workgroup meets.  Global stores are not waited for (__syncthreads would
// wait for them): nothing in the workgroup reads them back.
__device__ __forceinline__ void lds_barrier() {
    // LDS-only release / acquire around the barrier: the compiler keeps every
    // LDS access on its side of it (a plain s_barrier is no memory operation
    // to it) and waits only for LDS operations (lgkmcnt), not for loads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ inline void small_tables(const RouteParams &p, RouteLds &L) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int E = p.experts, K = p.top_k, M = p.rows;
    const int n_pos = M * K;
    for (int e = tid; e < E; e += blockDim.x) {
        L.first_pos[e] = INT_MAX;
        L.counts[e] = 0;
    }
    lds_barrier();
    // first appearance and count per expert (order-independent LDS atomics)
    for (int q = tid; q < n_pos; q += blockDim.x) {
        const int e = L.ids[q];
        if (e < 0 || e >= E) {
            p.list_pos[q] = -1;
            if (*p.error == 0) *p.error = p.error_code;  // prepare_route_tables rejects such ids (moonlight_metal.m:545)
            continue;
        }
        atomicMin(&L.first_pos[e], q);
        atomicAdd(&L.counts[e], 1);
    }
    lds_barrier();
    // first-appearance ranks: a bit per list position that is the first
    // occurrence of its expert; the rank of e counts those bits before it
    const int nwords = (n_pos + 63) / 64;
    const int nwaves = (int)blockDim.x >> 6;
    for (int w = wave; w < nwords; w += nwaves) {
        const int q = w * 64 + lane;
        bool first = false;
        if (q < n_pos) {
            const int e = L.ids[q];
            first = e >= 0 && e < E && L.first_pos[e] == q;
        }
        const unsigned long long m = __ballot(first);
        if (lane == 0) L.first_mask[w] = m;
    }
    lds_barrier();
    if (wave == 0) {  // word prefix (<= 16 words) by a wave scan
        const int cnt = lane < nwords ? __popcll(L.first_mask[lane]) : 0;
        int incl = cnt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o, 64);
            if (lane >= o) incl += v;
        }
        if (lane < nwords) L.word_prefix[lane] = incl - cnt;
        const int total = __shfl(incl, 63, 64);
        if (lane == 0) {
            L.unique_total = total;
            *p.n_unique = total;
        }
    }
    lds_barrier();
    for (int e = tid; e < E; e += blockDim.x) {
        L.rank_of[e] = -1;
        if (L.counts[e] > 0) {
            const int q = L.first_pos[e];
            const int rank = L.word_prefix[q / 64] +
                             __popcll(L.first_mask[q / 64] & ((1ull << (q % 64)) - 1ull));
            L.rank_of[e] = rank;
            L.count_by_rank[rank] = L.counts[e];
            L.unique[rank] = e;
            p.unique[rank] = e;
        }
        p.counts[e] = L.counts[e];
    }
    lds_barrier();
    if (wave == 0) {  // exclusive scan of the counts in rank order (<= 256 ranks)
        int c4[4], local = 0;
        const int n_unique = L.unique_total;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rk = lane * 4 + i;
            c4[i] = rk < n_unique ? L.count_by_rank[rk] : 0;
            local += c4[i];
        }
        int incl = local;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o, 64);
            if (lane >= o) incl += v;
        }
        int run = incl - local;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rk = lane * 4 + i;
            if (rk < n_unique) L.offset_by_rank[rk] = run;
            run += c4[i];
        }
    }
    lds_barrier();
    for (int e = tid; e < E; e += blockDim.x) {
        if (L.rank_of[e] >= 0) {
            L.offsets[e] = L.offset_by_rank[L.rank_of[e]];
            p.offsets[e] = L.offsets[e];
        }
    }
    lds_barrier();
    write_tasks(p, L.counts, L.offsets, L.rank_of, L.unique_total);
    // compact lists: entries of expert e in (row, slot) order
    for (int e = wave; e < E; e += nwaves) {
        if (L.counts[e] == 0) continue;
        int running = 0;
        const int base = L.offsets[e];
        for (int q0 = 0; q0 < n_pos; q0 += 64) {
            const int q = q0 + lane;
            const bool match = q < n_pos && L.ids[q] == e;
            const unsigned long long mask = __ballot(match);
            if (match) {
                const int j = running + __popcll(mask & ((1ull << lane) - 1ull));
                p.list_rows[base + j] = q / K;
                p.list_slots[base + j] = q % K;
                p.list_pos[q] = base + j;
            }
            running += __popcll(mask);
        }
    }
}


}  // namespace mlh

// moe.hip -- device routing, route tables, grouped expert FFN launches and the
// deterministic combine of the Moonlight MoE layer.
//
// References (c4pt0r/floyd):
//   routing   moonlight_route_sigmoid_topk (moonlight_kernels.metal:469-512) =
//             moe_route_select + moe_route_finalize (moe_route.h:47-99)
//   tables    prepare_route_tables (moonlight_metal.m:525-559), which the
//             reference runs on the HOST after a blocking wait; here they are
//             built on the device so a layer needs no host round trip
//   experts   encode_moe_residual_buffer (moonlight_metal.m:561-676)
//   combine   moonlight_scatter_expert + moonlight_add_f32
//             (moonlight_kernels.metal:543-569)
#include "mlh_device.h"
#include "moe.h"

#include <climits>
#include <cstdlib>

namespace mlh {

constexpr int kRouteLdsIds = 4096;

// One workgroup: routing of every token row, then the route tables (small
// batches whose logits already exist).
__global__ __launch_bounds__(256) void route_kernel(RouteParams p) {
    __shared__ RouteLds L;
    __shared__ __align__(16) unsigned long long keys[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (p.rows == 1 && p.experts <= 64) {
        if (wave == 0) route_single_64(p, lane, keys[0]);
        return;
    }
    for (int r = wave; r < p.rows; r += 4) route_any(p, r, lane, L.ids, keys[wave]);
    __syncthreads();
    small_tables(p, L);
}

// Larger batches: one wave per token row over many workgroups; the tables
// follow in route_lists_kernel.
__global__ __launch_bounds__(256) void route_select_kernel(RouteParams p) {
    __shared__ __align__(16) unsigned long long keys[4][64];
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r < p.rows) route_any(p, r, threadIdx.x & 63, nullptr, keys[threadIdx.x >> 6]);
}

// Route tables of a batch of more than a few rows (prepare_route_tables,
// moonlight_metal.m:525-559) with one workgroup per expert.  Every workgroup
// histograms all positions (counts and first appearance through LDS atomics,
// which do not depend on order), so each derives its expert's rank in
// first-appearance order and its list offset without waiting for another
// workgroup, then writes its expert's list entries in position order.
// Workgroup 0 also writes the batch-wide outputs (n_unique, invalid-id marks,
// the tail of the task table).
constexpr unsigned short kNoExpert = 0xFFFF;
__global__ __launch_bounds__(1024) void route_lists_kernel(RouteParams p) {
    __shared__ int counts[kMaxExperts], first_pos[kMaxExperts];
    __shared__ unsigned short ids16[kRouteMaxPositions];
    __shared__ int wave_count[16];
    __shared__ int s_rank, s_offset, s_unique;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = p.experts, K = p.top_k, n_pos = p.rows * p.top_k;
    const int e = blockIdx.x;
    for (int i = tid; i < E; i += blockDim.x) {
        counts[i] = 0;
        first_pos[i] = INT_MAX;
    }
    __syncthreads();
    for (int q = tid; q < n_pos; q += blockDim.x) {
        const int id = p.ids[q];
        const bool ok = id >= 0 && id < E;
        ids16[q] = ok ? (unsigned short)id : kNoExpert;
        if (ok) {
            atomicAdd(&counts[id], 1);
            atomicMin(&first_pos[id], q);
        } else if (e == 0) {
            p.list_pos[q] = -1;
            if (*p.error == 0) *p.error = p.error_code;  // prepare_route_tables rejects such ids (moonlight_metal.m:545)
        }
    }
    __syncthreads();
    if (wave == 0) {  // rank and offset of e: active experts that appear first
        const int fe = first_pos[e];
        int rk = 0, off = 0, nu = 0;
        for (int i = lane; i < E; i += 64) {
            const int c = counts[i];
            if (c > 0) {
                ++nu;
                if (first_pos[i] < fe) {
                    ++rk;
                    off += c;
                }
            }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            rk += __shfl_xor(rk, o, 64);
            off += __shfl_xor(off, o, 64);
            nu += __shfl_xor(nu, o, 64);
        }
        if (lane == 0) {
            s_rank = counts[e] > 0 ? rk : -1;
            s_offset = off;
            s_unique = nu;
        }
    }
    __syncthreads();
    const int rank = s_rank, offset = s_offset, n_unique = s_unique;
    if (tid == 0) {
        p.counts[e] = counts[e];
        if (rank >= 0) {
            p.offsets[e] = offset;
            p.unique[rank] = e;
        }
        if (e == 0) *p.n_unique = n_unique;
        if (p.tasks && rank >= 0 && rank < p.task_slots)
            store_task(p.tasks + rank, p.expert_table[e], counts[e], offset);
    }
    if (p.tasks && e == 0)
        for (int u = n_unique + tid; u < p.task_slots; u += blockDim.x)
            store_task(p.tasks + u, ExpertWeights{}, 0, 0);
    if (rank < 0) return;  // the whole workgroup: no list entries
    // list entries of e in position order: wave w takes the contiguous
    // positions [w * seg, (w + 1) * seg), counts its entries (ballots), the
    // waves' counts meet in one exclusive scan, then each wave writes its
    // entries from its start (two barriers whatever the batch)
    const int nw = (int)(blockDim.x >> 6);
    const int seg = (n_pos + nw - 1) / nw;
    const int q_lo = wave * seg, q_hi = min(n_pos, q_lo + seg);
    int mine_count = 0;
    for (int q0 = q_lo; q0 < q_hi; q0 += 64) {
        const int q = q0 + lane;
        mine_count += __popcll(__ballot(q < q_hi && ids16[q] == e));
    }
    if (lane == 0) wave_count[wave] = mine_count;
    __syncthreads();
    int j0 = offset;
    for (int w = 0; w < wave; ++w) j0 += wave_count[w];
    for (int q0 = q_lo; q0 < q_hi; q0 += 64) {
        const int q = q0 + lane;
        const bool mine = q < q_hi && ids16[q] == e;
        const unsigned long long m = __ballot(mine);
        if (mine) {
            const int j = j0 + __popcll(m & ((1ull << lane) - 1ull));
            p.list_rows[j] = q / K;
            p.list_slots[j] = q % K;
            p.list_pos[q] = j;
        }
        j0 += __popcll(m);
    }
}

// Router logits for many token rows (prefill): logits[r][e] = RMSNorm(x[r]) .
// W[e] with an f32 router [experts][width] (moonlight_kernels.metal:43-60, the
// post-attention norm of :23-41 applied to x), on fp32 MFMA
// (v_mfma_f32_16x16x4_f32: fp32 products and sums, like the VALU matmul, in
// another order).  The norm's 1 / rms is a per-row factor of the dot product,
// so one pass accumulates sum_k (x n)[k] w[e][k] and sum_k x[k]^2 together and
// scales at the end.  A workgroup owns 16 rows x 32 experts (two 16 x 16
// tiles); its 4 waves take the 16-wide k steps w, w + 4, ... and meet in LDS
// in wave order (deterministic).  Lane l feeds row / expert l % 16 and, per
// group of 4 MFMAs, the k values 4 (l / 16) .. + 3 of a 16-wide step; a
// wave's loads go out kRouterBatch steps ahead of their MFMAs.
typedef float f32x4v_r __attribute__((ext_vector_type(4)));
constexpr int kRouterRows = 16, kRouterCols = 32, kRouterBatch = 4;
__global__ __launch_bounds__(256) void router_logits_kernel(const float *x, const float *norm_w,
                                                            float eps, const float *w, int rows,
                                                            int experts, int width,
                                                            float *logits) {
    __shared__ float part[4][2][16][16];  // [wave][tile][row][expert]
    __shared__ float ssq[4][16];          // [wave][row]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, m16 = lane & 15;
    const int r0 = blockIdx.x * kRouterRows, e0 = blockIdx.y * kRouterCols;
    const int row = min(r0 + m16, rows - 1);  // rows / experts past the end are never stored
    const float *xr = x + (long)row * width;
    const float *wr0 = w + (long)min(e0 + m16, experts - 1) * width;
    const float *wr1 = w + (long)min(e0 + 16 + m16, experts - 1) * width;
    f32x4v_r acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    float ss = 0.0f;
    const int steps = width / 16;
    for (int s0 = wave; s0 < steps; s0 += 4 * kRouterBatch) {
        f32x4 xv[kRouterBatch], nv[kRouterBatch], w0[kRouterBatch], w1[kRouterBatch];
#pragma unroll
        for (int b = 0; b < kRouterBatch; ++b) {
            const int st = s0 + 4 * b;
            const int k = (st < steps ? st : s0) * 16 + 4 * g;  // clamped: loaded, unused
            xv[b] = load_f4(xr + k);
            w0[b] = load_f4(wr0 + k);
            w1[b] = load_f4(wr1 + k);
            nv[b] = norm_w ? load_f4(norm_w + k) : f32x4{1.f, 1.f, 1.f, 1.f};
        }
#pragma unroll
        for (int b = 0; b < kRouterBatch; ++b) {
            if (s0 + 4 * b < steps) {
                const f32x4 v = xv[b];
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                const float a[4] = {v.x * nv[b].x, v.y * nv[b].y, v.z * nv[b].z, v.w * nv[b].w};
                const float b0[4] = {w0[b].x, w0[b].y, w0[b].z, w0[b].w};
                const float b1[4] = {w1[b].x, w1[b].y, w1[b].z, w1[b].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b0[j], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b1[j], acc1, 0, 0, 0);
                }
            }
        }
    }
    // the 4 lane groups of a row hold disjoint k: sum them (row m16)
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    if (g == 0) ssq[wave][m16] = ss;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        part[wave][0][4 * g + i][m16] = acc0[i];
        part[wave][1][4 * g + i][m16] = acc1[i];
    }
    __syncthreads();
    for (int o = tid; o < kRouterRows * kRouterCols; o += blockDim.x) {
        const int rr = o / kRouterCols, c = o % kRouterCols;
        const int r = r0 + rr, e = e0 + c;
        if (r >= rows || e >= experts) continue;
        const int t = c >> 4, ec = c & 15;
        const float v = (part[0][t][rr][ec] + part[1][t][rr][ec]) +
                        (part[2][t][rr][ec] + part[3][t][rr][ec]);
        float inv = 1.0f;
        if (norm_w) {
            const float sq = (ssq[0][rr] + ssq[1][rr]) + (ssq[2][rr] + ssq[3][rr]);
            inv = 1.0f / sqrtf(sq / (float)width + eps);
        }
        logits[(long)r * experts + e] = v * inv;
    }
}

int router_logits(const float *x, const float *norm_w, float eps, const float *w, int rows,
                  int experts, int width, float *logits, hipStream_t stream) {
    if (!x || !w || !logits || rows <= 0 || experts <= 0 || width <= 0 || width % 16) return kErrArgs;
    hipLaunchKernelGGL(router_logits_kernel,
                       dim3((rows + kRouterRows - 1) / kRouterRows,
                            (experts + kRouterCols - 1) / kRouterCols),
                       dim3(256), 0, stream, x, norm_w, eps, w, rows, experts, width, logits);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// Router logits for batches of fewer rows than router_logits_kernel needs
// for its parallelism (decode batches, short prefill chunks): workgroup
// (expert e, group of up to kRsRows token rows), thread t taking 8
// consecutive k of every 2048 (one load of the expert's weights and the norm
// weight), the same sums as router_logits_kernel (sum_k (x n)[k] w[e][k] and
// sum_k x[k]^2 per row, the norm's 1 / rms applied at the end).  The 256
// threads' sums meet in LDS: thread (row, segment) adds 16 of them in
// order, then the row's 16 segments by a butterfly, so the result does not
// depend on timing.  One round of loads instead of the GEMV's passes.
constexpr int kRsRows = 16;
__global__ __launch_bounds__(256) void router_small_kernel(const float *x, const float *norm_w,
                                                           float eps, const float *w, int rows,
                                                           int experts, int width,
                                                           float *logits) {
    __shared__ float part[2][kRsRows][257];  // [dot, sum of squares][row][thread]
    const int t = threadIdx.x, e = blockIdx.x, r0 = blockIdx.y * kRsRows;
    const int nr = rows - r0 < kRsRows ? rows - r0 : kRsRows;
    const float *we = w + (long)e * width;
    float dot[kRsRows], ss[kRsRows];
#pragma unroll
    for (int r = 0; r < kRsRows; ++r) dot[r] = ss[r] = 0.0f;
    for (int k = 8 * t; k < width; k += 8 * 256) {
        const f32x4 w0 = load_f4(we + k), w1 = load_f4(we + k + 4);
        f32x4 n0 = {1.f, 1.f, 1.f, 1.f}, n1 = {1.f, 1.f, 1.f, 1.f};
        if (norm_w) {
            n0 = load_f4(norm_w + k);
            n1 = load_f4(norm_w + k + 4);
        }
        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        const float nv[8] = {n0.x, n0.y, n0.z, n0.w, n1.x, n1.y, n1.z, n1.w};
#pragma unroll
        for (int r = 0; r < kRsRows; ++r) {
            if (r < nr) {
                const float *xr = x + (long)(r0 + r) * width + k;
                const f32x4 a = load_f4(xr), b = load_f4(xr + 4);
                const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    ss[r] += xv[j] * xv[j];
                    dot[r] += (xv[j] * nv[j]) * wv[j];
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kRsRows; ++r) {
        part[0][r][t] = dot[r];
        part[1][r][t] = ss[r];
    }
    __syncthreads();
    const int row = t >> 4, seg = t & 15;
    float d = 0.0f, q = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        d += part[0][row][16 * seg + j];
        q += part[1][row][16 * seg + j];
    }
    d = group_sum<16>(d);
    q = group_sum<16>(q);
    if (seg == 0 && row < nr) {
        const float inv = norm_w ? 1.0f / sqrtf(q / (float)width + eps) : 1.0f;
        logits[(long)(r0 + row) * experts + e] = d * inv;
    }
}

int router_logits_small(const float *x, const float *norm_w, float eps, const float *w, int rows,
                        int experts, int width, float *logits, hipStream_t stream) {
    if (!x || !w || !logits || rows <= 0 || experts <= 0 || width <= 0 || width % 8)
        return kErrArgs;
    hipLaunchKernelGGL(router_small_kernel, dim3(experts, (rows + kRsRows - 1) / kRsRows),
                       dim3(256), 0, stream, x, norm_w, eps, w, rows, experts, width, logits);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int route_topk(const RouteParams &p, hipStream_t stream) {
    if (!p.logits || !p.bias || !p.ids || !p.weights || p.rows <= 0 || p.experts <= 0 ||
        p.experts > kMaxExperts || p.top_k <= 0 || p.top_k > kMaxTopK ||
        p.top_k > p.experts || !p.n_unique || !p.unique || !p.counts || !p.offsets ||
        !p.list_rows || !p.list_slots || !p.list_pos || !p.error ||
        p.rows * p.top_k > kRouteMaxPositions)
        return kErrArgs;
    if (p.rows <= kRouteOneGroupRows) {
        // a few rows: selection and tables in one workgroup
        hipLaunchKernelGGL(route_kernel, dim3(1), dim3(256), 0, stream, p);
    } else {
        hipLaunchKernelGGL(route_select_kernel, dim3((p.rows + 3) / 4), dim3(256), 0, stream, p);
        hipLaunchKernelGGL(route_lists_kernel, dim3(p.experts), dim3(1024), 0, stream, p);
    }
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// out[r] = resid[r] + (sum_k w[r,k] * y[pos[r,k]] + shared[r]); routed sum in
// slot order (tests/test_moonlight_metal_moe.c:118-135), deterministic.
__global__ __launch_bounds__(256) void combine_kernel(CombineParams p) {
    const int r = blockIdx.x;
    const int K = p.top_k;
    for (int d = blockIdx.y * blockDim.x + threadIdx.x; d < p.hidden;
         d += gridDim.y * blockDim.x) {
        float routed = 0.0f;
        for (int k = 0; k < K; ++k) {
            const int q = r * K + k;
            const int pos = p.list_pos[q];
            if (pos >= 0) routed += p.weights[q] * p.expert_out[(long)pos * p.hidden + d];
        }
        float shared = p.shared_out[(long)r * p.hidden + d];
        if (p.shared_out2) shared += p.shared_out2[(long)r * p.hidden + d];
        if (p.routed_copy) {
            p.routed_copy[(long)r * p.hidden + d] = routed;
            p.shared_out[(long)r * p.hidden + d] = shared;
        }
        float out = routed + shared;
        if (p.resid) out = p.resid[(long)r * p.hidden + d] + out;
        p.out[(long)r * p.hidden + d] = out;
    }
}

// The same sums, four hidden dims per thread (hidden a multiple of 4): the
// row's slot positions and weights are loaded once (the same for the whole
// workgroup), then every slot's expert output, the shared outputs and the
// residual are in flight together; per dim the terms are added in the order
// of combine_kernel, so the results are the same bits.
__global__ __launch_bounds__(256) void combine4_kernel(CombineParams p) {
    const int r = blockIdx.x, K = p.top_k;
    int pos[kMaxTopK];
    float wt[kMaxTopK];
#pragma unroll
    for (int k = 0; k < kMaxTopK; ++k) {
        pos[k] = k < K ? p.list_pos[r * K + k] : -1;
        wt[k] = k < K ? p.weights[r * K + k] : 0.0f;
    }
    const int d = 4 * (blockIdx.y * blockDim.x + threadIdx.x);
    if (d >= p.hidden) return;
    const long o = (long)r * p.hidden + d;
    f32x4 ev[kMaxTopK];
#pragma unroll
    for (int k = 0; k < kMaxTopK; ++k)
        ev[k] = pos[k] >= 0 ? load_f4(p.expert_out + (long)pos[k] * p.hidden + d)
                            : f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 sh = load_f4(p.shared_out + o);
    const f32x4 sh2 = p.shared_out2 ? load_f4(p.shared_out2 + o) : f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 rs = p.resid ? load_f4(p.resid + o) : f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 routed = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < kMaxTopK; ++k) {
        if (pos[k] >= 0) {
            routed.x += wt[k] * ev[k].x;
            routed.y += wt[k] * ev[k].y;
            routed.z += wt[k] * ev[k].z;
            routed.w += wt[k] * ev[k].w;
        }
    }
    if (p.shared_out2) {
        sh.x += sh2.x;
        sh.y += sh2.y;
        sh.z += sh2.z;
        sh.w += sh2.w;
    }
    if (p.routed_copy) {
        *reinterpret_cast<f32x4 *>(p.routed_copy + o) = routed;
        *reinterpret_cast<f32x4 *>(p.shared_out + o) = sh;
    }
    f32x4 out = {routed.x + sh.x, routed.y + sh.y, routed.z + sh.z, routed.w + sh.w};
    if (p.resid) out = f32x4{rs.x + out.x, rs.y + out.y, rs.z + out.z, rs.w + out.w};
    *reinterpret_cast<f32x4 *>(p.out + o) = out;
}

int moe_combine(const CombineParams &p, hipStream_t stream) {
    if (!p.weights || !p.list_pos || !p.expert_out || !p.shared_out || !p.out || p.rows <= 0 ||
        p.top_k <= 0 || p.top_k > kMaxTopK)
        return kErrArgs;
    if (p.hidden % 4 == 0) {  // 1024 dims a workgroup (measured on MI355X, T = 2048: 47.6 us
                              // for the one-float form)
        hipLaunchKernelGGL(combine4_kernel, dim3(p.rows, (p.hidden + 1023) / 1024), dim3(256), 0,
                           stream, p);
    } else {
        // one workgroup per 256 hidden dims of a row
        hipLaunchKernelGGL(combine_kernel, dim3(p.rows, (p.hidden + 255) / 256), dim3(256), 0,
                           stream, p);
    }
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// One-row MoE layer: the down projections and the combine in one launch.
// out = resid + (sum over slots k of w_k * down_k(h_k) + down_sh(h_sh)), the
// routed sum in slot order as in combine_kernel.  Workgroup over RPB output
// rows, one wave per unit: unit k < top_k is slot k's expert (list entry
// list_pos[k], weights from the task table), unit top_k + j the j-th
// inter-wide column slice of the shared down projection.  A wave splits its
// own input vector into limbs in its LDS row (per-chunk scales, as in the
// GEMV), multiplies its RPB x inter weight block (64 / RPB lanes per row, NJ
// chunks per lane, all loads issued first), and the units' rows meet in LDS.
constexpr int kDownCombineRows = 8;     // output rows per workgroup
constexpr int kDownCombineChunks = 11;  // 16-byte chunks per lane and row (q8: inter <= 1408)
constexpr int kDownCombineMaxUnits = 16;

struct DownCombineParams {
    int hidden = 0, inter = 0, top_k = 0, units = 0, shared_width = 0;
    const ExpertTask *tasks = nullptr;
    const int *list_pos = nullptr;
    const float *weights = nullptr;
    const float *expert_hidden = nullptr;  // [top_k][inter] list entries
    const float *shared_hidden = nullptr;  // [shared_width]
    const uint8_t *shared_down = nullptr;
    const float *shared_down_s = nullptr;
    const float *resid = nullptr;
    float *routed_copy = nullptr, *shared_copy = nullptr;
    float *out = nullptr;
};

template <int FMT, int RPB, int NJ>
__global__ __launch_bounds__(1024) void moe_down_combine_kernel(DownCombineParams p) {
    extern __shared__ __align__(16) unsigned char dc_lds[];
    constexpr int LPR = 64 / RPB;
    __shared__ float part[kDownCombineMaxUnits][RPB];
    const int lane = threadIdx.x & 63;
    const int u = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int rr = lane / LPR, li = lane % LPR;
    const int d0 = blockIdx.x * RPB;
    const int row = d0 + rr < p.hidden ? d0 + rr : p.hidden - 1;
    const int I = p.inter;
    const int nc = row_bytes_of(FMT, I) / 16;
    // ---- the unit: weights, row stride, scales, input vector
    const uint8_t *w;
    const float *s, *x;
    long stride;
    bool active = true;
    if (u < p.top_k) {
        // a slot without an expert (e.g. NaN logits: nothing is taken, and
        // the task table may hold no weights at all) reads the shared down
        // rows instead, in bounds at the routed stride, and contributes 0
        const int pos = p.list_pos[u];
        active = pos >= 0;
        if (active) {
            const ExpertTask tk = p.tasks[pos];
            w = tk.w.down;
            s = tk.w.down_s;
        } else {
            w = p.shared_down;
            s = p.shared_down_s;
        }
        stride = row_bytes_of(FMT, I);
        x = p.expert_hidden + (long)(active ? pos : 0) * I;
    } else {
        const int j = u - p.top_k;
        w = p.shared_down + (long)j * row_bytes_of(FMT, I);
        s = p.shared_down_s;
        stride = row_bytes_of(FMT, p.shared_width);
        x = p.shared_hidden + (long)j * I;
    }
    // ---- the input vector first, every pass unconditional (clamped), then
    // the weights (clamped addresses, zero past the row end): in-order
    // completion lets the limb split below wait for the input alone while
    // the weights stream
    constexpr int kXPass = (LPR * NJ * (FMT == kQ8 ? 16 : 32) + 511) / 512;  // inter <= this
    f32x4 xa[kXPass], xb[kXPass];
#pragma unroll
    for (int i = 0; i < kXPass; ++i) {
        const int e0 = lane * 8 + 512 * i;
        const int ec = e0 < I ? e0 : 0;
        xa[i] = load_f4(x + ec);
        xb[i] = load_f4(x + ec + 4);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the input loads ahead of the weights
    u32x4 wv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int c = li + LPR * j;
        const u32x4 v = load_stream16(w + (long)row * stride + (c < nc ? c : 0) * 16);
        wv[j] = c < nc ? v : u32x4{0u, 0u, 0u, 0u};
    }
    const float sw = load_global_f32(s + row);
    __builtin_amdgcn_sched_barrier(0);  // the split below waits for the input loads only
    // ---- this wave's input vector into limbs
    unsigned char *my = dc_lds + u * limb_row_lds(FMT, I);
#pragma unroll
    for (int i = 0; i < kXPass; ++i) {
        if (512 * i >= I) break;  // uniform: no loads past here
        const int e0 = lane * 8 + 512 * i;
        const bool in = e0 < I;
        const f32x4 a = xa[i], b = xb[i];
        const float v[8] = {in ? a.x : 0.f, in ? a.y : 0.f, in ? a.z : 0.f, in ? a.w : 0.f,
                            in ? b.x : 0.f, in ? b.y : 0.f, in ? b.z : 0.f, in ? b.w : 0.f};
        limb_quantise<FMT>(v, in, e0, my, I, nc);
    }
    __syncthreads();
    // ---- the wave's RPB rows
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int c = li + LPR * j;
        if (c < nc) {
            const LimbInfo info = reinterpret_cast<const LimbInfo *>(my + 3 * I)[c];
            acc = fmaf(limb_chunk_dot<FMT>(wv[j], my, I, nc, c, info), info.scale, acc);
        }
    }
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, kWave);
    if (li == 0) part[u][rr] = active ? acc * sw : 0.0f;
    __syncthreads();
    if ((int)threadIdx.x < RPB && d0 + (int)threadIdx.x < p.hidden) {
        const int t = threadIdx.x, d = d0 + t;
        float routed = 0.0f;
        for (int k = 0; k < p.top_k; ++k) routed += p.weights[k] * part[k][t];
        float shared = 0.0f;
        for (int k = p.top_k; k < p.units; ++k) shared += part[k][t];
        if (p.routed_copy) p.routed_copy[d] = routed;
        if (p.shared_copy) p.shared_copy[d] = shared;
        float out = routed + shared;
        if (p.resid) out = p.resid[d] + out;
        p.out[d] = out;
    }
}

bool down_combine_ok(const ExpertFfnParams &f) {
    if (f.rows != 1 || !f.has_shared || f.expert_fmt != f.shared_fmt ||
        (f.expert_fmt != kQ8 && f.expert_fmt != kQ4) || f.limb_x || !f.tasks || f.inter <= 0 ||
        f.shared_width % f.inter || f.top_k < 1 || f.hidden <= 0)
        return false;
    const int epc = f.expert_fmt == kQ8 ? 16 : 32;
    if (f.inter % epc) return false;
    const int units = f.top_k + f.shared_width / f.inter;
    const int nc = row_bytes_of(f.expert_fmt, f.inter) / 16;
    return units <= kDownCombineMaxUnits &&
           nc <= (64 / kDownCombineRows) * kDownCombineChunks &&
           units * limb_row_lds(f.expert_fmt, f.inter) <= 96 * 1024;
}

static int moe_down_combine(const ExpertFfnParams &f, hipStream_t stream) {
    DownCombineParams p;
    p.hidden = f.hidden;
    p.inter = f.inter;
    p.top_k = f.top_k;
    p.units = f.top_k + f.shared_width / f.inter;
    p.shared_width = f.shared_width;
    p.tasks = f.tasks;
    p.list_pos = f.list_pos;
    p.weights = f.route_weights;
    p.expert_hidden = f.expert_hidden;
    p.shared_hidden = f.shared_hidden;
    p.shared_down = f.shared_down;
    p.shared_down_s = f.shared_down_s;
    p.resid = f.combine_resid;
    p.routed_copy = f.combine_routed;
    p.shared_copy = f.combine_shared;
    p.out = f.combine_out;
    const int lds = p.units * limb_row_lds(f.expert_fmt, f.inter);
    const dim3 grid((unsigned)((f.hidden + kDownCombineRows - 1) / kDownCombineRows));
    const dim3 block((unsigned)(64 * p.units));
    if (f.expert_fmt == kQ8) {
        auto *k = &moe_down_combine_kernel<kQ8, kDownCombineRows, kDownCombineChunks>;
        static const bool attr = hipFuncSetAttribute(reinterpret_cast<const void *>(k),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     96 * 1024) == hipSuccess;
        (void)attr;
        hipLaunchKernelGGL(k, grid, block, lds, stream, p);
    } else {
        auto *k = &moe_down_combine_kernel<kQ4, kDownCombineRows, kDownCombineChunks>;
        static const bool attr = hipFuncSetAttribute(reinterpret_cast<const void *>(k),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     96 * 1024) == hipSuccess;
        (void)attr;
        hipLaunchKernelGGL(k, grid, block, lds, stream, p);
    }
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// Both grouped expert launches (gate/up + SwiGLU, then down).  The routed
// experts use one format (ebits) and the shared expert possibly another
// (dbits); one launch covers both when the formats agree.
int expert_ffn(const ExpertFfnParams &f, hipStream_t stream) {
    const int max_tasks = f.rows * f.top_k < f.experts ? f.rows * f.top_k : f.experts;
    const int max_rows = f.rows;  // token rows any task can hold
    const bool presplit = f.limb_x != nullptr;
    const bool fused_fmt = f.expert_fmt == f.shared_fmt;
    if (f.route.logits &&
        (f.rows != 1 || f.route.rows != 1 || f.route.experts > 64 || f.route.experts < 1 ||
         f.route.top_k < 1 || f.route.top_k > f.route.experts || presplit || !f.route.tasks ||
         !f.route.expert_table))
        return kErrArgs;
    const bool fused_down = f.combine_out != nullptr;
    if (fused_down && (!down_combine_ok(f) || !f.route_weights || !f.list_pos)) return kErrArgs;
    for (int stage = 0; stage < 2; ++stage) {
        if (stage == 1 && fused_down) return moe_down_combine(f, stream);
        if (presplit) {
            // the stage's inputs, split once: token rows (RMSNorm'ed) for
            // stage 0, list rows and shared rows for stage 1
            LimbRowsParams a, b;
            if (stage == 0) {
                a.fmt = f.expert_fmt;
                a.rows = f.rows;
                a.I = f.hidden;
                a.x = f.x;
                a.x_stride = f.hidden;
                a.norm_w = f.norm_w;
                a.eps = f.eps;
                a.out = f.limb_x;
                a.out_stride = f.limb_x_stride;
                if (f.has_shared && !fused_fmt) {
                    b = a;
                    b.fmt = f.shared_fmt;
                    b.out = f.limb_xs;
                }
            } else {
                a.fmt = f.expert_fmt;
                a.rows = f.rows * f.top_k;
                a.I = f.inter;
                a.x = f.expert_hidden;
                a.x_stride = f.inter;
                a.out = f.limb_h;
                a.out_stride = f.limb_h_stride;
                if (f.has_shared) {
                    b.fmt = f.shared_fmt;
                    b.rows = f.rows;
                    b.I = f.shared_width;
                    b.x = f.shared_hidden;
                    b.x_stride = f.shared_width;
                    b.out = f.limb_sh;
                    b.out_stride = f.limb_sh_stride;
                }
            }
            if (int err = limb_quantise_rows(a, b, stream)) return err;
        }
        GemvLaunch L;
        ExpertGemvParams &e = L.expert;
        if (presplit) {
            e.limbs = stage == 0 ? f.limb_x : f.limb_h;
            e.limb_stride = stage == 0 ? f.limb_x_stride : f.limb_h_stride;
            e.sh_limbs = stage == 0 ? (fused_fmt ? f.limb_x : f.limb_xs) : f.limb_sh;
            e.sh_limb_stride = stage == 0 ? f.limb_x_stride : f.limb_sh_stride;
        }
        e.stage = stage;
        if (stage == 0) e.route = f.route;  // stage 1 reads the tables it wrote
        e.tasks = f.tasks;
        e.experts = f.expert_table;
        e.n_unique = f.n_unique;
        e.unique = f.unique;
        e.counts = f.counts;
        e.offsets = f.offsets;
        e.rows = f.list_rows;
        e.shared_rows = f.rows;
        e.hidden = f.hidden;
        e.inter = f.inter;
        e.shared_width = f.shared_width;
        e.norm_w = f.norm_w;
        e.eps = f.eps;
        if (stage == 0) {
            e.x = f.x;
            e.y = f.expert_hidden;
            e.sh_w = f.shared_gate;
            e.sh_s = f.shared_gate_s;
            e.sh_w2 = f.shared_up;
            e.sh_s2 = f.shared_up_s;
            e.sh_y = f.shared_hidden;
        } else {
            e.x = f.expert_hidden;
            e.y = f.expert_out;
            e.sh_w = f.shared_down;
            e.sh_s = f.shared_down_s;
            e.sh_x = f.shared_hidden;
            e.sh_y = f.shared_out;
        }
        const bool dual = stage == 0;
        const int routed_O = stage == 0 ? f.inter : f.hidden;
        const int routed_I = stage == 0 ? f.hidden : f.inter;
        const int shared_O = stage == 0 ? f.shared_width : f.hidden;
        const int shared_I = stage == 0 ? f.hidden : f.shared_width;
        const bool fused = f.expert_fmt == f.shared_fmt && f.has_shared;
        // routed (+ shared when the formats agree)
        {
            const int widest_I = fused && shared_I > routed_I ? shared_I : routed_I;
            GemvPlan plan = plan_expert_gemv(f.expert_fmt, routed_O, routed_I, max_rows, dual,
                                             max_tasks + (fused ? 2 : 0), widest_I);
            GemvLaunch Lr = L;
            const int per_block = gemv_rows_per_block(plan, dual);
            Lr.expert.routed_tasks = max_tasks;
            Lr.expert.routed_blocks = (routed_O + per_block - 1) / per_block;
            Lr.expert.shared_task = fused ? 1 : 0;
            const int shared_blocks = fused ? (shared_O + per_block - 1) / per_block : 0;
            const dim3 grid(max_tasks * Lr.expert.routed_blocks + shared_blocks,
                            (max_rows + plan.b - 1) / plan.b);
            if (!dispatch_gemv(f.expert_fmt, Lr, 1, plan, grid, stream)) return kErrArgs;
        }
        if (f.has_shared && !fused) {
            GemvPlan plan = plan_expert_gemv(f.shared_fmt, shared_O, shared_I, max_rows, dual, 1,
                                             shared_I);
            GemvLaunch Ls = L;
            Ls.expert.routed_tasks = 0;
            Ls.expert.routed_blocks = 1;
            Ls.expert.shared_task = 1;
            const int per_block = gemv_rows_per_block(plan, dual);
            const dim3 grid((shared_O + per_block - 1) / per_block,
                            (max_rows + plan.b - 1) / plan.b);
            if (!dispatch_gemv(f.shared_fmt, Ls, 1, plan, grid, stream)) return kErrArgs;
        }
    }
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// y[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * w (moonlight_kernels.metal:23-41).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *x, const float *w, float *y,
                                                      int width, float eps, long in_stride,
                                                      long out_stride) {
    __shared__ float part[4];
    const float *src = x + (long)blockIdx.x * in_stride;
    float *dst = y + (long)blockIdx.x * out_stride;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < width; i += blockDim.x) ss += src[i] * src[i];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = (part[0] + part[1]) + (part[2] + part[3]);
    const float inv = 1.0f / sqrtf(total / (float)width + eps);
    for (int i = threadIdx.x; i < width; i += blockDim.x) dst[i] = src[i] * inv * w[i];
}

int rmsnorm_rows(const float *x, const float *w, float *y, int rows, int width, float eps,
                 long in_stride, long out_stride, hipStream_t stream) {
    if (!x || !w || !y || rows <= 0 || width <= 0) return kErrArgs;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, stream, x, w, y, width, eps,
                       in_stride, out_stride);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// out[r, :] = table[ids[r], :] (moonlight_kernels.metal:10-21).
__global__ __launch_bounds__(256) void embed_kernel(const float *table, const int *ids, float *out,
                                                    int width, int vocab, int *clear_flag) {
    const int r = blockIdx.x;
    if (clear_flag && r == 0 && threadIdx.x == 0) *clear_flag = 0;
    int id = ids[r];
    id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);  // host validated; clamp defensively
    const float *src = table + (long)id * width;
    for (int i = threadIdx.x; i < width; i += blockDim.x) out[(long)r * width + i] = src[i];
}

int embed_rows(const float *table, const int *ids, float *out, int rows, int width, int vocab,
               int *clear_flag, hipStream_t stream) {
    if (!table || !ids || !out || rows <= 0 || width <= 0) return kErrArgs;
    hipLaunchKernelGGL(embed_kernel, dim3(rows), dim3(256), 0, stream, table, ids, out, width,
                       vocab, clear_flag);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// out = a + b elementwise (moonlight_kernels.metal:563-569).
__global__ __launch_bounds__(256) void add_kernel(const float *a, const float *b, float *out,
                                                  long n) {
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (long)gridDim.x * blockDim.x)
        out[i] = a[i] + b[i];
}

int add_vectors(const float *a, const float *b, float *out, long n, hipStream_t stream) {
    if (!a || !b || !out || n <= 0) return kErrArgs;
    long blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(add_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a, b, out, n);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace mlh

// gemv_impl.h -- the bandwidth-bound dequant GEMV core (gfx950, wave64), shared by
// the plain GEMV launches (gemv_*.hip) and the grouped MoE expert launches.
//
// Semantics follow moonlight_matmul_f32 / _q8_reduction / _q4
// (moonlight_kernels.metal:43-130): y[b,o] = (sum_i x[b,i] * q[o,i]) * s[o] with
// fp32 accumulation; q8 is int8 row-major [O, I], q4 packs column 2j in the low
// nibble and 2j+1 in the high nibble of byte j, stored as q+8
// (tools/convert_moonlight.py:46-66).
//
// Work decomposition.  A workgroup is 4 wavefronts.  A row of W is cut into
// 16-byte chunks; a group of LPR lanes covers a row, each lane owning the chunks
// li, li+LPR, ... of every row it visits (k-tiles of KT chunks per lane).
//   KS = 1: every wave owns R rows (per lane group);
//   KS = 4: the 4 waves of a workgroup share the same R rows and split the
//           k-tiles between them (wide rows: the 11264-long down projections),
//           partial sums meet in LDS.
// Per k-tile a lane issues its R*KT 16-byte non-temporal weight loads back to
// back, then loads the matching x slice once and reuses it for the R rows.
// int8 / nibbles become floats with v_cvt_f32_ubyteN on byte-biased values (q+128
// resp. the stored nibble) and the bias is removed once per row:
//      sum x*q = sum x*(q+bias) - bias*sum x.
// R*B partial sums are reduced over the lane group with a transposed butterfly.
// Prologue: optional RMSNorm of x (moonlight_kernels.metal:23-41).  Epilogues:
// plain, residual add, and SwiGLU of a gate/up pair (moonlight_kernels.metal:533-541).
#pragma once

#include "mlh_device.h"
#include "mlh_host.h"

namespace mlh {

template <int FMT> struct FmtTraits;
template <> struct FmtTraits<kF32> { static constexpr int kElemsPerChunk = 4; };
template <> struct FmtTraits<kQ8> { static constexpr int kElemsPerChunk = 16; };
template <> struct FmtTraits<kQ4> { static constexpr int kElemsPerChunk = 32; };

template <int FMT>
__device__ __forceinline__ float chunk_dot(u32x4 w, const float *x, float acc) {
    if constexpr (FMT == kF32) {
        acc = fmaf(__uint_as_float(w.x), x[0], acc);
        acc = fmaf(__uint_as_float(w.y), x[1], acc);
        acc = fmaf(__uint_as_float(w.z), x[2], acc);
        acc = fmaf(__uint_as_float(w.w), x[3], acc);
    } else if constexpr (FMT == kQ8) {
        unsigned int d[4] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u, w.z ^ 0x80808080u,
                             w.w ^ 0x80808080u};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc = fmaf((float)(d[j] & 0xFFu), x[4 * j + 0], acc);
            acc = fmaf((float)((d[j] >> 8) & 0xFFu), x[4 * j + 1], acc);
            acc = fmaf((float)((d[j] >> 16) & 0xFFu), x[4 * j + 2], acc);
            acc = fmaf((float)(d[j] >> 24), x[4 * j + 3], acc);
        }
    } else {
        unsigned int d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            unsigned int lo = d[j] & 0x0F0F0F0Fu;
            unsigned int hi = (d[j] >> 4) & 0x0F0F0F0Fu;
            const float *xs = x + 8 * j;
            acc = fmaf((float)(lo & 0xFFu), xs[0], acc);
            acc = fmaf((float)(hi & 0xFFu), xs[1], acc);
            acc = fmaf((float)((lo >> 8) & 0xFFu), xs[2], acc);
            acc = fmaf((float)((hi >> 8) & 0xFFu), xs[3], acc);
            acc = fmaf((float)((lo >> 16) & 0xFFu), xs[4], acc);
            acc = fmaf((float)((hi >> 16) & 0xFFu), xs[5], acc);
            acc = fmaf((float)(lo >> 24), xs[6], acc);
            acc = fmaf((float)(hi >> 24), xs[7], acc);
        }
    }
    return acc;
}

template <int FMT> __device__ __forceinline__ constexpr float byte_bias() {
    return FMT == kQ8 ? 128.0f : (FMT == kQ4 ? 8.0f : 0.0f);
}

__host__ __device__ constexpr int row_bytes_of(int fmt, int width) {
    return fmt == kF32 ? width * 4 : (fmt == kQ8 ? width : (width + 1) / 2);
}

// One workgroup's job: rows [row_block * rows_per_block, ...) of W for up to B
// token rows addressed through row pointers (gathered x, scattered y).
template <int B>
struct GemvJob {
    const uint8_t *w = nullptr;
    const float *s = nullptr;
    const uint8_t *w2 = nullptr;  // up projection (SwiGLU epilogue)
    const float *s2 = nullptr;
    int O = 0, I = 0;
    int rows = 0;  // valid token rows (<= B)
    const float *x[B];
    float *y[B];
    const float *resid[B];
    const float *norm_w = nullptr;
    float eps = 0.0f;
    int epilogue = kEpiPlain;
    int row_block = 0;
};

// Output rows covered by one workgroup.
template <int LPR, int R, int KS>
__host__ __device__ constexpr int rows_per_block(bool dual) {
    return (dual ? R / 2 : R) * (64 / LPR) * (KS == 1 ? 4 : 1);
}

template <int FMT, int B, int KT, int LPR, int R, int KS>
__device__ __forceinline__ void gemv_block(const GemvJob<B> job) {
    constexpr int EPC = FmtTraits<FMT>::kElemsPerChunk;
    constexpr int GPW = kWave / LPR;
    constexpr int NV = R * B;
    static_assert(NV <= LPR, "partial sums exceed the lane group");
    static_assert(KS == 1 || LPR == kWave, "k-split needs whole-wave row groups");
    __shared__ float red[4][NV];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int group = lane / LPR;
    const int li = lane & (LPR - 1);
    const bool dual = job.epilogue == kEpiSiluDual;
    const int out_per_group = dual ? R / 2 : R;
    const int row_wave = KS == 1 ? job.row_block * 4 + wave : job.row_block;
    const int kpart = KS == 1 ? 0 : wave;
    const int out0 = (row_wave * GPW + group) * out_per_group;
    // Only whole waves leave early: the RMSNorm prologue reduces over all 64
    // lanes, so lane groups past the last row stay (their loads and stores
    // are masked by row < O).
    if (KS > 1 ? (job.row_block * out_per_group >= job.O)
               : (row_wave * GPW * out_per_group >= job.O))
        return;

    const int row_bytes = row_bytes_of(FMT, job.I);
    const int nc = row_bytes / 16;

    // RMSNorm prologue: full-row sum of squares per token row (x is small and
    // shared by every wave, so it comes from L1/L2).
    float inv_rms[B];
#pragma unroll
    for (int b = 0; b < B; ++b) inv_rms[b] = 1.0f;
    if (job.norm_w) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float ss = 0.0f;
            if (b < job.rows) {
                // loads in batches of 8 issued before their use: a load-use
                // chain per iteration would serialise the L2 latency
                for (int i0 = lane * 4; i0 < job.I; i0 += kWave * 4 * 8) {
                    f32x4 v[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int i = i0 + kWave * 4 * u;
                        v[u] = i < job.I ? load_f4(job.x[b] + i) : f32x4{0.f, 0.f, 0.f, 0.f};
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        ss += v[u].x * v[u].x + v[u].y * v[u].y + v[u].z * v[u].z +
                              v[u].w * v[u].w;
                }
            }
            ss = wave_sum(ss);
            inv_rms[b] = 1.0f / sqrtf(ss / (float)job.I + job.eps);
        }
    }

    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = 0.0f;
    float sumx[B];
#pragma unroll
    for (int b = 0; b < B; ++b) sumx[b] = 0.0f;

    for (int kt0 = kpart * KT * LPR; kt0 < nc; kt0 += KS * KT * LPR) {
        u32x4 wv[R][KT];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int row;
            const uint8_t *base;
            if (dual) {
                row = out0 + (r < R / 2 ? r : r - R / 2);
                base = r < R / 2 ? job.w : job.w2;
            } else {
                row = out0 + r;
                base = job.w;
            }
#pragma unroll
            for (int k = 0; k < KT; ++k) {
                const int c = kt0 + li + LPR * k;
                wv[r][k] = (row < job.O && c < nc)
                               ? load_stream16(base + (long)row * row_bytes + c * 16)
                               : u32x4{0u, 0u, 0u, 0u};
            }
        }
        float xr[B][KT][EPC];
#pragma unroll
        for (int k = 0; k < KT; ++k) {
            const int c = kt0 + li + LPR * k;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const bool ok = c < nc && b < job.rows;
#pragma unroll
                for (int e = 0; e < EPC; e += 4) {
                    f32x4 v = ok ? load_f4(job.x[b] + c * EPC + e) : f32x4{0.f, 0.f, 0.f, 0.f};
                    if (job.norm_w && ok) {
                        f32x4 n = load_f4(job.norm_w + c * EPC + e);
                        v.x = v.x * inv_rms[b] * n.x;
                        v.y = v.y * inv_rms[b] * n.y;
                        v.z = v.z * inv_rms[b] * n.z;
                        v.w = v.w * inv_rms[b] * n.w;
                    }
                    xr[b][k][e + 0] = v.x;
                    xr[b][k][e + 1] = v.y;
                    xr[b][k][e + 2] = v.z;
                    xr[b][k][e + 3] = v.w;
                    sumx[b] += (v.x + v.y) + (v.z + v.w);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int k = 0; k < KT; ++k)
#pragma unroll
                for (int b = 0; b < B; ++b)
                    acc[r * B + b] = chunk_dot<FMT>(wv[r][k], xr[b][k], acc[r * B + b]);
    }

    if constexpr (FMT != kF32) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int b = 0; b < B; ++b) acc[r * B + b] -= byte_bias<FMT>() * sumx[b];
    }

    butterfly_reduce<NV, LPR>(acc, lane);
    const int vi = butterfly_index<NV, LPR>(lane);
    const bool writer = butterfly_writer<NV, LPR>(lane);
    float value = acc[0];
    if constexpr (KS > 1) {
        if (writer) red[wave][vi] = value;
        __syncthreads();
        value = (red[0][vi] + red[1][vi]) + (red[2][vi] + red[3][vi]);
        __syncthreads();  // `red` may be reused by the caller's next job
        if (wave != 0) return;
    }
    const int r = vi / B, b = vi % B;
    // select the row pointers with a compare chain: indexing the pointer
    // arrays with the lane-dependent b would spill them to scratch
    float *yb = job.y[0];
    const float *rb = job.resid[0];
#pragma unroll
    for (int i = 1; i < B; ++i) {
        if (b == i) {
            yb = job.y[i];
            rb = job.resid[i];
        }
    }
    if (dual) {
        // the up-projection partner of value index vi is vi + NV/2, held by the
        // lane across the first butterfly offset
        const float partner = __shfl_xor(value, LPR / 2, kWave);
        const int row = out0 + r;
        if (writer && r < R / 2 && row < job.O && b < job.rows) {
            const float g = FMT == kF32 ? value : value * job.s[row];
            const float u = FMT == kF32 ? partner : partner * job.s2[row];
            yb[row] = silu(g) * u;
        }
        return;
    }
    const int row = out0 + r;
    if (writer && row < job.O && b < job.rows) {
        float out = FMT == kF32 ? value : value * job.s[row];
        if (job.epilogue == kEpiResidual) out = rb[row] + out;
        yb[row] = out;
    }
}

// Grouped expert launches (MoE): blockIdx.y selects a task -- one active routed
// expert (in first-appearance order) or, last, the fused shared expert -- and
// the workgroup loops over that task's token rows in groups of B.  Token rows are
// gathered / scattered through the device route tables, so no gather or scatter
// pass exists (moonlight_metal.m:577-638 issues gather_rows / scatter_expert per
// expert instead).
struct ExpertWeights {
    const uint8_t *gate, *up, *down;
    const float *gate_s, *up_s, *down_s;
};

struct ExpertGemvParams {
    int stage = 0;  // 0: gate/up + SwiGLU, 1: down
    const ExpertWeights *experts = nullptr;  // device table [E]
    const int *n_unique = nullptr;           // route tables (device)
    const int *unique = nullptr;
    const int *counts = nullptr;
    const int *offsets = nullptr;
    const int *rows = nullptr;  // token row of each compact list entry
    int routed_tasks = 0;       // grid.y slots for routed experts
    int shared_task = 0;        // 1: grid.y slot routed_tasks is the shared expert
    const uint8_t *sh_w = nullptr, *sh_w2 = nullptr;
    const float *sh_s = nullptr, *sh_s2 = nullptr;
    int shared_width = 0;  // fused shared FFN width (2 x moe_intermediate_size)
    int shared_rows = 0;   // token rows of the batch
    int hidden = 0, inter = 0;
    const float *x = nullptr;  // stage 0: residual stream [rows, hidden]; 1: expert hidden
    float *y = nullptr;        // stage 0: expert hidden [list, inter]; 1: expert out [list, hidden]
    const float *sh_x = nullptr;  // stage 1: shared hidden [rows, shared_width]
    float *sh_y = nullptr;        // stage 0: shared hidden; 1: shared out [rows, hidden]
    const float *norm_w = nullptr;  // stage 0: post-attention RMSNorm weight
    float eps = 0.0f;
};

struct GemvLaunch {
    GemvParams plain;
    ExpertGemvParams expert;
};

template <int MODE, int FMT, int B, int KT, int LPR, int R, int KS>
__global__ __launch_bounds__(256) void gemv_kernel(GemvLaunch L) {
    GemvJob<B> job;
    job.row_block = blockIdx.x;
    if constexpr (MODE == 0) {
        const GemvParams &p = L.plain;
        job.w = p.w;
        job.s = p.s;
        job.w2 = p.w2;
        job.s2 = p.s2;
        job.O = p.O;
        job.I = p.I;
        // blockIdx.y selects a slice of B token rows
        const int row0 = blockIdx.y * B;
        job.rows = p.rows - row0 < B ? p.rows - row0 : B;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const long r = row0 + (b < job.rows ? b : 0);
            job.x[b] = p.x + r * p.x_stride;
            job.y[b] = p.y + r * p.y_stride;
            job.resid[b] = p.resid ? p.resid + r * p.resid_stride : nullptr;
        }
        job.norm_w = p.norm_w;
        job.eps = p.eps;
        job.epilogue = p.epilogue;
        gemv_block<FMT, B, KT, LPR, R, KS>(job);
    } else {
        const ExpertGemvParams &p = L.expert;
        const int task = blockIdx.y;
        const bool shared = p.shared_task && task == p.routed_tasks;
        int n, off = 0;
        const int *list = nullptr;
        if (shared) {
            n = p.shared_rows;
            job.w = p.sh_w;  // stage 0: shared gate (sh_w2 = up); stage 1: shared down
            job.s = p.sh_s;
            job.w2 = p.sh_w2;
            job.s2 = p.sh_s2;
            job.O = p.stage == 0 ? p.shared_width : p.hidden;
            job.I = p.stage == 0 ? p.hidden : p.shared_width;
        } else {
            if (task >= *p.n_unique) return;
            const int e = p.unique[task];
            n = p.counts[e];
            off = p.offsets[e];
            list = p.rows + off;
            const ExpertWeights ew = p.experts[e];
            job.w = p.stage == 0 ? ew.gate : ew.down;
            job.s = p.stage == 0 ? ew.gate_s : ew.down_s;
            job.w2 = ew.up;
            job.s2 = ew.up_s;
            job.O = p.stage == 0 ? p.inter : p.hidden;
            job.I = p.stage == 0 ? p.hidden : p.inter;
        }
        job.norm_w = p.stage == 0 ? p.norm_w : nullptr;
        job.eps = p.eps;
        job.epilogue = p.stage == 0 ? kEpiSiluDual : kEpiPlain;
        for (int g0 = 0; g0 < n; g0 += B) {
            job.rows = n - g0 < B ? n - g0 : B;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const int j = g0 + (b < job.rows ? b : 0);  // list entry
                const int token = shared ? j : list[j];
                if (p.stage == 0) {
                    job.x[b] = p.x + (long)token * p.hidden;
                    job.y[b] = shared ? p.sh_y + (long)j * p.shared_width
                                      : p.y + (long)(off + j) * p.inter;
                } else {
                    job.x[b] = shared ? p.sh_x + (long)j * p.shared_width
                                      : p.x + (long)(off + j) * p.inter;
                    job.y[b] = shared ? p.sh_y + (long)j * p.hidden
                                      : p.y + (long)(off + j) * p.hidden;
                }
                job.resid[b] = nullptr;
            }
            gemv_block<FMT, B, KT, LPR, R, KS>(job);
        }
    }
}

// Launch geometry chosen by the host (see gemv.hip, plan_gemv).
struct GemvPlan {
    int b = 1, kt = 1, lpr = 64, r = 4, ks = 1;
};

// MODE 0 grids cover the plain matrix; MODE 1 callers pass their own grid.
template <int MODE, int FMT, int B, int KT, int LPR, int R, int KS>
static void launch_gemv(const GemvLaunch &L, dim3 grid, hipStream_t stream) {
    if constexpr (MODE == 0) {
        const int per_block = rows_per_block<LPR, R, KS>(L.plain.epilogue == kEpiSiluDual);
        grid = dim3((unsigned)((L.plain.O + per_block - 1) / per_block),
                    (unsigned)((L.plain.rows + B - 1) / B));
    }
    hipLaunchKernelGGL((gemv_kernel<MODE, FMT, B, KT, LPR, R, KS>), grid, dim3(256), 0, stream, L);
}

template <int MODE, int FMT, int B>
bool dispatch_gemv_b(const GemvLaunch &L, const GemvPlan &plan, dim3 grid, hipStream_t stream) {
    if (plan.lpr < 64) {
        constexpr int RS8 = 8 / B > 1 ? 8 / B : 2;
        constexpr int RS16 = 16 / B < 8 ? 16 / B : 8;
        constexpr int RS32 = 32 / B < 8 ? 32 / B : 8;
        switch (plan.lpr) {
        case 8: launch_gemv<MODE, FMT, B, 1, 8, RS8, 1>(L, grid, stream); return true;
        case 16: launch_gemv<MODE, FMT, B, 1, 16, RS16, 1>(L, grid, stream); return true;
        case 32: launch_gemv<MODE, FMT, B, 1, 32, RS32, 1>(L, grid, stream); return true;
        }
        return false;
    }
#define MLH_GEMV_CASE(KT_, R_, KS_)                                                      \
    if (plan.kt == KT_ && plan.r == R_ && plan.ks == KS_) {                              \
        if constexpr (R_ * B <= 16 && R_ * KT_ <= 16) {                                  \
            launch_gemv<MODE, FMT, B, KT_, 64, R_, KS_>(L, grid, stream);                \
            return true;                                                                 \
        }                                                                                \
    }
#define MLH_GEMV_KT(KT_)                                                                 \
    MLH_GEMV_CASE(KT_, 1, 1) MLH_GEMV_CASE(KT_, 2, 1) MLH_GEMV_CASE(KT_, 4, 1)          \
    MLH_GEMV_CASE(KT_, 8, 1) MLH_GEMV_CASE(KT_, 1, 4) MLH_GEMV_CASE(KT_, 2, 4)          \
    MLH_GEMV_CASE(KT_, 4, 4) MLH_GEMV_CASE(KT_, 8, 4)
    MLH_GEMV_KT(1)
    if constexpr (FMT != kQ4) { MLH_GEMV_KT(2) }
    if constexpr (FMT == kF32) { MLH_GEMV_KT(4) }
#undef MLH_GEMV_KT
#undef MLH_GEMV_CASE
    return false;
}

template <int FMT>
bool dispatch_gemv_fmt(const GemvLaunch &L, int mode, const GemvPlan &plan, dim3 grid,
                       hipStream_t stream) {
    if (mode == 0) {
        switch (plan.b) {
        case 1: return dispatch_gemv_b<0, FMT, 1>(L, plan, grid, stream);
        case 2: return dispatch_gemv_b<0, FMT, 2>(L, plan, grid, stream);
        case 4: return dispatch_gemv_b<0, FMT, 4>(L, plan, grid, stream);
        }
        return false;
    }
    if constexpr (FMT != kF32) {
        switch (plan.b) {
        case 1: return dispatch_gemv_b<1, FMT, 1>(L, plan, grid, stream);
        case 2: return dispatch_gemv_b<1, FMT, 2>(L, plan, grid, stream);
        case 4: return dispatch_gemv_b<1, FMT, 4>(L, plan, grid, stream);
        }
    }
    return false;
}

// Per-format entry points (gemv_f32.hip / gemv_q8.hip / gemv_q4.hip).
bool dispatch_gemv_f32(const GemvLaunch &L, int mode, const GemvPlan &plan, dim3 grid,
                       hipStream_t stream);
bool dispatch_gemv_q8(const GemvLaunch &L, int mode, const GemvPlan &plan, dim3 grid,
                      hipStream_t stream);
bool dispatch_gemv_q4(const GemvLaunch &L, int mode, const GemvPlan &plan, dim3 grid,
                      hipStream_t stream);
inline bool dispatch_gemv(int fmt, const GemvLaunch &L, int mode, const GemvPlan &plan,
                          dim3 grid, hipStream_t stream) {
    if (fmt == kF32) return dispatch_gemv_f32(L, mode, plan, grid, stream);
    if (fmt == kQ8) return dispatch_gemv_q8(L, mode, plan, grid, stream);
    return dispatch_gemv_q4(L, mode, plan, grid, stream);
}

}  // namespace mlh

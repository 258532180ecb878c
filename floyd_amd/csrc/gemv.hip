// gemv.hip -- launch planning for the dequant GEMV (kernel core in gemv_impl.h)
// and the generic fallback kernel for shapes the vector core does not take.
#include <cstdio>
#include <cstdlib>

#include <string>

#include "gemv_impl.h"
#include "moe.h"

namespace mlh {

// Generic fallback for shapes the vector kernel does not take (row bytes not
// a multiple of 16, unaligned pointers, odd q4 widths): one wave per output,
// byte loads, same arithmetic.
__global__ __launch_bounds__(64) void gemv_generic_kernel(GemvParams p, int fmt) {
    const int o = blockIdx.x;
    const int b = blockIdx.y;
    const int lane = threadIdx.x;
    const bool dual = p.epilogue == kEpiSiluDual;
    const float *x = p.x + (long)b * p.x_stride;
    float inv = 1.0f;
    if (p.norm_w) {
        float ss = 0.0f;
        for (int i = lane; i < p.I; i += kWave) ss += x[i] * x[i];
        ss = wave_sum(ss);
        inv = 1.0f / sqrtf(ss / (float)p.I + p.eps);
    }
    float sums[2] = {0.0f, 0.0f};
    for (int m = 0; m < (dual ? 2 : 1); ++m) {
        const uint8_t *w = m ? p.w2 : p.w;
        float sum = 0.0f;
        for (int i = lane; i < p.I; i += kWave) {
            float xv = p.norm_w ? x[i] * inv * p.norm_w[i] : x[i];
            float wvv;
            if (fmt == kF32) {
                wvv = reinterpret_cast<const float *>(w)[(long)o * p.I + i];
            } else if (fmt == kQ8) {
                wvv = (float)reinterpret_cast<const int8_t *>(w)[(long)o * p.I + i];
            } else {
                uint8_t packed = w[(long)o * ((p.I + 1) / 2) + i / 2];
                wvv = (float)((i & 1) ? (packed >> 4) - 8 : (packed & 15) - 8);
            }
            sum = fmaf(xv, wvv, sum);
        }
        sums[m] = wave_sum(sum);
    }
    if (lane != 0) return;
    if (dual) {
        float g = fmt == kF32 ? sums[0] : sums[0] * p.s[o];
        float u = fmt == kF32 ? sums[1] : sums[1] * p.s2[o];
        p.y[(long)b * p.y_stride + o] = silu(g) * u;
        return;
    }
    float out = fmt == kF32 ? sums[0] : sums[0] * p.s[o];
    if (p.epilogue == kEpiResidual) out = p.resid[(long)b * p.resid_stride + o] + out;
    p.y[(long)b * p.y_stride + o] = out;
}

// ---------------------------------------------------------------------------
// pre-split limb rows
// ---------------------------------------------------------------------------

template <int FMT>
__device__ void limb_row(const LimbRowsParams &p, int r) {
    __shared__ float ss_red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *x = p.x + (long)r * p.x_stride;
    const int nc = row_bytes_of(FMT, p.I) / 16;
    float inv_rms = 1.0f;
    if (p.norm_w) {
        float ss = 0.0f;
        for (int e0 = tid * 8; e0 < p.I; e0 += kLimbPassElems) {
            const f32x4 a = load_f4(x + e0), b = load_f4(x + e0 + 4);
            ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w + b.x * b.x + b.y * b.y +
                  b.z * b.z + b.w * b.w;
        }
        ss = wave_sum(ss);
        if (lane == 0) ss_red[wave] = ss;
        __syncthreads();
        inv_rms = 1.0f / sqrtf(((ss_red[0] + ss_red[1]) + (ss_red[2] + ss_red[3])) / (float)p.I +
                               p.eps);
    }
    unsigned char *out = p.out + (long)r * p.out_stride;
    // every thread of a chunk group takes part in the shuffles of
    // limb_quantise, so the loop bound is the workgroup-uniform pass count
    const int npass = (p.I + kLimbPassElems - 1) / kLimbPassElems;
    for (int j = 0; j < npass; ++j) {
        const int e0 = tid * 8 + j * kLimbPassElems;
        const bool in = e0 < p.I;
        const int ec = in ? e0 : 0;
        const f32x4 a = load_f4(x + ec), b = load_f4(x + ec + 4);
        float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        if (p.norm_w) {
            const f32x4 na = load_f4(p.norm_w + ec), nb = load_f4(p.norm_w + ec + 4);
            const float n[8] = {na.x, na.y, na.z, na.w, nb.x, nb.y, nb.z, nb.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = v[i] * inv_rms * n[i];
        }
        limb_quantise<FMT>(v, in, e0, out, p.I, nc);
    }
}

__global__ __launch_bounds__(256) void limb_rows_kernel(LimbRowsParams a, LimbRowsParams b) {
    const bool first = (int)blockIdx.x < a.rows;
    const LimbRowsParams &p = first ? a : b;
    const int r = first ? (int)blockIdx.x : (int)blockIdx.x - a.rows;
    if (p.fmt == kQ4)
        limb_row<kQ4>(p, r);
    else
        limb_row<kQ8>(p, r);
}

int limb_quantise_rows(const LimbRowsParams &a, const LimbRowsParams &b, hipStream_t stream) {
    for (const LimbRowsParams *p : {&a, &b}) {
        if (p->rows == 0) continue;
        if (p->rows < 0 || !p->x || !p->out || (p->fmt != kQ8 && p->fmt != kQ4) || p->I <= 0 ||
            p->I % 16 || (p->fmt == kQ4 && p->I % 32) || p->x_stride % 4 ||
            p->out_stride < limb_row_lds(p->fmt, p->I) || p->out_stride % 16)
            return kErrArgs;
    }
    if (a.rows + b.rows == 0) return kOk;
    hipLaunchKernelGGL(limb_rows_kernel, dim3(a.rows + b.rows), dim3(256), 0, stream, a, b);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// ---------------------------------------------------------------------------
// planning
// ---------------------------------------------------------------------------

// Waves the planner tries to keep in flight: with ~8 waves per CU the HBM
// latency (~1-2 us under load) is hidden without relying on deep per-wave
// queues.
static constexpr long kTargetWaves = 2048;

// Plans measured best on MI355X for the Moonlight decode shapes (batch 1):
// sweeps over kt x r x ks of back-to-back launches, 400+ MB weight rotation.
struct PlanEntry {
    int fmt, O, I, dual, kt, r, ks, waves;
};
static const PlanEntry kMeasuredPlans[] = {
    {kQ4, 11264, 2048, 0, 1, 4, 1, 4}, {kQ8, 11264, 2048, 0, 1, 4, 1, 4},
    {kQ4, 2048, 11264, 0, 2, 1, 1, 8}, {kQ8, 2048, 11264, 0, 2, 1, 1, 8},
    {kQ8, 3072, 2048, 0, 1, 2, 1, 8},  {kQ8, 2048, 2048, 0, 2, 1, 1, 8},
    {kQ8, 2048, 1408, 0, 2, 1, 1, 8},  {kQ8, 2048, 2816, 0, 2, 1, 1, 8},
    {kQ8, 576, 2048, 0, 2, 1, 1, 4},   {kF32, 64, 2048, 0, 4, 1, 4, 4},
    {kQ4, 2048, 1408, 0, 1, 2, 1, 4},  {kQ8, 1536, 2048, 0, 2, 1, 1, 8},
    {kQ8, 3072, 1536, 0, 2, 1, 1, 8},
};

GemvPlan plan_gemv(int fmt, int O, int I, int rows, bool dual) {
    GemvPlan plan;
    plan.b = rows <= 1 ? 1 : rows <= 2 ? 2 : 4;
    const int nc = row_bytes_of(fmt, I) / 16;
    if (nc <= 32) {
        // rows per lane group fixed by dispatch_gemv_b for narrow rows
        plan.lpr = nc <= 8 ? 8 : nc <= 16 ? 16 : 32;
        plan.kt = 1;
        plan.ks = 1;
        if (plan.lpr == 8) plan.r = 8 / plan.b > 1 ? 8 / plan.b : 2;
        else plan.r = plan.lpr / plan.b < 8 ? plan.lpr / plan.b : 8;
        return plan;
    }
    plan.lpr = 64;
    if (plan.b == 1) {
        for (const PlanEntry &e : kMeasuredPlans) {
            if (e.fmt == fmt && e.O == O && e.I == I && e.dual == (int)dual) {
                plan.kt = e.kt;
                plan.r = e.r;
                plan.ks = e.ks;
                plan.waves = e.waves;
                return plan;
            }
        }
    }
    // Fallback heuristic from the same sweeps.  Quantised formats: a lane
    // covers its chunks of the row in one tile (KT = 1 or 2 for rows of up to
    // 128 chunks), wider rows split k over the workgroup's 4 waves; rows per
    // wave sized for ~700 workgroups.  f32: up to 2 chunks per lane per tile.
    const int rmin = dual ? 2 : 1;
    if (fmt != kF32) {
        if (nc <= 128) {
            plan.ks = 1;
            plan.kt = nc > 64 ? 2 : 1;
        } else {
            plan.ks = 4;
            plan.kt = nc > 256 ? 2 : 1;
        }
        const long per_wave_target = (long)O * (dual ? 2 : 1) / (plan.ks == 4 ? 700 : 2800);
        int r = rmin;
        while (r < 8 && r * 2 <= per_wave_target && r * 2 * plan.b <= 16 && r * 2 * plan.kt <= 16)
            r *= 2;
        plan.r = r;
        return plan;
    }
    plan.kt = nc > 64 ? 2 : 1;
    const int tiles = (nc + 64 * plan.kt - 1) / (64 * plan.kt);
    const long out_rows_total = (long)O * (dual ? 2 : 1);
    // k split only pays when every wave of the workgroup gets a k-tile, or for
    // short plain matrices (few rows: more waves); not for the gate/up pairs
    plan.ks = (tiles >= 4 || (tiles >= 2 && out_rows_total <= 4096 && !dual)) ? 4 : 1;
    int chosen = 0;
    for (int r = 8; r >= rmin; r >>= 1) {
        if (r * plan.b > 16 || r * plan.kt > 16) continue;
        const long out_rows = dual ? r / 2 : r;
        const long waves = (O + out_rows - 1) / out_rows * (plan.ks == 4 ? 4 : 1);
        chosen = r;
        if (waves >= kTargetWaves) break;
    }
    plan.r = chosen ? chosen : rmin;
    return plan;
}

// Grouped expert launches: same core, the work spread over `tasks` matrices.
// Quantised formats: one tile covers a lane's chunks of the widest row of the
// launch (I = max_I, KT up to 3 columns of 64 chunks), 8 rows per wave when
// the registers allow (the x prologue of every workgroup is amortised over
// more rows; measured best for the Moonlight expert shapes).
GemvPlan plan_expert_gemv(int fmt, int O, int I, int rows, bool dual, int tasks, int max_I) {
    GemvPlan plan = plan_gemv(fmt, O, max_I, rows, dual);
    plan.waves = 4;  // grouped launches use 4-wave workgroups
    if (plan.lpr < 64) return plan;
    if (fmt != kF32) {
        {
            const int nc = row_bytes_of(fmt, max_I) / 16;
            if (nc <= 192) {
                plan.ks = 1;
                plan.kt = (nc + 63) / 64;
            } else {
                plan.ks = 4;
                plan.kt = (nc + 255) / 256 < 3 ? (nc + 255) / 256 : 3;
            }
            plan.r = 8;
            while (plan.r > 1 && (plan.r * plan.kt > 16 || plan.r * plan.b > 16)) plan.r /= 2;
        }
        if (plan.r * plan.b > 16) plan.r = 16 / plan.b;
        if (plan.r * plan.kt > 16) plan.r = 16 / plan.kt;
        if (dual && plan.r < 2) plan.r = 2;
        (void)tasks;
        (void)I;
        return plan;
    }
    if (tasks <= 1) return plan;
    const int rmin = dual ? 2 : 1;
    for (int r = plan.r; r <= 8; r <<= 1) {
        if (r * plan.b > 16 || r * plan.kt > 16) break;
        const long out_rows = dual ? r / 2 : r;
        const long waves = (O + out_rows - 1) / out_rows * (plan.ks == 4 ? 4 : 1) * tasks;
        plan.r = r;
        if (waves <= 4 * kTargetWaves) break;
    }
    if (plan.r < rmin) plan.r = rmin;
    return plan;
}

int gemv_rows_per_block(const GemvPlan &plan, bool dual) {
    const int out = dual ? plan.r / 2 : plan.r;
    return out * (64 / plan.lpr) * (plan.ks == 1 ? plan.waves : 1);
}

bool gemv_mfma(const GemvParams &p, hipStream_t stream, std::string *name = nullptr);  // gemv_mfma.hip

// Template name of the kernel gemv() launches for this shape (aligned
// operands, no pre-split x).
std::string gemv_kernel_name(int fmt, int O, int I, int rows, bool dual) {
    GemvParams q;
    q.fmt = fmt;
    q.O = O;
    q.I = I;
    q.rows = rows;
    q.epilogue = dual ? kEpiSiluDual : q.epilogue;
    std::string mfma;
    if (gemv_mfma(q, nullptr, &mfma)) return mfma;
    const GemvPlan pl = plan_gemv(fmt, O, I, rows < kMaxGemvRows ? rows : kMaxGemvRows, dual);
    char buf[96];
    snprintf(buf, sizeof(buf), "mlh::gemv_kernel<0, %d, %d, %d, %d, %d, %d, %d>", fmt, pl.b,
             pl.kt, pl.lpr, pl.r, pl.ks, pl.waves);
    return buf;
}

static bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15u) == 0; }

int gemv(const GemvParams &p_in, hipStream_t stream) {
    if (!p_in.w || !p_in.x || !p_in.y || p_in.O <= 0 || p_in.I <= 0 || p_in.rows <= 0)
        return kErrArgs;
    if (p_in.fmt != kF32 && !p_in.s) return kErrArgs;
    if (p_in.epilogue == kEpiSiluDual && (!p_in.w2 || (p_in.fmt != kF32 && !p_in.s2)))
        return kErrArgs;
    if (p_in.epilogue == kEpiResidual && !p_in.resid) return kErrArgs;
    // router partials: only the matrix-core kernels write them
    if (p_in.router_parts &&
        (!p_in.router_w || !p_in.router_nw || p_in.router_experts <= 0 ||
         p_in.router_experts > 64 || p_in.O % 4 || ((uintptr_t)p_in.router_w & 15u) ||
         !gemv_router_ok(p_in)))
        return kErrArgs;
    // q8 / q4 with up to 4 token rows: the matrix-core kernel when it takes the shape
    if (gemv_mfma(p_in, stream))
        return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
    if (p_in.router_parts) return kErrArgs;
    const long row_bytes = row_bytes_of(p_in.fmt, p_in.I);
    const bool vector_ok =
        row_bytes % 16 == 0 && (p_in.fmt != kQ4 || p_in.I % 2 == 0) &&
        gemv_lds_bytes_rt(p_in.fmt, 1, p_in.I) <= kMaxGemvLds && aligned16(p_in.w) &&
        (!p_in.w2 || aligned16(p_in.w2)) && aligned16(p_in.x) && p_in.x_stride % 4 == 0 &&
        (!p_in.norm_w || aligned16(p_in.norm_w));
    // token rows beyond 4 run as slices of 4 (register budget) along grid.y
    // of one launch
    bool done = false;
    if (vector_ok) {
        int plan_rows = p_in.rows < kMaxGemvRows ? p_in.rows : kMaxGemvRows;
        if (plan_rows == 3) plan_rows = 4;  // the kernel takes 1, 2 or 4 token rows
        // the quantised x rows of a workgroup must fit its LDS
        while (plan_rows > 1 && gemv_lds_bytes_rt(p_in.fmt, plan_rows, p_in.I) > kMaxGemvLds)
            plan_rows /= 2;
        const GemvPlan plan = plan_gemv(p_in.fmt, p_in.O, p_in.I, plan_rows,
                                        p_in.epilogue == kEpiSiluDual);
        GemvLaunch L;
        L.plain = p_in;
        done = dispatch_gemv(p_in.fmt, L, 0, plan, dim3(1), stream);
    }
    if (!done) {
        hipLaunchKernelGGL(gemv_generic_kernel, dim3(p_in.O, p_in.rows), dim3(64), 0, stream,
                           p_in, p_in.fmt);
    }
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace mlh

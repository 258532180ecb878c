// qgemm.hip -- grouped int8-MFMA GEMM for prefill (see qgemm.h for the
// numerics).  gfx950: v_mfma_i32_32x32x32_i8, wave64.
//
// Workgroup: 4 waves in a 2 x 2 arrangement over a 128 (token rows) x 128
// (weight rows) tile; each wave owns 64 x 64 = 2 x 2 MFMA blocks per limb.
// Pipeline: the next 64-wide k slice is fetched into registers while the
// current one is multiplied out of LDS (double-buffered, one barrier per
// slice).  MFMA operand layout (measured on gfx950): lane l supplies row
// (l % 32) and the 16-byte k chunk (l / 32) of a 32-wide k step, for A rows and
// for B columns alike; result register r of lane l is
// C[(r / 4) * 8 + (l / 32) * 4 + r % 4][l % 32].
#include "qgemm.h"

namespace mlh {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kLdsRow = kQgBK + 16;  // padded LDS row in bytes (conflict-free b128 reads)
constexpr int kQuantMax = 16384;     // |256 * hi + lo| bound

bool qgemm_shape_ok(int fmt, int k) {
    return (fmt == kQ8 || fmt == kQ4) && k > 0 && k % kQgBK == 0;
}

// ---------------------------------------------------------------------------
// activation quantisation: one wave per row
// ---------------------------------------------------------------------------

__device__ __forceinline__ void quant_pair(float v, float inv, int &h, int &l) {
    float q = rintf(v * inv);
    q = fminf(fmaxf(q, -(float)kQuantMax), (float)kQuantMax);
    const int qi = (int)q;
    h = (qi + 128) >> 8;  // floor: lo lands in [-128, 127]
    l = qi - h * 256;
}

__global__ __launch_bounds__(256) void quantize_act_kernel(const float *x, long x_stride, int rows,
                                                           int width, const float *norm_w,
                                                           float eps, int8_t *hi, int8_t *lo,
                                                           float *scale) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + (long)row * x_stride;
    float inv_rms = 1.0f;
    if (norm_w) {
        float ss = 0.0f;
        for (int i = lane * 4; i < width; i += kWave * 4) {
            const f32x4 v = load_f4(xr + i);
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ss = wave_sum(ss);
        inv_rms = 1.0f / sqrtf(ss / (float)width + eps);
    }
    float amax = 0.0f;
    for (int i = lane * 4; i < width; i += kWave * 4) {
        f32x4 v = load_f4(xr + i);
        if (norm_w) {
            const f32x4 n = load_f4(norm_w + i);
            v.x = v.x * inv_rms * n.x;
            v.y = v.y * inv_rms * n.y;
            v.z = v.z * inv_rms * n.z;
            v.w = v.w * inv_rms * n.w;
        }
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    amax = wave_max(amax);
    const float inv = amax > 0.0f ? (float)kQuantMax / amax : 0.0f;
    if (lane == 0) scale[row] = amax / (float)kQuantMax;
    int8_t *hr = hi + (long)row * width;
    int8_t *lr = lo + (long)row * width;
    for (int i = lane * 4; i < width; i += kWave * 4) {
        f32x4 v = load_f4(xr + i);
        if (norm_w) {
            const f32x4 n = load_f4(norm_w + i);
            v.x = v.x * inv_rms * n.x;
            v.y = v.y * inv_rms * n.y;
            v.z = v.z * inv_rms * n.z;
            v.w = v.w * inv_rms * n.w;
        }
        int h0, h1, h2, h3, l0, l1, l2, l3;
        quant_pair(v.x, inv, h0, l0);
        quant_pair(v.y, inv, h1, l1);
        quant_pair(v.z, inv, h2, l2);
        quant_pair(v.w, inv, h3, l3);
        const unsigned hp = (h0 & 0xFF) | ((h1 & 0xFF) << 8) | ((h2 & 0xFF) << 16) |
                            ((unsigned)(h3 & 0xFF) << 24);
        const unsigned lp = (l0 & 0xFF) | ((l1 & 0xFF) << 8) | ((l2 & 0xFF) << 16) |
                            ((unsigned)(l3 & 0xFF) << 24);
        *reinterpret_cast<unsigned *>(hr + i) = hp;
        *reinterpret_cast<unsigned *>(lr + i) = lp;
    }
}

int quantize_activations(const float *x, long x_stride, int rows, int width, const float *norm_w,
                         float eps, int8_t *hi, int8_t *lo, float *scale, hipStream_t stream) {
    if (!x || !hi || !lo || !scale || rows <= 0 || width <= 0 || width % 4 || x_stride % 4)
        return kErrArgs;
    hipLaunchKernelGGL(quantize_act_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, x,
                       x_stride, rows, width, norm_w, eps, hi, lo, scale);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// ---------------------------------------------------------------------------
// GEMM
// ---------------------------------------------------------------------------

// 16 packed nibbles (stored q + 8, column 2j low) -> 8 int8 values q.
__device__ __forceinline__ void unpack_q4_word(unsigned w, unsigned &out0, unsigned &out1) {
    const unsigned lo = w & 0x0F0F0F0Fu;         // even columns
    const unsigned hi = (w >> 4) & 0x0F0F0F0Fu;  // odd columns
    // bytes [lo0, hi0, lo1, hi1] and [lo2, hi2, lo3, hi3]
    const unsigned a = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    const unsigned b = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
    // stored u in [0, 15] -> u - 8 as int8: (u + 0x78) ^ 0x80, no carry between bytes
    out0 = (a + 0x78787878u) ^ 0x80808080u;
    out1 = (b + 0x78787878u) ^ 0x80808080u;
}

__device__ __forceinline__ int find_task(const int *tile_start, int n, int tile) {
    // last t in [0, n) with tile_start[t] <= tile
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tile_start[mid] <= tile) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

template <bool DUAL>
__device__ __forceinline__ int tiles_of(int rows, int n_out) {
    constexpr int outw = DUAL ? kQgBW / 2 : kQgBW;
    return ((rows + kQgBM - 1) / kQgBM) * ((n_out + outw - 1) / outw);
}

template <int FMT, bool DUAL>
__global__ __launch_bounds__(256, 2) void qgemm_kernel(QGemmLaunch L) {
    __shared__ __attribute__((aligned(16))) int8_t lds_a[2][2][kQgBM * kLdsRow];
    __shared__ __attribute__((aligned(16))) int8_t lds_b[2][kQgBW * kLdsRow];
    __shared__ float lds_scale[kQgBM];
    __shared__ int lds_arow[kQgBM];

    // ---- tile -> (task, row tile, column tile), XCD-contiguous order
    GemmTask tk;
    int local;
    {
        int begin = 0, end;
        int n_tasks = 1;
        if (L.tasks) {
            const int nr = *L.n_routed;
            n_tasks = nr + 1;
            end = L.range == 1 ? L.tile_start[nr] : L.tile_start[nr + 1];
            if (L.range == 2) begin = L.tile_start[nr];
        } else {
            end = tiles_of<DUAL>(L.single.rows, L.single.n_out);
        }
        const int total = end - begin;
        const int per = (total + 7) >> 3;
        const int slot = blockIdx.x >> 3;
        if (slot >= per) return;
        const int tile = begin + (blockIdx.x & 7) * per + slot;
        if (tile >= end) return;
        if (L.tasks) {
            const int t = find_task(L.tile_start, n_tasks, tile);
            tk = L.tasks[t];
            local = tile - L.tile_start[t];
        } else {
            tk = L.single;
            local = tile;
        }
    }
    constexpr int outw = DUAL ? kQgBW / 2 : kQgBW;
    const int n_tiles = (tk.n_out + outw - 1) / outw;
    const int m_tiles = (tk.rows + kQgBM - 1) / kQgBM;
    const int per_group = kQgGroup * n_tiles;
    const int grp = local / per_group;
    const int gsize = min(kQgGroup, m_tiles - grp * kQgGroup);
    const int rem = local - grp * per_group;
    const int m0 = (grp * kQgGroup + rem % gsize) * kQgBM;
    const int n0 = (rem / gsize) * outw;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;

    if (tid < kQgBM) {
        const int m = m0 + tid;
        int arow = -1;
        float sc = 0.0f;
        if (m < tk.rows) {
            arow = tk.a_rows ? tk.a_rows[m] : m;
            sc = tk.a_scale[arow];
        }
        lds_arow[tid] = arow;
        lds_scale[tid] = sc;
    }
    __syncthreads();

    // ---- per-thread global sources (fixed over k)
    // A: 4 chunks of 16 bytes: limb = c >> 9, row = (c >> 2) & 127, chunk = c & 3
    const int8_t *a_src[4];
    int a_dst[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int c = tid + 256 * q;
        const int limb = c >> 9, r = (c >> 2) & (kQgBM - 1), kc = c & 3;
        const int arow = lds_arow[r];
        a_src[q] = arow < 0 ? nullptr
                            : (limb ? tk.a_lo : tk.a_hi) + (long)arow * tk.a_stride + kc * 16;
        a_dst[q] = limb * (kQgBM * kLdsRow) + r * kLdsRow + kc * 16;
    }
    // B: LDS row j holds weight row `out` of w (SwiGLU: rows 32..63 of each
    // 64-row half come from the up matrix w2, matching gate rows 0..31)
    constexpr int kBChunks = FMT == kQ8 ? 2 : 1;
    const uint8_t *b_src[kBChunks];
    int b_dst[kBChunks];
    const long w_row_bytes = FMT == kQ8 ? tk.k : tk.k / 2;
    const uint8_t *const w_gate = tk.w;
    const uint8_t *const w_up = tk.w2;
#pragma unroll
    for (int q = 0; q < kBChunks; ++q) {
        const int j = FMT == kQ8 ? (tid + 256 * q) >> 2 : tid >> 1;
        const int out = DUAL ? n0 + (j >> 6) * 32 + (j & 31) : n0 + j;
        const bool up = DUAL && ((j >> 5) & 1);
        const uint8_t *base = up ? w_up : w_gate;
        const int col = FMT == kQ8 ? ((tid + 256 * q) & 3) * 16 : (tid & 1) * 16;
        b_src[q] = out < tk.n_out ? base + (long)out * w_row_bytes + col : nullptr;
        b_dst[q] = j * kLdsRow + (FMT == kQ8 ? col : col * 2);
    }

    u32x4 ra[4], rb[kBChunks];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            ra[q] = a_src[q] ? *reinterpret_cast<const u32x4 *>(a_src[q] + k0)
                             : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int q = 0; q < kBChunks; ++q) {
            const long off = FMT == kQ8 ? k0 : k0 / 2;
            rb[q] = b_src[q] ? *reinterpret_cast<const u32x4 *>(b_src[q] + off)
                             : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto stash = [&](int buf) {
        int8_t *a = &lds_a[buf][0][0];
#pragma unroll
        for (int q = 0; q < 4; ++q) *reinterpret_cast<u32x4 *>(a + a_dst[q]) = ra[q];
        int8_t *b = &lds_b[buf][0];
        if (FMT == kQ8) {
#pragma unroll
            for (int q = 0; q < kBChunks; ++q) *reinterpret_cast<u32x4 *>(b + b_dst[q]) = rb[q];
        } else {
            unsigned v[8];
            unpack_q4_word(rb[0].x, v[0], v[1]);
            unpack_q4_word(rb[0].y, v[2], v[3]);
            unpack_q4_word(rb[0].z, v[4], v[5]);
            unpack_q4_word(rb[0].w, v[6], v[7]);
            *reinterpret_cast<u32x4 *>(b + b_dst[0]) = u32x4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<u32x4 *>(b + b_dst[0] + 16) = u32x4{v[4], v[5], v[6], v[7]};
        }
    };

    i32x16 acc[2][2][2];  // [limb][row block][column block]
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[a][i][f][r] = 0;

    const int nk = tk.k / kQgBK;
    fetch(0);
    stash(0);
    __syncthreads();
    const int arow_l = lane & 31;
    const int kq = (lane >> 5) * 16;
    for (int ks = 0; ks < nk; ++ks) {
        const int cur = ks & 1;
        if (ks + 1 < nk) fetch((ks + 1) * kQgBK);
        const int8_t *ah = &lds_a[cur][0][0];
        const int8_t *al = &lds_a[cur][1][0];
        const int8_t *bb = &lds_b[cur][0];
#pragma unroll
        for (int ksub = 0; ksub < 2; ++ksub) {
            const int koff = ksub * 32 + kq;
            i32x4 fa_h[2], fa_l[2], fb[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = wm * 64 + i * 32 + arow_l;
                fa_h[i] = *reinterpret_cast<const i32x4 *>(ah + row * kLdsRow + koff);
                fa_l[i] = *reinterpret_cast<const i32x4 *>(al + row * kLdsRow + koff);
            }
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                const int row = wn * 64 + f * 32 + arow_l;
                fb[f] = *reinterpret_cast<const i32x4 *>(bb + row * kLdsRow + koff);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int f = 0; f < 2; ++f) {
                    acc[0][i][f] =
                        __builtin_amdgcn_mfma_i32_32x32x32_i8(fa_h[i], fb[f], acc[0][i][f], 0, 0, 0);
                    acc[1][i][f] =
                        __builtin_amdgcn_mfma_i32_32x32x32_i8(fa_l[i], fb[f], acc[1][i][f], 0, 0, 0);
                }
        }
        if (ks + 1 < nk) stash(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int ml = wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            const int m = m0 + ml;
            if (m >= tk.rows) continue;
            const float sx = lds_scale[ml];
            float *yrow = tk.y + (long)m * tk.y_stride;
            if (DUAL) {
                const int n = n0 + wn * 32 + (lane & 31);
                if (n < tk.n_out) {
                    const float g = ((float)acc[0][i][0][r] * 256.0f + (float)acc[1][i][0][r]) *
                                    sx * tk.s[n];
                    const float u = ((float)acc[0][i][1][r] * 256.0f + (float)acc[1][i][1][r]) *
                                    sx * tk.s2[n];
                    yrow[n] = silu(g) * u;
                }
            } else {
#pragma unroll
                for (int f = 0; f < 2; ++f) {
                    const int n = n0 + wn * 64 + f * 32 + (lane & 31);
                    if (n < tk.n_out) {
                        float v = ((float)acc[0][i][f][r] * 256.0f + (float)acc[1][i][f][r]) * sx *
                                  tk.s[n];
                        if (tk.resid) v = tk.resid[(long)m * tk.resid_stride + n] + v;
                        yrow[n] = v;
                    }
                }
            }
        }
    }
}

template <int FMT, bool DUAL>
static void launch_qgemm(const QGemmLaunch &L, int grid, hipStream_t stream) {
    hipLaunchKernelGGL((qgemm_kernel<FMT, DUAL>), dim3((unsigned)grid), dim3(256), 0, stream, L);
}

static int launch_qgemm_fmt(int fmt, bool dual, const QGemmLaunch &L, int tiles_bound,
                            hipStream_t stream) {
    if (tiles_bound <= 0) return kOk;
    const int grid = ((tiles_bound + 7) / 8) * 8;
    if (fmt == kQ8) {
        if (dual) launch_qgemm<kQ8, true>(L, grid, stream);
        else launch_qgemm<kQ8, false>(L, grid, stream);
    } else if (fmt == kQ4) {
        if (dual) launch_qgemm<kQ4, true>(L, grid, stream);
        else launch_qgemm<kQ4, false>(L, grid, stream);
    } else {
        return kErrArgs;
    }
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

static int host_tiles(bool dual, int rows, int n_out) {
    const int outw = dual ? kQgBW / 2 : kQgBW;
    return ((rows + kQgBM - 1) / kQgBM) * ((n_out + outw - 1) / outw);
}

int qgemm_single(int fmt, bool dual, const GemmTask &task, hipStream_t stream) {
    if (!qgemm_shape_ok(fmt, task.k) || task.rows <= 0 || task.n_out <= 0 || !task.w ||
        !task.s || !task.a_hi || !task.a_lo || !task.a_scale || !task.y ||
        (dual && (!task.w2 || !task.s2)) || task.a_stride % 16)
        return kErrArgs;
    QGemmLaunch L;
    L.single = task;
    return launch_qgemm_fmt(fmt, dual, L, host_tiles(dual, task.rows, task.n_out), stream);
}

// ---------------------------------------------------------------------------
// MoE prefill: device-built task tables
// ---------------------------------------------------------------------------

struct MoeScheduleParams {
    MoeGemmParams p;
};

__global__ __launch_bounds__(256) void moe_schedule_kernel(MoeScheduleParams sp) {
    const MoeGemmParams &p = sp.p;
    __shared__ int tiles[2][kQgMaxTasks];
    const int nr = *p.n_unique;
    GemmTask *t0 = p.tasks;
    GemmTask *t1 = p.tasks + kQgMaxTasks;
    for (int u = threadIdx.x; u < nr; u += blockDim.x) {
        const int e = p.unique[u];
        const int cnt = p.counts[e], off = p.offsets[e];
        const ExpertWeights ew = p.expert_table[e];
        GemmTask a;
        a.w = ew.gate;
        a.w2 = ew.up;
        a.s = ew.gate_s;
        a.s2 = ew.up_s;
        a.rows = cnt;
        a.n_out = p.inter;
        a.k = p.hidden;
        a.a_hi = p.xq_hi;
        a.a_lo = p.xq_lo;
        a.a_scale = p.xq_scale;
        a.a_stride = p.hidden;
        a.a_rows = p.list_rows + off;
        a.y = p.expert_hidden + (long)off * p.inter;
        a.y_stride = p.inter;
        t0[u] = a;
        tiles[0][u] = tiles_of<true>(cnt, p.inter);
        GemmTask b;
        b.w = ew.down;
        b.s = ew.down_s;
        b.rows = cnt;
        b.n_out = p.hidden;
        b.k = p.inter;
        b.a_hi = p.hq_hi + (long)off * p.inter;
        b.a_lo = p.hq_lo + (long)off * p.inter;
        b.a_scale = p.hq_scale + off;
        b.a_stride = p.inter;
        b.y = p.expert_out + (long)off * p.hidden;
        b.y_stride = p.hidden;
        t1[u] = b;
        tiles[1][u] = tiles_of<false>(cnt, p.hidden);
    }
    if (threadIdx.x == 0) {
        tiles[0][nr] = 0;
        tiles[1][nr] = 0;
        if (p.has_shared) {
            GemmTask a;
            a.w = p.shared_gate;
            a.w2 = p.shared_up;
            a.s = p.shared_gate_s;
            a.s2 = p.shared_up_s;
            a.rows = p.rows;
            a.n_out = p.shared_width;
            a.k = p.hidden;
            a.a_hi = p.xq_hi;
            a.a_lo = p.xq_lo;
            a.a_scale = p.xq_scale;
            a.a_stride = p.hidden;
            a.y = p.shared_hidden;
            a.y_stride = p.shared_width;
            t0[nr] = a;
            tiles[0][nr] = tiles_of<true>(p.rows, p.shared_width);
            GemmTask b;
            b.w = p.shared_down;
            b.s = p.shared_down_s;
            b.rows = p.rows;
            b.n_out = p.hidden;
            b.k = p.shared_width;
            b.a_hi = p.sq_hi;
            b.a_lo = p.sq_lo;
            b.a_scale = p.sq_scale;
            b.a_stride = p.shared_width;
            b.y = p.shared_out;
            b.y_stride = p.hidden;
            t1[nr] = b;
            tiles[1][nr] = tiles_of<false>(p.rows, p.hidden);
        }
    }
    __syncthreads();
    if (threadIdx.x < 2) {
        const int s = threadIdx.x;
        int *start = p.tile_start + s * (kQgMaxTasks + 1);
        int acc = 0;
        for (int u = 0; u <= nr; ++u) {
            start[u] = acc;
            acc += tiles[s][u];
        }
        start[nr + 1] = acc;
    }
}

int moe_gemm(const MoeGemmParams &p, hipStream_t stream) {
    if (p.rows <= 0 || p.experts <= 0 || p.experts + 1 > kQgMaxTasks || p.top_k <= 0 ||
        !qgemm_shape_ok(p.expert_fmt, p.hidden) || !qgemm_shape_ok(p.expert_fmt, p.inter) ||
        (p.has_shared && (!qgemm_shape_ok(p.shared_fmt, p.hidden) ||
                          !qgemm_shape_ok(p.shared_fmt, p.shared_width))))
        return kErrArgs;
    int st = quantize_activations(p.x, p.hidden, p.rows, p.hidden, p.norm_w, p.eps, p.xq_hi,
                                  p.xq_lo, p.xq_scale, stream);
    if (st) return st;
    MoeScheduleParams sp;
    sp.p = p;
    hipLaunchKernelGGL(moe_schedule_kernel, dim3(1), dim3(256), 0, stream, sp);
    if (hipGetLastError() != hipSuccess) return kErrLaunch;

    const int entries = p.rows * p.top_k;
    const int max_tasks = entries < p.experts ? entries : p.experts;
    const bool same = !p.has_shared || p.shared_fmt == p.expert_fmt;
    for (int stage = 0; stage < 2; ++stage) {
        const bool dual = stage == 0;
        QGemmLaunch L;
        L.tasks = p.tasks + stage * kQgMaxTasks;
        L.tile_start = p.tile_start + stage * (kQgMaxTasks + 1);
        L.n_routed = p.n_unique;
        // upper bounds of the tile counts: sum_e ceil(n_e / BM) <= entries / BM + tasks
        const int routed_mt = entries / kQgBM + max_tasks;
        const int routed_nt = host_tiles(dual, 1, dual ? p.inter : p.hidden);
        const int shared_t =
            p.has_shared ? host_tiles(dual, p.rows, dual ? p.shared_width : p.hidden) : 0;
        if (same) {
            L.range = 0;
            st = launch_qgemm_fmt(p.expert_fmt, dual, L, routed_mt * routed_nt + shared_t, stream);
        } else {
            L.range = 1;
            st = launch_qgemm_fmt(p.expert_fmt, dual, L, routed_mt * routed_nt, stream);
            if (!st) {
                L.range = 2;
                st = launch_qgemm_fmt(p.shared_fmt, dual, L, shared_t, stream);
            }
        }
        if (st) return st;
        if (stage == 0) {
            st = quantize_activations(p.expert_hidden, p.inter, entries, p.inter, nullptr, 0.0f,
                                      p.hq_hi, p.hq_lo, p.hq_scale, stream);
            if (!st && p.has_shared)
                st = quantize_activations(p.shared_hidden, p.shared_width, p.rows,
                                          p.shared_width, nullptr, 0.0f, p.sq_hi, p.sq_lo,
                                          p.sq_scale, stream);
            if (st) return st;
        }
    }
    return kOk;
}

}  // namespace mlh

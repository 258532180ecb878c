// gemv.hip -- bandwidth-bound dequant GEMV for decode (gfx950, wave64).
//
// Semantics follow moonlight_matmul_f32 / _q8_reduction / _q4
// (moonlight_kernels.metal:43-130): y[b,o] = (sum_i x[b,i] * q[o,i]) * s[o]
// with fp32 accumulation; q8 is int8 row-major [O, I], q4 packs column 2j in
// the low nibble and 2j+1 in the high nibble of byte j, stored as q+8
// (tools/convert_moonlight.py:46-66).
//
// Design (one wavefront = R weight rows x B token rows):
//  * each lane owns the same 16-byte column chunks of every row it visits, so
//    its slice of x is loaded once into registers and reused for R rows;
//  * weights stream with 16-byte non-temporal loads, R*KT of them issued back
//    to back per lane before any arithmetic (bytes in flight hide HBM latency);
//  * int8 / nibbles become floats with v_cvt_f32_ubyteN on byte-biased values
//    (q+128 resp. nibble) and the bias is removed once per row:
//      sum x*q = sum x*(q+128) - 128*sum x
//  * the R*B partial sums are reduced across the lane group with a transposed
//    butterfly (R*B values cost ~R*B + log2(G) shuffles instead of R*B*log2(G)).
// Optional fused prologue (RMSNorm of x) and epilogues (residual add; SwiGLU
// of a gate/up matrix pair) remove separate elementwise launches.
#include "mlh_device.h"
#include "mlh_host.h"

namespace mlh {

template <int FMT> struct FmtTraits;
template <> struct FmtTraits<kF32> { static constexpr int kElemsPerChunk = 4; };
template <> struct FmtTraits<kQ8> { static constexpr int kElemsPerChunk = 16; };
template <> struct FmtTraits<kQ4> { static constexpr int kElemsPerChunk = 32; };

// Dot product of one 16-byte weight chunk with EPC x values, accumulated on
// the byte-biased integer values (bias removed later through sum x).
template <int FMT>
__device__ __forceinline__ float chunk_dot(u32x4 w, const float *x, float acc) {
    if constexpr (FMT == kF32) {
        acc = fmaf(__uint_as_float(w.x), x[0], acc);
        acc = fmaf(__uint_as_float(w.y), x[1], acc);
        acc = fmaf(__uint_as_float(w.z), x[2], acc);
        acc = fmaf(__uint_as_float(w.w), x[3], acc);
    } else if constexpr (FMT == kQ8) {
        unsigned int d[4] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u,
                             w.z ^ 0x80808080u, w.w ^ 0x80808080u};
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

template <int FMT> __device__ __forceinline__ float bias_of() {
    return FMT == kQ8 ? 128.0f : (FMT == kQ4 ? 8.0f : 0.0f);
}

// Rows per wave pass for a (KT chunks per lane, B token rows) shape: keep
// about 16 weight loads in flight per lane and at most 16 partial sums.
template <int KT, int B, int LPR>
struct RowsPerGroup {
    static constexpr int kLoads = 16 / KT > 1 ? 16 / KT : 2;
    static constexpr int kSums = 16 / B > 1 ? 16 / B : 2;
    static constexpr int kMin = kLoads < kSums ? kLoads : kSums;
    static constexpr int value = kMin * B <= LPR ? kMin : (LPR / B > 1 ? LPR / B : 2);
};

template <int FMT, int B, int KT, int LPR>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams p) {
    constexpr int EPC = FmtTraits<FMT>::kElemsPerChunk;
    constexpr int R = RowsPerGroup<KT, B, LPR>::value;
    constexpr int GPW = kWave / LPR;  // row groups per wave
    constexpr int NV = R * B;
    static_assert(NV <= LPR, "partial sums exceed group width");

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    const int group = lane / LPR;
    const int li = lane & (LPR - 1);

    const int row_bytes = FMT == kF32 ? p.I * 4 : (FMT == kQ8 ? p.I : p.I / 2);
    const int nc = row_bytes / 16;  // chunks per row
    const bool dual = p.epilogue == kEpiSiluDual;
    // Logical row r of this group -> matrix row.  Dual mode: first half gate,
    // second half up, same output index.
    const int rows_per_group_out = dual ? R / 2 : R;
    const int out0 = (wave * GPW + group) * rows_per_group_out;
    if (out0 >= p.O) return;

    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = 0.0f;
    float sumx[B];
#pragma unroll
    for (int b = 0; b < B; ++b) sumx[b] = 0.0f;

    // RMSNorm prologue scale per token row (whole row must be one k-tile).
    float inv_rms[B];
#pragma unroll
    for (int b = 0; b < B; ++b) inv_rms[b] = 1.0f;
    if (p.norm_w) {
        float ss[B];
#pragma unroll
        for (int b = 0; b < B; ++b) ss[b] = 0.0f;
#pragma unroll
        for (int k = 0; k < KT; ++k) {
            const int c = li + LPR * k;
            if (c < nc) {
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    if (b < p.rows) {
                        const float *xs = p.x + (long)b * p.x_stride + c * EPC;
#pragma unroll
                        for (int e = 0; e < EPC; e += 4) {
                            f32x4 v = load_f4(xs + e);
                            ss[b] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            float t = group_sum<LPR>(ss[b]);
            inv_rms[b] = 1.0f / sqrtf(t / (float)p.I + p.eps);
        }
    }

    for (int kt0 = 0; kt0 < nc; kt0 += KT * LPR) {
        // weights first: R * KT independent 16-byte loads per lane
        u32x4 wv[R][KT];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t *base;
            int row;
            if (dual) {
                row = out0 + (r < R / 2 ? r : r - R / 2);
                base = r < R / 2 ? p.w : p.w2;
            } else {
                row = out0 + r;
                base = p.w;
            }
#pragma unroll
            for (int k = 0; k < KT; ++k) {
                const int c = kt0 + li + LPR * k;
                if (row < p.O && c < nc)
                    wv[r][k] = load_stream16(base + (long)row * row_bytes + c * 16);
                else
                    wv[r][k] = u32x4{0u, 0u, 0u, 0u};
            }
        }
        // activations for the same chunks
        float xr[B][KT][EPC];
#pragma unroll
        for (int k = 0; k < KT; ++k) {
            const int c = kt0 + li + LPR * k;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const bool ok = c < nc && b < p.rows;
                const float *xs = p.x + (long)b * p.x_stride + c * EPC;
                const float *ns = p.norm_w + c * EPC;
#pragma unroll
                for (int e = 0; e < EPC; e += 4) {
                    f32x4 v = ok ? load_f4(xs + e) : f32x4{0.f, 0.f, 0.f, 0.f};
                    if (p.norm_w && ok) {
                        f32x4 n = load_f4(ns + e);
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

    // remove the byte bias: sum x*(q+bias) - bias*sum x
    if constexpr (FMT != kF32) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int b = 0; b < B; ++b) acc[r * B + b] -= bias_of<FMT>() * sumx[b];
    }

    butterfly_reduce<NV, LPR>(acc, lane);
    const int vi = butterfly_index<NV, LPR>(lane);
    const int r = vi / B, b = vi % B;
    float value = acc[0];
    if (dual) {
        // the up-projection partner of value index vi is vi + NV/2, held by
        // the lane across the first butterfly offset
        float partner = __shfl_xor(value, LPR / 2, kWave);
        const int row = out0 + r;
        if (butterfly_writer<NV, LPR>(lane) && r < R / 2 && row < p.O && b < p.rows) {
            float g = FMT == kF32 ? value : value * p.s[row];
            float u = FMT == kF32 ? partner : partner * p.s2[row];
            p.y[(long)b * p.y_stride + row] = silu(g) * u;
        }
        return;
    }
    const int row = out0 + r;
    if (butterfly_writer<NV, LPR>(lane) && row < p.O && b < p.rows) {
        float out = FMT == kF32 ? value : value * p.s[row];
        if (p.epilogue == kEpiResidual) out = p.resid[(long)b * p.resid_stride + row] + out;
        p.y[(long)b * p.y_stride + row] = out;
    }
}

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
// host dispatch
// ---------------------------------------------------------------------------

template <int FMT, int B, int KT, int LPR>
static void launch_one(const GemvParams &p, hipStream_t stream) {
    constexpr int R = RowsPerGroup<KT, B, LPR>::value;
    constexpr int GPW = kWave / LPR;
    const int out_per_group = p.epilogue == kEpiSiluDual ? R / 2 : R;
    const long groups = (p.O + out_per_group - 1) / out_per_group;
    const long waves = (groups + GPW - 1) / GPW;
    const long blocks = (waves + 3) / 4;
    hipLaunchKernelGGL((gemv_kernel<FMT, B, KT, LPR>), dim3((unsigned)blocks), dim3(256),
                       0, stream, p);
}

template <int FMT, int B>
static bool dispatch_shape(const GemvParams &p, int nc, hipStream_t stream) {
    // Rows of at most 64 chunks: one chunk per lane, lane groups sized to the
    // row.  Longer rows: KT chunks per lane and k-tile; a row that fits one
    // k-tile stays resident in registers (required by the RMSNorm prologue).
    // KT is capped per format by the register cost of the x slice (q4 chunks
    // carry 32 x values, q8 16, f32 4).
    if (nc <= 8) { launch_one<FMT, B, 1, 8>(p, stream); return true; }
    if (nc <= 16) { launch_one<FMT, B, 1, 16>(p, stream); return true; }
    if (nc <= 32) { launch_one<FMT, B, 1, 32>(p, stream); return true; }
    if (nc <= 64) { launch_one<FMT, B, 1, 64>(p, stream); return true; }
    if (p.norm_w && nc > (FMT == kF32 ? 512 : FMT == kQ8 ? 128 : 64)) return false;
    if constexpr (FMT == kQ4) {
        launch_one<FMT, B, 1, 64>(p, stream);
    } else if constexpr (FMT == kQ8) {
        launch_one<FMT, B, 2, 64>(p, stream);
    } else {
        if (nc <= 128) launch_one<FMT, B, 2, 64>(p, stream);
        else if (nc <= 256) launch_one<FMT, B, 4, 64>(p, stream);
        else if (nc <= 512) launch_one<FMT, B, 8, 64>(p, stream);
        else launch_one<FMT, B, 4, 64>(p, stream);
    }
    return true;
}

template <int FMT>
static bool dispatch_fmt(const GemvParams &p, int nc, hipStream_t stream) {
    switch (p.rows <= 1 ? 1 : p.rows <= 2 ? 2 : 4) {
    case 1: return dispatch_shape<FMT, 1>(p, nc, stream);
    case 2: return dispatch_shape<FMT, 2>(p, nc, stream);
    default: return dispatch_shape<FMT, 4>(p, nc, stream);
    }
}

static bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15u) == 0; }

int gemv(const GemvParams &p_in, hipStream_t stream) {
    if (!p_in.w || !p_in.x || !p_in.y || p_in.O <= 0 || p_in.I <= 0 || p_in.rows <= 0)
        return kErrArgs;
    if (p_in.fmt != kF32 && !p_in.s) return kErrArgs;
    if (p_in.epilogue == kEpiSiluDual && (!p_in.w2 || (p_in.fmt != kF32 && !p_in.s2)))
        return kErrArgs;
    if (p_in.epilogue == kEpiResidual && !p_in.resid) return kErrArgs;
    const long row_bytes = p_in.fmt == kF32 ? (long)p_in.I * 4
                         : p_in.fmt == kQ8 ? p_in.I : (p_in.I + 1) / 2;
    const bool vector_ok =
        row_bytes % 16 == 0 && (p_in.fmt != kQ4 || p_in.I % 2 == 0) &&
        aligned16(p_in.w) && (!p_in.w2 || aligned16(p_in.w2)) && aligned16(p_in.x) &&
        p_in.x_stride % 4 == 0 && (!p_in.norm_w || aligned16(p_in.norm_w));
    // token rows beyond 4 are processed in slices of 4 (register budget)
    for (int r0 = 0; r0 < p_in.rows; r0 += kMaxGemvRows) {
        GemvParams p = p_in;
        p.rows = p_in.rows - r0 < kMaxGemvRows ? p_in.rows - r0 : kMaxGemvRows;
        p.x = p_in.x + (long)r0 * p_in.x_stride;
        p.y = p_in.y + (long)r0 * p_in.y_stride;
        if (p.resid) p.resid = p_in.resid + (long)r0 * p_in.resid_stride;
        bool done = false;
        if (vector_ok) {
            const int nc = (int)(row_bytes / 16);
            if (p.fmt == kF32) done = dispatch_fmt<kF32>(p, nc, stream);
            else if (p.fmt == kQ8) done = dispatch_fmt<kQ8>(p, nc, stream);
            else done = dispatch_fmt<kQ4>(p, nc, stream);
        }
        if (!done) {
            hipLaunchKernelGGL(gemv_generic_kernel, dim3(p.O, p.rows), dim3(64), 0, stream,
                               p, p.fmt);
        }
    }
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace mlh

// gemv_impl.h -- the bandwidth-bound dequant GEMV core (gfx950, wave64), shared by
// the plain GEMV launches (gemv_*.hip) and the grouped MoE expert launches.
//
// Semantics follow moonlight_matmul_f32 / _q8_reduction / _q4
// (moonlight_kernels.metal:43-130): y[b,o] = (sum_i x[b,i] * q[o,i]) * s[o] with
// fp32 accumulation; q8 is int8 row-major [O, I], q4 packs column 2j in the low
// nibble and 2j+1 in the high nibble of byte j, stored as q+8
// (tools/convert_moonlight.py:46-66).
//
// Work decomposition.  A workgroup is 4 (or, for the quantised formats, 8)
// wavefronts.  A row of W is cut into 16-byte chunks; a group of LPR lanes
// covers a row, each lane owning the chunks li, li+LPR, ... of every row it
// visits (k-tiles of KT chunks per lane).
//   KS = 1: every wave owns R rows (per lane group);
//   KS > 1: the waves of a workgroup share the same R rows and split the
//           k-tiles between them (wide rows: the 11264-long down projections),
//           partial sums meet in LDS.
// Per k-tile a lane issues its R*KT 16-byte non-temporal weight loads back to
// back, then uses them against the matching slice of x for the R rows.
//   f32 weights (lm_head, router): fp32 FMAs against x read from L1 / L2
//           (gemv_block).
//   q8 / q4 weights: int8-limb dot products against x split once per
//           workgroup into LDS (limb_block; the numerics are described there).
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

// One 16-byte chunk of f32 weights (4 values) against 4 values of x.
__device__ __forceinline__ float chunk_dot_f32(u32x4 w, const float *x, float acc) {
    acc = fmaf(__uint_as_float(w.x), x[0], acc);
    acc = fmaf(__uint_as_float(w.y), x[1], acc);
    acc = fmaf(__uint_as_float(w.z), x[2], acc);
    acc = fmaf(__uint_as_float(w.w), x[3], acc);
    return acc;
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
    // optional: x already split into limb rows (limb_quantise_rows), one per
    // token row, in the LDS row layout; the prologue then only copies them
    const unsigned char *limbs[B];
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
    static_assert(FMT == kF32, "q8 / q4 take limb_block");
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
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int k = 0; k < KT; ++k)
#pragma unroll
                for (int b = 0; b < B; ++b)
                    acc[r * B + b] = chunk_dot_f32(wv[r][k], xr[b][k], acc[r * B + b]);
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

// ---------------------------------------------------------------------------
// Quantised formats (q8, q4): int8-limb dot products.
//
// Every workgroup first splits its token rows of x (RMSNorm'ed when norm_w is
// set) into LDS: per 16-byte weight chunk (16 q8 or 32 q4 elements) a scale
// sc = amax / 2^22 and three int8 limbs per element,
//     v ~= sc * (65536 * hi + 256 * mid + lo),  |65536 hi + 256 mid + lo| <= 2^22,
// i.e. 23 significant bits against the chunk's own max -- the precision of an
// fp32 operand.  A chunk's share of a row is then exact integer dot products
// of the stored weights with each limb (v_dot4_i32_i8: 4 products and their
// sum per instruction), combined and scaled once in fp32:
//     sum_chunk q * v ~= sc * (65536 * dot(q, hi) + (256 * dot(q, mid) + dot(q, lo))).
// q8 weights are the stored int8 values; q4 weights enter as the stored
// nibbles u = q + 8 (0..15, valid int8 operands) and 8 * (sum of the limb
// values) of the chunk is subtracted once per chunk.  The rounding of v is at
// most 0.75 * amax_chunk / 2^22 per element and the in-chunk sums are exact,
// so results agree with the fp32 matmul to fp32 rounding (like a different
// summation order).  The arithmetic drops from ~2.3 VALU instructions per
// weight (convert + fma) to ~1.1 (q8) / ~1.3 (q4), which is what kept the fp32
// form from streaming at HBM rate.
//
// Loads are ordered for the in-order vector memory counter: x (and norm_w),
// the epilogue's scale / residual values, then the first weight tile, all
// unpredicated (clamped addresses), so the prologue waits only for x while the
// weights are in flight.
// ---------------------------------------------------------------------------
constexpr int kLimbQuantMax = 1 << 22;  // |65536 hi + 256 mid + lo| bound
constexpr int kLimbPassElems = 2048;    // x elements quantised per workgroup pass

struct LimbInfo {
    float scale;
    int bias_hi;   // q4: 8 * sum(hi) of the chunk, else 0
    int bias_low;  // q4: 8 * sum(256 mid + lo) of the chunk, else 0
    int pad;
};

// Bytes of one token row of width I in the limb layout: hi, mid and lo limbs
// (I bytes each) and a LimbInfo per 16-byte weight chunk, padded to 1 KB (the
// unit of the LDS DMA copy of pre-split rows).  The same layout serves the
// LDS rows and the pre-split rows in memory.
__host__ __device__ constexpr int limb_row_bytes(int fmt, int I) {
    return 3 * I + 16 * (row_bytes_of(fmt, I) / 16);
}
__host__ __device__ constexpr int limb_row_lds(int fmt, int I) {
    return (limb_row_bytes(fmt, I) + 1023) & ~1023;
}

__device__ __forceinline__ int sdot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

__device__ __forceinline__ unsigned pack_i8x4(int a, int b, int c, int d) {
    return (unsigned)(a & 255) | ((unsigned)(b & 255) << 8) | ((unsigned)(c & 255) << 16) |
           ((unsigned)(d & 255) << 24);
}

// Quantises the 8 elements e0 .. e0 + 7 of one token row held by this thread
// (TPG neighbouring threads share a chunk).  Limb layout per row: hi at 0, mid
// at I, lo at 2 I.  q4 limbs are stored per 8 elements as the even-element
// dword then the odd-element dword (the order the nibble masks produce), each
// chunk's 32 bytes split in two 16-byte halves held nc * 16 bytes apart so a
// lane's 16-byte LDS reads are contiguous across lanes.  The quantisation step
// is 1 / rcp(amax / 2^22) (any step works: the stored scale amax / 2^22 is
// exact and the limbs are clamped).
template <int FMT>
__device__ __forceinline__ void limb_quantise(const float (&v)[8], bool in, int e0,
                                              unsigned char *row_lds, int I, int nc) {
    constexpr int EPT = 8;
    constexpr int EPC = FmtTraits<FMT>::kElemsPerChunk;
    constexpr int TPG = EPC / EPT;
    float m = 0.0f, bad = 0.0f;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        m = fmaxf(m, fabsf(v[i]));
        bad = fmaf(v[i], 0.0f, bad);  // NaN when some element is not finite
    }
#pragma unroll
    for (int o = 1; o < TPG; o <<= 1) {
        m = fmaxf(m, __shfl_xor(m, o, kWave));
        bad += __shfl_xor(bad, o, kWave);
    }
    // rows with amax below 1e-30 (where the step would overflow) quantise to 0
    const float inv = m > 1e-30f ? (float)kLimbQuantMax * __builtin_amdgcn_rcpf(m) : 0.0f;
    // q = 65536 hi + 256 mid + lo with hi in [-64, 64], mid and lo in
    // [-128, 127] is the base-256 form of U = q + 128 (65536 + 256 + 1):
    // U < 2^24 is exact in fp32 and the limbs are its bytes, each XOR 0x80
    // (the byte minus 128 in two's complement).
    unsigned U[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        float q = rintf(v[i] * inv);
        q = fminf(fmaxf(q, -(float)kLimbQuantMax), (float)kLimbQuantMax);
        U[i] = (unsigned)(q + 8421504.0f);
    }
    // byte k of a, b, c, d (in that order) as one signed-limb dword
    auto gather = [](unsigned a, unsigned b, unsigned c, unsigned d, int k) -> unsigned {
        const unsigned lo = __builtin_amdgcn_perm(b, a, (unsigned)(k | ((4 + k) << 8)) | 0x0c0c0000u);
        const unsigned hi = __builtin_amdgcn_perm(d, c, 0x00000c0cu | (unsigned)((k << 16) | ((4 + k) << 24)));
        return (lo | hi) ^ 0x80808080u;
    };
    constexpr int ND = EPT / 4;  // limb dwords per limb
    unsigned H[ND], M[ND], L[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) {
        // q8: elements 4d .. 4d + 3; q4: dword 0 the even, dword 1 the odd
        // elements
        int e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) e[j] = FMT == kQ4 ? 2 * j + d : 4 * d + j;
        H[d] = gather(U[e[0]], U[e[1]], U[e[2]], U[e[3]], 2);
        M[d] = gather(U[e[0]], U[e[1]], U[e[2]], U[e[3]], 1);
        L[d] = gather(U[e[0]], U[e[1]], U[e[2]], U[e[3]], 0);
    }
    // q4 bias terms: sum of hi and of 256 mid + lo over the chunk
    int hs = 0, ms = 0;
    if constexpr (FMT == kQ4) {
#pragma unroll
        for (int d = 0; d < ND; ++d) {
            hs = sdot4((int)H[d], 0x01010101, hs);
            ms += 256 * sdot4((int)M[d], 0x01010101, 0) + sdot4((int)L[d], 0x01010101, 0);
        }
#pragma unroll
        for (int o = 1; o < TPG; o <<= 1) {
            hs += __shfl_xor(hs, o, kWave);
            ms += __shfl_xor(ms, o, kWave);
        }
    }
    const int c = e0 / EPC, within = e0 % EPC;
    if (in) {
        const int g = within / 8;
        const int off = (FMT == kQ4 ? (g >> 1) * 16 * nc : 0) + 16 * c + 8 * (g & 1);
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2 *>(row_lds + off) = u32x2{H[0], H[1]};
        *reinterpret_cast<u32x2 *>(row_lds + I + off) = u32x2{M[0], M[1]};
        *reinterpret_cast<u32x2 *>(row_lds + 2 * I + off) = u32x2{L[0], L[1]};
        if (within == 0) {
            LimbInfo info;
            info.scale = m / (float)kLimbQuantMax + bad;
            info.bias_hi = FMT == kQ4 ? 8 * hs : 0;
            info.bias_low = FMT == kQ4 ? 8 * ms : 0;
            info.pad = 0;
            reinterpret_cast<LimbInfo *>(row_lds + 3 * I)[c] = info;
        }
    }
}

// One 16-byte weight chunk against the limbs of chunk c of one token row:
// the chunk's integer dot product as 65536 * dot_hi + dot_low (bias removed),
// returned in fp32.
template <int FMT>
__device__ __forceinline__ float limb_chunk_dot(u32x4 w, const unsigned char *row_lds, int I,
                                                int nc, int c, const LimbInfo &info) {
    const unsigned d[4] = {w.x, w.y, w.z, w.w};
    int hd = 0, mdd = 0, ld = 0;
    if constexpr (FMT == kQ4) {
        u32x4 lv[3][2];
#pragma unroll
        for (int t = 0; t < 3; ++t) {
            lv[t][0] = *reinterpret_cast<const u32x4 *>(row_lds + t * I + 16 * c);
            lv[t][1] = *reinterpret_cast<const u32x4 *>(row_lds + t * I + 16 * nc + 16 * c);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int ev = (int)(d[j] & 0x0F0F0F0Fu), od = (int)((d[j] >> 4) & 0x0F0F0F0Fu);
            const int half = j >> 1, k = 2 * (j & 1);
            hd = sdot4(ev, (int)lv[0][half][k], hd);
            hd = sdot4(od, (int)lv[0][half][k + 1], hd);
            mdd = sdot4(ev, (int)lv[1][half][k], mdd);
            mdd = sdot4(od, (int)lv[1][half][k + 1], mdd);
            ld = sdot4(ev, (int)lv[2][half][k], ld);
            ld = sdot4(od, (int)lv[2][half][k + 1], ld);
        }
    } else {
        u32x4 lv[3];
#pragma unroll
        for (int t = 0; t < 3; ++t) lv[t] = *reinterpret_cast<const u32x4 *>(row_lds + t * I + 16 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            hd = sdot4((int)d[j], (int)lv[0][j], hd);
            mdd = sdot4((int)d[j], (int)lv[1][j], mdd);
            ld = sdot4((int)d[j], (int)lv[2][j], ld);
        }
    }
    // |hd| <= 2^17 and |256 mdd + ld| < 2^27: exact in int32, the fp32 sum
    // rounds once
    return fmaf((float)(hd - info.bias_hi), 65536.0f, (float)(mdd * 256 + ld - info.bias_low));
}

// x passes held in registers across the weight issue: as many as a row the
// plan covers in one tile can need (KS * KT * 64 chunks), at most 6 (an
// 11264-wide row), one for B > 1; the rest of a wider row is loaded after the
// weights.
template <int FMT, int B, int KT, int KS, int W>
constexpr int limb_pre_passes() {
    constexpr int elems = KS * KT * 64 * FmtTraits<FMT>::kElemsPerChunk;
    constexpr int pass = W * kWave * 8;
    constexpr int passes = (elems + pass - 1) / pass;
    return B == 1 ? (passes < 6 ? passes : 6) : 1;
}

// A job's token rows (RMSNorm'ed with job.norm_w) split into limbs in the
// LDS row layout, in two steps so that the loads can be issued well before
// the split: issue() loads the first passes of x (and norm_w) into
// registers; quantise() takes the RMSNorm statistics (one workgroup barrier)
// and stores the limb rows, loading any further passes on the way.  Every
// thread of the workgroup calls both; with `presplit` (limb rows copied in
// by DMA instead) both do nothing but the barrier.
template <int FMT, int B, int KT, int KS, int W>
struct LimbRowsX {
    static constexpr int NJP = limb_pre_passes<FMT, B, KT, KS, W>();
    static constexpr int EPT = 8;                 // x elements per thread per pass
    static constexpr int XV = EPT / 4;            // float4 loads per thread per pass and row
    static constexpr int PASS = W * kWave * EPT;  // x elements split per workgroup pass
    f32x4 xv[NJP][B][XV];
    f32x4 nv[NJP][XV];

    __device__ __forceinline__ void issue(const GemvJob<B> &job, bool presplit) {
        const int tid = threadIdx.x;
        const int I = job.I;
        const int npass = (I + PASS - 1) / PASS;
#pragma unroll
        for (int j = 0; j < NJP; ++j) {
            if (!presplit && j < npass) {
                const int e0 = tid * EPT + j * PASS;
                const int ec = e0 < I ? e0 : 0;
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    if (b < job.rows) {  // uniform: absent token rows cost nothing
#pragma unroll
                        for (int h = 0; h < XV; ++h) xv[j][b][h] = load_f4(job.x[b] + ec + 4 * h);
                    }
                }
                if (job.norm_w) {
#pragma unroll
                    for (int h = 0; h < XV; ++h) nv[j][h] = load_f4(job.norm_w + ec + 4 * h);
                }
            }
        }
    }

    __device__ __forceinline__ void quantise(const GemvJob<B> &job, unsigned char *lds,
                                             bool presplit) {
        __shared__ float ss_red[W][B];
        const int tid = threadIdx.x;
        const int lane = tid & (kWave - 1);
        const int wave = tid / kWave;
        const int I = job.I;
        const int nc = row_bytes_of(FMT, I) / 16;
        const int lds_row = limb_row_lds(FMT, I);
        const int npass = (I + PASS - 1) / PASS;
        // RMSNorm statistics (workgroup reduction)
        float inv_rms[B];
#pragma unroll
        for (int b = 0; b < B; ++b) inv_rms[b] = 1.0f;
        if (job.norm_w && !presplit) {
            float ss[B];
#pragma unroll
            for (int b = 0; b < B; ++b) ss[b] = 0.0f;
#pragma unroll
            for (int j = 0; j < NJP; ++j) {
                if (j < npass && tid * EPT + j * PASS < I) {
#pragma unroll
                    for (int b = 0; b < B; ++b)
                        if (b < job.rows)
#pragma unroll
                        for (int h = 0; h < XV; ++h)
                            ss[b] += xv[j][b][h].x * xv[j][b][h].x + xv[j][b][h].y * xv[j][b][h].y +
                                     xv[j][b][h].z * xv[j][b][h].z + xv[j][b][h].w * xv[j][b][h].w;
                }
            }
            for (int j = NJP; j < npass; ++j) {
                const int e0 = tid * EPT + j * PASS;
                if (e0 < I) {
#pragma unroll
                    for (int b = 0; b < B; ++b)
                        if (b < job.rows)
#pragma unroll
                        for (int h = 0; h < XV; ++h) {
                            const f32x4 t = load_f4(job.x[b] + e0 + 4 * h);
                            ss[b] += t.x * t.x + t.y * t.y + t.z * t.z + t.w * t.w;
                        }
                }
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const float w_ss = wave_sum(ss[b]);
                if (lane == 0) ss_red[wave][b] = w_ss;
            }
            __syncthreads();
#pragma unroll
            for (int b = 0; b < B; ++b) {
                float tot = (ss_red[0][b] + ss_red[1][b]) + (ss_red[2][b] + ss_red[3][b]);
#pragma unroll
                for (int w = 4; w < W; w += 4)
                    tot += (ss_red[w][b] + ss_red[w + 1][b]) + (ss_red[w + 2][b] + ss_red[w + 3][b]);
                inv_rms[b] = 1.0f / sqrtf(tot / (float)I + job.eps);
            }
        }
        // quantise x into LDS
        auto quantise_pass = [&](const f32x4 (&xp)[XV], const f32x4 (&np)[XV], int b, int e0) {
            float v[EPT];
#pragma unroll
            for (int h = 0; h < XV; ++h) {
                v[4 * h + 0] = xp[h].x;
                v[4 * h + 1] = xp[h].y;
                v[4 * h + 2] = xp[h].z;
                v[4 * h + 3] = xp[h].w;
            }
            if (job.norm_w) {
#pragma unroll
                for (int h = 0; h < XV; ++h) {
                    v[4 * h + 0] = v[4 * h + 0] * inv_rms[b] * np[h].x;
                    v[4 * h + 1] = v[4 * h + 1] * inv_rms[b] * np[h].y;
                    v[4 * h + 2] = v[4 * h + 2] * inv_rms[b] * np[h].z;
                    v[4 * h + 3] = v[4 * h + 3] * inv_rms[b] * np[h].w;
                }
            }
            limb_quantise<FMT>(v, e0 < I && b < job.rows, e0, lds + b * lds_row, I, nc);
        };
#pragma unroll
        for (int j = 0; j < NJP; ++j) {
            if (!presplit && j < npass) {
                const int e0 = tid * EPT + j * PASS;
#pragma unroll
                for (int b = 0; b < B; ++b)
                    if (b < job.rows) quantise_pass(xv[j][b], nv[j], b, e0);
            }
        }
        for (int j = presplit ? npass : NJP; j < npass; ++j) {
            const int e0 = tid * EPT + j * PASS;
            const int ec = e0 < I ? e0 : 0;
            f32x4 np[XV];
#pragma unroll
            for (int h = 0; h < XV; ++h)
                np[h] = job.norm_w ? load_f4(job.norm_w + ec + 4 * h) : f32x4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
            for (int b = 0; b < B; ++b) {
                if (b < job.rows) {
                    f32x4 xp[XV];
#pragma unroll
                    for (int h = 0; h < XV; ++h) xp[h] = load_f4(job.x[b] + ec + 4 * h);
                    quantise_pass(xp, np, b, e0);
                }
            }
        }
    }
};

// One job: the token rows of job.x against row block job.row_block of the
// weights.  W waves per workgroup (4 or 8); with KS > 1 the W waves split k.
// XR: the caller has already stored the job's limb rows in LDS (LimbRowsX)
// and passed a workgroup barrier since.
template <int FMT, int B, int KT, int LPR, int R, int KS, int W = 4, bool XR = false>
__device__ __forceinline__ void limb_block(const GemvJob<B> job, unsigned char *lds) {
    constexpr int GPW = kWave / LPR;
    constexpr int NV = R * B;
    static_assert(NV <= LPR, "partial sums exceed the lane group");
    static_assert(KS == 1 || (LPR == kWave && KS == W), "k-split needs whole-wave row groups");
    __shared__ float red[W][NV];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int group = lane / LPR;
    const int li = lane & (LPR - 1);
    const bool dual = job.epilogue == kEpiSiluDual;
    const bool residual = job.epilogue == kEpiResidual;
    const int out_per_group = dual ? R / 2 : R;
    const int row_wave = KS == 1 ? job.row_block * W + wave : job.row_block;
    const int kpart = KS == 1 ? 0 : wave;
    const int out0 = (row_wave * GPW + group) * out_per_group;
    const int rpb = out_per_group * GPW * (KS == 1 ? W : 1);  // outputs per row block
    // whole workgroups past the end leave (the prologue below synchronises)
    if (job.row_block * rpb >= job.O) return;

    const int I = job.I;
    const int row_bytes = row_bytes_of(FMT, I);
    const int nc = row_bytes / 16;
    const int lds_row = limb_row_lds(FMT, I);

    const bool presplit = !XR && job.limbs[0] != nullptr;
    if (presplit) {
        // ---- 1'. pre-split rows: 1 KB blocks straight into LDS (DMA)
        const int nblk = lds_row / 1024;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            if (b < job.rows) {
                for (int blk = wave; blk < nblk; blk += W) {
                    __builtin_amdgcn_global_load_lds(
                        (const __attribute__((address_space(1))) void *)(job.limbs[b] + blk * 1024 +
                                                                         lane * 16),
                        (__attribute__((address_space(3))) void *)(lds + b * lds_row + blk * 1024),
                        16, 0, 0);
                }
            }
        }
    }
    // ---- 1. x (and norm_w) of the first passes
    LimbRowsX<FMT, B, KT, KS, W> xr;
    if constexpr (!XR) xr.issue(job, presplit);
    // ---- 2. the value this lane writes, and its epilogue operands
    const int vi = butterfly_index<NV, LPR>(lane);
    const int vr = vi / B, vb = vi % B;
    float *yb = job.y[0];
    const float *rb = job.resid[0];
#pragma unroll
    for (int i = 1; i < B; ++i) {
        if (vb == i) {  // compare chain: a lane-indexed pointer array would spill
            yb = job.y[i];
            rb = job.resid[i];
        }
    }
    struct Epi {
        float s, s2, resid;
    };
    // (the conditional loads are issued before the weights, whose waits they
    // therefore do not disturb)
    auto load_epi = [&](int o0) {
        const int vrow = o0 + vr;
        const int vc = vrow < job.O ? vrow : job.O - 1;
        Epi e{load_global_f32(job.s + vc), 0.0f, 0.0f};
        if (dual) e.s2 = load_global_f32(job.s2 + vc);
        if (residual) e.resid = load_global_f32(rb + vc);
        return e;
    };
    const Epi epi_cur = load_epi(out0);
    // ---- 3. the first weight tile.  Column-major issue (all rows of chunk
    // column k, then k + 1); a column entirely past the row end is skipped --
    // a uniform branch after the columns the compute needs first, so their
    // waits stay exact.
    const int step = KS * KT * LPR;
    auto load_tile = [&](u32x4 (&wv)[R][KT], int kt0, int o0) {
#pragma unroll
        for (int k = 0; k < KT; ++k) {
            if (k > 0 && kt0 + LPR * k >= nc) {
#pragma unroll
                for (int r = 0; r < R; ++r) wv[r][k] = u32x4{0u, 0u, 0u, 0u};
                continue;
            }
            const int c = kt0 + li + LPR * k;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                int row;
                const uint8_t *base;
                if (dual) {
                    row = o0 + (r < R / 2 ? r : r - R / 2);
                    base = r < R / 2 ? job.w : job.w2;
                } else {
                    row = o0 + r;
                    base = job.w;
                }
                const int row_c = row < job.O ? row : job.O - 1;
                const u32x4 v = load_stream16(base + (long)row_c * row_bytes + (c < nc ? c : 0) * 16);
                wv[r][k] = (row < job.O && c < nc) ? v : u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    u32x4 wa[R][KT];
    load_tile(wa, kpart * KT * LPR, out0);

    // ---- 4, 5. RMSNorm statistics, x quantised into LDS
    if constexpr (!XR) xr.quantise(job, lds, presplit);
    if (presplit) __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA blocks have landed
    if constexpr (!XR) __syncthreads();

    // ---- 6. dot products of one k tile into acc
    auto dot_tile = [&](const u32x4 (&wv)[R][KT], int kt0, float (&acc)[NV]) {
#pragma unroll
        for (int k = 0; k < KT; ++k) {
            const int c = kt0 + li + LPR * k;
            const bool cok = c < nc;
            const int cc = cok ? c : 0;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                if (b < job.rows) {
                    const unsigned char *row_lds = lds + b * lds_row;
                    const LimbInfo info = reinterpret_cast<const LimbInfo *>(row_lds + 3 * I)[cc];
                    const float sc = cok ? info.scale : 0.0f;
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float dot = limb_chunk_dot<FMT>(wv[r][k], row_lds, I, nc, cc, info);
                        acc[r * B + b] = fmaf(dot, sc, acc[r * B + b]);
                    }
                }
            }
        }
    };
    // ---- 7. reduction and epilogue of the row block (o0: its out0)
    auto finish = [&](float (&acc)[NV], int o0, const Epi &ep) {
        butterfly_reduce<NV, LPR>(acc, lane);
        const bool writer = butterfly_writer<NV, LPR>(lane);
        float value = acc[0];
        if constexpr (KS > 1) {
            if (writer) red[wave][vi] = value;
            __syncthreads();
            value = (red[0][vi] + red[1][vi]) + (red[2][vi] + red[3][vi]);
#pragma unroll
            for (int w = 4; w < W; w += 4)
                value += (red[w][vi] + red[w + 1][vi]) + (red[w + 2][vi] + red[w + 3][vi]);
            if (wave != 0) return;
        }
        const int vrow = o0 + vr;
        if (dual) {
            // the up-projection partner of value index vi is vi + NV/2, held by
            // the lane across the first butterfly offset
            const float partner = __shfl_xor(value, LPR / 2, kWave);
            if (writer && vr < R / 2 && vrow < job.O && vb < job.rows)
                yb[vrow] = silu(value * ep.s) * (partner * ep.s2);
            return;
        }
        if (writer && vrow < job.O && vb < job.rows) {
            float out = value * ep.s;
            if (residual) out = ep.resid + out;
            yb[vrow] = out;
        }
    };

    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = 0.0f;
    for (int kt0 = kpart * KT * LPR; kt0 < nc; kt0 += step) {
        if (kt0 != kpart * KT * LPR) load_tile(wa, kt0, out0);
        dot_tile(wa, kt0, acc);
    }
    finish(acc, out0, epi_cur);
}

// Grouped expert launches (MoE): blockIdx.x selects a task -- one active routed
// expert (in first-appearance order) or, after them, the fused shared expert --
// and its row block(s); blockIdx.y selects a group of B of that task's token
// rows.  Token rows are gathered / scattered through the device route tables,
// so no gather or scatter pass exists (moonlight_metal.m:577-638 issues
// gather_rows / scatter_expert per expert instead).
struct ExpertWeights {
    const uint8_t *gate, *up, *down;
    const float *gate_s, *up_s, *down_s;
};

// One active routed expert of a batch, as the routing kernels write it: its
// weights, its token rows and their offset in the compact lists.
struct ExpertTask {
    ExpertWeights w;
    int count, offset;
};

// Sigmoid top-k + route tables for `rows` token rows (one workgroup).
struct RouteParams {
    const float *logits = nullptr;  // [rows, experts] router logits
    const float *bias = nullptr;    // [experts] e_score_correction_bias (selection only)
    int rows = 0, experts = 0, top_k = 0, normalize = 1;
    float routed_scale = 1.0f;
    int *ids = nullptr;        // [rows, top_k] selection order
    float *weights = nullptr;  // [rows, top_k] finalised weights
    int *trace = nullptr;      // optional copy of ids (per-layer route trace)
    int *n_unique = nullptr;   // [1]
    int *unique = nullptr;     // [experts] active experts, first-appearance order
    int *counts = nullptr;     // [experts] entries per expert
    int *offsets = nullptr;    // [experts] start of each expert's compact list
    int *list_rows = nullptr;  // [rows*top_k] token row per list entry
    int *list_slots = nullptr; // [rows*top_k] slot per list entry
    int *list_pos = nullptr;   // [rows*top_k] list entry of (row, slot), -1 if invalid
    int *error = nullptr;      // [1] set to error_code when an id is out of range (if still 0)
    int error_code = 1;        // the forward passes layer + 1, so the first failing layer is kept
    // optional [rows, top_k] expert ids given by the caller: weights come from
    // their scores (moe_route_fixed, moe_route.h:76-87) instead of a top-k
    const int *fixed_ids = nullptr;
    // optional: the per-task table of the grouped expert launches
    const ExpertWeights *expert_table = nullptr;  // device [experts]
    ExpertTask *tasks = nullptr;                  // out [task_slots]
    int task_slots = 0;
    // optional, one token row routed inside the first expert launch: the
    // logits come as partials of the GEMV that wrote the row (GemvParams
    // router_parts, n_parts per expert, then n_parts partial sums of
    // squares of the row's `width` values): logit[e] = sum_j
    // logit_parts[e * n_parts + j] / sqrt(sum_j logit_parts[experts *
    // n_parts + j] / width + eps), the sums in one fixed order; the launch's
    // workgroup 0 also stores them in logits_out
    const float *logit_parts = nullptr;
    float *logits_out = nullptr;
    int n_parts = 0, width = 0;
    float eps = 0.0f;
};
struct ExpertGemvParams {
    int stage = 0;  // 0: gate/up + SwiGLU, 1: down
    const ExpertWeights *experts = nullptr;  // device table [E]
    const ExpertTask *tasks = nullptr;       // optional per-task table (one lookup)
    const int *n_unique = nullptr;           // route tables (device)
    const int *unique = nullptr;
    const int *counts = nullptr;
    const int *offsets = nullptr;
    const int *rows = nullptr;  // token row of each compact list entry
    int routed_tasks = 0;       // task slots for routed experts
    int routed_blocks = 0;      // row blocks (workgroups) per routed task
    int shared_task = 0;        // 1: the workgroups after the routed ones run the shared expert
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
    // optional pre-split limb rows (limb_quantise_rows): stage 0 by token row,
    // stage 1 by list entry; the shared expert's rows in sh_limbs
    const unsigned char *limbs = nullptr, *sh_limbs = nullptr;
    long limb_stride = 0, sh_limb_stride = 0;
    // stage 0 of a one-row batch with at most 64 experts: when route.logits
    // is set, every routed workgroup selects its expert from the router
    // logits itself (the route tables, which stage 1 and the combine read,
    // are written by workgroup 0), so no routing launch precedes stage 0
    RouteParams route;
};

}  // namespace mlh

#include "route_impl.h"

namespace mlh {

struct GemvLaunch {
    GemvParams plain;
    ExpertGemvParams expert;
};

// MODE 0: plain GEMV; 1: grouped expert tasks.
template <int MODE, int FMT, int B, int KT, int LPR, int R, int KS, int W>
__device__ __forceinline__ void run_job(const GemvJob<B> &job, unsigned char *lds) {
    if constexpr (FMT == kF32)
        gemv_block<FMT, B, KT, LPR, R, KS>(job);  // 4-wave workgroups
    else
        limb_block<FMT, B, KT, LPR, R, KS, W>(job, lds);
}

// Dynamic LDS of a launch: the quantised x rows of its widest job.
template <int FMT, int B>
__host__ __device__ constexpr int gemv_lds_bytes(int max_I) {
    return FMT == kF32 ? 0 : B * limb_row_lds(FMT, max_I);
}

template <int MODE, int FMT, int B, int KT, int LPR, int R, int KS, int W = 4>
__global__ __launch_bounds__(W * 64) void gemv_kernel(GemvLaunch L) {
    extern __shared__ __align__(16) unsigned char gemv_lds[];
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
            job.limbs[b] = p.limbs ? p.limbs + r * p.limb_stride : nullptr;
        }
        job.norm_w = p.norm_w;
        job.eps = p.eps;
        job.epilogue = p.epilogue;
        run_job<MODE, FMT, B, KT, LPR, R, KS, W>(job, gemv_lds);
    } else {
        const ExpertGemvParams &p = L.expert;
        __shared__ __align__(16) unsigned long long route_keys[W][64];
        // flat grid: routed task t owns workgroups t * routed_blocks ..,
        // the shared expert the ones after them (no idle workgroups)
        const int routed_wgs = p.routed_tasks * p.routed_blocks;
        const bool shared = (int)blockIdx.x >= routed_wgs;
        const int task = shared ? p.routed_tasks : (int)blockIdx.x / p.routed_blocks;
        job.row_block = shared ? (int)blockIdx.x - routed_wgs : (int)blockIdx.x % p.routed_blocks;
        int n, off = 0;
        const int *list = nullptr;
        // one routed token row of q8 / q4 experts: the row is split into
        // limbs while the routing runs (its loads issued with the router
        // operands'), so that only the weight stream follows the selection
        constexpr bool kLimbX = FMT != kF32 && B == 1;
        bool x_ready = false;
        if (shared) {
            n = p.shared_rows;
            job.w = p.sh_w;  // stage 0: shared gate (sh_w2 = up); stage 1: shared down
            job.s = p.sh_s;
            job.w2 = p.sh_w2;
            job.s2 = p.sh_s2;
            job.O = p.stage == 0 ? p.shared_width : p.hidden;
            job.I = p.stage == 0 ? p.hidden : p.shared_width;
        } else {
            ExpertWeights ew;
            if (p.route.logits) {
                // one token row: the logits (from partials: the whole
                // workgroup, one barrier), the tables for the later launches,
                // then this workgroup's own selection (every wave)
                __shared__ float route_logits[kMaxExperts + 1];
                const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
                GemvJob<B> xjob;
                LimbRowsX<FMT, B, KT, KS, W> xr;
                if constexpr (kLimbX) {
                    xjob.I = p.hidden;
                    xjob.rows = 1;
                    xjob.x[0] = p.x;  // token row 0
                    xjob.limbs[0] = nullptr;
                    xjob.norm_w = p.norm_w;  // inline routing: stage 0 only
                    xjob.eps = p.eps;
                    xr.issue(xjob, false);
                }
                // the bias and the expert table entries are in flight while
                // the logits are summed
                LaneRoute lr;
                if (p.route.logit_parts) {
                    lr = lane_route_load<false>(p.route, lane);
                    logits_from_parts(p.route, route_logits);
                    lr.logit = lane < p.route.experts ? route_logits[lane] : 0.0f;
                } else {
                    lr = lane_route_load<true>(p.route, lane);
                }
                if constexpr (kLimbX) {
                    // the limb rows, published by the barrier below
                    xr.quantise(xjob, gemv_lds, false);
                    x_ready = true;
                }
                // wave 0 selects this workgroup's expert (one wave per
                // workgroup: fewer waves per SIMD compete for the issue
                // slots), wave 1 of workgroup 0 writes the route tables
                __shared__ ExpertWeights sel_ew;
                __shared__ int sel_ok;
                if (wave == 0) {
                    ExpertWeights e;
                    const int src = inline_task_expert(p.route, task, &e, route_keys[0], lr);
                    if (lane == 0) {
                        sel_ok = src >= 0;
                        sel_ew = e;
                    }
                } else if (wave == 1 && blockIdx.x == 0 && blockIdx.y == 0) {
                    route_single_64(p.route, lane, route_keys[1], lr);
                }
                __syncthreads();
                if (!sel_ok) return;
                ew = sel_ew;
                n = 1;
                off = task;
            } else if (p.tasks) {
                const ExpertTask tk = p.tasks[task];
                if (tk.count == 0) return;
                n = tk.count;
                off = tk.offset;
                ew = tk.w;
            } else {
                if (task >= *p.n_unique) return;
                const int e = p.unique[task];
                n = p.counts[e];
                off = p.offsets[e];
                ew = p.experts[e];
            }
            list = p.route.logits ? nullptr : p.rows + off;  // inline: token row 0
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
        // blockIdx.y selects the task's token rows g0 .. g0 + B - 1
        const int g0 = blockIdx.y * B;
        if (g0 >= n) return;
        {
            job.rows = n - g0 < B ? n - g0 : B;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const int j = g0 + (b < job.rows ? b : 0);  // list entry
                const int token = shared || !list ? j : list[j];
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
                // pre-split rows: token rows (stage 0) or list / shared rows
                const long lrow = p.stage == 0 ? token : (shared ? j : off + j);
                job.limbs[b] = shared ? (p.sh_limbs ? p.sh_limbs + lrow * p.sh_limb_stride : nullptr)
                                      : (p.limbs ? p.limbs + lrow * p.limb_stride : nullptr);
            }
            if constexpr (kLimbX) {
                if (x_ready) {
                    limb_block<FMT, B, KT, LPR, R, KS, W, true>(job, gemv_lds);
                    return;
                }
            }
            run_job<MODE, FMT, B, KT, LPR, R, KS, W>(job, gemv_lds);
        }
    }
}

// Splits token rows of x (RMSNorm'ed with norm_w when set) into limb rows of
// the GEMV's LDS layout for format fmt: rows of segment a, then of segment b
// (b.rows may be 0), one workgroup per row.
struct LimbRowsParams {
    int fmt = kQ8, rows = 0, I = 0;
    const float *x = nullptr;
    long x_stride = 0;
    const float *norm_w = nullptr;
    float eps = 1e-5f;
    unsigned char *out = nullptr;
    long out_stride = 0;  // >= limb_row_lds(fmt, I)
};
int limb_quantise_rows(const LimbRowsParams &a, const LimbRowsParams &b, hipStream_t stream);

// Largest dynamic LDS a GEMV launch may ask for (the quantised x rows).
constexpr int kMaxGemvLds = 150 * 1024;
inline int gemv_lds_bytes_rt(int fmt, int b, int I) {
    return fmt == kF32 ? 0 : b * limb_row_lds(fmt, I);
}

// Launch geometry chosen by the host (see gemv.hip, plan_gemv).
struct GemvPlan {
    int b = 1, kt = 1, lpr = 64, r = 4, ks = 1;
    int waves = 4;  // per workgroup (8: plain q8 / q4 launches without k split)
};

// MODE 0 grids cover the plain matrix; MODE 1 callers pass their own grid.
template <int MODE, int FMT, int B, int KT, int LPR, int R, int KS, int W = 4>
static void launch_gemv(const GemvLaunch &L, dim3 grid, hipStream_t stream) {
    int max_I;
    if constexpr (MODE == 0) {
        const int per_block =
            rows_per_block<LPR, R, KS>(L.plain.epilogue == kEpiSiluDual) * (KS == 1 ? W / 4 : 1);
        grid = dim3((unsigned)((L.plain.O + per_block - 1) / per_block),
                    (unsigned)((L.plain.rows + B - 1) / B));
        max_I = L.plain.I;
    } else {
        const ExpertGemvParams &e = L.expert;
        max_I = e.stage == 0 ? e.hidden : (e.inter > e.shared_width ? e.inter : e.shared_width);
    }
    const int lds = gemv_lds_bytes<FMT, B>(max_I);
    if (lds > 64 * 1024) {
        static bool raised = false;  // per instantiation
        if (!raised) {
            (void)hipFuncSetAttribute(
                reinterpret_cast<const void *>(&gemv_kernel<MODE, FMT, B, KT, LPR, R, KS, W>),
                hipFuncAttributeMaxDynamicSharedMemorySize, kMaxGemvLds);
            raised = true;
        }
    }
    hipLaunchKernelGGL((gemv_kernel<MODE, FMT, B, KT, LPR, R, KS, W>), grid, dim3(W * 64), lds,
                       stream, L);
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
    if constexpr (MODE == 0 && FMT != kF32) {
        // 8-wave workgroups: half the per-row share of the x split
        if (plan.waves == 8) {
            if (plan.ks != 1) return false;
#define MLH_GEMV_W8(KT_, R_)                                                             \
            if (plan.kt == KT_ && plan.r == R_) {                                        \
                if constexpr (R_ * B <= 16) {                                            \
                    launch_gemv<MODE, FMT, B, KT_, 64, R_, 1, 8>(L, grid, stream);       \
                    return true;                                                         \
                }                                                                        \
            }
            MLH_GEMV_W8(1, 2) MLH_GEMV_W8(1, 4) MLH_GEMV_W8(2, 1) MLH_GEMV_W8(2, 2)
            MLH_GEMV_W8(2, 4)
#undef MLH_GEMV_W8
            return false;
        }
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
    MLH_GEMV_KT(2)
    if constexpr (FMT != kF32) { MLH_GEMV_KT(3) }
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

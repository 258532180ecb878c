// gemv_mfma.hip -- q8 / q4 dequant GEMV for 1..4 token rows on int8 matrix
// cores (gfx950: v_mfma_i32_16x16x64_i8).
//
// Semantics are those of gemv() (moonlight_kernels.metal:43-130 and the
// RMSNorm / residual / SwiGLU variants, :23-41, :533-541):
//     y[b, o] = s[o] * sum_i W[o, i] * x'[b, i],  x' = RMSNorm(x) or x.
//
// Numerics.  Each wave splits its quarter of the k range of every token row
// b into four int8 limbs against a power-of-two step 2^-e (chosen so that
// the wave's largest |x| maps below 2^30):
//     x ~= 2^-e * q,  q = rint(x * 2^e) = 2^24 L0 + 2^16 L1 + 2^8 L2 + L3,
// L0 in [-64, 64], L1..L3 in [-128, 127].  x * 2^e is exact in fp32, so the
// only rounding is rint's (at most half a step, and never more than fp32's
// own rounding of x for the wave's larger elements); the four limbs are the
// bytes of (q + 0x808080) ^ 0x808080 (split_limbs8).  The products of the
// stored weights with each limb are exact int32 sums on the matrix cores;
// the limbs are combined and scaled in fp32 once per wave, the four waves'
// shares added in fp32 and multiplied by the row scale.  q4 weights enter as
// the stored nibbles u = q + 8 (0..15); 8 * (sum of the limbs) comes off
// with one extra MFMA against a ones operand.  With RMSNorm the limbs are
// taken of x * norm_w and the 1 / rms factor is applied to the sum.
//
// Work decomposition.  A workgroup (4 waves) owns 16 output rows (16 gate +
// 16 up rows for SwiGLU); wave w takes the k quarter [w I / 4, (w + 1) I /
// 4).  A wave copies its weight rows of the quarter into its own LDS region
// by DMA (global_load_lds, 1 KB per instruction, contiguous row runs: 256
// bytes and more per row), loads and splits its x quarter meanwhile, then
// runs one MFMA per 64-k step: A = the x limbs (MFMA row 4 L + b), B = the
// 16 weight rows.  Only the final cross-wave sum meets in LDS (one
// barrier).  LDS rows of weights are XOR-swizzled in 16-byte chunks so the
// 16 rows an operand read touches hit distinct banks.
//
// Four kernels share that scheme:
//   gemv_mfma_kernel         the LDS-DMA form above (any k, 8 or 16 rows);
//   gemv_mfma_direct_kernel  k = 2048: a wave's 512-element quarter of each
//                            weight row goes straight into registers in the
//                            MFMA B layout (no LDS copy of the weights);
//   gemv_mfma_wide_kernel    one token row, k a multiple of 1024 above 4096,
//                            2048 or 4096 rows: k / 1024 waves per
//                            workgroup of 8 rows, the MFMA's 16 columns
//                            holding the 8 rows at two k slices;
//   gemv_mfma_splitk_kernel  other k > 4096 with at most 4096 rows:
//                            workgroups of (16-row block, 2048-wide k
//                            split); each stores its share, and the block's
//                            last-arriving workgroup adds the shares in
//                            split order and applies the epilogue.
// Every kernel also sums x^2 over its k range; a non-finite sum (a NaN or
// infinite x, which the int8 limbs cannot carry) makes the row's output NaN.
#include "mlh_device.h"
#include "mlh_host.h"

#include <type_traits>

namespace mlh {

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

// 16-byte global load the compiler does not track.  The compiler treats LDS
// DMA and register loads as one out-of-order counter and would wait for the
// whole DMA before the first use of a register loaded ahead of it; these
// loads instead complete in issue order before the DMA (memory reads return
// in order) and are waited for explicitly with wait_loaded<N>.  Nothing may
// touch their registers before that wait; tests/test_gemv_mfma_isa.py checks
// the compiled code for it.
__device__ __forceinline__ f32x4 load16_untracked(const float *p) {
    f32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}
// s_waitcnt vmcnt(N), tying v to it: uses of v cannot move above the wait.
template <int N>
__device__ __forceinline__ void wait_loaded(f32x4 &v) {
    asm volatile("s_waitcnt vmcnt(%1)" : "+v"(v) : "n"(N));
}

// dpp_wave_sum / dpp_wave_max: mlh_device.h.

constexpr int kRows = 16;         // output rows per workgroup
constexpr int kXPad = 64;         // bytes of padding per LDS limb row (bank spread)

// Byte position of element e (0..15) of a 16-element k slice in the limb
// rows: q4 nibble unpacking yields elements 0,2,4,6 | 1,3,5,7 | 8,10,12,14 |
// 9,11,13,15, and the limbs are stored in that order.
template <int FMT>
__device__ __forceinline__ int slice_pos(int e) {
    if constexpr (FMT == kQ4) return (e & 8) + ((e & 1) << 2) + ((e & 7) >> 1);
    return e;
}

// The four limbs of 8 elements of x (already scaled by the step's inverse),
// packed as the limb rows store them: lw[L][w] holds limb L of the elements
// at byte positions 4 w .. 4 w + 3 (slice_pos order).  The balanced base-256
// digits of q are the bytes of (q + 0x808080) ^ 0x808080: adding 128 to each
// of the three low digits makes them the plain bytes of the sum (each in
// 0..255), the xor takes the 128 off again in int8, and the top byte is L0.
// So an element costs a rounding, a conversion, an add and an xor, and a 4 x
// 4 byte transpose by v_perm_b32 gathers the limbs of 4 elements.
__device__ __forceinline__ void limb_transpose(unsigned e0, unsigned e1, unsigned e2, unsigned e3,
                                               unsigned &l0, unsigned &l1, unsigned &l2,
                                               unsigned &l3) {
    const unsigned a01 = __builtin_amdgcn_perm(e1, e0, 0x06020400u);  // e0.b0 e1.b0 e0.b2 e1.b2
    const unsigned b01 = __builtin_amdgcn_perm(e1, e0, 0x07030501u);  // e0.b1 e1.b1 e0.b3 e1.b3
    const unsigned a23 = __builtin_amdgcn_perm(e3, e2, 0x06020400u);
    const unsigned b23 = __builtin_amdgcn_perm(e3, e2, 0x07030501u);
    l3 = __builtin_amdgcn_perm(a23, a01, 0x05040100u);  // byte 0 of e0..e3
    l2 = __builtin_amdgcn_perm(b23, b01, 0x05040100u);  // byte 1
    l1 = __builtin_amdgcn_perm(a23, a01, 0x07060302u);  // byte 2
    l0 = __builtin_amdgcn_perm(b23, b01, 0x07060302u);  // byte 3
}
template <int FMT>
__device__ __forceinline__ void split_limbs8(const float (&v8)[8], float step_inv,
                                             unsigned (&lw)[4][2]) {
    unsigned e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        e[i] = (unsigned)((int)rintf(v8[i] * step_inv) + 0x808080) ^ 0x808080u;
    // q8: bytes in element order; q4: elements 0,2,4,6 | 1,3,5,7 (slice_pos)
    constexpr int i1 = FMT == kQ4 ? 2 : 1, i2 = FMT == kQ4 ? 4 : 2, i3 = FMT == kQ4 ? 6 : 3;
    constexpr int j0 = FMT == kQ4 ? 1 : 4, j1 = FMT == kQ4 ? 3 : 5, j2 = FMT == kQ4 ? 5 : 6, j3 = 7;
    limb_transpose(e[0], e[i1], e[i2], e[i3], lw[0][0], lw[1][0], lw[2][0], lw[3][0]);
    limb_transpose(e[j0], e[j1], e[j2], e[j3], lw[0][1], lw[1][1], lw[2][1], lw[3][1]);
}

// A token row whose x holds a NaN or an infinity (its sum of squares of x is
// not finite) cannot go through the limb split, which carries neither: its
// outputs are NaN.  The reference's fp32 dot (moonlight_kernels.metal:62-130)
// gives NaN there too, except where one sign of infinity meets only nonzero
// weights, which gives that infinity: never a finite value.  (A finite x
// whose squares overflow fp32, |x| > 1.8e19, is treated the same way.)
__device__ __forceinline__ float nonfinite_guard(float tss, float v) {
    return isfinite(tss) ? v : __builtin_nanf("");
}

struct MfmaGemvArgs {
    GemvParams p;
    int ndma;  // DMA instructions per wave (selects the instantiation)
    int rw;    // output rows per workgroup
};

// Router operands of wave 0 (one token row, p.router_parts set): lane e's
// router weights over the workgroup's RW output rows and the RMSNorm weight
// of lane n's row (loaded with the epilogue operands, used after the
// products).
template <int RW>
struct RouterOperands {
    f32x4 w[RW / 4];
    float nw;
};
template <int RW>
__device__ __forceinline__ RouterOperands<RW> load_router(const GemvParams &p, int lane, int row0,
                                                          int erc) {
    RouterOperands<RW> r;
    const int e = lane < p.router_experts ? lane : 0;
    const float *src = p.router_w + (long)e * p.O + row0;
#pragma unroll
    for (int i = 0; i < RW / 4; ++i) r.w[i] = load_f4(src + 4 * i);
    r.nw = p.router_nw[erc];
    return r;
}
// Wave 0 after the epilogue: lane n < RW holds output y of row row0 + n (0
// past O).  Writes this workgroup's router logit partials (sum over its rows
// of w[e, o] * y[o] * nw[o], in row order) and its sum of y^2 (row order).
// hw: LDS [2 * RW] of wave 0.
template <int RW>
__device__ __forceinline__ void store_router_parts(const GemvParams &p, int lane, float y,
                                                   const RouterOperands<RW> &r, float *hw) {
    if (lane < RW) {
        hw[lane] = y * r.nw;
        hw[RW + lane] = y * y;
    }
    // a wave's LDS accesses complete in issue order: the reads below see
    // every lane's store
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < RW / 4; ++i) {
        const f32x4 h = *reinterpret_cast<const f32x4 *>(hw + 4 * i);
        part = fmaf(r.w[i].x, h.x, part);
        part = fmaf(r.w[i].y, h.y, part);
        part = fmaf(r.w[i].z, h.z, part);
        part = fmaf(r.w[i].w, h.w, part);
    }
    const long n = gridDim.x;
    if (lane < p.router_experts) p.router_parts[(long)lane * n + blockIdx.x] = part;
    if (lane == 0) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < RW; ++i) ss += hw[RW + i];
        p.router_parts[(long)p.router_experts * n + blockIdx.x] = ss;
    }
}

// ND: DMA instructions per wave (a compile-time count, so that the wait for
// the x loads issued before them is exact); RW: output rows per workgroup
// (16, or 8 for wide-k matrices with few rows: twice the workgroups, the
// MFMA's weight columns 8..15 repeat 0..7 and are not stored)
template <int FMT, int B, bool DUAL, int ND, int RW = kRows>
struct MgShape {
    static constexpr int kNr = DUAL ? 2 * RW : RW;            // weight rows
    static constexpr int kKqb = ND * 1024 / kNr;              // weight bytes per row and wave
    static constexpr int kKq = FMT == kQ8 ? kKqb : 2 * kKqb;  // k elements per wave
    static constexpr int kI = 4 * kKq;
    static constexpr int kPass = (kKq + 511) / 512;          // x passes of 8 elements per lane
    static constexpr int kXrow = kKq + kXPad;
    static constexpr int kWaveLds = 4 * B * kXrow + kNr * kKqb;
    static constexpr int kNch = kKqb / 16;
    static constexpr int kSwz = kNch % 16 == 0 ? 15 : kNch % 8 == 0 ? 7 : kNch % 4 == 0 ? 3 : 0;
};

template <int FMT, int B, bool DUAL, int ND, int RW>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(MfmaGemvArgs a) {
    using Sh = MgShape<FMT, B, DUAL, ND, RW>;
    const GemvParams &p = a.p;
    extern __shared__ __attribute__((aligned(16))) unsigned char gm_lds[];
    __shared__ float red[4][4][2][B][RW];  // [wave][limb][gate / up][token row][row]
    __shared__ float red_ss[4][B];
    __shared__ __attribute__((aligned(16))) float router_hw[2 * RW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = blockIdx.x * RW;
    constexpr int row_bytes = FMT == kQ8 ? Sh::kI : Sh::kI / 2;
    constexpr int kq = Sh::kKq, kqb = Sh::kKqb, xrow = Sh::kXrow, swz = Sh::kSwz;
    const int k0 = wave * kq;
    unsigned char *xl = gm_lds + wave * Sh::kWaveLds;  // [4 limbs][B][xrow]
    unsigned char *wl = xl + 4 * B * xrow;              // [nr][kqb], 16-byte chunks swizzled

    // ---- 1. x of this wave's quarter (and norm_w): 8 elements per lane and
    // pass, all loads unconditional (norm_w absent: x itself, unused; a
    // conditional untracked load lets the register allocator copy its
    // destination before the wait), issued before the weight DMA so that the
    // wait for them leaves the DMA in flight
    constexpr int kMaxPass = Sh::kPass;
    const bool has_norm = p.norm_w != nullptr;
    const float *nw = has_norm ? p.norm_w : p.x;
    f32x4 xv[kMaxPass][B][2];
    f32x4 nv[kMaxPass][2];
#pragma unroll
    for (int j = 0; j < kMaxPass; ++j) {
        const int e = j * 512 + lane * 8;
        const int ec = e < kq ? e : 0;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float *xb = p.x + (long)b * p.x_stride + k0 + ec;
            xv[j][b][0] = load16_untracked(xb);
            xv[j][b][1] = load16_untracked(xb + 4);
        }
        nv[j][0] = load16_untracked(nw + k0 + ec);
        nv[j][1] = load16_untracked(nw + k0 + ec + 4);
    }
    // ---- 2. the weight rows of the quarter into LDS: instruction d writes
    // bytes [1024 d, 1024 d + 1024) of the region; lane i the 16 bytes of row
    // r = (1024 d + 16 i) / kqb, physical chunk c, which holds the row's
    // logical chunk c ^ (r & swz) (rows past O repeat row O - 1)
#pragma unroll
    for (int d = 0; d < ND; ++d) {
        const int f = 1024 * d + 16 * lane;
        const int r = f / kqb, c = (f % kqb) >> 4;
        const int logical = c ^ (r & swz);
        int orow = row0 + (DUAL ? (r & (RW - 1)) : r);
        orow = orow < p.O ? orow : p.O - 1;
        const uint8_t *base = (DUAL && r >= RW) ? p.w2 : p.w;
        const uint8_t *src = base + (long)orow * row_bytes + (FMT == kQ8 ? k0 : k0 / 2) + logical * 16;
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                         (__attribute__((address_space(3))) void *)(wl + 1024 * d),
                                         16, 0, 0);
    }
    // the x loads have landed once at most the ND DMA instructions are in flight
#pragma unroll
    for (int j = 0; j < kMaxPass; ++j) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            wait_loaded<ND>(xv[j][b][0]);
            wait_loaded<ND>(xv[j][b][1]);
        }
        wait_loaded<ND>(nv[j][0]);
        wait_loaded<ND>(nv[j][1]);
    }
    // ---- 3. split x into limbs in registers while the DMA is in flight (an
    // LDS store would wait for the DMA: the compiler cannot tell the regions
    // apart)
    float ss[B], amax[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        ss[b] = 0.0f;
        amax[b] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kMaxPass; ++j) {
        if (j * 512 + lane * 8 < kq) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    f32x4 v = xv[j][b][h];
                    ss[b] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                    if (has_norm) {
                        v.x *= nv[j][h].x;
                        v.y *= nv[j][h].y;
                        v.z *= nv[j][h].z;
                        v.w *= nv[j][h].w;
                    }
                    xv[j][b][h] = v;
                    amax[b] = fmaxf(amax[b], fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)),
                                                   fmaxf(fabsf(v.z), fabsf(v.w))));
                }
            }
        }
    }
    float step_inv[B], step[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        amax[b] = dpp_wave_max(amax[b]);
        ss[b] = dpp_wave_sum(ss[b]);
        // 2^e with amax * 2^e < 2^30 (amax = 0: any e; the limbs are 0)
        int e2 = 0;
        (void)frexpf(amax[b], &e2);  // amax < 2^e2
        const int ex = amax[b] > 0.0f ? 30 - e2 : 0;
        step_inv[b] = ldexpf(1.0f, ex);
        step[b] = ldexpf(1.0f, -ex);
    }
    // the 8 elements of a pass fill bytes e .. e + 7 of each limb row (q4: in
    // the slice order, elements 0,2,4,6 then 1,3,5,7 of the 8)
    unsigned lw[kMaxPass][B][4][2];
#pragma unroll
    for (int j = 0; j < kMaxPass; ++j) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float v8[8] = {xv[j][b][0].x, xv[j][b][0].y, xv[j][b][0].z, xv[j][b][0].w,
                                 xv[j][b][1].x, xv[j][b][1].y, xv[j][b][1].z, xv[j][b][1].w};
            // balanced base-256 digits: q = 2^24 L0 + 2^16 L1 + 2^8 L2 + L3
            split_limbs8<FMT>(v8, step_inv[b], lw[j][b]);
        }
    }
    // this wave's DMA has landed; no LDS access may be scheduled above the
    // wait (the compiler would wait for the DMA at the first one instead)
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_sched_barrier(0);
    // the epilogue's operands of lane 16 b + n (row row0 + n, token row b),
    // in flight during the products and the reduction
    const int er = row0 + (lane & 15), eb = lane >> 4 < B ? lane >> 4 : 0;
    const int erc = er < p.O ? er : p.O - 1;
    const bool has_res = p.epilogue == kEpiResidual;
    float e_s = 0.0f, e_s2 = 0.0f, e_res = 0.0f;
    const bool router = !DUAL && B == 1 && p.router_parts != nullptr;
    RouterOperands<RW> ro{};
    if (wave == 0) {
        e_s = p.s[erc];
        if (DUAL) e_s2 = p.s2[erc];
        if (has_res) e_res = p.resid[(long)eb * p.resid_stride + erc];
        if (router) ro = load_router<RW>(p, lane, row0, erc);
    }
#pragma unroll
    for (int j = 0; j < kMaxPass; ++j) {
        const int e = j * 512 + lane * 8;
        if (e < kq) {
#pragma unroll
            for (int b = 0; b < B; ++b)
#pragma unroll
                for (int L = 0; L < 4; ++L)
                    *reinterpret_cast<uint2 *>(xl + (L * B + b) * xrow + e) =
                        uint2{lw[j][b][L][0], lw[j][b][L][1]};
        }
    }
    // (a wave reads only its own LDS region: its LDS stores complete in order
    // before its reads below)

    // ---- 4. MFMA over the 64-k steps: A row m = 4 L + b (lane m = l % 16
    // supplies it), B column n = weight row l % 16; lane group g = l / 16
    // supplies k bytes 16 g .. 16 g + 15 of the step
    const int m = lane & 15, g = lane >> 4;
    const int limb = m >> 2, tb = m & 3;
    // (rows of b >= B repeat token row 0: their products are not used)
    const unsigned char *arow = xl + (limb * B + (tb < B ? tb : 0)) * xrow;
    const int n = lane & 15;
    const int wn = n & (RW - 1);  // weight row of MFMA column n
    const unsigned char *wrow = wl + wn * kqb;
    const unsigned char *wrow2 = wl + (RW + wn) * kqb;
    i32x4 acc = {0, 0, 0, 0}, acc2 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
    constexpr int nsteps = kq / 64;
    // steps in groups of 8 (and one group of the rest): the group's LDS
    // reads issued before its products
    using WRaw = typename std::conditional<FMT == kQ8, u32x4, uint2>::type;
    const i32x4 ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    auto group = [&](int s0, auto count) {
        constexpr int U = decltype(count)::value;
        u32x4 av[U];
        WRaw wv[U], uv[U];
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const int s = s0 + i;
            av[i] = *reinterpret_cast<const u32x4 *>(arow + 64 * s + 16 * g);
            if constexpr (FMT == kQ8) {
                const int lc = 4 * s + g;  // logical chunk
                wv[i] = *reinterpret_cast<const u32x4 *>(wrow + 16 * (lc ^ (wn & swz)));
                if constexpr (DUAL) uv[i] = *reinterpret_cast<const u32x4 *>(wrow2 + 16 * (lc ^ (wn & swz)));
            } else {
                const int lc = 2 * s + (g >> 1);  // logical chunk; 8-byte half g & 1
                wv[i] = *reinterpret_cast<const uint2 *>(wrow + 16 * (lc ^ (wn & swz)) + 8 * (g & 1));
                if constexpr (DUAL)
                    uv[i] = *reinterpret_cast<const uint2 *>(wrow2 + 16 * (lc ^ (wn & swz)) + 8 * (g & 1));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const i32x4 A = i32x4{(int)av[i].x, (int)av[i].y, (int)av[i].z, (int)av[i].w};
            i32x4 Bw, Bu;
            if constexpr (FMT == kQ8) {
                Bw = i32x4{(int)wv[i].x, (int)wv[i].y, (int)wv[i].z, (int)wv[i].w};
                if constexpr (DUAL) Bu = i32x4{(int)uv[i].x, (int)uv[i].y, (int)uv[i].z, (int)uv[i].w};
            } else {
                const uint2 w = wv[i];
                Bw = i32x4{(int)(w.x & 0x0F0F0F0Fu), (int)((w.x >> 4) & 0x0F0F0F0Fu),
                           (int)(w.y & 0x0F0F0F0Fu), (int)((w.y >> 4) & 0x0F0F0F0Fu)};
                if constexpr (DUAL) {
                    const uint2 u = uv[i];
                    Bu = i32x4{(int)(u.x & 0x0F0F0F0Fu), (int)((u.x >> 4) & 0x0F0F0F0Fu),
                               (int)(u.y & 0x0F0F0F0Fu), (int)((u.y >> 4) & 0x0F0F0F0Fu)};
                }
                acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, ones, acc1, 0, 0, 0);
            }
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bw, acc, 0, 0, 0);
            if constexpr (DUAL) acc2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bu, acc2, 0, 0, 0);
        }
    };
    for (int s0 = 0; s0 + 8 <= nsteps; s0 += 8) group(s0, std::integral_constant<int, 8>{});
    if constexpr (nsteps % 8 != 0) group(nsteps - nsteps % 8, std::integral_constant<int, nsteps % 8>{});
    // ---- 5. lane (g, n) holds limb g of token rows b = 0..3 (registers) for
    // weight row n: combine the limbs across the lane groups, scale
    const float limb_w = g == 0 ? 16777216.0f : g == 1 ? 65536.0f : g == 2 ? 256.0f : 1.0f;
#pragma unroll
    for (int b = 0; b < B; ++b) {
        int c = acc[b], c2 = DUAL ? acc2[b] : 0;
        if constexpr (FMT == kQ4) {
            c -= 8 * acc1[b];
            if (DUAL) c2 -= 8 * acc1[b];
        }
        if (n < RW) {
            red[wave][g][0][b][n] = (float)c * limb_w * step[b];
            if (DUAL) red[wave][g][1][b][n] = (float)c2 * limb_w * step[b];
        }
        if (lane == 0) red_ss[wave][b] = ss[b];
    }
    __syncthreads();
    // ---- 6. the shares of the four limbs and four waves (limbs, then waves,
    // in order) and the epilogue
    if (wave != 0) return;
    const int b = g;  // lanes 16 b + n, b < B
    const int row = row0 + n;
    float y_out = 0.0f;  // this lane's output, for the router partials
    if (g < B && n < RW && row < p.O) {
        float inv_rms = 1.0f;
        if (p.norm_w) {
            const float tot = (red_ss[0][b] + red_ss[1][b]) + (red_ss[2][b] + red_ss[3][b]);
            inv_rms = 1.0f / sqrtf(tot / (float)Sh::kI + p.eps);
        }
        auto total = [&](int u) {
            float w4[4];
#pragma unroll
            for (int w = 0; w < 4; ++w)
                w4[w] = (red[w][0][u][b][n] + red[w][1][u][b][n]) + (red[w][2][u][b][n] + red[w][3][u][b][n]);
            return ((w4[0] + w4[1]) + (w4[2] + w4[3])) * inv_rms;
        };
        const float tss = (red_ss[0][b] + red_ss[1][b]) + (red_ss[2][b] + red_ss[3][b]);
        const float sum = nonfinite_guard(tss, total(0) * e_s);
        const float sum2 = DUAL ? total(1) * e_s2 : 0.0f;
        float *yb = p.y + (long)b * p.y_stride;
        if (DUAL) {
            yb[row] = silu(sum) * sum2;
        } else {
            float out = sum;
            if (has_res) out = e_res + out;
            yb[row] = out;
            y_out = out;
        }
    }
    // the whole of wave 0, converged: the partials read every lane's output
    if (router) store_router_parts<RW>(p, lane, y_out, ro, router_hw);
}


// Weights straight into registers in the MFMA B layout, for matrices whose
// wave k range (KQ elements) fits in registers: no LDS copy of the weights
// (the LDS traffic of the DMA kernel's product phase is shared by every
// workgroup of a CU), and no LDS DMA, so every load is an ordinary one the
// compiler waits for where its registers are used.  Lane (g, n) loads weight
// row row0 + n in 16-byte pieces: q8 piece s = k bytes 64 s + 16 g (MFMA
// step s), q4 piece j = bytes 64 j + 16 g (steps 2 j and 2 j + 1, one 8-byte
// half each), so a wave instruction reads 64 contiguous bytes of each of 16
// rows; the limb rows are read at the same k positions.
template <int FMT, int B, bool DUAL, int KQ>
struct DirectLds {
    static constexpr int kXrow = KQ + kXPad;
    unsigned char xl[4][4 * B * kXrow];  // per wave: [4 limbs][B][xrow]
    float red[4][4][2][B][kRows];        // [wave][limb][gate / up][token row][row]
    float red_ss[4][B];
};

// One wave's share of a register-direct workgroup: the k range [k0, k0 +
// KQ) of the workgroup's 16 output rows.  Issues the x (and norm_w) loads,
// then the weight loads, then `epilogue_loads()` (the caller's operands, in
// flight during the split and the products); splits x into limbs; leaves the
// wave's limb-combined shares in L.red[wave] and its sum of squares of x in
// L.red_ss[wave].
template <int FMT, int B, bool DUAL, int KQ, typename EpilogueLoads>
__device__ __forceinline__ void direct_wave(const GemvParams &p, int row0, int k0,
                                            DirectLds<FMT, B, DUAL, KQ> &L,
                                            EpilogueLoads &&epilogue_loads) {
    constexpr int S = KQ / 64;                  // MFMA steps per wave
    constexpr int NW = FMT == kQ8 ? S : S / 2;  // 16-byte weight pieces per lane and matrix
    constexpr int kPass = (KQ + 511) / 512;
    constexpr int xrow = KQ + kXPad;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long row_bytes = FMT == kQ8 ? p.I : p.I / 2;
    unsigned char *xl = L.xl[wave];
    const int n = lane & 15, g = lane >> 4;

    // ---- x of this wave's k range (and norm_w), then the weights, then
    // the epilogue's operands: in-order completion lets the split start
    // while the weights are still in flight
    const bool has_norm = p.norm_w != nullptr;
    const float *nw = p.norm_w;  // loaded only with a norm
    f32x4 xv[kPass][B][2];
    f32x4 nv[kPass][2] = {};
#pragma unroll
    for (int j = 0; j < kPass; ++j) {
        const int e = j * 512 + lane * 8;
        const int ec = e < KQ ? e : 0;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float *xb = p.x + (long)b * p.x_stride + k0 + ec;
            xv[j][b][0] = load_f4(xb);
            xv[j][b][1] = load_f4(xb + 4);
        }
        if (has_norm) {
            nv[j][0] = load_f4(nw + k0 + ec);
            nv[j][1] = load_f4(nw + k0 + ec + 4);
        }
    }
    const int wr_row = row0 + n < p.O ? row0 + n : p.O - 1;
    const long w_off = (long)wr_row * row_bytes + (FMT == kQ8 ? k0 : k0 / 2) + 16 * g;
    u32x4 wv[NW], uv[DUAL ? NW : 1];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        wv[i] = load_global16(p.w + w_off + 64 * i);
        if constexpr (DUAL) uv[i] = load_global16(p.w2 + w_off + 64 * i);
    }
    epilogue_loads();

    // ---- split x into limbs (as gemv_mfma_kernel) and store the limb rows
    float ss[B], amax[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        ss[b] = 0.0f;
        amax[b] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kPass; ++j) {
        if (j * 512 + lane * 8 < KQ) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    f32x4 v = xv[j][b][h];
                    ss[b] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                    if (has_norm) {
                        v.x *= nv[j][h].x;
                        v.y *= nv[j][h].y;
                        v.z *= nv[j][h].z;
                        v.w *= nv[j][h].w;
                    }
                    xv[j][b][h] = v;
                    amax[b] = fmaxf(amax[b], fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)),
                                                   fmaxf(fabsf(v.z), fabsf(v.w))));
                }
            }
        }
    }
    float step_inv[B], step[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        amax[b] = dpp_wave_max(amax[b]);
        ss[b] = dpp_wave_sum(ss[b]);
        int e2 = 0;
        (void)frexpf(amax[b], &e2);  // amax < 2^e2
        const int ex = amax[b] > 0.0f ? 30 - e2 : 0;
        step_inv[b] = ldexpf(1.0f, ex);
        step[b] = ldexpf(1.0f, -ex);
    }
#pragma unroll
    for (int j = 0; j < kPass; ++j) {
        const int e = j * 512 + lane * 8;
        if (e < KQ) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const float v8[8] = {xv[j][b][0].x, xv[j][b][0].y, xv[j][b][0].z, xv[j][b][0].w,
                                     xv[j][b][1].x, xv[j][b][1].y, xv[j][b][1].z, xv[j][b][1].w};
                unsigned lw[4][2];
                split_limbs8<FMT>(v8, step_inv[b], lw);
#pragma unroll
                for (int Lb = 0; Lb < 4; ++Lb)
                    *reinterpret_cast<uint2 *>(xl + (Lb * B + b) * xrow + e) =
                        uint2{lw[Lb][0], lw[Lb][1]};
            }
        }
    }
    // (a wave reads only its own limb rows: its LDS stores complete in order
    // before its reads below)

    // ---- MFMA steps: A row m = 4 L + b from LDS (rows of b >= B repeat
    // token row 0: their products are not used), B column n from registers
    const int m = lane & 15;
    const int limb = m >> 2, tb = m & 3;
    const unsigned char *arow = xl + (limb * B + (tb < B ? tb : 0)) * xrow;
    i32x4 acc = {0, 0, 0, 0}, acc2 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
    const i32x4 ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    u32x4 av[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int aoff = FMT == kQ8 ? 64 * s + 16 * g : 128 * (s >> 1) + 32 * g + 16 * (s & 1);
        av[s] = *reinterpret_cast<const u32x4 *>(arow + aoff);
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const i32x4 A = i32x4{(int)av[s].x, (int)av[s].y, (int)av[s].z, (int)av[s].w};
        i32x4 Bw, Bu;
        if constexpr (FMT == kQ8) {
            Bw = i32x4{(int)wv[s].x, (int)wv[s].y, (int)wv[s].z, (int)wv[s].w};
            if constexpr (DUAL) Bu = i32x4{(int)uv[s].x, (int)uv[s].y, (int)uv[s].z, (int)uv[s].w};
        } else {
            const u32x4 w4 = wv[s >> 1];
            const unsigned wx = (s & 1) ? w4.z : w4.x, wy = (s & 1) ? w4.w : w4.y;
            Bw = i32x4{(int)(wx & 0x0F0F0F0Fu), (int)((wx >> 4) & 0x0F0F0F0Fu),
                       (int)(wy & 0x0F0F0F0Fu), (int)((wy >> 4) & 0x0F0F0F0Fu)};
            if constexpr (DUAL) {
                const u32x4 u4 = uv[s >> 1];
                const unsigned ux = (s & 1) ? u4.z : u4.x, uy = (s & 1) ? u4.w : u4.y;
                Bu = i32x4{(int)(ux & 0x0F0F0F0Fu), (int)((ux >> 4) & 0x0F0F0F0Fu),
                           (int)(uy & 0x0F0F0F0Fu), (int)((uy >> 4) & 0x0F0F0F0Fu)};
            }
            acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, ones, acc1, 0, 0, 0);
        }
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bw, acc, 0, 0, 0);
        if constexpr (DUAL) acc2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bu, acc2, 0, 0, 0);
    }
    // ---- limbs combined into the wave's shares
    const float limb_w = g == 0 ? 16777216.0f : g == 1 ? 65536.0f : g == 2 ? 256.0f : 1.0f;
#pragma unroll
    for (int b = 0; b < B; ++b) {
        int c = acc[b], c2 = DUAL ? acc2[b] : 0;
        if constexpr (FMT == kQ4) {
            c -= 8 * acc1[b];
            if (DUAL) c2 -= 8 * acc1[b];
        }
        L.red[wave][g][0][b][n] = (float)c * limb_w * step[b];
        if (DUAL) L.red[wave][g][1][b][n] = (float)c2 * limb_w * step[b];
        if (lane == 0) L.red_ss[wave][b] = ss[b];
    }
}

// Sum of the shares of the four limbs and four waves (limbs, then waves, in
// order) for output row n, token row b, matrix u (0, or 1 = up).
template <int FMT, int B, bool DUAL, int KQ>
__device__ __forceinline__ float direct_total(const DirectLds<FMT, B, DUAL, KQ> &L, int u, int b,
                                              int n) {
    float w4[4];
#pragma unroll
    for (int w = 0; w < 4; ++w)
        w4[w] = (L.red[w][0][u][b][n] + L.red[w][1][u][b][n]) +
                (L.red[w][2][u][b][n] + L.red[w][3][u][b][n]);
    return (w4[0] + w4[1]) + (w4[2] + w4[3]);
}

template <int FMT, int B, bool DUAL, int KQ>
__global__ __launch_bounds__(256) void gemv_mfma_direct_kernel(GemvParams p) {
    __shared__ __attribute__((aligned(16))) DirectLds<FMT, B, DUAL, KQ> L;
    __shared__ __attribute__((aligned(16))) float router_hw[2 * kRows];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = blockIdx.x * kRows;
    const int n = lane & 15, g = lane >> 4;
    const int wr_row = row0 + n < p.O ? row0 + n : p.O - 1;
    const int eb = g < B ? g : 0;
    const bool has_res = p.epilogue == kEpiResidual;
    const bool router = !DUAL && B == 1 && p.router_parts != nullptr;
    float e_s = 0.0f, e_s2 = 0.0f, e_res = 0.0f;
    RouterOperands<kRows> ro{};
    direct_wave<FMT, B, DUAL, KQ>(p, row0, wave * KQ, L, [&] {
        e_s = p.s[wr_row];
        e_s2 = DUAL ? p.s2[wr_row] : 0.0f;
        e_res = has_res ? p.resid[(long)eb * p.resid_stride + wr_row] : 0.0f;
        if (router && wave == 0) ro = load_router<kRows>(p, lane, row0, wr_row);
    });
    __syncthreads();
    if (wave != 0) return;
    const int b = g;
    const int row = row0 + n;
    float y_out = 0.0f;  // this lane's output, for the router partials
    if (g < B && row < p.O) {
        float inv_rms = 1.0f;
        if (p.norm_w) {
            const float tot = (L.red_ss[0][b] + L.red_ss[1][b]) + (L.red_ss[2][b] + L.red_ss[3][b]);
            inv_rms = 1.0f / sqrtf(tot / (float)p.I + p.eps);
        }
        const float tss = (L.red_ss[0][b] + L.red_ss[1][b]) + (L.red_ss[2][b] + L.red_ss[3][b]);
        const float sum = nonfinite_guard(tss, (direct_total(L, 0, b, n) * inv_rms) * e_s);
        const float sum2 = DUAL ? (direct_total(L, 1, b, n) * inv_rms) * e_s2 : 0.0f;
        float *yb = p.y + (long)b * p.y_stride;
        if (DUAL) {
            yb[row] = silu(sum) * sum2;
        } else {
            float out = sum;
            if (has_res) out = e_res + out;
            yb[row] = out;
            y_out = out;
        }
    }
    // the whole of wave 0, converged: the partials read every lane's output
    if (router) store_router_parts<kRows>(p, lane, y_out, ro, router_hw);
}

// Split-k form for wide-k matrices with few rows (2048 x 11264): workgroup
// (row block, split) takes 16 output rows and the k chunk [split * 4 KQ,
// (split + 1) * 4 KQ) (one KQ range per wave as in the direct kernel; waves
// past I contribute nothing), so every workgroup streams as many weight
// bytes as a 2048-wide direct workgroup and splits a quarter of x per wave
// instead of all of it.  Each workgroup stores its share of every output
// (and its sum of squares of x) in sk_part / sk_ss; the workgroup of a row
// block that arrives last (sk_count, agent_handoff_arrive; it resets the
// counter to zero) adds the shares of the splits in split order and
// applies the epilogue, so the result does not depend on arrival order.
// The partial arrays are the library's own device memory (static, per
// GPU): launches on one GPU must not overlap (the library issues all its
// work on one stream per device).
constexpr int kSkMaxSplits = 16;
constexpr int kSkMaxRowBlocks = 256;  // O <= 4096
constexpr int kSkCountStride = 32;    // ints between counters (one per 128 bytes)
__device__ float sk_part[kSkMaxRowBlocks * kSkMaxSplits * kMaxGemvRows * kRows];
__device__ float sk_ss[kSkMaxRowBlocks * kSkMaxSplits * kMaxGemvRows];
__device__ int sk_count[kSkMaxRowBlocks * kSkCountStride];  // zero between launches

template <int FMT, int B, int KQ>
__global__ __launch_bounds__(256) void gemv_mfma_splitk_kernel(GemvParams p) {
    __shared__ __attribute__((aligned(16))) DirectLds<FMT, B, false, KQ> L;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rb = blockIdx.x, split = blockIdx.y, splits = gridDim.y;
    const int row0 = rb * kRows;
    const int n = lane & 15, g = lane >> 4;
    const int wr_row = row0 + n < p.O ? row0 + n : p.O - 1;
    const int eb = g < B ? g : 0;
    const bool has_res = p.epilogue == kEpiResidual;
    const int k0 = (split * 4 + wave) * KQ;
    float e_s = 0.0f, e_res = 0.0f;
    if (k0 < p.I) {
        direct_wave<FMT, B, false, KQ>(p, row0, k0, L, [&] {
            e_s = p.s[wr_row];
            e_res = has_res ? p.resid[(long)eb * p.resid_stride + wr_row] : 0.0f;
        });
    } else {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            L.red[wave][g][0][b][n] = 0.0f;
            if (lane == 0) L.red_ss[wave][b] = 0.0f;
        }
        e_s = p.s[wr_row];
        e_res = has_res ? p.resid[(long)eb * p.resid_stride + wr_row] : 0.0f;
    }
    __syncthreads();
    // this workgroup's shares: lane (b, n) of wave 0
    const long pbase = ((long)rb * kSkMaxSplits + split) * B;
    if (wave == 0 && g < B) {
        __hip_atomic_store(&sk_part[(pbase + g) * kRows + n], direct_total(L, 0, g, n),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (n == 0)
            __hip_atomic_store(&sk_ss[pbase + g],
                               (L.red_ss[0][g] + L.red_ss[1][g]) + (L.red_ss[2][g] + L.red_ss[3][g]),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    int *count = sk_count + rb * kSkCountStride;
    if (!agent_handoff_arrive(count, splits) || wave != 0) return;
    const int b = g;
    const int row = row0 + n;
    if (g < B) {
        float sum = 0.0f, tot = 0.0f;
        for (int k = 0; k < splits; ++k) {
            const long pb = ((long)rb * kSkMaxSplits + k) * B + b;
            sum += __hip_atomic_load(&sk_part[pb * kRows + n], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
            tot += __hip_atomic_load(&sk_ss[pb], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (row < p.O) {
            const float inv_rms = p.norm_w ? 1.0f / sqrtf(tot / (float)p.I + p.eps) : 1.0f;
            float out = nonfinite_guard(tot, sum * inv_rms * e_s);
            if (has_res) out = e_res + out;
            p.y[(long)b * p.y_stride + row] = out;
        }
    }
    if (lane == 0) __hip_atomic_store(count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wide-k form with no sum across workgroups, for one token row, k a multiple
// of 1024 in (4096, 16384] and 2048 or 4096 rows (config 1's 2048 x 11264,
// the dense down projection at decode).  A workgroup of k / 1024 waves owns
// 8 output rows and the whole k range; wave w takes the columns [1024 w,
// 1024 w + 1024) as two slices of 512.  The matrix-core B operand's 16
// columns hold the 8 rows at both slices (column n: row n % 8, slice n / 8)
// and A row 4 L + h holds limb L of x's slice h, so C[4 L + h][8 h + r] is
// limb L's product of row r over slice h; the other products are not used.
// A wave streams 8 rows x 1024 columns, as many weight bytes as a wave of
// the direct kernel (16 rows x 512), and splits 1024 elements of x once
// (one power-of-two step for both slices).  The waves' row totals meet in
// LDS and wave 0 adds them in wave order.
constexpr int kWideRows = 8;
constexpr int kWideSlice = 512;
constexpr int kWideMaxWaves = 16;

struct WideLds {
    static constexpr int kXrow = kWideSlice + kXPad;
    unsigned char xl[kWideMaxWaves][4 * 2 * kXrow];  // per wave: [limb][slice][xrow]
    float red[kWideMaxWaves][kWideRows];
    float red_ss[kWideMaxWaves];
};

template <int FMT>
__global__ __launch_bounds__(1024) void gemv_mfma_wide_kernel(GemvParams p) {
    __shared__ __attribute__((aligned(16))) WideLds L;
    constexpr int S = kWideSlice / 64;          // MFMA steps per slice
    constexpr int NW = FMT == kQ8 ? S : S / 2;  // 16-byte weight pieces per lane
    constexpr int xrow = WideLds::kXrow;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const int row0 = blockIdx.x * kWideRows;
    const int n = lane & 15, g = lane >> 4;
    const int h = n >> 3;  // this lane's B column: row row0 + (n & 7) at slice h
    const int wrow = row0 + (n & 7) < p.O ? row0 + (n & 7) : p.O - 1;
    const int k0 = wave * 2 * kWideSlice;
    const long row_bytes = FMT == kQ8 ? p.I : p.I / 2;
    unsigned char *xl = L.xl[wave];

    // ---- x (and norm_w) of both slices, then the weights, then the
    // epilogue's operands: in-order completion lets the split start while
    // the weights are in flight
    const bool has_norm = p.norm_w != nullptr;
    const float *nw = p.norm_w;  // loaded only with a norm
    f32x4 xv[2][2], nv[2][2] = {};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int e = k0 + j * kWideSlice + lane * 8;
        xv[j][0] = load_f4(p.x + e);
        xv[j][1] = load_f4(p.x + e + 4);
        if (has_norm) {
            nv[j][0] = load_f4(nw + e);
            nv[j][1] = load_f4(nw + e + 4);
        }
    }
    const int kw = k0 + h * kWideSlice;
    const long w_off = (long)wrow * row_bytes + (FMT == kQ8 ? kw : kw / 2) + 16 * g;
    u32x4 wv[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) wv[i] = load_global16(p.w + w_off + 64 * i);
    const bool has_res = p.epilogue == kEpiResidual;
    float e_s = 0.0f, e_res = 0.0f;
    if (wave == 0) {
        e_s = p.s[wrow];
        e_res = has_res ? p.resid[wrow] : 0.0f;
    }

    // ---- split x into four limbs against one step for the wave's range
    float ss = 0.0f, amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            f32x4 v = xv[j][q];
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            if (has_norm) {
                v.x *= nv[j][q].x;
                v.y *= nv[j][q].y;
                v.z *= nv[j][q].z;
                v.w *= nv[j][q].w;
            }
            xv[j][q] = v;
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    }
    amax = dpp_wave_max(amax);
    ss = dpp_wave_sum(ss);
    int e2 = 0;
    (void)frexpf(amax, &e2);  // amax < 2^e2
    const int ex = amax > 0.0f ? 30 - e2 : 0;
    const float step_inv = ldexpf(1.0f, ex), step = ldexpf(1.0f, -ex);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float v8[8] = {xv[j][0].x, xv[j][0].y, xv[j][0].z, xv[j][0].w,
                             xv[j][1].x, xv[j][1].y, xv[j][1].z, xv[j][1].w};
        unsigned lw[4][2];
        split_limbs8<FMT>(v8, step_inv, lw);
#pragma unroll
        for (int Lb = 0; Lb < 4; ++Lb)
            *reinterpret_cast<uint2 *>(xl + (Lb * 2 + j) * xrow + lane * 8) = uint2{lw[Lb][0], lw[Lb][1]};
    }
    // (a wave reads only its own limb rows: its LDS stores complete in order
    // before its reads below)

    // ---- MFMA steps: A row m = 4 L + slice from LDS, B column n from
    // registers (A rows 4 L + 2 and 4 L + 3 repeat slice 0 and 1: their
    // products are not used)
    const int m = lane & 15;
    const unsigned char *arow = xl + ((m >> 2) * 2 + (m & 1)) * xrow;
    i32x4 acc = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
    const i32x4 ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    u32x4 av[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int aoff = FMT == kQ8 ? 64 * s + 16 * g : 128 * (s >> 1) + 32 * g + 16 * (s & 1);
        av[s] = *reinterpret_cast<const u32x4 *>(arow + aoff);
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const i32x4 A = i32x4{(int)av[s].x, (int)av[s].y, (int)av[s].z, (int)av[s].w};
        i32x4 Bw;
        if constexpr (FMT == kQ8) {
            Bw = i32x4{(int)wv[s].x, (int)wv[s].y, (int)wv[s].z, (int)wv[s].w};
        } else {
            const u32x4 w4 = wv[s >> 1];
            const unsigned wx = (s & 1) ? w4.z : w4.x, wy = (s & 1) ? w4.w : w4.y;
            Bw = i32x4{(int)(wx & 0x0F0F0F0Fu), (int)((wx >> 4) & 0x0F0F0F0Fu),
                       (int)(wy & 0x0F0F0F0Fu), (int)((wy >> 4) & 0x0F0F0F0Fu)};
            acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, ones, acc1, 0, 0, 0);
        }
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bw, acc, 0, 0, 0);
    }
    // ---- lane (g, n) holds limb g of slices 0..1 (registers 0..1) for
    // column n; its own product is slice h.  Limbs, then the two slices, are
    // added across lanes (each sum is commutative, so every lane of a row
    // ends with the same bits)
    int c = h ? acc[1] : acc[0];
    if constexpr (FMT == kQ4) c -= 8 * (h ? acc1[1] : acc1[0]);
    const float limb_w = g == 0 ? 16777216.0f : g == 1 ? 65536.0f : g == 2 ? 256.0f : 1.0f;
    float v = (float)c * limb_w * step;
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    v += __shfl_xor(v, 8);
    if (lane < kWideRows) L.red[wave][lane] = v;
    if (lane == 0) L.red_ss[wave] = ss;
    __syncthreads();
    if (wave != 0 || lane >= kWideRows || row0 + lane >= p.O) return;
    float tot = 0.0f, tss = 0.0f;
    for (int w = 0; w < nwaves; ++w) {
        tot += L.red[w][lane];
        tss += L.red_ss[w];
    }
    const float inv_rms = has_norm ? 1.0f / sqrtf(tss / (float)p.I + p.eps) : 1.0f;
    const float sum = nonfinite_guard(tss, (tot * inv_rms) * e_s);
    p.y[row0 + lane] = has_res ? e_res + sum : sum;
}

// The wide-k kernel takes p (one token row, k a multiple of 1024 in (4096,
// 16384], 2048 or 4096 rows: one or two workgroups per CU).  Measured on
// MI355X against the split-k kernel (same box, medians of graph replays):
// q4 2048 x 11264 6.10 against 7.42 us, q8 2048 x 11264 7.74 against 8.80,
// q4 2048 x 16384 7.13 against 8.69; q8 3000 x 7168 (375 workgroups, spread
// unevenly over the CUs) 8.52 against 8.28, which stays on split-k.
bool wide_ok(const GemvParams &p) {
    return (p.fmt == kQ8 || p.fmt == kQ4) && p.rows == 1 && p.epilogue != kEpiSiluDual &&
           !p.limbs && !p.router_parts && p.I > 4096 && p.I <= 1024 * kWideMaxWaves &&
           p.I % 1024 == 0 && (p.O == 2048 || p.O == 4096);
}
template <int FMT>
bool launch_wide(const GemvParams &p, hipStream_t stream, std::string *name) {
    if (name) {
        char buf[96];
        snprintf(buf, sizeof(buf), "mlh::(anonymous namespace)::gemv_mfma_wide_kernel<%d>", FMT);
        *name = buf;
        return true;
    }
    hipLaunchKernelGGL((gemv_mfma_wide_kernel<FMT>), dim3((p.O + kWideRows - 1) / kWideRows),
                       dim3(64 * (p.I / 1024)), 0, stream, p);
    return true;
}

template <int FMT, int B, bool DUAL, int KQ>
bool launch_direct(const GemvParams &p, hipStream_t stream, std::string *name) {
    if (name) {
        char buf[96];
        snprintf(buf, sizeof(buf), "mlh::(anonymous namespace)::gemv_mfma_direct_kernel<%d, %d, %s, %d>",
                 FMT, B, DUAL ? "true" : "false", KQ);
        *name = buf;
        return true;
    }
    hipLaunchKernelGGL((gemv_mfma_direct_kernel<FMT, B, DUAL, KQ>), dim3((p.O + kRows - 1) / kRows),
                       dim3(256), 0, stream, p);
    return true;
}
template <int FMT, bool DUAL>
bool launch_direct_b(const GemvParams &p, hipStream_t stream, std::string *name) {
    switch (p.rows) {
    case 1: return launch_direct<FMT, 1, DUAL, 512>(p, stream, name);
    case 2: return launch_direct<FMT, 2, DUAL, 512>(p, stream, name);
    case 4: return launch_direct<FMT, 4, DUAL, 512>(p, stream, name);
    default: return false;
    }
}

// Splits of 4 x 512 k per workgroup for the split-k kernel, or 0 when it
// does not take the shape.
constexpr int kSkQuarter = 512;
int splitk_splits(const GemvParams &p) {
    const int chunk = 4 * kSkQuarter;
    const int splits = (p.I + chunk - 1) / chunk;
    if ((p.fmt != kQ8 && p.fmt != kQ4) || p.epilogue == kEpiSiluDual || p.rows < 1 ||
        p.rows > 4 || p.rows == 3 || p.limbs || p.router_parts || p.I <= 4096 || p.O > 4096 ||
        p.I % kSkQuarter || splits > kSkMaxSplits || (p.O + kRows - 1) / kRows > kSkMaxRowBlocks)
        return 0;
    return splits;
}
template <int FMT, int B>
bool launch_splitk(const GemvParams &p, int splits, hipStream_t stream, std::string *name) {
    if (name) {
        char buf[96];
        snprintf(buf, sizeof(buf), "mlh::(anonymous namespace)::gemv_mfma_splitk_kernel<%d, %d, %d>",
                 FMT, B, kSkQuarter);
        *name = buf;
        return true;
    }
    hipLaunchKernelGGL((gemv_mfma_splitk_kernel<FMT, B, kSkQuarter>),
                       dim3((p.O + kRows - 1) / kRows, splits), dim3(256), 0, stream, p);
    return true;
}
template <int FMT>
bool launch_splitk_b(const GemvParams &p, int splits, hipStream_t stream, std::string *name) {
    switch (p.rows) {
    case 1: return launch_splitk<FMT, 1>(p, splits, stream, name);
    case 2: return launch_splitk<FMT, 2>(p, splits, stream, name);
    case 4: return launch_splitk<FMT, 4>(p, splits, stream, name);
    default: return false;
    }
}

// With `name` set nothing is launched: the kernel's template name is stored.
template <int FMT, int B, bool DUAL, int ND, int RW>
bool launch_one(const MfmaGemvArgs &a, hipStream_t stream, std::string *name) {
    using Sh = MgShape<FMT, B, DUAL, ND, RW>;
    // shapes whose x passes exceed the register budget are not instantiated
    // (the dynamic LDS plus the static reduction arrays within the 160 KB)
    if constexpr (Sh::kPass > (B == 1 ? 6 : B == 2 ? 3 : 2) || 4 * Sh::kWaveLds > 150 * 1024) {
        return false;
    } else {
    if (Sh::kI != a.p.I) return false;
    if (name) {
        char buf[96];
        snprintf(buf, sizeof(buf), "mlh::(anonymous namespace)::gemv_mfma_kernel<%d, %d, %s, %d, %d>",
                 FMT, B, DUAL ? "true" : "false", ND, RW);
        *name = buf;
        return true;
    }
    constexpr int lds = 4 * Sh::kWaveLds;
    static const bool attr = [] {
        if (lds <= 64 * 1024) return true;
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_mfma_kernel<FMT, B, DUAL, ND, RW>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, lds) == hipSuccess)
            return true;
        (void)hipGetLastError();  // not sticky: the caller falls back
        return false;
    }();
    if (!attr) return false;
    hipLaunchKernelGGL((gemv_mfma_kernel<FMT, B, DUAL, ND, RW>), dim3((a.p.O + RW - 1) / RW),
                       dim3(256), lds, stream, a);
    return true;
    }
}

// DMA counts of the Moonlight shapes: 16 or 32 rows x (I / 4) weight bytes
// per wave, I = 2048 or 11264; 8 rows at I = 11264
template <int FMT, int B, bool DUAL>
bool launch_nd(const MfmaGemvArgs &a, hipStream_t stream, std::string *name) {
    if (a.rw == 8) {
        if constexpr (DUAL || B != 1) {
            return false;
        } else {
            switch (a.ndma) {
            case 11: return launch_one<FMT, B, DUAL, 11, 8>(a, stream, name);
            case 22: return launch_one<FMT, B, DUAL, 22, 8>(a, stream, name);
            default: return false;
            }
        }
    }
    switch (a.ndma) {
    case 4: return launch_one<FMT, B, DUAL, 4, kRows>(a, stream, name);
    case 8: return launch_one<FMT, B, DUAL, 8, kRows>(a, stream, name);
    case 16: return launch_one<FMT, B, DUAL, 16, kRows>(a, stream, name);
    case 22: return launch_one<FMT, B, DUAL, 22, kRows>(a, stream, name);
    case 44: return launch_one<FMT, B, DUAL, 44, kRows>(a, stream, name);
    default: return false;
    }
}

template <int FMT, bool DUAL>
bool launch_b(const MfmaGemvArgs &a, hipStream_t stream, std::string *name) {
    switch (a.p.rows) {
    case 1: return launch_nd<FMT, 1, DUAL>(a, stream, name);
    case 2: return launch_nd<FMT, 2, DUAL>(a, stream, name);
    case 4: return launch_nd<FMT, 4, DUAL>(a, stream, name);
    default: return false;
    }
}

}  // namespace

// The matrix-core GEMV for the shapes it covers (q8 / q4, 1, 2 or 4 token
// rows, I a multiple of 256 (q8) or 512 (q4), aligned operands, no pre-split
// x); returns false, launching nothing, otherwise.  Measured on MI355X
// against the vector kernel (gemv_impl.h), graph replays: q4 11264 x 2048
// 5.27 against 5.95 us, q8 3648 x 2048 4.16 against 4.72 us, q8 11264 x 2048
// at 4 rows 9.9 against 12.7 us.  Wide-k matrices with few rows (2048 x
// 11264) take 8-row workgroups at one token row (256 workgroups rather than
// 128), else the vector kernel.  With `name` set it
// launches nothing and stores the template name of the kernel it would
// launch (operand alignment not checked).
// Output rows per workgroup when the matrix-core kernels take p (operand
// alignment checked when `aligned`), else 0.
static int mfma_rows(const GemvParams &p, bool aligned) {
    if ((p.fmt != kQ8 && p.fmt != kQ4) || p.rows < 1 || p.rows > 4 || p.rows == 3 || p.limbs)
        return 0;
    const bool dual = p.epilogue == kEpiSiluDual;
    const int rw = p.O < 4096 && p.I > 4096 ? 8 : kRows;
    if (rw == 8 && (dual || p.rows != 1)) return 0;
    const int max_pass = p.rows == 1 ? 6 : p.rows == 2 ? 3 : 2;
    if (p.I % (p.fmt == kQ8 ? 256 : 512) || p.I / 4 > max_pass * 512) return 0;
    auto al = [](const void *q) { return ((uintptr_t)q & 15u) == 0; };
    if (aligned && (!al(p.w) || (dual && !al(p.w2)) || !al(p.x) || p.x_stride % 4 ||
                    (p.norm_w && !al(p.norm_w))))
        return 0;
    return rw;
}

bool gemv_mfma(const GemvParams &p, hipStream_t stream, std::string *name);

bool gemv_router_ok(const GemvParams &p) {
    const int rw = mfma_rows(p, true);
    if (!(rw > 0 && p.rows == 1 && p.epilogue != kEpiSiluDual && p.O % rw == 0)) return false;
    // a kernel of the dispatch below exists for the shape (instantiated DMA
    // counts, register and LDS budgets): asked in name-only mode, which
    // launches nothing
    GemvParams q = p;
    q.router_parts = nullptr;
    std::string name;
    return splitk_splits(q) == 0 && !wide_ok(q) && gemv_mfma(q, nullptr, &name);
}

int gemv_router_parts(const GemvParams &p) {
    const int rw = mfma_rows(p, false);
    return rw > 0 ? p.O / rw : 0;
}

bool gemv_mfma(const GemvParams &p, hipStream_t stream, std::string *name) {
    auto al = [](const void *q) { return ((uintptr_t)q & 15u) == 0; };
    // wide-k matrices with few rows: at one token row and 2048 rows or more
    // the wide kernel, else the split-k kernel
    if (wide_ok(p)) {
        if (!name && (!al(p.w) || !al(p.x) || (p.norm_w && !al(p.norm_w)))) return false;
        return p.fmt == kQ8 ? launch_wide<kQ8>(p, stream, name) : launch_wide<kQ4>(p, stream, name);
    }
    if (const int splits = splitk_splits(p)) {
        if (!name && (!al(p.w) || !al(p.x) || p.x_stride % 4 || (p.norm_w && !al(p.norm_w))))
            return false;
        return p.fmt == kQ8 ? launch_splitk_b<kQ8>(p, splits, stream, name)
                            : launch_splitk_b<kQ4>(p, splits, stream, name);
    }
    const int rw = mfma_rows(p, !name);
    if (!rw) return false;
    const bool dual = p.epilogue == kEpiSiluDual;
    if (p.router_parts && !gemv_router_ok(p)) return false;
    // k quarters of 512: weights straight into registers, except q8 at one
    // token row (measured on MI355X, graph replays: q4 11264 x 2048 5.27 ->
    // 5.21 us, q8 at 4 rows 9.3 -> 8.6 us median, q8 at one row 6.43 -> 6.60
    // us, so that stays on the DMA kernel)
    if (p.I == 2048 && rw == kRows && !(p.fmt == kQ8 && p.rows == 1))
        return dual ? (p.fmt == kQ8 ? launch_direct_b<kQ8, true>(p, stream, name)
                                    : launch_direct_b<kQ4, true>(p, stream, name))
                    : (p.fmt == kQ8 ? launch_direct_b<kQ8, false>(p, stream, name)
                                    : launch_direct_b<kQ4, false>(p, stream, name));
    MfmaGemvArgs a;
    a.p = p;
    const int kqb = p.fmt == kQ8 ? p.I / 4 : p.I / 8;  // weight bytes per row and wave
    a.rw = rw;
    a.ndma = (dual ? 2 * rw : rw) * kqb / 1024;
    return dual ? (p.fmt == kQ8 ? launch_b<kQ8, true>(a, stream, name)
                                : launch_b<kQ4, true>(a, stream, name))
                : (p.fmt == kQ8 ? launch_b<kQ8, false>(a, stream, name)
                                : launch_b<kQ4, false>(a, stream, name));
}

}  // namespace mlh

// mla.hip -- compressed-MLA attention over the 512+64 latent KV cache (gfx950).
//
// References (c4pt0r/floyd):
//   cache append   moonlight_cache_append   (moonlight_kernels.metal:132-170)
//   query RoPE     moonlight_rope_query     (moonlight_kernels.metal:172-200)
//   absorb         moonlight_attention_absorb_query (moonlight_kernels.metal:218-245)
//   scores         moonlight_attention_scores       (moonlight_kernels.metal:247-282)
//   softmax + lc   moonlight_attention_latent_context (moonlight_kernels.metal:284-343)
//   value          moonlight_attention_decode_value (moonlight_kernels.metal:345-375)
//   orchestration  encode_attention_buffer  (moonlight_metal.m:287-440)
//
// Launches per decode attention call (groups of up to kMlaDecodeRows rows):
//   mla_prep    (row, cache-append | head x 128 latent columns): RMSNorm +
//               RoPE into the caches, RoPE of the query's rope part, and the
//               absorbed query qa_h = W_UK_h^T q_nope_h, each wave reading
//               128-column runs of 4 kv_b rows per instruction.
//   mla_attend  (split, row): a run of kMlaTileKeys-key tiles per workgroup;
//               every latent row read once scores ALL heads (the reference
//               re-reads the cache per head); per split a running max /
//               exp-sum and the partial latent context of every head.
//   mla_merge_value (row, head, kMlaValueDims latent dims): one-pass
//               log-sum-exp merge of the splits into that slice of lc_h,
//               its share of ctx_h = W_UV_h lc_h, and the sum of the shares
//               by the head's last workgroup.
// Prefill (more than one row, outside a captured graph) runs mla_prep for
// the cache and the query rope, then, for 64 rows or more, kv_b applied to
// every cached key (mla_expand) and a flash-attention kernel per head on the
// expanded keys and values (mla_flash); for fewer rows the absorb and value
// as per-head MFMA GEMMs around a flash-attention kernel in the absorbed
// form (mla_prefill_attend).
#include "mla.h"

#include "mlh_device.h"

namespace mlh {

// The attention call's first position: from device memory when the call is
// part of a replayed graph, else the launch argument.
__device__ __forceinline__ int mla_position(const MlaParams &p) {
    return p.position_dev ? *p.position_dev : p.position;
}

// The attention products take their fp32 operands as split-f16 pairs
// (split_f16), which need |v| < 65504; the reference's fp32 products have no
// such limit.  The kernels that write the operands (the cache rows, the
// query rope, the absorbed query) check every value and report a finite one
// outside the range through p.range_error instead of letting the products
// turn it into inf / NaN.  NaN and inf inputs propagate as in fp32.
constexpr float kSplitF16Max = 65504.0f;
// halves per row of an expanded value block (32 keys + 4 pad)
constexpr int kFlashVRow = 36;
__device__ __forceinline__ bool outside_f16(float v) {
    const float a = fabsf(v);
    return a >= kSplitF16Max && a < INFINITY;
}
// The f16 halves of one cache value as split_f16 (below) makes them: hi =
// x with its low 13 mantissa bits cleared, lo = f16(x - hi), as bits.
__device__ __forceinline__ void split_f16_bits(float x, uint16_t &hi, uint16_t &lo) {
    const float h = __uint_as_float(__float_as_uint(x) & 0xFFFFE000u);
    hi = __builtin_bit_cast(uint16_t, (_Float16)h);
    lo = __builtin_bit_cast(uint16_t, (_Float16)(x - h));
}

__device__ __forceinline__ void report_range(const MlaParams &p, bool bad) {
    if (bad && p.range_error && *p.range_error == 0) *p.range_error = p.range_code;
}

// Eight consecutive dequantised kv_b values w[row, col..col+7] (col % 8 ==
// 0), moonlight_weight_value (moonlight_kernels.metal:202-216) per element,
// in two steps for a format known at compile time: kvb_fetch8 issues the
// loads, kvb_decode8 dequantises, so a thread can have many rows in flight
// before it decodes the first (a run-time format switch would make every
// load wait before the next is issued).
template <int FMT> struct Kvb8 {
    f32x4 a, b;   // kF32
    uint2 q8;     // kQ8
    unsigned q4;  // kQ4
    float s;
};
template <int FMT>
__device__ __forceinline__ void kvb_fetch8(const MatrixRef &m, int row, int col, int width,
                                           Kvb8<FMT> &r) {
    if constexpr (FMT == kF32) {
        const float *p = reinterpret_cast<const float *>(m.w) + (long)row * width + col;
        r.a = load_f4(p);
        r.b = load_f4(p + 4);
    } else if constexpr (FMT == kQ8) {
        r.s = m.s[row];
        r.q8 = *reinterpret_cast<const uint2 *>(m.w + (long)row * width + col);
    } else {
        r.s = m.s[row];
        r.q4 = *reinterpret_cast<const unsigned *>(m.w + (long)row * ((width + 1) / 2) + col / 2);
    }
}
template <int FMT>
__device__ __forceinline__ void kvb_decode8(const Kvb8<FMT> &r, float (&out)[8]) {
    if constexpr (FMT == kF32) {
        out[0] = r.a.x; out[1] = r.a.y; out[2] = r.a.z; out[3] = r.a.w;
        out[4] = r.b.x; out[5] = r.b.y; out[6] = r.b.z; out[7] = r.b.w;
    } else if constexpr (FMT == kQ8) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[i] = (float)(int8_t)((r.q8.x >> (8 * i)) & 0xFF) * r.s;
            out[4 + i] = (float)(int8_t)((r.q8.y >> (8 * i)) & 0xFF) * r.s;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = (float)((int)((r.q4 >> (8 * i)) & 15) - 8) * r.s;
            out[2 * i + 1] = (float)((int)((r.q4 >> (8 * i + 4)) & 15) - 8) * r.s;
        }
    }
}

// grid (rows, 1 + heads * chunks), chunks = ceil(latent / 128): role 0
// appends the cache rows and ropes every head's query; role 1 + h * chunks
// + c absorbs head h's query into the latent columns 128 c .. 128 c + 127:
// qa_h[l] = sum_i q_nope[i] kv_b[h (nope + v) + i][l].  chunks = -1 (prefill,
// which absorbs by GEMM or not at all): grid (rows, 1), role 0 alone.
// (chunks = 0, grid (rows, 1 + heads): role 1 + h ropes head h's query.)  A wave instruction covers 4 nope rows x 128 columns
// (16 lanes per row, 8 columns per lane: contiguous row runs), wave w rows
// 4 (w + 4 j) .. + 3 for j = 0, 1, ...; a lane issues the loads of 8 rows
// before decoding any; the 4 lanes of a column set and the 4 waves meet by
// shuffles and LDS.
constexpr int kMlaAbsorbCols = 128;
template <int FMT>
__global__ __launch_bounds__(256) void mla_prep_kernel(MlaParams p, int chunks) {
    const int r = blockIdx.x;
    const int role = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int hw = p.nope + p.rope;
    const int half = p.rope / 2;
    if (role == 0) {
        __shared__ float part[4];
        const float *c = p.compressed + (long)r * p.compressed_stride;
        // loads first, unconditional (clamped): the compressed row, and with
        // the absorb (chunks > 0) the rope halves of every head's query,
        // pairs t and t + 256 of heads x rope / 2
        float cv[kMlaMaxLatent / 256];
#pragma unroll
        for (int u = 0; u < kMlaMaxLatent / 256; ++u) {
            const int i = t + 256 * u;
            const float v = c[i < p.latent ? i : 0];
            cv[u] = i < p.latent ? v : 0.0f;
        }
        constexpr int kQPairs = 2;
        static_assert(kMlaMaxHeads * 64 / 2 <= 256 * kQPairs, "rope pairs of every head");
        const int npair = chunks ? p.heads * half : 0;
        float q1[kQPairs], q2[kQPairs], fq[kQPairs];
#pragma unroll
        for (int k = 0; k < kQPairs; ++k) {
            const int j = t + 256 * k, jc = j < npair ? j : 0;
            const float *qh = p.query + (long)r * p.query_stride + (long)(jc / half) * hw + p.nope;
            q1[k] = qh[2 * (jc % half)];
            q2[k] = qh[2 * (jc % half) + 1];
            fq[k] = p.inv_freq[jc % half];
        }
        const int pos = mla_position(p) + r;
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < kMlaMaxLatent / 256; ++u) ss += cv[u] * cv[u];
        ss = wave_sum(ss);
        if (lane == 0) part[wave] = ss;
        __syncthreads();
        const float total = (part[0] + part[1]) + (part[2] + part[3]);
        const float inv = 1.0f / sqrtf(total / (float)p.latent + p.eps);
        float *lat = p.latent_cache + (long)pos * p.latent;
        uint16_t *lsp = p.latent_split + (long)pos * 2 * p.latent;
        bool bad = false;
#pragma unroll
        for (int u = 0; u < kMlaMaxLatent / 256; ++u) {
            const int i = t + 256 * u;
            if (i < p.latent) {
                const float v = cv[u] * inv * p.kv_norm[i];
                lat[i] = v;
                uint16_t hi, lo;
                split_f16_bits(v, hi, lo);
                lsp[i] = hi;
                lsp[p.latent + i] = lo;
                bad |= outside_f16(v);
            }
        }
        float *rp = p.rope_cache + (long)pos * p.rope;
        if (t < half) {
            const float angle = (float)pos * p.inv_freq[t];
            const float cs = cosf(angle), sn = sinf(angle);
            const float first = c[p.latent + 2 * t], second = c[p.latent + 2 * t + 1];
            const float a = first * cs - second * sn, b = second * cs + first * sn;
            rp[t] = a;
            rp[half + t] = b;
            bad |= outside_f16(a) || outside_f16(b);
        }
        // the query rope of every head (same angles as the key's)
#pragma unroll
        for (int k = 0; k < kQPairs; ++k) {
            const int j = t + 256 * k;
            if (j < npair) {
                const int hh = j / half, i = j % half;
                const float angle = (float)pos * fq[k];
                const float cs = cosf(angle), sn = sinf(angle);
                float *qr = p.query_rope + ((long)r * p.heads + hh) * p.rope;
                const float a = q1[k] * cs - q2[k] * sn, b = q2[k] * cs + q1[k] * sn;
                qr[i] = a;
                qr[half + i] = b;
                bad |= outside_f16(a) || outside_f16(b);
            }
        }
        report_range(p, bad);
        return;
    }
    // chunks == 0: the query rope only (prefill absorbs with mla_head_gemm);
    // with the absorb the query rope is role 0's
    const int h = chunks ? (role - 1) / chunks : role - 1;
    const int cc = chunks ? (role - 1) % chunks : 0;
    const float *q = p.query + (long)r * p.query_stride + (long)h * hw;
    if (!chunks && t < half) {
        const int pos = mla_position(p) + r;
        const float angle = (float)pos * p.inv_freq[t];
        const float cs = cosf(angle), sn = sinf(angle);
        const float first = q[p.nope + 2 * t], second = q[p.nope + 2 * t + 1];
        float *qr = p.query_rope + ((long)r * p.heads + h) * p.rope;
        const float a = first * cs - second * sn, b = second * cs + first * sn;
        qr[t] = a;
        qr[half + t] = b;
        report_range(p, outside_f16(a) || outside_f16(b));
    }
    if (!chunks) return;
    constexpr int kBatch = 8;  // wave instructions (4 rows each) in flight per lane
    __shared__ float red[4][kMlaAbsorbCols];
    const int sub = lane >> 4;                              // row within an instruction
    const int col = cc * kMlaAbsorbCols + 8 * (lane & 15);  // first of the lane's 8 columns
    const bool col_ok = col < p.latent;
    const int wrow = h * (p.nope + p.vdim);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int steps = (p.nope + 15) / 16;  // instructions per wave
    for (int j0 = 0; j0 < steps; j0 += kBatch) {
        Kvb8<FMT> raw[kBatch];
        float qc[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int i = 4 * (wave + 4 * (j0 + j)) + sub;  // nope row
            const bool ok = j0 + j < steps && i < p.nope;
            qc[j] = ok ? q[i] : 0.0f;
            kvb_fetch8<FMT>(p.kv_b, wrow + (ok ? i : 0), col_ok ? col : 0, p.latent, raw[j]);
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            float w[8];
            kvb_decode8<FMT>(raw[j], w);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(qc[j], w[e], acc[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        acc[e] += __shfl_xor(acc[e], 16, 64);
        acc[e] += __shfl_xor(acc[e], 32, 64);
    }
    if (sub == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) red[wave][8 * (lane & 15) + e] = acc[e];
    }
    __syncthreads();
    if (t < kMlaAbsorbCols && cc * kMlaAbsorbCols + t < p.latent) {
        const float v = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
        p.query_absorbed[((long)r * p.heads + h) * p.latent + cc * kMlaAbsorbCols + t] = v;
        report_range(p, outside_f16(v));
    }
}


// The keys before a row's own position in tiles of kMlaTileKeys, spread over
// `splits` workgroups per row (the reference's scores + softmax + latent
// context, moonlight_kernels.metal:247-343, per workgroup): with at most
// `splits` tiles workgroup b takes tile b, else tiles b * tiles / splits ..
// (b + 1) * tiles / splits - 1, so the merge finds min(tiles, splits)
// partials.  A workgroup keeps a running max / exp-sum per head across its
// tiles and writes one partial (max, sum, latent context of every head).
// The products run on the f16 matrix cores as split-f16 triples (split_f16:
// ~22-bit operands, fp32 accumulation, another order than the reference;
// measured against the oracle: the same rel-L2, 1.7-2.7e-6, as the former
// fp32 16x16x4 products), with fp32 operands in LDS and registers.  The
// row's own (new) key joins in mla_merge_value.  Per tile, all 8 waves:
//   scores  S[key][head] = [lat | rope][key] . [qa | q_rope][head]: wave w
//           takes the 32-dim steps w, w + 8, w + 16
//           (v_mfma_f32_16x16x32_f16; query slices split once, in
//           registers); the 8 partials meet in LDS.
//   softmax 16 lanes per head: tile max, running max, P = exp(S - max), the
//           rescale of the running sum and context.
//   context LC[head][d] += P[head][key] lat[key][d]: wave w takes the 16-wide
//           d tiles w, w + 8, w + 16, w + 24 (v_mfma_f32_16x16x16_f16 over
//           the tile's 16 keys).
// The rows of the next two tiles are in flight in registers (coalesced
// 16-byte loads) while a tile is in use, and go into LDS (two buffers) at
// the top of their step: three barriers per tile.  Loops have
// compile-time trip counts (steps past the latent + rope width multiply a
// zero query slice), so every LDS read of a phase is issued ahead of its
// MFMAs.
constexpr int kAttnDims = kMlaMaxLatent + 64;       // latent + rope
constexpr int kAttnRowStride = kAttnDims + 4;       // floats (16-byte aligned rows, banks spread)
constexpr int kAttnPStride = kMlaTileKeys + 4;      // floats, P[head][key]
constexpr int kAttnTileFloats = kMlaTileKeys * kAttnRowStride;
constexpr size_t kAttnMfmaLds =
    sizeof(float) * (2 * (size_t)kAttnTileFloats + 8 * kMlaTileKeys * kMlaMaxHeads +
                     kMlaMaxHeads * kAttnPStride);
static_assert(kMlaTileKeys == 16, "one 16-key MFMA tile per key tile");
static_assert(kMlaMaxLatent / 4 * kMlaTileKeys <= 4 * 512 && 64 / 4 * kMlaTileKeys <= 512,
              "a tile is at most 4 latent and 1 rope 16-byte loads per thread");

typedef float f32x4v __attribute__((ext_vector_type(4)));

// Sum / max over the 16 lanes of a DPP row, every lane receiving it (pairs
// exchanged symmetrically, so all lanes add in the same order).
#define MLH_DPP(v, ctrl) \
    __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), ctrl, 0xF, 0xF, false))
__device__ __forceinline__ float row16_sum(float v) {
    v += MLH_DPP(v, 0xB1);   // quad_perm [1,0,3,2]
    v += MLH_DPP(v, 0x4E);   // quad_perm [2,3,0,1]
    v += MLH_DPP(v, 0x141);  // row_half_mirror
    return v + MLH_DPP(v, 0x140);  // row_mirror
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, MLH_DPP(v, 0xB1));
    v = fmaxf(v, MLH_DPP(v, 0x4E));
    v = fmaxf(v, MLH_DPP(v, 0x141));
    return fmaxf(v, MLH_DPP(v, 0x140));
}
#undef MLH_DPP

// fp32 products on the f16 matrix cores: x = hi + lo with hi = x truncated
// to 11 significant bits and lo = f16(x - hi) (21 significant bits), and
// a.b ~ hi_a.hi_b + hi_a.lo_b + lo_a.hi_b in fp32 accumulation (the dropped
// lo_a.lo_b and the rounding of lo are ~2^-20 relative).  Values must lie
// inside the f16 range (|x| < 65504; a larger one turns the products to
// inf / NaN, not to a wrong finite
// value).  gfx950 operand layouts (measured): v_mfma_f32_16x16x32_f16 lane l
// supplies A[l % 16][8 (l / 16) .. + 7] and B[8 (l / 16) .. + 7][l % 16];
// v_mfma_f32_16x16x16_f16 A[l % 16][4 (l / 16) .. + 3] and B[4 (l / 16) ..
// + 3][l % 16]; both return D[4 (l / 16) + i][l % 16] in register i, as the
// fp32 16x16x4 instruction does.
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
// hi is x with its low 13 mantissa bits cleared (11 significant bits: exact
// in f16 for |x| in [2^-14, 65504)), lo = x - hi is exact in fp32 and
// rounded once to f16, so a split costs a mask, a subtraction and half of
// each of two packed conversions per value.
template <int N, typename V>
__device__ __forceinline__ void split_f16(const float (&x)[N], V &hi, V &lo) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float h = __uint_as_float(__float_as_uint(x[i]) & 0xFFFFE000u);
        hi[i] = (_Float16)h;
        lo[i] = (_Float16)(x[i] - h);
    }
}

__global__ __launch_bounds__(512) void mla_attend_mfma_kernel(MlaParams p) {
    constexpr int H = kMlaMaxHeads;
    constexpr int TK = kMlaTileKeys;
    constexpr int NS = (kAttnDims / 32 + 7) / 8;  // 32-dim score steps per wave
    constexpr int NT = kMlaMaxLatent / 16 / 8;    // 16-wide context tiles per wave
    constexpr int DL = kMlaValueDims;
    extern __shared__ __attribute__((aligned(16))) float attn_lds[];
    float *const buf0 = attn_lds;
    float *const buf1 = attn_lds + kAttnTileFloats;
    float *const sp = attn_lds + 2 * kAttnTileFloats;  // score partials [wave][key][head]
    float *const p_s = sp + 8 * TK * H;                // P [head][key]
    __shared__ float smax[H], ssum[H];
    __shared__ __attribute__((aligned(16))) float sscale[H];
    const int b = blockIdx.x, r = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int g = lane >> 4, m16 = lane & 15;
    const int D = p.latent, R = p.rope;
    const int KD = D + R;  // a multiple of 16 (launch condition)
    // the position first (memory reads complete in issue order)
    const int keys = mla_position(p) + r;  // the keys before row r's own
    const int tiles = (keys + TK - 1) / TK;
    const int G = p.splits;
    int t_begin = b, t_end = b < tiles ? b + 1 : b;
    if (tiles > G) {  // 32-bit products: b * tiles < 2^31 for any cache that fits in HBM
        t_begin = (int)((unsigned)(b * tiles) / (unsigned)G);
        t_end = (int)((unsigned)((b + 1) * tiles) / (unsigned)G);
    }
    if (t_begin >= t_end) return;  // no partial: the merge reads min(tiles, splits)
    if (t < H) {
        smax[t] = -INFINITY;
        ssum[t] = 0.0f;
    }
    // ---- tile rows through registers: 16-byte piece f = t + 512 u of the
    // latent part (key f / (D / 4)), piece t of the rope part (key t / (R /
    // 4)); pieces past the tile repeat a piece of the tile (the same value
    // stored twice), so loads and stores need no branches; keys past the
    // causal end load the last valid row (finite values, zero probability)
    const int D4 = D >> 2, R4 = R >> 2;
    int lkey[4], lcol[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int f = (t + 512 * u) % (TK * D4);
        lkey[u] = f / D4;
        lcol[u] = 4 * (f % D4);
    }
    const int rkey = (t % (TK * R4)) / R4, rcol = 4 * (t % R4);
    f32x4 la[4], ra, lb[4], rb;
    // a tile past the run loads the cache's first 16 bytes into every lane
    // (offsets masked, no branches: every path has the same loads in flight)
    auto load_tile = [&](int tile, f32x4 (&lr)[4], f32x4 &rr) {
        const long live = -(long)(tile < t_end);
        const int k0 = tile * TK, last = (keys - k0 < TK ? keys - k0 : TK) - 1;
#pragma unroll
        for (int u = 0; u < 4; ++u)  // the split row of a key: as many bytes as D floats
            lr[u] = load_f4(reinterpret_cast<const float *>(p.latent_split) +
                            (((long)(k0 + (lkey[u] < last ? lkey[u] : last)) * D + lcol[u]) & live));
        rr = load_f4(p.rope_cache + (((long)(k0 + (rkey < last ? rkey : last)) * R + rcol) & live));
    };
    auto store_tile = [&](float *buf, const f32x4 (&lr)[4], const f32x4 &rr) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            *reinterpret_cast<f32x4 *>(buf + lkey[u] * kAttnRowStride + lcol[u]) = lr[u];
        *reinterpret_cast<f32x4 *>(buf + rkey * kAttnRowStride + D + rcol) = rr;
    };
    load_tile(t_begin, la, ra);
    // ---- this wave's query slices, split into f16 halves: dims 32 (w + 8 j)
    // + 8 g .. + 7 of head m16 (D and KD are multiples of 16, so the 8 dims
    // lie in one part and wholly inside or past KD); absent heads read head
    // 0 (their outputs are unused), dims past KD are zero
    half8 qh8[NS], ql8[NS];
    {
        const long qh = (long)r * p.heads + (m16 < p.heads ? m16 : 0);
        const float *qa = p.query_absorbed + qh * D;
        const float *qr = p.query_rope + qh * R;
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            // branch-free: every slice loads (dims past KD reload dim 0)
            const int d = 32 * (wave + 8 * j) + 8 * g;
            const float *src = d < D ? qa + d : d < KD ? qr + (d - D) : qa;
            const f32x4 v0 = load_f4(src), v1 = load_f4(src + 4);
            const bool in = d < KD;
            const float x[8] = {in ? v0.x : 0.f, in ? v0.y : 0.f, in ? v0.z : 0.f, in ? v0.w : 0.f,
                                in ? v1.x : 0.f, in ? v1.y : 0.f, in ? v1.z : 0.f, in ? v1.w : 0.f};
            split_f16<8>(x, qh8[j], ql8[j]);
        }
    }
    // every load so far (query slices included) has landed: inside the tile
    // loop only prefetched rows are in flight, waited for at their store
    __builtin_amdgcn_s_waitcnt(0);
    f32x4v cacc[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) cacc[i] = f32x4v{0.f, 0.f, 0.f, 0.f};
    // one tile from its LDS buffer: scores, softmax, context
    auto process = [&](const float *cur, int tile) {
        const int nk = keys - tile * TK < TK ? keys - tile * TK : TK;
        // ---- scores: 32-dim steps w + 8 j on the f16 matrix cores (three
        // products each, two accumulator chains); a lane's 8 dims past KD
        // read row columns 0.. (finite) against a zero query slice
        {
            // latent dims: the cached halves (hi at half d, lo at half D + d
            // of the row); rope dims (d >= D, wave-uniform): fp32, split here
            half8 kh[NS], kl[NS];
            f32x4 av[NS][2];
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                const int d = 32 * (wave + 8 * j) + 8 * g;
                const float *row = cur + m16 * kAttnRowStride;
                if (d < D) {
                    const _Float16 *hr = reinterpret_cast<const _Float16 *>(row) + d;
                    kh[j] = *reinterpret_cast<const half8 *>(hr);
                    kl[j] = *reinterpret_cast<const half8 *>(hr + D);
                } else {
                    const float *rr = row + (d < KD ? d : D);
                    av[j][0] = *reinterpret_cast<const f32x4 *>(rr);
                    av[j][1] = *reinterpret_cast<const f32x4 *>(rr + 4);
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // all row reads issued before the products
            f32x4v a0 = f32x4v{0.f, 0.f, 0.f, 0.f}, a1 = a0;
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                if (32 * (wave + 8 * j) + 8 * g >= D) {
                    const float x[8] = {av[j][0].x, av[j][0].y, av[j][0].z, av[j][0].w,
                                        av[j][1].x, av[j][1].y, av[j][1].z, av[j][1].w};
                    split_f16<8>(x, kh[j], kl[j]);
                }
                a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[j], qh8[j], a0, 0, 0, 0);
                a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh[j], ql8[j], a1, 0, 0, 0);
                a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl[j], qh8[j], a0, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) sp[(wave * TK + 4 * g + i) * H + m16] = a0[i] + a1[i];
        }
        __syncthreads();
        // ---- softmax: 16 lanes (one DPP row) per head, one key each
        if (t < 256) {
            const int h = t >> 4, j = t & 15;
            const float *q = sp + j * H + h;
            const float s8 = ((q[0 * TK * H] + q[1 * TK * H]) + (q[2 * TK * H] + q[3 * TK * H])) +
                             ((q[4 * TK * H] + q[5 * TK * H]) + (q[6 * TK * H] + q[7 * TK * H]));
            const float s = j < nk ? s8 * p.scale : -INFINITY;
            const float mo = smax[h];
            const float mn = fmaxf(mo, row16_max(s));  // finite: key 0 of the tile is valid
            const float e = j < nk ? expf(s - mn) : 0.0f;
            p_s[h * kAttnPStride + j] = e;
            const float sum = row16_sum(e);
            if (j == 0) {
                const float f = expf(mo - mn);  // 0 on the first tile
                sscale[h] = f;
                ssum[h] = ssum[h] * f + sum;
                smax[h] = mn;
            }
        }
        __syncthreads();
        // ---- context: rescale, then P x lat for the wave's d tiles (tiles
        // past D read tile 0 and store nothing)
        {
            const f32x4 f = *reinterpret_cast<const f32x4 *>(sscale + 4 * g);
            const f32x4 pv = *reinterpret_cast<const f32x4 *>(p_s + m16 * kAttnPStride + 4 * g);
            // keys 4 g .. 4 g + 3 of latent dim col: the cached halves
            constexpr int RS = 2 * kAttnRowStride;  // halves per LDS row
            half4 bh[NT], bl[NT];
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                const int dt = wave + 8 * i;
                const int col = (dt < D / 16 ? dt : 0) * 16 + m16;
                const _Float16 *hb = reinterpret_cast<const _Float16 *>(cur) + (4 * g) * RS + col;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    bh[i][j] = hb[j * RS];
                    bl[i][j] = hb[j * RS + D];
                }
            }
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                cacc[i][0] *= f.x;
                cacc[i][1] *= f.y;
                cacc[i][2] *= f.z;
                cacc[i][3] *= f.w;
            }
            // P [head][keys 4 g ..] against lat [keys 4 g ..][d] on the f16
            // matrix cores (the same operands as four fp32 16x16x4 steps)
            const float pj[4] = {pv.x, pv.y, pv.z, pv.w};
            half4 ph, pl;
            split_f16<4>(pj, ph, pl);
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                cacc[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, bh[i], cacc[i], 0, 0, 0);
                cacc[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, bl[i], cacc[i], 0, 0, 0);
                cacc[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, bh[i], cacc[i], 0, 0, 0);
            }
        }
    };
    // two tiles in flight: register set A holds the even tiles of the run,
    // B the odd ones; a tile's rows go into its buffer at the top of its
    // step (the buffer was last read two steps before, ahead of this step's
    // first barrier), then the set loads the tile two ahead
    // (pairs of steps in a loop without a mid exit, an odd last tile after
    // it, so that the compiler sees the same loads in flight on every path)
    load_tile(t_begin + 1, lb, rb);
    int tile = t_begin;
    for (; tile + 1 < t_end; tile += 2) {
        store_tile(buf0, la, ra);
        __syncthreads();
        load_tile(tile + 2, la, ra);
        process(buf0, tile);
        store_tile(buf1, lb, rb);
        __syncthreads();
        load_tile(tile + 3, lb, rb);
        process(buf1, tile + 1);
    }
    if (tile < t_end) {
        store_tile(buf0, la, ra);
        __syncthreads();
        process(buf0, tile);
    }
    // ---- the partial: max / sum at [row][head][split], the latent context
    // at [row][head][chunk of DL dims][split][DL] (streaming stores: read
    // once, by the next launch; measured 1 us faster per call at ctx 4096)
    const int nc = D / DL;
    if (t < H) {
        const long at = ((long)r * H + t) * p.max_splits + b;
        p.part_max[at] = smax[t];
        p.part_sum[at] = ssum[t];
    }
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int dt = wave + 8 * i;
        if (dt < D / 16) {
            const int d = dt * 16 + m16;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int h = 4 * g + q;
                if (h < p.heads)
                    __builtin_nontemporal_store(
                        cacc[i][q],
                        p.part_lc + ((((long)r * H + h) * nc + d / DL) * p.max_splits + b) * DL + d % DL);
            }
        }
    }
}

// Four consecutive dequantised kv_b values w[row, col..col+3] (col % 4 == 0),
// moonlight_weight_value (moonlight_kernels.metal:202-216) per element.
__device__ __forceinline__ f32x4 kvb_load4(const MatrixRef &m, long row, int col, int width) {
    if (m.fmt == kF32) return load_f4(reinterpret_cast<const float *>(m.w) + row * width + col);
    const float s = m.s[row];
    if (m.fmt == kQ8) {
        const unsigned v = *reinterpret_cast<const unsigned *>(m.w + row * width + col);
        return f32x4{(float)(int8_t)(v & 0xFF) * s, (float)(int8_t)((v >> 8) & 0xFF) * s,
                     (float)(int8_t)((v >> 16) & 0xFF) * s, (float)(int8_t)(v >> 24) * s};
    }
    const unsigned v =
        *reinterpret_cast<const unsigned short *>(m.w + row * ((width + 1) / 2) + col / 2);
    return f32x4{(float)((int)(v & 15) - 8) * s, (float)((int)((v >> 4) & 15) - 8) * s,
                 (float)((int)((v >> 8) & 15) - 8) * s, (float)((int)((v >> 12) & 15) - 8) * s};
}

// Per-head products of the prefill path on fp32 MFMA (16x16x4), kv_b
// dequantised on its way into LDS:
//   ABSORB (moonlight_attention_absorb_query, moonlight_kernels.metal:218-245):
//     qa[r][h][n] = sum_k q_nope[r][h][k] kv_b[h (nope + v) + k][n]   K = nope, N = latent
//   value (moonlight_attention_decode_value, :345-375):
//     ctx[r][h][n] = sum_k lc[r][h][k] kv_b[h (nope + v) + nope + n][k] K = latent, N = vdim
// Workgroup: 64 token rows x 64 outputs of one head (grid z); wave w owns
// rows 16 w .. + 15 as four 16 x 16 tiles; k in steps of 16 through LDS, the
// next step's loads in flight during the MFMAs.  fp32 products and sums, in
// another order than the per-row kernels.
template <bool ABSORB>
__global__ __launch_bounds__(256) void mla_head_gemm_kernel(MlaParams p) {
    constexpr int BM = 64, BK = 16, LS = BK + 4;
    __shared__ __attribute__((aligned(16))) float xs[BM][LS];
    __shared__ __attribute__((aligned(16))) float ws[64][LS];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int g = lane >> 4, m16 = lane & 15;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * 64, h = blockIdx.z;
    const int K = ABSORB ? p.nope : p.latent;
    const int N = ABSORB ? p.latent : p.vdim;
    const long wrow0 = (long)h * (p.nope + p.vdim) + (ABSORB ? 0 : p.nope);
    // staging: thread t copies x[m0 + t / 4][k0 + 4 (t % 4) .. + 3] and 4 weights
    const int xr = t >> 2, xc = 4 * (t & 3);
    const long xrow = m0 + xr < p.rows ? m0 + xr : p.rows - 1;  // past the end: loaded, unused
    const float *xsrc = ABSORB ? p.query + xrow * p.query_stride + (long)h * (p.nope + p.rope)
                               : p.latent_context + (xrow * p.heads + h) * p.latent;
    f32x4 xv, wv;
    auto fetch = [&](int k0) {
        xv = load_f4(xsrc + k0 + xc);
        if constexpr (ABSORB) {  // 4 outputs n of one k: a kv_b row segment
            const int n = n0 + 4 * (t & 15);
            wv = kvb_load4(p.kv_b, wrow0 + k0 + (t >> 4), n + 4 <= N ? n : N - 4, p.latent);
        } else {  // 4 k of one output n: a kv_b row segment
            const int n = n0 + (t >> 2) < N ? n0 + (t >> 2) : N - 1;
            wv = kvb_load4(p.kv_b, wrow0 + n, k0 + 4 * (t & 3), p.latent);
        }
    };
    auto stash = [&]() {
        *reinterpret_cast<f32x4 *>(&xs[xr][xc]) = xv;
        if constexpr (ABSORB) {
            const int k = t >> 4, n = 4 * (t & 15);
            ws[n][k] = wv.x;
            ws[n + 1][k] = wv.y;
            ws[n + 2][k] = wv.z;
            ws[n + 3][k] = wv.w;
        } else {
            *reinterpret_cast<f32x4 *>(&ws[t >> 2][4 * (t & 3)]) = wv;
        }
    };
    f32x4v acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = f32x4v{0.f, 0.f, 0.f, 0.f};
    fetch(0);
    for (int k0 = 0; k0 < K; k0 += BK) {
        __syncthreads();  // the previous step's LDS reads are done
        stash();
        __syncthreads();
        if (k0 + BK < K) fetch(k0 + BK);
        const f32x4 a = *reinterpret_cast<const f32x4 *>(&xs[16 * wave + m16][4 * g]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f32x4 b = *reinterpret_cast<const f32x4 *>(&ws[16 * q + m16][4 * g]);
            acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, acc[q], 0, 0, 0);
            acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, acc[q], 0, 0, 0);
            acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, acc[q], 0, 0, 0);
            acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, acc[q], 0, 0, 0);
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int n = n0 + 16 * q + m16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long r = m0 + 16 * wave + 4 * g + i;
            if (r < p.rows && n < N) {
                if constexpr (ABSORB) {
                    p.query_absorbed[(r * p.heads + h) * p.latent + n] = acc[q][i];
                    report_range(p, outside_f16(acc[q][i]));
                } else
                    p.context[(r * p.heads + h) * p.vdim + n] = acc[q][i];
            }
        }
    }
}

// ---- expanded per-head keys and values (prefill of many rows)
// For every cached key and head, kv_b applied to the latent row once:
// k_nope (nope dims) and the value (vdim dims), as the f16 halves of
// mla_flash_kernel's split-f16 operands, in the layout its LDS tiles take
// by straight copies.  Per head h, from kv_expanded:
//   keys:   [h][key][KROW]  hi of dims 0 .. QKP - 1, then lo, then 8 pad
//           (dims: k_nope, the key's rope, zeros up to QKP = nope + rope
//           rounded up to 32)
//   values: after every head's keys, [h][key / 32][hi, lo][vdim][VROW],
//           the 32 keys of a block consecutive for each value dim, 4 pad
// The pads put consecutive rows of a tile on different LDS banks.
struct ExpandLayout {
    int qkp, krow, vdim;
    long keys;  // capacity (a multiple of 64)
    __host__ __device__ ExpandLayout(const MlaParams &p)
        : qkp((p.nope + p.rope + 31) / 32 * 32), krow(2 * qkp + 8), vdim(p.vdim),
          keys(p.expand_keys) {}
    __host__ __device__ long key_row(int h, long key) const { return ((long)h * keys + key) * krow; }
    // value block (hi, lo halves) of keys 32 b .. 32 b + 31
    __host__ __device__ long value_block(int heads, int h, long b) const {
        return (long)heads * keys * krow + (((long)h * (keys / 32) + b) * 2) * vdim * kFlashVRow;
    }
};

// The split halves of four consecutive values as two 8-byte stores.
__device__ __forceinline__ void store_split4(uint16_t *hi, uint16_t *lo, const float (&v)[4]) {
    ushort4 h4, l4;
    split_f16_bits(v[0], h4.x, l4.x);
    split_f16_bits(v[1], h4.y, l4.y);
    split_f16_bits(v[2], h4.z, l4.z);
    split_f16_bits(v[3], h4.w, l4.w);
    *reinterpret_cast<ushort4 *>(hi) = h4;
    *reinterpret_cast<ushort4 *>(lo) = l4;
}

// The rope and padding dims (nope .. QKP - 1) of the key rows m0 .. m0 + 63
// for head h: the key's rope values, zeros past rope or nrows.
__device__ __forceinline__ void expand_rope(const MlaParams &p, int h, long m0, long nrows,
                                            int t, bool &bad) {
    const ExpandLayout L(p);
    const int w4 = (L.qkp - p.nope) / 4;  // 4-dim groups a row
    for (int i = t; i < 64 * w4; i += 256) {
        const long key = m0 + i / w4;
        const int d = 4 * (i % w4);  // rope dim of the group
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (key < nrows && d < p.rope) {
            const f32x4 x = load_f4(p.rope_cache + key * p.rope + d);
            v[0] = x.x, v[1] = x.y, v[2] = x.z, v[3] = x.w;
        }
        uint16_t *row = p.kv_expanded + L.key_row(h, key) + p.nope + d;
        store_split4(row, row + L.qkp, v);
#pragma unroll
        for (int j = 0; j < 4; ++j) bad |= outside_f16(v[j]);
    }
}

// The same products on the f16 matrix cores for q8 / q4 kv_b.  The stored
// integers are exact in f16, so an fp32 activation x costs two products
// instead of one fp32 MFMA at a sixteenth of the rate: hi = x with its low
// 13 mantissa bits cleared (exact in f16) and lo' = f16((x - hi) 2^11) go
// into two accumulators, combined as acc_hi + 2^-11 acc_lo (lo' scaled up
// keeps lo out of f16's subnormal range, where it would lose its bits for
// small x).  kv_b's per-row scale goes with the activation in the absorb
// (its rows are the contraction index), divided by the head's largest scale
// so that the activation stays near the magnitude of q (that scale multiplies
// the result), and onto the sum in the value projection (its rows are the
// outputs):
//   absorb: qa[r][h][n] = smax sum_k (q_nope[r][h][k] s[h (nope + v) + k] / smax) w[h (nope + v) + k][n]
//   value:  ctx[r][h][n] = s[h (nope + v) + nope + n] sum_k lc[r][h][k] w[h (nope + v) + nope + n][k]
// Workgroup: 64 token rows x 64 outputs of one head (grid z); wave w: rows
// 16 w .. + 15 against four 16-output tiles, KS steps of 32 k on
// v_mfma_f32_16x16x32_f16 (lane (m16, g) supplies A[m16][8 g .. + 7] and
// B[8 g .. + 7][m16]; D[4 g + i][m16] in register i).  The workgroup's
// weights go into LDS once, [output][k]: the value projection's rows as
// int8, as they are stored (8 k of one output are one 8-byte read,
// converted at each use); the absorb's [k][output] block transposed through
// registers, 8 values of a row a thread, and stored as f16 (its few steps
// are read by four waves, so the conversion is done once).  A wave reads
// its own activation rows from global memory, D steps ahead (the absorb:
// all at once).  Measured on MI355X (2048-token prefill, kernel trace):
// value 53.5 -> 40.0 us with the int8 LDS rows instead of every wave
// loading its weights; the absorb's block transposed by v_perm_b32 in 4 x 4
// byte blocks took 50.5 us as int8 rows and 48.9 as f16 rows, against 46.3
// for the 8-value rows kept here.
enum HeadGemmMode { kHgAbsorb, kHgValue };
template <int MODE, int FMT, int KS>
__global__ __launch_bounds__(256) void mla_head_gemm_f16_kernel(MlaParams p) {
    constexpr bool ABSORB = MODE == kHgAbsorb;
    constexpr int BK = 32, K = KS * BK;
    constexpr int D = ABSORB ? KS : (KS < 4 ? KS : 4);  // steps in flight
    // LDS weights [output][k]: the absorb's as f16 (K + 8 halves a row), the
    // value's as int8 (K + 16 bytes a row; converted at each use)
    constexpr int WB = ABSORB ? 2 * (K + 8) : K + 16;
    __shared__ __attribute__((aligned(16))) int8_t wt[64][WB];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int g = lane >> 4, m16 = lane & 15;
    const int m0 = blockIdx.x * 64, n0 = blockIdx.y * 64, h = blockIdx.z;
    const int N = ABSORB ? p.latent : p.vdim;
    const long wrow0 = (long)h * (p.nope + p.vdim) + (MODE == kHgValue ? p.nope : 0);
    const long rbytes = FMT == kQ8 ? p.latent : p.latent / 2;  // bytes per kv_b row
    // this lane's activation row (rows past the end load the last, unused)
    const long r = m0 + 16 * wave + m16 < p.rows ? m0 + 16 * wave + m16 : p.rows - 1;
    const float *xrow = ABSORB ? p.query + r * p.query_stride + (long)h * (p.nope + p.rope)
                               : p.latent_context + (r * p.heads + h) * p.latent;
    struct Step {
        f32x4 x0, x1, s0, s1;
    };
    Step st[KS];
    auto load = [&](int j) {
        const int k0 = j * BK + 8 * g;
        st[j].x0 = load_f4(xrow + k0);
        st[j].x1 = load_f4(xrow + k0 + 4);
        if constexpr (ABSORB) {
            st[j].s0 = load_f4(p.kv_b.s + wrow0 + k0);
            st[j].s1 = load_f4(p.kv_b.s + wrow0 + k0 + 4);
        }
    };
    // four stored integers (q8 bytes, or q4 nibbles of 2 bytes) as int8 bytes
    auto int8x4 = [](const uint8_t *src) -> unsigned {
        if constexpr (FMT == kQ8) {
            return *reinterpret_cast<const unsigned *>(src);
        } else {
            const unsigned v = *reinterpret_cast<const unsigned short *>(src);
            unsigned o = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) o |= (unsigned)(((int)((v >> (4 * i)) & 15) - 8) & 0xFF) << (8 * i);
            return o;
        }
    };
#pragma unroll
    for (int j = 0; j < D; ++j) load(j);
    // ---- the weights into LDS, [output][k]
    if constexpr (ABSORB) {
        // thread t: rows k = t / 8 + 32 u of the [K][64] block, columns
        // n0 + 8 (t % 8) .. + 7, stored transposed as f16
        const int sk = t >> 3, sn = 8 * (t & 7);
        uint2 wv[KS];
#pragma unroll
        for (int u = 0; u < KS; ++u) {
            const uint8_t *src = p.kv_b.w + (wrow0 + sk + 32 * u) * rbytes;
            if constexpr (FMT == kQ8)
                wv[u] = *reinterpret_cast<const uint2 *>(src + n0 + sn);
            else
                wv[u] = uint2{*reinterpret_cast<const unsigned *>(src + (n0 + sn) / 2), 0u};
        }
#pragma unroll
        for (int u = 0; u < KS; ++u) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int v = FMT == kQ8 ? (int)(int8_t)(((i < 4 ? wv[u].x : wv[u].y) >> (8 * (i & 3))) & 0xFF)
                                         : (int)((wv[u].x >> (4 * i)) & 15) - 8;
                reinterpret_cast<_Float16 *>(&wt[sn + i][0])[sk + 32 * u] = (_Float16)v;
            }
        }
    } else {
        // 64 output rows of K bytes (q4: unpacked), 4 bytes per thread and pass
        constexpr int NW4 = 64 * K / 4;
#pragma unroll
        for (int i = t; i < NW4; i += 256) {
            const int row = i / (K / 4), c = 4 * (i % (K / 4));
            const int n = n0 + row < N ? n0 + row : N - 1;
            const uint8_t *src = p.kv_b.w + (wrow0 + n) * rbytes;
            *reinterpret_cast<unsigned *>(&wt[row][c]) = int8x4(src + (FMT == kQ8 ? c : c / 2));
        }
    }
    float smax = 1.0f, sinv = 1.0f;
    if constexpr (ABSORB) {  // the head's largest absorb-row scale (every wave)
        float m = 0.0f;
        for (int k = lane; k < K; k += 64) m = fmaxf(m, fabsf(p.kv_b.s[wrow0 + k]));
        m = wave_max(m);
        smax = m;
        sinv = m > 0.0f ? 1.0f / m : 0.0f;
    }
    __syncthreads();
    f32x4v acc[4], accl[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = accl[q] = f32x4v{0.f, 0.f, 0.f, 0.f};
    bool bad = false;
#pragma unroll
    for (int j = 0; j < KS; ++j) {
        if (j + D < KS) load(j + D);
        float x[8] = {st[j].x0.x, st[j].x0.y, st[j].x0.z, st[j].x0.w,
                      st[j].x1.x, st[j].x1.y, st[j].x1.z, st[j].x1.w};
        if constexpr (ABSORB) {
            const float sc[8] = {st[j].s0.x, st[j].s0.y, st[j].s0.z, st[j].s0.w,
                                 st[j].s1.x, st[j].s1.y, st[j].s1.z, st[j].s1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] *= sc[i] * sinv;
        }
        half8 ah, al;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            bad |= outside_f16(2.0f * x[i]);  // lo' below is at most 2 |x|
            const float hv = __uint_as_float(__float_as_uint(x[i]) & 0xFFFFE000u);
            ah[i] = (_Float16)hv;
            al[i] = (_Float16)((x[i] - hv) * 2048.0f);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            half8 b;
            if constexpr (ABSORB) {
                b = *reinterpret_cast<const half8 *>(&wt[16 * q + m16][2 * (j * BK + 8 * g)]);
            } else {
                const uint2 wb = *reinterpret_cast<const uint2 *>(&wt[16 * q + m16][j * BK + 8 * g]);
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    b[i] = (_Float16)(int8_t)(((i < 4 ? wb.x : wb.y) >> (8 * (i & 3))) & 0xFF);
            }
            acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, b, acc[q], 0, 0, 0);
            accl[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, b, accl[q], 0, 0, 0);
        }
    }
    report_range(p, bad);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int n = n0 + 16 * q + m16;
        const float sv = ABSORB ? smax : n < N ? p.kv_b.s[wrow0 + n] : 1.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long rr = m0 + 16 * wave + 4 * g + i;
            const float v = fmaf(accl[q][i], 1.0f / 2048.0f, acc[q][i]) * sv;
            if (rr < p.rows && n < N) {
                if constexpr (ABSORB) {
                    p.query_absorbed[(rr * p.heads + h) * p.latent + n] = v;
                    report_range(p, outside_f16(v));
                } else {
                    p.context[(rr * p.heads + h) * p.vdim + n] = v;
                }
            }
        }
    }
}

// The f16 head GEMM for K = KS * 32 (absorb: nope, value: latent); false
// when no instantiation covers K.
template <int MODE, int FMT>
bool launch_head_gemm_f16(const MlaParams &p, dim3 grid, hipStream_t stream) {
    const int K = MODE == kHgAbsorb ? p.nope : p.latent;
    if (K % 32) return false;
#define MLH_HG(KS)                                                                                 \
    case KS:                                                                                       \
        hipLaunchKernelGGL((mla_head_gemm_f16_kernel<MODE, FMT, KS>), grid, dim3(256), 0,          \
                           stream, p);                                                             \
        return true;
    if constexpr (MODE == kHgAbsorb) {  // nope <= 256
        switch (K / 32) {
            MLH_HG(1) MLH_HG(2) MLH_HG(4) MLH_HG(8)
        default: return false;
        }
    } else {  // latent: a multiple of 64, <= 512
        switch (K / 32) {
            MLH_HG(2) MLH_HG(4) MLH_HG(8) MLH_HG(16)
        default: return false;
        }
    }
#undef MLH_HG
}

// Expansion of the cached latent rows into the per-head keys and values of
// mla_flash_kernel (ExpandLayout), for every key 0 .. position + rows - 1:
//   kv[key][h][n] = s[h (nope + v) + n] sum_k lat[key][k] w[h (nope + v) + n][k]
// (n < nope: k_nope, else the value), on the f16 matrix cores as the head
// GEMMs do it (the integers exact in f16; the activation as hi and lo' =
// (x - hi) 2^11 in two accumulators).  Workgroup: 64 keys x every output of
// one head (nope + vdim <= 256 in tiles of 16; wave w takes tiles w, w + 4,
// ..), so each latent row is read and split once per head and the head's
// kv_b rows once per 64 keys.  Per chunk of 64 k the split keys and the
// weights converted to f16 go into LDS, the next chunk's loads in flight in
// registers meanwhile.  k_nope tiles take the weights as A (D[n][key]: four
// dims of one key a lane, one 8-byte store a half), value tiles the keys as
// A (D[key][n]: four keys of one value dim a lane, as the value blocks hold
// them); the workgroup also writes its keys' rope and padding dims.
constexpr int kExKC = 64;               // k per chunk
constexpr int kExARow = 2 * kExKC + 8;  // halves per key row in LDS (hi, lo', pad)
constexpr int kExBRow = kExKC + 8;      // halves per weight row in LDS
template <int FMT>
__global__ __launch_bounds__(256, 2) void mla_expand_kernel(MlaParams p) {
    __shared__ __attribute__((aligned(16))) _Float16 as[64 * kExARow];
    __shared__ __attribute__((aligned(16))) _Float16 bs[256 * kExBRow];
    const ExpandLayout L(p);
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int g = lane >> 4, m16 = lane & 15;
    const long m0 = (long)blockIdx.x * 64;
    const int h = blockIdx.y;
    const long nk = (long)mla_position(p) + p.rows;
    const int N = p.nope + p.vdim, NT = N / 16;
    const long wrow0 = (long)h * N;
    const long rbytes = FMT == kQ8 ? p.latent : p.latent / 2;  // bytes per kv_b row
    constexpr int NB = FMT == kQ8 ? 4 : 2;  // 16-byte weight pieces a thread and chunk
    f32x4 ra[4];
    uint4 rb[NB];
    // chunk c: latent float4 (t + 256 u) = key / 16, k 4 (% 16); weight
    // piece (t + 256 u) = row / (4 or 2), 16 bytes (% 4 or 2)
    auto load = [&](int c) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = t + 256 * u;
            const long key = m0 + idx / 16 < nk ? m0 + idx / 16 : nk - 1;
            ra[u] = load_f4(p.latent_cache + key * p.latent + kExKC * c + 4 * (idx % 16));
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int idx = t + 256 * u, row = idx / NB;
            const int n = row < N ? row : N - 1;
            rb[u] = *reinterpret_cast<const uint4 *>(p.kv_b.w + (wrow0 + n) * rbytes +
                                                     (FMT == kQ8 ? kExKC : kExKC / 2) * c +
                                                     16 * (idx % NB));
        }
    };
    bool bad = false;
    auto store = [&]() {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = t + 256 * u;
            const float x[4] = {ra[u].x, ra[u].y, ra[u].z, ra[u].w};
            half4 hv, lv;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                bad |= outside_f16(2.0f * x[i]);  // lo' is at most 2 |x|
                const float hx = __uint_as_float(__float_as_uint(x[i]) & 0xFFFFE000u);
                hv[i] = (_Float16)hx;
                lv[i] = (_Float16)((x[i] - hx) * 2048.0f);
            }
            _Float16 *dst = as + (idx / 16) * kExARow + 4 * (idx % 16);
            *reinterpret_cast<half4 *>(dst) = hv;
            *reinterpret_cast<half4 *>(dst + kExKC) = lv;
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int idx = t + 256 * u, row = idx / NB;
            if (row >= N) continue;
            const unsigned wv[4] = {rb[u].x, rb[u].y, rb[u].z, rb[u].w};
            _Float16 *dst = bs + row * kExBRow + (FMT == kQ8 ? 16 : 32) * (idx % NB);
#pragma unroll
            for (int v = 0; v < (FMT == kQ8 ? 2 : 4); ++v) {
                half8 o;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if constexpr (FMT == kQ8)
                        o[i] = (_Float16)(int8_t)((wv[2 * v + i / 4] >> (8 * (i & 3))) & 0xFF);
                    else
                        o[i] = (_Float16)((int)((wv[v] >> (4 * i)) & 15) - 8);
                }
                *reinterpret_cast<half8 *>(dst + 8 * v) = o;
            }
        }
    };
    f32x4v acc[4][4], accl[4][4];
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) acc[qq][mt] = accl[qq][mt] = f32x4v{0.f, 0.f, 0.f, 0.f};
    const int nch = p.latent / kExKC;
    load(0);
    for (int c = 0; c < nch; ++c) {
        if (c) __syncthreads();  // the previous chunk's LDS reads are done
        store();
        __syncthreads();
        if (c + 1 < nch) load(c + 1);
#pragma unroll
        for (int s2 = 0; s2 < kExKC / 32; ++s2) {
            half8 ah[4], al[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const _Float16 *src = as + (16 * mt + m16) * kExARow + 32 * s2 + 8 * g;
                ah[mt] = *reinterpret_cast<const half8 *>(src);
                al[mt] = *reinterpret_cast<const half8 *>(src + kExKC);
            }
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                const int q = wave + 4 * qq;
                if (q >= NT) continue;
                const half8 b =
                    *reinterpret_cast<const half8 *>(bs + (16 * q + m16) * kExBRow + 32 * s2 + 8 * g);
                if (16 * q < p.nope) {
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) {
                        acc[qq][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, ah[mt], acc[qq][mt], 0, 0, 0);
                        accl[qq][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, al[mt], accl[qq][mt], 0, 0, 0);
                    }
                } else {
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) {
                        acc[qq][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[mt], b, acc[qq][mt], 0, 0, 0);
                        accl[qq][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[mt], b, accl[qq][mt], 0, 0, 0);
                    }
                }
            }
        }
    }
    // ---- results into the expanded layout (keys from nk on: zeros)
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
        const int q = wave + 4 * qq, nq = 16 * q;
        if (q >= NT) continue;
        if (nq < p.nope) {  // D[n][key]: dims nq + 4 g .. + 3 of key m0 + 16 mt + m16
            const f32x4 sc = load_f4(p.kv_b.s + wrow0 + nq + 4 * g);
            const float s4[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const long key = m0 + 16 * mt + m16;
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[i] = key < nk ? fmaf(accl[qq][mt][i], 1.0f / 2048.0f, acc[qq][mt][i]) * s4[i] : 0.0f;
                    bad |= outside_f16(v[i]);
                }
                uint16_t *row = p.kv_expanded + L.key_row(h, key) + nq + 4 * g;
                store_split4(row, row + L.qkp, v);
            }
        } else {  // D[key][n]: keys m0 + 16 mt + 4 g .. + 3 of value dim nq + m16 - nope
            const int dv = nq + m16 - p.nope;
            const float sv = p.kv_b.s[wrow0 + nq + m16];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const long key = m0 + 16 * mt + 4 * g;
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[i] = key + i < nk ? fmaf(accl[qq][mt][i], 1.0f / 2048.0f, acc[qq][mt][i]) * sv : 0.0f;
                    bad |= outside_f16(v[i]);
                }
                uint16_t *hi = p.kv_expanded + L.value_block(p.heads, h, key / 32) +
                               (long)dv * kFlashVRow + key % 32;
                store_split4(hi, hi + (long)p.vdim * kFlashVRow, v);
            }
        }
    }
    expand_rope(p, h, m0, nk, t, bad);
    report_range(p, bad);
}

// Prefill attention (rows > 1, causal; moonlight_kernels.metal:247-343 with
// key_count = position + row + 1), flash form: a workgroup takes RB query
// rows and every head, and streams key tiles of kPfKeys cache rows
// through two LDS buffers (DMA of tile t + 1 in flight while tile t is
// used).  Per tile and row, on the f16 matrix cores as split-f16 triples
// (split_f16) with the operand layouts of mla_attend_mfma_kernel: scores
// S[key][head] (the 4 waves split the latent + rope dims in 32-dim steps;
// partials summed in LDS in wave order), the causal mask, an
// online softmax (running max and sum per row and head; the context is
// rescaled when the max grows), and the context LC[head][d] += P . lat (the
// waves split the 16-wide d tiles).  The normalised lc goes straight to
// latent_context: no split partials, no merge launch, and every key tile is
// read once per RB rows instead of once per row.
// Query rows and waves per workgroup.  Measured on MI355X (2048-token
// prefill): 2 rows on 4 waves 47.6 ms; 4 rows on 8 waves 48.4 ms (the key
// tiles' f16 splits serve twice the rows, but the kernel is bound by its
// per-tile barriers and latencies rather than by the vector work); 4 rows
// on 4 waves exceed the register file.
constexpr int kPfRowsPerGroup = 2;
constexpr int kPfWaves = 4;
constexpr int kPfKeys = 16;
constexpr int kPfRowStride = kMlaMaxLatent + 4;  // latent rows in LDS (rope in registers)
// The running max of a (row, head) moves only when a tile's max exceeds it
// by more than this (e^8 ~ 3e3 keeps every exp term and sum far inside fp32);
// the context rescale then runs on few tiles.
constexpr float kPfLazyMax = 8.0f;
template <int RB, int NW>
constexpr size_t pf_lds_bytes() {
    return sizeof(float) * (2 * (size_t)kPfKeys * kPfRowStride +     // key tiles (latent)
                            NW * RB * kPfKeys * kMlaMaxHeads +       // score partials
                            RB * kMlaMaxHeads * (kPfKeys + 4) +      // P [row][head][key]
                            3 * RB * kMlaMaxHeads);                  // max, sum, rescale
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations, not for its loads in flight (__syncthreads() would also wait
// for the next key tile's DMA and serialise the double buffering).
__device__ __forceinline__ void lds_barrier() {
    // The empty asm statements clobber memory, so the compiler keeps every
    // memory access on its side of the barrier (s_barrier alone is no memory
    // operation to it).  An LDS release fence would do the same but also wait
    // for the key tile's LDS DMA in flight (vmcnt(0)).
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt, expcnt not waited
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// RB query rows per workgroup of NW waves (4 or 8): wave w takes the 32-dim
// score steps w, w + NW, ... and the 16-wide context d tiles w, w + NW, ...
template <int RB, int NW>
__global__ __launch_bounds__(64 * NW, 8 / NW) void mla_prefill_attend_kernel(MlaParams p) {
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    constexpr int H = kMlaMaxHeads, KS = kPfKeys;
    constexpr int NJ = (kAttnDims / 32 + NW - 1) / NW;  // 32-dim score steps per wave
    constexpr int NQ = kMlaMaxLatent / 16 / NW;         // d tiles per wave
    constexpr int PS = KS + 4;                 // P row stride
    extern __shared__ __attribute__((aligned(16))) float pf_lds[];
    float *kbuf = pf_lds;                            // [2][KS][kPfRowStride]
    float *part = kbuf + 2 * KS * kPfRowStride;      // [NW waves][RB][KS][H]
    float *p_s = part + NW * RB * KS * H;            // [RB][H][PS]
    float *m_s = p_s + RB * H * PS;                  // [RB][H]
    float *l_s = m_s + RB * H;
    float *sc_s = l_s + RB * H;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int g = lane >> 4, m16 = lane & 15;
    const int r0 = blockIdx.x * RB;
    const int nrow = p.rows - r0 < RB ? p.rows - r0 : RB;
    const int pos0 = mla_position(p) + r0;  // position of row r0; row b sees keys <= pos0 + b
    const int keys = pos0 + nrow;
    const int ntiles = (keys + KS - 1) / KS;
    const int D = p.latent, R = p.rope, KD = D + R;  // KD a multiple of 16 (launch condition)
    // ---- queries of the rows split into f16 halves (split_f16): dims
    // 32 (w + NW j) + 8 g .. + 7 of head m16 (absent rows repeat row r0,
    // absent heads head 0, dims past KD are zero)
    half8 qh8[RB][NJ], ql8[RB][NJ];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const long qh = (long)(r0 + (b < nrow ? b : 0)) * p.heads + (m16 < p.heads ? m16 : 0);
        const float *qa = p.query_absorbed + qh * D;
        const float *qr = p.query_rope + qh * R;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int d = 32 * (wave + NW * j) + 8 * g;
            const float *src = d < D ? qa + d : d < KD ? qr + (d - D) : qa;
            const f32x4 v0 = load_f4(src), v1 = load_f4(src + 4);
            const bool in = d < KD;
            const float x[8] = {in ? v0.x : 0.f, in ? v0.y : 0.f, in ? v0.z : 0.f, in ? v0.w : 0.f,
                                in ? v1.x : 0.f, in ? v1.y : 0.f, in ? v1.z : 0.f, in ? v1.w : 0.f};
            split_f16<8>(x, qh8[b][j], ql8[b][j]);
        }
    }
    for (int i = t; i < RB * H; i += blockDim.x) {
        m_s[i] = -INFINITY;
        l_s[i] = 0.0f;
    }
    // ---- latent rows of a key tile -> LDS buffer by DMA (16 bytes per lane
    // into M0 + 16 lane); the rope part goes to registers: 32-dim step st =
    // D / 32 + s (dims D + 32 s ..) belongs to wave st % NW, which holds dims
    // D + 32 s + 8 g .. + 7 of key m16 (rope dims past R read dim 0 against a
    // zero query).  Rows past the last key copy the last key (finite, masked).
    const int rope_s = ((wave - D / 32) % NW + NW) % NW;  // this wave's rope step
    const bool has_rope = 32 * rope_s < R;
    const int rope_col = 32 * rope_s + 8 * g < R ? 32 * rope_s + 8 * g : 0;
    auto issue = [&](int tile, int buf, f32x4 (&rope_next)[2]) {
        float *kb = kbuf + buf * KS * kPfRowStride;
        for (int row = wave; row < KS; row += NW) {
            const int k = tile * KS + row < keys ? tile * KS + row : keys - 1;
            // the key's f16 halves (2 D halves: as many bytes as D floats)
            const float *lsrc = reinterpret_cast<const float *>(p.latent_split + (long)k * 2 * D);
            __attribute__((address_space(3))) float *dst =
                (__attribute__((address_space(3))) float *)(kb + row * kPfRowStride);
            for (int c0 = 0; c0 < D; c0 += 256)
                if (c0 + 4 * lane < D)
                    __builtin_amdgcn_global_load_lds(
                        (const __attribute__((address_space(1))) void *)(lsrc + c0 + 4 * lane),
                        dst + c0, 16, 0, 0);
        }
        if (has_rope) {
            const int k = tile * KS + m16 < keys ? tile * KS + m16 : keys - 1;
            rope_next[0] = load_f4(p.rope_cache + (long)k * R + rope_col);
            rope_next[1] = load_f4(p.rope_cache + (long)k * R + rope_col + 4);
        }
    };
    f32x4v acc[RB][NQ];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int q = 0; q < NQ; ++q) acc[b][q] = f32x4v{0.f, 0.f, 0.f, 0.f};
    f32x4 rope_cur[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    f32x4 rope_next[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    issue(0, 0, rope_next);
    for (int kt = 0; kt < ntiles; ++kt) {
        __builtin_amdgcn_s_waitcnt(0);  // this wave's part of tile kt has landed
        __syncthreads();                // every part visible; tile kt - 1 and P free
        rope_cur[0] = rope_next[0];
        rope_cur[1] = rope_next[1];
        if (kt + 1 < ntiles) issue(kt + 1, (kt + 1) & 1, rope_next);
        const float *kb = kbuf + (kt & 1) * KS * kPfRowStride;
        // ---- scores of the tile: wave w takes the 32-dim steps w, w + NW, ...
        // (v_mfma_f32_16x16x32_f16, split-f16 triples, two accumulator chains)
        {
            f32x4v sacc[RB][2];
#pragma unroll
            for (int b = 0; b < RB; ++b) sacc[b][0] = sacc[b][1] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int d0 = 32 * (wave + NW * j);
                if (d0 < KD) {
                    half8 kh, kl;
                    if (d0 < D) {  // the cached halves: hi at dims .., lo at D + dims
                        const _Float16 *row =
                            reinterpret_cast<const _Float16 *>(kb + m16 * kPfRowStride) + d0 + 8 * g;
                        kh = *reinterpret_cast<const half8 *>(row);
                        kl = *reinterpret_cast<const half8 *>(row + D);
                    } else {
                        const float x[8] = {rope_cur[0].x, rope_cur[0].y, rope_cur[0].z,
                                            rope_cur[0].w, rope_cur[1].x, rope_cur[1].y,
                                            rope_cur[1].z, rope_cur[1].w};
                        split_f16<8>(x, kh, kl);
                    }
#pragma unroll
                    for (int b = 0; b < RB; ++b) {
                        sacc[b][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh8[b][j], sacc[b][0], 0, 0, 0);
                        sacc[b][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql8[b][j], sacc[b][1], 0, 0, 0);
                        sacc[b][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh8[b][j], sacc[b][0], 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int b = 0; b < RB; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    part[((wave * RB + b) * KS + 4 * g + i) * H + m16] = sacc[b][0][i] + sacc[b][1][i];
        }
        lds_barrier();
        // ---- causal mask and online softmax: 16 lanes per (row, head), one key each
        for (int idx = t; idx < RB * H * KS; idx += blockDim.x) {
            const int b = idx / (H * KS), h = (idx / KS) % H, k = idx % KS;
            auto pw = [&](int w) { return part[((w * RB + b) * KS + k) * H + h]; };
            float sum = (pw(0) + pw(1)) + (pw(2) + pw(3));
            if constexpr (NW == 8) sum += (pw(4) + pw(5)) + (pw(6) + pw(7));
            const int key = kt * KS + k;
            const bool valid = b < nrow && key <= pos0 + b;
            const float sv = valid ? sum * p.scale : -INFINITY;
            // the 16 keys of (b, h) are the 16 lanes of one DPP row
            const float mt = row16_max(sv);
            const float mo = m_s[b * H + h];
            const float mn = mt > mo + kPfLazyMax ? mt : mo;  // -inf mo: the tile max
            const float e = valid ? __expf(sv - mn) : 0.0f;
            const float es = row16_sum(e);
            p_s[(b * H + h) * PS + k] = e;
            if (k == 0) {
                const float sc = mn == mo ? 1.0f : __expf(mo - mn);  // 0 while mo is -inf
                l_s[b * H + h] = l_s[b * H + h] * sc + es;
                m_s[b * H + h] = mn;
                sc_s[b * H + h] = sc;
            }
        }
        lds_barrier();
        // ---- context: wave w takes the d tiles w, w + NW, ...; each latent
        // operand is split once and multiplies the P of every row
        half4 ph[RB], pl[RB];
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            const f32x4 pv = *reinterpret_cast<const f32x4 *>(p_s + (b * H + m16) * PS + 4 * g);
            const float pj[4] = {pv.x, pv.y, pv.z, pv.w};
            float scl[4];
            bool rescale = false;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                scl[i] = sc_s[b * H + 4 * g + i];
                rescale |= scl[i] != 1.0f;
            }
            if (rescale) {  // rare: the lazy max moved for one of this lane's heads
#pragma unroll
                for (int q = 0; q < NQ; ++q)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[b][q][i] *= scl[i];
            }
            split_f16<4>(pj, ph[b], pl[b]);
        }
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int dt = wave + NW * q;
            if (dt < D / 16) {
                // keys 4 g .. 4 g + 3 of latent dim dt * 16 + m16, cached halves
                constexpr int RS = 2 * kPfRowStride;  // halves per LDS row
                const _Float16 *lb =
                    reinterpret_cast<const _Float16 *>(kb + (4 * g) * kPfRowStride) + dt * 16 + m16;
                const half4 bh = {lb[0], lb[RS], lb[2 * RS], lb[3 * RS]};
                const half4 bl = {lb[D], lb[RS + D], lb[2 * RS + D], lb[3 * RS + D]};
#pragma unroll
                for (int b = 0; b < RB; ++b) {
                    acc[b][q] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph[b], bh, acc[b][q], 0, 0, 0);
                    acc[b][q] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph[b], bl, acc[b][q], 0, 0, 0);
                    acc[b][q] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl[b], bh, acc[b][q], 0, 0, 0);
                }
            }
        }
    }
    __syncthreads();  // the last tile's sums in l_s
    // ---- normalised latent context of each row and head
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        if (b >= nrow) continue;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int dt = wave + NW * q;
            if (dt >= D / 16) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int h = 4 * g + i;
                if (h < p.heads)
                    p.latent_context[((long)(r0 + b) * p.heads + h) * D + dt * 16 + m16] =
                        acc[b][q][i] / l_s[b * H + h];
            }
        }
    }
}

// Prefill attention on the expanded keys and values (moonlight_kernels.metal
// :247-343 with key_count = position + row + 1, its latent form multiplied
// out: q_absorbed . lat = q_nope . (W_UK lat) and W_UV (sum_k p_k lat_k) =
// sum_k p_k (W_UV lat_k)), one head per workgroup, causal flash form.
// Workgroup (head, 64 query rows), wave w: rows 16 w .. + 15; every wave
// holds its rows' queries (QKP dims) as f16 halves and its rows' value
// context transposed, O^T[dv][row], in registers.  Per tile of 32 keys,
// copied with its values into LDS by DMA (one buffer, 43.5 KB at Moonlight's
// shape, so three workgroups share a CU and hide each other's copies;
// measured on MI355X against two buffers and one workgroup a CU: 165.7
// against 180.1 us per layer, 2048-token prefill; workgroups ordered so that
// the XCD of workgroup i (i % 8) takes one head after another measured
// 181.9 against 162.3 us with the same L2 hit rate, 89 %):
//   scores S^T[key][row] = K . Q^T, v_mfma_f32_16x16x32_f16 with the key
//     rows as A (16 keys a product) and the query as B, split-f16 triples:
//     a lane ends with four keys of one row;
//   softmax: per row a running max (lazy, kPfLazyMax) and sum, the row's
//     four lanes meeting by row swaps (quad_rows_max / quad_rows_sum);
//   context O^T += V^T . P^T with the lane's probabilities as B directly
//     (its 8 k slots: keys 4 g .. + 3 and 16 + 4 g .. + 3) and the value
//     block rows as A; a rescale touches the lane's own row only.
// NKS: 32-dim score steps (QKP / 32); NV: 16-dim value tiles (vdim / 16).
// Max / sum over the four 16-lane rows of a wave for each lane position
// (lanes l, l ^ 16, l ^ 32, l ^ 48), by the gfx950 row swaps: the same
// order of terms in every lane, so the four copies agree bit for bit.
__device__ __forceinline__ float quad_rows_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float quad_rows_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float m = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int NKS, int NV>
constexpr size_t flash_lds_bytes() {
    return sizeof(uint16_t) * (32 * (2 * 32 * NKS + 8) + 2 * 16 * NV * kFlashVRow);
}

template <int NKS, int NV>
__global__ __launch_bounds__(256, 1) void mla_flash_kernel(MlaParams p) {
    constexpr int QKP = 32 * NKS, KROW = 2 * QKP + 8, VD = 16 * NV;
    constexpr int KHALVES = 32 * KROW, VHALVES = 2 * VD * kFlashVRow;
    extern __shared__ __attribute__((aligned(16))) uint16_t fl_lds[];
    const ExpandLayout L(p);
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int g = lane >> 4, m16 = lane & 15;
    const int h = blockIdx.x;
    const int nrb = (p.rows + 63) / 64;
    const int r0 = (nrb - 1 - (int)blockIdx.y) * 64;  // the longest rows first
    const int pos0 = mla_position(p);
    const int rl = r0 + 16 * wave + m16;               // this lane's query row
    const int rc = rl < p.rows ? rl : p.rows - 1;      // (absent rows repeat the last)
    const int rpos = pos0 + rc;                         // keys 0 .. rpos are visible
    const int wlast = pos0 + min(r0 + 16 * wave + 15, p.rows - 1);  // the wave's last key
    const int nk = pos0 + min(r0 + 64, p.rows);         // keys of the workgroup
    const int ntiles = (nk + 31) / 32;
    // ---- the query row as f16 halves: dims 32 j + 8 g .. + 7 (k_nope dims,
    // then the rope, zeros past nope + rope), scaled by the softmax scale and
    // log2(e), so that the scores come out in base-2 exponent units
    constexpr float kLog2e = 1.4426950408889634f;
    const float qscale = p.scale * kLog2e;
    half8 qh[NKS], ql[NKS];
    bool bad = false;
    {
        const float *qn = p.query + (long)rc * p.query_stride + (long)h * (p.nope + p.rope);
        const float *qr = p.query_rope + ((long)rc * p.heads + h) * p.rope;
#pragma unroll
        for (int j = 0; j < NKS; ++j) {
            const int d = 32 * j + 8 * g;
            float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (d < p.nope + p.rope) {
                const float *src = d < p.nope ? qn + d : qr + (d - p.nope);
                const f32x4 v0 = load_f4(src), v1 = load_f4(src + 4);
                x[0] = v0.x, x[1] = v0.y, x[2] = v0.z, x[3] = v0.w;
                x[4] = v1.x, x[5] = v1.y, x[6] = v1.z, x[7] = v1.w;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                bad |= outside_f16(x[i]);
                x[i] *= qscale;
            }
            split_f16<8>(x, qh[j], ql[j]);
        }
    }
    report_range(p, bad);
    // ---- DMA of key tile kt (its key rows, then its value block) into LDS:
    // 1 KB per wave instruction, 16 bytes a lane
    auto issue = [&](int kt) {
        uint16_t *dst = fl_lds;
        const uint16_t *ks = p.kv_expanded + L.key_row(h, 32L * kt);
        const uint16_t *vs = p.kv_expanded + L.value_block(p.heads, h, kt);
        constexpr int KC = KHALVES / 8, VC = VHALVES / 8;  // 16-byte chunks
        // unrolled over compile-time trip counts (the lane test matters for
        // the last, partial instruction only): 153.8 against 160.9 us per
        // layer for the runtime loops
#pragma unroll
        for (int i = 0; i < (KC + 255) / 256; ++i) {
            const int c0 = 64 * wave + 256 * i;
            if (c0 < KC && (KC % 64 == 0 || c0 + lane < KC))
                __builtin_amdgcn_global_load_lds(
                    (const __attribute__((address_space(1))) void *)(ks + 8L * (c0 + lane)),
                    (__attribute__((address_space(3))) void *)(dst + 8 * c0), 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < (VC + 255) / 256; ++i) {
            const int c0 = 64 * wave + 256 * i;
            if (c0 < VC && (VC % 64 == 0 || c0 + lane < VC))
                __builtin_amdgcn_global_load_lds(
                    (const __attribute__((address_space(1))) void *)(vs + 8L * (c0 + lane)),
                    (__attribute__((address_space(3))) void *)(dst + KHALVES + 8 * c0), 16, 0, 0);
        }
    };
    f32x4v acc[NV];
#pragma unroll
    for (int q = 0; q < NV; ++q) acc[q] = f32x4v{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;
    issue(0);
    for (int kt = 0; kt < ntiles; ++kt) {
        __builtin_amdgcn_s_waitcnt(0);  // this wave's part of tile kt has landed
        __syncthreads();                // every part visible
        if (32 * kt > wlast) {  // every key of the tile is after the wave's rows
            __syncthreads();
            if (kt + 1 < ntiles) issue(kt + 1);
            continue;
        }
        const uint16_t *kb = fl_lds;
        const uint16_t *vb = kb + KHALVES;
        // ---- scores: keys 16 s + m16 as A rows, this wave's rows as B columns
        f32x4v sa[2][2];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) sa[s2][0] = sa[s2][1] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NKS; ++j) {
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const uint16_t *kr = kb + (16 * s2 + m16) * KROW + 32 * j + 8 * g;
                const half8 kh = *reinterpret_cast<const half8 *>(kr);
                const half8 kl = *reinterpret_cast<const half8 *>(kr + QKP);
                sa[s2][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[j], sa[s2][0], 0, 0, 0);
                sa[s2][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[j], sa[s2][1], 0, 0, 0);
                sa[s2][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[j], sa[s2][0], 0, 0, 0);
            }
        }
        // ---- causal mask (tiles the diagonal crosses only), online softmax
        // of the lane's row in base 2 (v_exp_f32)
        float sv[8], e[8];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[4 * s2 + i] = sa[s2][0][i] + sa[s2][1][i];
        const bool whole = 32 * kt + 31 <= pos0 + r0 + 16 * wave;  // every key visible (wave)
        float mt = -INFINITY;
        if (whole) {
#pragma unroll
            for (int i = 0; i < 8; ++i) mt = fmaxf(mt, sv[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int key = 32 * kt + 16 * (i >> 2) + 4 * g + (i & 3);
                if (key > rpos) sv[i] = -INFINITY;
                mt = fmaxf(mt, sv[i]);
            }
        }
        mt = quad_rows_max(mt);
        const float mn = mt > m + kPfLazyMax * kLog2e ? mt : m;  // -inf m: the tile max
        float es = 0.0f;
        if (mn == -INFINITY) {  // no visible key yet for the row
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = 0.0f;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                e[i] = __builtin_amdgcn_exp2f(sv[i] - mn);  // masked keys: 2^-inf = 0
                es += e[i];
            }
        }
        es = quad_rows_sum(es);
        const float sc = mn == m ? 1.0f : __builtin_amdgcn_exp2f(m - mn);  // 0 while m is -inf
        l = l * sc + es;
        m = mn;
        if (__ballot(sc != 1.0f)) {  // rare: a row's max moved
#pragma unroll
            for (int q = 0; q < NV; ++q)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[q][i] *= sc;
        }
        half8 ph, pl;
        split_f16<8>(e, ph, pl);
        // ---- context: value dims 16 q + m16 as A rows (keys 4 g .. + 3 and
        // 16 + 4 g .. + 3 of the block), the probabilities as B
#pragma unroll
        for (int q = 0; q < NV; ++q) {
            const uint16_t *vr = vb + (16 * q + m16) * kFlashVRow + 4 * g;
            const half4 h0 = *reinterpret_cast<const half4 *>(vr);
            const half4 h1 = *reinterpret_cast<const half4 *>(vr + 16);
            const half4 l0 = *reinterpret_cast<const half4 *>(vr + VD * kFlashVRow);
            const half4 l1 = *reinterpret_cast<const half4 *>(vr + VD * kFlashVRow + 16);
            const half8 vh = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
            const half8 vl = {l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
            acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph, acc[q], 0, 0, 0);
            acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pl, acc[q], 0, 0, 0);
            acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vl, ph, acc[q], 0, 0, 0);
        }
        __syncthreads();  // every wave is done with the tile
        if (kt + 1 < ntiles) issue(kt + 1);
    }
    // ---- the row's context: O^T[16 q + 4 g + i][row] / l
    if (rl < p.rows) {
        const float inv = 1.0f / l;
        float *out = p.context + ((long)rl * p.heads + h) * p.vdim + 4 * g;
#pragma unroll
        for (int q = 0; q < NV; ++q)
            *reinterpret_cast<f32x4 *>(out + 16 * q) =
                f32x4{acc[q][0] * inv, acc[q][1] * inv, acc[q][2] * inv, acc[q][3] * inv};
    }
}

// Merge of the key splits and the value projection, one launch.  Workgroup
// (row, head h, chunk c of kMlaValueDims latent dims), 8 waves:
//   merge  lc_h[d] = sum_s e^{m_s - M} lc_s[d] / sum_s e^{m_s - M} l_s for
//          the chunk's dims in one pass over its contiguous partials: thread
//          t takes dims 4 (t % 8) .. + 3 of the splits t / 8, t / 8 + 64, ...
//          with a running max (rescaling on a new max), loading kMergeBatch
//          splits before using them; the 8 slots of a wave meet by
//          shuffles, the 8 waves in LDS.  The row's own key (not in any
//          split) joins as one more term: its score [qa | q_rope] . [lat |
//          rope] over the whole workgroup, its weight 1 and its latent row.
//   value  y_c[v] = W_UV_h[v, chunk] . lc_h[chunk] for every value row v:
//          thread t takes row t / 4 (+ 128 per pass), dims 8 (t % 4) .. + 7;
//          the first pass's weights are loaded before the merge starts.
//   sum    ctx_h[v] = sum_c y_c[v] in chunk order, by the chunk workgroup
//          that arrives last (merge_count; it resets the counter).  The
//          shares travel as device-coherent (agent-scope) stores and loads,
//          which on gfx950 bypass the per-XCD L2 copies
//          (agent_handoff_arrive, mlh_device.h).
constexpr int kMergeBatch = 4;
template <int FMT>
__global__ __launch_bounds__(512) void mla_merge_value_kernel(MlaParams p) {
    constexpr int H = kMlaMaxHeads;
    constexpr int TK = kMlaTileKeys;
    constexpr int DL = kMlaValueDims, NB = kMergeBatch;
    constexpr int NG = 8;  // waves
    static_assert(DL == 32, "8 threads of 4 dims per split");
    __shared__ float gm[NG], gl[NG];
    __shared__ __attribute__((aligned(16))) float gacc[NG][DL];
    __shared__ float lcs[DL];
    __shared__ float ownp[8];
    const int r = blockIdx.x, h = blockIdx.y, c = blockIdx.z;
    const int nchunks = gridDim.z;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    // ---- loads, in this order and all unconditional (indices clamped; no
    // load under a branch, whose join would wait for every load before it):
    // the split partials (a row has at most kMlaAttendGroups <= 64 NB
    // splits: one batch of NB per thread, masked once the position is
    // known), the first value-weight rows, the position, the own key's
    // score terms and latent value
    static_assert(64 * NB >= kMlaAttendGroups, "one batch covers every split");
    const long mbase = ((long)r * H + h) * p.max_splits;
    const int dq = t & 7, slot = t >> 3;
    const float *lc = p.part_lc + (((long)r * H + h) * nchunks + c) * p.max_splits * DL + 4 * dq;
    float mv[NB], lv[NB];
    f32x4 v[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int s = slot + 64 * i < p.max_splits ? slot + 64 * i : p.max_splits - 1;
        mv[i] = p.part_max[mbase + s];
        lv[i] = p.part_sum[mbase + s];
        v[i] = load_f4(lc + (long)s * DL);
    }
    // value rows of this thread: v = t / 4 + 128 i; dims c * DL + 8 (t % 4) ..
    const int vq = t & 3, vr = t >> 2;
    const int wrow0 = h * (p.nope + p.vdim) + p.nope;
    const int vcol = c * DL + 8 * vq;
    Kvb8<FMT> wraw;
    kvb_fetch8<FMT>(p.kv_b, wrow0 + (vr < p.vdim ? vr : 0), vcol, p.latent, wraw);
    const int pos = mla_position(p) + r;  // row r's own key; the splits hold keys 0 .. pos - 1
    const int keys = pos;
    // thread t: latent dim t, rope dim t of the own key's score, latent
    // value t of this chunk
    const float *qa = p.query_absorbed + ((long)r * p.heads + h) * p.latent;
    const float *qr = p.query_rope + ((long)r * p.heads + h) * p.rope;
    const float *lnew = p.latent_cache + (long)pos * p.latent;
    const float *rnew = p.rope_cache + (long)pos * p.rope;
    const int tl = t < p.latent ? t : 0, tr = t < p.rope ? t : 0, tv = t < DL ? t : 0;
    const float qa_t = qa[tl], ln_t = lnew[tl], qr_t = qr[tr], rn_t = rnew[tr];
    const float lv_t = lnew[c * DL + tv];
    // (selects, not branches: a load the compiler sinks into a branch is
    // waited for at the join)
    float own = (t < p.latent ? qa_t : 0.0f) * ln_t;
    own = fmaf(t < p.rope ? qr_t : 0.0f, rn_t, own);
    const float own_v = t < DL ? lv_t : 0.0f;

    const int tiles = (keys + TK - 1) / TK;
    const int ns = tiles < p.splits ? tiles : p.splits;  // partials of this row
    float M = -INFINITY, L = 0.0f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    {
        bool ok[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) ok[i] = slot + 64 * i < ns;
        float mn = M;
#pragma unroll
        for (int i = 0; i < NB; ++i) mn = fmaxf(mn, ok[i] ? mv[i] : -INFINITY);
        // no valid split for this thread: mn is -inf and nothing changes
        // (M - mn would be NaN); else the rescale is 0 while M is -inf
        const float sc = mn == -INFINITY ? 1.0f : expf(M - mn);
        acc.x *= sc;
        acc.y *= sc;
        acc.z *= sc;
        acc.w *= sc;
        L *= sc;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            // masked slots hold stale memory (possibly NaN): zero their
            // values, not only their weight
            const float e = ok[i] ? expf(mv[i] - mn) : 0.0f;
            const f32x4 vi = ok[i] ? v[i] : f32x4{0.f, 0.f, 0.f, 0.f};
            acc.x = fmaf(e, vi.x, acc.x);
            acc.y = fmaf(e, vi.y, acc.y);
            acc.z = fmaf(e, vi.z, acc.z);
            acc.w = fmaf(e, vi.w, acc.w);
            L = fmaf(e, ok[i] ? lv[i] : 0.0f, L);
        }
        M = mn;
    }
    // the 8 slots of the wave (lanes 8 apart), then the waves in LDS
#pragma unroll
    for (int o = 8; o <= 32; o <<= 1) {
        const float M2 = __shfl_xor(M, o, 64), L2 = __shfl_xor(L, o, 64);
        const f32x4 a2 = {__shfl_xor(acc.x, o, 64), __shfl_xor(acc.y, o, 64),
                          __shfl_xor(acc.z, o, 64), __shfl_xor(acc.w, o, 64)};
        const float mn = fmaxf(M, M2);
        const float e1 = M == -INFINITY ? 0.0f : expf(M - mn);
        const float e2 = M2 == -INFINITY ? 0.0f : expf(M2 - mn);
        acc.x = acc.x * e1 + a2.x * e2;
        acc.y = acc.y * e1 + a2.y * e2;
        acc.z = acc.z * e1 + a2.z * e2;
        acc.w = acc.w * e1 + a2.w * e2;
        L = L * e1 + L2 * e2;
        M = mn;
    }
    if (lane < 8) {
        if (lane == 0) {
            gm[wave] = M;
            gl[wave] = L;
        }
        *reinterpret_cast<f32x4 *>(&gacc[wave][4 * dq]) = acc;
    }
    own = wave_sum(own);
    if (lane == 0) ownp[t >> 6] = own;
    __syncthreads();
    if (t < DL) {
        const float snew =
            (((ownp[0] + ownp[1]) + (ownp[2] + ownp[3])) + ((ownp[4] + ownp[5]) + (ownp[6] + ownp[7]))) *
            p.scale;
        float mt = snew;  // groups without a split hold -inf
        for (int i = 0; i < NG; ++i) mt = fmaxf(mt, gm[i]);
        float a = 0.0f, l = 0.0f;
        for (int i = 0; i < NG; ++i) {
            const float e = gm[i] == -INFINITY ? 0.0f : expf(gm[i] - mt);
            a = fmaf(e, gacc[i][t], a);
            l = fmaf(e, gl[i], l);
        }
        const float en = expf(snew - mt);
        a = fmaf(en, own_v, a);
        l += en;
        lcs[t] = a / l;
    }
    __syncthreads();
    float *part = p.value_part + (((long)r * p.heads + h) * nchunks + c) * p.vdim;
    for (int v0 = 0; v0 < p.vdim; v0 += 128) {
        const int v = v0 + vr;
        if (v0 > 0) kvb_fetch8<FMT>(p.kv_b, wrow0 + (v < p.vdim ? v : 0), vcol, p.latent, wraw);
        float wv[8];
        kvb_decode8<FMT>(wraw, wv);
        float y = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) y = fmaf(wv[e], lcs[8 * vq + e], y);
        y += __shfl_xor(y, 1, 64);
        y += __shfl_xor(y, 2, 64);
        if (vq == 0 && v < p.vdim)
            __hip_atomic_store(part + v, y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // the last of the head's chunk workgroups sums the shares
    int *count = p.merge_count + (r * p.heads + h) * kMlaCountStride;
    if (!agent_handoff_arrive(count, nchunks)) return;
    constexpr int kMaxChunks = kMlaMaxLatent / kMlaValueDims;
    const float *parts = p.value_part + ((long)r * p.heads + h) * nchunks * p.vdim;
    for (int v = t; v < p.vdim; v += 512) {
        float sh[kMaxChunks];  // all shares in flight before the first add
#pragma unroll
        for (int i = 0; i < kMaxChunks; ++i)
            sh[i] = i < nchunks ? __hip_atomic_load(parts + (long)i * p.vdim + v,
                                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                : 0.0f;
        float y = 0.0f;
#pragma unroll
        for (int i = 0; i < kMaxChunks; ++i) y += sh[i];
        p.context[((long)r * p.heads + h) * p.vdim + v] = y;
    }
    if (t == 0) __hip_atomic_store(count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


__global__ __launch_bounds__(256) void split_cache_kernel(const float *latent, uint16_t *split,
                                                          long rows, int width) {
    const long n = rows * width;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (long)gridDim.x * blockDim.x) {
        const long r = i / width;
        const int c = (int)(i - r * width);
        uint16_t hi, lo;
        split_f16_bits(latent[i], hi, lo);
        split[r * 2 * width + c] = hi;
        split[r * 2 * width + width + c] = lo;
    }
}

int mla_split_cache(const float *latent, uint16_t *split, long rows, int width,
                    hipStream_t stream) {
    if (rows < 0 || width <= 0 || (rows && (!latent || !split))) return kErrArgs;
    if (rows == 0) return kOk;
    const long n = rows * width;
    const int blocks = (int)std::min<long>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(split_cache_kernel, dim3(blocks), dim3(256), 0, stream, latent, split,
                       rows, width);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// The flash kernel's instantiations: (QKP / 32, vdim / 16) of Moonlight
// (nope 128 + rope 64, value 128) and of the small test models (32 + 16, 32).
static bool flash_shape(int nope, int rope, int vdim, int *nks, int *nv) {
    if (nope <= 0 || rope <= 0 || vdim <= 0 || nope % 16 || rope % 8 || vdim % 16) return false;
    *nks = (nope + rope + 31) / 32;
    *nv = vdim / 16;
    return (*nks == 6 && *nv == 8) || (*nks == 2 && *nv == 2);
}

size_t mla_expand_kv_bytes(int heads, int nope, int rope, int vdim, int latent, int kv_b_fmt) {
    int nks, nv;
    if (heads <= 0 || !flash_shape(nope, rope, vdim, &nks, &nv) || latent <= 0 ||
        latent % kExKC || nope + vdim > 256 || (kv_b_fmt != kQ8 && kv_b_fmt != kQ4))
        return 0;
    const size_t krow = 2 * 32 * (size_t)nks + 8;
    return (size_t)heads * (krow + 2 * (size_t)vdim * kFlashVRow / 32) * sizeof(uint16_t);
}

template <int NKS, int NV>
static void launch_flash(const MlaParams &p, hipStream_t stream) {
    static const bool attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&mla_flash_kernel<NKS, NV>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)(flash_lds_bytes<NKS, NV>())) == hipSuccess;
    (void)attr;
    constexpr size_t lds = flash_lds_bytes<NKS, NV>();
    hipLaunchKernelGGL((mla_flash_kernel<NKS, NV>), dim3(p.heads, (p.rows + 63) / 64), dim3(256),
                       lds, stream, p);
}

// Prefill on the expanded keys and values: the expansion of every key
// 0 .. position + rows - 1 (a head GEMM over the latent cache), then the
// flash kernel.  False (nothing launched) when the shape or format has no
// instantiation or the keys exceed the expanded buffer.
static bool mla_prefill_expanded(const MlaParams &p, hipStream_t stream) {
    int nks, nv;
    const long nk = (long)p.position + p.rows;
    if (!p.kv_expanded || p.rows < kMlaExpandMinRows || nk > p.expand_keys ||
        !mla_expand_kv_bytes(p.heads, p.nope, p.rope, p.vdim, p.latent, p.kv_b.fmt) ||
        !flash_shape(p.nope, p.rope, p.vdim, &nks, &nv))
        return false;
    const dim3 ge((unsigned)((nk + 63) / 64), (unsigned)p.heads);
    if (p.kv_b.fmt == kQ8)
        hipLaunchKernelGGL(mla_expand_kernel<kQ8>, ge, dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(mla_expand_kernel<kQ4>, ge, dim3(256), 0, stream, p);
    if (nks == 6)
        launch_flash<6, 8>(p, stream);
    else
        launch_flash<2, 2>(p, stream);
    return true;
}

int mla_attention_core(const MlaParams &p, hipStream_t stream) {
    if (p.heads <= 0 || p.heads > kMlaMaxHeads || p.latent <= 0 || p.latent % 64 ||
        p.latent > kMlaMaxLatent || p.rope <= 0 || p.rope > 64 || (p.rope & 1) ||
        p.nope <= 0 || p.nope > 256 || p.vdim <= 0 || p.rows <= 0 || p.max_splits <= 0 ||
        !p.latent_context || p.position < 0 || p.query_stride < (long)p.heads * (p.nope + p.rope) ||
        p.compressed_stride < p.latent + p.rope ||
        (p.grid_splits && (!p.position_dev || p.grid_splits > p.max_splits)))
        return kErrArgs;
    // the fp32-MFMA score tiles take 16 dims per step (mla_session_shape_ok)
    if (p.rope % 16 || p.latent + p.rope > kAttnDims) return kErrArgs;
    if (p.rows > 1 && !p.grid_splits && p.nope % 16 == 0 && p.vdim % 16 == 0) {
        // prefill: cache append + query rope, the absorb as a per-head GEMM,
        // flash attention writing lc directly, the value as a per-head GEMM
        constexpr int RB = kPfRowsPerGroup, NW = kPfWaves;
        static const bool attr = hipFuncSetAttribute(
            reinterpret_cast<const void *>(&mla_prefill_attend_kernel<RB, NW>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)pf_lds_bytes<RB, NW>()) == hipSuccess;
        (void)attr;
        const unsigned mt = (unsigned)((p.rows + 63) / 64);
        // the cache rows and every head's query rope, one workgroup a row
        // (measured on MI355X, 2048-token prefill: 12.5 us per layer against
        // 28.2 with a workgroup per (row, head) for the rope)
        hipLaunchKernelGGL(mla_prep_kernel<kF32>, dim3(p.rows, 1), dim3(256), 0, stream, p, -1);
        if (mla_prefill_expanded(p, stream))
            return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
        // the head GEMMs on the f16 matrix cores for integer kv_b (K a
        // multiple of 32 with an instantiation), else on fp32 MFMA
        const dim3 ga(mt, (unsigned)((p.latent + 63) / 64), (unsigned)p.heads);
        const dim3 gv(mt, (unsigned)((p.vdim + 63) / 64), (unsigned)p.heads);
        const bool q8 = p.kv_b.fmt == kQ8, q4 = p.kv_b.fmt == kQ4;
        const bool fa = (q8 && launch_head_gemm_f16<kHgAbsorb, kQ8>(p, ga, stream)) ||
                        (q4 && launch_head_gemm_f16<kHgAbsorb, kQ4>(p, ga, stream));
        if (!fa) hipLaunchKernelGGL(mla_head_gemm_kernel<true>, ga, dim3(256), 0, stream, p);
        hipLaunchKernelGGL((mla_prefill_attend_kernel<RB, NW>), dim3((p.rows + RB - 1) / RB),
                           dim3(64 * NW), (pf_lds_bytes<RB, NW>()), stream, p);
        const bool fv = (q8 && launch_head_gemm_f16<kHgValue, kQ8>(p, gv, stream)) ||
                        (q4 && launch_head_gemm_f16<kHgValue, kQ4>(p, gv, stream));
        if (!fv) hipLaunchKernelGGL(mla_head_gemm_kernel<false>, gv, dim3(256), 0, stream, p);
        return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
    }
    // decode: groups of at most kMlaDecodeRows rows (the partial buffers'
    // capacity), three launches each
    if (!p.value_part || !p.merge_count || p.latent % kMlaValueDims ||
        (p.position_dev && p.rows > kMlaDecodeRows) ||
        (p.kv_b.fmt != kF32 && p.kv_b.fmt != kQ8 && p.kv_b.fmt != kQ4))
        return kErrArgs;
    static const bool attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&mla_attend_mfma_kernel),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)kAttnMfmaLds) == hipSuccess;
    (void)attr;
    for (int r0 = 0; r0 < p.rows; r0 += kMlaDecodeRows) {
        MlaParams q = p;
        q.rows = p.rows - r0 < kMlaDecodeRows ? p.rows - r0 : kMlaDecodeRows;
        q.position = p.position + r0;
        q.query = p.query + (long)r0 * p.query_stride;
        q.compressed = p.compressed + (long)r0 * p.compressed_stride;
        q.context = p.context + (long)r0 * p.heads * p.vdim;
        const int chunks = (q.latent + kMlaAbsorbCols - 1) / kMlaAbsorbCols;
        const dim3 pgrid(q.rows, 1 + q.heads * chunks);
        const dim3 mgrid(q.rows, q.heads, q.latent / kMlaValueDims);
        switch (q.kv_b.fmt) {
        case kF32: hipLaunchKernelGGL(mla_prep_kernel<kF32>, pgrid, dim3(256), 0, stream, q, chunks); break;
        case kQ8: hipLaunchKernelGGL(mla_prep_kernel<kQ8>, pgrid, dim3(256), 0, stream, q, chunks); break;
        default: hipLaunchKernelGGL(mla_prep_kernel<kQ4>, pgrid, dim3(256), 0, stream, q, chunks); break;
        }
        // row r's splits hold keys 0 .. position + r - 1 (its own key joins
        // in the merge): kMlaAttendGroups workgroups over the group's rows,
        // at most one per key tile of the last row
        const int tiles = (q.position + q.rows - 1 + kMlaTileKeys - 1) / kMlaTileKeys;
        int splits = (kMlaAttendGroups + q.rows - 1) / q.rows;
        if (splits > tiles) splits = tiles;
        if (splits > q.max_splits) splits = q.max_splits;
        if (splits < 1) splits = 1;
        q.splits = q.grid_splits ? q.grid_splits : splits;
        hipLaunchKernelGGL(mla_attend_mfma_kernel, dim3(q.splits, q.rows), dim3(512), kAttnMfmaLds,
                           stream, q);
        switch (q.kv_b.fmt) {
        case kF32: hipLaunchKernelGGL(mla_merge_value_kernel<kF32>, mgrid, dim3(512), 0, stream, q); break;
        case kQ8: hipLaunchKernelGGL(mla_merge_value_kernel<kQ8>, mgrid, dim3(512), 0, stream, q); break;
        default: hipLaunchKernelGGL(mla_merge_value_kernel<kQ4>, mgrid, dim3(512), 0, stream, q); break;
        }
    }
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace mlh

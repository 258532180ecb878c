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
// Launches per attention call:
//   mla_prep    (row, cache-append | head): RMSNorm + RoPE into the caches,
//               RoPE of the query's rope part, and the absorbed query
//               qa_h = W_UK_h^T q_nope_h with each wave streaming whole kv_b
//               rows (coalesced 8-column lane slices).
//   mla_attend  (key split of kMlaKeysPerSplit keys, row): every latent row
//               read once scores ALL heads (the reference re-reads the cache
//               per head); per split a local max / exp-sum and the partial
//               latent context of every head (the split's latent rows are
//               re-read from L2 for the context pass).
//   mla_merge   (row, head, 128-wide latent chunk): log-sum-exp merge of the
//               splits into lc_h.
//   mla_value   (row, head, 32 value rows): ctx_h = W_UV_h lc_h.
#include "mla.h"

#include "mlh_device.h"

namespace mlh {

// Eight consecutive dequantised kv_b values w[row, col..col+7] (col % 8 == 0),
// moonlight_weight_value (moonlight_kernels.metal:202-216) applied per element.
__device__ __forceinline__ void kvb_load8(const MatrixRef &m, int row, int col, int width,
                                          float (&out)[8]) {
    if (m.fmt == kF32) {
        const float *p = reinterpret_cast<const float *>(m.w) + (long)row * width + col;
        const f32x4 a = load_f4(p), b = load_f4(p + 4);
        out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
        out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
        return;
    }
    const float s = m.s[row];
    if (m.fmt == kQ8) {
        const uint2 v = *reinterpret_cast<const uint2 *>(m.w + (long)row * width + col);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[i] = (float)(int8_t)((v.x >> (8 * i)) & 0xFF) * s;
            out[4 + i] = (float)(int8_t)((v.y >> (8 * i)) & 0xFF) * s;
        }
        return;
    }
    const unsigned v =
        *reinterpret_cast<const unsigned *>(m.w + (long)row * ((width + 1) / 2) + col / 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = (float)((int)((v >> (8 * i)) & 15) - 8) * s;
        out[2 * i + 1] = (float)((int)((v >> (8 * i + 4)) & 15) - 8) * s;
    }
}

__global__ __launch_bounds__(256) void mla_prep_kernel(MlaParams p) {
    const int r = blockIdx.x;
    const int role = blockIdx.y;  // 0: cache append, 1 + h: query head h
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int pos = p.position + r;
    const int hw = p.nope + p.rope;
    const int half = p.rope / 2;
    if (role == 0) {
        __shared__ float part[4];
        const float *c = p.compressed + (long)r * p.compressed_stride;
        float ss = 0.0f;
        for (int i = t; i < p.latent; i += blockDim.x) ss += c[i] * c[i];
        ss = wave_sum(ss);
        if (lane == 0) part[wave] = ss;
        __syncthreads();
        const float total = (part[0] + part[1]) + (part[2] + part[3]);
        const float inv = 1.0f / sqrtf(total / (float)p.latent + p.eps);
        float *lat = p.latent_cache + (long)pos * p.latent;
        for (int i = t; i < p.latent; i += blockDim.x) lat[i] = c[i] * inv * p.kv_norm[i];
        float *rp = p.rope_cache + (long)pos * p.rope;
        if (t < half) {
            const float angle = (float)pos * p.inv_freq[t];
            const float cs = cosf(angle), sn = sinf(angle);
            const float first = c[p.latent + 2 * t], second = c[p.latent + 2 * t + 1];
            rp[t] = first * cs - second * sn;
            rp[half + t] = second * cs + first * sn;
        }
        return;
    }
    const int h = role - 1;
    const float *q = p.query + (long)r * p.query_stride + (long)h * hw;
    if (t < half) {
        const float angle = (float)pos * p.inv_freq[t];
        const float cs = cosf(angle), sn = sinf(angle);
        const float first = q[p.nope + 2 * t], second = q[p.nope + 2 * t + 1];
        float *qr = p.query_rope + ((long)r * p.heads + h) * p.rope;
        qr[t] = first * cs - second * sn;
        qr[half + t] = second * cs + first * sn;
    }
    // qa[l] = sum_c q_nope[c] * kv_b[h*(nope+v) + c, l]: wave w takes rows
    // c = w, w+4, ...; lane owns columns 8*lane .. 8*lane+7 (+512 per pass)
    __shared__ float red[4][kMlaMaxLatent];
    const int wrow = h * (p.nope + p.vdim);
    for (int col0 = 0; col0 < p.latent; col0 += 512) {
        const int col = col0 + 8 * lane;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (col < p.latent) {
            // 8 rows per step: all loads issued before the FMAs
            for (int c0 = wave; c0 < p.nope; c0 += 32) {
                float wv[8][8];
                float qc[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int c = c0 + 4 * j;
                    qc[j] = c < p.nope ? q[c] : 0.0f;
                    if (c < p.nope) {
                        kvb_load8(p.kv_b, wrow + c, col, p.latent, wv[j]);
                    } else {
#pragma unroll
                        for (int i = 0; i < 8; ++i) wv[j][i] = 0.0f;
                    }
                }
#pragma unroll
                for (int j = 0; j < 8; ++j)
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[i] = fmaf(qc[j], wv[j][i], acc[i]);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) red[wave][col - col0 + i] = acc[i];
        }
        __syncthreads();
        float *qa = p.query_absorbed + ((long)r * p.heads + h) * p.latent;
        for (int i = t; i < 512 && col0 + i < p.latent; i += blockDim.x)
            qa[col0 + i] = (red[0][i] + red[1][i]) + (red[2][i] + red[3][i]);
        __syncthreads();
    }
}

// Latent slice of a lane: LPL values per lane, float4 groups at 4*lane and
// 256 + 4*lane for the 512-wide cache (coalesced 1 KB per wave load).
template <int LPL>
__device__ __forceinline__ int lat_index(int lane, int i) {
    if constexpr (LPL >= 4) return (i / 4) * 256 + 4 * lane + (i % 4);
    else if constexpr (LPL == 2) return 2 * lane + i;
    else return lane;
}

template <int LPL>
__device__ __forceinline__ void load_lat(const float *row, int lane, float (&v)[LPL]) {
    if constexpr (LPL >= 4) {
#pragma unroll
        for (int g = 0; g < LPL / 4; ++g) {
            const f32x4 a = load_f4(row + g * 256 + 4 * lane);
            v[4 * g + 0] = a.x; v[4 * g + 1] = a.y; v[4 * g + 2] = a.z; v[4 * g + 3] = a.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < LPL; ++i) v[i] = row[lat_index<LPL>(lane, i)];
    }
}

// One workgroup per (split of KS keys, token row).  Wave w scores heads
// 4w..4w+3 against every key of the split (8 keys per step, all loads issued
// first); the transposed butterfly leaves one (key, head) score per writer
// lane.  The context pass gives each thread latent dims t, t+256 and loads
// KB cache values of its dims at a time before their FMAs.
template <int LPL>
__global__ __launch_bounds__(256) void mla_attend_kernel(MlaParams p) {
    constexpr int H = kMlaMaxHeads;
    constexpr int KS = kMlaKeysPerSplit;
    constexpr int HW = H / 4;  // heads per wave
    constexpr int KB = 8;      // keys per scoring step
    __shared__ float prob[KS][H];  // scores, then probabilities, key-major
    __shared__ float smax[H], ssum[H];
    const int split = blockIdx.x;
    const int r = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int keys = p.position + r + 1;
    const int k0 = split * KS;
    const int nk = keys - k0 < KS ? keys - k0 : KS;
    const long part = ((long)r * p.max_splits + split) * H;
    if (nk <= 0) {
        if (t < H) {
            p.part_max[part + t] = -INFINITY;
            p.part_sum[part + t] = 0.0f;
        }
        return;
    }
    float qa[HW][LPL];
    float qr[HW];
#pragma unroll
    for (int i = 0; i < HW; ++i) {
        const int h = wave * HW + i;
        const bool hv = h < p.heads;
        if (hv) {
            load_lat<LPL>(p.query_absorbed + ((long)r * p.heads + h) * p.latent, lane, qa[i]);
        } else {
#pragma unroll
            for (int e = 0; e < LPL; ++e) qa[i][e] = 0.0f;
        }
        qr[i] = (hv && lane < p.rope) ? p.query_rope[((long)r * p.heads + h) * p.rope + lane]
                                      : 0.0f;
    }
    for (int j0 = 0; j0 < nk; j0 += KB) {
        float lv[KB][LPL];
        float rv[KB];
#pragma unroll
        for (int b = 0; b < KB; ++b) {
            const int j = j0 + b < nk ? j0 + b : nk - 1;  // clamp: duplicates are not written
            const long k = k0 + j;
            load_lat<LPL>(p.latent_cache + k * p.latent, lane, lv[b]);
            rv[b] = lane < p.rope ? p.rope_cache[k * p.rope + lane] : 0.0f;
        }
        float s[KB * HW];
#pragma unroll
        for (int b = 0; b < KB; ++b)
#pragma unroll
            for (int i = 0; i < HW; ++i) {
                float a = qr[i] * rv[b];
#pragma unroll
                for (int e = 0; e < LPL; ++e) a = fmaf(qa[i][e], lv[b][e], a);
                s[b * HW + i] = a;
            }
        butterfly_reduce<KB * HW, 64>(s, lane);
        const int vi = butterfly_index<KB * HW, 64>(lane);
        const int b = vi / HW, i = vi % HW;
        if (butterfly_writer<KB * HW, 64>(lane) && j0 + b < nk)
            prob[j0 + b][wave * HW + i] = s[0] * p.scale;
    }
    __syncthreads();
    {  // local softmax statistics: 16 lanes per head
        const int h = t >> 4, sub = t & 15;
        float m = -INFINITY;
        for (int j = sub; j < nk; j += 16) m = fmaxf(m, prob[j][h]);
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        float sum = 0.0f;
        for (int j = sub; j < nk; j += 16) {
            const float e = expf(prob[j][h] - m);
            prob[j][h] = e;
            sum += e;
        }
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
        if (sub == 0) {
            smax[h] = m;
            ssum[h] = sum;
        }
    }
    __syncthreads();
    if (t < H) {
        p.part_max[part + t] = smax[t];
        p.part_sum[part + t] = ssum[t];
    }
    for (int l = t; l < p.latent; l += blockDim.x) {
        float acc[H];
#pragma unroll
        for (int h = 0; h < H; ++h) acc[h] = 0.0f;
        for (int j0 = 0; j0 < nk; j0 += KB) {
            float v[KB];
#pragma unroll
            for (int b = 0; b < KB; ++b)
                v[b] = j0 + b < nk ? p.latent_cache[(long)(k0 + j0 + b) * p.latent + l] : 0.0f;
#pragma unroll
            for (int b = 0; b < KB; ++b) {
                // probabilities past nk are never read: v is 0 and the row is skipped
                if (j0 + b < nk) {
                    const f32x4 *pj = reinterpret_cast<const f32x4 *>(prob[j0 + b]);
#pragma unroll
                    for (int g = 0; g < H / 4; ++g) {
                        const f32x4 w = pj[g];
                        acc[4 * g + 0] = fmaf(w.x, v[b], acc[4 * g + 0]);
                        acc[4 * g + 1] = fmaf(w.y, v[b], acc[4 * g + 1]);
                        acc[4 * g + 2] = fmaf(w.z, v[b], acc[4 * g + 2]);
                        acc[4 * g + 3] = fmaf(w.w, v[b], acc[4 * g + 3]);
                    }
                }
            }
        }
#pragma unroll
        for (int h = 0; h < H; ++h)
            if (h < p.heads) p.part_lc[(part + h) * p.latent + l] = acc[h];
    }
}

// lc_h = sum_s e^{m_s - M} lc_s / sum_s e^{m_s - M} l_s over the key splits.
__global__ __launch_bounds__(128) void mla_merge_kernel(MlaParams p) {
    constexpr int H = kMlaMaxHeads;
    constexpr int KS = kMlaKeysPerSplit;
    __shared__ float weight[kMlaMaxSplitsInLds];
    __shared__ float red[2];
    const int r = blockIdx.x, h = blockIdx.y;
    const int t = threadIdx.x;
    const int keys = p.position + r + 1;
    const int ns = (keys + KS - 1) / KS;
    const long base = (long)r * p.max_splits * H + h;
    float m = -INFINITY;
    for (int s = t; s < ns; s += blockDim.x) m = fmaxf(m, p.part_max[base + (long)s * H]);
    m = wave_max(m);
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    m = fmaxf(red[0], red[1]);
    __syncthreads();
    float l = 0.0f;
    for (int s = t; s < ns; s += blockDim.x) {
        const float w = expf(p.part_max[base + (long)s * H] - m);
        weight[s] = w;
        l += w * p.part_sum[base + (long)s * H];
    }
    l = wave_sum(l);
    if ((t & 63) == 0) red[t >> 6] = l;
    __syncthreads();
    const float inv = 1.0f / (red[0] + red[1]);
    const int d = blockIdx.z * 128 + t;
    if (d < p.latent) {
        // 8 splits per step: loads first, then the FMAs in split order
        float acc = 0.0f;
        for (int s0 = 0; s0 < ns; s0 += 8) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                v[i] = s0 + i < ns ? p.part_lc[(base + (long)(s0 + i) * H) * p.latent + d] : 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (s0 + i < ns) acc = fmaf(weight[s0 + i], v[i], acc);
        }
        p.latent_context[((long)r * p.heads + h) * p.latent + d] = acc * inv;
    }
}

// ctx_h[v] = W_UV_h[v, :] . lc_h: one wave per 8 value rows, lanes over
// 8-column slices, transposed-butterfly reduction of the 8 rows.
__global__ __launch_bounds__(256) void mla_value_kernel(MlaParams p) {
    const int r = blockIdx.x, h = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int v0 = blockIdx.z * 32 + wave * 8;
    const float *lc = p.latent_context + ((long)r * p.heads + h) * p.latent;
    const int wrow0 = h * (p.nope + p.vdim) + p.nope;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int col = 8 * lane; col < p.latent; col += 512) {
        float x[8];
        const f32x4 a = load_f4(lc + col), b = load_f4(lc + col + 4);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
        float wv[8][8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int row = wrow0 + (v0 + i < p.vdim ? v0 + i : v0);
            kvb_load8(p.kv_b, row, col, p.latent, wv[i]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[i] = fmaf(x[e], wv[i][e], acc[i]);
    }
    butterfly_reduce<8, 64>(acc, lane);
    const int vi = butterfly_index<8, 64>(lane);
    if (butterfly_writer<8, 64>(lane) && v0 + vi < p.vdim)
        p.context[((long)r * p.heads + h) * p.vdim + v0 + vi] = acc[0];
}

int mla_attention_core(const MlaParams &p, hipStream_t stream) {
    if (p.heads <= 0 || p.heads > kMlaMaxHeads || p.latent <= 0 || p.latent % 64 ||
        p.latent > kMlaMaxLatent || p.rope <= 0 || p.rope > 64 || (p.rope & 1) ||
        p.nope <= 0 || p.nope > 256 || p.vdim <= 0 || p.rows <= 0 || p.max_splits <= 0 ||
        !p.latent_context || p.position < 0 || p.query_stride < (long)p.heads * (p.nope + p.rope) ||
        p.compressed_stride < p.latent + p.rope ||
        (p.position + p.rows + kMlaKeysPerSplit - 1) / kMlaKeysPerSplit >
            (p.max_splits < kMlaMaxSplitsInLds ? p.max_splits : kMlaMaxSplitsInLds))
        return kErrArgs;
    hipLaunchKernelGGL(mla_prep_kernel, dim3(p.rows, 1 + p.heads), dim3(256), 0, stream, p);
    const int splits = (p.position + p.rows + kMlaKeysPerSplit - 1) / kMlaKeysPerSplit;
    const dim3 grid(splits, p.rows);
    switch (p.latent / 64) {
    case 1: hipLaunchKernelGGL(mla_attend_kernel<1>, grid, dim3(256), 0, stream, p); break;
    case 2: hipLaunchKernelGGL(mla_attend_kernel<2>, grid, dim3(256), 0, stream, p); break;
    case 4: hipLaunchKernelGGL(mla_attend_kernel<4>, grid, dim3(256), 0, stream, p); break;
    case 8: hipLaunchKernelGGL(mla_attend_kernel<8>, grid, dim3(256), 0, stream, p); break;
    default: return kErrArgs;
    }
    hipLaunchKernelGGL(mla_merge_kernel, dim3(p.rows, p.heads, (p.latent + 127) / 128),
                       dim3(128), 0, stream, p);
    hipLaunchKernelGGL(mla_value_kernel, dim3(p.rows, p.heads, (p.vdim + 31) / 32), dim3(256), 0,
                       stream, p);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace mlh

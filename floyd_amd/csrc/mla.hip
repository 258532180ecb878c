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
// Decomposition:
//   mla_prep        one workgroup per (token row, cache append | query head):
//                   RMSNorm + RoPE into the caches; RoPE of the query's rope
//                   part; absorbed query qa_h = W_UK_h^T q_nope_h.
//   mla_attend      split-K over keys (flash-decoding): one workgroup per
//                   (key split of 64 keys, token row) scores ALL heads against
//                   each latent row it reads (the cache is read once, not once
//                   per head as moonlight_attention_scores does), keeps a local
//                   max / exp-sum and the partial latent context of every head.
//   mla_merge_value one workgroup per (token row, head): log-sum-exp merge of
//                   the splits, then ctx_h = W_UV_h lc_h.
#include "mla.h"

#include "mlh_device.h"

namespace mlh {

// Dequantised kv_b element, moonlight_weight_value (moonlight_kernels.metal:202-216).
__device__ __forceinline__ float kvb_value(const MatrixRef &m, int row, int col, int width) {
    if (m.fmt == kF32) return reinterpret_cast<const float *>(m.w)[(long)row * width + col];
    if (m.fmt == kQ8)
        return (float)reinterpret_cast<const int8_t *>(m.w)[(long)row * width + col] * m.s[row];
    const uint8_t packed = m.w[(long)row * ((width + 1) / 2) + col / 2];
    const int v = (col & 1) ? (packed >> 4) - 8 : (packed & 15) - 8;
    return (float)v * m.s[row];
}

__global__ __launch_bounds__(256) void mla_prep_kernel(MlaParams p) {
    const int r = blockIdx.x;
    const int role = blockIdx.y;  // 0: cache append, 1 + h: query head h
    const int t = threadIdx.x;
    const int pos = p.position + r;
    const int hw = p.nope + p.rope;
    if (role == 0) {
        __shared__ float part[4];
        const float *c = p.compressed + (long)r * (p.latent + p.rope);
        float ss = 0.0f;
        for (int i = t; i < p.latent; i += blockDim.x) ss += c[i] * c[i];
        ss = wave_sum(ss);
        if ((t & 63) == 0) part[t >> 6] = ss;
        __syncthreads();
        const float total = (part[0] + part[1]) + (part[2] + part[3]);
        const float inv = 1.0f / sqrtf(total / (float)p.latent + p.eps);
        float *lat = p.latent_cache + (long)pos * p.latent;
        for (int i = t; i < p.latent; i += blockDim.x) lat[i] = c[i] * inv * p.kv_norm[i];
        const int half = p.rope / 2;
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
    const float *q = p.query + ((long)r * p.heads + h) * hw;
    // RoPE of the rope part into the half layout (moonlight_kernels.metal:186-199)
    const int half = p.rope / 2;
    if (t < half) {
        const float angle = (float)pos * p.inv_freq[t];
        const float cs = cosf(angle), sn = sinf(angle);
        const float first = q[p.nope + 2 * t], second = q[p.nope + 2 * t + 1];
        float *qr = p.query_rope + ((long)r * p.heads + h) * p.rope;
        qr[t] = first * cs - second * sn;
        qr[half + t] = second * cs + first * sn;
    }
    // absorbed query: qa[l] = sum_c q_nope[c] * kv_b[h*(nope+v) + c, l]
    __shared__ float qn[256];
    __shared__ float halves[2][512];
    for (int i = t; i < p.nope; i += blockDim.x) qn[i] = q[i];
    __syncthreads();
    const int wrow = h * (p.nope + p.vdim);
    const int chalf = (p.nope + 1) / 2;
    for (int base = 0; base < p.latent; base += 512) {
        // thread -> (column quad, row half): 128 x 4 columns x 2 halves of the rows
        const int quad = t & 127, hh = t >> 7;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        const int c0 = hh * chalf, c1 = hh ? p.nope : chalf;
        for (int c = c0; c < c1; ++c) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int l = base + quad * 4 + i;
                if (l < p.latent) acc[i] = fmaf(qn[c], kvb_value(p.kv_b, wrow + c, l, p.latent), acc[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) halves[hh][quad * 4 + i] = acc[i];
        __syncthreads();
        float *qa = p.query_absorbed + ((long)r * p.heads + h) * p.latent;
        for (int i = t; i < 512 && base + i < p.latent; i += blockDim.x)
            qa[base + i] = halves[0][i] + halves[1][i];
        __syncthreads();
    }
}

// LPL latent values per lane (latent = 64 * LPL), up to kMlaMaxHeads heads.
template <int LPL>
__global__ __launch_bounds__(256) void mla_attend_kernel(MlaParams p) {
    constexpr int H = kMlaMaxHeads;
    constexpr int KS = kMlaKeysPerSplit;
    __shared__ float sc[H][KS];
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
    // query slices in registers: qa[h][lane + 64 i], q_rope[h][lane]
    float qa[H][LPL];
    float qr[H];
#pragma unroll
    for (int h = 0; h < H; ++h) {
        const bool hv = h < p.heads;
        const float *src = p.query_absorbed + ((long)r * p.heads + h) * p.latent;
#pragma unroll
        for (int i = 0; i < LPL; ++i) qa[h][i] = hv ? src[lane + 64 * i] : 0.0f;
        qr[h] = (hv && lane < p.rope) ? p.query_rope[((long)r * p.heads + h) * p.rope + lane]
                                      : 0.0f;
    }
    // scores: each wave takes every 4th key of the split
    for (int j = wave; j < nk; j += 4) {
        const int k = k0 + j;
        const float *lat = p.latent_cache + (long)k * p.latent;
        float lv[LPL];
#pragma unroll
        for (int i = 0; i < LPL; ++i) lv[i] = lat[lane + 64 * i];
        const float rv = lane < p.rope ? p.rope_cache[(long)k * p.rope + lane] : 0.0f;
        float s[H];
#pragma unroll
        for (int h = 0; h < H; ++h) {
            float a = qr[h] * rv;
#pragma unroll
            for (int i = 0; i < LPL; ++i) a = fmaf(qa[h][i], lv[i], a);
            s[h] = a;
        }
        butterfly_reduce<H, 64>(s, lane);
        if (butterfly_writer<H, 64>(lane)) sc[butterfly_index<H, 64>(lane)][j] = s[0] * p.scale;
    }
    __syncthreads();
    // local softmax statistics: 16 lanes per head (heads spread over waves)
    {
        const int h = t >> 4, sub = t & 15;
        float m = -INFINITY;
        for (int j = sub; j < nk; j += 16) m = fmaxf(m, sc[h][j]);
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        float sum = 0.0f;
        for (int j = sub; j < nk; j += 16) {
            const float e = expf(sc[h][j] - m);
            sc[h][j] = e;
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
    // partial latent context: thread -> latent dims t, t + 256, ...
    for (int l = t; l < p.latent; l += blockDim.x) {
        float acc[H];
#pragma unroll
        for (int h = 0; h < H; ++h) acc[h] = 0.0f;
        for (int j = 0; j < nk; ++j) {
            const float v = p.latent_cache[(long)(k0 + j) * p.latent + l];
#pragma unroll
            for (int h = 0; h < H; ++h) acc[h] = fmaf(sc[h][j], v, acc[h]);
        }
#pragma unroll
        for (int h = 0; h < H; ++h)
            if (h < p.heads) p.part_lc[(part + h) * p.latent + l] = acc[h];
    }
}

__global__ __launch_bounds__(256) void mla_merge_value_kernel(MlaParams p) {
    constexpr int H = kMlaMaxHeads;
    constexpr int KS = kMlaKeysPerSplit;
    __shared__ float lc[kMlaMaxLatent];
    __shared__ float weight[kMlaMaxSplitsInLds];
    __shared__ float denom;
    const int r = blockIdx.x, h = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int keys = p.position + r + 1;
    const int ns = (keys + KS - 1) / KS;
    // log-sum-exp merge of the splits
    if (wave == 0) {
        float m = -INFINITY;
        for (int s = lane; s < ns; s += 64)
            m = fmaxf(m, p.part_max[((long)r * p.max_splits + s) * H + h]);
        m = wave_max(m);
        float l = 0.0f;
        for (int s = lane; s < ns; s += 64) {
            const long idx = ((long)r * p.max_splits + s) * H + h;
            const float w = expf(p.part_max[idx] - m);
            weight[s] = w;
            l += w * p.part_sum[idx];
        }
        l = wave_sum(l);
        if (lane == 0) denom = l;
    }
    __syncthreads();
    const float inv = 1.0f / denom;
    for (int i = t; i < p.latent; i += blockDim.x) {
        float acc = 0.0f;
        for (int s = 0; s < ns; ++s)
            acc = fmaf(weight[s], p.part_lc[(((long)r * p.max_splits + s) * H + h) * p.latent + i], acc);
        lc[i] = acc * inv;
    }
    __syncthreads();
    // ctx_h[v] = sum_l lc[l] * W_UV[h*(nope+v) + nope + v, l]: one wave per value row
    const int wrow0 = h * (p.nope + p.vdim) + p.nope;
    float *ctx = p.context + ((long)r * p.heads + h) * p.vdim;
    for (int v = wave; v < p.vdim; v += 4) {
        float acc = 0.0f;
        for (int l = lane; l < p.latent; l += 64)
            acc = fmaf(lc[l], kvb_value(p.kv_b, wrow0 + v, l, p.latent), acc);
        acc = wave_sum(acc);
        if (lane == 0) ctx[v] = acc;
    }
}

int mla_attention_core(const MlaParams &p, hipStream_t stream) {
    if (p.heads <= 0 || p.heads > kMlaMaxHeads || p.latent <= 0 || p.latent % 64 ||
        p.latent > kMlaMaxLatent || p.rope <= 0 || p.rope > 64 || (p.rope & 1) ||
        p.nope <= 0 || p.nope > 256 || p.vdim <= 0 || p.rows <= 0 || p.max_splits <= 0 ||
        p.position < 0 || (p.position + p.rows + kMlaKeysPerSplit - 1) / kMlaKeysPerSplit >
                              (p.max_splits < kMlaMaxSplitsInLds ? p.max_splits
                                                                 : kMlaMaxSplitsInLds))
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
    hipLaunchKernelGGL(mla_merge_value_kernel, dim3(p.rows, p.heads), dim3(256), 0, stream, p);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace mlh

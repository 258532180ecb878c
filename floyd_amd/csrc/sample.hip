// sample.hip -- next-token choice on the device (gfx950, wave64).
//
// choose_token (moonlight_chat.c:96-131):
//   temperature <= 0 : the first index of the maximum (serial scan, strict >);
//   otherwise        : p_t = expf((logit_t - max) / T), p_t /= (float)sum_t p_t
//                      (the sum in double), qsort by descending p, keep the
//                      smallest prefix whose double sum reaches top_p, draw
//                      u * kept and return the first candidate whose running sum
//                      reaches the draw.
// Device form, each pass one sweep over HBM-resident data:
//   max_kernel    per-workgroup (value, index) maxima of 1024 logits; NaN never
//                 wins, equal values keep the lower index (the serial scan's
//                 result; a NaN at index 0 makes it 0, handled by the greedy fold)
//   greedy_kernel one workgroup folds the partials into the token
//   prob_kernel   every workgroup folds the partials (the same total order), p in
//                 fp32 from an exp in double rounded once, per-workgroup double sums
//   key_kernel    every workgroup folds the sums in the same order, p /= (float)
//                 total, sort key ~bits(p) over the 30 low bits of p's pattern
//                 (0 <= p <= 1 keeps the top two at 0): ascending keys are
//                 descending p
//   rocPRIM radix sort of the (key, token) pairs over the 30 key bits: the
//                 sort is stable, so equal p stay in token order, which is
//                 what the reference's qsort yields (glibc 2.35 sorts arrays
//                 of this size with a stable merge sort); then an inclusive
//                 scan (double) of the sorted p
//   count_kernel  the first prefix sum >= top_p ends the nucleus (atomic min)
//   pick_kernel   the first prefix sum >= u * kept inside the nucleus
//   finish_kernel the token
// Two departures, both far below the resolution of a draw: exp is rounded once
// from double (glibc's expf misrounds about 0.06 % of arguments by one ulp), and
// the double sums are tree-ordered instead of serial.
#include "sample.h"

#include <cstring>

#include <rocprim/rocprim.hpp>

#include <math.h>

namespace mlh {

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 4;
constexpr int kPerBlock = kThreads * kPerThread;
constexpr int kWaves = kThreads / 64;
// p lies in [0, 1]: bit patterns up to 0x3f800000, so 30 bits order them
constexpr uint32_t kRankMask = 0x3fffffffu;
constexpr int kRankBits = 30;

struct Best {
    float v;
    int i;
};

// The serial scan's preference: a non-NaN value beats NaN, a larger value a
// smaller one, and of equal values the lower index wins.
__device__ __forceinline__ Best better(Best a, Best b) {
    const bool an = isnan(a.v), bn = isnan(b.v);
    if (an != bn) return an ? b : a;
    if (!an && a.v != b.v) return a.v > b.v ? a : b;
    return a.i < b.i ? a : b;
}

__device__ __forceinline__ Best wave_best(Best b) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        Best other{__shfl_xor(b.v, o, 64), __shfl_xor(b.i, o, 64)};
        b = better(b, other);
    }
    return b;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
    return v;
}

// All threads of the workgroup receive the fold of the `n` partial maxima.
__device__ Best fold_best(const float *part_v, const int *part_i, int n) {
    __shared__ Best red[kWaves];
    Best b{__int_as_float(0x7fc00000), 0x7fffffff};
    for (int t = threadIdx.x; t < n; t += kThreads) b = better(b, Best{part_v[t], part_i[t]});
    b = wave_best(b);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = b;
    __syncthreads();
    Best r = red[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) r = better(r, red[w]);
    return r;
}

// All threads receive the sum of the `n` partial sums, added in the same order
// by every workgroup.
__device__ double fold_sum(const double *part, int n) {
    __shared__ double red[kWaves];
    double s = 0.0;
    for (int t = threadIdx.x; t < n; t += kThreads) s += part[t];
    s = wave_sum_f64(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = s;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ __launch_bounds__(kThreads) void max_kernel(const float *logits, int V, float *part_v,
                                                       int *part_i, int *ctl) {
    __shared__ Best red[kWaves];
    const int base = blockIdx.x * kPerBlock + threadIdx.x * kPerThread;
    Best b{__int_as_float(0x7fc00000), 0x7fffffff};
#pragma unroll
    for (int k = 0; k < kPerThread; ++k)
        if (base + k < V) b = better(b, Best{logits[base + k], base + k});
    b = wave_best(b);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = b;
    __syncthreads();
    if (threadIdx.x == 0) {
        Best r = red[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) r = better(r, red[w]);
        part_v[blockIdx.x] = r.v;
        part_i[blockIdx.x] = r.i;
        if (blockIdx.x == 0) {
            ctl[0] = V - 1;
            ctl[1] = V - 1;
            ctl[2] = 0;
        }
    }
}

__global__ __launch_bounds__(kThreads) void greedy_kernel(const float *logits, const float *part_v,
                                                          const int *part_i, int n, int *ctl) {
    const Best b = fold_best(part_v, part_i, n);
    if (threadIdx.x == 0) ctl[3] = isnan(logits[0]) ? 0 : b.i;
}

__global__ __launch_bounds__(kThreads) void prob_kernel(const float *logits, int V, float temperature,
                                                        const float *part_v, const int *part_i,
                                                        int n, float *probs, double *part_sum,
                                                        int *ctl) {
    __shared__ double red[kWaves];
    const float maximum = fold_best(part_v, part_i, n).v;
    const int base = blockIdx.x * kPerBlock + threadIdx.x * kPerThread;
    double s = 0.0;
    bool bad = !isfinite(maximum);
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        if (base + k < V) {
            const float e = (logits[base + k] - maximum) / temperature;
            const float p = (float)exp((double)e);
            bad |= isnan(p);
            probs[base + k] = p;
            s += (double)p;
        }
    }
    s = wave_sum_f64(s);
    if (bad) ctl[2] = 1;
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = s;
    __syncthreads();
    if (threadIdx.x == 0) part_sum[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ __launch_bounds__(kThreads) void key_kernel(const float *probs, int V, const double *part_sum,
                                                       int n, uint32_t *keys, int *tokens) {
    const float total = (float)fold_sum(part_sum, n);
    const int base = blockIdx.x * kPerBlock + threadIdx.x * kPerThread;
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        if (base + k < V) {
            const float p = probs[base + k] / total;
            keys[base + k] = ~__float_as_uint(p) & kRankMask;
            tokens[base + k] = base + k;
        }
    }
}

// ctl[slot] = min(ctl[slot], first i < limit with scan[i] >= threshold), where
// limit and threshold come from the nucleus (pick) or top_p (count).
template <bool PICK>
__global__ __launch_bounds__(kThreads) void search_kernel(const double *scan, int V, double top_p,
                                                          double u, int *ctl) {
    __shared__ int red[kWaves];
    int limit = V;
    double threshold = top_p;
    if (PICK) {
        limit = ctl[0] + 1;
        threshold = u * scan[limit - 1];
    }
    const int base = blockIdx.x * kPerBlock + threadIdx.x * kPerThread;
    int first = 0x7fffffff;
#pragma unroll
    for (int k = kPerThread - 1; k >= 0; --k)
        if (base + k < limit && scan[base + k] >= threshold) first = base + k;
    first = wave_min_i(first);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = first;
    __syncthreads();
    if (threadIdx.x == 0) {
        const int m = min(min(red[0], red[1]), min(red[2], red[3]));
        if (m != 0x7fffffff) atomicMin(&ctl[PICK ? 1 : 0], m);
    }
}

__global__ void finish_kernel(const int *sorted_tokens, int *ctl) {
    if (threadIdx.x == 0) ctl[3] = sorted_tokens[min(ctl[1], ctl[0])];
}

// p of a sort key, widened to double for the scan
struct KeyProb {
    __host__ __device__ double operator()(uint32_t key) const {
        return (double)__builtin_bit_cast(float, ~key & kRankMask);
    }
};

using ProbIter = rocprim::transform_iterator<const uint32_t *, KeyProb, double>;

}  // namespace

void sample_free(SampleWork *w) {
    void *bufs[] = {w->probs, w->keys, w->sorted, w->tokens, w->sorted_tokens, w->scan,
                    w->part_v, w->part_i, w->part_sum, w->ctl, w->temp};
    for (void *p : bufs)
        if (p) (void)hipFree(p);
    *w = SampleWork();
}

int sample_alloc(SampleWork *w, int vocab) {
    if (vocab <= 0 || vocab > (1 << 30)) return -1;
    sample_free(w);
    w->vocab = vocab;
    w->blocks = (vocab + kPerBlock - 1) / kPerBlock;
    const size_t V = (size_t)vocab, nb = (size_t)w->blocks;
    size_t sort_bytes = 0, scan_bytes = 0;
    bool ok =
        hipMalloc((void **)&w->probs, V * sizeof(float)) == hipSuccess &&
        hipMalloc((void **)&w->keys, V * sizeof(uint32_t)) == hipSuccess &&
        hipMalloc((void **)&w->sorted, V * sizeof(uint32_t)) == hipSuccess &&
        hipMalloc((void **)&w->tokens, V * sizeof(int)) == hipSuccess &&
        hipMalloc((void **)&w->sorted_tokens, V * sizeof(int)) == hipSuccess &&
        hipMalloc((void **)&w->scan, V * sizeof(double)) == hipSuccess &&
        hipMalloc((void **)&w->part_v, nb * sizeof(float)) == hipSuccess &&
        hipMalloc((void **)&w->part_i, nb * sizeof(int)) == hipSuccess &&
        hipMalloc((void **)&w->part_sum, nb * sizeof(double)) == hipSuccess &&
        hipMalloc((void **)&w->ctl, 4 * sizeof(int)) == hipSuccess &&
        rocprim::radix_sort_pairs(nullptr, sort_bytes, w->keys, w->sorted, w->tokens,
                                  w->sorted_tokens, (unsigned)V, 0, kRankBits) == hipSuccess &&
        rocprim::inclusive_scan(nullptr, scan_bytes, ProbIter(w->sorted, KeyProb{}), w->scan, V,
                                rocprim::plus<double>()) == hipSuccess;
    if (ok) {
        w->temp_bytes = sort_bytes > scan_bytes ? sort_bytes : scan_bytes;
        ok = hipMalloc(&w->temp, w->temp_bytes ? w->temp_bytes : 16) == hipSuccess;
    }
    if (!ok) {
        sample_free(w);
        return -3;
    }
    return 0;
}

int sample_enqueue(SampleWork *w, const float *logits, float temperature, float top_p, double u,
                   hipStream_t stream) {
    if (!w->ctl || !logits) return -1;
    const int V = w->vocab, nb = w->blocks;
    hipLaunchKernelGGL(max_kernel, dim3(nb), dim3(kThreads), 0, stream, logits, V, w->part_v,
                       w->part_i, w->ctl);
    if (!(temperature > 0.0f)) {
        hipLaunchKernelGGL(greedy_kernel, dim3(1), dim3(kThreads), 0, stream, logits, w->part_v,
                           w->part_i, nb, w->ctl);
        return hipGetLastError() == hipSuccess ? 0 : -2;
    }
    hipLaunchKernelGGL(prob_kernel, dim3(nb), dim3(kThreads), 0, stream, logits, V, temperature,
                       w->part_v, w->part_i, nb, w->probs, w->part_sum, w->ctl);
    hipLaunchKernelGGL(key_kernel, dim3(nb), dim3(kThreads), 0, stream, w->probs, V, w->part_sum,
                       nb, w->keys, w->tokens);
    size_t bytes = w->temp_bytes;
    if (rocprim::radix_sort_pairs(w->temp, bytes, w->keys, w->sorted, w->tokens, w->sorted_tokens,
                                  (unsigned)V, 0, kRankBits, stream) != hipSuccess)
        return -2;
    bytes = w->temp_bytes;
    if (rocprim::inclusive_scan(w->temp, bytes, ProbIter(w->sorted, KeyProb{}), w->scan,
                                (size_t)V, rocprim::plus<double>(), stream) != hipSuccess)
        return -2;
    hipLaunchKernelGGL(search_kernel<false>, dim3(nb), dim3(kThreads), 0, stream, w->scan, V,
                       (double)top_p, u, w->ctl);
    hipLaunchKernelGGL(search_kernel<true>, dim3(nb), dim3(kThreads), 0, stream, w->scan, V,
                       (double)top_p, u, w->ctl);
    hipLaunchKernelGGL(finish_kernel, dim3(1), dim3(64), 0, stream, w->sorted_tokens, w->ctl);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace mlh

// sample.hip -- next-token choice on the device (gfx950, wave64).
//
// choose_token (moonlight_chat.c:96-131):
//   temperature <= 0 : the first index of the maximum (serial scan, strict >);
//   otherwise        : p_t = expf((logit_t - max) / T), p_t /= (float)sum_t p_t
//                      (the sum in double), qsort by descending p, keep the
//                      smallest prefix whose double sum reaches top_p, draw
//                      u * kept and return the first candidate whose running sum
//                      reaches the draw.
// Device form, without a sort: the two prefix searches of the sorted order
// (the nucleus end, then the draw) are radix selections by probability mass.
//   Order.  p as the rank key ~bits(p) & 0x3fffffff (0 <= p <= 1 keeps the top
//   two bits at 0): ascending key is descending p, equal keys are equal p,
//   and equal p go in token order, as a stable sort leaves them (glibc
//   2.35's qsort sorts arrays of this size with a stable merge sort).
//   Mass.  Each p as the integer M = p * 2^62, truncated.  Running sums of M
//   are exact.  The reference's running sums in double are exact too while
//   every p they add is >= 2^-30 (a multiple of 2^-53) and the sum stays
//   below 1, and there "sum >= x" is "sum of M >= ceil(x * 2^62)": the
//   nucleus end, kept and the drawn candidate are the reference's.
//   Selection of the first candidate whose running sum reaches a threshold
//   T: key bits 29..22, then 21..14, by histograms of count and mass over
//   the whole vocabulary (the first bin holding a key whose inclusive
//   prefix reaches T); the keys under the selected 16-bit prefix go to one
//   workgroup, which selects bits 13..6 and 5..0 the same way and then,
//   among the keys equal to the selected one (each of mass m), the j-th in
//   token order for the first j with before + (j + 1) m >= T.
// Kernels (a round per threshold: T = top_p, then T = u * kept):
//   max_kernel     per-workgroup (value, index) maxima of 1024 logits; NaN never
//                  wins, equal values keep the lower index (the serial scan's
//                  result; a NaN at index 0 makes it 0, handled by the greedy
//                  fold); clears the selection histograms and list lengths
//   greedy_kernel  one workgroup folds the partials into the token
//   prob_kernel    every workgroup folds the partials (the same total order), p
//                  in fp32 from an exp in double rounded once, per-workgroup
//                  double sums
//   key_kernel     every workgroup folds the sums in the same order, p /=
//                  (float) total, the keys, the bits 29..22 histogram
//   level1_kernel  per round: every workgroup selects the bits 29..22 bin from
//                  the histogram (all reach the same answer), then histograms
//                  bits 21..14 of the keys in that bin
//   collect_kernel per round: selects both levels, lists the keys under that
//                  16-bit prefix with their tokens
//   final_kernel   per round, one workgroup: bits 13..6, 5..0 and the tie from
//                  the list (from all keys when the list overflowed); round 0
//                  writes round 1's threshold ceil(u * kept * 2^62), round 1
//                  the token
// Departures, all far below the resolution of a draw: exp is rounded once from
// double (glibc's expf misrounds about 0.06 % of arguments by one ulp), the
// normalising sum is tree-ordered instead of serial, and the running sums are
// exact where the reference's round (a p below 2^-30 added to a large sum).
#include "sample.h"

#include <math.h>
#include <stddef.h>

namespace mlh {

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 4;
constexpr int kPerBlock = kThreads * kPerThread;
constexpr int kWaves = kThreads / 64;

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
                                                       int *part_i, int *ctl, unsigned *clear,
                                                       int clear_words) {
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < clear_words; i += gridDim.x * kThreads)
        clear[i] = 0u;
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
        if (blockIdx.x == 0) ctl[2] = 0;
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


constexpr uint32_t kRankMask = 0x3fffffffu;
constexpr int kBins = 256;             // 8 key bits per histogram level
constexpr int kCandMax = 8192;         // list capacity per round (64 KB of LDS)
constexpr int kFinalThreads = 1024;
constexpr int kTieMax = kFinalThreads;  // equal keys ranked from the list

struct Hist {
    unsigned count[kBins];
    unsigned long long mass[kBins];
};

// The selection scratch (SampleWork::select).  max_kernel clears h0, h1 and
// n; the lists and thr1 are written before they are read.
struct Select {
    Hist h0;                               // key bits 29..22, both rounds
    Hist h1[2];                            // key bits 21..14, per round
    unsigned n[2];                         // list lengths (may exceed kCandMax)
    unsigned long long thr1;               // round 1's threshold
    unsigned long long list[2][kCandMax];  // key << 32 | token
};
constexpr int kSelectClearWords = (int)(offsetof(Select, thr1) / sizeof(unsigned));
static_assert(offsetof(Select, thr1) % sizeof(unsigned) == 0, "cleared words");

// M(p) = p * 2^62 truncated, p from its rank key
__device__ __forceinline__ unsigned long long key_mass(uint32_t key) {
    return (unsigned long long)(__uint_as_float(~key & kRankMask) * 0x1p62f);
}

struct Pick {
    int bin;                    // -1: no bin reaches T
    unsigned long long before;  // before + the mass of the bins ahead of it
    unsigned count;             // keys in the bin
};

// One full wave, histogram bins [0, 64 PL) in order: the first bin that holds
// a key and whose inclusive mass prefix, added to `before`, reaches T.  Every
// lane gets the result; *total (if given) = before + the whole mass.
template <int PL>
__device__ Pick wave_pick(const unsigned *count, const unsigned long long *mass,
                          unsigned long long before, unsigned long long T,
                          unsigned long long *total) {
    const int lane = threadIdx.x & 63;
    unsigned c[PL];
    unsigned long long m[PL], s = 0;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
        c[i] = count[PL * lane + i];
        m[i] = mass[PL * lane + i];
        s += m[i];
    }
    unsigned long long incl = s;  // inclusive prefix over lanes
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
    }
    if (total) *total = before + __shfl(incl, 63, 64);
    unsigned long long run = before + (incl - s);
    int first = -1;
    unsigned long long at = 0;
    unsigned cf = 0;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
        const unsigned long long next = run + m[i];
        if (first < 0 && c[i] > 0 && next >= T) {
            first = i;
            at = run;
            cf = c[i];
        }
        run = next;
    }
    const unsigned long long hit = __ballot(first >= 0);
    Pick r{-1, before, 0};
    if (hit) {
        const int src = __builtin_ctzll(hit);
        r.bin = __shfl(PL * lane + first, src, 64);
        r.before = __shfl(at, src, 64);
        r.count = __shfl(cf, src, 64);
    }
    return r;
}

// Levels 0 and 1 of a round, by one full wave: the key prefix (8 bits, or 16
// with level 1) whose keys hold the crossing, the mass of all keys below it,
// and T clamped to the total mass (a threshold above it keeps every
// candidate, as the reference's loop that runs to the end of the vocabulary).
struct Path {
    unsigned prefix;
    unsigned long long before, T;
};
__device__ Path descend(const Select &S, int round, unsigned long long T, bool level1) {
    unsigned long long total = 0;
    Pick a = wave_pick<4>(S.h0.count, S.h0.mass, 0, T, &total);
    if (a.bin < 0) {
        T = total;
        a = wave_pick<4>(S.h0.count, S.h0.mass, 0, T, nullptr);
    }
    Path p{a.bin < 0 ? 0u : (unsigned)a.bin, a.before, T};
    if (level1) {
        const Pick b = wave_pick<4>(S.h1[round].count, S.h1[round].mass, a.before, T, nullptr);
        p.prefix = (p.prefix << 8) | (b.bin < 0 ? 0u : (unsigned)b.bin);
        p.before = b.before;
    }
    return p;
}

__global__ __launch_bounds__(kThreads) void key_kernel(const float *probs, int V, const double *part_sum,
                                                       int n, uint32_t *keys, Select *S) {
    __shared__ unsigned cnt[kBins];
    __shared__ unsigned long long ms[kBins];
    const int t = threadIdx.x;
    cnt[t] = 0;
    ms[t] = 0;
    const float total = (float)fold_sum(part_sum, n);  // (its barrier orders the clears)
    const int base = blockIdx.x * kPerBlock + t * kPerThread;
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        if (base + k < V) {
            const float p = probs[base + k] / total;
            const uint32_t key = ~__float_as_uint(p) & kRankMask;
            keys[base + k] = key;
            atomicAdd(&cnt[key >> 22], 1u);
            atomicAdd(&ms[key >> 22], key_mass(key));
        }
    }
    __syncthreads();
    if (cnt[t]) {
        atomicAdd(&S->h0.count[t], cnt[t]);
        atomicAdd(&S->h0.mass[t], ms[t]);
    }
}

// Round `round` (threshold T0, or thr1 for round 1): bits 21..14 of the keys
// in the selected bits 29..22 bin.
__global__ __launch_bounds__(kThreads) void level1_kernel(const uint32_t *keys, int V, Select *S,
                                                          int round, unsigned long long T0) {
    __shared__ unsigned cnt[kBins];
    __shared__ unsigned long long ms[kBins];
    __shared__ unsigned sel;
    const int t = threadIdx.x;
    const int base = blockIdx.x * kPerBlock + t * kPerThread;
    uint32_t kv[kPerThread];
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) kv[k] = keys[base + k < V ? base + k : V - 1];
    cnt[t] = 0;
    ms[t] = 0;
    if (t < 64) {
        const Path p = descend(*S, round, round == 0 ? T0 : S->thr1, false);
        if (t == 0) sel = p.prefix;
    }
    __syncthreads();
    const unsigned b0 = sel;
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        if (base + k < V && (kv[k] >> 22) == b0) {
            const unsigned d = (kv[k] >> 14) & 255u;
            atomicAdd(&cnt[d], 1u);
            atomicAdd(&ms[d], key_mass(kv[k]));
        }
    }
    __syncthreads();
    if (cnt[t]) {
        atomicAdd(&S->h1[round].count[t], cnt[t]);
        atomicAdd(&S->h1[round].mass[t], ms[t]);
    }
}

// Round `round`: the keys under the selected 16-bit prefix, with their
// tokens, appended to the round's list (one counter update per wave; entries
// past kCandMax are counted, not stored).
__global__ __launch_bounds__(kThreads) void collect_kernel(const uint32_t *keys, int V, Select *S,
                                                           int round, unsigned long long T0) {
    __shared__ unsigned sel;
    const int t = threadIdx.x, lane = t & 63;
    const int base = blockIdx.x * kPerBlock + t * kPerThread;
    uint32_t kv[kPerThread];
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) kv[k] = keys[base + k < V ? base + k : V - 1];
    if (t < 64) {
        const Path p = descend(*S, round, round == 0 ? T0 : S->thr1, true);
        if (t == 0) sel = p.prefix;
    }
    __syncthreads();
    const unsigned pf = sel;
    const unsigned long long below = (1ull << lane) - 1;
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        const bool match = base + k < V && (kv[k] >> 14) == pf;
        const unsigned long long bal = __ballot(match);
        if (bal) {
            const int leader = __builtin_ctzll(bal);
            unsigned slot0 = 0;
            if (lane == leader) slot0 = atomicAdd(&S->n[round], (unsigned)__popcll(bal));
            slot0 = __shfl(slot0, leader, 64);
            if (match) {
                const unsigned slot = slot0 + (unsigned)__popcll(bal & below);
                if (slot < (unsigned)kCandMax)
                    S->list[round][slot] = ((unsigned long long)kv[k] << 32) | (unsigned)(base + k);
            }
        }
    }
}

// Exclusive prefix sum of v over the workgroup (kFinalThreads threads).
__device__ unsigned block_exclusive(unsigned v, unsigned *wsum) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    unsigned incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned x = __shfl_up(incl, o, 64);
        if (lane >= o) incl += x;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    unsigned off = 0;
    for (int w = 0; w < wave; ++w) off += wsum[w];
    return off + incl - v;
}

// Round `round`, one workgroup: the last 14 key bits and the tie.  Round 0
// writes S->thr1 = min(ceil(u * kept * 2^62), kept) (the reference's sample
// = random_unit * kept in double, as an integer threshold); round 1 writes
// the token to ctl[3].
__global__ __launch_bounds__(kFinalThreads) void final_kernel(const uint32_t *keys, int V, Select *S,
                                                              int round, unsigned long long T0, double u,
                                                              int *ctl) {
    constexpr int NT = kFinalThreads;
    __shared__ unsigned long long cand[kCandMax];
    __shared__ unsigned cnt[kBins];
    __shared__ unsigned long long ms[kBins];
    __shared__ unsigned tie_tok[kTieMax];
    __shared__ unsigned wsum[NT / 64];
    __shared__ unsigned sh_prefix, sh_count, tie_n;
    __shared__ int sh_bin;
    __shared__ unsigned long long sh_before, sh_T;
    const int t = threadIdx.x;
    if (t < 64) {
        const Path p = descend(*S, round, round == 0 ? T0 : S->thr1, true);
        if (t == 0) {
            sh_prefix = p.prefix;
            sh_before = p.before;
            sh_T = p.T;
        }
    }
    const unsigned n = S->n[round];
    const bool fits = n <= (unsigned)kCandMax;
    if (fits)
        for (unsigned i = t; i < n; i += NT) cand[i] = S->list[round][i];
    if (t < kBins) {
        cnt[t] = 0;
        ms[t] = 0;
    }
    if (t == 0) tie_n = 0;
    __syncthreads();
    unsigned prefix = sh_prefix;
    const unsigned long long T = sh_T;
    auto add = [&](uint32_t key, unsigned d) {
        atomicAdd(&cnt[d], 1u);
        atomicAdd(&ms[d], key_mass(key));
    };
    // ---- bits 13..6 of the keys under the 16-bit prefix
    if (fits) {
        for (unsigned i = t; i < n; i += NT) {
            const uint32_t key = (uint32_t)(cand[i] >> 32);
            add(key, (key >> 6) & 255u);
        }
    } else {
        for (int i = t; i < V; i += NT) {
            const uint32_t key = keys[i];
            if ((key >> 14) == prefix) add(key, (key >> 6) & 255u);
        }
    }
    __syncthreads();
    if (t < 64) {
        const Pick q = wave_pick<4>(cnt, ms, sh_before, T, nullptr);
        if (t == 0) {
            sh_bin = q.bin;
            sh_before = q.before;
        }
    }
    __syncthreads();
    prefix = (prefix << 8) | (sh_bin < 0 ? 0u : (unsigned)sh_bin);
    if (t < kBins) {
        cnt[t] = 0;
        ms[t] = 0;
    }
    __syncthreads();
    // ---- bits 5..0 of the keys under the 24-bit prefix
    if (fits) {
        for (unsigned i = t; i < n; i += NT) {
            const uint32_t key = (uint32_t)(cand[i] >> 32);
            if ((key >> 6) == prefix) add(key, key & 63u);
        }
    } else {
        for (int i = t; i < V; i += NT) {
            const uint32_t key = keys[i];
            if ((key >> 6) == prefix) add(key, key & 63u);
        }
    }
    __syncthreads();
    if (t < 64) {
        const Pick q = wave_pick<1>(cnt, ms, sh_before, T, nullptr);
        if (t == 0) {
            sh_bin = q.bin;
            sh_before = q.before;
            sh_count = q.count;
        }
    }
    __syncthreads();
    const uint32_t K = (prefix << 6) | (sh_bin < 0 ? 0u : (unsigned)sh_bin);
    const unsigned long long before = sh_before, mK = key_mass(K);
    const unsigned cK = sh_count;
    // the first j with before + (j + 1) mK >= T (j = 0 when T <= before)
    unsigned long long j = 0;
    if (T > before && mK > 0) j = (T - before + mK - 1) / mK - 1;
    if (cK > 0 && j > cK - 1) j = cK - 1;
    if (round == 0) {
        if (t == 0) {
            const unsigned long long kept = before + (j + 1) * mK;
            const double sample = u * ((double)kept * 0x1p-62);
            const double x = ceil(sample * 0x1p62);
            unsigned long long thr = x >= 0x1p64 ? ~0ull : x <= 0.0 ? 0ull : (unsigned long long)x;
            S->thr1 = thr < kept ? thr : kept;
        }
        return;
    }
    // ---- the j-th token (token order) among the keys equal to K
    if (t == 0) ctl[3] = 0;  // (only reached for inconsistent, non-finite input)
    if (fits && cK <= (unsigned)kTieMax) {
        for (unsigned i = t; i < n; i += NT) {
            if ((uint32_t)(cand[i] >> 32) == K) {
                const unsigned slot = atomicAdd(&tie_n, 1u);
                if (slot < (unsigned)kTieMax) tie_tok[slot] = (unsigned)cand[i];
            }
        }
        __syncthreads();
        const unsigned m = tie_n < (unsigned)kTieMax ? tie_n : (unsigned)kTieMax;
        if ((unsigned)t < m) {
            const unsigned mine = tie_tok[t];
            unsigned rank = 0;
            for (unsigned q = 0; q < m; ++q) rank += tie_tok[q] < mine;
            if (rank == j) ctl[3] = (int)mine;
        }
    } else {
        // thread t counts the keys equal to K in its contiguous token range;
        // the range holding the j-th is walked by its thread
        const int per = (V + NT - 1) / NT;
        const int lo = t * per < V ? t * per : V, hi = lo + per < V ? lo + per : V;
        unsigned c = 0;
        for (int i = lo; i < hi; ++i) c += keys[i] == K;
        const unsigned ex = block_exclusive(c, wsum);
        if (ex <= j && j < (unsigned long long)ex + c) {
            unsigned long long left = j - ex;
            for (int i = lo; i < hi; ++i) {
                if (keys[i] == K) {
                    if (left == 0) {
                        ctl[3] = i;
                        break;
                    }
                    --left;
                }
            }
        }
    }
}

}  // namespace

void sample_free(SampleWork *w) {
    void *bufs[] = {w->probs, w->keys, w->part_v, w->part_i, w->part_sum, w->ctl, w->select};
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
    const bool ok =
        hipMalloc((void **)&w->probs, V * sizeof(float)) == hipSuccess &&
        hipMalloc((void **)&w->keys, V * sizeof(uint32_t)) == hipSuccess &&
        hipMalloc((void **)&w->part_v, nb * sizeof(float)) == hipSuccess &&
        hipMalloc((void **)&w->part_i, nb * sizeof(int)) == hipSuccess &&
        hipMalloc((void **)&w->part_sum, nb * sizeof(double)) == hipSuccess &&
        hipMalloc((void **)&w->ctl, 4 * sizeof(int)) == hipSuccess &&
        hipMalloc(&w->select, sizeof(Select)) == hipSuccess;
    if (!ok) {
        sample_free(w);
        return -3;
    }
    return 0;
}

int sample_enqueue(SampleWork *w, const float *logits, float temperature, float top_p, double u,
                   hipStream_t stream) {
    if (!w->ctl || !w->select || !logits) return -1;
    const int V = w->vocab, nb = w->blocks;
    Select *S = static_cast<Select *>(w->select);
    hipLaunchKernelGGL(max_kernel, dim3(nb), dim3(kThreads), 0, stream, logits, V, w->part_v,
                       w->part_i, w->ctl, reinterpret_cast<unsigned *>(S), kSelectClearWords);
    if (!(temperature > 0.0f)) {
        hipLaunchKernelGGL(greedy_kernel, dim3(1), dim3(kThreads), 0, stream, logits, w->part_v,
                           w->part_i, nb, w->ctl);
        return hipGetLastError() == hipSuccess ? 0 : -2;
    }
    // round 0's threshold: ceil(top_p * 2^62) (top_p <= 0: the first candidate;
    // beyond the total mass: clamped to it on the device)
    const double tp = (double)top_p * 0x1p62;
    const unsigned long long T0 =
        !(tp > 0.0) ? 0ull : tp >= 0x1p64 ? ~0ull : (unsigned long long)ceil(tp);
    hipLaunchKernelGGL(prob_kernel, dim3(nb), dim3(kThreads), 0, stream, logits, V, temperature,
                       w->part_v, w->part_i, nb, w->probs, w->part_sum, w->ctl);
    hipLaunchKernelGGL(key_kernel, dim3(nb), dim3(kThreads), 0, stream, w->probs, V, w->part_sum,
                       nb, w->keys, S);
    for (int round = 0; round < 2; ++round) {
        hipLaunchKernelGGL(level1_kernel, dim3(nb), dim3(kThreads), 0, stream, w->keys, V, S, round,
                           T0);
        hipLaunchKernelGGL(collect_kernel, dim3(nb), dim3(kThreads), 0, stream, w->keys, V, S, round,
                           T0);
        hipLaunchKernelGGL(final_kernel, dim3(1), dim3(kFinalThreads), 0, stream, w->keys, V, S,
                           round, T0, u, w->ctl);
    }
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace mlh

// mlh_device.h -- device building blocks shared by the Moonlight HIP kernels
// (gfx950 / CDNA4, wave64).  Header-only; included by the .hip sources.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlh {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// 16-byte global load.  Weights are streamed exactly once per launch, so the
// load is marked non-temporal to keep L2 / MALL for the activations.
__device__ __forceinline__ u32x4 load_stream16(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// 16-byte load through the global address space.  Pointers that reach a
// kernel through a table in memory are generic; a generic (flat) load also
// counts against the LDS wait counter, so a wait for LDS reads would wait for
// every outstanding flat load as well.
__device__ __forceinline__ u32x4 load_global16(const void *p) {
    return *(const __attribute__((address_space(1))) u32x4 *)(p);
}

__device__ __forceinline__ float load_global_f32(const float *p) {
    return *(const __attribute__((address_space(1))) float *)(p);
}

// 4-byte store through the global address space (a flat store would also
// count against the LDS wait counter, see load_global16).
__device__ __forceinline__ void store_global(float *p, float v) {
    *(__attribute__((address_space(1))) float *)(p) = v;
}

__device__ __forceinline__ f32x4 load_f4(const float *p) {
    return *reinterpret_cast<const f32x4 *>(p);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Wave reductions on DPP only (no LDS instruction: with an LDS DMA in flight
// the compiler would wait for it before any LDS instruction, ds_bpermute
// included).  Lane 63 ends with the total; every lane gets it by readlane.
#define MLH_DPP(v, ctrl, rmask) \
    __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), ctrl, rmask, 0xF, false))
__device__ __forceinline__ float dpp_wave_sum(float v) {
    v += MLH_DPP(v, 0xB1, 0xF);   // quad_perm [1,0,3,2]
    v += MLH_DPP(v, 0x4E, 0xF);   // quad_perm [2,3,0,1]
    v += MLH_DPP(v, 0x141, 0xF);  // row_half_mirror
    v += MLH_DPP(v, 0x140, 0xF);  // row_mirror
    // row_bcast15 / row_bcast31 write only the masked rows: the others add
    // their own value, so they are not read below
    const float b15 = MLH_DPP(v, 0x142, 0xA);
    v = (threadIdx.x & 16) ? v + b15 : v;
    const float b31 = MLH_DPP(v, 0x143, 0xC);
    v = (threadIdx.x & 32) ? v + b31 : v;
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float dpp_wave_max(float v) {
    v = fmaxf(v, MLH_DPP(v, 0xB1, 0xF));
    v = fmaxf(v, MLH_DPP(v, 0x4E, 0xF));
    v = fmaxf(v, MLH_DPP(v, 0x141, 0xF));
    v = fmaxf(v, MLH_DPP(v, 0x140, 0xF));
    v = fmaxf(v, MLH_DPP(v, 0x142, 0xA));
    v = fmaxf(v, MLH_DPP(v, 0x143, 0xC));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
#undef MLH_DPP

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Sum over groups of G lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = G / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Transposed butterfly: NV partial sums per lane, reduced over groups of G
// lanes.  After the call v[0] of a lane holds the group total of value index
// butterfly_index<NV, G>(lane); every lane of the group ends up holding one
// total (NV <= G), lanes whose low bits are zero are the designated writers.
// Step s exchanges half of the live values across lane offset G >> (s + 1);
// the recursion keeps every array index a compile-time constant (a runtime
// index would turn each access into a compare/select chain over the array).
template <int NV, int G, int STEP>
struct ButterflyStep {
    static __device__ __forceinline__ void run(float (&v)[NV], int lane) {
        constexpr int N = NV >> STEP;
        if constexpr (N > 1) {
            constexpr int HALF = N / 2;
            constexpr int O = G >> (STEP + 1);
            const bool upper = (lane & O) != 0;
#pragma unroll
            for (int i = 0; i < HALF; ++i) {
                const float send = upper ? v[i] : v[i + HALF];
                const float keep = upper ? v[i + HALF] : v[i];
                v[i] = keep + __shfl_xor(send, O, kWave);
            }
            ButterflyStep<NV, G, STEP + 1>::run(v, lane);
        } else {
#pragma unroll
            for (int o = G >> (STEP + 1); o >= 1; o >>= 1) v[0] += __shfl_xor(v[0], o, kWave);
        }
    }
};

template <int NV, int G>
__device__ __forceinline__ void butterfly_reduce(float (&v)[NV], int lane) {
    static_assert(NV <= G, "more values than lanes in the group");
    static_assert((NV & (NV - 1)) == 0, "NV must be a power of two");
    ButterflyStep<NV, G, 0>::run(v, lane);
}

// Value index a lane holds after butterfly_reduce<NV, G>.
template <int NV, int G>
__device__ __forceinline__ int butterfly_index(int lane) {
    int idx = 0, n = NV, o = G / 2;
    while (n > 1) {
        n >>= 1;
        if (lane & o) idx += n;
        o >>= 1;
    }
    return idx;
}

// Lanes that write: the bits below the last transposed offset are zero.
template <int NV, int G>
__device__ __forceinline__ bool butterfly_writer(int lane) {
    int steps = 0;
    while ((1 << steps) < NV) ++steps;
    int low = G >> steps;  // lanes in the final plain-reduction subgroup
    return (lane & (low - 1)) == 0;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Hand-off between the workgroups of one launch: every workgroup stores its
// shares with agent-scope atomic stores, arrives at a counter, and the
// workgroup that arrives last reads all the shares with agent-scope atomic
// loads (and resets the counter for the next launch).  On gfx950 agent-scope
// stores and loads act at the device-coherent level (they bypass the
// non-coherent state of the per-XCD L2 caches), so once a store has
// completed, an agent-scope load from any XCD returns it.  The order is kept
// at both levels:
//  - hardware: every thread waits for its own stores (s_waitcnt) before the
//    workgroup barrier that precedes the counter increment;
//  - compiler: the empty asm statements clobber memory, so no load or store
//    moves across the wait, the barriers or the increment.
// An agent-scope release / acquire on the counter states the same order in
// the HIP memory model, but on gfx950 each one writes back or invalidates
// the XCD's L2 (buffer_wbl2 / buffer_inv sc1) in every workgroup; measured
// on a 768-workgroup split-k GEMV: 17.4 us against 6.1 us with this form.
// Every thread of the workgroup calls it; returns whether this workgroup
// arrived last (the same value in every thread).
__device__ __forceinline__ bool agent_handoff_arrive(int *count, int total) {
    __shared__ int arrived_last;
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        arrived_last = __hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT) == total - 1;
    __syncthreads();
    asm volatile("" ::: "memory");
    return arrived_last != 0;
}

}  // namespace mlh

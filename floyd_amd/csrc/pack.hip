// pack.hip -- device-side container packing and synthetic weight generation.
//
// quantize_rows restates quant_int8 / quant_int4 (tools/convert_moonlight.py:46-66)
// bit for bit: per row amax = max|w|, s = max(amax / qmax, 1e-8f) in f32,
// q = clip(rint(w / s)) with round-half-even, int8 bytes or q+8 nibbles (even
// column low, odd width leaves the last high nibble 0).  Used to build
// synthetic containers directly in HBM (the 17 GB Moonlight q8 model would
// otherwise have to be generated and copied through the host).
#include "mlh_device.h"
#include "mlh_host.h"

namespace mlh {

__global__ __launch_bounds__(256) void quantize_rows_kernel(int bits, const float *w, int rows,
                                                            int cols, uint8_t *q, float *s) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    if (row >= rows) return;
    const float *src = w + (long)row * cols;
    float amax = 0.0f;
    for (int c = lane; c < cols; c += kWave) amax = fmaxf(amax, fabsf(src[c]));
    amax = wave_max(amax);
    const float qmax = bits == 8 ? 127.0f : 7.0f;
    float scale = amax / qmax;
    scale = scale > 1e-8f ? scale : 1e-8f;
    if (lane == 0) s[row] = scale;
    if (bits == 8) {
        uint8_t *dst = q + (long)row * cols;
        for (int c = lane; c < cols; c += kWave) {
            float v = rintf(src[c] / scale);
            v = fminf(fmaxf(v, -128.0f), 127.0f);
            dst[c] = (uint8_t)(int8_t)(int)v;
        }
    } else {
        const int row_bytes = (cols + 1) / 2;
        uint8_t *dst = q + (long)row * row_bytes;
        for (int j = lane; j < row_bytes; j += kWave) {
            float v0 = fminf(fmaxf(rintf(src[2 * j] / scale), -8.0f), 7.0f);
            unsigned byte = (unsigned)((int)v0 + 8);
            if (2 * j + 1 < cols) {
                float v1 = fminf(fmaxf(rintf(src[2 * j + 1] / scale), -8.0f), 7.0f);
                byte |= (unsigned)((int)v1 + 8) << 4;
            }
            dst[j] = (uint8_t)byte;
        }
    }
}

int quantize_rows(int bits, const float *w, int rows, int cols, uint8_t *q, float *s,
                  hipStream_t stream) {
    if ((bits != 8 && bits != 4) || !w || !q || !s || rows <= 0 || cols <= 0) return kErrArgs;
    const int blocks = (rows + 3) / 4;
    hipLaunchKernelGGL(quantize_rows_kernel, dim3(blocks), dim3(256), 0, stream, bits, w, rows,
                       cols, q, s);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

__device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t k) {
    uint64_t z = seed + (k + 1) * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float bf16_round(float x) {
    unsigned u = __float_as_uint(x);
    if ((u & 0x7F800000u) == 0x7F800000u) return x;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return __uint_as_float(u & 0xFFFF0000u);
}

__global__ __launch_bounds__(256) void fill_normal_kernel(float *out, int64_t n, uint64_t seed,
                                                          float mean, float stdv, int bf16) {
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        uint64_t a = splitmix64_at(seed, 2 * (uint64_t)i);
        uint64_t b = splitmix64_at(seed, 2 * (uint64_t)i + 1);
        double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53;
        double u2 = (double)(b >> 11) * 0x1.0p-53;
        double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        float v = (float)((double)mean + (double)stdv * z);
        out[i] = bf16 ? bf16_round(v) : v;
    }
}

int fill_normal(float *out, int64_t n, uint64_t seed, float mean, float stdv, int bf16,
                hipStream_t stream) {
    if (!out || n < 0) return kErrArgs;
    if (n == 0) return kOk;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fill_normal_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, out, n,
                       seed, mean, stdv, bf16);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace mlh

namespace mlh {

// Plain 16-byte streaming copy: the bandwidth yardstick for the GEMVs and the
// calibration kernel for rocprof FETCH_SIZE / WRITE_SIZE readings.
__global__ __launch_bounds__(256) void copy16_kernel(const u32x4 *src, u32x4 *dst, long n) {
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (long)gridDim.x * blockDim.x)
        __builtin_nontemporal_store(load_stream16(src + i), dst + i);
}

// Read-only streaming yardstick: every workgroup folds its share of `src`
// into one word.  Measures what pure HBM reads of a given size cost,
// launch ramp and tail included (the ceiling for a GEMV of that size).
__global__ __launch_bounds__(256) void read16_kernel(const u32x4 *src, long n, unsigned *out) {
    unsigned acc = 0;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (long)gridDim.x * blockDim.x) {
        u32x4 v = load_stream16(src + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    acc = __reduce_xor_sync(~0ull, acc);
    if ((threadIdx.x & 63) == 0) out[blockIdx.x * 4 + threadIdx.x / 64] = acc;
}

int read16(const void *src, size_t bytes, int blocks, unsigned *out, hipStream_t stream) {
    if (!src || !out || bytes % 16 || blocks <= 0 || ((uintptr_t)src & 15)) return kErrArgs;
    hipLaunchKernelGGL(read16_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const u32x4 *>(src), (long)(bytes / 16), out);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int copy16(const void *src, void *dst, size_t bytes, hipStream_t stream) {
    if (!src || !dst || bytes % 16 || ((uintptr_t)src | (uintptr_t)dst) & 15) return kErrArgs;
    const long n = (long)(bytes / 16);
    long blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(copy16_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const u32x4 *>(src), static_cast<u32x4 *>(dst), n);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // namespace mlh

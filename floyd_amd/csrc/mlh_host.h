// mlh_host.h -- host-side interface of the Moonlight HIP kernels (internal).
// The public C ABI (include/*.h) is implemented on top of these launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace mlh {

enum Fmt { kF32 = 0, kQ8 = 1, kQ4 = 2 };
enum Epilogue { kEpiPlain = 0, kEpiResidual = 1, kEpiSiluDual = 2 };
enum Status { kOk = 0, kErrArgs = -1, kErrLaunch = -2, kErrDevice = -3, kErrSize = -4 };

constexpr int kMaxGemvRows = 4;

// y[b, o] = epilogue((sum_i xn[b, i] * W[o, i]) * s[o]) for b < rows, where
// xn = RMSNorm(x) * norm_w when norm_w is set, else x.
struct GemvParams {
    int fmt = kQ8;
    const uint8_t *w = nullptr;   // [O, row_bytes]
    const float *s = nullptr;     // [O] (unused for f32)
    const uint8_t *w2 = nullptr;  // up projection for kEpiSiluDual
    const float *s2 = nullptr;
    int O = 0;                    // output width (rows of W)
    int I = 0;                    // input width
    int rows = 0;                 // token rows
    const float *x = nullptr;
    long x_stride = 0;            // floats between token rows of x
    const float *norm_w = nullptr;
    float eps = 1e-5f;
    float *y = nullptr;
    long y_stride = 0;
    const float *resid = nullptr;  // kEpiResidual: y = resid + result
    long resid_stride = 0;
    int epilogue = kEpiPlain;
    // optional (q8 / q4): x already split into limb rows (limb_quantise_rows,
    // same format and width), row stride limb_stride bytes; norm_w is then
    // already applied
    const unsigned char *limbs = nullptr;
    long limb_stride = 0;
    // optional, one token row of a plain or residual epilogue on the int8
    // matrix-core kernels (gemv_router_ok): router logit partials of the
    // output row y for the next MoE layer's router.  Workgroup j of the
    // launch writes router_parts[e * n + j] = sum over its output rows o of
    // router_w[e, o] * (y[o] * router_nw[o]) for e < router_experts and
    // router_parts[router_experts * n + j] = sum of y[o]^2 (n = the launch's
    // workgroups, gemv_router_parts)
    const float *router_w = nullptr;   // [router_experts, O] f32
    const float *router_nw = nullptr;  // [O] the router input's RMSNorm weight
    float *router_parts = nullptr;
    int router_experts = 0;
};

int gemv(const GemvParams &p, hipStream_t stream);
// Whether gemv() can write router logit partials for p (router fields
// aside), and how many partials per expert it then writes.
bool gemv_router_ok(const GemvParams &p);
int gemv_router_parts(const GemvParams &p);

struct GemvPlan;
// Launch geometry the planner picks for a GEMV shape (exposed for the grouped
// expert launches, which share the GEMV core).
GemvPlan plan_gemv(int fmt, int O, int I, int rows, bool dual);
std::string gemv_kernel_name(int fmt, int O, int I, int rows, bool dual);

// Packs f32 rows like tools/convert_moonlight.py:46-66 (bits 8 or 4).
int quantize_rows(int bits, const float *w, int rows, int cols, uint8_t *q, float *s,
                  hipStream_t stream);
// out[i] = bf16_round(mean + std * N(0,1)) from a counter-based generator
// (synthetic weights; the distribution, not the stream, is the contract).
int fill_normal(float *out, int64_t n, uint64_t seed, float mean, float std, int bf16,
                hipStream_t stream);

// dst = src with 16-byte non-temporal loads/stores (bandwidth yardstick).
int copy16(const void *src, void *dst, size_t bytes, hipStream_t stream);
// Reads `bytes` of src with `blocks` workgroups (out: blocks*4 words).
int read16(const void *src, size_t bytes, int blocks, unsigned *out, hipStream_t stream);

}  // namespace mlh

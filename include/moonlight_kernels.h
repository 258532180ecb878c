/*
 * moonlight_kernels.h -- kernel-level C ABI of the MI355X Moonlight library.
 *
 * These entry points take DEVICE pointers (from mlk_malloc) and run on the
 * library's HIP stream; they are what moonlight_hip.h's session runtime is
 * built from, exposed for callers that keep their own buffers in HBM (and for
 * the parity tests and bench).  Every function returns 0 on success or a
 * negative status (-1 bad arguments, -2 launch failure, -3 device error,
 * -4 size limit); mlk_last_error() describes the last failure.
 *
 * Reference interfaces replaced (paths in c4pt0r/floyd):
 *   mlk_gemv           moonlight_matmul_f32 / _q8_reduction / _q4
 *                      (moonlight_kernels.metal:43-130) as encoded by
 *                      encode_matmul_at (moonlight_metal.m:164-197)
 *   mlk_gemv_swiglu    gate + up matmuls + moonlight_silu_multiply
 *                      (moonlight_metal.m:459-472, moonlight_kernels.metal:533-541)
 *   mlk_route_topk     moonlight_route_sigmoid_topk (moonlight_kernels.metal:469-512)
 *                      = moe_route_select + moe_route_finalize (moe_route.h:47-99)
 *   mlk_quantize       quant_int8 / quant_int4 (tools/convert_moonlight.py:46-66)
 *   mlk_sample         choose_token (moonlight_chat.c:96-131), the caller-side
 *                      sampler, on device logits
 */
#ifndef MOONLIGHT_KERNELS_H
#define MOONLIGHT_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { MLK_F32 = 0, MLK_Q8 = 1, MLK_Q4 = 2 };

/* ---- device plumbing (no counterpart in the reference: Metal used shared
 *      memory buffers, moonlight_metal.m:733-755) ---------------------------- */
int mlk_init(void);
const char *mlk_device_name(void);
const char *mlk_last_error(void);
void *mlk_malloc(size_t bytes);
int mlk_free(void *ptr);
int mlk_memcpy_h2d(void *dst, const void *src, size_t bytes);
int mlk_memcpy_d2h(void *dst, const void *src, size_t bytes);
int mlk_memcpy_d2d(void *dst, const void *src, size_t bytes);
int mlk_memset(void *dst, int value, size_t bytes);
int mlk_synchronize(void);

/* ---- dequant matmul ------------------------------------------------------
 * y[b, o] = (sum_i xn[b, i] * W[o, i]) * s[o] (+ resid[b, o]) for b < rows,
 * with W f32 [O, I], int8 [O, I] or packed int4 [O, ceil(I/2)] and one f32
 * scale per output row; xn = RMSNorm(x) * norm_w when norm_w != NULL
 * (moonlight_kernels.metal:23-41), else x.  x, y, resid are dense [rows, *]. */
int mlk_gemv(int fmt, const void *w, const float *s, const float *x, float *y,
             int out_width, int in_width, int rows, const float *norm_w,
             float eps, const float *resid);
/* h[b, j] = silu(gate_j . xn_b) * (up_j . xn_b), gate/up of one format. */
int mlk_gemv_swiglu(int fmt, const void *w_gate, const float *s_gate,
                    const void *w_up, const float *s_up, const float *x,
                    float *h, int out_width, int in_width, int rows,
                    const float *norm_w, float eps);
/* Name of the kernel instantiation mlk_gemv (swiglu = 0) or mlk_gemv_swiglu
 * (swiglu = 1) launches for this shape, as profilers print it; written into
 * name[name_size]. */
int mlk_gemv_kernel_name(int fmt, int out_width, int in_width, int rows,
                         int swiglu, char *name, size_t name_size);
/* Average device time per launch (microseconds) of `iters` back-to-back
 * mlk_gemv launches that rotate over n_copies weight copies (defeats the
 * 256 MB last-level cache), measured with HIP events on the library stream.
 * use_graph != 0 replays the launches from one captured hipGraph. */
int mlk_time_gemv(int fmt, const void *const *w_copies,
                  const float *const *s_copies, int n_copies, const float *x,
                  float *y, int out_width, int in_width, int rows, int warmup,
                  int iters, int use_graph, double *avg_us);

/* Average device time per launch (microseconds) of a plain 16-byte streaming
 * copy of `bytes` (rotating over n_buffers source/destination pairs): the
 * measured HBM yardstick reported beside the GEMV roofline. */
int mlk_time_copy(void *const *src, void *const *dst, int n_buffers,
                  size_t bytes, int warmup, int iters, double *avg_us);

/* Same for a read-only stream of `bytes` split over `blocks` workgroups
 * (scratch: blocks * 4 words of device memory): the ceiling a GEMV reading
 * that many bytes can reach, launch ramp and tail included. */
int mlk_time_read(void *const *src, int n_buffers, size_t bytes, int blocks,
                  unsigned *scratch, int warmup, int iters, double *avg_us);

/* ---- routing --------------------------------------------------------------
 * Sigmoid top-k of rows x experts router logits: ids[r, k] is the expert with
 * the k-th largest sigmoid(logit) + bias (lower index on ties; NaN and -inf
 * never taken, -1 when fewer than top_k can be), weights[r, k] its sigmoid
 * score, divided by the row's sum (+ 1e-20) when normalize, times
 * routed_scale.  Runs the decode path's routing kernels and waits for them. */
int mlk_route_topk(const float *logits, const float *bias, int rows, int experts,
                   int top_k, int normalize, float routed_scale, int *ids,
                   float *weights);

/* ---- token choice ---------------------------------------------------------
 * The token choose_token (moonlight_chat.c:96-131) picks from `vocab` device
 * logits with the caller's draw u in [0, 1) (random_unit,
 * moonlight_chat.c:89-94): the first index of the maximum when temperature
 * <= 0, else the top-p draw.  The device sampler that
 * moonlight_session_sample runs; writes *token (host memory) and waits.
 * Non-finite logits under a top-p draw return -1 ("logits are not finite"). */
int mlk_sample(const float *logits, int vocab, float temperature, float top_p,
               double u, int *token);

/* ---- packing / synthetic weights ---------------------------------------- */
int mlk_quantize(int bits, const float *w, int rows, int cols, uint8_t *q,
                 float *s);
int mlk_fill_normal(float *out, int64_t n, uint64_t seed, float mean,
                    float std, int bf16);

#ifdef __cplusplus
}
#endif
#endif

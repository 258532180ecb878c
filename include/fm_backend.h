/*
 * fm_backend.h -- the legacy q8/q4 matmul C API on MI355X.
 *
 * Same ABI as floyd's backend_metal.h:15-41 (fm_init, fm_device_name,
 * fm_matmul_q8/q4 and the DeepSeek-V4 fp8/fp4 entry points), so callers such
 * as deepseek_v4_quant.h:110-117 and tests/test_backend_metal.c link against
 * this library unchanged.
 *
 *   fm_init                     backend_metal.m:29-45   1 = ready, 0 = no gfx950 device
 *   fm_device_name              backend_metal.m:46      borrowed string
 *   fm_matmul_q8 / fm_matmul_q4 backend_metal.m:124-127 y[S,O] = x[S,I] W[O,I]^T * s[O];
 *        host pointers in and out, synchronous.  cache = 1 keeps a device copy
 *        of (w, s) keyed by the host pointer for the life of the process
 *        (thread-safe, as backend_metal.m:19-70); cache = 0 uploads per call.
 *   fm_matmul_deepseek_v4_fp8 / _fp4  backend_metal.m:128-139: the DeepSeek-V4
 *        formats are outside this library's scope; they return 0, which
 *        deepseek_v4_quant.h:110-117 treats as "use the CPU path".
 */
#ifndef FM_BACKEND_H
#define FM_BACKEND_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int fm_init(void);
const char *fm_device_name(void);
void fm_matmul_q8(float *y, const float *x, const int8_t *w, const float *s,
                  int O, int I, int S, int cache);
void fm_matmul_q4(float *y, const float *x, const uint8_t *w, const float *s,
                  int O, int I, int S, int cache);
int fm_matmul_deepseek_v4_fp8(float *y, const float *x, const uint8_t *w,
                              const uint8_t *s, int O, int I, int S,
                              int block_size);
int fm_matmul_deepseek_v4_fp4(float *y, const float *x, const uint8_t *w,
                              const uint8_t *s, int O, int I, int S);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (serving loops and harnesses that forbid hipMalloc): fm_matmul_q8
 * (bits = 8) or fm_matmul_q4 (bits = 4) with cache = 0, the same kernels and
 * results, but x, y, w and s are staged in a static device array of
 * FM_STATIC_SCRATCH_BYTES per GPU (held from load to process end) instead of
 * library-allocated memory; the call allocates nothing.  Limit: the staging,
 * 256-byte aligned S*I*4 + S*O*4 + weight bytes, plus O*4, must fit the array
 * (e.g. a q8 [11264 x 2048] matrix with S <= 32).  Returns 1, or 0 with y
 * filled with NaN and the reason in mlk_last_error() (bad arguments, sizes
 * beyond the limit, device failure).  Synchronous.  The array keeps the last
 * call's contents; every byte a call reads is written by that call first.
 * Calls on one GPU share the array, so overlapping calls would race: calls of
 * one process are serialised by a lock. */
#define FM_STATIC_SCRATCH_BYTES (32u << 20)
int fm_matmul_static(int bits, float *y, const float *x, const void *w,
                     const float *s, int O, int I, int S);

#ifdef __cplusplus
}
#endif
#endif

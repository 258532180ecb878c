// fm_backend.cpp -- the legacy synchronous q8/q4 matmul API (include/fm_backend.h)
// over the HIP GEMV.  Mirrors backend_metal.m:19-139: weights optionally cached
// by host pointer (cache = 1), transient otherwise; x and y always transient.
#include "device_context.h"
#include "mlh_host.h"
#include "../../include/fm_backend.h"

#include <cmath>
#include <cstring>
#include <limits>
#include <mutex>
#include <unordered_map>

namespace {

struct CachedWeight {
    void *w = nullptr;
    float *s = nullptr;
};

std::mutex g_mutex;  // guards every device's cache and staging buffer

// Per device: the weights cached by host pointer and the staging buffer of
// x, y and transient weights.
struct DeviceState {
    std::unordered_map<const void *, CachedWeight> cache;
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
};
constexpr int kMaxDevices = 64;
DeviceState g_state[kMaxDevices];

bool ensure_scratch(DeviceState &d, size_t bytes) {
    if (bytes <= d.scratch_bytes) return true;
    if (d.scratch) (void)hipFree(d.scratch);
    d.scratch = nullptr;
    d.scratch_bytes = 0;
    if (hipMalloc(&d.scratch, bytes) != hipSuccess) return false;
    d.scratch_bytes = bytes;
    return true;
}

void fill_nan(float *y, long count) {
    const float nan = std::numeric_limits<float>::quiet_NaN();
    for (long i = 0; i < count; ++i) y[i] = nan;
}

void run(int fmt, float *y, const float *x, const void *w, size_t w_bytes, const float *s,
         int O, int I, int S, int cache) {
    if (!y) return;
    if (!x || !w || !s || O <= 0 || I <= 0 || S <= 0) {
        mlh::set_last_error("fm_matmul: invalid arguments");
        if (O > 0 && S > 0) fill_nan(y, (long)O * S);
        return;
    }
    mlh::DeviceContext *ctx = mlh::context();
    if (!ctx) {
        fill_nan(y, (long)O * S);
        return;
    }
    if (ctx->device >= kMaxDevices) {
        mlh::set_last_error("fm_matmul: device index out of range");
        fill_nan(y, (long)O * S);
        return;
    }
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState &d = g_state[ctx->device];
    hipStream_t st = ctx->stream;
    const size_t x_bytes = (size_t)S * I * sizeof(float);
    const size_t y_bytes = (size_t)S * O * sizeof(float);
    auto align = [](size_t v) { return (v + 255) & ~(size_t)255; };
    CachedWeight dev;
    bool transient = true;
    if (cache) {
        auto it = d.cache.find(w);
        if (it != d.cache.end()) {
            dev = it->second;  // a hit ignores sizes: one stable pointer per tensor
            transient = false;
        }
    }
    size_t need = align(x_bytes) + align(y_bytes);
    if (transient && !cache) need += align(w_bytes) + align((size_t)O * sizeof(float));
    bool ok = ensure_scratch(d, need);
    char *base = static_cast<char *>(d.scratch);
    if (ok && transient) {
        if (cache) {
            ok = hipMalloc(&dev.w, w_bytes) == hipSuccess &&
                 hipMalloc((void **)&dev.s, (size_t)O * sizeof(float)) == hipSuccess;
        } else {
            dev.w = base + align(x_bytes) + align(y_bytes);
            dev.s = reinterpret_cast<float *>(base + align(x_bytes) + align(y_bytes) +
                                              align(w_bytes));
        }
        ok = ok && hipMemcpyAsync(dev.w, w, w_bytes, hipMemcpyHostToDevice, st) == hipSuccess &&
             hipMemcpyAsync(dev.s, s, (size_t)O * sizeof(float), hipMemcpyHostToDevice, st) ==
                 hipSuccess;
        if (ok && cache) d.cache[w] = dev;
    }
    float *dx = reinterpret_cast<float *>(base);
    float *dy = reinterpret_cast<float *>(base + align(x_bytes));
    if (ok) ok = hipMemcpyAsync(dx, x, x_bytes, hipMemcpyHostToDevice, st) == hipSuccess;
    if (ok) {
        mlh::GemvParams p;
        p.fmt = fmt;
        p.w = static_cast<const uint8_t *>(dev.w);
        p.s = dev.s;
        p.O = O;
        p.I = I;
        p.rows = S;
        p.x = dx;
        p.x_stride = I;
        p.y = dy;
        p.y_stride = O;
        ok = mlh::gemv(p, st) == mlh::kOk;
    }
    if (ok) ok = hipMemcpyAsync(y, dy, y_bytes, hipMemcpyDeviceToHost, st) == hipSuccess;
    if (ok) ok = hipStreamSynchronize(st) == hipSuccess;
    if (!ok) {
        mlh::set_last_error("fm_matmul: device failure");
        fill_nan(y, (long)O * S);
    }
}

}  // namespace

namespace mlh {
bool fm_static_setup();  // fm_static.hip
}

extern "C" {

// Also looks up the device address of fm_matmul_static's static scratch.
int fm_init(void) { return mlh::context() && mlh::fm_static_setup() ? 1 : 0; }

const char *fm_device_name(void) {
    mlh::DeviceContext *ctx = mlh::context();
    return ctx ? ctx->name.c_str() : "(none)";
}

void fm_matmul_q8(float *y, const float *x, const int8_t *w, const float *s, int O, int I,
                  int S, int cache) {
    run(mlh::kQ8, y, x, w, (size_t)O * I, s, O, I, S, cache);
}

void fm_matmul_q4(float *y, const float *x, const uint8_t *w, const float *s, int O, int I,
                  int S, int cache) {
    run(mlh::kQ4, y, x, w, (size_t)O * ((I + 1) / 2), s, O, I, S, cache);
}

int fm_matmul_deepseek_v4_fp8(float *, const float *, const uint8_t *, const uint8_t *, int,
                              int, int, int) {
    return 0;
}

int fm_matmul_deepseek_v4_fp4(float *, const float *, const uint8_t *, const uint8_t *, int,
                              int, int) {
    return 0;
}

}  // extern "C"

// fm_static.hip -- fm_matmul_static (include/fm_backend.h): the q8 / q4
// matmul of fm_matmul_q8 / fm_matmul_q4 (cache = 0) for callers that cannot
// allocate device memory.  x, y, the weights and their scales are staged in
// `scratch`, a static device array of FM_STATIC_SCRATCH_BYTES that every GPU
// holds from module load to process end, instead of the library-allocated
// staging of fm_backend.cpp; the call itself allocates nothing.
#include "device_context.h"
#include "mlh_host.h"
#include "../../include/fm_backend.h"

#include <cstdio>
#include <limits>
#include <mutex>

namespace {

constexpr size_t kScratchBytes = FM_STATIC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

// Host code may not use this name as a device address (it is a host-side
// stand-in); the address of each GPU's copy comes from hipGetSymbolAddress.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_static_mutex;  // serialises the calls that share a GPU's array
void *g_scratch_ptr[kMaxDevices] = {};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// The device address of `device`'s copy of scratch, looked up once per device
// with that device current.  Caller holds g_static_mutex.
void *scratch_of(int device) {
    if (device < 0 || device >= kMaxDevices) {
        mlh::set_last_error("fm_matmul_static: device index out of range");
        return nullptr;
    }
    if (g_scratch_ptr[device]) return g_scratch_ptr[device];
    int current = -1;
    if (hipGetDevice(&current) != hipSuccess) current = -1;
    if (current != device && hipSetDevice(device) != hipSuccess) {
        mlh::set_last_error("fm_matmul_static: cannot select the device");
        return nullptr;
    }
    void *ptr = nullptr;
    const hipError_t status = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (current >= 0 && current != device) (void)hipSetDevice(current);
    if (status != hipSuccess || !ptr) {
        mlh::set_last_error(std::string("fm_matmul_static: hipGetSymbolAddress: ") +
                            hipGetErrorString(status));
        return nullptr;
    }
    g_scratch_ptr[device] = ptr;
    return ptr;
}

int fail(float *y, int O, int S, const char *message) {
    mlh::set_last_error(message);
    if (y && O > 0 && S > 0) {
        const float nan = std::numeric_limits<float>::quiet_NaN();
        for (long i = 0; i < (long)O * S; ++i) y[i] = nan;
    }
    return 0;
}

}  // namespace

namespace mlh {

// Set-up of the static scratch for the library's device (fm_init).
bool fm_static_setup() {
    DeviceContext *ctx = context();
    if (!ctx) return false;
    std::lock_guard<std::mutex> lock(g_static_mutex);
    return scratch_of(ctx->device) != nullptr;
}

}  // namespace mlh

extern "C" int fm_matmul_static(int bits, float *y, const float *x, const void *w,
                                const float *s, int O, int I, int S) {
    if (!y) {
        mlh::set_last_error("fm_matmul_static: y is required");
        return 0;
    }
    if ((bits != 8 && bits != 4) || !x || !w || !s || O <= 0 || I <= 0 || S <= 0)
        return fail(y, O, S, "fm_matmul_static: invalid arguments");
    const size_t w_bytes = (size_t)O * (bits == 8 ? (size_t)I : (size_t)(I + 1) / 2);
    const size_t x_bytes = (size_t)S * I * sizeof(float);
    const size_t y_bytes = (size_t)S * O * sizeof(float);
    const size_t s_bytes = (size_t)O * sizeof(float);
    const size_t need = align256(x_bytes) + align256(y_bytes) + align256(w_bytes) + s_bytes;
    if (need > kScratchBytes) {
        char msg[160];
        snprintf(msg, sizeof(msg),
                 "fm_matmul_static: %zu bytes of staging exceed the %zu-byte static scratch",
                 need, kScratchBytes);
        return fail(y, O, S, msg);
    }
    mlh::DeviceContext *ctx = mlh::context();
    if (!ctx) return fail(y, O, S, "fm_matmul_static: no gfx950 device");
    std::lock_guard<std::mutex> lock(g_static_mutex);
    unsigned char *base = static_cast<unsigned char *>(scratch_of(ctx->device));
    if (!base) {
        const std::string why = mlh::last_error();
        return fail(y, O, S, why.c_str());
    }
    // layout: x | y | w | s, each 256-byte aligned; every byte the kernel
    // reads is written here first, so nothing needs clearing between calls
    float *dx = reinterpret_cast<float *>(base);
    float *dy = reinterpret_cast<float *>(base + align256(x_bytes));
    unsigned char *dw = base + align256(x_bytes) + align256(y_bytes);
    float *ds = reinterpret_cast<float *>(dw + align256(w_bytes));
    hipStream_t st = ctx->stream;
    bool ok = hipMemcpyAsync(dx, x, x_bytes, hipMemcpyHostToDevice, st) == hipSuccess &&
              hipMemcpyAsync(dw, w, w_bytes, hipMemcpyHostToDevice, st) == hipSuccess &&
              hipMemcpyAsync(ds, s, s_bytes, hipMemcpyHostToDevice, st) == hipSuccess;
    if (ok) {
        mlh::GemvParams p;
        p.fmt = bits == 8 ? mlh::kQ8 : mlh::kQ4;
        p.w = dw;
        p.s = ds;
        p.O = O;
        p.I = I;
        p.rows = S;
        p.x = dx;
        p.x_stride = I;
        p.y = dy;
        p.y_stride = O;
        ok = mlh::gemv(p, st) == mlh::kOk;
    }
    ok = ok && hipMemcpyAsync(y, dy, y_bytes, hipMemcpyDeviceToHost, st) == hipSuccess;
    ok = hipStreamSynchronize(st) == hipSuccess && ok;
    if (!ok) return fail(y, O, S, "fm_matmul_static: device failure");
    return 1;
}

// kernels_api.cpp -- the kernel-level C ABI (include/moonlight_kernels.h) and
// the process-wide device context.
#include "device_context.h"
#include "mlh_host.h"
#include "../../include/moonlight_kernels.h"
#include "moe.h"
#include "sample.h"

#include <mutex>
#include <vector>

namespace mlh {

static std::mutex g_context_mutex;
static constexpr int kMaxDevices = 64;
static DeviceContext g_contexts[kMaxDevices];
static thread_local std::string g_last_error;

void set_last_error(const std::string &message) { g_last_error = message; }
const char *last_error() { return g_last_error.c_str(); }

int check_hip(hipError_t status, const char *what) {
    if (status == hipSuccess) return kOk;
    set_last_error(std::string(what) + ": " + hipGetErrorString(status));
    return kErrDevice;
}

DeviceContext *context() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        set_last_error("no HIP device is available");
        return nullptr;
    }
    return context_of(device);
}

DeviceContext *context_of(int device) {
    std::lock_guard<std::mutex> lock(g_context_mutex);
    if (device < 0 || device >= kMaxDevices) {
        set_last_error("HIP device index out of range");
        return nullptr;
    }
    DeviceContext &ctx = g_contexts[device];
    if (ctx.ready) return &ctx;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= device) {
        set_last_error("no HIP device is available");
        return nullptr;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        set_last_error("cannot query HIP device " + std::to_string(device));
        return nullptr;
    }
    std::string arch = prop.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0) {
        set_last_error("device " + std::to_string(device) + " is " + arch +
                       "; this library is built for gfx950 (MI355X)");
        return nullptr;
    }
    {
        DeviceScope scope(device);
        if (hipStreamCreateWithFlags(&ctx.stream, hipStreamNonBlocking) != hipSuccess) {
            set_last_error("cannot create the HIP stream");
            return nullptr;
        }
    }
    ctx.device = device;
    // Marketing names can be empty inside containers; the architecture is
    // always appended so callers can tell the device class.
    ctx.name = std::string(prop.name[0] ? prop.name : "AMD Instinct GPU") + " [" +
               arch.substr(0, arch.find(':')) + "]";
    ctx.arch = arch;
    ctx.cu_count = prop.multiProcessorCount;
    ctx.ready = true;
    return &ctx;
}

}  // namespace mlh

using namespace mlh;

static hipStream_t lib_stream() {
    DeviceContext *ctx = context();
    return ctx ? ctx->stream : nullptr;
}

extern "C" {

int mlk_init(void) { return context() ? kOk : kErrDevice; }

const char *mlk_device_name(void) {
    DeviceContext *ctx = context();
    return ctx ? ctx->name.c_str() : "(none)";
}

const char *mlk_last_error(void) { return last_error(); }

void *mlk_malloc(size_t bytes) {
    if (!context()) return nullptr;
    void *ptr = nullptr;
    if (check_hip(hipMalloc(&ptr, bytes ? bytes : 1), "hipMalloc") != kOk) return nullptr;
    return ptr;
}

int mlk_free(void *ptr) {
    if (!ptr) return kOk;
    return check_hip(hipFree(ptr), "hipFree");
}

int mlk_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    hipStream_t s = lib_stream();
    if (!s) return kErrDevice;
    int st = check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s), "H2D copy");
    return st ? st : check_hip(hipStreamSynchronize(s), "H2D sync");
}

int mlk_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    hipStream_t s = lib_stream();
    if (!s) return kErrDevice;
    int st = check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s), "D2H copy");
    return st ? st : check_hip(hipStreamSynchronize(s), "D2H sync");
}

int mlk_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    hipStream_t s = lib_stream();
    if (!s) return kErrDevice;
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s), "D2D copy");
}

int mlk_memset(void *dst, int value, size_t bytes) {
    hipStream_t s = lib_stream();
    if (!s) return kErrDevice;
    return check_hip(hipMemsetAsync(dst, value, bytes, s), "memset");
}

int mlk_synchronize(void) {
    hipStream_t s = lib_stream();
    if (!s) return kErrDevice;
    return check_hip(hipStreamSynchronize(s), "stream sync");
}

static int finish(int status, const char *what) {
    if (status == kOk) return kOk;
    if (status == kErrArgs) set_last_error(std::string(what) + ": invalid arguments");
    else if (status == kErrLaunch) set_last_error(std::string(what) + ": kernel launch failed");
    return status;
}

int mlk_gemv(int fmt, const void *w, const float *s, const float *x, float *y, int out_width,
             int in_width, int rows, const float *norm_w, float eps, const float *resid) {
    hipStream_t st = lib_stream();
    if (!st) return kErrDevice;
    if (fmt < MLK_F32 || fmt > MLK_Q4) return finish(kErrArgs, "mlk_gemv");
    GemvParams p;
    p.fmt = fmt;
    p.w = static_cast<const uint8_t *>(w);
    p.s = s;
    p.O = out_width;
    p.I = in_width;
    p.rows = rows;
    p.x = x;
    p.x_stride = in_width;
    p.norm_w = norm_w;
    p.eps = eps;
    p.y = y;
    p.y_stride = out_width;
    p.resid = resid;
    p.resid_stride = out_width;
    p.epilogue = resid ? kEpiResidual : kEpiPlain;
    return finish(gemv(p, st), "mlk_gemv");
}

int mlk_gemv_kernel_name(int fmt, int out_width, int in_width, int rows, int swiglu, char *name,
                         size_t name_size) {
    if (!name || name_size == 0 || fmt < kF32 || fmt > kQ4 || out_width <= 0 || in_width <= 0 ||
        rows <= 0)
        return finish(kErrArgs, "mlk_gemv_kernel_name");
    const std::string n = gemv_kernel_name(fmt, out_width, in_width, rows, swiglu != 0);
    snprintf(name, name_size, "%s", n.c_str());
    return kOk;
}

int mlk_gemv_swiglu(int fmt, const void *w_gate, const float *s_gate, const void *w_up,
                    const float *s_up, const float *x, float *h, int out_width, int in_width,
                    int rows, const float *norm_w, float eps) {
    hipStream_t st = lib_stream();
    if (!st) return kErrDevice;
    if (fmt < MLK_F32 || fmt > MLK_Q4) return finish(kErrArgs, "mlk_gemv_swiglu");
    GemvParams p;
    p.fmt = fmt;
    p.w = static_cast<const uint8_t *>(w_gate);
    p.s = s_gate;
    p.w2 = static_cast<const uint8_t *>(w_up);
    p.s2 = s_up;
    p.O = out_width;
    p.I = in_width;
    p.rows = rows;
    p.x = x;
    p.x_stride = in_width;
    p.norm_w = norm_w;
    p.eps = eps;
    p.y = h;
    p.y_stride = out_width;
    p.epilogue = kEpiSiluDual;
    return finish(gemv(p, st), "mlk_gemv_swiglu");
}

int mlk_time_gemv(int fmt, const void *const *w_copies, const float *const *s_copies,
                  int n_copies, const float *x, float *y, int out_width, int in_width, int rows,
                  int warmup, int iters, int use_graph, double *avg_us) {
    hipStream_t st = lib_stream();
    if (!st) return kErrDevice;
    if (!w_copies || n_copies <= 0 || iters <= 0 || !avg_us) return finish(kErrArgs, "mlk_time_gemv");
    auto launch = [&](int i) {
        GemvParams p;
        p.fmt = fmt;
        p.w = static_cast<const uint8_t *>(w_copies[i % n_copies]);
        p.s = s_copies ? s_copies[i % n_copies] : nullptr;
        p.O = out_width;
        p.I = in_width;
        p.rows = rows;
        p.x = x;
        p.x_stride = in_width;
        p.y = y;
        p.y_stride = out_width;
        return gemv(p, st);
    };
    for (int i = 0; i < warmup; ++i)
        if (int e = launch(i)) return finish(e, "mlk_time_gemv warmup");
    hipGraphExec_t exec = nullptr;
    hipGraph_t graph = nullptr;
    if (use_graph) {
        if (int e = check_hip(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "capture"))
            return e;
        for (int i = 0; i < iters; ++i) launch(i);
        if (int e = check_hip(hipStreamEndCapture(st, &graph), "end capture")) return e;
        if (int e = check_hip(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate"))
            return e;
        // one untimed replay to load the graph
        if (int e = check_hip(hipGraphLaunch(exec, st), "graph launch")) return e;
    }
    hipEvent_t start, stop;
    (void)hipEventCreate(&start);
    (void)hipEventCreate(&stop);
    (void)hipEventRecord(start, st);
    int status = kOk;
    if (use_graph) {
        status = check_hip(hipGraphLaunch(exec, st), "graph launch");
    } else {
        for (int i = 0; i < iters && status == kOk; ++i) status = launch(i);
    }
    (void)hipEventRecord(stop, st);
    int sync = check_hip(hipEventSynchronize(stop), "event sync");
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, start, stop);
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (status) return finish(status, "mlk_time_gemv");
    if (sync) return sync;
    *avg_us = (double)ms * 1000.0 / iters;
    return kOk;
}

int mlk_time_copy(void *const *src, void *const *dst, int n_buffers, size_t bytes, int warmup,
                  int iters, double *avg_us) {
    hipStream_t st = lib_stream();
    if (!st) return kErrDevice;
    if (!src || !dst || n_buffers <= 0 || iters <= 0 || !avg_us)
        return finish(kErrArgs, "mlk_time_copy");
    for (int i = 0; i < warmup; ++i)
        if (int e = copy16(src[i % n_buffers], dst[i % n_buffers], bytes, st))
            return finish(e, "mlk_time_copy");
    hipEvent_t start, stop;
    (void)hipEventCreate(&start);
    (void)hipEventCreate(&stop);
    (void)hipEventRecord(start, st);
    int status = kOk;
    for (int i = 0; i < iters && status == kOk; ++i)
        status = copy16(src[i % n_buffers], dst[i % n_buffers], bytes, st);
    (void)hipEventRecord(stop, st);
    int sync = check_hip(hipEventSynchronize(stop), "event sync");
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, start, stop);
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
    if (status) return finish(status, "mlk_time_copy");
    if (sync) return sync;
    *avg_us = (double)ms * 1000.0 / iters;
    return kOk;
}

int mlk_time_read(void *const *src, int n_buffers, size_t bytes, int blocks, unsigned *scratch,
                  int warmup, int iters, double *avg_us) {
    hipStream_t st = lib_stream();
    if (!st) return kErrDevice;
    if (!src || n_buffers <= 0 || iters <= 0 || !avg_us || !scratch)
        return finish(kErrArgs, "mlk_time_read");
    for (int i = 0; i < warmup; ++i)
        if (int e = read16(src[i % n_buffers], bytes, blocks, scratch, st))
            return finish(e, "mlk_time_read");
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    if (int e = check_hip(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "capture"))
        return e;
    for (int i = 0; i < iters; ++i) read16(src[i % n_buffers], bytes, blocks, scratch, st);
    if (int e = check_hip(hipStreamEndCapture(st, &graph), "end capture")) return e;
    if (int e = check_hip(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate"))
        return e;
    (void)hipGraphLaunch(exec, st);
    hipEvent_t start, stop;
    (void)hipEventCreate(&start);
    (void)hipEventCreate(&stop);
    (void)hipEventRecord(start, st);
    int status = check_hip(hipGraphLaunch(exec, st), "graph launch");
    (void)hipEventRecord(stop, st);
    int sync = check_hip(hipEventSynchronize(stop), "event sync");
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, start, stop);
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
    (void)hipGraphExecDestroy(exec);
    (void)hipGraphDestroy(graph);
    if (status) return status;
    if (sync) return sync;
    *avg_us = (double)ms * 1000.0 / iters;
    return kOk;
}

int mlk_route_topk(const float *logits, const float *bias, int rows, int experts, int top_k,
                   int normalize, float routed_scale, int *ids, float *weights) {
    hipStream_t st = lib_stream();
    if (!st) return kErrDevice;
    if (!logits || !bias || !ids || !weights || rows <= 0 || experts <= 0 || top_k <= 0)
        return finish(kErrArgs, "mlk_route_topk");
    // the route tables the kernels also write, in one scratch allocation
    const size_t pos = (size_t)rows * top_k;
    const size_t n_int = 2 + 3 * (size_t)experts + 3 * pos;
    int *tab = nullptr;
    if (int e = check_hip(hipMalloc(&tab, n_int * sizeof(int)), "mlk_route_topk")) return e;
    RouteParams p;
    p.logits = logits;
    p.bias = bias;
    p.rows = rows;
    p.experts = experts;
    p.top_k = top_k;
    p.normalize = normalize;
    p.routed_scale = routed_scale;
    p.ids = ids;
    p.weights = weights;
    p.n_unique = tab;
    p.error = tab + 1;
    p.unique = tab + 2;
    p.counts = p.unique + experts;
    p.offsets = p.counts + experts;
    p.list_rows = p.offsets + experts;
    p.list_slots = p.list_rows + pos;
    p.list_pos = p.list_slots + pos;
    int status = check_hip(hipMemsetAsync(tab, 0, n_int * sizeof(int), st), "mlk_route_topk");
    if (status == kOk) status = finish(route_topk(p, st), "mlk_route_topk");
    const int sync = check_hip(hipStreamSynchronize(st), "mlk_route_topk");
    (void)hipFree(tab);
    return status != kOk ? status : sync;
}

int mlk_sample(const float *logits, int vocab, float temperature, float top_p, double u,
               int *token) {
    hipStream_t st = lib_stream();
    if (!st) return kErrDevice;
    if (!logits || !token || vocab <= 0 || !(u >= 0.0 && u < 1.0)) return finish(kErrArgs, "mlk_sample");
    SampleWork w;
    if (sample_alloc(&w, vocab) != 0) {
        set_last_error("mlk_sample: device allocation failed");
        return kErrDevice;
    }
    int out[2] = {0, -1};
    int status = sample_enqueue(&w, logits, temperature, top_p, u, st) == 0 ? kOk : kErrLaunch;
    if (status == kOk)
        status = check_hip(hipMemcpyAsync(out, w.ctl + 2, sizeof(out), hipMemcpyDeviceToHost, st),
                           "mlk_sample");
    const int sync = check_hip(hipStreamSynchronize(st), "mlk_sample");
    sample_free(&w);
    if (status == kOk) status = sync;
    if (status != kOk) return finish(status, "mlk_sample");
    if (out[0] && temperature > 0.0f) {
        set_last_error("mlk_sample: logits are not finite");
        return kErrArgs;
    }
    *token = out[1];
    return kOk;
}

int mlk_quantize(int bits, const float *w, int rows, int cols, uint8_t *q, float *s) {
    hipStream_t st = lib_stream();
    if (!st) return kErrDevice;
    return finish(quantize_rows(bits, w, rows, cols, q, s, st), "mlk_quantize");
}

int mlk_fill_normal(float *out, int64_t n, uint64_t seed, float mean, float stdv, int bf16) {
    hipStream_t st = lib_stream();
    if (!st) return kErrDevice;
    return finish(fill_normal(out, n, seed, mean, stdv, bf16, st), "mlk_fill_normal");
}

}  // extern "C"

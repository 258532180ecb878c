// device_context.h -- process-wide HIP context of the library (internal).
#pragma once

#include <hip/hip_runtime.h>

#include <string>

namespace mlh {

struct DeviceContext {
    bool ready = false;
    int device = 0;
    hipStream_t stream = nullptr;  // default priority, non-blocking
    std::string name;              // marketing name, e.g. "AMD Instinct MI355X"
    std::string arch;              // gcnArchName, e.g. "gfx950:sramecc+:xnack-"
    int cu_count = 0;
};

// The context of the calling thread's current HIP device (hipGetDevice: 0
// unless the caller selected another), initialised with its library stream on
// first use; nullptr (and the last error set) when that device is not a
// usable gfx950 device.
DeviceContext *context();
// The context of `device`, initialised on first use (the stream is created
// with `device` current; the caller's current device is restored).
DeviceContext *context_of(int device);

// Makes `device` current for the scope's lifetime and restores the caller's
// device afterwards (nothing happens when it already is current, or for a
// negative device).
class DeviceScope {
public:
    explicit DeviceScope(int device) {
        int current = -1;
        if (device >= 0 && hipGetDevice(&current) == hipSuccess && current != device &&
            hipSetDevice(device) == hipSuccess)
            previous_ = current;
    }
    ~DeviceScope() {
        if (previous_ >= 0) (void)hipSetDevice(previous_);
    }
    DeviceScope(const DeviceScope &) = delete;
    DeviceScope &operator=(const DeviceScope &) = delete;

private:
    int previous_ = -1;
};
void set_last_error(const std::string &message);
const char *last_error();
// Translates a HIP status into a library status, recording the message.
int check_hip(hipError_t status, const char *what);

}  // namespace mlh

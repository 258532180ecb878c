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

// Initialises device 0 and the library stream once; returns nullptr (and sets
// the last error) when no usable gfx950 device is present.
DeviceContext *context();
void set_last_error(const std::string &message);
const char *last_error();
// Translates a HIP status into a library status, recording the message.
int check_hip(hipError_t status, const char *what);

}  // namespace mlh

// gemv_f32.hip -- instantiations of the GEMV core for the f32 format
// (split per format so the three compile in parallel).
#include "gemv_impl.h"

namespace mlh {

bool dispatch_gemv_f32(const GemvLaunch &L, int mode, const GemvPlan &plan, dim3 grid,
                      hipStream_t stream) {
    return dispatch_gemv_fmt<kF32>(L, mode, plan, grid, stream);
}

}  // namespace mlh

// gemv_q8.hip -- instantiations of the GEMV core for the q8 format
// (split per format so the three compile in parallel).
#include "gemv_impl.h"

namespace mlh {

bool dispatch_gemv_q8(const GemvLaunch &L, int mode, const GemvPlan &plan, dim3 grid,
                      hipStream_t stream) {
    return dispatch_gemv_fmt<kQ8>(L, mode, plan, grid, stream);
}

}  // namespace mlh

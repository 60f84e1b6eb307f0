// Decode GEMV launch unit: fp8 A rows staged in LDS once per workgroup (kernel template in gemv.h).
#include "gemv.h"

namespace w4a8 {

bool launch_gemv_staged(const GemmArgs& p, dim3 grid, const GemvPlan& pl, hipStream_t stream) {
  return launch_gemv_amode<kAStage>(p, grid, pl, stream);
}

}  // namespace w4a8

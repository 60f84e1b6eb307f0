// Decode GEMV launch unit: bf16/fp16 A rows quantized per token into LDS by the GEMV itself, so a
// decode call is a single launch (kernel template in gemv.h).
#include "gemv.h"

namespace w4a8 {

bool launch_gemv_fused(const GemmArgs& p, dim3 grid, const GemvPlan& pl, hipStream_t stream) {
  return launch_gemv_amode<kAQuant>(p, grid, pl, stream);
}

}  // namespace w4a8

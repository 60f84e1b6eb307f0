// Decode GEMV launch unit: the fused act quant (bf16/fp16 A rows quantized into LDS by the GEMV) on
// e2m1 weights, MXFP4 and NVFP4 (kernel template in gemv.h).
#include "gemv.h"

namespace w4a8 {

bool launch_gemv_fused_e2m1(const GemmArgs& p, dim3 grid, const GemvPlan& pl, hipStream_t stream) {
  return gemv_launch_quant<false, true>(p, grid, stream, pl);
}

}  // namespace w4a8

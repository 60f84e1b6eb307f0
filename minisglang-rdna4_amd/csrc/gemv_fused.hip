// Decode GEMV launch unit: bf16/fp16 A rows quantized per token into LDS by the GEMV itself, so a
// decode call is a single launch (kernel template in gemv.h). int4 weights here; the e2m1 formats
// in gemv_fused_e2m1.hip.
#include "gemv.h"

namespace w4a8 {

bool launch_gemv_fused(const GemmArgs& p, dim3 grid, const GemvPlan& pl, hipStream_t stream) {
  if (p.wfmt == kE2M1) return launch_gemv_fused_e2m1(p, grid, pl, stream);
  return gemv_launch_quant<true, false>(p, grid, stream, pl);
}

}  // namespace w4a8

// Decode GEMV launch unit: fp8 A rows staged in LDS once per workgroup (kernel template in gemv.h).
#include "gemv.h"

namespace w4a8 {

bool launch_gemv_staged(const GemmArgs& p, dim3 grid, const GemvPlan& pl, hipStream_t stream) {
  const int ns = p.silu ? 2 * pl.nstr : pl.nstr;
  if (ns == 1) return gemv_launch_fmt<kAStage, 1, kGemvChunk, kWinWaitAll, true, true>(p, grid, stream, pl);
  if (ns == 2) return gemv_launch_fmt<kAStage, 2, kGemvChunk, kWinWaitAll, true, true>(p, grid, stream, pl);
  return false;
}

}  // namespace w4a8

// Routed decode GEMV: gemm1 (+ silu) of a decode-sized MoE batch with the router in the kernel's
// prologue (gemv_kernel's kARoute source). One launch does the route (softmax + top-k +
// renormalize, moe_route.h), the one-block-per-slot assignment, the per-token act quant of x and
// the grouped gemm1 with the fused silu epilogue, where the batch otherwise runs the route + slots
// launch and then gemm1. Its own unit, built in parallel with the other GEMV units.
//
// Bits: the plan (strips, K split) is the grouped gemm1's for the same call, the A codes and row
// scale are the act-quant kernel's, and the routing is the route kernel's code: the gemm1 buffer
// and every route output equal those of the two-launch path bit for bit.
#include "gemv.h"

namespace w4a8 {

// p: the grouped gemm1's arguments (sorted_ids non-null for the grouped plan, silu set) plus the
// route fields; row_blocks: the grouped gemm1's row blocks, for its plan. kErrUnsupported when the
// routed kernel does not cover the call.
int launch_moe_route_gemm1(const GemmArgs& p, int64_t row_blocks, hipStream_t stream) {
  GemvPlan pl = plan_gemv(p, row_blocks, false);
  if (!p.silu || pl.nstr != 1) return kErrUnsupported;
  const int64_t threads = (int64_t)pl.waves * 64;
  const int64_t chunks = p.KT * (kTileK / 8);  // 16-byte loads of the token's row
  const size_t stage = (size_t)((stage_stride((int)p.KT) + 15) / 16) * 16;
  if (chunks > kStageMax * threads || stage > (size_t)kStageLdsMax) return kErrUnsupported;
  pl.amode = kARoute;
  pl.sm = chunks <= threads ? 1 : chunks <= 2 * threads ? 2 : chunks <= 4 * threads ? 4 : 8;
  pl.stage_bytes = stage;
  pl.af = kWinAfterA;
  pl.ch = kGemvChunk;
  const dim3 grid((unsigned)(p.N / kTileN / 2), 1, (unsigned)p.num_slots);
  if (!gemv_launch_fmt<kARoute, 2, kGemvChunk, kWinAfterA, true, true>(p, grid, stream, pl)) return kErrUnsupported;
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

}  // namespace w4a8

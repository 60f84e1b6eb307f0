// Decode GEMV launch unit for the sub-tile-group formats: int4 with group 32/64, e2m1 with fp16
// group scales and NVFP4 (e2m1 with e4m3 group-16 scales and a per-channel global) (kernel template in gemv.h). Groups per tile are a template constant so the
// per-tile sub-group loop is straight-line code.
#include "gemv.h"

namespace w4a8 {

template <int NS, int CHK, int MD, bool SY>
static void launch_gpt(const GemmArgs& p, dim3 grid, dim3 block, size_t lds, int tpw, hipStream_t stream) {
  const int gpt = p.group >= kTileK ? 1 : kTileK / p.group;
  if constexpr (MD == kModeE2M1F16) {
    if (gpt == 8) {
      hipLaunchKernelGGL((gemv_kernel<NS, CHK, MD, kAGlobal, SY, 4, 8, kWinAfterA>), grid, block, lds, stream, p, tpw);
      return;
    }
  }
  if (gpt == 4)
    hipLaunchKernelGGL((gemv_kernel<NS, CHK, MD, kAGlobal, SY, 4, 4, kWinAfterA>), grid, block, lds, stream, p, tpw);
  else if (gpt == 2)
    hipLaunchKernelGGL((gemv_kernel<NS, CHK, MD, kAGlobal, SY, 4, 2, kWinAfterA>), grid, block, lds, stream, p, tpw);
  else if constexpr (MD == kModeE2M1F16)
    hipLaunchKernelGGL((gemv_kernel<NS, CHK, MD, kAGlobal, SY, 4, 1, kWinAfterA>), grid, block, lds, stream, p, tpw);
}

template <int NS, int CHK>
static void launch_fmt(const GemmArgs& p, dim3 grid, dim3 block, size_t lds, int tpw, hipStream_t stream) {
  if (p.wfmt == kInt4) {
    if (p.zeros == nullptr) launch_gpt<NS, CHK, kModeI4Sub, true>(p, grid, block, lds, tpw, stream);
    else launch_gpt<NS, CHK, kModeI4Sub, false>(p, grid, block, lds, tpw, stream);
  } else {
    launch_gpt<NS, CHK, kModeE2M1F16, false>(p, grid, block, lds, tpw, stream);
  }
}

bool launch_gemv_generic(const GemmArgs& p, dim3 grid, const GemvPlan& pl, hipStream_t stream) {
  if (p.wfmt == kInt4 && p.group >= kTileK) return false;  // the fast int4 path covers these
  const int nstr_k = p.silu ? 2 * pl.nstr : pl.nstr;
  const int ch = nstr_k >= 4 ? 4 : gemv_chunk(pl.tpw);
  const size_t lds = (size_t)pl.waves * nstr_k * 4 * 64 * sizeof(float);
  const dim3 block(pl.waves * 64);
  if (nstr_k == 1 && ch == 4) launch_fmt<1, 4>(p, grid, block, lds, pl.tpw, stream);
  else if (nstr_k == 1) launch_fmt<1, 8>(p, grid, block, lds, pl.tpw, stream);
  else if (nstr_k == 2 && ch == 4) launch_fmt<2, 4>(p, grid, block, lds, pl.tpw, stream);
  else if (nstr_k == 2) launch_fmt<2, 8>(p, grid, block, lds, pl.tpw, stream);
  else if (nstr_k == 4) launch_fmt<4, 4>(p, grid, block, lds, pl.tpw, stream);
  else return false;
  return true;
}

}  // namespace w4a8

// Per-token fp8-e4m3 activation quantization.
//
// Contract (python/minisgl/quant/kernels.py:1703-1712, python/minisgl/layers/norm.py:27-46):
// per row, amax = max |x|; s = max(amax / 448, 1e-8); q = e4m3_rne(x * (1 / s)), unclamped.
// The division and reciprocal are IEEE-rounded f32 operations; v_cvt_pk_fp8_f32 rounds to
// nearest even (checked bit-for-bit against the CPU restatement).
//
// One workgroup per row (grid-stride over rows), 16-byte vector loads; rows up to 32768 elements
// are read once into registers (one memory round trip), longer rows take two passes. Batches of
// 64 or more rows of up to 4096 elements take one wave per row instead. An optional
// device-side row count (the MoE padded row count) lets a graph-captured launch size the grid for
// the maximum and skip the tail.
#include "act_quant.h"

namespace w4a8 {

template <int CPT>
__global__ void __launch_bounds__(kAqThreads)
act_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t K, int dtype,
                 uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scales,
                 const int32_t* __restrict__ row_count) {
  __shared__ float red[kAqThreads / 64];
  int64_t rows = M;
  if (row_count) {
    const int64_t rc = *row_count;
    rows = rc < M ? rc : M;
  }
  for (int64_t m = blockIdx.x; m < rows; m += gridDim.x) quant_row<CPT>(x + m * ldx, K, dtype, q + m * ldq, scales + m, red);
}

// Many short rows (M >= 64, K <= 4096): one wave per row, 8 elements per lane per 16-byte chunk
// and CPW chunks per lane, reduced with wave_max alone (no LDS, no barrier). Same arithmetic as
// quant_row, bit for bit.
template <int CPW>
__global__ void __launch_bounds__(256)
act_quant_wave_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t K, int dtype,
                      uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scales,
                      const int32_t* __restrict__ row_count) {
  const int lane = threadIdx.x & 63;
  int64_t rows = M;
  if (row_count) {
    const int64_t rc = *row_count;
    rows = rc < M ? rc : M;
  }
  const int64_t stride = (int64_t)gridDim.x * (blockDim.x >> 6);
  for (int64_t m = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); m < rows; m += stride)
    quant_row_wave<CPW>(x + m * ldx, K, dtype, q + m * ldq, scales + m, lane);
}

int launch_act_quant(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* q,
                     int64_t ldq, float* scales, const int32_t* row_count, hipStream_t stream) {
  if (M <= 0) return kOk;
  if (M >= 64 && K <= 64 * 8 * 8) {
    const int cpw = (int)((K + 511) / 512);
    const int64_t blocks = (M + 3) / 4;
    dim3 g((unsigned)(blocks < 16384 ? blocks : 16384)), b(256);
    const uint16_t* xp = reinterpret_cast<const uint16_t*>(x);
#define W4A8_AQW(C) hipLaunchKernelGGL(act_quant_wave_kernel<C>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count)
    if (cpw <= 1) W4A8_AQW(1);
    else if (cpw <= 2) W4A8_AQW(2);
    else if (cpw <= 4) W4A8_AQW(4);
    else W4A8_AQW(8);
#undef W4A8_AQW
    return hipGetLastError() == hipSuccess ? kOk : kErrHip;
  }
  const int64_t grid = M < 8192 ? M : 8192;
  const uint16_t* xp = reinterpret_cast<const uint16_t*>(x);
  dim3 g((unsigned)grid), b(kAqThreads);
  switch (quant_row_cpt(K)) {
    case 1: hipLaunchKernelGGL(act_quant_kernel<1>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count); break;
    case 2: hipLaunchKernelGGL(act_quant_kernel<2>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count); break;
    case 4: hipLaunchKernelGGL(act_quant_kernel<4>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count); break;
    case 8: hipLaunchKernelGGL(act_quant_kernel<8>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count); break;
    case 16: hipLaunchKernelGGL(act_quant_kernel<16>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count); break;
    default: hipLaunchKernelGGL(act_quant_kernel<0>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count);
  }
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

}  // namespace w4a8

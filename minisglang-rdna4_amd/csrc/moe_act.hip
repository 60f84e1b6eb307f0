// Gated tanh-GELU between the unfused gemm1 and gemm2 of the MoE FFN, for experts whose checkpoint
// declares HF `gelu_pytorch_tanh` (Gemma4's routed experts). Restates the reference's
// gelu_tanh_and_mul (python/minisgl/layers/activation.py:11-22, 47-64), which w4a8_moe runs on the
// (P, 2*inter) output of its unfused gemm1 (python/minisgl/quant/kernels.py:777-783):
//   out[r, i] = dtype(gelu_tanh(f32(y[r, i])) * f32(y[r, inter + i])),
//   gelu_tanh(a) = 0.5 a (1 + tanh(sqrt(2/pi) (a + 0.044715 a^3))),
// in f32 with one rounding to the activation dtype at the end (the gate and up values are already
// in that dtype: gemm1 stored them so). Rows at and past the device-side row count (the align's
// ntp) are skipped, so a graph-captured launch can be sized for the padded capacity.
#include "w4a8_common.h"

namespace w4a8 {

__device__ __forceinline__ float gelu_tanh(float a) {
  const float kBeta = 0.7978845608028654f;  // sqrt(2 / pi)
  const float kKappa = 0.044715f;
  const float cube = a * a * a;
  const float inner = kBeta * (a + kKappa * cube);
  return 0.5f * a * (1.0f + tanhf(inner));
}

// one workgroup of 256 threads per row (grid-stride over rows), 8 channels per thread per pass
__global__ void __launch_bounds__(256) gelu_tanh_mul_kernel(const uint16_t* __restrict__ y, int64_t ldy, int64_t rows,
                                                            int64_t inter, int dtype, uint16_t* __restrict__ out,
                                                            int64_t ldo, const int32_t* __restrict__ row_count) {
  int64_t nr = rows;
  if (row_count) {
    const int64_t rc = *row_count;
    nr = rc < rows ? rc : rows;
  }
  for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
    const uint16_t* yr = y + r * ldy;
    for (int64_t i = (int64_t)threadIdx.x * 8; i < inter; i += 256 * 8) {
      const uint4 g = *reinterpret_cast<const uint4*>(yr + i);
      const uint4 u = *reinterpret_cast<const uint4*>(yr + inter + i);
      float gf[8], uf[8];
      unpack8(g, dtype, gf);
      unpack8(u, dtype, uf);
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = to_dtype(gelu_tanh(gf[2 * e]) * uf[2 * e], dtype);
        const uint32_t hi = to_dtype(gelu_tanh(gf[2 * e + 1]) * uf[2 * e + 1], dtype);
        w[e] = lo | (hi << 16);
      }
      *reinterpret_cast<uint4*>(out + r * ldo + i) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

int launch_gelu_tanh_mul(const void* y, int64_t ldy, int64_t rows, int64_t inter, int dtype, void* out, int64_t ldo,
                         const int32_t* row_count, hipStream_t stream) {
  if (rows <= 0) return kOk;
  const int64_t grid = rows < 8192 ? rows : 8192;
  hipLaunchKernelGGL(gelu_tanh_mul_kernel, dim3((unsigned)grid), dim3(256), 0, stream,
                     reinterpret_cast<const uint16_t*>(y), ldy, rows, inter, dtype, reinterpret_cast<uint16_t*>(out),
                     ldo, row_count);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

}  // namespace w4a8

// Per-token fp8-e4m3 activation quantization.
//
// Contract (python/minisgl/quant/kernels.py:1703-1712, python/minisgl/layers/norm.py:27-46):
// per row, amax = max |x|; s = max(amax / 448, 1e-8); q = e4m3_rne(x * (1 / s)), unclamped.
// The division and reciprocal are IEEE-rounded f32 operations; v_cvt_pk_fp8_f32 rounds to
// nearest even (checked bit-for-bit against the CPU restatement).
//
// One workgroup per row (grid-stride over rows), 16-byte vector loads; rows up to 32768 elements
// are read once into registers (one memory round trip), longer rows take two passes. An optional
// device-side row count (the MoE padded row count) lets a graph-captured launch size the grid for
// the maximum and skip the tail.
#include "w4a8_common.h"

namespace w4a8 {

constexpr int kAqThreads = 256;

__device__ __forceinline__ float block_max(float v, float* red) {
  const int tid = threadIdx.x;
  v = wave_max(v);
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  if (tid < 64) {
    float t = tid < kAqThreads / 64 ? red[tid] : 0.0f;
    t = wave_max(t);
    if (tid == 0) red[0] = t;
  }
  __syncthreads();
  v = red[0];
  __syncthreads();
  return v;
}

// CPT > 0: the row (<= 256*8*CPT elements) is read once into registers. CPT == 0: two passes.
template <int CPT>
__global__ void __launch_bounds__(kAqThreads)
act_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t K, int dtype,
                 uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scales,
                 const int32_t* __restrict__ row_count) {
  __shared__ float red[kAqThreads / 64];
  const int tid = threadIdx.x;
  int64_t rows = M;
  if (row_count) {
    const int64_t rc = *row_count;
    rows = rc < M ? rc : M;
  }
  for (int64_t m = blockIdx.x; m < rows; m += gridDim.x) {
    const uint16_t* xr = x + m * ldx;
    uint8_t* qr = q + m * ldq;
    float amax = 0.0f;
    if (CPT > 0) {
      uint4 raw[CPT > 0 ? CPT : 1];
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int64_t k = ((int64_t)c * kAqThreads + tid) * 8;
        raw[c] = k < K ? *reinterpret_cast<const uint4*>(xr + k) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        float f[8];
        unpack8(raw[c], dtype, f);
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
      }
      const float s = act_row_scale(block_max(amax, red));
      const float inv = 1.0f / s;
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int64_t k = ((int64_t)c * kAqThreads + tid) * 8;
        if (k < K) {
          float f[8];
          unpack8(raw[c], dtype, f);
          *reinterpret_cast<uint2*>(qr + k) = quant8(f, inv);
        }
      }
      if (tid == 0) scales[m] = s;
    } else {
      for (int64_t k = (int64_t)tid * 8; k < K; k += kAqThreads * 8) {
        float f[8];
        unpack8(*reinterpret_cast<const uint4*>(xr + k), dtype, f);
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
      }
      const float s = act_row_scale(block_max(amax, red));
      const float inv = 1.0f / s;
      for (int64_t k = (int64_t)tid * 8; k < K; k += kAqThreads * 8) {
        float f[8];
        unpack8(*reinterpret_cast<const uint4*>(xr + k), dtype, f);
        *reinterpret_cast<uint2*>(qr + k) = quant8(f, inv);
      }
      if (tid == 0) scales[m] = s;
    }
  }
}

int launch_act_quant(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* q,
                     int64_t ldq, float* scales, const int32_t* row_count, hipStream_t stream) {
  if (M <= 0) return kOk;
  const int64_t grid = M < 8192 ? M : 8192;
  const int64_t chunks = (K + kAqThreads * 8 - 1) / (kAqThreads * 8);
  const uint16_t* xp = reinterpret_cast<const uint16_t*>(x);
  dim3 g((unsigned)grid), b(kAqThreads);
  if (chunks <= 1)
    hipLaunchKernelGGL(act_quant_kernel<1>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count);
  else if (chunks <= 2)
    hipLaunchKernelGGL(act_quant_kernel<2>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count);
  else if (chunks <= 4)
    hipLaunchKernelGGL(act_quant_kernel<4>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count);
  else if (chunks <= 8)
    hipLaunchKernelGGL(act_quant_kernel<8>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count);
  else if (chunks <= 16)
    hipLaunchKernelGGL(act_quant_kernel<16>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count);
  else
    hipLaunchKernelGGL(act_quant_kernel<0>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

}  // namespace w4a8

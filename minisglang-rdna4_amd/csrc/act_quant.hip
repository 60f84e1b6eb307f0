// Per-token fp8-e4m3 activation quantization.
//
// Contract (python/minisgl/quant/kernels.py:1703-1712, python/minisgl/layers/norm.py:27-46):
// per row, amax = max |x|; s = max(amax / 448, 1e-8); q = e4m3_rne(x * (1 / s)), unclamped.
// The division and reciprocal are IEEE-rounded f32 operations; v_cvt_pk_fp8_f32 rounds to
// nearest even (checked bit-for-bit against the CPU restatement).
//
// One workgroup per row (grid-stride over rows), 16-byte vector loads, two passes over the row
// (the second pass re-reads it from L2). An optional device-side row count (the MoE padded row
// count) lets a graph-captured launch size the grid for the maximum and skip the tail.
#include "w4a8_common.h"

namespace w4a8 {

constexpr int kAqThreads = 256;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ void unpack8(const uint4& u, int dtype, float* f) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = from_dtype((uint16_t)(w[i] & 0xffffu), dtype);
    f[2 * i + 1] = from_dtype((uint16_t)(w[i] >> 16), dtype);
  }
}

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
    float amax = 0.0f;
    for (int64_t k = (int64_t)tid * 8; k < K; k += kAqThreads * 8) {
      float f[8];
      unpack8(*reinterpret_cast<const uint4*>(xr + k), dtype, f);
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
    }
    amax = wave_max(amax);
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    if (tid < 64) {
      float v = tid < kAqThreads / 64 ? red[tid] : 0.0f;
      v = wave_max(v);
      if (tid == 0) red[0] = v;
    }
    __syncthreads();
    amax = red[0];
    __syncthreads();
    float s = amax / 448.0f;
    if (s < 1e-8f) s = 1e-8f;
    const float inv = 1.0f / s;
    uint8_t* qr = q + m * ldq;
    for (int64_t k = (int64_t)tid * 8; k < K; k += kAqThreads * 8) {
      float f[8];
      unpack8(*reinterpret_cast<const uint4*>(xr + k), dtype, f);
      uint32_t lo = 0, hi = 0;
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[0] * inv, f[1] * inv, lo, false);
      lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[2] * inv, f[3] * inv, lo, true);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[4] * inv, f[5] * inv, hi, false);
      hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[6] * inv, f[7] * inv, hi, true);
      *reinterpret_cast<uint2*>(qr + k) = make_uint2(lo, hi);
    }
    if (tid == 0) scales[m] = s;
  }
}

int launch_act_quant(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* q,
                     int64_t ldq, float* scales, const int32_t* row_count, hipStream_t stream) {
  if (M <= 0) return kOk;
  int64_t grid = M < 8192 ? M : 8192;
  hipLaunchKernelGGL(act_quant_kernel, dim3((unsigned)grid), dim3(kAqThreads), 0, stream,
                     reinterpret_cast<const uint16_t*>(x), ldx, M, K, dtype, q, ldq, scales,
                     row_count);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

}  // namespace w4a8

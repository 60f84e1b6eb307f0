// Load-time weight repack: reference op layout -> W4 tile layout (see w4a8_common.h).
//
// Input is the reference's op layout (python/minisgl/quant/kernels.py:255-346 and
// python/minisgl/quant/mxfp4.py:55-69): w_packed (N, K/8) int32, nibble j of word k/8 holds the
// code of input k = 8*(k/8) + j. A stacked MoE weight (E, N, K/8) is the same matrix with E*N
// rows, which lands expert-major in the tile order too.
// Each thread writes one lane's 16 bytes of one tile.
#include "w4a8_common.h"

namespace w4a8 {

__device__ __forceinline__ uint32_t code_at(const int32_t* w, int64_t K8, int64_t n, int64_t k) {
  return ((uint32_t)w[n * K8 + (k >> 3)] >> (4 * (k & 7))) & 15u;
}

__global__ void repack_int4_kernel(const int32_t* __restrict__ w, int64_t N, int64_t K, int64_t KT,
                                   uint4* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (N / kTileN) * KT * 64;
  if (gid >= total) return;
  const int lane = (int)(gid & 63);
  const int64_t tile = gid >> 6;
  const int64_t kt = tile % KT, ns = tile / KT;
  const int64_t n = ns * kTileN + (lane & 15);
  const int q = lane >> 4;
  const int64_t K8 = K / 8;
  uint32_t dw[4] = {0, 0, 0, 0};
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const int64_t k = kt * kTileK + (e < 16 ? 16 * q + e : 64 + 16 * q + (e - 16));
    uint32_t c = 0;  // padding (beyond K): activations there are zero
    if (k < K) {
      const uint32_t code = code_at(w, K8, n, k);
      c = code >= 8 ? code - 8 : 15 - code;
    }
    const int d = e >> 3, within = e & 7;
    const int byte = within & 3, shift = 8 * byte + (within >= 4 ? 4 : 0);
    dw[d] |= c << shift;
  }
  out[gid] = make_uint4(dw[0], dw[1], dw[2], dw[3]);
}

__global__ void repack_e2m1_kernel(const int32_t* __restrict__ w, int64_t N, int64_t K, int64_t KT,
                                   uint4* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (N / kTileN) * KT * 64;
  if (gid >= total) return;
  const int lane = (int)(gid & 63);
  const int64_t tile = gid >> 6;
  const int64_t kt = tile % KT, ns = tile / KT;
  const int64_t n = ns * kTileN + (lane & 15);
  const int q = lane >> 4;
  const int64_t K8 = K / 8;
  uint32_t dw[4] = {0, 0, 0, 0};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int64_t k = kt * kTileK + 32 * q + 8 * d;
    if (k < K) dw[d] = (uint32_t)w[n * K8 + (k >> 3)];
  }
  out[gid] = make_uint4(dw[0], dw[1], dw[2], dw[3]);
}

int launch_repack(const int32_t* w, int64_t N, int64_t K, int wfmt, void* out, hipStream_t stream) {
  const int64_t KT = (K + kTileK - 1) / kTileK;
  const int64_t total = (N / kTileN) * KT * 64;
  if (total == 0) return kOk;
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  if (wfmt == kInt4)
    hipLaunchKernelGGL(repack_int4_kernel, dim3((unsigned)blocks), dim3(threads), 0, stream, w, N, K,
                       KT, reinterpret_cast<uint4*>(out));
  else
    hipLaunchKernelGGL(repack_e2m1_kernel, dim3((unsigned)blocks), dim3(threads), 0, stream, w, N, K,
                       KT, reinterpret_cast<uint4*>(out));
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

}  // namespace w4a8

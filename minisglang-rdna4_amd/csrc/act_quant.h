// Per-token fp8-e4m3 activation quantization of one row by one 256-thread workgroup; shared by the
// act-quant kernel and the MoE route/align kernel, which quantizes the tokens in the same launch.
//
// Contract (python/minisgl/quant/kernels.py:1703-1712, python/minisgl/layers/norm.py:27-46):
// amax = max |x|; s = max(amax / 448, 1e-8); q = e4m3_rne(x * (1 / s)), unclamped. The division
// and reciprocal are IEEE-rounded f32 operations; v_cvt_pk_fp8_f32 rounds to nearest even.
#pragma once
#include "w4a8_common.h"

namespace w4a8 {

constexpr int kAqThreads = 256;

// workgroup (NT threads) maximum; every thread of the workgroup must call it; red holds NT/64 floats
template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
  const int tid = threadIdx.x;
  v = wave_max(v);
  if ((tid & 63) == 0) red[tid >> 6] = v;
  lds_barrier();
  v = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) v = fmaxf(v, red[w]);
  lds_barrier();
  return v;
}

// One row (K <= CPW*512) quantized by one wave: CPW 16-byte loads per lane, all issued before the
// first use, the maximum by wave_max alone (no LDS, no barrier). Same arithmetic as quant_row, bit
// for bit. All 64 lanes active.
template <int CPW>
__device__ __forceinline__ void quant_row_wave(const uint16_t* __restrict__ xr, int64_t K, int dtype,
                                               uint8_t* __restrict__ qr, float* __restrict__ scale_out, int lane) {
  uint4 raw[CPW];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int64_t k = ((int64_t)c * 64 + lane) * 8;
    raw[c] = k < K ? *reinterpret_cast<const uint4*>(xr + k) : make_uint4(0, 0, 0, 0);
  }
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < CPW; ++c) amax = fmaxf(amax, amax8(raw[c], dtype));
  const float s = act_row_scale(wave_max(amax));
  const float inv = 1.0f / s;
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int64_t k = ((int64_t)c * 64 + lane) * 8;
    if (k < K) {
      float f[8];
      unpack8(raw[c], dtype, f);
      *reinterpret_cast<uint2*>(qr + k) = quant8(f, inv);
    }
  }
  if (lane == 0) *scale_out = s;
}

// One row quantized by a workgroup of NT threads, 8 elements per thread per pass. CPT > 0: the row
// (<= NT*8*CPT elements) is read once into registers. CPT == 0: two passes.
template <int CPT, int NT = kAqThreads>
__device__ __forceinline__ void quant_row(const uint16_t* __restrict__ xr, int64_t K, int dtype,
                                          uint8_t* __restrict__ qr, float* __restrict__ scale_out, float* red) {
  const int tid = threadIdx.x;
  float amax = 0.0f;
  if (CPT > 0) {
    uint4 raw[CPT > 0 ? CPT : 1];
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int64_t k = ((int64_t)c * NT + tid) * 8;
      raw[c] = k < K ? *reinterpret_cast<const uint4*>(xr + k) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < CPT; ++c) amax = fmaxf(amax, amax8(raw[c], dtype));
    const float s = act_row_scale(block_max<NT>(amax, red));
    const float inv = 1.0f / s;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int64_t k = ((int64_t)c * NT + tid) * 8;
      if (k < K) {
        float f[8];
        unpack8(raw[c], dtype, f);
        *reinterpret_cast<uint2*>(qr + k) = quant8(f, inv);
      }
    }
    if (tid == 0) *scale_out = s;
  } else {
    for (int64_t k = (int64_t)tid * 8; k < K; k += NT * 8)
      amax = fmaxf(amax, amax8(*reinterpret_cast<const uint4*>(xr + k), dtype));
    const float s = act_row_scale(block_max<NT>(amax, red));
    const float inv = 1.0f / s;
    for (int64_t k = (int64_t)tid * 8; k < K; k += NT * 8) {
      float f[8];
      unpack8(*reinterpret_cast<const uint4*>(xr + k), dtype, f);
      *reinterpret_cast<uint2*>(qr + k) = quant8(f, inv);
    }
    if (tid == 0) *scale_out = s;
  }
}

// registers-per-thread depth of quant_row for a row of K elements (0: two passes)
inline int quant_row_cpt(int64_t K, int nt = kAqThreads) {
  const int64_t chunks = (K + nt * 8 - 1) / (nt * 8);
  return chunks <= 1 ? 1 : chunks <= 2 ? 2 : chunks <= 4 ? 4 : chunks <= 8 ? 8 : chunks <= 16 ? 16 : 0;
}

}  // namespace w4a8

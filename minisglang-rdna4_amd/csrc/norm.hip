// RMSNorm with an optional fused residual add, and the per-token fp8 quant of its output as an
// epilogue: the producer side of the W4A8 linears.
//
// Restates tail_hip's rms_norm / rms_norm_add / rms_norm_quant / rms_norm_add_quant (called from
// python/minisgl/layers/norm.py:9-58 and 134-168; contract there and in
// tools/w4a8_producer_actquant.py:113-136):
//   residual <- x + residual (in the activation dtype; rms_norm_add only, in place)
//   normed    = dtype(v * rsqrt(mean(v^2) + eps))      over the f32-widened row v
//   out       = dtype(normed * g)  with g = weight, dtype(weight + 1) (plus_one) or no gain
//   (x_fp8, act_scales) = the act-quant of out, bit for bit what w4a8_act_quant(out) returns
// The mean is a fixed-order f32 sum: each of the NT threads accumulates its 8-element chunks
// (elements (c*NT + t)*8 + i, chunk order then element order, fused multiply-add), each wave sums
// in DPP tree order, the NT/64 wave sums in a balanced pairwise tree. rsqrt is 1 / sqrt, both
// correctly rounded. NT depends on K only (256 up to 2048, 512 up to 4096, else 1024), so a row's
// result does not depend on the batch it comes in.
//
// One workgroup per row (grid-stride over rows); the row is read once into registers, 8 elements
// per thread per 16-byte chunk, CPT chunks per thread. Rows are wide and few at decode, so the
// per-element work is spread over as many threads as a row has chunks (up to 1024).
#include "act_quant.h"

namespace w4a8 {

// fixed-order workgroup sum of NW waves (a balanced pairwise tree over the wave sums); every
// thread must call it
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  lds_barrier();
  float t[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) t[w] = red[w];
#pragma unroll
  for (int s = 1; s < NW; s <<= 1)
#pragma unroll
    for (int w = 0; w + s < NW; w += 2 * s) t[w] = t[w] + t[w + s];
  lds_barrier();
  return t[0];
}

// DT (bf16 / fp16) is a template constant: per-element conversions carry no dtype branch
template <int NT, int CPT, bool ADD, bool QUANT, int DT>
__global__ void __launch_bounds__(NT)
rms_norm_kernel(const uint16_t* x, int64_t ldx, uint16_t* __restrict__ res, int64_t ldr,
                const uint16_t* __restrict__ weight, int plus_one, float eps, int64_t M, int64_t K,
                uint16_t* out, int64_t ldo, uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scales) {
  constexpr int dtype = DT;
  __shared__ float red[NT / 64];
  const int tid = threadIdx.x;
  // the gain is the same for every row: loaded once, widened (and shifted by one) per use
  uint4 wv[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int64_t k = ((int64_t)c * NT + tid) * 8;
    wv[c] = (weight && k < K) ? *reinterpret_cast<const uint4*>(weight + k) : make_uint4(0, 0, 0, 0);
  }
  // out may be x itself: each thread reads its chunks of a row before writing them, and no
  // thread touches another's chunks
  for (int64_t m = blockIdx.x; m < M; m += gridDim.x) {
    uint4 v[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int64_t k = ((int64_t)c * NT + tid) * 8;
      v[c] = k < K ? *reinterpret_cast<const uint4*>(x + m * ldx + k) : make_uint4(0, 0, 0, 0);
    }
    if (ADD) {
      // residual <- x + residual, one rounding per element (the dtype add). Every residual chunk is
      // loaded before the first store, so the loads are not held behind the stores.
      uint4 rv[CPT];
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int64_t k = ((int64_t)c * NT + tid) * 8;
        rv[c] = k < K ? *reinterpret_cast<const uint4*>(res + m * ldr + k) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int64_t k = ((int64_t)c * NT + tid) * 8;
        if (k < K) {
          uint16_t* rp = res + m * ldr + k;
          float fx[8], fr[8];
          unpack8(v[c], dtype, fx);
          unpack8(rv[c], dtype, fr);
          uint32_t w4[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            w4[i] = (uint32_t)to_dtype(fx[2 * i] + fr[2 * i], dtype) |
                    ((uint32_t)to_dtype(fx[2 * i + 1] + fr[2 * i + 1], dtype) << 16);
          v[c] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
          *reinterpret_cast<uint4*>(rp) = v[c];
        }
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      float f[8];
      unpack8(v[c], dtype, f);  // chunks past K are zero
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(f[i], f[i], ss);
    }
    const float mean = block_sum<NT / 64>(ss, red) / (float)K;
    const float rstd = 1.0f / sqrtf(mean + eps);
    float amax = 0.f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int64_t k = ((int64_t)c * NT + tid) * 8;
      float f[8];
      unpack8(v[c], dtype, f);
      float g[8];
      if (weight) {
        unpack8(wv[c], dtype, g);
        if (plus_one) {
#pragma unroll
          for (int i = 0; i < 8; ++i) g[i] = from_dtype(to_dtype(g[i] + 1.0f, dtype), dtype);
        }
      }
      uint32_t w4[4];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float o = from_dtype(to_dtype(f[i] * rstd, dtype), dtype);
        if (weight) o = from_dtype(to_dtype(o * g[i], dtype), dtype);
        f[i] = o;
        amax = fmaxf(amax, fabsf(o));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w4[i] = (uint32_t)to_dtype(f[2 * i], dtype) | ((uint32_t)to_dtype(f[2 * i + 1], dtype) << 16);
      v[c] = make_uint4(w4[0], w4[1], w4[2], w4[3]);  // out, rounded
      if (k < K) *reinterpret_cast<uint4*>(out + m * ldo + k) = v[c];
    }
    if (QUANT) {
      // the act-quant of the rounded output row (quant_row's arithmetic)
      const float s = act_row_scale(block_max<NT>(amax, red));
      const float inv = 1.0f / s;
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        const int64_t k = ((int64_t)c * NT + tid) * 8;
        if (k < K) {
          float f[8];
          unpack8(v[c], dtype, f);
          *reinterpret_cast<uint2*>(q + m * ldq + k) = quant8(f, inv);
        }
      }
      if (tid == 0) scales[m] = s;
    }
  }
}

template <int NT, int CPT, int DT>
static void launch_norm_dt(dim3 g, hipStream_t st, const uint16_t* x, int64_t ldx, uint16_t* res, int64_t ldr,
                           const uint16_t* w, int plus_one, float eps, int64_t M, int64_t K, uint16_t* out, int64_t ldo,
                           uint8_t* q, int64_t ldq, float* scales) {
  const dim3 b(NT);
  if (res && q)
    hipLaunchKernelGGL((rms_norm_kernel<NT, CPT, true, true, DT>), g, b, 0, st, x, ldx, res, ldr, w, plus_one, eps, M,
                       K, out, ldo, q, ldq, scales);
  else if (res)
    hipLaunchKernelGGL((rms_norm_kernel<NT, CPT, true, false, DT>), g, b, 0, st, x, ldx, res, ldr, w, plus_one, eps, M,
                       K, out, ldo, q, ldq, scales);
  else if (q)
    hipLaunchKernelGGL((rms_norm_kernel<NT, CPT, false, true, DT>), g, b, 0, st, x, ldx, res, ldr, w, plus_one, eps, M,
                       K, out, ldo, q, ldq, scales);
  else
    hipLaunchKernelGGL((rms_norm_kernel<NT, CPT, false, false, DT>), g, b, 0, st, x, ldx, res, ldr, w, plus_one, eps,
                       M, K, out, ldo, q, ldq, scales);
}

template <int NT, int CPT>
static void launch_norm_cpt(dim3 g, hipStream_t st, const uint16_t* x, int64_t ldx, uint16_t* res, int64_t ldr,
                            const uint16_t* w, int plus_one, float eps, int64_t M, int64_t K, int dtype, uint16_t* out,
                            int64_t ldo, uint8_t* q, int64_t ldq, float* scales) {
  if (dtype == kBF16)
    launch_norm_dt<NT, CPT, kBF16>(g, st, x, ldx, res, ldr, w, plus_one, eps, M, K, out, ldo, q, ldq, scales);
  else
    launch_norm_dt<NT, CPT, kF16>(g, st, x, ldx, res, ldr, w, plus_one, eps, M, K, out, ldo, q, ldq, scales);
}

// Threads per row from K alone: 256 up to 2048, 512 up to 4096, 1024 beyond (the oracle mirrors
// this, since the f32 sum order follows it).
int rms_norm_threads(int64_t K) { return K <= 2048 ? 256 : K <= 4096 ? 512 : 1024; }

// Rows of up to 32768 elements; returns kErrUnsupported beyond.
int launch_rms_norm(const void* x, int64_t ldx, void* res, int64_t ldr, const void* weight, int plus_one, float eps,
                    int64_t M, int64_t K, int dtype, void* out, int64_t ldo, uint8_t* q, int64_t ldq, float* scales,
                    hipStream_t stream) {
  if (M <= 0) return kOk;
  if (K > 32768) return kErrUnsupported;
  const int nt = rms_norm_threads(K);
  const int64_t chunks = (K + nt * 8 - 1) / (nt * 8);  // 1..4
  const dim3 g((unsigned)(M < 8192 ? M : 8192));
  auto xp = reinterpret_cast<const uint16_t*>(x);
  auto rp = reinterpret_cast<uint16_t*>(res);
  auto wp = reinterpret_cast<const uint16_t*>(weight);
  auto op = reinterpret_cast<uint16_t*>(out);
#define W4A8_NORM(NT_, C_) launch_norm_cpt<NT_, C_>(g, stream, xp, ldx, rp, ldr, wp, plus_one, eps, M, K, dtype, op, ldo, \
                                                    q, ldq, scales)
  if (nt == 256) W4A8_NORM(256, 1);
  else if (nt == 512) W4A8_NORM(512, 1);
  else if (chunks <= 1) W4A8_NORM(1024, 1);
  else if (chunks <= 2) W4A8_NORM(1024, 2);
  else W4A8_NORM(1024, 4);
#undef W4A8_NORM
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

}  // namespace w4a8

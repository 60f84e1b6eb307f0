// W4A16 (unquantized activations) on the fp8 MFMA kernels: the activation pieces.
//
// The reference's W4A16 arm (python/minisgl/quant/kernels.py:1125-1178, 1756-1786) multiplies the
// 4-bit weights against bf16/fp16 activations that are never rounded. Here each activation row is
// split, exactly, into T fp8-e4m3 rows with power-of-two scales,
//   x = 2^E * (a_0 + a_1 / 16 + ... + a_{T-1} / 16^(T-1)),   a_t = e4m3(16^t * r_t),
// where r_0 = x / 2^E and r_{t+1} = 16 * r_t - a_t. 2^E is the smallest power of two with
// amax / 2^E <= 448. Every step is exact in f32 (scaling by powers of two, and the subtraction of a
// value's own rounding), and each term carries the next 4 significant bits: two terms hold every
// bf16 value (8 bits) and three every fp16 value (11 bits) whose scaled magnitude is at least 2^-6
// (smaller ones keep what the e4m3 subnormals hold, an absolute error under 2^(E-13)). The T rows go
// through the ordinary W4A8 GEMM (row t of token m at row T*m + t, scale 2^(E-4t)) into an f32
// buffer, and the sum kernel adds each token's T rows in row order and rounds once to the
// activation dtype (for the fused gate_up arm: silu(gate) * up, rounded as the W4A8 fused arm does).
#include "act_quant.h"

namespace w4a16 {
using namespace w4a8;

constexpr int kSplitThreads = 256;

// smallest E with amax <= 448 * 2^E (amax = m * 2^e, m in [1, 2): E = e - 8 if m <= 1.75, else
// e - 7); 0 for a zero row
__device__ __forceinline__ int split_exponent(float amax) {
  if (!(amax > 0.0f)) return 0;
  int e;
  const float m = 2.0f * frexpf(amax, &e);  // amax = (m / 2) * 2^e, m in [1, 2)
  e -= 1;
  return m <= 1.75f ? e - 8 : e - 7;
}

// r <- 16 * (r - e4m3(c)) for the 8 values just rounded to c (exact)
__device__ __forceinline__ void split_residual(float (&r)[8], uint2 c) {
  float a[8];
  a[0] = __builtin_amdgcn_cvt_f32_fp8((int)c.x, 0);
  a[1] = __builtin_amdgcn_cvt_f32_fp8((int)c.x, 1);
  a[2] = __builtin_amdgcn_cvt_f32_fp8((int)c.x, 2);
  a[3] = __builtin_amdgcn_cvt_f32_fp8((int)c.x, 3);
  a[4] = __builtin_amdgcn_cvt_f32_fp8((int)c.y, 0);
  a[5] = __builtin_amdgcn_cvt_f32_fp8((int)c.y, 1);
  a[6] = __builtin_amdgcn_cvt_f32_fp8((int)c.y, 2);
  a[7] = __builtin_amdgcn_cvt_f32_fp8((int)c.y, 3);
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (r[i] - a[i]) * 16.0f;
}

// one workgroup per row (grid-stride over rows); the row is read twice (max, then split)
template <int T>
__global__ void __launch_bounds__(kSplitThreads)
act_split_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t K, int dtype,
                 uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scales) {
  __shared__ float red[kSplitThreads / 64];
  const int tid = threadIdx.x;
  for (int64_t m = blockIdx.x; m < M; m += gridDim.x) {
    const uint16_t* xr = x + m * ldx;
    float amax = 0.0f;
    for (int64_t k = (int64_t)tid * 8; k < K; k += kSplitThreads * 8)
      amax = fmaxf(amax, amax8(*reinterpret_cast<const uint4*>(xr + k), dtype));
    const int E = split_exponent(block_max<kSplitThreads>(amax, red));
    for (int64_t k = (int64_t)tid * 8; k < K; k += kSplitThreads * 8) {
      float r[8];
      unpack8(*reinterpret_cast<const uint4*>(xr + k), dtype, r);
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = ldexpf(r[i], -E);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const uint2 c = quant8(r, 1.0f);
        *reinterpret_cast<uint2*>(q + (T * m + t) * ldq + k) = c;
        if (t + 1 < T) split_residual(r, c);
      }
    }
    if (tid < T) scales[T * m + tid] = ldexpf(1.0f, E - 4 * tid);
  }
}

// python/minisgl/quant/kernels.py:1756-1786 (bit-exact to w4a16_linear + silu_and_mul): gate and
// up rounded to the dtype, silu in f32, rounded, times up (the caller rounds the product)
template <int DT>
__device__ __forceinline__ float silu_mul_dt(float gate, float up) {
  const float gg = from_dtype(to_dtype(gate, DT), DT);
  const float uu = from_dtype(to_dtype(up, DT), DT);
  const float sg = gg / (1.0f + expf(-gg));
  return from_dtype(to_dtype(sg, DT), DT) * uu;
}

// out[m, c] = dtype(sum_t y[T*m + t, c]) (sum in t order); silu: out[m, c] over gate column c and
// up column c + N/2. One thread per 4 output columns.
template <int T, int DT, bool SILU>
__global__ void __launch_bounds__(256)
tsum_kernel(const float* __restrict__ y, int64_t N, int64_t M, void* __restrict__ out, int64_t ldo) {
  const int64_t nout = SILU ? N / 2 : N;
  const int64_t per_row = nout / 4;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * per_row) return;
  const int64_t m = idx / per_row, c = (idx % per_row) * 4;
  float g[4] = {0.f, 0.f, 0.f, 0.f}, u[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const float* yr = y + (T * m + t) * N;
    const float4 a = *reinterpret_cast<const float4*>(yr + c);
    g[0] += a.x; g[1] += a.y; g[2] += a.z; g[3] += a.w;
    if (SILU) {
      const float4 b = *reinterpret_cast<const float4*>(yr + nout + c);
      u[0] += b.x; u[1] += b.y; u[2] += b.z; u[3] += b.w;
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float v = SILU ? silu_mul_dt<DT>(g[i], u[i]) : g[i];
    reinterpret_cast<uint16_t*>(out)[m * ldo + c + i] = to_dtype(v, DT);
  }
}

constexpr int kMidThreads = 128;
constexpr int64_t kMidMaxInter = 32768;  // the h row lives in LDS: 2 bytes per column

// The middle of the MoE W4A16 arm, one workgroup per routed slot s = m*top_k + j (grid-stride):
// silu_and_mul between the reference's two grouped W4A16 GEMMs (python/minisgl/quant/kernels.py:
// 962-975), whose gemm2 then reads h unquantized. gemm1 ran over the split activations under a
// route with T virtual tokens per token (virtual token T*m + t carries term t and token m's
// experts), so the slot's gate|up row is the sum, in t order, of the f32 rows at padded positions
// pos_t = inv_pos[(T*m + t)*top_k + j]. h = silu(gate) * up in the dtype (silu_mul_dt), then split
// exactly as act_split_kernel splits a row: term t goes to row pos_t of q with scale 2^(E - 4t), so
// gemm2 over the same route reads the slot's T terms by padded position (every pos_t belongs to
// the slot's expert). h_out (optional): h at row s. A slot with pos_0 < 0 (dropped) is skipped.
template <int T, int DT>
__global__ void __launch_bounds__(kMidThreads)
moe_silu_split_kernel(const float* __restrict__ y, int64_t ldy, const int32_t* __restrict__ inv_pos, int64_t numel,
                      int top_k, int64_t I, uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scales,
                      uint16_t* __restrict__ h_out, int64_t ldh) {
  extern __shared__ uint4 hs4[];  // h of this slot; each thread reads back only what it wrote
  __shared__ float red[kMidThreads / 64];
  uint16_t* hs = reinterpret_cast<uint16_t*>(hs4);
  const int tid = threadIdx.x;
  for (int64_t s = blockIdx.x; s < numel; s += gridDim.x) {
    const int64_t m = s / top_k, j = s - m * top_k;
    int64_t pos[T];
#pragma unroll
    for (int t = 0; t < T; ++t) pos[t] = inv_pos[(T * m + t) * top_k + j];
    if (pos[0] < 0) continue;  // the same for the whole workgroup
    float amax = 0.0f;
    for (int64_t c = (int64_t)tid * 8; c < I; c += kMidThreads * 8) {
      float g[8], u[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) g[i] = u[i] = 0.0f;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float* yr = y + pos[t] * ldy + c;
        const float4 g0 = *reinterpret_cast<const float4*>(yr), g1 = *reinterpret_cast<const float4*>(yr + 4);
        const float4 u0 = *reinterpret_cast<const float4*>(yr + I), u1 = *reinterpret_cast<const float4*>(yr + I + 4);
        g[0] += g0.x; g[1] += g0.y; g[2] += g0.z; g[3] += g0.w;
        g[4] += g1.x; g[5] += g1.y; g[6] += g1.z; g[7] += g1.w;
        u[0] += u0.x; u[1] += u0.y; u[2] += u0.z; u[3] += u0.w;
        u[4] += u1.x; u[5] += u1.y; u[6] += u1.z; u[7] += u1.w;
      }
      uint16_t hb[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        hb[i] = to_dtype(silu_mul_dt<DT>(g[i], u[i]), DT);
        amax = fmaxf(amax, fabsf(from_dtype(hb[i], DT)));
      }
      uint4 w;
      w.x = hb[0] | ((uint32_t)hb[1] << 16); w.y = hb[2] | ((uint32_t)hb[3] << 16);
      w.z = hb[4] | ((uint32_t)hb[5] << 16); w.w = hb[6] | ((uint32_t)hb[7] << 16);
      *reinterpret_cast<uint4*>(hs + c) = w;
      if (h_out) *reinterpret_cast<uint4*>(h_out + s * ldh + c) = w;
    }
    const int E = split_exponent(block_max<kMidThreads>(amax, red));
    for (int64_t c = (int64_t)tid * 8; c < I; c += kMidThreads * 8) {
      float r[8];
      unpack8(*reinterpret_cast<const uint4*>(hs + c), DT, r);
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = ldexpf(r[i], -E);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const uint2 cw = quant8(r, 1.0f);
        *reinterpret_cast<uint2*>(q + pos[t] * ldq + c) = cw;
        if (t + 1 < T) split_residual(r, cw);
      }
    }
    if (tid < T) scales[pos[tid]] = ldexpf(1.0f, E - 4 * tid);
  }
}

}  // namespace w4a16

namespace w4a8 {

// terms per activation value: 2 for bf16, 3 for fp16
int w4a16_terms(int dtype) { return dtype == kBF16 ? 2 : 3; }

int launch_act_split(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* q, int64_t ldq,
                     float* scales, hipStream_t stream) {
  if (M <= 0) return kOk;
  const dim3 g((unsigned)(M < 16384 ? M : 16384)), b(w4a16::kSplitThreads);
  auto xp = reinterpret_cast<const uint16_t*>(x);
  if (w4a16_terms(dtype) == 2)
    hipLaunchKernelGGL(w4a16::act_split_kernel<2>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales);
  else
    hipLaunchKernelGGL(w4a16::act_split_kernel<3>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

template <int T, int DT>
static void tsum_dt(const float* y, int64_t N, int64_t M, void* out, int64_t ldo, int silu, hipStream_t st) {
  const int64_t n = M * ((silu ? N / 2 : N) / 4);
  const dim3 g((unsigned)((n + 255) / 256)), b(256);
  if (silu) hipLaunchKernelGGL((w4a16::tsum_kernel<T, DT, true>), g, b, 0, st, y, N, M, out, ldo);
  else hipLaunchKernelGGL((w4a16::tsum_kernel<T, DT, false>), g, b, 0, st, y, N, M, out, ldo);
}

// y: (T*M, N) f32 rows of the split GEMM; out: (M, N or N/2) in dtype, row stride ldo
int launch_tsum(const float* y, int64_t N, int64_t M, int dtype, void* out, int64_t ldo, int silu, hipStream_t st) {
  if (M <= 0) return kOk;
  if (dtype == kBF16) tsum_dt<2, kBF16>(y, N, M, out, ldo, silu, st);
  else tsum_dt<3, kF16>(y, N, M, out, ldo, silu, st);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

int64_t w4a16_moe_max_inter() { return w4a16::kMidMaxInter; }

// y: gemm1's (P, 2I) f32 rows over the virtual route; inv_pos: (T*terms*top_k,) of that route
int launch_moe_silu_split(const float* y, int64_t ldy, const int32_t* inv_pos, int64_t T, int top_k, int64_t I,
                          int dtype, uint8_t* q, int64_t ldq, float* scales, void* h, int64_t ldh, hipStream_t st) {
  const int64_t numel = T * top_k;
  if (numel <= 0) return kOk;
  const dim3 g((unsigned)(numel < 65536 ? numel : 65536)), b(w4a16::kMidThreads);
  const size_t lds = (size_t)I * 2;
  auto hp = reinterpret_cast<uint16_t*>(h);
  if (dtype == kBF16)
    hipLaunchKernelGGL((w4a16::moe_silu_split_kernel<2, kBF16>), g, b, lds, st, y, ldy, inv_pos, numel, top_k, I, q,
                       ldq, scales, hp, ldh);
  else
    hipLaunchKernelGGL((w4a16::moe_silu_split_kernel<3, kF16>), g, b, lds, st, y, ldy, inv_pos, numel, top_k, I, q,
                       ldq, scales, hp, ldh);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

}  // namespace w4a8

// MoE routing, token-slot alignment and top-k combine for the grouped W4A8 FFN.
//
// route: restates the softmax + top-k + renormalize half of moe_hip.moe_route_align
//   (python/minisgl/quant/kernels.py:423-447): softmax over f32-widened logits, top-k with exact
//   ties keeping the LOWER expert index (python/minisgl/layers/moe.py:1218-1227), weights
//   renormalised by sum + 1e-8 (python/minisgl/moe/fused.py:52-53). One wave per token; experts
//   are selected on the logits, which orders them exactly as the softmax does.
// align: restates moe_align_block_size (python/minisgl/moe/fused.py:120-176): slots sorted by
//   expert, stable in slot order, each expert padded to a multiple of block_m with the sentinel
//   numel, per-block expert id (blocks past the end clamp to E-1), padded total ntp. A single
//   workgroup builds it deterministically: an LDS histogram, a scan, then chunks of 1024 slots
//   ranked with wave ballots (lanes holding the same expert) and per-wave counts in LDS.
// combine: out[t] = sum_j tw[t,j] * y[pos(t,j)] in f32, j in slot order, cast to the activation
//   dtype (mmq_fp8_moe_gather_reduce, kernels.py:876-882).
#include "w4a8_common.h"

namespace w4a8 {

constexpr int kMaxExperts = 512;
constexpr int kRouteMaxPerLane = kMaxExperts / 64;

__device__ __forceinline__ float load_logit(const void* p, int dtype, int64_t i) {
  if (dtype == kF32) return reinterpret_cast<const float*>(p)[i];
  return from_dtype(reinterpret_cast<const uint16_t*>(p)[i], dtype);
}

__global__ void __launch_bounds__(256)
moe_route_kernel(const void* __restrict__ logits, int dtype, int64_t T, int E, int top_k, int renorm,
                 float* __restrict__ tw, int32_t* __restrict__ ids) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  float v[kRouteMaxPerLane];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kRouteMaxPerLane; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? load_logit(logits, dtype, t * E + e) : -INFINITY;
    mx = fmaxf(mx, v[i]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < kRouteMaxPerLane; ++i) {
    const int e = lane + 64 * i;
    if (e < E) sum += expf(v[i] - mx);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);

  unsigned used = 0;  // bit i: expert lane + 64*i taken
  float wsum = 0.f;
  float myw = 0.f;
  int myid = 0;
  for (int j = 0; j < top_k; ++j) {
    // lane-local best unused (largest logit, lowest index)
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < kRouteMaxPerLane; ++i) {
      const int e = lane + 64 * i;
      if (e < E && !((used >> i) & 1u) && (v[i] > bv || (v[i] == bv && e < bi))) {
        bv = v[i];
        bi = e;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if ((bi & 63) == lane) used |= 1u << (bi >> 6);
    const float p = expf(bv - mx) / sum;
    wsum += p;
    if (lane == j) {
      myw = p;
      myid = bi;
    }
  }
  if (lane < top_k) {
    tw[t * top_k + lane] = renorm ? myw / (wsum + 1e-8f) : myw;
    ids[t * top_k + lane] = myid;
  }
}

constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / 64;

__global__ void __launch_bounds__(kAlignThreads)
moe_align_kernel(const int32_t* __restrict__ ids, int64_t numel, int E, int bm, int64_t P,
                 int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
                 int32_t* __restrict__ ntp_out, int32_t* __restrict__ inv_pos) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int base[kMaxExperts];
  __shared__ int wcount[kAlignWaves][kMaxExperts];
  __shared__ int wsums[kAlignWaves];
  __shared__ int total_s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < kMaxExperts; e += kAlignThreads) cnt[e] = 0;
  for (int i = tid; i < kAlignWaves * kMaxExperts; i += kAlignThreads) (&wcount[0][0])[i] = 0;
  __syncthreads();
  for (int64_t i = tid; i < numel; i += kAlignThreads) {
    const int e = ids[i];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // exclusive scan of padded counts over experts (E <= 1024 = one element per thread)
  int padded = 0;
  if (tid < E) padded = (cnt[tid] + bm - 1) / bm * bm;
  int incl = padded;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int n = __shfl_up(incl, o, 64);
    if (lane >= o) incl += n;
  }
  if (lane == 63) wsums[wave] = incl;
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int w = 0; w < kAlignWaves; ++w) {
      const int s = wsums[w];
      wsums[w] = run;
      run += s;
    }
    total_s = run;
  }
  __syncthreads();
  const int excl = incl - padded + wsums[wave];
  if (tid < E) base[tid] = excl;
  const int total = total_s;
  __syncthreads();
  // fill sentinel and block owners
  for (int64_t i = tid; i < P; i += kAlignThreads) sorted_ids[i] = (int32_t)numel;
  const int64_t nblocks = (P + bm - 1) / bm;
  for (int64_t b = tid; b < nblocks; b += kAlignThreads) expert_ids[b] = E - 1;
  __syncthreads();
  if (tid < E) {
    const int b0 = base[tid] / bm, nb = (cnt[tid] + bm - 1) / bm;
    for (int b = 0; b < nb; ++b) expert_ids[b0 + b] = tid;
  }
  if (tid == 0) *ntp_out = total;
  // stable scatter in chunks of kAlignThreads slots
  for (int64_t c0 = 0; c0 < numel; c0 += kAlignThreads) {
    const int64_t i = c0 + tid;
    int e = -1;
    if (i < numel) {
      e = ids[i];
      if (e < 0 || e >= E) e = -1;
    }
    const int key = e < 0 ? 0x7ff : e;  // 11-bit key; invalid slots group together and are dropped
    uint64_t peers = __ballot(1);
#pragma unroll
    for (int b = 0; b < 11; ++b) {
      const int bit = (key >> b) & 1;
      const uint64_t bal = __ballot(bit);
      peers &= bit ? bal : ~bal;
    }
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int rank = __popcll(peers & below);
    const int leader = __ffsll((long long)peers) - 1;
    if (e >= 0 && lane == leader) wcount[wave][e] = __popcll(peers);
    if (e < 0 && i < numel && inv_pos) inv_pos[i] = -1;  // dropped slot: the combine skips it
    __syncthreads();
    if (e >= 0) {
      int off = base[e] + rank;
      for (int w = 0; w < wave; ++w) off += wcount[w][e];
      sorted_ids[off] = (int32_t)i;
      if (inv_pos) inv_pos[i] = off;
    }
    __syncthreads();
    if (tid < E) {
      int add = 0;
      for (int w = 0; w < kAlignWaves; ++w) {
        add += wcount[w][tid];
        wcount[w][tid] = 0;
      }
      base[tid] += add;
    }
    __syncthreads();
  }
}

__global__ void moe_combine_kernel(const float* __restrict__ y, int64_t ldy,
                                   const int32_t* __restrict__ inv_pos, const float* __restrict__ tw,
                                   int64_t T, int top_k, int64_t H, void* __restrict__ out, int dtype) {
  const int64_t h = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= H) return;
  for (int64_t t = blockIdx.y; t < T; t += gridDim.y) {
    float acc = 0.f;
    for (int j = 0; j < top_k; ++j) {
      const int64_t pos = inv_pos[t * top_k + j];
      if (pos >= 0) acc += tw[t * top_k + j] * y[pos * ldy + h];
    }
    if (dtype == kF32)
      reinterpret_cast<float*>(out)[t * H + h] = acc;
    else
      reinterpret_cast<uint16_t*>(out)[t * H + h] = to_dtype(acc, dtype);
  }
}

int launch_moe_route(const void* logits, int dtype, int64_t T, int E, int top_k, int renorm, float* tw,
                     int32_t* ids, hipStream_t stream) {
  if (T <= 0) return kOk;
  const int per_block = 4;
  hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)((T + per_block - 1) / per_block)),
                     dim3(per_block * 64), 0, stream, logits, dtype, T, E, top_k, renorm, tw, ids);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

int launch_moe_align(const int32_t* ids, int64_t numel, int E, int bm, int64_t P, int32_t* sorted_ids,
                     int32_t* expert_ids, int32_t* ntp, int32_t* inv_pos, hipStream_t stream) {
  hipLaunchKernelGGL(moe_align_kernel, dim3(1), dim3(kAlignThreads), 0, stream, ids, numel, E, bm, P,
                     sorted_ids, expert_ids, ntp, inv_pos);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

int launch_moe_combine(const float* y, int64_t ldy, const int32_t* inv_pos, const float* tw, int64_t T,
                       int top_k, int64_t H, void* out, int dtype, hipStream_t stream) {
  if (T <= 0) return kOk;
  dim3 grid((unsigned)((H + 255) / 256), (unsigned)(T < 65535 ? T : 65535));
  hipLaunchKernelGGL(moe_combine_kernel, grid, dim3(256), 0, stream, y, ldy, inv_pos, tw, T, top_k, H,
                     out, dtype);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

}  // namespace w4a8

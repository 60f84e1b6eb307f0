// Router of the grouped W4A8 FFN, shared by the route kernels (moe.hip) and the routed decode GEMV
// (gemv.h). Restates the softmax + top-k + renormalize half of moe_hip.moe_route_align
// (python/minisgl/quant/kernels.py:423-447): softmax over f32-widened logits, top-k with exact ties
// keeping the LOWER expert index (python/minisgl/layers/moe.py:1218-1227), weights renormalised by
// sum + 1e-8 (python/minisgl/moe/fused.py:52-53).
//
// One wave routes one token (all 64 lanes active); lane l holds experts l + 64*i, i < PER. Softmax:
// max, then the sum of exp in a fixed tree order. Top-k: repeated wave argmax on the logits (which
// orders the experts exactly as the probabilities do), on one 64-bit key per (logit, expert) so
// that a single integer maximum settles value and tie at once. Renormalisation: by the selected
// probabilities' sum, taken in selection order, + 1e-8.
#pragma once
#include "w4a8_common.h"

namespace w4a8 {

// DPP broadcasts of lane 15 of each row to the next row, and of lane 31 to rows 2 and 3 (gfx9)
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

// Loads of token t's logits (raw bits), all issued before any use, whatever the dtype.
template <int PER>
__device__ __forceinline__ void route_load(const void* __restrict__ logits, int dtype, int64_t t, int E,
                                           uint32_t (&raw)[PER]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    const int64_t idx = t * E + (e < E ? e : 0);
    raw[i] = dtype == kF32 ? __float_as_uint(reinterpret_cast<const float*>(logits)[idx])
                           : (uint32_t)reinterpret_cast<const uint16_t*>(logits)[idx];
  }
}

__device__ __forceinline__ float route_logit(uint32_t raw, int dtype) {
  return dtype == kF32 ? __uint_as_float(raw) : from_dtype((uint16_t)raw, dtype);
}

// Selection key of (logit v, expert e): the larger key is the larger logit, then the lower expert
// index, exactly as the float comparison orders them (-0 is taken as +0, since -0 == +0). The
// logit's bits map to an order-preserving unsigned (negatives inverted, positives with the sign
// bit set) in the high word, ~e in the low word. 0: no candidate (expert past E, or a NaN logit,
// which the float comparison never selects).
__device__ __forceinline__ uint64_t route_key(float v, int e, bool ok) {
  uint32_t b = __float_as_uint(v);
  b = b == 0x80000000u ? 0u : b;
  const uint32_t u = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (ok && v == v) ? ((uint64_t)u << 32) | (uint32_t)(0xffffffffu - (uint32_t)e) : 0ull;
}
__device__ __forceinline__ float route_key_logit(uint64_t k) {
  const uint32_t u = (uint32_t)(k >> 32);
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

// max of the key with the DPP partner's (rows outside RM keep their own)
template <int CTRL, int RM = 0xf>
__device__ __forceinline__ uint64_t key_max_step(uint64_t k) {
  const uint32_t lo = (uint32_t)k, hi = (uint32_t)(k >> 32);
  uint32_t olo, ohi;
  if constexpr (RM == 0xf) {  // every row written: no old value to keep
    olo = (uint32_t)__builtin_amdgcn_mov_dpp((int)lo, CTRL, 0xf, 0xf, false);
    ohi = (uint32_t)__builtin_amdgcn_mov_dpp((int)hi, CTRL, 0xf, 0xf, false);
  } else {
    olo = (uint32_t)__builtin_amdgcn_update_dpp((int)lo, (int)lo, CTRL, RM, 0xf, false);
    ohi = (uint32_t)__builtin_amdgcn_update_dpp((int)hi, (int)hi, CTRL, RM, 0xf, false);
  }
  const uint64_t o = ((uint64_t)ohi << 32) | olo;
  return o > k ? o : k;
}
// the wave's largest key, uniform: four steps leave each 16-lane row's maximum in all its lanes,
// the two broadcasts carry rows 0-2 into row 3, whose lane 63 then holds the wave's maximum
__device__ __forceinline__ uint64_t wave_key_max(uint64_t k) {
  k = key_max_step<kDppXor1>(k);
  k = key_max_step<kDppXor2>(k);
  k = key_max_step<kDppHalfMirror>(k);
  k = key_max_step<kDppRowMirror>(k);
  k = key_max_step<kDppRowBcast15, 0xa>(k);
  k = key_max_step<kDppRowBcast31, 0xc>(k);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

// The first n choices of a token: lane j < n holds choice j (logit myv, expert myid). Each round
// takes the wave's largest key and clears it where it sits. A round with no candidate left (NaN
// logits) gives logit -inf and expert 0x7fffffff, outside every [0, E). n is uniform.
struct RoutePick {
  float myv;
  int myid;
};

// 16-bit logits (bf16, fp16): the same order in one 32-bit key, the logit's 16 bits mapped the same
// way in the high half and ~e in the low half (E < 65536), so each reduction step is one unsigned
// maximum instead of a 64-bit compare and two selects. 0: no candidate, as above (a mapped value
// of 0 would be the bits 0xffff, a NaN).
__device__ __forceinline__ uint32_t route_key16(uint32_t raw, int dtype, int e, bool ok) {
  const float v = from_dtype((uint16_t)raw, dtype);
  uint32_t b = raw & 0xffffu;
  b = b == 0x8000u ? 0u : b;
  const uint32_t u = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
  return (ok && v == v) ? (u << 16) | (0xffffu - (uint32_t)e) : 0u;
}
__device__ __forceinline__ float route_key16_logit(uint32_t k, int dtype) {
  const uint32_t u = k >> 16;
  const uint32_t b = (u & 0x8000u) ? (u & 0x7fffu) : (~u & 0xffffu);
  return from_dtype((uint16_t)b, dtype);
}
template <int CTRL, int RM = 0xf>
__device__ __forceinline__ uint32_t key16_max_step(uint32_t k) {
  uint32_t o;
  if constexpr (RM == 0xf) o = (uint32_t)__builtin_amdgcn_mov_dpp((int)k, CTRL, 0xf, 0xf, false);
  else o = (uint32_t)__builtin_amdgcn_update_dpp((int)k, (int)k, CTRL, RM, 0xf, false);
  return o > k ? o : k;
}
__device__ __forceinline__ uint32_t wave_key16_max(uint32_t k) {
  k = key16_max_step<kDppXor1>(k);
  k = key16_max_step<kDppXor2>(k);
  k = key16_max_step<kDppHalfMirror>(k);
  k = key16_max_step<kDppRowMirror>(k);
  k = key16_max_step<kDppRowBcast15, 0xa>(k);
  k = key16_max_step<kDppRowBcast31, 0xc>(k);
  return (uint32_t)__builtin_amdgcn_readlane((int)k, 63);
}

template <int PER>
__device__ __forceinline__ RoutePick route_pick(const uint32_t (&raw)[PER], int dtype, int E, int n) {
  const int lane = threadIdx.x & 63;
  if (dtype != kF32) {
    uint32_t key[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = lane + 64 * i;
      key[i] = route_key16(raw[i], dtype, e, e < E);
    }
    uint32_t mine = 0;
    for (int j = 0; j < n; ++j) {
      uint32_t m = key[0];
#pragma unroll
      for (int i = 1; i < PER; ++i) m = key[i] > m ? key[i] : m;
      const uint32_t top = wave_key16_max(m);
#pragma unroll
      for (int i = 0; i < PER; ++i) key[i] = key[i] == top ? 0u : key[i];
      mine = lane == j ? top : mine;
    }
    if (mine == 0u) return RoutePick{-INFINITY, 0x7fffffff};
    return RoutePick{route_key16_logit(mine, dtype), (int)(0xffffu - (mine & 0xffffu))};
  }
  uint64_t key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    key[i] = route_key(route_logit(raw[i], dtype), e, e < E);
  }
  uint64_t mine = 0;
  for (int j = 0; j < n; ++j) {
    uint64_t m = key[0];
#pragma unroll
    for (int i = 1; i < PER; ++i) m = key[i] > m ? key[i] : m;
    const uint64_t top = wave_key_max(m);
#pragma unroll
    for (int i = 0; i < PER; ++i) key[i] = key[i] == top ? 0ull : key[i];
    mine = lane == j ? top : mine;
  }
  if (mine == 0ull) return RoutePick{-INFINITY, 0x7fffffff};
  return RoutePick{route_key_logit(mine), (int)(0xffffffffu - (uint32_t)mine)};
}

// Softmax max and denominator over the token's E logits (experts past E excluded).
template <int PER>
__device__ __forceinline__ void route_softmax(const uint32_t (&raw)[PER], int dtype, int E, float& mx, float& sum) {
  const int lane = threadIdx.x & 63;
  float v[PER];
  mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    v[i] = lane + 64 * i >= E ? -INFINITY : route_logit(raw[i], dtype);
    mx = fmaxf(mx, v[i]);
  }
  mx = wave_max(mx);
  float part = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (lane + 64 * i < E) part += expf(v[i] - mx);
  sum = wave_sum(part);
}

// Routing weight of lane j's choice (lanes j < top_k; the whole wave takes part).
__device__ __forceinline__ float route_weight(const RoutePick& r, float mx, float sum, int top_k, int renorm) {
  const int lane = threadIdx.x & 63;
  const float p = lane < top_k ? expf(r.myv - mx) / sum : 0.f;
  float wsum = 0.f;
  for (int j = 0; j < top_k; ++j) wsum += lane_f(p, j);
  return renorm ? p / (wsum + 1e-8f) : p;
}

// Route of token t: writes the k weights and ids to global memory and the ids to ids_s (LDS,
// optional).
template <int PER>
__device__ __forceinline__ void route_token(const void* __restrict__ logits, int dtype, int64_t t, int E,
                                            int top_k, int renorm, float* __restrict__ tw,
                                            int32_t* __restrict__ ids, int32_t* ids_s) {
  const int lane = threadIdx.x & 63;
  uint32_t raw[PER];
  route_load<PER>(logits, dtype, t, E, raw);
  const RoutePick r = route_pick<PER>(raw, dtype, E, top_k);
  float mx, sum;
  route_softmax<PER>(raw, dtype, E, mx, sum);
  const float w = route_weight(r, mx, sum, top_k, renorm);
  if (lane < top_k) {
    tw[t * top_k + lane] = w;
    ids[t * top_k + lane] = r.myid;
    if (ids_s) ids_s[t * top_k + lane] = r.myid;
  }
}

// Two tokens per wave with 16-bit logits: the two routes' selection rounds, softmax reductions and
// weights are independent chains, so the wave runs them interleaved in about the time of one
// (each token's results are route_token's bits).
template <int PER>
__device__ __forceinline__ void route_token_pair(const void* __restrict__ logits, int dtype, int64_t t0, int64_t t1,
                                                 int E, int top_k, int renorm, float* __restrict__ tw,
                                                 int32_t* __restrict__ ids, int32_t* ids_s) {
  const int lane = threadIdx.x & 63;
  uint32_t raw0[PER], raw1[PER];
  route_load<PER>(logits, dtype, t0, E, raw0);
  route_load<PER>(logits, dtype, t1, E, raw1);
  uint32_t k0[PER], k1[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    k0[i] = route_key16(raw0[i], dtype, e, e < E);
    k1[i] = route_key16(raw1[i], dtype, e, e < E);
  }
  uint32_t mine0 = 0, mine1 = 0;
  for (int j = 0; j < top_k; ++j) {
    uint32_t m0 = k0[0], m1 = k1[0];
#pragma unroll
    for (int i = 1; i < PER; ++i) {
      m0 = k0[i] > m0 ? k0[i] : m0;
      m1 = k1[i] > m1 ? k1[i] : m1;
    }
    const uint32_t top0 = wave_key16_max(m0), top1 = wave_key16_max(m1);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      k0[i] = k0[i] == top0 ? 0u : k0[i];
      k1[i] = k1[i] == top1 ? 0u : k1[i];
    }
    mine0 = lane == j ? top0 : mine0;
    mine1 = lane == j ? top1 : mine1;
  }
  const RoutePick r0 = mine0 == 0u ? RoutePick{-INFINITY, 0x7fffffff}
                                   : RoutePick{route_key16_logit(mine0, dtype), (int)(0xffffu - (mine0 & 0xffffu))};
  const RoutePick r1 = mine1 == 0u ? RoutePick{-INFINITY, 0x7fffffff}
                                   : RoutePick{route_key16_logit(mine1, dtype), (int)(0xffffu - (mine1 & 0xffffu))};
  float mx0, sum0, mx1, sum1;
  route_softmax<PER>(raw0, dtype, E, mx0, sum0);
  route_softmax<PER>(raw1, dtype, E, mx1, sum1);
  const float w0 = route_weight(r0, mx0, sum0, top_k, renorm);
  const float w1 = route_weight(r1, mx1, sum1, top_k, renorm);
  if (lane < top_k) {
    tw[t0 * top_k + lane] = w0;
    ids[t0 * top_k + lane] = r0.myid;
    tw[t1 * top_k + lane] = w1;
    ids[t1 * top_k + lane] = r1.myid;
    if (ids_s) {
      ids_s[t0 * top_k + lane] = r0.myid;
      ids_s[t1 * top_k + lane] = r1.myid;
    }
  }
}

}  // namespace w4a8

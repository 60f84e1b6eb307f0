// Argument block shared by the dense and grouped (MoE) W4A8 GEMM kernels.
#pragma once
#include "w4a8_common.h"

namespace w4a8 {

// most experts the routed decode GEMV's in-kernel router covers (four per lane of a wave)
constexpr int kRouteMaxExperts = 256;

struct GemmArgs {
  // activations: fp8 rows (row stride ldx bytes) + per-row f32 scale
  const uint8_t* xq;
  int64_t ldx;
  const float* act_scales;
  // bf16/fp16 activations for the decode GEMV's fused quant prologue (null otherwise)
  const uint16_t* xsrc;
  int64_t ldxs;       // elements
  int xdtype;
  int64_t M;          // dense: rows of x/out. grouped: padded row capacity P
  // weights
  int64_t N;          // output channels of the weight (2*inter for the fused-silu arms)
  int64_t K;
  int64_t KT;         // tiles along K = ceil(K/128)
  const uint4* wt;    // W4 tiles
  const void* scales; // (K/g, N) group-major, fp16 or E8M0 uint8
  int sfmt;
  const int32_t* zeros;  // (K/g, N/8) packed or null (symmetric, zero = 8)
  int group;
  int wfmt;
  // grouped rows (null sorted_ids => dense)
  const int32_t* sorted_ids;
  const int32_t* expert_ids;
  const int32_t* ntp;
  int top_k;
  int64_t num_slots;  // T * top_k; sorted ids >= this are padding
  int bm;             // align block size
  int a_by_token;     // 1: A row = token = slot / top_k (gemm1); 0: A row = padded position (gemm2)
  int64_t w_expert_tiles;  // tiles per expert
  int64_t s_expert_stride; // scale elements per expert
  int64_t z_expert_stride; // zero words per expert
  // routed decode GEMV (kARoute): router logits (T, num_experts) and the route it writes, per slot
  // the weight, expert and padded row, per 16-row block the sorted ids and the owner, and ntp
  const void* logits;
  int ldtype;
  int num_experts;
  int renorm;
  float* tw_out;
  int32_t* ids_out;
  int32_t* inv_out;
  int32_t* sorted_out;
  int32_t* eid_out;
  int32_t* ntp_out;
  // output
  void* out;
  int out_dtype;
  int64_t ldo;        // elements
  int silu;           // 1: out[:, j] = silu(y[:, j]) * y[:, j + N/2]
  // 1: rows 2m and 2m+1 are the two fp8 terms of bf16 activation row m (W4A16): out row m is
  // bf16((0 + y[2m]) + y[2m+1]), silu applied to those sums (prefill DMA kernel only)
  int tsum2;
  // 1 (dense prefill DMA kernel): xq holds the fp8 codes in MFMA operand order (act_quant_tiled_kernel, act_tile_kernel:
  // per 16-row block and K tile one 2 KiB block, the block at ((row/16) * KT + kt) * 2048), and for
  // symmetric int4 seeds[kt * seeds_ld + row] holds the row-sum seed MFMA's result for that block
  int a_tiled;
  const float* seeds;
  int64_t seeds_ld;
  // split-K
  float* partial;     // (SK, M, N) f32 when SK > 1
  int SK;
  int64_t kps;        // tiles per split
};

}  // namespace w4a8

// Large-M W4A8 GEMM (prefill band) on the 16x16x128 f8f6f4 MFMA.
//
// Restates the math of the reference's wmma_tiled_tuned arm of mmq_fp8_gemm
// (python/minisgl/quant/kernels.py:1632, 1686-1734) and of the grouped MoE GEMMs
// (kernels.py:744-773, 851-874): y[m,n] = s_m * sum_g scale[g,n] * sum_{k in g} e4m3(x[m,k]) w(n,k),
// f32 accumulation, output in the activation dtype (or f32 for the MoE down projection).
//
// Tiling: a workgroup of WM x WN waves owns BM = WM*RB*16 rows and BN = WN*NSB*16 channels; a
// wave owns RB 16-row blocks x NSB 16-channel strips and walks all K tiles. Per K tile a wave
// loads its A fragments (two 16-byte reads per row block) and one 1 KB weight tile per strip,
// unpacks int4 tiles to fp8 once per strip and reuses them across its RB row blocks.
//   * int4, group 128, symmetric: the -0.5 code shift is folded into the MFMA accumulator seed
//     (an MFMA of the A fragment against a constant -0.5 operand), so each group costs one FMA per
//     output element: acc += scale * MFMA(A, B, -R/2).
//   * int4 otherwise (zero points, groups of 32/64): row sums R from an MFMA against +0.5, then
//     acc += scale * (C + (15 - 2z) * R/2); narrower groups mask the other K blocks out through
//     the MFMA's per-block B scale.
//   * e2m1 with E8M0 scales: the checkpoint's block exponents feed the scaled MFMA directly.
// For the grouped form every workgroup's rows lie inside one align block (bm % BM == 0), so one
// expert's tiles serve the whole workgroup.
#include "gemm_args.h"

namespace w4a8 {

__device__ __forceinline__ bool prow_source(const GemmArgs& p, int64_t r, int64_t& ar) {
  if (!p.sorted_ids) {
    ar = r;
    return r < p.M;
  }
  if (r >= p.M || r >= (int64_t)(*p.ntp)) return false;
  const int64_t slot = p.sorted_ids[r];
  if (slot >= p.num_slots) return false;
  ar = p.a_by_token ? (int64_t)((uint32_t)slot / (uint32_t)p.top_k) : r;  // slots < 2^31
  return true;
}

__device__ __forceinline__ float psilu_mul(float gate, float up, int dt) {
  const float g = from_dtype(to_dtype(gate, dt), dt);
  const float u = from_dtype(to_dtype(up, dt), dt);
  const float den = 1.0f + expf(-g);
  const float sg = g / den;
  const float sh = from_dtype(to_dtype(sg, dt), dt);
  return sh * u;
}

__device__ __forceinline__ void pstore(const GemmArgs& p, int64_t row, int64_t col, float v) {
  if (p.out_dtype == kF32)
    reinterpret_cast<float*>(p.out)[row * p.ldo + col] = v;
  else
    reinterpret_cast<uint16_t*>(p.out)[row * p.ldo + col] = to_dtype(v, p.out_dtype);
}

// MODE: 0 = int4 sym g128 fast, 1 = int4 general, 2 = e2m1 + E8M0, 3 = e2m1 + fp16 scales
template <int WM, int WN, int RB, int NSB, int MODE>
__global__ void __launch_bounds__(WM * WN * 64) gemm_prefill_kernel(const GemmArgs p) {
  constexpr int BM = WM * RB * 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t blk_row0 = (int64_t)blockIdx.y * BM;
  const int64_t row0 = blk_row0 + (int64_t)wm * RB * 16;

  int64_t expert = 0;
  if (p.sorted_ids) {
    if (blk_row0 >= (int64_t)(*p.ntp)) return;
    expert = p.expert_ids[(uint32_t)blk_row0 / (uint32_t)p.bm];  // padded rows < 2^31
  }

  const uint8_t* arow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    int64_t ar;
    arow[rb] = prow_source(p, row0 + rb * 16 + (lane & 15), ar) ? p.xq + ar * p.ldx : nullptr;
  }

  const int64_t nstrips = p.N / kTileN;
  constexpr int HALF = NSB / 2;
  int64_t strip[NSB];
  bool sval[NSB];
#pragma unroll
  for (int j = 0; j < NSB; ++j) {
    if (p.silu) {
      const int64_t gs = ((int64_t)blockIdx.x * WN + wn) * HALF + (j < HALF ? j : j - HALF);
      sval[j] = gs < nstrips / 2;
      strip[j] = j < HALF ? gs : nstrips / 2 + gs;
    } else {
      strip[j] = ((int64_t)blockIdx.x * WN + wn) * NSB + j;
      sval[j] = strip[j] < nstrips;
    }
  }

  const uint4* wt = p.wt + (size_t)(expert * p.w_expert_tiles) * 64;
  const size_t esz = p.sfmt == kScaleF16 ? 2 : 1;
  const void* scales = reinterpret_cast<const char*>(p.scales) + (size_t)(expert * p.s_expert_stride) * esz;
  const int32_t* zeros = p.zeros ? p.zeros + expert * p.z_expert_stride : nullptr;
  const int64_t N = p.N, K = p.K, KT = p.KT;
  const int group = p.group;
  const int gpt = group >= kTileK ? 1 : kTileK / group;

  v4f acc[RB][NSB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < NSB; ++j) acc[rb][j] = v4f{0.f, 0.f, 0.f, 0.f};

  const v4f zero4 = v4f{0.f, 0.f, 0.f, 0.f};
  for (int64_t kt = 0; kt < KT; ++kt) {
    const int64_t kbase = kt * kTileK;
    const int kvalid = (int)(K - kbase < kTileK ? K - kbase : kTileK);
    v8i a[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) a[rb] = load_a_operand(arow[rb] ? arow[rb] + kbase : nullptr, kvalid, lane);
    uint4 raw[NSB];
#pragma unroll
    for (int j = 0; j < NSB; ++j)
      raw[j] = sval[j] ? wt[(size_t)(strip[j] * KT + kt) * 64 + lane] : make_uint4(0, 0, 0, 0);

    if (MODE == 2) {
      const int64_t blk = kt * 4 + (lane >> 4);
      const bool bin = blk * 32 < K;
#pragma unroll
      for (int j = 0; j < NSB; ++j) {
        const int64_t n = strip[j] * kTileN + (lane & 15);
        const int sb = (bin && sval[j]) ? (int)reinterpret_cast<const uint8_t*>(scales)[blk * N + n] : 127;
        const v8i b = fp4_operand(raw[j]);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb][j] = mfma_f8f4_sb(a[rb], b, acc[rb][j], sb);
      }
    } else if (MODE == 0) {
      const v8i nhalf8 = splat8(0xB0B0B0B0u);  // -0.5 in every byte
      v4f seed[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) seed[rb] = mfma_f8f8(a[rb], nhalf8, zero4);
      const int64_t g = kbase / group;
#pragma unroll
      for (int j = 0; j < NSB; ++j) {
        const int64_t n = strip[j] * kTileN + (lane & 15);
        const v8i b = unpack_tile_int4(raw[j]);
        const float sc = sval[j] ? load_scale(scales, kScaleF16, g * N + n) : 0.f;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const v4f c = mfma_f8f8(a[rb], b, seed[rb]);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[rb][j][r] += sc * c[r];
        }
      }
    } else {
      const v8i half8 = splat8(kE4M3Half4);
      // the tile's group scales, all loads issued before the first MFMA (each sub-group's MFMAs
      // would otherwise wait on their own dependent load)
      constexpr int SMAX = MODE == 3 ? 8 : 4;
      float scv[SMAX][NSB];
#pragma unroll
      for (int ss = 0; ss < SMAX; ++ss) {
        const bool in = ss < gpt && kbase + (int64_t)ss * (kTileK / gpt) < K;
        const int64_t g = in ? (kbase + (int64_t)ss * (kTileK / gpt)) / group : 0;
#pragma unroll
        for (int j = 0; j < NSB; ++j) {
          const int64_t n = strip[j] * kTileN + (lane & 15);
          scv[ss][j] = (in && sval[j]) ? group_scale(scales, p.sfmt, g * N + n, zeros, n) : 0.f;
        }
      }
#pragma unroll
      for (int ss = 0; ss < SMAX; ++ss) {
        if (ss >= gpt || kbase + (int64_t)ss * (kTileK / gpt) >= K) break;
        const int msk = gpt == 1 ? 127 : subgroup_mask_scale(lane, gpt, ss);
        const int64_t g = (kbase + (int64_t)ss * (kTileK / gpt)) / group;
        v4f rh[RB];
        if (MODE == 1) {
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) rh[rb] = mfma_f8f8_sb(a[rb], half8, zero4, msk);
        }
#pragma unroll
        for (int j = 0; j < NSB; ++j) {
          const int64_t n = strip[j] * kTileN + (lane & 15);
          v8i b = MODE == 1 ? unpack_tile_int4(raw[j]) : fp4_operand(raw[j]);
          if (MODE == 3 && gpt == 8) b = fp4_half_operand(b, ss);
          const float sc = scv[ss][j];
          float coef = -1.0f;
          if (MODE == 1 && zeros && sval[j]) {
            const uint32_t zw = (uint32_t)zeros[g * (N / 8) + n / 8];
            coef = 15.0f - 2.0f * (float)((zw >> (4 * (n & 7))) & 15u);
          }
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) {
            const v4f c = MODE == 1 ? mfma_f8f8_sb(a[rb], b, zero4, msk) : mfma_f8f4_sb(a[rb], b, zero4, msk);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float t = MODE == 1 ? c[r] + coef * rh[rb][r] : c[r];
              acc[rb][j][r] += sc * t;
            }
          }
        }
      }
    }
  }

  // epilogue: lane holds rows 4*(lane>>4)+r of each row block, channel strip*16 + (lane & 15)
  const int jn = p.silu ? HALF : NSB;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = row0 + rb * 16 + 4 * (lane >> 4) + r;
      int64_t ar;
      if (!prow_source(p, row, ar)) continue;
      const float s = p.act_scales[ar];
#pragma unroll
      for (int j = 0; j < NSB; ++j) {
        if (j >= jn || !sval[j]) continue;
        const int64_t col = strip[j] * kTileN + (lane & 15);
        if (p.silu)
          pstore(p, row, col, psilu_mul(acc[rb][j][r] * s, acc[rb][j + HALF][r] * s, p.out_dtype));
        else
          pstore(p, row, col, acc[rb][j][r] * s);
      }
    }
  }
}

template <int WM, int WN, int RB, int NSB>
static int launch_prefill_cfg(const GemmArgs& p, int64_t row_tiles, hipStream_t stream) {
  constexpr int BN = WN * NSB * 16;
  const int64_t ncols = p.silu ? p.N / 2 : p.N;
  const int64_t colw = p.silu ? BN / 2 : BN;
  dim3 grid((unsigned)((ncols + colw - 1) / colw), (unsigned)row_tiles);
  dim3 block(WM * WN * 64);
  int mode;
  if (p.wfmt == kInt4)
    mode = (p.zeros == nullptr && p.group % kTileK == 0 && p.sfmt == kScaleF16) ? 0 : 1;
  else
    mode = p.sfmt == kScaleE8M0 ? 2 : 3;
  switch (mode) {
    case 0: hipLaunchKernelGGL((gemm_prefill_kernel<WM, WN, RB, NSB, 0>), grid, block, 0, stream, p); break;
    case 1: hipLaunchKernelGGL((gemm_prefill_kernel<WM, WN, RB, NSB, 1>), grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL((gemm_prefill_kernel<WM, WN, RB, NSB, 2>), grid, block, 0, stream, p); break;
    default: hipLaunchKernelGGL((gemm_prefill_kernel<WM, WN, RB, NSB, 3>), grid, block, 0, stream, p); break;
  }
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

// bm_rows: rows per workgroup required by the caller (grouped: must divide the align block).
int launch_prefill(const GemmArgs& p, int64_t rows_to_cover, int bm_rows, hipStream_t stream) {
  if (bm_rows == 64) {
    const int64_t tiles = (rows_to_cover + 63) / 64;
    return launch_prefill_cfg<1, 4, 4, 4>(p, tiles, stream);
  }
  const int64_t tiles = (rows_to_cover + 127) / 128;
  return launch_prefill_cfg<2, 2, 4, 4>(p, tiles, stream);
}

}  // namespace w4a8

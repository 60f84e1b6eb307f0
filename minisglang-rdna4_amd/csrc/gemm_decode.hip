// Skinny-M W4A8 GEMM (decode band, up to 16 rows per row block) on the 16x16x128 f8f6f4 MFMA.
//
// Restates the math of the reference's decode_gemv arm of mmq_fp8_gemm
// (python/minisgl/quant/kernels.py:1562-1563, 1686-1734) and of its fused gate_up+silu twin
// mmq_fp8_gemm_silu (kernels.py:1737-1753; epilogue tools/w4a8_gemm_silu_parity.py:52-54):
//   y[m,n] = s_m * sum_g scale[g,n] * sum_{k in g} e4m3(x[m,k]) * w(n,k)
// with f32 accumulation. The grouped (MoE) form follows mmq_fp8_moe_gemm / _gemm1_silu
// (kernels.py:744-773): rows are padded positions of the align, A rows are gathered by slot.
//
// Work split: blockIdx.x = group of 16-channel strips, blockIdx.y = K split, blockIdx.z = block of
// 16 rows. The waves of a workgroup take the K tiles of their split round-robin; each tile is one
// coalesced 1 KB weight load per strip and one MFMA per strip (plus one MFMA against a constant
// 0.5 operand that yields the row sums the int4 code shift needs). Waves reduce through LDS; K
// splits, if any, go through an f32 workspace and a second kernel. Both reductions run in a fixed
// order, so results do not depend on timing.
#include "gemm_args.h"

namespace w4a8 {

__device__ __forceinline__ bool row_source(const GemmArgs& p, int64_t r, int64_t& ar) {
  if (!p.sorted_ids) {
    ar = r;
    return r < p.M;
  }
  if (r >= p.M || r >= (int64_t)(*p.ntp)) return false;
  const int64_t slot = p.sorted_ids[r];
  if (slot >= p.num_slots) return false;
  ar = p.a_by_token ? slot / p.top_k : r;
  return true;
}

__device__ __forceinline__ const void* expert_scales(const GemmArgs& p, int64_t e) {
  const size_t esz = p.sfmt == kScaleF16 ? 2 : 1;
  return reinterpret_cast<const char*>(p.scales) + (size_t)(e * p.s_expert_stride) * esz;
}

__device__ __forceinline__ float silu_mul(float gate, float up, int dt) {
  // tools/w4a8_gemm_silu_parity.py:52-54: round to dtype, silu in f32, round, multiply in dtype.
  const float g = from_dtype(to_dtype(gate, dt), dt);
  const float u = from_dtype(to_dtype(up, dt), dt);
  const float den = 1.0f + expf(-g);
  const float sg = g / den;
  const float sh = from_dtype(to_dtype(sg, dt), dt);
  return sh * u;
}

__device__ __forceinline__ void store_out(const GemmArgs& p, int64_t row, int64_t col, float v) {
  if (p.out_dtype == kF32) {
    reinterpret_cast<float*>(p.out)[row * p.ldo + col] = v;
  } else {
    reinterpret_cast<uint16_t*>(p.out)[row * p.ldo + col] = to_dtype(v, p.out_dtype);
  }
}

// Final value for (row, col) of the output (col < N, or < N/2 for silu) from unscaled totals.
__device__ __forceinline__ void finish(const GemmArgs& p, int64_t row, int64_t col, float tot,
                                       float tot_up) {
  int64_t ar;
  if (!row_source(p, row, ar)) return;
  const float s = p.act_scales[ar];
  if (p.silu) {
    store_out(p, row, col, silu_mul(tot * s, tot_up * s, p.out_dtype));
  } else {
    store_out(p, row, col, tot * s);
  }
}

// Strip j of workgroup sg; for the fused-silu arm strips [0, half) are gate, [half, 2*half) up.
__device__ __forceinline__ bool strip_of(int silu, int64_t sg, int j, int half, int nstr,
                                         int64_t nstrips, int64_t& strip) {
  if (silu) {
    const int64_t gs = sg * half + (j < half ? j : j - half);
    strip = j < half ? gs : nstrips / 2 + gs;
    return gs < nstrips / 2;
  }
  strip = sg * nstr + j;
  return strip < nstrips;
}

template <int NSTR, int WFMT>
__global__ void __launch_bounds__(512) gemv_kernel(const GemmArgs p) {
  extern __shared__ float red[];  // [W][NSTR][4][64]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
  const int64_t sg = blockIdx.x;
  const int ks = blockIdx.y;
  const int64_t m0 = (int64_t)blockIdx.z * 16;

  int64_t expert = 0;
  if (p.sorted_ids) {
    if (m0 >= (int64_t)(*p.ntp)) return;
    expert = p.expert_ids[m0 / p.bm];
  }
  int64_t ar;
  const uint8_t* arow = row_source(p, m0 + (lane & 15), ar) ? p.xq + ar * p.ldx : nullptr;

  const int64_t nstrips = p.N / kTileN;
  const int half = p.silu ? NSTR / 2 : NSTR;
  int64_t strip[NSTR];
  bool sval[NSTR];
#pragma unroll
  for (int j = 0; j < NSTR; ++j) sval[j] = strip_of(p.silu, sg, j, half, NSTR, nstrips, strip[j]);

  const uint4* wt = p.wt + (size_t)(expert * p.w_expert_tiles) * 64;
  const void* scales = expert_scales(p, expert);
  const int32_t* zeros = p.zeros ? p.zeros + expert * p.z_expert_stride : nullptr;
  const int64_t N = p.N, K = p.K, KT = p.KT;
  const int group = p.group;
  const int gpt = group >= kTileK ? 1 : kTileK / group;

  v4f acc[NSTR];
#pragma unroll
  for (int j = 0; j < NSTR; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};

  const v8i half8 = splat8(kE4M3Half4);
  const int64_t kt_begin = (int64_t)ks * p.kps;
  const int64_t kt_end = kt_begin + p.kps < KT ? kt_begin + p.kps : KT;
  const bool e8m0_fast = (WFMT == kE2M1) && p.sfmt == kScaleE8M0;

  for (int64_t kt = kt_begin + wave; kt < kt_end; kt += W) {
    const int64_t kbase = kt * kTileK;
    const int kvalid = (int)(K - kbase < kTileK ? K - kbase : kTileK);
    const v8i a = load_a_operand(arow ? arow + kbase : nullptr, kvalid, lane);
    uint4 raw[NSTR];
#pragma unroll
    for (int j = 0; j < NSTR; ++j)
      raw[j] = sval[j] ? wt[(size_t)(strip[j] * KT + kt) * 64 + lane] : make_uint4(0, 0, 0, 0);

    if (e8m0_fast) {
      // MXFP4: E8M0 block scales go straight into the MFMA; no per-group VALU work.
      const int64_t blk = kt * 4 + (lane >> 4);
      const bool bin = blk * 32 < K;
#pragma unroll
      for (int j = 0; j < NSTR; ++j) {
        const int64_t n = strip[j] * kTileN + (lane & 15);
        const int sb = (bin && sval[j]) ? (int)reinterpret_cast<const uint8_t*>(scales)[blk * N + n] : 127;
        acc[j] = mfma_f8f4_sb(a, fp4_operand(raw[j]), acc[j], sb);
      }
      continue;
    }

    v4f rh[4];
    if (WFMT == kInt4) {
#pragma unroll
      for (int ss = 0; ss < 4; ++ss) {
        if (ss >= gpt) break;
        rh[ss] = gpt == 1 ? mfma_f8f8(a, half8, v4f{0.f, 0.f, 0.f, 0.f})
                          : mfma_f8f8_sb(a, half8, v4f{0.f, 0.f, 0.f, 0.f},
                                         subgroup_mask_scale(lane, gpt, ss));
      }
    }
#pragma unroll
    for (int j = 0; j < NSTR; ++j) {
      if (!sval[j]) continue;
      const int64_t n = strip[j] * kTileN + (lane & 15);
      const v8i b = WFMT == kInt4 ? unpack_tile_int4(raw[j]) : fp4_operand(raw[j]);
#pragma unroll
      for (int ss = 0; ss < 4; ++ss) {
        if (ss >= gpt || kbase + (int64_t)ss * (kTileK / gpt) >= K) break;
        const int msk = gpt == 1 ? 127 : subgroup_mask_scale(lane, gpt, ss);
        v4f c = v4f{0.f, 0.f, 0.f, 0.f};
        c = WFMT == kInt4 ? mfma_f8f8_sb(a, b, c, msk) : mfma_f8f4_sb(a, b, c, msk);
        const int64_t g = (kbase + (int64_t)ss * (kTileK / gpt)) / group;
        const float sc = load_scale(scales, p.sfmt, g * N + n);
        if (WFMT == kInt4) {
          float coef = -1.0f;
          if (zeros) {
            const uint32_t zw = (uint32_t)zeros[g * (N / 8) + n / 8];
            coef = 15.0f - 2.0f * (float)((zw >> (4 * (n & 7))) & 15u);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[j][r] += sc * (c[r] + coef * rh[ss][r]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[j][r] += sc * c[r];
        }
      }
    }
  }

#pragma unroll
  for (int j = 0; j < NSTR; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[((wave * NSTR + j) * 4 + r) * 64 + lane] = acc[j][r];
  __syncthreads();

  const int nent = half * 4 * 64;
  for (int e = threadIdx.x; e < nent; e += blockDim.x) {
    const int j = e >> 8, r = (e >> 6) & 3, l = e & 63;
    int64_t sj;
    if (!strip_of(p.silu, sg, j, half, NSTR, nstrips, sj)) continue;
    float tot = 0.f, tot_up = 0.f;
    for (int w = 0; w < W; ++w) {
      tot += red[((w * NSTR + j) * 4 + r) * 64 + l];
      if (p.silu) tot_up += red[((w * NSTR + j + half) * 4 + r) * 64 + l];
    }
    const int64_t row = m0 + 4 * (l >> 4) + r;
    const int64_t col = sj * kTileN + (l & 15);
    if (p.SK == 1) {
      finish(p, row, col, tot, tot_up);
    } else {
      if (row < p.M) {
        float* part = p.partial + ((size_t)ks * p.M + row) * N;
        part[col] = tot;
        if (p.silu) part[col + N / 2] = tot_up;
      }
    }
  }
}

__global__ void splitk_reduce_kernel(const GemmArgs p, int64_t nout) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.M * nout) return;
  const int64_t row = idx / nout, col = idx % nout;
  int64_t ar;
  if (!row_source(p, row, ar)) return;
  float tot = 0.f, tot_up = 0.f;
  for (int s = 0; s < p.SK; ++s) {
    const float* part = p.partial + ((size_t)s * p.M + row) * p.N;
    tot += part[col];
    if (p.silu) tot_up += part[col + p.N / 2];
  }
  finish(p, row, col, tot, tot_up);
}

// Split/shape policy. Depends only on (rows, N, K) so the fused-silu arm and the plain arm run
// the same per-channel arithmetic (same K split, same wave assignment) and agree bit-for-bit.
struct GemvPlan {
  int nstr;   // strips per workgroup (plain arm)
  int waves;
  int sk;
  int64_t kps;
};

GemvPlan plan_gemv(int64_t rows, int64_t N, int64_t K, int64_t row_blocks) {
  GemvPlan pl;
  pl.nstr = rows <= 2 ? 1 : (rows <= 8 ? 2 : 4);
  pl.waves = 4;
  const int64_t KT = (K + kTileK - 1) / kTileK;
  const int64_t nstrips = N / kTileN;
  const int64_t sg = (nstrips + pl.nstr - 1) / pl.nstr;
  int sk = 1;
  const int64_t target = 1024;
  while (sg * row_blocks * sk < target && (KT + 2 * sk - 1) / (2 * sk) >= pl.waves) sk *= 2;
  pl.sk = sk;
  pl.kps = (KT + sk - 1) / sk;
  return pl;
}

template <int NSTR, int WFMT>
static void launch_gemv_t(const GemmArgs& p, dim3 grid, int waves, hipStream_t stream) {
  const size_t lds = (size_t)waves * NSTR * 4 * 64 * sizeof(float);
  hipLaunchKernelGGL((gemv_kernel<NSTR, WFMT>), grid, dim3(waves * 64), lds, stream, p);
}

// row_blocks: number of 16-row blocks to launch (dense: ceil(M/16); grouped: a bound on the
// padded rows that can hold data).
int launch_gemv(GemmArgs p, int64_t row_blocks, hipStream_t stream) {
  const GemvPlan pl = plan_gemv(p.sorted_ids ? 16 : p.M, p.N, p.K, row_blocks);
  p.SK = pl.sk;
  p.kps = pl.kps;
  const int nstr = p.silu ? 2 * pl.nstr : pl.nstr;
  const int64_t nstrips = p.N / kTileN;
  const int64_t per = p.silu ? pl.nstr : pl.nstr;
  const int64_t sg = ((p.silu ? nstrips / 2 : nstrips) + per - 1) / per;
  if (p.SK > 1 && p.partial == nullptr) return kErrInvalid;
  dim3 grid((unsigned)sg, (unsigned)pl.sk, (unsigned)row_blocks);
  const bool i4 = p.wfmt == kInt4;
  switch (nstr) {
    case 1: i4 ? launch_gemv_t<1, kInt4>(p, grid, pl.waves, stream) : launch_gemv_t<1, kE2M1>(p, grid, pl.waves, stream); break;
    case 2: i4 ? launch_gemv_t<2, kInt4>(p, grid, pl.waves, stream) : launch_gemv_t<2, kE2M1>(p, grid, pl.waves, stream); break;
    case 4: i4 ? launch_gemv_t<4, kInt4>(p, grid, pl.waves, stream) : launch_gemv_t<4, kE2M1>(p, grid, pl.waves, stream); break;
    case 8: i4 ? launch_gemv_t<8, kInt4>(p, grid, pl.waves, stream) : launch_gemv_t<8, kE2M1>(p, grid, pl.waves, stream); break;
    default: return kErrInvalid;
  }
  if (hipGetLastError() != hipSuccess) return kErrHip;
  if (p.SK > 1) {
    const int64_t nout = p.silu ? p.N / 2 : p.N;
    const int64_t total = p.M * nout;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       stream, p, nout);
    if (hipGetLastError() != hipSuccess) return kErrHip;
  }
  return kOk;
}

size_t gemv_workspace_bytes(int64_t M, int64_t N, int64_t K, int grouped, int64_t row_blocks) {
  const GemvPlan pl = plan_gemv(grouped ? 16 : M, N, K, row_blocks);
  return pl.sk > 1 ? (size_t)pl.sk * (size_t)M * (size_t)N * sizeof(float) : 0;
}

}  // namespace w4a8

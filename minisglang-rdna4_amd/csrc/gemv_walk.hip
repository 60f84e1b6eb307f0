// Strip-walking decode GEMV: a decode call of up to 16 bf16/fp16 rows in one launch.
//
// Each workgroup quantizes every row of the call per token into LDS once (the act-quant kernel's
// arithmetic, bit for bit), then walks a contiguous range of strip groups; the grid is sized to
// about one workgroup per CU. The row phase is paid once per CU instead of once per strip group,
// and one rolling window of weight loads runs across the whole range, so a wave's loads never
// drain between strips.
//
// Arithmetic: the K split (waves, tiles per wave) is the one-row plan of the weight (gemm_decode.hip
// plan_gemv), each wave accumulates its K tiles in order with the same per-tile MFMA and FMA steps
// as gemv_kernel, and the waves' partial sums of a strip are added in wave order. A row's output
// bits are therefore those of gemv_kernel's one-row call, whatever the other rows of the call
// (reference: the decode_gemv arm of mmq_fp8_gemm / mmq_fp8_gemm_silu,
// python/minisgl/quant/kernels.py:1562-1563, 1686-1753, and its M-invariance record
// _qminv_dense.txt:30-33).
#include "gemv.h"

namespace w4a8 {

// Thread mapping of the row phase: rows padded to a power of two, 2^tpr_log threads per row, thread t
// on row t >> tpr_log, reading its row's 16-byte chunks j0 + i * tpr (SM of them). Per-row maxima:
// each thread's chunks as packed 16-bit magnitudes, a 16-lane DPP reduction, then the row's 16-lane
// groups through LDS. DT: the activation dtype (kBF16 / kF16).
//
// Walk: the first sets * kw waves form `sets` sets of kw waves (kw: the plan's K-split waves); set s
// takes the workgroup's strip groups s, s + sets, ...; wave w of a set owns K tiles [w * tpw, (w + 1) * tpw)
// of each and keeps CH tiles of weight loads in flight across its groups.
//   NS: strips per group (plain arm 1; fused silu 2: a gate strip and its up strip).
template <int NS, int CH, int MODE, bool SYM, int SM, int DT>
__global__ void __launch_bounds__(512) gemv_walk_kernel(const GemmArgs p, const WalkArgs wa) {
  static_assert(MODE == kModeI4 || MODE == kModeE8M0 || MODE == kModeNV, "int4 (groups of 128+), MXFP4, NVFP4");
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float amax16[32];  // maxima of the 16-lane groups (8 waves x 4)
  __shared__ float srow[16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kw = wa.kw, tpw = wa.tpw, tpr_log = wa.tpr_log;
  const int M = (int)p.M, K = (int)p.K;

  // ---- row loads first, before any other work: rows past M and chunks past K read zeros (out of
  // the descriptor's range). Row stride ldxs is a multiple of 8 elements, so 32-bit offsets hold
  // rows of up to 2^31 bytes in all.
  const int tpr = 1 << tpr_log;
  const int r = tid >> tpr_log, j0 = tid & (tpr - 1);
  const bool rin = r < M;
  const uint32_t ldb = (uint32_t)p.ldxs * 2u;
  const uint32_t xbytes = (uint32_t)(M - 1) * ldb + (uint32_t)K * 2u;
  const BufRsrc rs_x = make_rsrc(p.xsrc, xbytes);
  uint4 stg[SM];
#pragma unroll
  for (int i = 0; i < SM; ++i) {
    const int j = j0 + i * tpr;
    const bool ok = rin && j * 8 < K;
    stg[i] = bload128(rs_x, ok ? (uint32_t)r * ldb + (uint32_t)j * 16u : xbytes, 0u);
  }

  // sets of kw waves (1 or 2): wave w is wave wk of set w >= kw; waves past the sets (a plan of 5-7
  // waves in an 8-wave workgroup) only help with the row phase
  const int set = (wa.sets == 2 && wave >= kw) ? 1 : 0, wk = wave - set * kw, sets = wa.sets;
  const bool walker = wave < sets * kw;
  const int N = (int)p.N, KT = (int)p.KT;
  const int nstrips = N / kTileN;
  const int half = p.silu ? NS / 2 : NS;
  // this workgroup's strip groups [g0, g0 + ng): base + 1 groups for the first `extra` workgroups,
  // base for the rest; consecutive workgroups of one XCD get consecutive ranges, so strips that
  // share scale lines meet in one L2
  const int b = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int ng = wa.gbase + (b < wa.gextra ? 1 : 0);
  const int g0 = b * wa.gbase + (b < wa.gextra ? b : wa.gextra);

  // ---- weight window, issued behind the row loads
  const int kb = wk * tpw;
  const int ke = kb + tpw < KT ? kb + tpw : KT;
  const int nt = ke - kb;  // >= 1: the plan gives every wave at least one tile
  const int ngs = !walker ? 0 : sets == 2 ? (ng - set + 1) >> 1 : ng;  // this set's groups
  const int nitems = ngs * nt;
  constexpr int kEsz = MODE == kModeI4 ? 2 : 1;
  const int ngr = K >> (31 - __builtin_clz((unsigned)p.group));
  const int gshift = 31 - __builtin_clz((unsigned)(p.group >= kTileK ? p.group / kTileK : 1));
  const BufRsrc rs_w = make_rsrc(p.wt, (uint32_t)(nstrips * KT * kTileBytes));
  const BufRsrc rs_s = make_rsrc(p.scales, (uint32_t)(ngr * N * kEsz));
  const BufRsrc rs_z = make_rsrc(p.zeros, p.zeros ? (uint32_t)(ngr * (N / 8) * 4) : 0u);
  uint4 raw[CH][NS];
  typedef unsigned short v2h __attribute__((ext_vector_type(2)));
  v2h sc[(CH + 1) / 2][NS];
  uint32_t zw[SYM ? 1 : CH][NS];
  int sb[MODE == kModeE8M0 ? CH : 1][NS];
  // NVFP4: the 8 group-16 scale bytes of a tile, two per register (d16 loads into the halves)
  typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
  v2u16 nvs[MODE == kModeNV ? CH : 1][NS][4];
  // item (g, t): K tile kb + t of strip group g0 + g; past the last item the last one is loaded
  // again (a cache hit that keeps the loads unconditional)
  auto load_item = [&](int s, int g, int t) {
    if (g >= ngs) {
      g = ngs > 0 ? ngs - 1 : 0;
      t = nt - 1;
    }
    g = set + g * sets;
    if (g >= ng) g = ng - 1;  // a set with no group: any valid address
    const int kt = kb + t;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      int64_t st;
      strip_of(p.silu, g0 + g, j, half, NS, nstrips, st);
      const int stc = (int)(st < nstrips ? st : nstrips - 1);
      raw[s][j] = bload128_nt(rs_w, (uint32_t)lane * 16, (uint32_t)((stc * KT + kt) * kTileBytes));
      const int n = stc * kTileN + (lane & 15);
      if (MODE == kModeI4) {
        const int gi = kt >> gshift;
        sc[s >> 1][j][s & 1] = bload16(rs_s, (uint32_t)n * 2, (uint32_t)(gi * N * 2));
        if (!SYM) zw[s][j] = bload32(rs_z, (uint32_t)(n / 8) * 4, (uint32_t)(gi * (N / 8) * 4));
      } else if (MODE == kModeE8M0) {
        sb[s][j] = (int)bload8(rs_s, (uint32_t)((lane >> 4) * N + n), (uint32_t)(kt * 4 * N));
      } else {
        // groups past K read as 0 from the descriptor's bound (a zero scale)
#pragma unroll
        for (int ss = 0; ss < 8; ++ss)
          nvs[MODE == kModeNV ? s : 0][j][ss >> 1][ss & 1] =
              (unsigned short)bload8(rs_s, (uint32_t)n, (uint32_t)((kt * 8 + ss) * N));
      }
    }
  };
  int lg = 0, lt = 0;  // next item to load
  auto adv = [&](int& g, int& t) {
    if (++t == nt) {
      t = 0;
      ++g;
    }
  };
#pragma unroll
  for (int s = 0; s < CH; ++s) {
    load_item(s, lg, lt);
    adv(lg, lt);
  }

  // ---- per-token quant of the rows into LDS (padded to whole tiles with zero codes)
  // |x| maxima as packed 16-bit magnitudes: for bf16 and fp16 the integer order of the magnitude bits
  // is the order of the finite values, +inf above them; a NaN sorts above +inf, and a thread that
  // holds one takes the f32 path instead, whose fmaxf skips NaNs as the act-quant kernel does
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  u16x2 m2 = {0, 0};
#pragma unroll
  for (int i = 0; i < SM; ++i) {
    const uint32_t w4[4] = {stg[i].x, stg[i].y, stg[i].z, stg[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, w4[e] & 0x7fff7fffu));
  }
  const uint32_t mbits = m2[0] > m2[1] ? m2[0] : m2[1];
  constexpr uint32_t kInfBits = DT == kBF16 ? 0x7f80u : 0x7c00u;
  float v = DT == kBF16 ? __uint_as_float(mbits << 16) : f16_to_f32((uint16_t)mbits);
  if (mbits > kInfBits) {
    v = 0.f;
#pragma unroll
    for (int i = 0; i < SM; ++i) v = fmaxf(v, amax8(stg[i], DT));
  }
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppRowMirror>(v));
  if ((lane & 15) == 0) amax16[tid >> 4] = v;
  lds_barrier();
  // the row's 16-lane groups [gb, gb + tpr / 16): all 32 entries read at once (8 independent
  // 16-byte reads), the others masked out
  float am = 0.f;
  {
    const int gb = (r * tpr) >> 4, ge = gb + (tpr >> 4);
    const float4* a4 = reinterpret_cast<const float4*>(amax16);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 t = a4[q];
      am = fmaxf(am, (4 * q + 0 >= gb && 4 * q + 0 < ge) ? t.x : 0.f);
      am = fmaxf(am, (4 * q + 1 >= gb && 4 * q + 1 < ge) ? t.y : 0.f);
      am = fmaxf(am, (4 * q + 2 >= gb && 4 * q + 2 < ge) ? t.z : 0.f);
      am = fmaxf(am, (4 * q + 3 >= gb && 4 * q + 3 < ge) ? t.w : 0.f);
    }
  }
  // the raw rows are unpacked again for the codes: the compiler would otherwise keep f32 values of
  // every chunk live across the barrier (8 VGPRs per chunk)
#pragma unroll
  for (int i = 0; i < SM; ++i) asm volatile("" : "+v"(stg[i].x), "+v"(stg[i].y), "+v"(stg[i].z), "+v"(stg[i].w));
  const float s_row = act_row_scale(am);
  const float inv = 1.0f / s_row;
  const int lstride = stage_stride(KT);
  const int cpr = KT * (kTileK / 8);
  unsigned char* a_lds = smem;
  if (rin) {
#pragma unroll
    for (int i = 0; i < SM; ++i) {
      const int j = j0 + i * tpr;
      if (j < cpr) {
        float f[8];
        unpack8(stg[i], DT, f);
        *reinterpret_cast<uint2*>(a_lds + r * lstride + j * 8) = quant8(f, inv);
      }
    }
    if (j0 == 0) srow[r] = s_row;
  }
  lds_barrier();

  // ---- the walk
  float* red = reinterpret_cast<float*>(smem + ((M * lstride + 15) / 16) * 16);  // [ngmax][kw][NS][M][16]
  const int lrow = (lane & 15) < M ? (lane & 15) : 0;
  const v4f zero4 = v4f{0.f, 0.f, 0.f, 0.f};
  v4f acc[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) acc[j] = zero4;
  auto compute = [&](int s, int t) {
    const unsigned char* src = a_lds + lrow * lstride + (kb + t) * kTileK + 16 * (lane >> 4);
    const uint4 lo = *reinterpret_cast<const uint4*>(src);
    const uint4 hi = *reinterpret_cast<const uint4*>(src + 64);
    v8i at;
    at[0] = (int)lo.x; at[1] = (int)lo.y; at[2] = (int)lo.z; at[3] = (int)lo.w;
    at[4] = (int)hi.x; at[5] = (int)hi.y; at[6] = (int)hi.z; at[7] = (int)hi.w;
    if (MODE == kModeE8M0) {
#pragma unroll
      for (int j = 0; j < NS; ++j) acc[j] = mfma_f8f4_sb(at, fp4_operand(raw[s][j]), acc[j], sb[s][j]);
    } else if (MODE == kModeNV) {
      // 16-wide groups: one MFMA per group on half of a lane's 32-element block (the other half
      // zeroed), only that block's scale open, then acc += e4m3(scale) * partial
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const v8i b = fp4_operand(raw[s][j]);
#pragma unroll
        for (int ss = 0; ss < 8; ++ss) {
          const v4f c = mfma_f8f4_sb(at, fp4_half_operand(b, ss), zero4, subgroup_mask_scale(lane, 8, ss));
          const v2u16 pr = nvs[MODE == kModeNV ? s : 0][j][ss >> 1];
          const float scf = __builtin_amdgcn_cvt_f32_fp8((int)(uint32_t)pr[ss & 1], 0);
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[j][q] = fmaf(scf, c[q], acc[j][q]);
        }
      }
    } else if (SYM) {
      const v4f seed = mfma_f8f8(at, splat8(0xB0B0B0B0u), zero4);  // -R/2
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const v4f c = mfma_f8f8(at, unpack_tile_int4(raw[s][j]), seed);
        const float scf = f16_to_f32(sc[s >> 1][j][s & 1]);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[j][q] = fmaf(scf, c[q], acc[j][q]);
      }
    } else {
      const v4f rh = mfma_f8f8(at, splat8(kE4M3Half4), zero4);
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const v4f c = mfma_f8f8(at, unpack_tile_int4(raw[s][j]), zero4);
        const float coef = 15.0f - 2.0f * (float)((zw[SYM ? 0 : s][j] >> (4 * (lane & 7))) & 15u);
        const float scf = f16_to_f32(sc[s >> 1][j][s & 1]);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[j][q] = fmaf(scf, fmaf(coef, rh[q], c[q]), acc[j][q]);
      }
    }
  };
  // a group's last tile: the wave's partial sums of the group go to LDS (rows < M only)
  auto flush = [&](int gs) {
    const int g = set + gs * sets, qq = lane >> 4, c = lane & 15;
#pragma unroll
    for (int j = 0; j < NS; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (4 * qq + q < M) red[(((g * kw + wk) * NS + j) * M + 4 * qq + q) * 16 + c] = acc[j][q];
      acc[j] = zero4;
    }
  };
  int cg = 0, ct = 0;
  int i0 = 0;
  for (; i0 + CH < nitems; i0 += CH) {
#pragma unroll
    for (int s = 0; s < CH; ++s) {
      compute(s, ct);
      if (ct == nt - 1) flush(cg);
      adv(cg, ct);
      load_item(s, lg, lt);
      adv(lg, lt);
    }
  }
#pragma unroll
  for (int s = 0; s < CH; ++s) {
    if (i0 + s < nitems) {
      compute(s, ct);
      if (ct == nt - 1) flush(cg);
      adv(cg, ct);
    }
  }
  lds_barrier();

  // ---- outputs: the waves' partial sums added in wave order, times the row scale
  const int per = M * 16;
  const int total = ng * half * per;
  // e = ((g * half + j) * M + i) * 16 + c with half = 1 (NS is 2 only on the silu arm, whose group
  // is one gate strip and its up strip: one output strip either way). q / M by a float reciprocal:
  // q + 1/2 lies at least 1/(2M) >= 1/32 from a multiple of M, and for q < 2^16 the product's
  // rounding error is below 2^-7, so the truncation is exact (no integer division on the tail)
  const float inv_m = 1.0f / (float)M;
  for (int e = tid; e < total; e += blockDim.x) {
    const int c = e & 15, q = e >> 4;
    const int g = (int)(((float)q + 0.5f) * inv_m);
    const int i = q - g * M;
    constexpr int j = 0;
    int64_t sj;
    if (!strip_of(p.silu, g0 + g, j, half, NS, nstrips, sj)) continue;
    // up to 8 partials read at once; the missing ones add +0, which changes no sum (the running sum
    // starts at +0 and is never -0)
    float pr[8], pu[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const int wc = w < kw ? w : 0;
      pr[w] = red[(((g * kw + wc) * NS + j) * M + i) * 16 + c];
      pu[w] = p.silu ? red[(((g * kw + wc) * NS + j + half) * M + i) * 16 + c] : 0.f;
    }
    float tot = 0.f, tot_up = 0.f;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      tot += w < kw ? pr[w] : 0.f;
      tot_up += w < kw ? pu[w] : 0.f;
    }
    const float scl = srow[i];
    const int64_t col = sj * kTileN + c;
    if (MODE == kModeNV) {
      // the per-output-channel global (f32 bits in the zeros slot)
      tot *= __int_as_float(p.zeros[col]);
      if (p.silu) {
        int64_t su;
        strip_of(p.silu, g0 + g, j + half, half, NS, nstrips, su);
        tot_up *= __int_as_float(p.zeros[su * kTileN + c]);
      }
    }
    if (p.silu)
      store_out(p, i, col, silu_mul(tot * scl, tot_up * scl, p.out_dtype));
    else
      store_out(p, i, col, tot * scl);
  }
}

namespace {


template <int NS, int CH, int MODE, bool SYM, int SM, int DT>
void walk_launch_dt(const GemmArgs& p, const WalkPlan& wp, hipStream_t stream) {
  auto kern = gemv_walk_kernel<NS, CH, MODE, SYM, SM, DT>;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, kWalkLdsMax);
  (void)attr;
  const WalkArgs wa{wp.waves, wp.sets, wp.tpw, wp.ngroups / wp.grid, wp.ngroups % wp.grid, wp.tpr_log};
  hipLaunchKernelGGL(kern, dim3(wp.grid), dim3(wp.block_waves * 64), wp.lds, stream, p, wa);
}

template <int NS, int CH, int MODE, bool SYM, int SM>
void walk_launch(const GemmArgs& p, const WalkPlan& wp, hipStream_t stream) {
  if (p.xdtype == kF16) walk_launch_dt<NS, CH, MODE, SYM, SM, kF16>(p, wp, stream);
  else walk_launch_dt<NS, CH, MODE, SYM, SM, kBF16>(p, wp, stream);
}

template <int NS, int CH, int MODE, bool SYM>
bool walk_sm(const GemmArgs& p, const WalkPlan& wp, hipStream_t stream) {
  switch (wp.sm) {
    case 1: walk_launch<NS, CH, MODE, SYM, 1>(p, wp, stream); return true;
    case 2: walk_launch<NS, CH, MODE, SYM, 2>(p, wp, stream); return true;
    case 4: walk_launch<NS, CH, MODE, SYM, 4>(p, wp, stream); return true;
    case 8: walk_launch<NS, CH, MODE, SYM, 8>(p, wp, stream); return true;
    case 16: walk_launch<NS, CH, MODE, SYM, 16>(p, wp, stream); return true;
    default: return false;
  }
}

template <int NS, int CH>
bool walk_fmt(const GemmArgs& p, const WalkPlan& wp, hipStream_t stream) {
  if (p.wfmt == kInt4) {
    if (p.zeros == nullptr) return walk_sm<NS, CH, kModeI4, true>(p, wp, stream);
    return walk_sm<NS, CH, kModeI4, false>(p, wp, stream);
  }
  if (gemv_nvfp4(p)) return walk_sm<NS, CH, kModeNV, false>(p, wp, stream);
  return walk_sm<NS, CH, kModeE8M0, false>(p, wp, stream);
}

}  // namespace

bool launch_gemv_walk(const GemmArgs& p, const WalkPlan& wp, hipStream_t stream) {
  constexpr int kCh = 4;  // tiles of weight loads in flight per wave
  return p.silu ? walk_fmt<2, kCh>(p, wp, stream) : walk_fmt<1, kCh>(p, wp, stream);
}

}  // namespace w4a8

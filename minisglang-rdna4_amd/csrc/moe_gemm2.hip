// Fused gemm2 + top-k weighted combine of the MoE FFN for decode-sized batches: one launch does
// the per-row act quant of the gemm1 buffer, the down projection and the per-token reduction.
// Restates fp8_wmma.mmq_fp8_moe_gemm2_gather_reduce (python/minisgl/quant/kernels.py:831-850):
//   out[t, n] = sum_j tw[t, j] * s_(t,j) * sum_g scale[e, g, n] * sum_{k in g} e4m3(q_(t,j)[k]) * w_e(n, k)
// with q_(t,j), s_(t,j) the per-row fp8 quant of the gemm1 row of slot (t, j) (act_quant.h's
// arithmetic) and e the slot's expert; f32 throughout, cast to the output dtype once.
//
// Work split: workgroup = (16-channel strip, token), one wave per top-k slot. Each wave quantizes
// its slot's gemm1 row into LDS, streams its expert's weight tiles for the strip and leaves the
// slot's 16 outputs in LDS; then 16 threads sum the token's slots in slot order. No workgroup
// talks to another, so there are no atomics and no device-scope fences, and the result does not
// depend on timing. Experts shared by several tokens are read once per token (from L2 or MALL
// after the first): the grid's strips map to XCDs by strip index, so every token's workgroup for
// a strip meets the same L2.
//
// Bits: a slot's row sum follows the grouped gemm2's K split (K tiles in runs of tpw, one
// accumulator per run started from zero, the runs summed in order) with the same per-tile MFMA
// and FMA sequence, and the combine is the unfused combine's FMA chain, so the output equals the
// unfused path (act quant, w4a8_moe_gemm decode arm into row_dtype, w4a8_moe_combine) bit for bit.
// row_dtype follows the reference: its fused gemm2 + gather-reduce sums the slot rows unrounded
// (f32), its unfused gemm2 (NVFP4 two-level weights, or MINISGL_MOE_G2FUSE=0) hands them over in
// the activation dtype.
#include "gemv.h"

namespace w4a8 {

struct G2CArgs {
  const uint16_t* a;      // gemm1 buffer (P, K) bf16/fp16, rows at padded positions
  int64_t lda;            // elements
  int adtype;
  const int32_t* inv_pos; // (T*top_k) slot -> padded row, < 0 for a dropped slot
  const int32_t* ids;     // (T*top_k) expert of each slot
  const float* tw;        // (T*top_k) routing weights
  int top_k;
  int E;
  const uint4* wt;        // W4 tiles of every expert
  int64_t w_expert_tiles;
  const void* scales;
  int64_t s_expert_stride;
  const int32_t* zeros;   // AWQ zero words (E, K/g, N/8), the NVFP4 global (E, N), or null
  int64_t z_expert_stride;
  int group;
  int N, K, KT;
  int tpw;                // K tiles per run of the grouped gemm2's split
  void* out;
  int out_dtype;
  int64_t ldo;
  int row_dtype;          // each slot's gemm2 row rounded to this dtype before the combine (kF32: not)
};

constexpr int kG2cMaxSlots = 16;

// MODE: kModeI4 (int4, group a multiple of 128), kModeE8M0 (MXFP4), kModeNV (NVFP4). SYM: int4
// without zero points. KTMAX: most K tiles (weights of every tile are loaded up front). SLOTS: most
// top-k slots (waves) of the launch, 8 or 16: a 16-wave workgroup leaves each wave 128 VGPRs, an
// 8-wave one 256, which the 16-tile NVFP4 and asymmetric int4 kernels need. NSG: strips per
// workgroup; each wave quantizes its slot's row once for all of them.
template <int MODE, bool SYM, int KTMAX, int SLOTS, int NSG>
__global__ void __launch_bounds__(SLOTS * 64) moe_gemm2_combine_kernel(const G2CArgs p) {
  extern __shared__ __align__(16) unsigned char arows[];  // per wave: KT*128 fp8 codes + 16 bytes
  __shared__ float ys[SLOTS][kTileN * NSG];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // top-k slot j
  const int strip0 = blockIdx.x * NSG;
  const int64_t t = blockIdx.y;
  const int64_t slot = t * p.top_k + wave;
  const int pos = p.inv_pos[slot];
  const int e = p.ids[slot];
  const bool valid = pos >= 0 && e >= 0 && e < p.E;  // uniform across the wave
  const int N = p.N, K = p.K, KT = p.KT;
  const int astride = KT * kTileK + 16;
  unsigned char* arow = arows + wave * astride;
  const int nstrips = N / kTileN;
  // strip q of the workgroup (past the last strip: the last one again, never stored) and this
  // lane's output channel in it
  int stq[NSG], nq[NSG];
#pragma unroll
  for (int q = 0; q < NSG; ++q) {
    stq[q] = strip0 + q < nstrips ? strip0 + q : nstrips - 1;
    nq[q] = stq[q] * kTileN + (lane & 15);
  }
  float yv[NSG];
#pragma unroll
  for (int q = 0; q < NSG; ++q) yv[q] = 0.f;

  if (valid) {
    // ---- the slot's gemm1 row: per-row fp8 quant into this wave's LDS row (act_quant.h's
    // arithmetic: s = max(amax / 448, 1e-8), codes = e4m3(x * (1 / s)), the max being exact). The
    // row's loads go out before the weight loads, so its quant does not wait behind them (T=1..8:
    // 1-2% per call)
    constexpr int kAch = (KTMAX * kTileK / 8 + 63) / 64;  // 16-byte loads per lane
    const uint16_t* src = p.a + (int64_t)pos * p.lda;
    const int nch = K / 8;
    uint4 xa[kAch];
#pragma unroll
    for (int i = 0; i < kAch; ++i) {
      const int c = lane + 64 * i;
      xa[i] = c < nch ? *reinterpret_cast<const uint4*>(src + c * 8) : make_uint4(0u, 0u, 0u, 0u);
    }
    // ---- weight tiles, scales and zero words of every K tile, all in flight before the quant
    const uint4* wt = p.wt + (size_t)((int64_t)e * p.w_expert_tiles) * 64;
    const int kEsz = MODE == kModeI4 ? 2 : 1;
    const void* scales = reinterpret_cast<const char*>(p.scales) + (size_t)((int64_t)e * p.s_expert_stride) * kEsz;
    const int32_t* zeros = p.zeros ? p.zeros + (int64_t)e * p.z_expert_stride : nullptr;
    const BufRsrc rs_w = make_rsrc(wt, (uint32_t)((N / kTileN) * KT * kTileBytes));
    const int ngroups = K >> (31 - __builtin_clz((unsigned)p.group));
    const BufRsrc rs_s = make_rsrc(scales, (uint32_t)(ngroups * N * kEsz));
    const BufRsrc rs_z = make_rsrc(zeros, (MODE == kModeI4 && zeros) ? (uint32_t)(ngroups * (N / 8) * 4) : 0u);
    const int gshift = 31 - __builtin_clz((unsigned)(p.group >= kTileK ? p.group / kTileK : 1));
    uint4 raw[KTMAX][NSG];
    // fp16 scales and NVFP4 block-scale bytes land in the 16-bit halves of their registers (a d16
    // load writes one half without waiting): two scales per VGPR, two NVFP4 bytes per VGPR. Kept
    // as one value per VGPR, the KTMAX=16 NVFP4 and asymmetric int4 kernels spilled to scratch.
    typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
    v2u16 sc[(KTMAX + 1) / 2][NSG];
    uint32_t zw[(MODE == kModeI4 && !SYM) ? KTMAX : 1][NSG];
    int sb[MODE == kModeE8M0 ? KTMAX : 1][NSG];
    v2u16 nvs[MODE == kModeNV ? KTMAX : 1][NSG][4];
    // every slot up to KTMAX is loaded, those past KT from tile KT-1 again (a cache hit, never
    // used): a guard per tile made the compiler finish each tile's scale before issuing the next
    // tile, one memory round trip per K tile
#pragma unroll
    for (int kt = 0; kt < KTMAX; ++kt) {
      const int kc = kt < KT ? kt : KT - 1;
#pragma unroll
      for (int q = 0; q < NSG; ++q) {
        const int n = nq[q];
        raw[kt][q] = bload128_nt(rs_w, (uint32_t)lane * 16, (uint32_t)((stq[q] * KT + kc) * kTileBytes));
        if (MODE == kModeI4) {
          const int g = kc >> gshift;
          sc[kt >> 1][q][kt & 1] = bload16(rs_s, (uint32_t)n * 2, (uint32_t)(g * N * 2));
          if (!SYM)
            zw[(MODE == kModeI4 && !SYM) ? kt : 0][q] = bload32(rs_z, (uint32_t)(n / 8) * 4, (uint32_t)(g * (N / 8) * 4));
        } else if (MODE == kModeE8M0) {
          sb[MODE == kModeE8M0 ? kt : 0][q] = (int)bload8(rs_s, (uint32_t)((lane >> 4) * N + n), (uint32_t)(kc * 4 * N));
        } else {
#pragma unroll
          for (int ss = 0; ss < 8; ++ss)
            nvs[MODE == kModeNV ? kt : 0][q][ss >> 1][ss & 1] =
                (unsigned short)bload8(rs_s, (uint32_t)n, (uint32_t)((kc * 8 + ss) * N));
        }
      }
    }

    float am = 0.f;
#pragma unroll
    for (int i = 0; i < kAch; ++i) am = fmaxf(am, amax8(xa[i], p.adtype));
    const float s = act_row_scale(wave_max(am));
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < kAch; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
        float f[8];
        unpack8(xa[i], p.adtype, f);
        *reinterpret_cast<uint2*>(arow + c * 8) = quant8(f, inv);
      }
    }
    // the row is read back by other lanes of this wave only: LDS serves one wave's accesses in
    // order, so waiting for the writes (and keeping the compiler from moving the reads above them)
    // is all the ordering needed -- no workgroup barrier, which waves on dropped slots never reach
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // ---- K loop: A row 0 of the MFMA is the slot's row (the other rows are zero and unused)
    const v4f zero4 = v4f{0.f, 0.f, 0.f, 0.f};
    v4f acc[NSG], tot[NSG];
#pragma unroll
    for (int q = 0; q < NSG; ++q) acc[q] = tot[q] = zero4;
    const bool arow_lane = (lane & 15) == 0;
#pragma unroll
    for (int kt = 0; kt < KTMAX; ++kt) {
      if (kt < KT) {
        v8i at;
        uint4 lo = make_uint4(0u, 0u, 0u, 0u), hi = lo;
        if (arow_lane) {
          const unsigned char* ap = arow + kt * kTileK + 16 * (lane >> 4);
          lo = *reinterpret_cast<const uint4*>(ap);
          hi = *reinterpret_cast<const uint4*>(ap + 64);
        }
        at[0] = (int)lo.x; at[1] = (int)lo.y; at[2] = (int)lo.z; at[3] = (int)lo.w;
        at[4] = (int)hi.x; at[5] = (int)hi.y; at[6] = (int)hi.z; at[7] = (int)hi.w;
        const v4f seed = (MODE == kModeI4 && SYM) ? mfma_f8f8(at, splat8(0xB0B0B0B0u), zero4) : zero4;  // -R/2
        const v4f rh = (MODE == kModeI4 && !SYM) ? mfma_f8f8(at, splat8(kE4M3Half4), zero4) : zero4;
#pragma unroll
        for (int q = 0; q < NSG; ++q) {
          if (MODE == kModeE8M0) {
            acc[q] = mfma_f8f4_sb(at, fp4_operand(raw[kt][q]), acc[q], sb[MODE == kModeE8M0 ? kt : 0][q]);
          } else if (MODE == kModeI4 && SYM) {
            const v4f c = mfma_f8f8(at, unpack_tile_int4(raw[kt][q]), seed);
            const float scf = f16_to_f32(sc[kt >> 1][q][kt & 1]);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[q][r] = fmaf(scf, c[r], acc[q][r]);
          } else if (MODE == kModeI4) {
            const v4f c = mfma_f8f8(at, unpack_tile_int4(raw[kt][q]), zero4);
            const uint32_t z = zw[(MODE == kModeI4 && !SYM) ? kt : 0][q];
            const float coef = 15.0f - 2.0f * (float)((z >> (4 * (nq[q] & 7))) & 15u);
            const float scf = f16_to_f32(sc[kt >> 1][q][kt & 1]);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[q][r] = fmaf(scf, fmaf(coef, rh[r], c[r]), acc[q][r]);
          } else {
            const v8i b = fp4_operand(raw[kt][q]);
#pragma unroll
            for (int ss = 0; ss < 8; ++ss) {
              const v4f c = mfma_f8f4_sb(at, fp4_half_operand(b, ss), zero4, subgroup_mask_scale(lane, 8, ss));
              const float scf =
                  __builtin_amdgcn_cvt_f32_fp8((int)(uint32_t)nvs[MODE == kModeNV ? kt : 0][q][ss >> 1][ss & 1], 0);
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[q][r] = fmaf(scf, c[r], acc[q][r]);
            }
          }
        }
        // end of a run of the grouped gemm2's split: fold it into the total in run order
        if ((kt + 1) % p.tpw == 0 || kt + 1 == KT) {
#pragma unroll
          for (int q = 0; q < NSG; ++q) {
#pragma unroll
            for (int r = 0; r < 4; ++r) tot[q][r] = tot[q][r] + acc[q][r];
            acc[q] = zero4;
          }
        }
      }
    }
    // row 0 of the C fragment: element 0 of lanes 0..15 (column = lane)
#pragma unroll
    for (int q = 0; q < NSG; ++q) {
      float v = tot[q][0];
      if (MODE == kModeNV) v *= __int_as_float(zeros[nq[q]]);  // the per-output-channel global
      yv[q] = v * s;
      if (p.row_dtype != kF32) yv[q] = from_dtype(to_dtype(yv[q], p.row_dtype), p.row_dtype);
    }
  }
  if (lane < kTileN) {
#pragma unroll
    for (int q = 0; q < NSG; ++q) ys[wave][q * kTileN + lane] = yv[q];
  }
  __syncthreads();
  if (threadIdx.x < kTileN * NSG) {
    const int q = threadIdx.x / kTileN, c = threadIdx.x % kTileN;
    if (strip0 + q < nstrips) {
      float acc = 0.f;
      for (int j = 0; j < p.top_k; ++j) {
        const int64_t sl = t * p.top_k + j;
        if (p.inv_pos[sl] >= 0) acc = fmaf(p.tw[sl], ys[j][threadIdx.x], acc);
      }
      const int64_t col = (int64_t)(strip0 + q) * kTileN + c;
      if (p.out_dtype == kF32)
        reinterpret_cast<float*>(p.out)[t * p.ldo + col] = acc;
      else
        reinterpret_cast<uint16_t*>(p.out)[t * p.ldo + col] = to_dtype(acc, p.out_dtype);
    }
  }
}

// True when the fused kernel serves these weights: int4 with groups of 128 or more, MXFP4 (E8M0)
// or NVFP4, K a multiple of 128 up to 2048, top_k up to 16; NVFP4 and asymmetric int4 past 8 K
// tiles only for up to 8 slots (their 16-tile kernel does not fit 128 VGPRs).
bool moe_gemm2_combine_fits(int64_t K, int scale_fmt, bool has_zeros, int wfmt, int64_t group, int top_k) {
  const bool i4 = wfmt == kInt4 && scale_fmt == kScaleF16 && group % kTileK == 0;
  const bool nv = wfmt == kE2M1 && scale_fmt == kScaleE4M3 && has_zeros && group == 16;
  const bool fmt = i4 || nv || (wfmt == kE2M1 && scale_fmt == kScaleE8M0 && !has_zeros && group == 32);
  const bool wide_ok = !(nv || (i4 && has_zeros)) || K <= 8 * kTileK || top_k <= 8;
  return fmt && wide_ok && K % kTileK == 0 && K <= 16 * kTileK && top_k >= 1 && top_k <= kG2cMaxSlots;
}

// The 8-tile, 8-slot kernel (the configs[4] decode shape) takes two strips per workgroup from 8
// tokens on: each wave quantizes its slot's row once for both and keeps twice the weight bytes in
// flight (configs[4], whole call: T=8 39.8 -> 38.5 us, T=12 55.7 -> 54.7, T=16 64.0 -> 62.9); below
// 8 tokens the grid of half as many workgroups leaves CUs idle (T=1 15.5 -> 16.9). Four strips
// were slower at every T. Each strip's arithmetic is the same, so the bits are too. K of up to 6
// tiles (inter 768, the configs[4] experts) takes a 6-tile kernel: the registers of the two tiles
// the 8-tile one loads and never uses went to occupancy (two strips: 108 -> 88 VGPRs, 4 -> 5 waves
// per SIMD; T=16 whole call 56.7 -> 54.4 us, T=1..12 within the runs' noise). The tiles past KT
// are never used either way, so the bits are the same.
template <int MODE, bool SYM>
static void g2c_launch(const G2CArgs& a, int64_t T, size_t lds, hipStream_t st) {
  const bool few = a.top_k <= 8;
  const int nstrips = a.N / kTileN;
  const dim3 block((unsigned)(a.top_k * 64));
  auto grid = [&](int nsg) { return dim3((unsigned)((nstrips + nsg - 1) / nsg), (unsigned)T); };
  if (a.KT <= 6 && few && T >= 8)
    hipLaunchKernelGGL((moe_gemm2_combine_kernel<MODE, SYM, 6, 8, 2>), grid(2), block, lds, st, a);
  else if (a.KT <= 6 && few)
    hipLaunchKernelGGL((moe_gemm2_combine_kernel<MODE, SYM, 6, 8, 1>), grid(1), block, lds, st, a);
  else if (a.KT <= 8 && few && T >= 8)
    hipLaunchKernelGGL((moe_gemm2_combine_kernel<MODE, SYM, 8, 8, 2>), grid(2), block, lds, st, a);
  else if (a.KT <= 8 && few)
    hipLaunchKernelGGL((moe_gemm2_combine_kernel<MODE, SYM, 8, 8, 1>), grid(1), block, lds, st, a);
  else if (a.KT <= 8)
    hipLaunchKernelGGL((moe_gemm2_combine_kernel<MODE, SYM, 8, 16, 1>), grid(1), block, lds, st, a);
  else if (few)
    hipLaunchKernelGGL((moe_gemm2_combine_kernel<MODE, SYM, 16, 8, 1>), grid(1), block, lds, st, a);
  else if constexpr (MODE != kModeNV && (MODE != kModeI4 || SYM))
    hipLaunchKernelGGL((moe_gemm2_combine_kernel<MODE, SYM, 16, 16, 1>), grid(1), block, lds, st, a);
}

// p: the grouped gemm2's arguments as w4a8_moe_gemm would build them for the decode arm (for the
// K split); the rest is the fused kernel's. The caller checked moe_gemm2_combine_fits.
int launch_moe_gemm2_combine(const GemmArgs& p, int64_t row_blocks, const uint16_t* a, int64_t lda, int adtype,
                             const int32_t* inv_pos, const int32_t* ids, const float* tw, int64_t T, int E,
                             int row_dtype, hipStream_t stream) {
  int waves = 0, tpw = 0;
  gemv_ksplit(p, row_blocks, waves, tpw);
  G2CArgs g = {};
  g.a = a; g.lda = lda; g.adtype = adtype;
  g.inv_pos = inv_pos; g.ids = ids; g.tw = tw; g.top_k = p.top_k; g.E = E;
  g.wt = p.wt; g.w_expert_tiles = p.w_expert_tiles;
  g.scales = p.scales; g.s_expert_stride = p.s_expert_stride;
  g.zeros = p.zeros; g.z_expert_stride = p.z_expert_stride;
  g.group = p.group; g.N = (int)p.N; g.K = (int)p.K; g.KT = (int)p.KT; g.tpw = tpw;
  g.out = p.out; g.out_dtype = p.out_dtype; g.ldo = p.ldo; g.row_dtype = row_dtype;
  const size_t lds = (size_t)p.top_k * (p.KT * kTileK + 16);
  if (p.wfmt == kE2M1 && p.sfmt == kScaleE8M0) g2c_launch<kModeE8M0, false>(g, T, lds, stream);
  else if (p.wfmt == kE2M1) g2c_launch<kModeNV, false>(g, T, lds, stream);
  else if (p.zeros == nullptr) g2c_launch<kModeI4, true>(g, T, lds, stream);
  else g2c_launch<kModeI4, false>(g, T, lds, stream);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

}  // namespace w4a8

// Large-M W4A8 GEMM (prefill band and the grouped MoE GEMMs) with LDS-staged operands, for the
// formats whose scale changes at most once per 128-wide K tile: int4 with a group multiple of 128
// (fp16 scales, with or without zero points) and MXFP4 (E8M0 block-32 scales).
//
// Same arithmetic as gemm_prefill.hip (python/minisgl/quant/kernels.py:1632, 1686-1734, 744-773):
// y[m,n] = s_m * sum_g scale[g,n] * sum_{k in g} e4m3(x[m,k]) w(n,k), f32 accumulation.
//
// Workgroup tile BM x BN x 128 (K step = one group or less), WM x WN waves, wave tile RB row blocks
// x NSB strips of 16. Per K step the workgroup copies, into the other half of a double-buffered
// LDS stage while it computes from this one:
//   A  (BM x 128 fp8)  in MFMA operand order [row block][half][lane][16 B], so each wave's fragment
//                      read is two contiguous, conflict-free 1 KiB ds_read_b128;
//   B  int4: W4 tiles unpacked ONCE per workgroup to the fp8 operand [strip][half][lane][16 B]
//      (each wave that uses a strip reads it, none unpacks it again); e2m1: the fp4 bytes as is;
//   per-strip scales (fp16 for the stage's group, or the E8M0 bytes of its four 32-blocks in lane
//   order) and zero-point words.
// Global loads for step k+1 are issued before step k's MFMAs and written to LDS after them, one
// barrier per step. int4 symmetric: the MFMA accumulator is seeded with -R/2 (an MFMA of the A
// fragment against a constant -0.5 operand, once per row block per step); asymmetric: row sums
// R/2 from an MFMA against +0.5 and acc += s * (C + (15 - 2z) R/2); MXFP4: E8M0 bytes feed the
// scaled MFMA and the accumulator stays in the MFMA.
#include <cstdlib>
#include <type_traits>

#include "prefill.h"

namespace w4a8 {

// WPE: waves per SIMD the register budget is sized for (2: 256 registers per wave; 1: 512, for
// the large wave tiles whose accumulators live in AGPRs).
template <int WM, int WN, int RB, int NSB, int MODE, int WPE>
__global__ void __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
gemm_lds_kernel(const GemmArgs p) {
  constexpr int T = WM * WN * 64;
  constexpr int BM = WM * RB * 16, BN = WN * NSB * 16;
  constexpr int NSTRIP = BN / 16;
  using S = LdsStage<BM, BN, MODE>;
  constexpr int A_PER = BM * 8 / T;   // 16-byte A chunks per thread per step
  constexpr int B_PER = NSTRIP * 64 / T;  // 16-byte weight chunks per thread per step
  static_assert(A_PER * T == BM * 8 && B_PER * T == NSTRIP * 64, "tile / thread mismatch");
  extern __shared__ __align__(16) unsigned char lds[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int64_t blk_row0 = (int64_t)blockIdx.y * BM;

  int64_t expert = 0;
  if (p.sorted_ids) {
    if (blk_row0 >= (int64_t)(*p.ntp)) return;
    expert = p.expert_ids[(uint32_t)blk_row0 / (uint32_t)p.bm];  // padded rows < 2^31
  }
  const int N = (int)p.N, K = (int)p.K, KT = (int)p.KT;
  const int nstrips = N / kTileN;
  const int gshift = 31 - __builtin_clz((unsigned)(p.group >= kTileK ? p.group / kTileK : 1));

  // global strip of LDS strip s. Wave wn computes LDS strips [wn * NSB, wn * NSB + NSB); with silu
  // the first half of each wave's strips are gate strips and the second half the matching up strips,
  // so a wave's strips sit at fixed LDS offsets whatever the activation.
  auto gstrip = [&](int s, bool& ok) __attribute__((always_inline)) {
    int gs;
    if (p.silu) {
      constexpr int hj = NSB / 2;
      const int j = s % NSB;
      const int h = (int)blockIdx.x * (NSTRIP / 2) + (s / NSB) * hj + (j < hj ? j : j - hj);
      gs = j < hj ? h : nstrips / 2 + h;
      ok = h < nstrips / 2;
    } else {
      gs = (int)blockIdx.x * NSTRIP + s;
      ok = gs < nstrips;
    }
    return ok ? gs : nstrips - 1;
  };

  const uint4* wt = p.wt + (size_t)(expert * p.w_expert_tiles) * 64;
  constexpr int kEsz = MODE == kPE8M0 ? 1 : 2;
  const unsigned char* scales = reinterpret_cast<const unsigned char*>(p.scales) + (size_t)(expert * p.s_expert_stride) * kEsz;
  const int32_t* zeros = p.zeros ? p.zeros + expert * p.z_expert_stride : nullptr;

  // ---- per-thread copy assignments (fixed across K steps): buffer loads with a 32-bit per-lane
  // offset and a scalar per-step offset, no 64-bit address math in the loop
  const BufRsrc rs_a = make_rsrc(p.xq, 0xffffffffu);
  const BufRsrc rs_w = make_rsrc(wt, (uint32_t)((size_t)nstrips * KT * kTileBytes));
  const int ngroups = K >> (31 - __builtin_clz((unsigned)p.group));
  const BufRsrc rs_s = make_rsrc(scales, (uint32_t)((size_t)(MODE == kPE8M0 ? K / 32 : ngroups) * N * kEsz));
  const BufRsrc rs_z = make_rsrc(zeros, zeros ? (uint32_t)((size_t)ngroups * (N / 8) * 4) : 0u);
  uint32_t a_voff[A_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int c = (int)threadIdx.x + i * T;  // = (rb * 2 + h) * 64 + l
    const int l = c & 63, h = (c >> 6) & 1, rb = c >> 7;
    int64_t ar;
    const bool ok = lrow_source(p, blk_row0 + rb * 16 + (l & 15), ar);
    a_voff[i] = (uint32_t)((ok ? ar : 0) * p.ldx) + h * 64 + 16 * (l >> 4);
  }
  uint32_t b_voff[B_PER];
#pragma unroll
  for (int i = 0; i < B_PER; ++i) {
    const int c = (int)threadIdx.x + i * T;  // = s * 64 + l
    bool ok;
    const int gs = gstrip(c >> 6, ok);
    b_voff[i] = (uint32_t)(((size_t)gs * KT * 64 + (c & 63)) * 16);
  }

  // two register sets of prefetched operands (steps k+1 and k+2 in flight while step k computes);
  // native vectors, since whole-struct uint4 copies keep arrays out of registers
  v4u ra[2][A_PER], rbw[2][B_PER];
  uint4 rs[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
  uint2 rz[2] = {make_uint2(0, 0), make_uint2(0, 0)};
  using Set0 = std::integral_constant<int, 0>;
  using Set1 = std::integral_constant<int, 1>;
  // scale / zero copy roles: int4 fp16 -> 2 chunks of 16 B per strip; E8M0 -> 4 chunks per strip.
  // Threads past the chunk count load a duplicate of the last chunk (unconditional loads keep the
  // wait counts exact).
  constexpr int S_CHUNKS = MODE == kPE8M0 ? NSTRIP * 4 : NSTRIP * 2;
  const int sc_c = (int)threadIdx.x < S_CHUNKS ? (int)threadIdx.x : S_CHUNKS - 1;
  bool sc_ok;
  const int sc_gs = gstrip(MODE == kPE8M0 ? (sc_c >> 2) : (sc_c >> 1), sc_ok);
  const uint32_t s_voff = MODE == kPE8M0 ? (uint32_t)((sc_c & 3) * N + sc_gs * 16)
                                         : (uint32_t)((sc_gs * 16 + (sc_c & 1) * 8) * 2);
  const int z_c = (int)threadIdx.x < NSTRIP ? (int)threadIdx.x : NSTRIP - 1;
  bool z_ok;
  const uint32_t z_voff = (uint32_t)(gstrip(z_c, z_ok) * 2 * 4);

  auto issue = [&](int kt, auto set) __attribute__((always_inline)) {
    constexpr int R = decltype(set)::value;
    // the step offsets are wave-uniform; readfirstlane keeps them in SGPRs (a VGPR soffset makes
    // the compiler wrap every load in a waterfall loop)
    const uint32_t so_a = (uint32_t)__builtin_amdgcn_readfirstlane(kt * kTileK);
    const uint32_t so_b = (uint32_t)__builtin_amdgcn_readfirstlane(kt * kTileBytes);
    const int g = kt >> gshift;
    const uint32_t so_s = (uint32_t)__builtin_amdgcn_readfirstlane(MODE == kPE8M0 ? kt * 4 * N : g * N * 2);
#pragma unroll
    for (int i = 0; i < A_PER; ++i) ra[R][i] = bload128v(rs_a, a_voff[i], so_a);
#pragma unroll
    for (int i = 0; i < B_PER; ++i) rbw[R][i] = bload128v(rs_w, b_voff[i], so_b);
    rs[R] = bload128(rs_s, s_voff, so_s);
    if (MODE == kPAsym)
      rz[R] = bload64(rs_z, z_voff, (uint32_t)__builtin_amdgcn_readfirstlane(g * (N / 8) * 4));
  };
  auto commit = [&](int buf, auto set) __attribute__((always_inline)) {
    constexpr int R = decltype(set)::value;
    unsigned char* st = lds + buf * S::kBytes;
#pragma unroll
    for (int i = 0; i < A_PER; ++i) *reinterpret_cast<v4u*>(st + ((int)threadIdx.x + i * T) * 16) = ra[R][i];
    unsigned char* sb = st + S::kA;
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int c = (int)threadIdx.x + i * T;
      const int s = c >> 6, l = c & 63;
      if (MODE == kPE8M0) {
        *reinterpret_cast<v4u*>(sb + (s * 64 + l) * 16) = rbw[R][i];
      } else {
        const v8i u = unpack_tile_int4(make_uint4(rbw[R][i].x, rbw[R][i].y, rbw[R][i].z, rbw[R][i].w));
        *reinterpret_cast<uint4*>(sb + ((s * 2 + 0) * 64 + l) * 16) = make_uint4(u[0], u[1], u[2], u[3]);
        *reinterpret_cast<uint4*>(sb + ((s * 2 + 1) * 64 + l) * 16) = make_uint4(u[4], u[5], u[6], u[7]);
      }
    }
    // threads past the chunk count write the same bytes as the last chunk's owner (identical values,
    // no branch among the writes)
    *reinterpret_cast<uint4*>(st + S::kA + S::kB + sc_c * 16) = rs[R];
    if (MODE == kPAsym) *reinterpret_cast<uint2*>(st + S::kA + S::kB + S::kS + z_c * 8) = rz[R];
  };

  // wave's strips in LDS order
  int sl[NSB];
#pragma unroll
  for (int j = 0; j < NSB; ++j) sl[j] = wn * NSB + j;

  v4f acc[RB][NSB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < NSB; ++j) acc[rb][j] = v4f{0.f, 0.f, 0.f, 0.f};
  const v4f zero4 = v4f{0.f, 0.f, 0.f, 0.f};

  // per-lane LDS offsets of this wave's operands, computed once; the empty asm keeps each in one
  // VGPR so every read in the K loop is that VGPR plus an immediate
  uint32_t oa = (uint32_t)(wm * RB * 2048 + lane * 16);
  uint32_t ob = (uint32_t)(S::kA + wn * NSB * (MODE == kPE8M0 ? 1024 : 2048) + lane * 16);
  uint32_t os = (uint32_t)(S::kA + S::kB + (MODE == kPE8M0 ? wn * NSB * 64 + lane : (wn * NSB * 16 + (lane & 15)) * 2));
  uint32_t oz = (uint32_t)(S::kA + S::kB + S::kS + (wn * NSB * 2 + ((lane & 15) >> 3)) * 4);
  asm volatile("" : "+v"(oa), "+v"(ob), "+v"(os), "+v"(oz));
  const int zsh = 4 * (lane & 7);

  // MFMA work of one K step from LDS stage `cur`. Operands are read one strip (or row block) ahead
  // of the MFMAs that use them, so a wave's LDS latency hides under its own MFMAs.
  auto compute = [&](int cur) __attribute__((always_inline)) {
    const unsigned char* st = lds + cur * S::kBytes;
    if (MODE == kPE8M0) {
      // all of the wave's fp4 strips and scale bytes (4 VGPRs + 1 per strip), then row blocks
      uint4 braw[NSB];
      int sbyte[NSB];
#pragma unroll
      for (int j = 0; j < NSB; ++j) {
        braw[j] = *reinterpret_cast<const uint4*>(st + ob + j * 1024);
        sbyte[j] = (int)st[os + j * 64];
      }
      v8i a0 = lds_operand(st + oa, 0);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        v8i a1;
        if (rb + 1 < RB) a1 = lds_operand(st + oa + (rb + 1) * 2048, 0);
        __builtin_amdgcn_sched_barrier(0);  // the read stays ahead of this row block's MFMAs
#pragma unroll
        for (int j = 0; j < NSB; ++j) acc[rb][j] = mfma_f8f4_sb(a0, fp4_operand(braw[j]), acc[rb][j], sbyte[j]);
        if (rb + 1 < RB) a0 = a1;
      }
      return;
    }
    v8i a[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) a[rb] = lds_operand(st + oa + rb * 2048, 0);
    v4f pre[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)  // symmetric: -R/2; zero points: +R/2
      pre[rb] = mfma_f8f8(a[rb], splat8(MODE == kPSym ? 0xB0B0B0B0u : kE4M3Half4), zero4);
    if (MODE == kPAsym) {
      // zero points: acc += s * (C + (15 - 2z) R/2); strip j's MFMAs run while strip j-1's
      // partials are scaled in (operands read at use: no registers to spare for a lookahead at
      // two waves per SIMD)
      v4f cp[RB];
      float scp = 0.f, cfp = 0.f;
#pragma unroll
      for (int j = 0; j <= NSB; ++j) {
        v4f cj[RB];
        float scj = 0.f, cfj = 0.f;
        if (j < NSB) {
          const v8i b = lds_operand(st + ob + j * 2048, 0);
          scj = f16_to_f32(*reinterpret_cast<const uint16_t*>(st + os + j * 32));
          const uint32_t zw = *reinterpret_cast<const uint32_t*>(st + oz + j * 8);
          cfj = 15.0f - 2.0f * (float)((zw >> zsh) & 15u);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) cj[rb] = mfma_f8f8(a[rb], b, zero4);
        }
        if (j > 0) {
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[rb][j - 1][r] += scp * (cp[rb][r] + cfp * pre[rb][r]);
        }
        if (j < NSB) {
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) cp[rb] = cj[rb];
          scp = scj;
          cfp = cfj;
        }
      }
      return;
    }
    // symmetric: strip j's MFMAs run while strip j+1's operand is read and strip j-1's partials
    // are scaled into the accumulators
    v8i bn = lds_operand(st + ob, 0);
    float scn = f16_to_f32(*reinterpret_cast<const uint16_t*>(st + os));
    v4f cp[RB];
    float scp = 0.f;
#pragma unroll
    for (int j = 0; j <= NSB; ++j) {
      v4f cj[RB];
      float scj = 0.f;
      if (j < NSB) {
        const v8i b = bn;
        scj = scn;
        if (j + 1 < NSB) {
          bn = lds_operand(st + ob + (j + 1) * 2048, 0);
          scn = f16_to_f32(*reinterpret_cast<const uint16_t*>(st + os + (j + 1) * 32));
        }
        __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of this strip's MFMAs
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) cj[rb] = mfma_f8f8(a[rb], b, pre[rb]);
      }
      if (j > 0) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[rb][j - 1][r] += scp * cp[rb][r];
      }
      if (j < NSB) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) cp[rb] = cj[rb];
        scp = scj;
      }
    }
  };

  // step k computes from stage k & 1; the loads for step k + 2 are issued before its MFMAs and the
  // registers of step k + 1 go to the other stage after them (K loop unrolled by two so each
  // register set is a compile-time index). The steady loop has no branch inside, so the MFMAs stay
  // ahead of the LDS writes (and the waits for their loads); the scheduling fences hold that order.
  issue(0, Set0{});
  commit(0, Set0{});
  if (KT > 1) issue(1, Set1{});
  lds_barrier();
  int kt = 0;
  for (; kt + 3 < KT; kt += 2) {
    issue(kt + 2, Set0{});
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    __builtin_amdgcn_sched_barrier(0);
    commit(1, Set1{});
    lds_barrier();
    issue(kt + 3, Set1{});
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    __builtin_amdgcn_sched_barrier(0);
    commit(0, Set0{});
    lds_barrier();
  }
  // drain: 1, 2 or 3 steps left (step kt is in stage 0, step kt + 1 in registers set 1)
  const int left = KT - kt;
  if (left == 3) {
    issue(kt + 2, Set0{});
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    __builtin_amdgcn_sched_barrier(0);
    commit(1, Set1{});
    lds_barrier();
    compute(1);
    __builtin_amdgcn_sched_barrier(0);
    commit(0, Set0{});
    lds_barrier();
    compute(0);
  } else if (left == 2) {
    compute(0);
    __builtin_amdgcn_sched_barrier(0);
    commit(1, Set1{});
    lds_barrier();
    compute(1);
  } else {
    compute(0);
  }

  // epilogue: lane holds rows 4*(lane>>4)+r of each row block, channel (lane & 15) of each strip
  const int64_t row0 = blk_row0 + (int64_t)wm * RB * 16;
  store_tile(p, acc, row0, lane, [&](int j, bool& ok) __attribute__((always_inline)) { return gstrip(sl[j], ok); });
}

template <int WM, int WN, int RB, int NSB, int MODE, int WPE>
static void launch_lds_one(const GemmArgs& p, dim3 grid, dim3 block, hipStream_t stream) {
  constexpr int BM = WM * RB * 16, BN = WN * NSB * 16;
  constexpr size_t lds = 2 * (size_t)LdsStage<BM, BN, MODE>::kBytes;
  auto kern = gemm_lds_kernel<WM, WN, RB, NSB, MODE, WPE>;
  // dynamic LDS above 64 KiB must be allowed per kernel, once
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  (void)attr;
  hipLaunchKernelGGL(kern, grid, block, lds, stream, p);
}

template <int WM, int WN, int RB, int NSB, int WPE = 2>
static int launch_lds_cfg(const GemmArgs& p, int mode, int64_t row_tiles, hipStream_t stream) {
  constexpr int BN = WN * NSB * 16;
  const int64_t ncols = p.silu ? p.N / 2 : p.N;
  const int64_t colw = p.silu ? BN / 2 : BN;
  const dim3 grid((unsigned)((ncols + colw - 1) / colw), (unsigned)row_tiles);
  const dim3 block(WM * WN * 64);
  if (mode == kPSym) launch_lds_one<WM, WN, RB, NSB, kPSym, WPE>(p, grid, block, stream);
  else if (mode == kPAsym) launch_lds_one<WM, WN, RB, NSB, kPAsym, WPE>(p, grid, block, stream);
  else launch_lds_one<WM, WN, RB, NSB, kPE8M0, WPE>(p, grid, block, stream);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

// Returns kErrUnsupported for formats this kernel does not cover (the caller then uses the
// per-wave kernel). bm_rows: rows per workgroup the caller requires (grouped: divides the align
// block; 0 for dense).
int launch_prefill_lds(const GemmArgs& p, int64_t rows_to_cover, int bm_rows, hipStream_t stream) {
  // NVFP4 on the fp16 MFMA, then the DMA-staged pipeline (three stages, A by LDS-DMA); this
  // kernel covers what those leave
  int rc = launch_prefill_nv(p, rows_to_cover, bm_rows, stream);
  if (rc != kErrUnsupported) return rc;
  rc = launch_prefill_dma(p, rows_to_cover, bm_rows, stream);
  if (rc != kErrUnsupported) return rc;
  int mode;
  if (p.wfmt == kInt4 && p.sfmt == kScaleF16 && p.group % kTileK == 0)
    mode = p.zeros ? kPAsym : kPSym;
  else if (p.wfmt == kE2M1 && p.sfmt == kScaleE8M0)
    mode = kPE8M0;
  else
    return kErrUnsupported;
  if (p.silu && (p.N / kTileN) % 2) return kErrUnsupported;
  if (p.K % kTileK) return kErrUnsupported;  // whole K tiles only (no masked tail)
  // grouped rows: a workgroup's rows must sit inside one align block (one expert)
  if (p.sorted_ids && bm_rows != 64 && bm_rows != 128) return kErrUnsupported;
  // 32-bit offsets within one matrix
  if ((int64_t)p.N * p.KT * 64 >= (int64_t)1 << 31) return kErrUnsupported;
  if (bm_rows == 64) return launch_lds_cfg<2, 4, 2, 2>(p, mode, (rows_to_cover + 63) / 64, stream);
  if (bm_rows == 128) return launch_lds_cfg<4, 2, 2, 4>(p, mode, (rows_to_cover + 127) / 128, stream);
  // dense: 256 x 128 tiles on 8 waves (two waves per SIMD hide each other's LDS and barrier
  // waits; measured faster than 128 x 128 on 4 waves for every format).
  // W4A8_PREFILL_ROWS=128|256 overrides the choice (tuning).
  static const int forced = [] {
    const char* e = getenv("W4A8_PREFILL_ROWS");
    return e ? atoi(e) : 0;
  }();
  const int rows = forced == 128 ? 128 : 256;
  if (rows == 128) return launch_lds_cfg<4, 2, 2, 4>(p, mode, (rows_to_cover + 127) / 128, stream);
  return launch_lds_cfg<4, 2, 4, 4>(p, mode, (rows_to_cover + 255) / 256, stream);
}

}  // namespace w4a8

// Large-M W4A8 GEMM (prefill band and grouped MoE GEMMs) with the activation tile copied straight
// from global memory into LDS by the buffer unit (buffer_load ... lds), three LDS stages deep.
//
// Same arithmetic and tile shapes as gemm_prefill_lds.hip (python/minisgl/quant/kernels.py:1632,
// 1686-1734, 744-773): y[m,n] = s_m * sum_g scale[g,n] * sum_{k in g} e4m3(x[m,k]) w(n,k), f32
// accumulation, one MFMA per (row block, strip, K step) of 128.
//
// What changes is how a K step's operands reach LDS:
//   A (BM x 128 fp8) and, for MXFP4, the fp4 weight strips and their E8M0 bytes are loaded by
//   LDS-DMA: one 1 KiB block per wave instruction, written in lane order, which is exactly the
//   MFMA operand order, so no VGPR holds them and no ds_write is issued;
//   int4 weights still go through registers: each workgroup unpacks every strip once (to the fp8
//   operand) and writes it to LDS, with its fp16 scales and zero words.
// Each stage is its own __shared__ array and every stage index is a compile-time constant (the K
// loop is unrolled by three), so the compiler tells the stages apart: reading stage k does not
// wait for the DMAs in flight to stages k+1 and k+2. Step k issues the loads of step k+2 (int4:
// between its MFMAs), computes step k, writes the int4 registers of step k+1, then waits for its
// own step-k+1 loads (a counted vmcnt, the loads of step k+2 stay in flight) and meets the other
// waves at one s_barrier.
#include <cstdlib>

#include "prefill.h"

namespace w4a8 {

template <int WM, int WN, int RB, int NSB, int MODE, bool AT>
__global__ void __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_dma_kernel(const GemmArgs p) {
  constexpr int T = WM * WN * 64, NW = WM * WN;
  constexpr int BM = WM * RB * 16, BN = WN * NSB * 16;
  constexpr int NSTRIP = BN / 16;
  constexpr bool kFp4 = MODE == kPE8M0;
  using S = LdsStage<BM, BN, MODE>;
  constexpr int A_PER = (BM / 8) / NW;                 // A 1 KiB blocks per wave per step
  static_assert(A_PER * NW == BM / 8, "A blocks / waves");
  constexpr int B_DMA = kFp4 ? NSTRIP / NW : 0;        // fp4 strips per wave per step
  constexpr int S_DMA = kFp4 ? NSTRIP / NW : 0;        // E8M0 strips per wave per step
  // E8M0 bytes: one 256-byte slot per strip (a wave's dword DMA covers 64 lanes x 4 bytes; lanes
  // 0-15 carry the strip's 64 bytes, the rest repeat them into the slot's unused tail)
  constexpr int kSE8 = NSTRIP * 256;
  // AT (p.a_tiled): A in operand order, and for symmetric int4 the row-sum seeds travel by LDS-DMA
  // (one dword per row, kSeedB bytes per stage) instead of four MFMAs per wave and step
  constexpr bool kSeedL = AT && MODE == kPSym;
  constexpr int kSeedOff = kFp4 ? S::kA + S::kB + kSE8 : S::kBytes;
  constexpr int kSeedB = kSeedL ? BM * 4 : 0;
  constexpr int kStage = kSeedOff + kSeedB;
  static_assert(!kFp4 || B_DMA * NW == NSTRIP, "fp4 strips / waves");
  constexpr int B_PER = kFp4 ? 0 : NSTRIP * 64 / T;    // int4 16-byte chunks per thread per step
  static_assert(kFp4 || B_PER * T == NSTRIP * 64, "int4 chunks / threads");
  // vector-memory operations every wave issues per step (all unconditional, so one count holds)
  constexpr int NOPS = (kFp4 ? S_DMA + A_PER + B_DMA : A_PER + B_PER + 1 + (MODE == kPAsym ? 1 : 0)) + (kSeedL ? 1 : 0);

  __shared__ __align__(16) unsigned char st0[kStage];
  __shared__ __align__(16) unsigned char st1[kStage];
  __shared__ __align__(16) unsigned char st2[kStage];
  auto stage = [&](auto I) __attribute__((always_inline)) -> unsigned char* {
    if constexpr (decltype(I)::value == 0) return st0;
    else if constexpr (decltype(I)::value == 1) return st1;
    else return st2;
  };

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  int bx = (int)blockIdx.x, by = (int)blockIdx.y;
  int64_t expert = 0;
  if (p.sorted_ids) {
    // Grouped: tiles in XCD order. Workgroup i runs on XCD i % 8; each XCD takes a contiguous
    // range of the tiles that hold rows (row tiles below ntp, every column tile of each), so a
    // row tile's A rows and an expert's weight strips, read by the neighbouring tiles, stay in one
    // L2 (in grid order a row tile's column tiles and an expert's row tiles sat on different XCDs).
    // The grid is a multiple of 8 workgroups, so every XCD has the same number of slots.
    const int gx = (int)gridDim.x;
    const int i = by * gx + bx;
    const int used = ((*p.ntp) + BM - 1) / BM * gx;
    const int share = (used + 7) / 8;
    const int v = (i & 7) * share + (i >> 3);
    if ((i >> 3) >= share || v >= used) return;
    bx = v % gx;
    by = v / gx;
    expert = p.expert_ids[(uint32_t)(by * BM) / (uint32_t)p.bm];  // padded rows < 2^31
  }
  const int64_t blk_row0 = (int64_t)by * BM;
  const int N = (int)p.N, K = (int)p.K, KT = (int)p.KT;
  const int nstrips = N / kTileN;
  const int gshift = 31 - __builtin_clz((unsigned)(p.group >= kTileK ? p.group / kTileK : 1));

  // global strip of LDS strip s: wave wn computes LDS strips [wn*NSB, wn*NSB + NSB); with silu the
  // first half of each wave's strips are gate strips and the second half the matching up strips
  auto gstrip = [&](int s, bool& ok) __attribute__((always_inline)) {
    int gs;
    if (p.silu) {
      constexpr int hj = NSB / 2;
      const int j = s % NSB;
      const int h = bx * (NSTRIP / 2) + (s / NSB) * hj + (j < hj ? j : j - hj);
      gs = j < hj ? h : nstrips / 2 + h;
      ok = h < nstrips / 2;
    } else {
      gs = bx * NSTRIP + s;
      ok = gs < nstrips;
    }
    return ok ? gs : nstrips - 1;
  };

  const uint4* wt = p.wt + (size_t)(expert * p.w_expert_tiles) * 64;
  constexpr int kEsz = kFp4 ? 1 : 2;
  const unsigned char* scales = reinterpret_cast<const unsigned char*>(p.scales) + (size_t)(expert * p.s_expert_stride) * kEsz;
  const int32_t* zeros = p.zeros ? p.zeros + expert * p.z_expert_stride : nullptr;
  const int ngroups = K >> (31 - __builtin_clz((unsigned)p.group));
  const BufRsrc rs_a = make_rsrc(p.xq, 0xffffffffu);
  const BufRsrc rs_w = make_rsrc(wt, (uint32_t)((size_t)nstrips * KT * kTileBytes));
  const BufRsrc rs_s = make_rsrc(scales, (uint32_t)((size_t)(kFp4 ? K / 32 : ngroups) * N * kEsz));
  const BufRsrc rs_z = make_rsrc(zeros, zeros ? (uint32_t)((size_t)ngroups * (N / 8) * 4) : 0u);

  // ---- per-lane source offsets (fixed across K steps; the step adds a scalar offset)
  // A block b = wave + i*NW of a step is row block b/2, half b%2; lane l reads row (l & 15) of it,
  // bytes [64*half + 16*(l >> 4), +16) of the step's 128
  // AT: block b's 1 KiB sits whole in the tiled codes (row blocks past M read the last one)
  uint32_t a_voff[A_PER];
  const int64_t nblk16 = (p.M + 15) / 16;
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int b = wave + i * NW;
    if constexpr (AT) {
      int64_t rbg = blk_row0 / 16 + (b >> 1);
      rbg = rbg < nblk16 ? rbg : nblk16 - 1;
      a_voff[i] = (uint32_t)((rbg * KT * 2 + (b & 1)) * 1024 + lane * 16);
    } else {
      int64_t ar;
      const bool ok = lrow_source(p, blk_row0 + (b >> 1) * 16 + (lane & 15), ar);
      a_voff[i] = (uint32_t)((ok ? ar : 0) * p.ldx) + (b & 1) * 64 + 16 * (lane >> 4);
    }
  }
  // seeds: wave w copies rows 64 (w % (BM / 64)) + lane of the tile (waves past BM / 64 copy the same
  // rows again, so every wave issues one DMA per step and one vmcnt count holds)
  constexpr int kSeedW = BM / 64 > 0 ? BM / 64 : 1;
  const BufRsrc rs_seed = make_rsrc(p.seeds, kSeedL ? (uint32_t)((size_t)KT * p.seeds_ld * 4) : 0u);
  uint32_t seed_voff = 0;
  if constexpr (kSeedL) {
    int64_t sr = blk_row0 + 64 * (wave % kSeedW) + lane;
    sr = sr < p.seeds_ld ? sr : p.seeds_ld - 1;
    seed_voff = (uint32_t)(sr * 4);
  }
  // The epilogue's rows: one per thread, its source looked up in the same round trip as the A
  // rows' and its act scale loaded ahead of step 0's loads; both go to LDS at the end of the
  // prologue, so the epilogue starts with no load to wait for (grouped rows had three dependent
  // ones there: ntp, sorted id, act scale). LDS rather than registers: the int4 tiles already use
  // nearly every VGPR through the K loop.
  __shared__ float e_sc[BM];
  __shared__ int e_ok[BM];
  const int er = (int)threadIdx.x;
  float er_sc = 0.f;
  bool er_ok = false;
  if (er < BM) {
    int64_t ar;
    er_ok = lrow_source(p, blk_row0 + er, ar);
    er_sc = p.act_scales[er_ok ? ar : 0];
  }
  // fp4: wave strip s = wave + i*NW; E8M0 dword of DMA lane m (< 16): 32-block m >> 2, channels
  // 4 * (m & 3) .. +3 (LDS byte (m >> 2) * 16 + channel = the MFMA lane whose scale it is)
  int b_gs[kFp4 ? B_DMA : 1];
  uint32_t e_voff[kFp4 ? S_DMA : 1];
  if constexpr (kFp4) {
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) {
      bool ok;
      b_gs[i] = gstrip(wave + i * NW, ok);
      const int m = lane & 15;
      e_voff[i] = (uint32_t)((m >> 2) * N + b_gs[i] * 16 + (m & 3) * 4);
    }
  }
  // int4: chunk c = tid + i*T is lane c & 63 of strip c >> 6; scales 2 chunks of 16 B per strip,
  // zero words 8 B per strip (threads past the counts load duplicates of the last and write the
  // same bytes again)
  uint32_t b_voff[kFp4 ? 1 : B_PER];
  constexpr int S_CHUNKS = NSTRIP * 2;
  const int sc_c = (int)threadIdx.x < S_CHUNKS ? (int)threadIdx.x : S_CHUNKS - 1;
  const int z_c = (int)threadIdx.x < NSTRIP ? (int)threadIdx.x : NSTRIP - 1;
  uint32_t s_voff = 0, z_voff = 0;
  if constexpr (!kFp4) {
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int c = (int)threadIdx.x + i * T;
      bool ok;
      const int gs = gstrip(c >> 6, ok);
      b_voff[i] = (uint32_t)(((size_t)gs * KT * 64 + (c & 63)) * 16);
    }
    bool ok;
    s_voff = (uint32_t)((gstrip(sc_c >> 1, ok) * 16 + (sc_c & 1) * 8) * 2);
    z_voff = (uint32_t)(gstrip(z_c, ok) * 2 * 4);
  }

  // int4 register sets, one per stage index (two are live at a time)
  v4u rbw[3][kFp4 ? 1 : B_PER];
  uint4 rsc[3];
  uint2 rzp[3];

  // loads of K step kt into stage I (DMA) / register set I (int4 weights, scales, zeros)
  // part: 1 = the A DMAs (and fp4 strips / E8M0 bytes), 2 = the int4 weight, scale and zero loads
  auto issue = [&](auto I, int kt, int part = 3) __attribute__((always_inline)) {
    constexpr int R = decltype(I)::value;
    unsigned char* st = stage(I);
    if constexpr (kFp4) {
#pragma unroll
      for (int i = 0; i < S_DMA; ++i)
        lds_dma4(rs_s, st + S::kA + S::kB + (wave + i * NW) * 256, e_voff[i],
                 (uint32_t)__builtin_amdgcn_readfirstlane(kt * 4 * N));
    }
    const uint32_t so_a = (uint32_t)__builtin_amdgcn_readfirstlane(AT ? kt * 2048 : kt * kTileK);
    if (part & 1) {
#pragma unroll
      for (int i = 0; i < A_PER; ++i)
        lds_dma16(rs_a, st + (wave + i * NW) * 1024, a_voff[i], so_a);
      if constexpr (kSeedL)
        lds_dma4(rs_seed, st + kSeedOff + (wave % kSeedW) * 256, seed_voff,
                 (uint32_t)__builtin_amdgcn_readfirstlane(kt * (int)p.seeds_ld * 4));
    }
    if constexpr (kFp4) {
#pragma unroll
      for (int i = 0; i < B_DMA; ++i)
        lds_dma16(rs_w, st + S::kA + (wave + i * NW) * 1024, (uint32_t)lane * 16,
                    (uint32_t)__builtin_amdgcn_readfirstlane((b_gs[i] * KT + kt) * kTileBytes));
    } else if (part & 2) {
      const uint32_t so_b = (uint32_t)__builtin_amdgcn_readfirstlane(kt * kTileBytes);
#pragma unroll
      for (int i = 0; i < B_PER; ++i) rbw[R][i] = bload128v(rs_w, b_voff[i], so_b);
      const int g = kt >> gshift;
      rsc[R] = bload128(rs_s, s_voff, (uint32_t)__builtin_amdgcn_readfirstlane(g * N * 2));
      if (MODE == kPAsym) rzp[R] = bload64(rs_z, z_voff, (uint32_t)__builtin_amdgcn_readfirstlane(g * (N / 8) * 4));
    }
  };
  // int4: unpack register set R into stage I
  auto commit = [&](auto I, auto R_) __attribute__((always_inline)) {
    if constexpr (!kFp4) {
      constexpr int R = decltype(R_)::value;
      unsigned char* st = stage(I);
      unsigned char* sb = st + S::kA;
#pragma unroll
      for (int i = 0; i < B_PER; ++i) {
        const int c = (int)threadIdx.x + i * T;
        const int s = c >> 6, l = c & 63;
        const v8i u = unpack_tile_int4(make_uint4(rbw[R][i].x, rbw[R][i].y, rbw[R][i].z, rbw[R][i].w));
        *reinterpret_cast<uint4*>(sb + ((s * 2 + 0) * 64 + l) * 16) = make_uint4(u[0], u[1], u[2], u[3]);
        *reinterpret_cast<uint4*>(sb + ((s * 2 + 1) * 64 + l) * 16) = make_uint4(u[4], u[5], u[6], u[7]);
      }
      *reinterpret_cast<uint4*>(st + S::kA + S::kB + sc_c * 16) = rsc[R];
      if (MODE == kPAsym) *reinterpret_cast<uint2*>(st + S::kA + S::kB + S::kS + z_c * 8) = rzp[R];
    }
  };

  v4f acc[RB][NSB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < NSB; ++j) acc[rb][j] = v4f{0.f, 0.f, 0.f, 0.f};
  const v4f zero4 = v4f{0.f, 0.f, 0.f, 0.f};

  // per-lane LDS offsets of this wave's operands within a stage; the empty asm keeps each in one
  // VGPR so every read is that VGPR plus an immediate
  uint32_t oa = (uint32_t)(wm * RB * 2048 + lane * 16);
  uint32_t ob = (uint32_t)(S::kA + wn * NSB * (kFp4 ? 1024 : 2048) + lane * 16);
  uint32_t os = (uint32_t)(S::kA + S::kB + (kFp4 ? wn * NSB * 256 + lane : (wn * NSB * 16 + (lane & 15)) * 2));
  uint32_t oz = (uint32_t)(S::kA + S::kB + S::kS + (wn * NSB * 2 + ((lane & 15) >> 3)) * 4);
  asm volatile("" : "+v"(oa), "+v"(ob), "+v"(os), "+v"(oz));
  const int zsh = 4 * (lane & 7);

  // MFMA work of one K step from stage I (operands read one row block / strip ahead of their
  // MFMAs). mid(i) runs right after the MFMAs of int4 strip i (i = 0, 1) or MXFP4 row block i, so
  // its work (the loads of a later step, the unpack of the next step's weights) overlaps MFMAs in
  // flight.
  auto compute = [&](auto I, auto mid) __attribute__((always_inline)) {
    const unsigned char* st = stage(I);
    if constexpr (kFp4) {
      uint4 braw[NSB];
      int sbyte[NSB];
#pragma unroll
      for (int j = 0; j < NSB; ++j) {
        braw[j] = *reinterpret_cast<const uint4*>(st + ob + j * 1024);
        sbyte[j] = (int)st[os + j * 256];
      }
      v8i a0 = lds_operand(st + oa, 0);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        v8i a1;
        if (rb + 1 < RB) a1 = lds_operand(st + oa + (rb + 1) * 2048, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < NSB; ++j) acc[rb][j] = mfma_f8f4_sb(a0, fp4_operand(braw[j]), acc[rb][j], sbyte[j]);
        mid(rb);
        if (rb + 1 < RB) a0 = a1;
      }
    } else {
      v8i a[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) a[rb] = lds_operand(st + oa + rb * 2048, 0);
      v4f pre[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {  // symmetric: -R/2; zero points: +R/2
        if constexpr (kSeedL)
          pre[rb] = *reinterpret_cast<const v4f*>(st + kSeedOff + (wm * RB * 16 + rb * 16 + 4 * (lane >> 4)) * 4);
        else
          pre[rb] = mfma_f8f8(a[rb], splat8(MODE == kPSym ? 0xB0B0B0B0u : kE4M3Half4), zero4);
      }
      v4f cp[RB];
      float scp = 0.f, cfp = 0.f;
      v8i bn = lds_operand(st + ob, 0);
      float scn = f16_to_f32(*reinterpret_cast<const uint16_t*>(st + os));
      uint32_t zn = MODE == kPAsym ? *reinterpret_cast<const uint32_t*>(st + oz) : 0u;
#pragma unroll
      for (int j = 0; j <= NSB; ++j) {
        v4f cj[RB];
        float scj = 0.f, cfj = 0.f;
        if (j < NSB) {
          const v8i b = bn;
          scj = scn;
          if (MODE == kPAsym) cfj = 15.0f - 2.0f * (float)((zn >> zsh) & 15u);
          if (j + 1 < NSB) {
            bn = lds_operand(st + ob + (j + 1) * 2048, 0);
            scn = f16_to_f32(*reinterpret_cast<const uint16_t*>(st + os + (j + 1) * 32));
            if (MODE == kPAsym) zn = *reinterpret_cast<const uint32_t*>(st + oz + (j + 1) * 8);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) cj[rb] = mfma_f8f8(a[rb], b, MODE == kPSym ? pre[rb] : zero4);
          if (j < 2) mid(j);
        }
        if (j > 0) {
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              if (MODE == kPSym)
                acc[rb][j - 1][r] += scp * cp[rb][r];
              else
                acc[rb][j - 1][r] += scp * (cp[rb][r] + cfp * pre[rb][r]);
            }
          // issue the previous strip's scale FMAs between this strip's MFMAs (one MFMA, then four
          // VALU ops), so they run while the matrix pipe works instead of after it
          if (j < NSB) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
              __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
            }
          }
        }
        if (j < NSB) {
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) cp[rb] = cj[rb];
          scp = scj;
          cfp = cfj;
        }
      }
    }
  };

  // one pipelined step kt (stage C = kt % 3): loads of kt+2, MFMAs of kt, int4 registers of kt+1
  // to LDS, wait for kt+1's loads, barrier. The loads of kt+2 are issued between the step's MFMAs
  // instead of ahead of them all (int4: the weight loads after the first strip's, ahead of the
  // unpack of kt+1's weights, and the A DMAs after the second's; MXFP4: all after the second row
  // block's): at the top of the step every wave's loads would meet in the address unit's queue
  // while the step's first MFMAs wait (1-4% on configs[3] and configs[5] shapes). The weight
  // registers go first because the unpack one step later waits on them, while the A DMAs are only
  // waited for at the end of the next step (weights first: configs[3] 2-8% faster, MoE T=4096 2%).
  auto step = [&](auto C, int kt) __attribute__((always_inline)) {
    constexpr int c = decltype(C)::value, n1 = (c + 1) % 3, n2 = (c + 2) % 3;
    static_assert(kFp4 || NSB >= 2, "int4 steps issue their loads after strips 0 and 1");
    if constexpr (kFp4) {
      compute(C, [&](int rb) __attribute__((always_inline)) {
        if (rb == 1) issue(IC<n2>{}, kt + 2);
      });
    } else {
      compute(C, [&](int j) __attribute__((always_inline)) {
        if (j == 0) {
          issue(IC<n2>{}, kt + 2, 2);
          commit(IC<n1>{}, IC<n1>{});
        } else {
          issue(IC<n2>{}, kt + 2, 1);
        }
      });
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_lgkm0<NOPS>();
    __builtin_amdgcn_s_barrier();
  };
  // the same step near the end of K: loads only while steps remain, a full wait otherwise
  auto step_tail = [&](auto C, int kt) __attribute__((always_inline)) {
    constexpr int c = decltype(C)::value, n1 = (c + 1) % 3, n2 = (c + 2) % 3;
    if (kt >= KT) return;
    const bool more = kt + 2 < KT;
    if (more) issue(IC<n2>{}, kt + 2);
    compute(C, [&](int j) __attribute__((always_inline)) {
      if (j == 0 && kt + 1 < KT) commit(IC<n1>{}, IC<n1>{});
    });
    if (more) wait_vm_lgkm0<NOPS>();
    else wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();
  };

  // prologue: steps 0 and 1 in flight, step 0 in LDS. The epilogue rows' loads above are older
  // than both, so the counted wait covers them; their LDS writes land before the first step's
  // barrier (its wait takes lgkmcnt to 0), long before the epilogue reads them.
  issue(IC<0>{}, 0);
  issue(IC<1>{}, 1);
  commit(IC<0>{}, IC<0>{});
  wait_vm_lgkm0<NOPS>();
  if (er < BM) {
    e_sc[er] = er_sc;
    e_ok[er] = er_ok ? 1 : 0;
  }
  __builtin_amdgcn_s_barrier();
  int kt = 0;
  for (; kt + 4 < KT; kt += 3) {
    step(IC<0>{}, kt);
    step(IC<1>{}, kt + 1);
    step(IC<2>{}, kt + 2);
  }
  step_tail(IC<0>{}, kt);
  step_tail(IC<1>{}, kt + 1);
  step_tail(IC<2>{}, kt + 2);
  step_tail(IC<0>{}, kt + 3);
  step_tail(IC<1>{}, kt + 4);

  // epilogue: lane holds rows 4*(lane>>4)+r of each row block, channel (lane & 15) of each strip
  const int64_t row0 = blk_row0 + (int64_t)wm * RB * 16;
  float e_rsc[RB][4];
  uint32_t e_valid = 0;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int lr = wm * RB * 16 + rb * 16 + 4 * (lane >> 4) + r;
      e_rsc[rb][r] = e_sc[lr];
      e_valid |= (e_ok[lr] ? 1u : 0u) << (rb * 4 + r);
    }
  // the stages are free: the last step's barrier followed every wave's reads and every DMA
  constexpr int kScr = 16 * (NSB * 16 * 4 + 16);  // one wave's row-major tile, f32 worst case
  constexpr int kWps = kStage / kScr;
  static_assert(3 * kWps >= NW, "epilogue scratch");
  unsigned char* scr = (wave < kWps ? st0 : wave < 2 * kWps ? st1 : st2) + (wave % kWps) * kScr;
  store_tile_scaled(p, acc, e_rsc, e_valid, row0, lane,
                    [&](int j, bool& ok) __attribute__((always_inline)) { return gstrip(wn * NSB + j, ok); }, scr);
}

template <int WM, int WN, int RB, int NSB, int MODE, bool AT = false>
static int launch_dma_cfg_at(const GemmArgs& p, int64_t row_tiles, hipStream_t stream) {
  constexpr int BN = WN * NSB * 16;
  const int64_t ncols = p.silu ? p.N / 2 : p.N;
  const int64_t colw = p.silu ? BN / 2 : BN;
  const int64_t gx = (ncols + colw - 1) / colw;
  int64_t gy = row_tiles;
  if (p.sorted_ids)  // the grouped tile order needs a multiple of 8 workgroups
    while ((gx * gy) % 8) ++gy;
  const dim3 grid((unsigned)gx, (unsigned)gy);
  const dim3 block(WM * WN * 64);
  auto kern = gemm_dma_kernel<WM, WN, RB, NSB, MODE, AT>;
  hipLaunchKernelGGL(kern, grid, block, 0, stream, p);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

// dense calls with p.a_tiled take the tiled-A instantiation (grouped ones: launch_dma_modes_grouped)
template <int WM, int WN, int RB, int NSB, int MODE>
static int launch_dma_cfg(const GemmArgs& p, int64_t row_tiles, hipStream_t stream) {
  if (p.a_tiled) return launch_dma_cfg_at<WM, WN, RB, NSB, MODE, true>(p, row_tiles, stream);
  return launch_dma_cfg_at<WM, WN, RB, NSB, MODE, false>(p, row_tiles, stream);
}

template <int WM, int WN, int RB, int NSB>
static int launch_dma_modes(const GemmArgs& p, int mode, int64_t row_tiles, hipStream_t stream) {
  if (mode == kPSym) return launch_dma_cfg<WM, WN, RB, NSB, kPSym>(p, row_tiles, stream);
  if (mode == kPAsym) return launch_dma_cfg<WM, WN, RB, NSB, kPAsym>(p, row_tiles, stream);
  return launch_dma_cfg<WM, WN, RB, NSB, kPE8M0>(p, row_tiles, stream);
}
// grouped tiles: A rows gathered through the sorted ids, or (p.a_tiled, symmetric int4, A rows at
// their padded positions: gemm2) the padded rows' codes in operand order with their seeds
template <int WM, int WN, int RB, int NSB>
static int launch_dma_modes_grouped(const GemmArgs& p, int mode, int64_t row_tiles, hipStream_t stream) {
  if (mode == kPSym && p.a_tiled) return launch_dma_cfg_at<WM, WN, RB, NSB, kPSym, true>(p, row_tiles, stream);
  if (mode == kPSym) return launch_dma_cfg_at<WM, WN, RB, NSB, kPSym>(p, row_tiles, stream);
  if (mode == kPAsym) return launch_dma_cfg_at<WM, WN, RB, NSB, kPAsym>(p, row_tiles, stream);
  return launch_dma_cfg_at<WM, WN, RB, NSB, kPE8M0>(p, row_tiles, stream);
}

// Formats and shapes as launch_prefill_lds, plus at least three K steps (the pipeline's depth).
// bm_rows: rows per workgroup the caller requires (grouped: 64 or 128; 0 for dense).
int launch_prefill_dma(const GemmArgs& p, int64_t rows_to_cover, int bm_rows, hipStream_t stream) {
  int mode;
  if (p.wfmt == kInt4 && p.sfmt == kScaleF16 && p.group % kTileK == 0)
    mode = p.zeros ? kPAsym : kPSym;
  else if (p.wfmt == kE2M1 && p.sfmt == kScaleE8M0)
    mode = kPE8M0;
  else
    return kErrUnsupported;
  if (p.silu && (p.N / kTileN) % 2) return kErrUnsupported;
  if (p.K % kTileK || p.KT < 3) return kErrUnsupported;
  if (p.sorted_ids && bm_rows != 64 && bm_rows != 128) return kErrUnsupported;
  if ((int64_t)p.N * p.KT * 64 >= (int64_t)1 << 31) return kErrUnsupported;
  if (p.ldx % 16) return kErrUnsupported;  // A rows are read in 16-byte pieces
  // W4A8_PREFILL_DMA=0 leaves every call to the register-staged kernel (A/B measurements)
  static const bool enabled = [] {
    const char* e = getenv("W4A8_PREFILL_DMA");
    return !(e && atoi(e) == 0);
  }();
  if (!enabled) return kErrUnsupported;
  // Tiles (waves WM x WN, wave tile RB x NSB blocks of 16): the largest whose three stages fit
  // the 160 KiB of LDS and whose registers fit two waves per SIMD. MXFP4 keeps its weights as fp4
  // in LDS and its accumulators are the only per-step state, so it takes 64 x 128 wave tiles
  // (256 x 256 per workgroup: a quarter less LDS read per MFMA than 64 x 64); int4 holds the
  // unpacked fp8 weights plus the partials of its per-group scaling and stays at 64 x 64.
  if (p.a_tiled && (p.sorted_ids ? (mode != kPSym || p.a_by_token != 0) : (bm_rows != 0 || mode == kPAsym)))
    return kErrUnsupported;
  if (bm_rows == 64) return launch_dma_modes_grouped<2, 4, 2, 2>(p, mode, (rows_to_cover + 63) / 64, stream);
  if (bm_rows == 128) return launch_dma_modes_grouped<2, 4, 4, 4>(p, mode, (rows_to_cover + 127) / 128, stream);
  // Grids of at most half a workgroup per CU take smaller tiles. int4: 128 x 128 when that gives
  // 192 or more workgroups, else 64 x 128 (the configs[2] M=512 calls, M=1024 on 4096-wide
  // weights): K=4096 N=6144 M=512 39.5 -> 29.9 us, K=4096 N=4096 M=1024 42.4 -> 32.4 us, K=14336
  // N=4096 M=1024 126.7 -> 94.2 us (128 x 128); K=4096 N=4096 M=512 50.7 -> 21.8 us, K=14336
  // N=4096 M=512 146.9 -> 64.6 us (64 x 128; 128 x 128 gave 28.2 and 85.5 there). A grid of 144
  // (K=4096 N=6144 M=768) measured slower with 128 x 128 tiles (55.5 against 48.2 us) and keeps
  // 256 x 128. MXFP4 (256 x 256) takes 64 x 128 tiles. The tile shape does not change any
  // output's arithmetic.
  const int64_t ncols = p.silu ? p.N / 2 : p.N;
  const int64_t bn_default = mode == kPE8M0 ? 256 : 128;
  const int64_t g_default = (ncols + bn_default - 1) / bn_default * ((rows_to_cover + 255) / 256);
  if (mode != kPE8M0 && g_default <= 128) {
    if ((ncols + 127) / 128 * ((rows_to_cover + 127) / 128) >= 192)
      return launch_dma_modes<4, 2, 2, 4>(p, mode, (rows_to_cover + 127) / 128, stream);
    return launch_dma_modes<2, 4, 2, 2>(p, mode, (rows_to_cover + 63) / 64, stream);
  }
  // a default grid of 257-384 workgroups runs one and a half rounds of the CUs; 128 x 128 tiles
  // even it out (K=4096 N=6144 M=2048: 384 workgroups, 96.5 -> 91.6 us; a grid of 576 measured
  // slower that way, 143.3 -> 146.7 us)
  if (mode != kPE8M0 && g_default > 256 && g_default <= 384)
    return launch_dma_modes<4, 2, 2, 4>(p, mode, (rows_to_cover + 127) / 128, stream);
  if (mode == kPE8M0 && g_default <= 128)
    return launch_dma_modes<2, 4, 2, 2>(p, mode, (rows_to_cover + 63) / 64, stream);
  if (mode == kPE8M0) return launch_dma_cfg<4, 2, 4, 8, kPE8M0>(p, (rows_to_cover + 255) / 256, stream);
  return launch_dma_modes<4, 2, 4, 4>(p, mode, (rows_to_cover + 255) / 256, stream);
}

}  // namespace w4a8

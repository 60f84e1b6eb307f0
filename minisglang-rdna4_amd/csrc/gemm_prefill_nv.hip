// NVFP4 prefill / grouped GEMM on the fp16 MFMA (v_mfma_f32_16x16x32_f16).
//
// Same contract as the other prefill kernels (python/minisgl/quant/kernels.py:1686-1734, 744-773,
// with NVFP4's two-level scale of :518-559): y[m,n] = s_m * g_n * sum_k e4m3(x[m,k]) *
// (e2m1(w[n,k]) * e4m3(sb[k/16, n])), f32 accumulation, g_n the per-channel f32 global.
//
// NVFP4's block scales cover 16 elements and are e4m3 (4 significant bits), so the scaled fp8 x
// fp4 MFMA (one power-of-two scale per 32 elements) cannot take them. But every dequantized weight
// e2m1 * e4m3 is exact in fp16: at most 6 significant bits, magnitudes 2^-10 .. 2688, all inside
// fp16's normal range; and so is every e4m3 activation code. The fp16 MFMA at half the fp8 rate
// therefore computes the same products exactly, with one f32 accumulator per output over all of K;
// the global and the activation scale are applied once in the epilogue.
//
// Per K step of 128 (one W4 tile per strip):
//   A (BM x 128 fp8) goes to LDS by LDS-DMA in operand order, three stages deep (as in
//     gemm_prefill_dma.hip); each wave converts its fragments to fp16 in registers
//     (v_cvt_scalef32_pk_f16_fp8, two values per instruction).
//   B: each thread loads one lane of one strip's fp4 tile (16 bytes, two 16-element blocks) and
//     the two e4m3 block scales, converts the codes to fp16 (v_cvt_scalef32_pk_f16_fp4), scales
//     them with packed fp16 multiplies (exact) and writes them to LDS in MFMA operand order, two
//     stages deep (the registers of step k+1 are written while step k computes).
// K order inside a step: lane group q of the A tile holds K [16q, 16q+16) and [64+16q, 64+16q+16)
// (the fp8 operand order); sub-step s of the four fp16 MFMAs takes bytes [8s, 8s+8) of those 32,
// i.e. K = 64*(s>>1) + 16q + 8*(s&1) + e. B is written so that the same (s, q, e) holds the same K.
#include <cstdlib>

#include "prefill.h"

namespace w4a8 {

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// 8 fp8 codes (two dwords, byte order) -> 8 fp16 values, exact
__device__ __forceinline__ v8h fp8x8_to_f16(uint32_t lo, uint32_t hi) {
  const v2h p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false);
  const v2h p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true);
  const v2h p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false);
  const v2h p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true);
  const auto l = __builtin_shufflevector(p0, p1, 0, 1, 2, 3);
  const auto h = __builtin_shufflevector(p2, p3, 0, 1, 2, 3);
  return __builtin_shufflevector(l, h, 0, 1, 2, 3, 4, 5, 6, 7);
}

// byte B of w: two e2m1 codes (low nibble first) -> fp16, times the block scale pair sc (exact)
template <int B>
__device__ __forceinline__ v2h fp4x2_scaled(uint32_t w, v2h sc) {
  return __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, B) * sc;
}

__device__ __forceinline__ uint32_t h2_bits(v2h v) { return __builtin_bit_cast(uint32_t, v); }

// the 16 codes of one 16-element block (dwords d0, d1) -> two 16-byte operand chunks (K 0..7, 8..15)
__device__ __forceinline__ void block16(uint32_t d0, uint32_t d1, v2h sc, uint4& lo, uint4& hi) {
  lo = make_uint4(h2_bits(fp4x2_scaled<0>(d0, sc)), h2_bits(fp4x2_scaled<1>(d0, sc)),
                  h2_bits(fp4x2_scaled<2>(d0, sc)), h2_bits(fp4x2_scaled<3>(d0, sc)));
  hi = make_uint4(h2_bits(fp4x2_scaled<0>(d1, sc)), h2_bits(fp4x2_scaled<1>(d1, sc)),
                  h2_bits(fp4x2_scaled<2>(d1, sc)), h2_bits(fp4x2_scaled<3>(d1, sc)));
}

}  // namespace

template <int WM, int WN, int RB, int NSB>
__global__ void __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_nv_kernel(const GemmArgs p) {
  constexpr int T = WM * WN * 64, NW = WM * WN;
  constexpr int BM = WM * RB * 16, BN = WN * NSB * 16;
  constexpr int NSTRIP = BN / 16;
  constexpr int kA = BM * 128;          // fp8 A in operand order: 2 KiB per 16-row block
  constexpr int kB = NSTRIP * 4096;     // fp16 B: [strip][sub-step 4][lane 64][16 bytes]
  constexpr int A_PER = (BM / 8) / NW;  // A 1 KiB blocks per wave per step
  static_assert(A_PER * NW == BM / 8, "A blocks / waves");
  constexpr int B_PER = NSTRIP * 64 / T;  // fp4 tile lanes per thread per step
  static_assert(B_PER * T == NSTRIP * 64, "fp4 lanes / threads");
  // vector-memory operations every wave issues per step: A DMAs, fp4 loads, two scale bytes each
  constexpr int NOPS = A_PER + 3 * B_PER;
  static_assert(3 * kA + 2 * kB <= 160 * 1024, "LDS");

  // every stage its own array, every stage index a compile-time constant (the K loop is unrolled
  // by six): the compiler then tells the stages apart, so the B writes of step k+1 do not wait for
  // the A DMAs of step k+2
  __shared__ __align__(16) unsigned char sa0[kA];
  __shared__ __align__(16) unsigned char sa1[kA];
  __shared__ __align__(16) unsigned char sa2[kA];
  __shared__ __align__(16) unsigned char sb0[kB];
  __shared__ __align__(16) unsigned char sb1[kB];
  auto astage = [&](auto I) __attribute__((always_inline)) -> unsigned char* {
    if constexpr (decltype(I)::value == 0) return sa0;
    else if constexpr (decltype(I)::value == 1) return sa1;
    else return sa2;
  };
  auto bstage = [&](auto I) __attribute__((always_inline)) -> unsigned char* {
    if constexpr (decltype(I)::value == 0) return sb0;
    else return sb1;
  };

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

  // global strip of LDS strip s (silu: each wave's first NSB/2 strips are gate, the rest up)
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
  const unsigned char* scales = reinterpret_cast<const unsigned char*>(p.scales) + (size_t)(expert * p.s_expert_stride);
  const int32_t* glob = p.zeros + expert * p.z_expert_stride;
  const BufRsrc rs_a = make_rsrc(p.xq, 0xffffffffu);
  const BufRsrc rs_w = make_rsrc(wt, (uint32_t)((size_t)nstrips * KT * kTileBytes));
  const BufRsrc rs_s = make_rsrc(scales, (uint32_t)((size_t)(K / 16) * N));

  // A block b = wave + i*NW of a step is row block b/2, half b%2; lane l reads row (l & 15) of it,
  // bytes [64*half + 16*(l >> 4), +16) of the step's 128
  uint32_t a_voff[A_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int b = wave + i * NW;
    int64_t ar;
    const bool ok = lrow_source(p, blk_row0 + (b >> 1) * 16 + (lane & 15), ar);
    a_voff[i] = (uint32_t)((ok ? ar : 0) * p.ldx) + (b & 1) * 64 + 16 * (lane >> 4);
  }
  // B: fp4 tile lane c = tid + i*T is lane c & 63 of strip c >> 6; its 16 bytes are the two
  // 16-element blocks 2q', 2q'+1 (q' = lane >> 4) of channel lane & 15; their scale bytes are
  // rows 2q' and 2q'+1 of the step's 8 scale rows
  uint32_t w_voff[B_PER], s_voff[B_PER];
#pragma unroll
  for (int i = 0; i < B_PER; ++i) {
    const int c = (int)threadIdx.x + i * T;
    bool ok;
    const int gs = gstrip(c >> 6, ok);
    w_voff[i] = (uint32_t)(((size_t)gs * KT * 64 + (c & 63)) * 16);
    s_voff[i] = (uint32_t)(2 * ((c & 63) >> 4) * N + gs * 16 + (c & 15));
  }

  v4u rw[3][B_PER];
  uint32_t rs0[3][B_PER], rs1[3][B_PER];

  auto issue = [&](auto I, int kt) __attribute__((always_inline)) {
    constexpr int R = decltype(I)::value;
    unsigned char* st = astage(I);
    const uint32_t so_a = (uint32_t)__builtin_amdgcn_readfirstlane(kt * kTileK);
#pragma unroll
    for (int i = 0; i < A_PER; ++i) lds_dma16(rs_a, st + (wave + i * NW) * 1024, a_voff[i], so_a);
    const uint32_t so_w = (uint32_t)__builtin_amdgcn_readfirstlane(kt * kTileBytes);
    const uint32_t so_s = (uint32_t)__builtin_amdgcn_readfirstlane(kt * 8 * N);
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      rw[R][i] = bload128v(rs_w, w_voff[i], so_w);
      rs0[R][i] = bload8(rs_s, s_voff[i], so_s);
      rs1[R][i] = bload8(rs_s, s_voff[i] + N, so_s);
    }
  };
  // B registers of set R -> fp16 operands in B stage BI
  auto commit = [&](auto R_, auto BI) __attribute__((always_inline)) {
    constexpr int R = decltype(R_)::value;
    unsigned char* bs = bstage(BI);
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int c = (int)threadIdx.x + i * T;
      const int s = c >> 6, q = (c & 63) >> 4, cc = c & 15;
      const v2h sc = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(rs0[R][i] | (rs1[R][i] << 8), 1.0f, false);
      const v2h sc0 = __builtin_shufflevector(sc, sc, 0, 0), sc1 = __builtin_shufflevector(sc, sc, 1, 1);
      // block g = 2q + h: sub-steps 2*(g >> 2) and +1, operand lane 16*(g & 3) + cc
      const int sub = 2 * (q >> 1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint4 lo, hi;
        block16(h ? rw[R][i].z : rw[R][i].x, h ? rw[R][i].w : rw[R][i].y, h ? sc1 : sc0, lo, hi);
        const int L = 16 * (2 * (q & 1) + h) + cc;
        *reinterpret_cast<uint4*>(bs + ((s * 4 + sub) * 64 + L) * 16) = lo;
        *reinterpret_cast<uint4*>(bs + ((s * 4 + sub + 1) * 64 + L) * 16) = hi;
      }
    }
  };

  v4f acc[RB][NSB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < NSB; ++j) acc[rb][j] = v4f{0.f, 0.f, 0.f, 0.f};

  uint32_t oa = (uint32_t)(wm * RB * 2048 + lane * 16);
  uint32_t ob = (uint32_t)((wn * NSB * 4 * 64 + lane) * 16);
  asm volatile("" : "+v"(oa), "+v"(ob));

  // the four fp16 sub-steps of a K step from A stage I and B stage BI (each sub-step's B fragments
  // read one sub-step ahead of its MFMAs); mid(s) runs after sub-step s's MFMAs are issued (the
  // next step's B decode and later loads overlap them)
  auto compute = [&](auto I, auto BI, auto mid) __attribute__((always_inline)) {
    const unsigned char* sa = astage(I);
    const unsigned char* bs = bstage(BI);
    v8h bc[NSB], bn[NSB];
#pragma unroll
    for (int j = 0; j < NSB; ++j) bc[j] = *reinterpret_cast<const v8h*>(bs + ob + (j * 4) * 1024);
    uint4 alo[RB], ahi[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      alo[rb] = *reinterpret_cast<const uint4*>(sa + oa + rb * 2048);
      ahi[rb] = *reinterpret_cast<const uint4*>(sa + oa + rb * 2048 + 1024);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s < 3) {
#pragma unroll
        for (int j = 0; j < NSB; ++j) bn[j] = *reinterpret_cast<const v8h*>(bs + ob + (j * 4 + s + 1) * 1024);
      }
      v8h a[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const uint4 w = s < 2 ? alo[rb] : ahi[rb];
        a[rb] = (s & 1) ? fp8x8_to_f16(w.z, w.w) : fp8x8_to_f16(w.x, w.y);
      }
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int j = 0; j < NSB; ++j) acc[rb][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[rb], bc[j], acc[rb][j], 0, 0, 0);
      mid(s);
      if (s < 3) {
#pragma unroll
        for (int j = 0; j < NSB; ++j) bc[j] = bn[j];
      }
    }
  };

  // one pipelined step kt (A stage C = kt % 3, B stage D = kt % 2): MFMAs of kt, B registers of
  // kt+1 to LDS (after the first sub-step's MFMAs), loads of kt+2 (after the second's, rather than
  // ahead of all of them, where every wave's loads would meet in the address unit's queue while the
  // first MFMAs wait: 4-6% at M=4096), wait for kt+1's loads, barrier
  auto step = [&](auto C, auto D, int kt) __attribute__((always_inline)) {
    constexpr int c = decltype(C)::value, d = decltype(D)::value, n1 = (c + 1) % 3, n2 = (c + 2) % 3;
    compute(C, D, [&](int s) __attribute__((always_inline)) {
      if (s == 0) commit(IC<n1>{}, IC<1 - d>{});
      if (s == 1) issue(IC<n2>{}, kt + 2);
    });
    __builtin_amdgcn_sched_barrier(0);
    wait_vm_lgkm0<NOPS>();
    __builtin_amdgcn_s_barrier();
  };
  // the same step near the end of K: loads only while steps remain, a full wait otherwise
  auto step_tail = [&](auto C, auto D, int kt) __attribute__((always_inline)) {
    constexpr int c = decltype(C)::value, d = decltype(D)::value, n1 = (c + 1) % 3, n2 = (c + 2) % 3;
    if (kt >= KT) return;
    const bool more = kt + 2 < KT;
    if (more) issue(IC<n2>{}, kt + 2);
    compute(C, D, [&](int s) __attribute__((always_inline)) {
      if (s == 0 && kt + 1 < KT) commit(IC<n1>{}, IC<1 - d>{});
    });
    if (more) wait_vm_lgkm0<NOPS>();
    else wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();
  };

  issue(IC<0>{}, 0);
  issue(IC<1>{}, 1);
  commit(IC<0>{}, IC<0>{});
  wait_vm_lgkm0<NOPS>();
  __builtin_amdgcn_s_barrier();
  int kt = 0;
  for (; kt + 7 < KT; kt += 6) {
    step(IC<0>{}, IC<0>{}, kt);
    step(IC<1>{}, IC<1>{}, kt + 1);
    step(IC<2>{}, IC<0>{}, kt + 2);
    step(IC<0>{}, IC<1>{}, kt + 3);
    step(IC<1>{}, IC<0>{}, kt + 4);
    step(IC<2>{}, IC<1>{}, kt + 5);
  }
  step_tail(IC<0>{}, IC<0>{}, kt);
  step_tail(IC<1>{}, IC<1>{}, kt + 1);
  step_tail(IC<2>{}, IC<0>{}, kt + 2);
  step_tail(IC<0>{}, IC<1>{}, kt + 3);
  step_tail(IC<1>{}, IC<0>{}, kt + 4);
  step_tail(IC<2>{}, IC<1>{}, kt + 5);
  step_tail(IC<0>{}, IC<0>{}, kt + 6);
  step_tail(IC<1>{}, IC<1>{}, kt + 7);

  // epilogue: the per-channel global, then the row scale and the store (silu pairs strips j and
  // j + NSB/2 inside the wave)
  auto wstrip = [&](int j, bool& ok) __attribute__((always_inline)) { return gstrip(wn * NSB + j, ok); };
#pragma unroll
  for (int j = 0; j < NSB; ++j) {
    bool ok;
    const int gs = wstrip(j, ok);
    const float g = __int_as_float(glob[gs * kTileN + (lane & 15)]);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[rb][j][r] *= g;
  }
  const int64_t row0 = blk_row0 + (int64_t)wm * RB * 16;
  constexpr int kScr = 16 * (NSB * 16 * 4 + 16);
  constexpr int kWps = kA / kScr;
  static_assert(3 * kWps >= NW, "epilogue scratch");
  unsigned char* scr = (wave < kWps ? sa0 : wave < 2 * kWps ? sa1 : sa2) + (wave % kWps) * kScr;
  store_tile(p, acc, row0, lane, wstrip, scr);
}

template <int WM, int WN, int RB, int NSB>
static int launch_nv_cfg(const GemmArgs& p, int64_t row_tiles, hipStream_t stream) {
  constexpr int BN = WN * NSB * 16;
  const int64_t ncols = p.silu ? p.N / 2 : p.N;
  const int64_t colw = p.silu ? BN / 2 : BN;
  const dim3 grid((unsigned)((ncols + colw - 1) / colw), (unsigned)row_tiles);
  hipLaunchKernelGGL((gemm_nv_kernel<WM, WN, RB, NSB>), grid, dim3(WM * WN * 64), 0, stream, p);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

// NVFP4 (e2m1 codes, e4m3 block-16 scales, the f32 global in the zeros slot) with whole 128-K
// steps, at least two of them, and 16-byte aligned activation rows; kErrUnsupported otherwise.
// bm_rows: rows per workgroup the caller requires (grouped: 64 or 128; 0 for dense).
int launch_prefill_nv(const GemmArgs& p, int64_t rows_to_cover, int bm_rows, hipStream_t stream) {
  if (!(p.wfmt == kE2M1 && p.sfmt == kScaleE4M3 && p.group == 16 && p.zeros)) return kErrUnsupported;
  if (p.silu && (p.N / kTileN) % 2) return kErrUnsupported;
  if (p.K % kTileK || p.KT < 2) return kErrUnsupported;
  if (p.sorted_ids && bm_rows != 64 && bm_rows != 128) return kErrUnsupported;
  if ((int64_t)p.N * p.KT * 64 >= (int64_t)1 << 31) return kErrUnsupported;
  if ((p.K / 16) * p.N >= (int64_t)1 << 32) return kErrUnsupported;
  if (p.ldx % 16) return kErrUnsupported;
  // W4A8_PREFILL_NV=0 leaves NVFP4 to the per-wave kernel (A/B measurements)
  static const bool enabled = [] {
    const char* e = getenv("W4A8_PREFILL_NV");
    return !(e && atoi(e) == 0);
  }();
  if (!enabled) return kErrUnsupported;
  // LDS: three A stages and two fp16 B stages; 256 x 128 uses all 160 KiB
  if (bm_rows == 64) return launch_nv_cfg<2, 4, 2, 2>(p, (rows_to_cover + 63) / 64, stream);
  if (bm_rows == 128) return launch_nv_cfg<4, 2, 2, 4>(p, (rows_to_cover + 127) / 128, stream);
  const int64_t ncols = p.silu ? p.N / 2 : p.N;
  if ((ncols + 127) / 128 * ((rows_to_cover + 255) / 256) <= 128)
    return launch_nv_cfg<2, 4, 2, 2>(p, (rows_to_cover + 63) / 64, stream);
  return launch_nv_cfg<4, 2, 4, 4>(p, (rows_to_cover + 255) / 256, stream);
}

}  // namespace w4a8

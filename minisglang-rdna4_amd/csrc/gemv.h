// Skinny-M W4A8 GEMM (decode band, up to 16 rows per row block) on the 16x16x128 f8f6f4 MFMA:
// the kernel template, shared by the launch units gemm_decode.hip (A read per tile from global
// memory), gemv_staged.hip (fp8 A staged in LDS), gemv_fused.hip and gemv_fused_e2m1.hip (bf16/fp16
// A quantized to fp8 in LDS by the kernel itself, so a decode call is one launch), gemv_generic.hip
// (sub-tile groups) and gemv_routed.hip (MoE gemm1 with the router in the prologue).
//
// Restates the math of the reference's decode_gemv arm of mmq_fp8_gemm
// (python/minisgl/quant/kernels.py:1562-1563, 1686-1734) and of its fused gate_up+silu twin
// mmq_fp8_gemm_silu (kernels.py:1737-1753; epilogue tools/w4a8_gemm_silu_parity.py:52-54):
//   y[m,n] = s_m * sum_g scale[g,n] * sum_{k in g} e4m3(x[m,k]) * w(n,k)
// with f32 accumulation. The grouped (MoE) form follows mmq_fp8_moe_gemm / _gemm1_silu
// (kernels.py:744-773): rows are padded positions of the align, A rows are gathered by slot.
//
// Work split: blockIdx.x = group of 16-channel strips, blockIdx.z = block of 16 rows; a workgroup
// covers all of K and its waves split K into contiguous ranges. Each K tile is one coalesced 1 KB
// weight load per strip and one MFMA per strip (plus, for int4, one MFMA against a constant
// operand that yields the row sums the code shift needs). A wave issues every load of a chunk of
// tiles before its first MFMA, so it keeps a chunk's worth of weight bytes in flight. Waves reduce
// through LDS in a fixed order: results do not depend on timing, and no second kernel is needed.
#pragma once
#include "gemm_args.h"
#include "moe_route.h"


namespace w4a8 {

__device__ __forceinline__ bool row_source(const GemmArgs& p, int64_t r, int64_t& ar) {
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

// Workgroups go to the 8 XCDs round-robin (block i to XCD i % 8), each XCD with its own L2. The
// remap hands each XCD a contiguous range of strip groups, so neighbouring strips, which share
// scale cache lines (one 128-byte line holds the fp16 scales of 4 strips), meet in one L2 instead
// of being fetched from HBM by up to 4 XCDs. Bijective on [0, n) for any n.
__device__ __forceinline__ int xcd_remap(int i, int n) {
  const int q = n >> 3, r = n & 7, x = i & 7, j = i >> 3;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + j;
}

// Per-tile accumulate of one wave for the sub-tile-group formats and the peeled partial tile: A
// fragment a, weight tiles raw[j] of its strips, K tile kt. GPT (groups per tile: 1, 2 or 4) is a
// compile-time constant and sub-groups past K are masked by a zero scale rather than skipped, so
// the body is straight-line code. SYM: int4 without zero points (zero 8).
template <int NSTR, int WFMT, int GPT, bool SYM>
__device__ __forceinline__ void gemv_tile(const GemmArgs& p, const v8i& a, const uint4* raw, const bool* sval,
                                          const int64_t* strip, int kt, const void* scales,
                                          const int32_t* zeros, int lane, v4f* acc) {
  const int N = (int)p.N, K = (int)p.K;
  const int kbase = kt * kTileK;
  if (WFMT == kE2M1 && p.sfmt == kScaleE8M0) {
    // MXFP4: E8M0 block scales go straight into the MFMA; blocks past K carry zero activations
    // and a 2^-127 scale.
    const int blk = kt * 4 + (lane >> 4);
    const bool bin = blk * 32 < K;
#pragma unroll
    for (int j = 0; j < NSTR; ++j) {
      const int n = (int)strip[j] * kTileN + (lane & 15);
      const int sb = (bin && sval[j]) ? (int)reinterpret_cast<const uint8_t*>(scales)[blk * N + n] : 0;
      acc[j] = mfma_f8f4_sb(a, fp4_operand(raw[j]), acc[j], sb);
    }
    return;
  }
  constexpr int kSub = kTileK / GPT;  // K width of one sub-group
  const int group = p.group;
  const int ngroups = K / group;
  const v8i half8 = splat8(kE4M3Half4);
  const v4f zero4 = v4f{0.f, 0.f, 0.f, 0.f};
  v4f rh[GPT];
  if (WFMT == kInt4) {
#pragma unroll
    for (int ss = 0; ss < GPT; ++ss)
      rh[ss] = GPT == 1 ? mfma_f8f8(a, half8, zero4) : mfma_f8f8_sb(a, half8, zero4, subgroup_mask_scale(lane, GPT, ss));
  }
  static_assert(GPT < 8 || WFMT == kE2M1, "16-wide groups are e2m1 only");
#pragma unroll
  for (int j = 0; j < NSTR; ++j) {
    if (!sval[j]) continue;
    const int n = (int)strip[j] * kTileN + (lane & 15);
    const v8i b = WFMT == kInt4 ? unpack_tile_int4(raw[j]) : fp4_operand(raw[j]);
#pragma unroll
    for (int ss = 0; ss < GPT; ++ss) {
      const int msk = GPT == 1 ? 127 : subgroup_mask_scale(lane, GPT, ss);
      const v4f c = WFMT == kInt4 ? mfma_f8f8_sb(a, b, zero4, msk)
                                  : mfma_f8f4_sb(a, GPT == 8 ? fp4_half_operand(b, ss) : b, zero4, msk);
      const bool in = kbase + ss * kSub < K;
      int g = (kbase + ss * kSub) / group;
      g = g < ngroups ? g : ngroups - 1;
      const float sc = in ? group_scale(scales, p.sfmt, (int64_t)g * N + n, zeros, n) : 0.0f;
      if (WFMT == kInt4) {
        float coef = -1.0f;
        if (!SYM) {
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

// Kernel modes: which per-tile work a wave does.
//   0: int4, group a multiple of 128 (one scale per strip per tile, preloaded with the weights)
//   1: int4, group 32/64 (sub-tile groups, scales loaded per sub-group)
//   2: e2m1 with E8M0 block scales (bytes preloaded, fed to the scaled MFMA)
//   3: e2m1 with fp16 group scales (sub-tile groups)
//   4: NVFP4 (e2m1, e4m3 group-16 scales preloaded with the weights, per-channel global applied in
//      the epilogue)
constexpr int kModeI4 = 0, kModeI4Sub = 1, kModeE8M0 = 2, kModeE2M1F16 = 3, kModeNV = 4;

// Where a wave's A fragments come from.
//   kAGlobal: fp8 rows in global memory, loaded per tile with the weights (grouped rows, or blocks
//             too large to stage).
//   kAStage:  fp8 rows copied once per workgroup into LDS.
//   kAQuant:  bf16/fp16 rows read once per workgroup, quantized per token (the act-quant kernel's
//             arithmetic, bit for bit) into LDS.
//   kARoute:  kAQuant for gemm1 of a decode-sized MoE batch, one slot per workgroup row block
//             (blockIdx.z = slot, output row slot * bm): the workgroup routes the slot's token
//             itself (moe_route.h, on the logits in p.logits), takes the slot's expert and
//             quantizes the token's row; strip group 0 of each token's first slot writes the route
//             (weights, ids, inverse positions, sorted ids, block owners, ntp) as the route + slot
//             launch would, so the batch needs no launch before gemm1.
constexpr int kAGlobal = 0, kAStage = 1, kAQuant = 2, kARoute = 3;
constexpr int kRoutePer = kRouteMaxExperts / 64;  // experts per lane of the in-kernel router
constexpr int kStageMax = 8;                // most 16-byte staging loads per thread (SM <= this)

// When a wave issues its first window of weight loads (compile-time, so that the compiler's wait
// counts stay exact; with a run-time choice it had to merge both orders and waited for every load,
// the weights included, before it touched the A data).
//   kWinAfterA: right after the A loads. The A data is waited for with a counted vmcnt, so the quant
//               or staging runs while the weights are in flight.
//   kWinAFirst: after A is quantized into LDS (fused quant): the activation row's loads meet no
//               weight load of the workgroup on their way (one-row calls on narrow weights).
//   kWinWaitAll: right after the A loads, and the fp8 staging waits for every load of the window
//               before it writes LDS (staged fp8 A; measured equal or up to 2% faster than
//               kWinAfterA on the decode sweep's staged calls).
constexpr int kWinAfterA = 0, kWinAFirst = 1, kWinWaitAll = 2;
// s_waitcnt vmcnt(0) in the gfx9 encoding (expcnt and lgkmcnt at their maxima: not waited for)
constexpr int kWaitVmcnt0 = 0x0F70;
constexpr int kStageLdsMax = 32 * 1024;     // LDS bytes of a staged A block

// LDS row stride of a staged A block: K padded to whole tiles (zeros) + 16 bytes of bank skew.
__host__ __device__ inline int stage_stride(int KT) { return KT * kTileK + 16; }

// Workgroup = one group of strips (blockIdx.x) x one block of 16 rows (blockIdx.z), all of K. Wave
// w owns the contiguous K tiles [w*tpw, (w+1)*tpw) and walks them in chunks of CH tiles: it issues
// every global load of a chunk up front, in per-tile groups (weights, scales, zero words; and the A
// fragment when A is not staged), then computes tile by tile as the groups land.
//   SYM: int4 with no zero points (zero 8): the MFMA is seeded with -R/2 from an MFMA against a
//        constant -0.5 operand, so no zero decode and one FMA per output element per tile.
//   SM:  16-byte A staging loads per thread (1, 2, 4 or 8): the registers they hold while the first
//        window of weights is in flight set the kernel's peak register count, so it is sized to the
//        block.
//   GPT: groups per K tile for the sub-tile-group modes (1 for the others).
//   AF:  when the first window of weight loads is issued (kWinAfterA / kWinAFirst / kWinWaitAll).
template <int NSTR, int CH, int MODE, int AMODE, bool SYM, int SM, int GPT, int AF>
__global__ void __launch_bounds__(512) gemv_kernel(const GemmArgs p, int tpw) {
  constexpr int WFMT = (MODE == kModeE8M0 || MODE == kModeE2M1F16 || MODE == kModeNV) ? kE2M1 : kInt4;
  static_assert(MODE != kModeNV || GPT == 8, "NVFP4 tiles hold 8 groups");
  static_assert(AF != kWinAFirst || AMODE == kAQuant, "A-first applies to the fused quant");
  static_assert(AF != kWinWaitAll || AMODE == kAStage, "wait-all applies to fp8 staging");
  constexpr bool kStaged = AMODE != kAGlobal;
  constexpr bool kRoute = AMODE == kARoute;
  constexpr bool kQuant = AMODE == kAQuant || kRoute;  // bf16/fp16 rows quantized in the prologue
  // grouped (MoE) rows only reach the global-A kernels: the staged and fused kernels are compiled
  // without the align lookups, so their prologue has no chain of dependent argument loads
  constexpr bool kMayGroup = AMODE == kAGlobal;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float amax_w[8 * 16];  // per-wave row maxima (fused quant)
  __shared__ float srow[16];
  __shared__ int rvalid[16];
  // the wave index is uniform across the wave: readfirstlane lets the compiler keep everything
  // derived from it (K range, loop bounds, branches) in scalar registers
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), W = blockDim.x >> 6;
  if constexpr (AMODE == kAGlobal) {
    // every argument field this source uses, loaded in one batch at entry: left to the compiler the
    // loads follow the branches on them, four dependent scalar-cache rounds before the first weight
    // load (measured: M=8/16 calls 0.15-0.5 us faster this way; the staged and fused-quant sources
    // measured 0.1-0.3 us slower and keep the compiler's order)
    asm volatile("" ::"s"(p.silu), "s"(p.out_dtype), "s"(p.ldo), "s"(p.out), "s"(p.N), "s"(p.K), "s"(p.KT), "s"(p.M),
                 "s"(p.wt), "s"(p.scales), "s"(p.zeros), "s"(p.group), "s"(p.sfmt), "s"(tpw));
    asm volatile("" ::"s"(p.xq), "s"(p.ldx), "s"(p.act_scales), "s"(p.sorted_ids), "s"(p.expert_ids), "s"(p.ntp),
                 "s"(p.bm), "s"(p.num_slots), "s"(p.top_k), "s"(p.a_by_token), "s"(p.w_expert_tiles),
                 "s"(p.s_expert_stride), "s"(p.z_expert_stride));
  }
  const int64_t sg = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  // routed: the block is slot blockIdx.z (output row slot * bm), its A row the slot's token
  const int64_t m0 = kRoute ? (int64_t)blockIdx.z * p.bm : (int64_t)blockIdx.z * 16;
  const int64_t tok = kRoute ? (int64_t)(blockIdx.z / (uint32_t)p.top_k) : 0;
  uint32_t logit_raw[kRoute ? kRoutePer : 1];
  if constexpr (kRoute) route_load<kRoutePer>(p.logits, p.ldtype, tok, p.num_experts, logit_raw);

  int64_t expert = 0;
  if (kMayGroup && p.sorted_ids) {
    if (m0 >= (int64_t)(*p.ntp)) return;
    expert = p.expert_ids[(uint32_t)m0 / (uint32_t)p.bm];  // padded rows < 2^31
  }
  // A row of this lane. A row that holds no data reads row 0 instead: an A row only feeds its
  // own output row, which is never stored, and a valid address keeps the loads branch-free.
  int64_t ar = m0 + (lane & 15);
  bool row_ok = kRoute ? (lane & 15) == 0 : kMayGroup ? row_source(p, m0 + (lane & 15), ar) : ar < p.M;
  const uint8_t* arow = p.xq + (row_ok ? ar : 0) * p.ldx;
  // act scale of the row, loaded now so the epilogue does not wait on a dependent load
  float row_scale = (!kQuant && row_ok) ? p.act_scales[ar] : 0.f;

  const int64_t nstrips = p.N / kTileN;
  const int half = p.silu ? NSTR / 2 : NSTR;
  int64_t strip[NSTR];
  bool sval[NSTR];
#pragma unroll
  for (int j = 0; j < NSTR; ++j) sval[j] = strip_of(p.silu, sg, j, half, NSTR, nstrips, strip[j]);

  // 32-bit index math on the hot path (tile, scale and zero indices of one matrix fit easily)
  const int N = (int)p.N, K = (int)p.K, KT = (int)p.KT;
  const int gshift = 31 - __builtin_clz((unsigned)(p.group >= kTileK ? p.group / kTileK : 1));  // tiles per group
  const v4f zero4 = v4f{0.f, 0.f, 0.f, 0.f};

  // ---- A staging loads, issued before any weight load so that waiting for them never waits for
  // weights. Rows [0, rv) of the block; each row padded with zeros to whole tiles.
  const int rv = kRoute ? 1 : kStaged ? (int)(p.M - m0 < 16 ? p.M - m0 : 16) : 0;
  const int64_t xr0 = kRoute ? tok : m0;  // source row of the block's row 0
  const int lstride = stage_stride(KT);
  unsigned char* a_lds = smem;
  constexpr int kEl = kQuant ? 8 : 16;  // elements per 16-byte load
  const int cpr = KT * (kTileK / kEl);  // loads per padded row
  const int nchunks = rv * cpr;
  uint4 stg[kStaged ? SM : 1];
  auto issue_stage = [&]() {
#pragma unroll
    for (int i = 0; i < SM; ++i) {
      int c = (int)threadIdx.x + i * (int)blockDim.x;
      c = c < nchunks ? c : nchunks - 1;
      const int r = c / cpr;
      int k = (c - r * cpr) * kEl;
      k = k < K ? k : K - kEl;  // padding: any valid address, the value is replaced by zeros
      if (kQuant)
        stg[i] = *reinterpret_cast<const uint4*>(p.xsrc + (xr0 + r) * p.ldxs + k);
      else
        stg[i] = *reinterpret_cast<const uint4*>(p.xq + (xr0 + r) * p.ldx + k);
    }
  };
  if constexpr (kRoute) {
    // the row's loads go out behind the logits' and ahead of the route, whose wait for the
    // logits leaves them in flight
    issue_stage();
    // the slot's choice needs the first jj + 1 rounds; the wave that writes the route, all top_k
    const int jj = (int)((int64_t)blockIdx.z - tok * p.top_k);
    const bool writer = blockIdx.x == 0 && wave == 0 && jj == 0;
    const RoutePick rp = route_pick<kRoutePer>(logit_raw, p.ldtype, p.num_experts, writer ? p.top_k : jj + 1);
    const int e = __builtin_amdgcn_readlane(rp.myid, jj);
    const bool eok = e >= 0 && e < p.num_experts;
    // a slot left without an expert (NaN logits) is dropped: no output row, expert E-1's
    // weights for valid addresses
    expert = eok ? e : p.num_experts - 1;
    row_ok = row_ok && eok;
    if (writer) {
      // the token's route, written once: per slot s the weight, the expert, the padded row; the
      // slot's block holds s in its first row and the sentinel S in the others
      float mx, sum;
      route_softmax<kRoutePer>(logit_raw, p.ldtype, p.num_experts, mx, sum);
      const float w = route_weight(rp, mx, sum, p.top_k, p.renorm);
      const int S = (int)p.num_slots, bm = p.bm;
      const int64_t s0 = tok * p.top_k;
      const bool mine_ok = rp.myid >= 0 && rp.myid < p.num_experts;
      if (lane < p.top_k) {
        p.tw_out[s0 + lane] = w;
        p.ids_out[s0 + lane] = rp.myid;
        p.inv_out[s0 + lane] = mine_ok ? (int32_t)((s0 + lane) * bm) : -1;
        p.eid_out[s0 + lane] = mine_ok ? rp.myid : p.num_experts - 1;
      }
      for (int j = 0; j < p.top_k; ++j) {
        const int ej = __builtin_amdgcn_readlane(rp.myid, j);
        const bool ok = ej >= 0 && ej < p.num_experts;
        if (lane < bm) p.sorted_out[(s0 + j) * bm + lane] = (lane == 0 && ok) ? (int32_t)(s0 + j) : S;
      }
      if (tok == 0 && lane == 0) *p.ntp_out = S * bm;
    }
  }

  const uint4* wt = p.wt + (size_t)(expert * p.w_expert_tiles) * 64;
  // scale element size from the mode (E8M0 bytes, else fp16), so that the scale base stays in
  // scalar registers
  const int kEsz = (MODE == kModeE8M0 || MODE == kModeNV || (MODE == kModeE2M1F16 && p.sfmt == kScaleE4M3)) ? 1 : 2;
  const void* scales = reinterpret_cast<const char*>(p.scales) + (size_t)(expert * p.s_expert_stride) * kEsz;
  const int32_t* zeros = p.zeros ? p.zeros + expert * p.z_expert_stride : nullptr;
  if (kStaged && !kRoute) issue_stage();

  const int kt_begin = wave * tpw;
  const int kt_last = kt_begin + tpw < KT ? kt_begin + tpw : KT;
  // full tiles [kt_begin, kt_end); with A in global memory a partial last tile (K % 128 != 0) is
  // peeled below, with A in LDS it reads the zero padding like any other tile
  const int kfull = K / kTileK;
  const int kt_end = kStaged ? kt_last : (kt_last < kfull ? kt_last : kfull);
  int strip_c[NSTR];
#pragma unroll
  for (int j = 0; j < NSTR; ++j) strip_c[j] = (int)(strip[j] < nstrips ? strip[j] : nstrips - 1);

  v8i a[kStaged ? 1 : CH];
  uint4 raw[CH][NSTR];
  // raw fp16 bits, two tiles per VGPR (the loads fill the low and high halves): converting at load
  // time would force a wait per load, and a VGPR per scale would cost the kernel occupancy
  typedef unsigned short v2h __attribute__((ext_vector_type(2)));
  v2h sc[(CH + 1) / 2][NSTR];
  uint32_t zw[SYM ? 1 : CH][NSTR];
  int sb[CH][NSTR];
  // NVFP4: the 8 group-scale bytes of a tile, two per register (loaded into the halves directly)
  typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
  v2u16 nvs[MODE == kModeNV ? CH : 1][NSTR][4];
  v4f acc[NSTR];
#pragma unroll
  for (int j = 0; j < NSTR; ++j) acc[j] = zero4;

  // global loads of K tile kt into register slot t: weights, scales, zero words; and the A
  // fragment unless A is staged
  // buffer descriptors: this expert's tiles, scales, zero words; per-lane offsets fixed, per-tile
  // offsets scalar
  const BufRsrc rs_w = make_rsrc(wt, (uint32_t)(nstrips * KT * kTileBytes));
  const int ngroups = K >> (31 - __builtin_clz((unsigned)p.group));  // group is a power of two
  const BufRsrc rs_s = make_rsrc(scales, (uint32_t)(ngroups * N * kEsz));
  const BufRsrc rs_z = make_rsrc(zeros, zeros ? (uint32_t)(ngroups * (N / 8) * 4) : 0u);
  const BufRsrc rs_a = make_rsrc(p.xq, 0xffffffffu);
  // A fragment of tile kt: row-major rows (lane (l & 15)'s row, bytes 16 (l >> 4) and 64 + 16 (l >> 4)
  // of the tile), or with p.a_tiled (grouped gemm2) the block's operand-order codes, two 1 KiB runs
  const bool a_t = kMayGroup && p.a_tiled;
  const uint32_t a_voff = a_t ? (uint32_t)((m0 >> 4) * KT * 2048 + lane * 16)
                              : (uint32_t)((row_ok ? ar : 0) * p.ldx) + 16 * (lane >> 4);
  const uint32_t a_step = a_t ? 2048u : (uint32_t)kTileK, a_hi = a_t ? 1024u : 64u;
  // global loads of K tile kt into register slot t: weights, scales, zero words; and the A
  // fragment unless A is staged
  auto load_tile = [&](int t, int kt) {
    if (!kStaged) {
      const uint4 lo = bload128(rs_a, a_voff, (uint32_t)kt * a_step);
      const uint4 hi = bload128(rs_a, a_voff + a_hi, (uint32_t)kt * a_step);
      a[t][0] = (int)lo.x; a[t][1] = (int)lo.y; a[t][2] = (int)lo.z; a[t][3] = (int)lo.w;
      a[t][4] = (int)hi.x; a[t][5] = (int)hi.y; a[t][6] = (int)hi.z; a[t][7] = (int)hi.w;
    }
#pragma unroll
    for (int j = 0; j < NSTR; ++j) {
      raw[t][j] = bload128_nt(rs_w, (uint32_t)lane * 16, (uint32_t)((strip_c[j] * KT + kt) * kTileBytes));
      const int n = strip_c[j] * kTileN + (lane & 15);
      if (MODE == kModeI4) {
        const int g = kt >> gshift;
        sc[t >> 1][j][t & 1] = bload16(rs_s, (uint32_t)n * 2, (uint32_t)(g * N * 2));
        if (!SYM) zw[t][j] = zeros ? bload32(rs_z, (uint32_t)(n / 8) * 4, (uint32_t)(g * (N / 8) * 4)) : 0x88888888u;
      } else if (MODE == kModeE8M0) {
        // blocks past K read as 0 (2^-127) from the descriptor's bound; their activations are 0
        sb[t][j] = (int)bload8(rs_s, (uint32_t)((lane >> 4) * N + n), (uint32_t)(kt * 4 * N));
      } else if (MODE == kModeNV) {
        // groups past K read as 0 from the descriptor's bound (a zero scale)
#pragma unroll
        for (int ss = 0; ss < 8; ++ss)
          nvs[MODE == kModeNV ? t : 0][j][ss >> 1][ss & 1] =
              (unsigned short)bload8(rs_s, (uint32_t)n, (uint32_t)((kt * 8 + ss) * N));
      }
    }
  };
  // tile index for a slot load; past the range end it repeats the last tile (a cache hit that
  // keeps the loads unconditional)
  auto clamp_kt = [&](int kt) { return kt < kt_end ? kt : (kt_end > 0 ? kt_end - 1 : 0); };
  // fill the window: the first CH tiles' loads are in flight while A is staged (A-first: after)
  if constexpr (AF != kWinAFirst) {
#pragma unroll
    for (int t = 0; t < CH; ++t) load_tile(t, clamp_kt(kt_begin + t));
  }

  if (kQuant) {
    // per-row amax: lane r (< 16) of each wave ends with the wave's maximum of row r
    float rowmax = 0.f;
    if (rv == 1) {
      float v = 0.f;
#pragma unroll
      for (int i = 0; i < SM; ++i) {
        const int c = (int)threadIdx.x + i * (int)blockDim.x;
        if (c < nchunks && c * 8 < K) v = fmaxf(v, amax8(stg[i], p.xdtype));
      }
      rowmax = wave_max(v);
    } else {
#pragma unroll
      for (int i = 0; i < SM; ++i) {
        const int c = (int)threadIdx.x + i * (int)blockDim.x;
        const int r = c < nchunks ? c / cpr : 0;
        const bool valid = c < nchunks && (c - r * cpr) * 8 < K;
        const float v = valid ? amax8(stg[i], p.xdtype) : 0.f;
        // the rows present in this wave, one at a time (a wave's loads span one or two rows when
        // K >= 512)
        uint64_t rem = __ballot(valid);
        while (rem) {
          const int leader = __ffsll((unsigned long long)rem) - 1;
          const int rr = __shfl(r, leader, 64);
          const bool mine = valid && r == rr;
          const float m = wave_max(mine ? v : 0.f);
          if (lane == rr) rowmax = fmaxf(rowmax, m);
          rem &= ~__ballot(mine);
        }
      }
    }
    if (lane < 16) amax_w[wave * 16 + lane] = rowmax;
    __syncthreads();
    // every thread derives the scales of the rows it touches from the per-wave maxima (no second
    // barrier): s = max(amax / 448, 1e-8), codes = e4m3(x * (1 / s))
    auto row_s = [&](int r) {
      float am = 0.f;
      for (int w = 0; w < W; ++w) am = fmaxf(am, amax_w[w * 16 + r]);
      return act_row_scale(am);
    };
    const float inv0 = 1.0f / row_s(0);
#pragma unroll
    for (int i = 0; i < SM; ++i) {
      const int c = (int)threadIdx.x + i * (int)blockDim.x;
      if (c < nchunks) {
        const int r = c / cpr, k = (c - r * cpr) * 8;
        uint2 q = make_uint2(0u, 0u);
        if (k < K) {
          float f[8];
          unpack8(stg[i], p.xdtype, f);
          q = quant8(f, r == 0 ? inv0 : 1.0f / row_s(r));
        }
        *reinterpret_cast<uint2*>(a_lds + r * lstride + k) = q;
      }
    }
    if (row_ok) row_scale = row_s(lane & 15);
    __syncthreads();
  } else if (AMODE == kAStage) {
    // every load of the window lands before the staging writes: vmcnt(0)
    if constexpr (AF == kWinWaitAll) __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
#pragma unroll
    for (int i = 0; i < SM; ++i) {
      const int c = (int)threadIdx.x + i * (int)blockDim.x;
      if (c < nchunks) {
        const int r = c / cpr, k = (c - r * cpr) * 16;
        *reinterpret_cast<uint4*>(a_lds + r * lstride + k) = k < K ? stg[i] : make_uint4(0u, 0u, 0u, 0u);
      }
    }
    __syncthreads();
  }
  if constexpr (AF == kWinAFirst) {
#pragma unroll
    for (int t = 0; t < CH; ++t) load_tile(t, clamp_kt(kt_begin + t));
  }
  const int lrow = kStaged ? ((lane & 15) < rv ? (lane & 15) : 0) : 0;

  // MFMA work of K tile kt held in slot t
  auto compute_tile = [&](int t, int kt) {
    v8i at;
    if (kStaged) {
      const unsigned char* src = a_lds + lrow * lstride + kt * kTileK + 16 * (lane >> 4);
      const uint4 lo = *reinterpret_cast<const uint4*>(src);
      const uint4 hi = *reinterpret_cast<const uint4*>(src + 64);
      at[0] = (int)lo.x; at[1] = (int)lo.y; at[2] = (int)lo.z; at[3] = (int)lo.w;
      at[4] = (int)hi.x; at[5] = (int)hi.y; at[6] = (int)hi.z; at[7] = (int)hi.w;
    } else {
      at = a[t];
    }
    if (MODE == kModeE8M0) {
      // K blocks past the end carry zero activations; their (clamped) scale is harmless.
#pragma unroll
      for (int j = 0; j < NSTR; ++j) {
        if (!sval[j]) continue;
        acc[j] = mfma_f8f4_sb(at, fp4_operand(raw[t][j]), acc[j], sb[t][j]);
      }
    } else if (MODE == kModeI4 && SYM) {
      const v4f seed = mfma_f8f8(at, splat8(0xB0B0B0B0u), zero4);  // -R/2
#pragma unroll
      for (int j = 0; j < NSTR; ++j) {
        if (!sval[j]) continue;
        const v4f c = mfma_f8f8(at, unpack_tile_int4(raw[t][j]), seed);
        const float scf = f16_to_f32(sc[t >> 1][j][t & 1]);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[j][r] = fmaf(scf, c[r], acc[j][r]);
      }
    } else if (MODE == kModeI4) {
      const v4f rh = mfma_f8f8(at, splat8(kE4M3Half4), zero4);
#pragma unroll
      for (int j = 0; j < NSTR; ++j) {
        if (!sval[j]) continue;
        const int n = strip_c[j] * kTileN + (lane & 15);
        const v4f c = mfma_f8f8(at, unpack_tile_int4(raw[t][j]), zero4);
        const float coef = 15.0f - 2.0f * (float)((zw[SYM ? 0 : t][j] >> (4 * (n & 7))) & 15u);
        const float scf = f16_to_f32(sc[t >> 1][j][t & 1]);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[j][r] = fmaf(scf, fmaf(coef, rh[r], c[r]), acc[j][r]);
      }
    } else if (MODE == kModeNV) {
      // 16-wide groups: each 32-element block of a lane's operand holds two groups, so each group
      // is one MFMA on half the block (the other half zeroed) with only its block's scale open
#pragma unroll
      for (int j = 0; j < NSTR; ++j) {
        if (!sval[j]) continue;
        const v8i b = fp4_operand(raw[t][j]);
#pragma unroll
        for (int ss = 0; ss < 8; ++ss) {
          const v4f c = mfma_f8f4_sb(at, fp4_half_operand(b, ss), zero4, subgroup_mask_scale(lane, 8, ss));
          const v2u16 pr = nvs[MODE == kModeNV ? t : 0][j][ss >> 1];
          const float scf = __builtin_amdgcn_cvt_f32_fp8((int)(uint32_t)pr[ss & 1], 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[j][r] = fmaf(scf, c[r], acc[j][r]);
        }
      }
    } else {
      gemv_tile<NSTR, WFMT, GPT, SYM>(p, at, raw[t], sval, strip, kt, scales, zeros, lane, acc);
    }
  };

  // Rolling window of CH tiles. Steady state: slot t is consumed, then refilled with the tile CH
  // further on, so a wave keeps CH tiles of loads in flight until its range runs out. The steady
  // body has no branch (a branch out of it would make the compiler's wait counts drain the window
  // every tile); the last (at most CH) tiles, already in flight, drain after it.
  int c0 = kt_begin;
  for (; c0 + CH < kt_end; c0 += CH) {
#pragma unroll
    for (int t = 0; t < CH; ++t) {
      compute_tile(t, c0 + t);
      load_tile(t, clamp_kt(c0 + t + CH));
    }
  }
#pragma unroll
  for (int t = 0; t < CH; ++t)
    if (c0 + t < kt_end) compute_tile(t, c0 + t);

  if (!kStaged && kt_last > kfull && kt_begin <= kfull) {
    // partial last tile: masked A fragment (zeros past K), per-sub-group scale loads
    uint4 rawp[NSTR];
#pragma unroll
    for (int j = 0; j < NSTR; ++j) rawp[j] = wt[(strip_c[j] * KT + kfull) * 64 + lane];
    const v8i ap = load_a_operand(arow + kfull * kTileK, K - kfull * kTileK, lane);
    gemv_tile<NSTR, WFMT, GPT, SYM>(p, ap, rawp, sval, strip, kfull, scales, MODE == kModeNV ? nullptr : zeros, lane,
                                    acc);
  }

  // Cross-wave reduction through LDS, over the block's existing rows only (row i = 4q + r of the
  // C fragment lives in lane 16q + c, element r): a one-row decode call moves 16 floats per wave.
  float* red = reinterpret_cast<float*>(smem + (kStaged ? ((rv * lstride + 15) / 16) * 16 : 0));
  const int nr = kRoute ? 1 : (kMayGroup && p.sorted_ids) ? 16 : (int)(p.M - m0 < 16 ? p.M - m0 : 16);
  if (wave == 0 && lane < 16) {
    srow[lane] = row_scale;
    rvalid[lane] = row_ok ? 1 : 0;
  }
  {
    const int q = lane >> 4, c = lane & 15;
#pragma unroll
    for (int j = 0; j < NSTR; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (4 * q + r < nr) red[((wave * NSTR + j) * nr + 4 * q + r) * 16 + c] = acc[j][r];
  }
  __syncthreads();

  const int per = nr * 16;
  // e = (j * nr + i) * 16 + c; q / nr by a float reciprocal (exact: q + 1/2 lies at least 1/32 from
  // a multiple of nr <= 16, and q < 2^16 keeps the rounding error below 2^-7)
  const float inv_nr = 1.0f / (float)nr;
  for (int e = threadIdx.x; e < half * per; e += blockDim.x) {
    const int c = e & 15, q = e >> 4;
    const int j = (int)(((float)q + 0.5f) * inv_nr), i = q - j * nr;
    int64_t sj;
    if (!strip_of(p.silu, sg, j, half, NSTR, nstrips, sj)) continue;
    if (!rvalid[i]) continue;
    float tot = 0.f, tot_up = 0.f;
    for (int w = 0; w < W; ++w) {
      tot += red[((w * NSTR + j) * nr + i) * 16 + c];
      if (p.silu) tot_up += red[((w * NSTR + j + half) * nr + i) * 16 + c];
    }
    const float scl = srow[i];
    const int64_t row = m0 + i, col = sj * kTileN + c;
    if (MODE == kModeNV) {
      // the per-output-channel global (f32 bits in the zeros slot)
      tot *= __int_as_float(zeros[col]);
      if (p.silu) {
        int64_t su;
        strip_of(p.silu, sg, j + half, half, NSTR, nstrips, su);
        tot_up *= __int_as_float(zeros[su * kTileN + c]);
      }
    }
    if (p.silu)
      store_out(p, row, col, silu_mul(tot * scl, tot_up * scl, p.out_dtype));
    else
      store_out(p, row, col, tot * scl);
  }
}

// Launch shape of one decode call. The per-channel arithmetic depends only on (waves, tpw), which
// the planner derives from (M, N, K, row_blocks) alone, so the fused-silu arm, the plain arm and
// every A source agree bit for bit.
struct GemvPlan {
  int nstr;     // strips per workgroup of the plain arm (the silu arm runs 2*nstr: gate + up)
  int waves;    // waves per workgroup, wave w owning K tiles [w*tpw, (w+1)*tpw)
  int tpw;      // K tiles per wave
  int amode;    // kAGlobal / kAStage / kAQuant
  int sm;       // staging loads per thread (4 or 8) for kAStage / kAQuant
  size_t stage_bytes;  // LDS bytes of the staged A block (0 for kAGlobal)
  int af;       // when the first window of weight loads is issued (kWinAfterA / kWinAFirst / kWinWaitAll)
  int ch;       // window of the int4 fused-quant kernels (3 or 4 tiles; the other kernels roll 4)
};

// Launch shape of the strip-walking GEMV (gemv_walk.hip): one row block of bf16/fp16 rows quantized
// into LDS once per workgroup, `grid` workgroups each walking a contiguous range of the `ngroups`
// strip groups (a strip, or a gate strip and its up strip), the one-row K split (waves, tpw).
struct WalkPlan {
  int grid;
  int waves;    // the plan's K-split waves (one set)
  int sets;     // wave sets per workgroup, each walking every sets-th strip group
  int block_waves;  // waves per workgroup: the sets, plus helper waves of the row phase
  int tpw;
  int ngroups;
  int ngmax;    // most strip groups of one workgroup
  int tpr_log;  // log2 of the threads per row in the row phase
  int sm;       // 16-byte row loads per thread
  size_t lds;   // dynamic LDS: the row codes plus the waves' partial sums
};
// dynamic LDS a walking launch may use (the kernel's static arrays take the rest of the 160 KiB)
constexpr int kWalkLdsMax = 160 * 1024 - 512;
// the walking kernel's own arguments
struct WalkArgs {
  int kw;       // K-split waves per set
  int sets;     // 1 or 2
  int tpw;
  int gbase;    // strip groups per workgroup (ngroups / grid) ...
  int gextra;   // ... plus one for the first ngroups % grid workgroups
  int tpr_log;
};
bool launch_gemv_walk(const GemmArgs& p, const WalkPlan& wp, hipStream_t stream);
// false when the walking GEMV does not cover the call
bool plan_gemv_walk(const GemmArgs& p, int64_t row_blocks, WalkPlan& wp);

// Kernel launch of one A source; defined in the unit that instantiates it. `grid` is
// (strip groups, 1, row blocks); returns false when no kernel matches the call's formats.
bool launch_gemv_global(const GemmArgs& p, dim3 grid, const GemvPlan& pl, hipStream_t stream);
bool launch_gemv_staged(const GemmArgs& p, dim3 grid, const GemvPlan& pl, hipStream_t stream);
bool launch_gemv_fused(const GemmArgs& p, dim3 grid, const GemvPlan& pl, hipStream_t stream);
// the fused quant on e2m1 weights (MXFP4, NVFP4): its own unit, built in parallel with the int4 one
bool launch_gemv_fused_e2m1(const GemmArgs& p, dim3 grid, const GemvPlan& pl, hipStream_t stream);
// sub-tile groups (int4 group 32/64, e2m1 with fp16 scales), A read per tile
bool launch_gemv_generic(const GemmArgs& p, dim3 grid, const GemvPlan& pl, hipStream_t stream);
// K split (waves, tiles per wave) the GEMV runs for these arguments and row blocks
void gemv_ksplit(const GemmArgs& p, int64_t row_blocks, int& waves, int& tpw);
// the planner itself (quant_src: p.xsrc holds bf16/fp16 rows the kernel may quantize)
GemvPlan plan_gemv(const GemmArgs& p, int64_t row_blocks, bool quant_src);
// gemm1 of a decode-sized MoE batch with the router in the prologue (gemv_routed.hip)
int launch_moe_route_gemm1(const GemmArgs& p, int64_t row_blocks, hipStream_t stream);

// NVFP4 (e2m1 weights, e4m3 group-16 scales, per-channel global): the fast path's dedicated mode
inline bool gemv_nvfp4(const GemmArgs& p) {
  return p.wfmt == kE2M1 && p.sfmt == kScaleE4M3 && p.group == 16 && p.zeros != nullptr;
}

// Chunk length (tiles per strip held in registers at once) of the sub-tile-group kernels: 4 for
// short K ranges, else 8 (longer ranges roll the window through the range).
inline int gemv_chunk(int tpw) { return tpw <= 4 ? 4 : 8; }
// The fast-path kernels roll a 4-tile window (3 or 4 for int4 with the fused-quant A source, chosen
// by the planner). Measured on MI355X at the Llama-3-8B decode shapes (one row): against an 8-tile
// window it costs fewer VGPRs (68 against 80, so seven waves per SIMD and the whole gate_up grid
// resident at once instead of two rounds), and it queues fewer weight loads ahead of each wave's A
// loads on the CU, so A is ready sooner; gate_up 15.5 us against 18.1 us, down 10.5 against 11.0,
// qkv and o_proj 4-8% faster. The window does not change the summation order.
constexpr int kGemvChunk = 4;

// Block size and dynamic LDS of a launch: the staged A block plus the cross-wave reduction tile.
inline void gemv_block_lds(const GemmArgs& p, const GemvPlan& pl, dim3& block, size_t& lds) {
  const int nstr_k = p.silu ? 2 * pl.nstr : pl.nstr;
  lds = pl.stage_bytes + (size_t)pl.waves * nstr_k * 4 * 64 * sizeof(float);
  block = dim3(pl.waves * 64);
}

// Launch of one kernel variant; the staging depth only exists for staged A sources.
template <int NS, int CHK, int MD, int AM, bool SY, int AF>
void gemv_launch_sm(const GemmArgs& p, dim3 grid, hipStream_t stream, const GemvPlan& pl) {
  constexpr int G = MD == kModeNV ? 8 : 1;
  dim3 block;
  size_t lds;
  gemv_block_lds(p, pl, block, lds);
  if constexpr (AM == kAGlobal) {
    hipLaunchKernelGGL((gemv_kernel<NS, CHK, MD, AM, SY, 4, G, AF>), grid, block, lds, stream, p, pl.tpw);
  } else if constexpr (AM == kAStage) {
    if (pl.sm <= 4)
      hipLaunchKernelGGL((gemv_kernel<NS, CHK, MD, AM, SY, 4, G, AF>), grid, block, lds, stream, p, pl.tpw);
    else
      hipLaunchKernelGGL((gemv_kernel<NS, CHK, MD, AM, SY, 8, G, AF>), grid, block, lds, stream, p, pl.tpw);
  } else {
    if (pl.sm == 1)
      hipLaunchKernelGGL((gemv_kernel<NS, CHK, MD, AM, SY, 1, G, AF>), grid, block, lds, stream, p, pl.tpw);
    else if (pl.sm == 2)
      hipLaunchKernelGGL((gemv_kernel<NS, CHK, MD, AM, SY, 2, G, AF>), grid, block, lds, stream, p, pl.tpw);
    else if (pl.sm == 4)
      hipLaunchKernelGGL((gemv_kernel<NS, CHK, MD, AM, SY, 4, G, AF>), grid, block, lds, stream, p, pl.tpw);
    else
      hipLaunchKernelGGL((gemv_kernel<NS, CHK, MD, AM, SY, 8, G, AF>), grid, block, lds, stream, p, pl.tpw);
  }
}

// Format dispatch of one (A source, strips, int4 window, window order) choice. I4 / E2: which
// weight formats the calling unit instantiates (int4 with 128-multiple groups; MXFP4 and NVFP4).
template <int AMODE, int NS, int CHI4, int AF, bool I4, bool E2>
bool gemv_launch_fmt(const GemmArgs& p, dim3 grid, hipStream_t stream, const GemvPlan& pl) {
  if constexpr (I4) {
    if (p.wfmt == kInt4 && p.group % kTileK == 0) {
      if (p.zeros == nullptr) gemv_launch_sm<NS, CHI4, kModeI4, AMODE, true, AF>(p, grid, stream, pl);
      else gemv_launch_sm<NS, CHI4, kModeI4, AMODE, false, AF>(p, grid, stream, pl);
      return true;
    }
  }
  if constexpr (E2) {
    if (gemv_nvfp4(p)) {
      gemv_launch_sm<NS, kGemvChunk, kModeNV, AMODE, false, AF>(p, grid, stream, pl);
      return true;
    }
    if (p.wfmt == kE2M1 && p.sfmt == kScaleE8M0) {
      gemv_launch_sm<NS, kGemvChunk, kModeE8M0, AMODE, false, AF>(p, grid, stream, pl);
      return true;
    }
  }
  return false;
}

// The fused-quant kernels: strips per workgroup (1, 2, 4), int4 window (3, 4) and window order
// (A-first or after A) as the planner chose them.
template <bool I4, bool E2>
bool gemv_launch_quant(const GemmArgs& p, dim3 grid, hipStream_t stream, const GemvPlan& pl) {
  const int ns = p.silu ? 2 * pl.nstr : pl.nstr;
  const bool first = pl.af == kWinAFirst, ch4 = pl.ch == 4;
#define W4A8_GEMV_Q(NS, CH, AF) return gemv_launch_fmt<kAQuant, NS, CH, AF, I4, E2>(p, grid, stream, pl)
  if (ns == 1) {
    if (first) W4A8_GEMV_Q(1, 3, kWinAFirst);
    if (ch4) W4A8_GEMV_Q(1, 4, kWinAfterA);
    W4A8_GEMV_Q(1, 3, kWinAfterA);
  }
  if (ns == 2) {
    if (first) W4A8_GEMV_Q(2, 3, kWinAFirst);
    if (ch4) W4A8_GEMV_Q(2, 4, kWinAfterA);
    W4A8_GEMV_Q(2, 3, kWinAfterA);
  }
  if (ns == 4 && !first) {
    if (ch4) W4A8_GEMV_Q(4, 4, kWinAfterA);
    W4A8_GEMV_Q(4, 3, kWinAfterA);
  }
#undef W4A8_GEMV_Q
  return false;
}

}  // namespace w4a8

// Pieces shared by the LDS-staged prefill / grouped GEMM kernels (gemm_prefill_lds.hip,
// gemm_prefill_dma.hip): weight-format modes, grouped-row lookup, the silu epilogue, the 1 KiB
// MFMA operand read and the per-stage LDS layout.
#pragma once
#include <type_traits>

#include "gemm_args.h"

namespace w4a8 {

template <int N>
using IC = std::integral_constant<int, N>;

// s_waitcnt vmcnt(n) lgkmcnt(0), expcnt untouched (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}

constexpr int kPSym = 0, kPAsym = 1, kPE8M0 = 2;

__device__ __forceinline__ bool lrow_source(const GemmArgs& p, int64_t r, int64_t& ar) {
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

// With a bf16 output the exponential is the hardware one (__expf): the rounded result of
// g / (1 + e^-g) depends only on the bf16 value g, and over all 65536 bf16 values it equals the
// one with expf (checked on the GPU, NaN and inf included; so it also equals torch's f32 replica
// bit for bit). fp16 keeps expf (there __expf changes 2 of the 65536 results). dt is a
// compile-time constant at every call, so the choice costs nothing.
__device__ __forceinline__ float lsilu_mul(float gate, float up, int dt) {
  // tools/w4a8_gemm_silu_parity.py:52-54: round to dtype, silu in f32, round, multiply in dtype
  const float g = from_dtype(to_dtype(gate, dt), dt);
  const float u = from_dtype(to_dtype(up, dt), dt);
  const float sg = g / (1.0f + (dt == kBF16 ? __expf(-g) : expf(-g)));
  return from_dtype(to_dtype(sg, dt), dt) * u;
}

__device__ __forceinline__ v8i lds_operand(const unsigned char* base, int lane) {
  const uint4 lo = *reinterpret_cast<const uint4*>(base + lane * 16);
  const uint4 hi = *reinterpret_cast<const uint4*>(base + 1024 + lane * 16);
  v8i a;
  a[0] = (int)lo.x; a[1] = (int)lo.y; a[2] = (int)lo.z; a[3] = (int)lo.w;
  a[4] = (int)hi.x; a[5] = (int)hi.y; a[6] = (int)hi.z; a[7] = (int)hi.w;
  return a;
}

template <int BM, int BN, int MODE>
struct LdsStage {
  static constexpr int kA = BM * 128;                          // fp8 operand order
  static constexpr int kB = MODE == kPE8M0 ? BN * 64 : BN * 128;  // fp4 bytes, or unpacked fp8
  static constexpr int kS = MODE == kPE8M0 ? BN * 4 : BN * 2;  // E8M0 [strip][lane] | fp16 [strip][16]
  static constexpr int kZ = MODE == kPAsym ? BN / 2 : 0;       // zero words [strip][2]
  static constexpr int kBytes = kA + kB + kS + kZ;
};

// Epilogue of the LDS-staged GEMMs. Lane layout: rows row0 + rb*16 + 4*(lane>>4) + r, channel
// (lane & 15) of each strip j, strip(j, ok) giving strip j's global index. y = acc * s_row, or for
// the fused arm silu(gate) * up over the strip pairs (j, j + NSB/2), rounded to the output dtype.
// The dtype and the arm are compile-time here, so the store loops hold no branches and no loads.
template <int DT, bool SILU, int RB, int NSB, typename SF>
__device__ __forceinline__ void store_tile_dt(const GemmArgs& p, const v4f (&acc)[RB][NSB], const float (&sc)[RB][4],
                                              uint32_t valid, int64_t row0, int lane, SF strip) {
  constexpr int JN = SILU ? NSB / 2 : NSB;
#pragma unroll
  for (int j = 0; j < JN; ++j) {
    bool ok;
    const int gs = strip(j, ok);
    if (!ok) continue;
    const int64_t col = (int64_t)gs * kTileN + (lane & 15);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (!((valid >> (rb * 4 + r)) & 1u)) continue;
        const int64_t row = row0 + rb * 16 + 4 * (lane >> 4) + r;
        const float s = sc[rb][r];
        float v;
        if constexpr (SILU)
          v = lsilu_mul(acc[rb][j][r] * s, acc[rb][j + NSB / 2][r] * s, DT);
        else
          v = acc[rb][j][r] * s;
        if constexpr (DT == kF32)
          reinterpret_cast<float*>(p.out)[row * p.ldo + col] = v;
        else
          reinterpret_cast<uint16_t*>(p.out)[row * p.ldo + col] = to_dtype(v, DT);
      }
  }
}

// The same epilogue through a per-wave LDS tile, for output rows whose stride and base are
// 16-byte aligned: each 16-row block is written to LDS in the MFMA lane layout (2 or 4 bytes per
// lane and element), read back row-major and stored 16 bytes per lane, so a store instruction
// covers whole row segments (the wave's strips are contiguous columns) instead of 32-byte pieces
// of four rows. scr: this wave's 16 * (JN*16*E + 16) bytes; nvs: the wave's strips inside N.
template <int DT, bool SILU, int RB, int NSB>
__device__ __forceinline__ void store_tile_lds(const GemmArgs& p, const v4f (&acc)[RB][NSB], const float (&sc)[RB][4],
                                               uint32_t valid, int64_t row0, int lane, int64_t col0, int nvs,
                                               unsigned char* scr) {
  constexpr int JN = SILU ? NSB / 2 : NSB;
  constexpr int E = DT == kF32 ? 4 : 2;
  constexpr int W = JN * 16 * E;       // bytes of one row of the wave's tile
  constexpr int P = W + 16;            // LDS row pitch (16-byte aligned; offsets the banks of rows 4 apart)
  constexpr int CPR = W / 16;          // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;        // rows per store instruction (lanes past row 15 idle)
  static_assert(CPR <= 64 && 64 % CPR == 0 && (RPI >= 16 || 16 % RPI == 0), "chunk layout");
  const int q = lane >> 4, c = lane & 15;
  const int crow = lane / CPR, chunk = lane % CPR;
  const bool cok = chunk * 16 / (16 * E) < nvs;  // the chunk's strip lies inside N
  unsigned char* outb = reinterpret_cast<unsigned char*>(p.out) + col0 * E + chunk * 16;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float s = sc[rb][r];
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        float v;
        if constexpr (SILU)
          v = lsilu_mul(acc[rb][j][r] * s, acc[rb][j + NSB / 2][r] * s, DT);
        else
          v = acc[rb][j][r] * s;
        unsigned char* d = scr + (4 * q + r) * P + j * 16 * E + c * E;
        if constexpr (DT == kF32) *reinterpret_cast<float*>(d) = v;
        else *reinterpret_cast<uint16_t*>(d) = to_dtype(v, DT);
      }
    }
    // rows of this block that hold data: bit 4q+r from any lane of group q
    uint32_t rv = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint64_t b = __ballot((valid >> (rb * 4 + r)) & 1u);
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) rv |= (uint32_t)((b >> (16 * qq)) & 1u) << (4 * qq + r);
    }
    // LDS operations of one wave complete in order: the reads see the writes above, and the next
    // block's writes come after these reads
#pragma unroll
    for (int i = 0; i < (16 + RPI - 1) / RPI; ++i) {
      const int rr = i * RPI + crow;
      const uint4 d = *reinterpret_cast<const uint4*>(scr + (rr < 16 ? rr : 15) * P + chunk * 16);
      if (cok && rr < 16 && ((rv >> rr) & 1u)) {
        const int64_t row = row0 + rb * 16 + rr;
        *reinterpret_cast<uint4*>(outb + row * p.ldo * E) = d;
      }
    }
  }
}

// One W4A16 bf16 output value from its two term rows: y_t = acc_t * s_t rounded to f32 as the f32
// output of the split GEMM stores them, then (0 + y_0) + y_1 as the term-sum kernel adds them (the
// empty asm keeps the products from contracting into the additions).
__device__ __forceinline__ float tsum2_value(float a0, float s0, float a1, float s1) {
  float y0 = a0 * s0, y1 = a1 * s1;
  asm volatile("" : "+v"(y0), "+v"(y1));
  return (0.0f + y0) + y1;
}

// The W4A16 bf16 epilogue (p.tsum2): the lane's rows 4q + r hold term r & 1 of activation row
// 2q + (r >> 1) of the block's 8, so each lane sums its own row pairs and writes bf16 token rows
// (silu over the summed gate and up, rounded as the fused silu arms round) through the per-wave LDS
// tile as store_tile_lds does: 8 token rows per 16-row block. row0: the wave's first term row
// (even); token rows are row / 2.
template <bool SILU, int RB, int NSB>
__device__ __forceinline__ void store_tile_tsum2(const GemmArgs& p, const v4f (&acc)[RB][NSB], const float (&sc)[RB][4],
                                                 uint32_t valid, int64_t row0, int lane, int64_t col0, int nvs,
                                                 unsigned char* scr) {
  constexpr int JN = SILU ? NSB / 2 : NSB;
  constexpr int E = 2;
  constexpr int W = JN * 16 * E;
  constexpr int P = W + 16;
  constexpr int CPR = W / 16;
  constexpr int RPI = 64 / CPR;
  static_assert(CPR <= 64 && 64 % CPR == 0 && (RPI >= 8 || 8 % RPI == 0), "chunk layout");
  const int q = lane >> 4, c = lane & 15;
  const int crow = lane / CPR, chunk = lane % CPR;
  const bool cok = chunk * 16 / (16 * E) < nvs;
  unsigned char* outb = reinterpret_cast<unsigned char*>(p.out) + col0 * E + chunk * 16;
  const int64_t trow0 = row0 / 2;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float s0 = sc[rb][2 * h], s1 = sc[rb][2 * h + 1];
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        float v;
        if constexpr (SILU)
          v = lsilu_mul(tsum2_value(acc[rb][j][2 * h], s0, acc[rb][j][2 * h + 1], s1),
                        tsum2_value(acc[rb][j + NSB / 2][2 * h], s0, acc[rb][j + NSB / 2][2 * h + 1], s1), kBF16);
        else
          v = tsum2_value(acc[rb][j][2 * h], s0, acc[rb][j][2 * h + 1], s1);
        *reinterpret_cast<uint16_t*>(scr + (2 * q + h) * P + j * 16 * E + c * E) = to_dtype(v, kBF16);
      }
    }
    // token rows of this block that hold data: bit 2q + h from row 4q + 2h of any lane of group q
    uint32_t rv = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint64_t b = __ballot((valid >> (rb * 4 + 2 * h)) & 1u);
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) rv |= (uint32_t)((b >> (16 * qq)) & 1u) << (2 * qq + h);
    }
#pragma unroll
    for (int i = 0; i < (8 + RPI - 1) / RPI; ++i) {
      const int rr = i * RPI + crow;
      const uint4 d = *reinterpret_cast<const uint4*>(scr + (rr < 8 ? rr : 7) * P + chunk * 16);
      if (cok && rr < 8 && ((rv >> rr) & 1u)) {
        const int64_t trow = trow0 + rb * 8 + rr;
        *reinterpret_cast<uint4*>(outb + trow * p.ldo * E) = d;
      }
    }
  }
}

// Every row's source lookup and activation scale is loaded before the first store: a load issued
// between stores makes the wait for its value also wait for all the stores issued before it (one
// vector-memory counter covers both), which serialized the whole epilogue.
// scr (may be null): this wave's LDS scratch for the row-major store path, at least
// 16 * (NSB*16*4 + 16) bytes, free to overwrite.
// The epilogue rows' sources, split from their scales so a kernel can look them up early (with
// its A rows) and load the scales behind its first loads: bit rb*4+r of the result is set when the
// lane's row row0 + rb*16 + 4*(lane>>4) + r holds data, ar[rb][r] its activation row.
template <int RB>
__device__ __forceinline__ uint32_t tile_row_sources(const GemmArgs& p, int64_t row0, int lane, int64_t (&ar)[RB][4]) {
  static_assert(RB * 4 <= 32, "row mask");
  uint32_t valid = 0;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = lrow_source(p, row0 + rb * 16 + 4 * (lane >> 4) + r, ar[rb][r]);
      valid |= (ok ? 1u : 0u) << (rb * 4 + r);
    }
  return valid;
}
template <int RB>
__device__ __forceinline__ void tile_row_scales(const GemmArgs& p, const int64_t (&ar)[RB][4], uint32_t valid,
                                                float (&sc)[RB][4]) {
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[rb][r] = p.act_scales[((valid >> (rb * 4 + r)) & 1u) ? ar[rb][r] : 0];
}

// The epilogue with the rows' scales and validity already in registers.
template <int RB, int NSB, typename SF>
__device__ __forceinline__ void store_tile_scaled(const GemmArgs& p, const v4f (&acc)[RB][NSB], const float (&sc)[RB][4],
                                                  uint32_t valid, int64_t row0, int lane, SF strip,
                                                  unsigned char* scr = nullptr) {
  const int esz = p.out_dtype == kF32 ? 4 : 2;
  if (scr && ((reinterpret_cast<uintptr_t>(p.out) | (uintptr_t)(p.ldo * esz)) & 15) == 0) {
    // the wave's strips are consecutive columns; count those inside N
    const int jn = p.silu ? NSB / 2 : NSB;
    int nvs = 0;
    bool ok0;
    const int gs0 = strip(0, ok0);
#pragma unroll
    for (int j = 0; j < NSB; ++j) {
      bool ok;
      (void)strip(j, ok);
      nvs += (j < jn && ok) ? 1 : 0;
    }
    const int64_t col0 = (int64_t)gs0 * kTileN;
    if (p.tsum2) {  // the host sets it for bf16 output rows with 16-byte aligned stride only
      if (p.silu) store_tile_tsum2<true>(p, acc, sc, valid, row0, lane, col0, nvs, scr);
      else store_tile_tsum2<false>(p, acc, sc, valid, row0, lane, col0, nvs, scr);
      return;
    }
    if (p.out_dtype == kBF16) {
      if (p.silu) store_tile_lds<kBF16, true>(p, acc, sc, valid, row0, lane, col0, nvs, scr);
      else store_tile_lds<kBF16, false>(p, acc, sc, valid, row0, lane, col0, nvs, scr);
    } else if (p.out_dtype == kF16) {
      if (p.silu) store_tile_lds<kF16, true>(p, acc, sc, valid, row0, lane, col0, nvs, scr);
      else store_tile_lds<kF16, false>(p, acc, sc, valid, row0, lane, col0, nvs, scr);
    } else {
      store_tile_lds<kF32, false>(p, acc, sc, valid, row0, lane, col0, nvs, scr);
    }
    return;
  }
  if (p.out_dtype == kBF16) {
    if (p.silu) store_tile_dt<kBF16, true>(p, acc, sc, valid, row0, lane, strip);
    else store_tile_dt<kBF16, false>(p, acc, sc, valid, row0, lane, strip);
  } else if (p.out_dtype == kF16) {
    if (p.silu) store_tile_dt<kF16, true>(p, acc, sc, valid, row0, lane, strip);
    else store_tile_dt<kF16, false>(p, acc, sc, valid, row0, lane, strip);
  } else {
    store_tile_dt<kF32, false>(p, acc, sc, valid, row0, lane, strip);
  }
}

template <int RB, int NSB, typename SF>
__device__ __forceinline__ void store_tile(const GemmArgs& p, const v4f (&acc)[RB][NSB], int64_t row0, int lane,
                                           SF strip, unsigned char* scr = nullptr) {
  int64_t ar[RB][4];
  const uint32_t valid = tile_row_sources<RB>(p, row0, lane, ar);
  float sc[RB][4];
  tile_row_scales<RB>(p, ar, valid, sc);
  store_tile_scaled(p, acc, sc, valid, row0, lane, strip, scr);
}

// Launch of the DMA-staged kernel (gemm_prefill_dma.hip); kErrUnsupported when it does not apply.
int launch_prefill_dma(const GemmArgs& p, int64_t rows_to_cover, int bm_rows, hipStream_t stream);
// NVFP4 on the fp16 MFMA (gemm_prefill_nv.hip); kErrUnsupported for other formats and shapes.
int launch_prefill_nv(const GemmArgs& p, int64_t rows_to_cover, int bm_rows, hipStream_t stream);

}  // namespace w4a8

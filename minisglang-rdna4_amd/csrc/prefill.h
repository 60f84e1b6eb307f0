// Pieces shared by the LDS-staged prefill / grouped GEMM kernels (gemm_prefill_lds.hip,
// gemm_prefill_dma.hip): weight-format modes, grouped-row lookup, the silu epilogue, the 1 KiB
// MFMA operand read and the per-stage LDS layout.
#pragma once
#include "gemm_args.h"

namespace w4a8 {

constexpr int kPSym = 0, kPAsym = 1, kPE8M0 = 2;

__device__ __forceinline__ bool lrow_source(const GemmArgs& p, int64_t r, int64_t& ar) {
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

__device__ __forceinline__ float lsilu_mul(float gate, float up, int dt) {
  // tools/w4a8_gemm_silu_parity.py:52-54: round to dtype, silu in f32, round, multiply in dtype
  const float g = from_dtype(to_dtype(gate, dt), dt);
  const float u = from_dtype(to_dtype(up, dt), dt);
  const float sg = g / (1.0f + expf(-g));
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

// Launch of the DMA-staged kernel (gemm_prefill_dma.hip); kErrUnsupported when it does not apply.
int launch_prefill_dma(const GemmArgs& p, int64_t rows_to_cover, int bm_rows, hipStream_t stream);

}  // namespace w4a8

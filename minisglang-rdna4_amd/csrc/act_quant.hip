// Per-token fp8-e4m3 activation quantization.
//
// Contract (python/minisgl/quant/kernels.py:1703-1712, python/minisgl/layers/norm.py:27-46):
// per row, amax = max |x|; s = max(amax / 448, 1e-8); q = e4m3_rne(x * (1 / s)), unclamped.
// The division and reciprocal are IEEE-rounded f32 operations; v_cvt_pk_fp8_f32 rounds to
// nearest even (checked bit-for-bit against the CPU restatement).
//
// One workgroup per row (grid-stride over rows), 16-byte vector loads; rows up to 32768 elements
// are read once into registers (one memory round trip), longer rows take two passes. Batches of
// 64 or more rows of up to 4096 elements take one wave per row instead. An optional
// device-side row count (the MoE padded row count) lets a graph-captured launch size the grid for
// the maximum and skip the tail.
#include "act_quant.h"

namespace w4a8 {

template <int CPT>
__global__ void __launch_bounds__(kAqThreads)
act_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t K, int dtype,
                 uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scales,
                 const int32_t* __restrict__ row_count) {
  __shared__ float red[kAqThreads / 64];
  int64_t rows = M;
  if (row_count) {
    const int64_t rc = *row_count;
    rows = rc < M ? rc : M;
  }
  for (int64_t m = blockIdx.x; m < rows; m += gridDim.x) quant_row<CPT>(x + m * ldx, K, dtype, q + m * ldq, scales + m, red);
}

// Many short rows (M >= 64, K <= 4096): one wave per row, 8 elements per lane per 16-byte chunk
// and CPW chunks per lane, reduced with wave_max alone (no LDS, no barrier). Same arithmetic as
// quant_row, bit for bit.
template <int CPW>
__global__ void __launch_bounds__(256)
act_quant_wave_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t K, int dtype,
                      uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scales,
                      const int32_t* __restrict__ row_count) {
  const int lane = threadIdx.x & 63;
  int64_t rows = M;
  if (row_count) {
    const int64_t rc = *row_count;
    rows = rc < M ? rc : M;
  }
  const int64_t stride = (int64_t)gridDim.x * (blockDim.x >> 6);
  for (int64_t m = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); m < rows; m += stride)
    quant_row_wave<CPW>(x + m * ldx, K, dtype, q + m * ldq, scales + m, lane);
}

// The codes of act_quant_kernel rewritten for the dense prefill GEMM in its A-operand order: per
// 16-row block and 128-wide K tile one 2 KiB block at ((row / 16) * KT + kt) * 2048 whose two 1 KiB
// halves hold, at lane l * 16, row (l & 15)'s bytes [16 (l >> 4), +16) and [64 + 16 (l >> 4), +16) of
// the tile -- what the GEMM's operand read gives lane l, so its LDS-DMA copies whole 1 KiB runs
// instead of 64-byte pieces of 16 rows. With them, per block and K tile, the GEMM's row-sum seed (the
// e4m3 -0.5 splat MFMA on that operand: the same instruction on the same bytes, so the same bits) at
// seeds[kt * seeds_ld + row], seeds_ld = M rounded up to 16. Rows past M in the last block are zero
// codes. One wave per (block, 4 K tiles), four per workgroup; every lane active at the MFMA.
__global__ void __launch_bounds__(256)
act_tile_kernel(const uint8_t* __restrict__ q, int64_t ldq, int64_t M, int KT, uint8_t* __restrict__ qt,
                float* __restrict__ seeds, int64_t seeds_ld) {
  // A wave takes a 16-row block and 4 consecutive K tiles: it reads the 16 rows' 512 bytes in row
  // order (two rows per instruction, 16 bytes per lane), stages them in LDS (rows padded to 33
  // chunks, so the operand reads below hit 16 different bank groups), then writes each tile's two
  // 1 KiB operand halves and its seeds. A wave per single tile read 16 rows' 64-byte pieces per
  // instruction and ran at about a third of HBM speed.
  __shared__ uint4 stg[4][16 * 33];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t nblk = (M + 15) / 16;
  const int KG = (KT + 3) / 4;  // groups of 4 K tiles
  const int64_t units = nblk * KG;
  const int r = lane & 15, qd = lane >> 4;
  uint4* st = stg[wave];
  for (int64_t u = (int64_t)blockIdx.x * 4 + wave; u < units; u += (int64_t)gridDim.x * 4) {
    const int64_t blk = u / KG;
    const int kt0 = (int)(u - blk * KG) * 4;
    const int nt = KT - kt0 < 4 ? KT - kt0 : 4;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rr = 2 * i + (lane >> 5), c = lane & 31;
      const int64_t m = blk * 16 + rr;
      const bool ok = m < M && c < nt * 8;
      st[rr * 33 + c] = ok ? *reinterpret_cast<const uint4*>(q + m * ldq + (int64_t)kt0 * kTileK + c * 16)
                           : make_uint4(0u, 0u, 0u, 0u);
    }
    // the wave reads back only what it wrote: LDS serves one wave's accesses in order
    for (int t = 0; t < nt; ++t) {
      const uint4 h0 = st[r * 33 + t * 8 + qd];
      const uint4 h1 = st[r * 33 + t * 8 + 4 + qd];
      uint8_t* dst = qt + (blk * KT + kt0 + t) * 2048 + lane * 16;
      *reinterpret_cast<uint4*>(dst) = h0;
      *reinterpret_cast<uint4*>(dst + 1024) = h1;
      v8i a;
      a[0] = (int)h0.x; a[1] = (int)h0.y; a[2] = (int)h0.z; a[3] = (int)h0.w;
      a[4] = (int)h1.x; a[5] = (int)h1.y; a[6] = (int)h1.z; a[7] = (int)h1.w;
      v4f pre = mfma_f8f8(a, splat8(0xB0B0B0B0u), v4f{0.f, 0.f, 0.f, 0.f});
      asm volatile("" : "+v"(pre));  // the MFMA runs with every lane active, before the lane branch
      // output lane l holds rows 4 (l >> 4) + i of column l & 15; column 0's lanes store them
      if (r == 0)
        *reinterpret_cast<float4*>(seeds + (int64_t)(kt0 + t) * seeds_ld + blk * 16 + 4 * qd) =
            make_float4(pre[0], pre[1], pre[2], pre[3]);
    }
  }
}

// act_quant_kernel and act_tile_kernel in one launch, for bf16/fp16 rows: one workgroup of 16 waves
// per 16-row block (grid-stride). Wave w first takes row w's maximum (the act-quant arithmetic: 16-byte
// chunks, wave_max), then the block's K tiles w, w + 16, ...: lane l quantizes row (l & 15)'s values
// [16 (l >> 4), +16) and [64 + 16 (l >> 4), +16) of the tile (the row is read a second time, from
// cache) into the operand-order block and runs the seed MFMA on them, as act_tile_kernel does on
// act_quant_kernel's codes. Same codes, scales and seeds, bit for bit; no row-major codes.
__global__ void __launch_bounds__(1024)
act_quant_tiled_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t K, int dtype,
                       uint8_t* __restrict__ qt, float* __restrict__ scales, float* __restrict__ seeds,
                       int64_t seeds_ld, const int32_t* __restrict__ row_count) {
  __shared__ float inv_s[16];
  int64_t rows = M;  // a device-side row count (the MoE padded row count) bounds the rows
  if (row_count) {
    const int64_t rc = *row_count;
    rows = rc < M ? rc : M;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int KT = (int)(K / kTileK);
  const int64_t nblk = (rows + 15) / 16;
  const int r = lane & 15, qd = lane >> 4;
  for (int64_t blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    {
      const int64_t m = blk * 16 + wave;
      float amax = 0.f;
      if (m < rows) {  // wave-uniform
        const uint16_t* xr = x + m * ldx;
        int64_t k = (int64_t)lane * 8;
        for (; k + 3 * 512 < K; k += 4 * 512) {
          const uint4 c0 = *reinterpret_cast<const uint4*>(xr + k);
          const uint4 c1 = *reinterpret_cast<const uint4*>(xr + k + 512);
          const uint4 c2 = *reinterpret_cast<const uint4*>(xr + k + 1024);
          const uint4 c3 = *reinterpret_cast<const uint4*>(xr + k + 1536);
          amax = fmaxf(amax, fmaxf(fmaxf(amax8(c0, dtype), amax8(c1, dtype)), fmaxf(amax8(c2, dtype), amax8(c3, dtype))));
        }
        for (; k < K; k += 512) amax = fmaxf(amax, amax8(*reinterpret_cast<const uint4*>(xr + k), dtype));
      }
      const float s = act_row_scale(wave_max(amax));
      if (lane == 0) {
        inv_s[wave] = 1.0f / s;
        if (m < rows) scales[m] = s;
      }
    }
    __syncthreads();
    const int64_t m = blk * 16 + r;
    const float inv = inv_s[r];
    const uint16_t* xr = x + (m < rows ? m : 0) * ldx;
    for (int kt = wave; kt < KT; kt += 16) {
      uint4 half[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t k = (int64_t)kt * kTileK + 64 * h + 16 * qd;
        float f[16];
        if (m < rows) {
          unpack8(*reinterpret_cast<const uint4*>(xr + k), dtype, f);
          unpack8(*reinterpret_cast<const uint4*>(xr + k + 8), dtype, f + 8);
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) f[i] = 0.f;
        }
        const uint2 c0 = quant8(f, inv), c1 = quant8(f + 8, inv);
        half[h] = make_uint4(c0.x, c0.y, c1.x, c1.y);
        *reinterpret_cast<uint4*>(qt + ((blk * KT + kt) * 2 + h) * 1024 + lane * 16) = half[h];
      }
      v8i a;
      a[0] = (int)half[0].x; a[1] = (int)half[0].y; a[2] = (int)half[0].z; a[3] = (int)half[0].w;
      a[4] = (int)half[1].x; a[5] = (int)half[1].y; a[6] = (int)half[1].z; a[7] = (int)half[1].w;
      v4f pre = mfma_f8f8(a, splat8(0xB0B0B0B0u), v4f{0.f, 0.f, 0.f, 0.f});
      asm volatile("" : "+v"(pre));  // the MFMA runs with every lane active, before the lane branch
      if (r == 0)
        *reinterpret_cast<float4*>(seeds + (int64_t)kt * seeds_ld + blk * 16 + 4 * qd) =
            make_float4(pre[0], pre[1], pre[2], pre[3]);
    }
    __syncthreads();  // inv_s is rewritten for the next block
  }
}

// act_quant_tiled_kernel's outputs for rows of up to 4096 elements, with x read once: wave w holds row
// w of the block in registers (lane l: the 8-element chunks l + 64 i), takes its maximum with wave_max,
// quantizes it (the act-quant arithmetic) and writes each chunk's 8 codes to its operand-order place
// in LDS; after one barrier wave w copies the block's K tiles w, w + 16, ... to global memory as 1 KiB
// runs and runs the seed MFMA on them. The two-pass kernel re-reads each row for its tiles, and with
// 16 rows of 8 KiB per workgroup those re-reads mostly miss L2 (M=8192 K=4096: 34.7 us against the
// row-major quant's 17). 16 * K bytes of LDS per workgroup; longer rows (16 chunks per lane spill)
// keep the two-pass kernel.
template <int CPL>
__global__ void __launch_bounds__(1024)
act_quant_tiled_lds_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t K, int dtype,
                           uint8_t* __restrict__ qt, float* __restrict__ scales, float* __restrict__ seeds,
                           int64_t seeds_ld, const int32_t* __restrict__ row_count) {
  extern __shared__ __align__(16) unsigned char cb[];  // [KT][2 halves][64 lanes][16 B]
  int64_t rows = M;  // as act_quant_tiled_kernel
  if (row_count) {
    const int64_t rc = *row_count;
    rows = rc < M ? rc : M;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int KT = (int)(K / kTileK);
  const int nch = (int)(K / 8);  // 16-byte chunks of a row
  const int64_t nblk = (rows + 15) / 16;
  for (int64_t blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    const int64_t m = blk * 16 + wave;
    const bool mok = m < rows;  // wave-uniform; rows past the bound give zero codes
    const uint16_t* xr = x + (mok ? m : 0) * ldx;
    uint4 raw[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = lane + 64 * i;
      raw[i] = (mok && c < nch) ? *reinterpret_cast<const uint4*>(xr + (int64_t)c * 8) : make_uint4(0u, 0u, 0u, 0u);
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) amax = fmaxf(amax, amax8(raw[i], dtype));
    const float s = act_row_scale(wave_max(amax));
    const float inv = 1.0f / s;
    if (lane == 0 && mok) scales[m] = s;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
        float f[8];
        unpack8(raw[i], dtype, f);
        // element k = 8c: tile k / 128, half (k % 128) / 64, operand lane row + 16 ((k % 64) / 16), byte k % 16
        const int k = c * 8, kk = k & 127;
        const int off = (((k >> 7) * 2 + (kk >> 6)) * 64 + wave + 16 * ((kk & 63) >> 4)) * 16 + (kk & 15);
        *reinterpret_cast<uint2*>(cb + off) = quant8(f, inv);
      }
    }
    __syncthreads();
    const int r = lane & 15, qd = lane >> 4;
    for (int kt = wave; kt < KT; kt += 16) {
      const uint4 h0 = *reinterpret_cast<const uint4*>(cb + (kt * 2) * 1024 + lane * 16);
      const uint4 h1 = *reinterpret_cast<const uint4*>(cb + (kt * 2 + 1) * 1024 + lane * 16);
      uint8_t* dst = qt + (blk * KT + kt) * 2048 + lane * 16;
      *reinterpret_cast<uint4*>(dst) = h0;
      *reinterpret_cast<uint4*>(dst + 1024) = h1;
      v8i a;
      a[0] = (int)h0.x; a[1] = (int)h0.y; a[2] = (int)h0.z; a[3] = (int)h0.w;
      a[4] = (int)h1.x; a[5] = (int)h1.y; a[6] = (int)h1.z; a[7] = (int)h1.w;
      v4f pre = mfma_f8f8(a, splat8(0xB0B0B0B0u), v4f{0.f, 0.f, 0.f, 0.f});
      asm volatile("" : "+v"(pre));  // the MFMA runs with every lane active, before the lane branch
      if (r == 0)
        *reinterpret_cast<float4*>(seeds + (int64_t)kt * seeds_ld + blk * 16 + 4 * qd) =
            make_float4(pre[0], pre[1], pre[2], pre[3]);
    }
    __syncthreads();  // the codes of the next block overwrite cb
  }
}

// The same for rows of up to 1024 elements (the MoE gemm2's K = inter, e.g. 768): a workgroup of 4
// waves per 16-row block, a 16-lane quarter of a wave per row (lane l of quarter q: row 4w + q,
// chunks (l & 15) + 16 i), the row maximum by a 16-lane DPP reduction; then wave w copies tiles
// w, w + 4, ... Short rows leave most of a 16-wave workgroup idle in the tile phase and allow only
// two of them per CU; these allow eight (K=768: the MoE gemm2's 41k padded rows 21.0 -> 18.8 us,
// M=32768 14.4 against 16.7).
template <int CPL>
__global__ void __launch_bounds__(256)
act_quant_tiled_short_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t K, int dtype,
                             uint8_t* __restrict__ qt, float* __restrict__ scales, float* __restrict__ seeds,
                             int64_t seeds_ld, const int32_t* __restrict__ row_count) {
  extern __shared__ __align__(16) unsigned char cb[];  // [KT][2 halves][64 lanes][16 B]
  int64_t rows = M;  // as act_quant_tiled_kernel
  if (row_count) {
    const int64_t rc = *row_count;
    rows = rc < M ? rc : M;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rib = 4 * wave + (lane >> 4), j = lane & 15;  // row in the block, lane in the row
  const int KT = (int)(K / kTileK);
  const int nch = (int)(K / 8);
  const int64_t nblk = (rows + 15) / 16;
  for (int64_t blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    const int64_t m = blk * 16 + rib;
    const bool mok = m < rows;  // rows past the bound give zero codes
    const uint16_t* xr = x + (mok ? m : 0) * ldx;
    uint4 raw[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = j + 16 * i;
      raw[i] = (mok && c < nch) ? *reinterpret_cast<const uint4*>(xr + (int64_t)c * 8) : make_uint4(0u, 0u, 0u, 0u);
    }
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) v = fmaxf(v, amax8(raw[i], dtype));
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppRowMirror>(v));
    const float s = act_row_scale(v);
    const float inv = 1.0f / s;
    if (j == 0 && mok) scales[m] = s;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = j + 16 * i;
      if (c < nch) {
        float f[8];
        unpack8(raw[i], dtype, f);
        const int k = c * 8, kk = k & 127;
        const int off = (((k >> 7) * 2 + (kk >> 6)) * 64 + rib + 16 * ((kk & 63) >> 4)) * 16 + (kk & 15);
        *reinterpret_cast<uint2*>(cb + off) = quant8(f, inv);
      }
    }
    __syncthreads();
    const int r = lane & 15, qd = lane >> 4;
    for (int kt = wave; kt < KT; kt += 4) {
      const uint4 h0 = *reinterpret_cast<const uint4*>(cb + (kt * 2) * 1024 + lane * 16);
      const uint4 h1 = *reinterpret_cast<const uint4*>(cb + (kt * 2 + 1) * 1024 + lane * 16);
      uint8_t* dst = qt + (blk * KT + kt) * 2048 + lane * 16;
      *reinterpret_cast<uint4*>(dst) = h0;
      *reinterpret_cast<uint4*>(dst + 1024) = h1;
      v8i a;
      a[0] = (int)h0.x; a[1] = (int)h0.y; a[2] = (int)h0.z; a[3] = (int)h0.w;
      a[4] = (int)h1.x; a[5] = (int)h1.y; a[6] = (int)h1.z; a[7] = (int)h1.w;
      v4f pre = mfma_f8f8(a, splat8(0xB0B0B0B0u), v4f{0.f, 0.f, 0.f, 0.f});
      asm volatile("" : "+v"(pre));  // the MFMA runs with every lane active, before the lane branch
      if (r == 0)
        *reinterpret_cast<float4*>(seeds + (int64_t)kt * seeds_ld + blk * 16 + 4 * qd) =
            make_float4(pre[0], pre[1], pre[2], pre[3]);
    }
    __syncthreads();  // the codes of the next block overwrite cb
  }
}

template <int CPL>
static int launch_act_quant_tiled_short(const uint16_t* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* qt,
                                        float* scales, float* seeds, int64_t seeds_ld, const int32_t* row_count,
                                        hipStream_t stream) {
  const int64_t nblk = (M + 15) / 16;
  const dim3 g((unsigned)(nblk < 65536 ? nblk : 65536)), b(256);
  hipLaunchKernelGGL(act_quant_tiled_short_kernel<CPL>, g, b, (size_t)(16 * K), stream, x, ldx, M, K, dtype, qt,
                     scales, seeds, seeds_ld, row_count);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

template <int CPL>
static int launch_act_quant_tiled_lds(const uint16_t* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* qt,
                                      float* scales, float* seeds, int64_t seeds_ld, const int32_t* row_count,
                                      hipStream_t stream) {
  auto kern = act_quant_tiled_lds_kernel<CPL>;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, 16 * 4096);
  (void)attr;
  const int64_t nblk = (M + 15) / 16;
  const dim3 g((unsigned)(nblk < 8192 ? nblk : 8192)), b(1024);
  hipLaunchKernelGGL(kern, g, b, (size_t)(16 * K), stream, x, ldx, M, K, dtype, qt, scales, seeds, seeds_ld, row_count);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

int launch_act_quant_tiled(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* qt, float* scales,
                           float* seeds, int64_t seeds_ld, const int32_t* row_count, hipStream_t stream) {
  if (M <= 0) return kOk;
  const uint16_t* xp = reinterpret_cast<const uint16_t*>(x);
  const int64_t c16 = (K / 8 + 15) / 16;  // 16-byte chunks per lane, 16 lanes per row
  if (c16 <= 4) return launch_act_quant_tiled_short<4>(xp, dtype, M, K, ldx, qt, scales, seeds, seeds_ld, row_count, stream);
  if (c16 <= 8) return launch_act_quant_tiled_short<8>(xp, dtype, M, K, ldx, qt, scales, seeds, seeds_ld, row_count, stream);
  const int64_t cpl = (K / 8 + 63) / 64;  // 16-byte chunks per lane for one row
  if (cpl <= 1) return launch_act_quant_tiled_lds<1>(xp, dtype, M, K, ldx, qt, scales, seeds, seeds_ld, row_count, stream);
  if (cpl <= 2) return launch_act_quant_tiled_lds<2>(xp, dtype, M, K, ldx, qt, scales, seeds, seeds_ld, row_count, stream);
  if (cpl <= 4) return launch_act_quant_tiled_lds<4>(xp, dtype, M, K, ldx, qt, scales, seeds, seeds_ld, row_count, stream);
  if (cpl <= 8) return launch_act_quant_tiled_lds<8>(xp, dtype, M, K, ldx, qt, scales, seeds, seeds_ld, row_count, stream);
  const int64_t nblk = (M + 15) / 16;
  const dim3 g((unsigned)(nblk < 8192 ? nblk : 8192)), b(1024);
  hipLaunchKernelGGL(act_quant_tiled_kernel, g, b, 0, stream, reinterpret_cast<const uint16_t*>(x), ldx, M, K, dtype,
                     qt, scales, seeds, seeds_ld, row_count);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

int launch_act_tile(const uint8_t* q, int64_t ldq, int64_t M, int64_t K, uint8_t* qt, float* seeds,
                    int64_t seeds_ld, hipStream_t stream) {
  if (M <= 0) return kOk;
  const int KT = (int)(K / kTileK);
  const int64_t units = (M + 15) / 16 * ((KT + 3) / 4);
  const int64_t wgs = (units + 3) / 4;
  const dim3 g((unsigned)(wgs < 65536 ? wgs : 65536)), b(256);
  hipLaunchKernelGGL(act_tile_kernel, g, b, 0, stream, q, ldq, M, KT, qt, seeds, seeds_ld);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

int launch_act_quant(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* q,
                     int64_t ldq, float* scales, const int32_t* row_count, hipStream_t stream) {
  if (M <= 0) return kOk;
  if (M >= 64 && K <= 64 * 8 * 8) {
    const int cpw = (int)((K + 511) / 512);
    const int64_t blocks = (M + 3) / 4;
    dim3 g((unsigned)(blocks < 16384 ? blocks : 16384)), b(256);
    const uint16_t* xp = reinterpret_cast<const uint16_t*>(x);
#define W4A8_AQW(C) hipLaunchKernelGGL(act_quant_wave_kernel<C>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count)
    if (cpw <= 1) W4A8_AQW(1);
    else if (cpw <= 2) W4A8_AQW(2);
    else if (cpw <= 4) W4A8_AQW(4);
    else W4A8_AQW(8);
#undef W4A8_AQW
    return hipGetLastError() == hipSuccess ? kOk : kErrHip;
  }
  const int64_t grid = M < 8192 ? M : 8192;
  const uint16_t* xp = reinterpret_cast<const uint16_t*>(x);
  dim3 g((unsigned)grid), b(kAqThreads);
  switch (quant_row_cpt(K)) {
    case 1: hipLaunchKernelGGL(act_quant_kernel<1>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count); break;
    case 2: hipLaunchKernelGGL(act_quant_kernel<2>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count); break;
    case 4: hipLaunchKernelGGL(act_quant_kernel<4>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count); break;
    case 8: hipLaunchKernelGGL(act_quant_kernel<8>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count); break;
    case 16: hipLaunchKernelGGL(act_quant_kernel<16>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count); break;
    default: hipLaunchKernelGGL(act_quant_kernel<0>, g, b, 0, stream, xp, ldx, M, K, dtype, q, ldq, scales, row_count);
  }
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

}  // namespace w4a8

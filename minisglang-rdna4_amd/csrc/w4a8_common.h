// Shared definitions for the gfx950 (CDNA4) W4A8 kernels.
//
// MFMA operand layouts used throughout (v_mfma_scale_f32_16x16x128_f8f6f4, measured on MI355X):
//   * fp8 operand (A activations, or B weights after int4 unpack): lane l, q = l >> 4, holds the
//     32 bytes of row/column (l & 15) at K offsets [16q, 16q+16) in bytes 0..15 and
//     [64+16q, 64+16q+16) in bytes 16..31 of its 8 VGPRs.
//   * fp4 operand (B weights, MXFP4): lane l holds K offsets [32q, 32q+32) in 4 VGPRs, element
//     32q+e in nibble (e & 1) of byte e/2 -- the checkpoint's own packing order.
//   * E8M0 block scales: the scale of row/column i for K block b (32 wide) is read from lane i+16b.
//   * C (16x16 f32): lane l holds rows 4q + r (r = 0..3) of column l & 15.
//
// Weight tile layout in HBM ("W4 tile"): a matrix of N output channels x K inputs is cut into
// 16-channel x 128-K tiles of 1024 bytes, ordered [N/16][ceil(K/128)][64 lanes][16 bytes], so a
// wave loads one tile as one coalesced 1 KB request and each lane receives exactly its MFMA
// operand. Codes stay 4-bit.
//   * int4: the 16 bytes of lane l are four dwords d; byte i of dword d holds operand element
//     8d+i in its low nibble and 8d+4+i in its high nibble, where operand element e maps to K as
//     in the fp8 layout above. The nibble is a sign-magnitude code of (q - 7.5):
//     c = q >= 8 ? q - 8 : 15 - q, value = (c & 8 ? -1 : 1) * ((c & 7) + 0.5). One v_perm over an
//     8-entry e4m3 table plus a sign OR turns it into fp8. The -0.5 shift is undone with the row
//     sums R (sum_k x) that an extra MFMA against a constant 0.5 operand provides:
//       sum_k x (q - z) = sum_k x v + (7.5 - z) * R.
//   * e2m1: lane l's 16 bytes are the checkpoint's 4 words for K [32q, 32q+32), unchanged.
// K is padded to a multiple of 128 with code 0 (activations there are zero).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a8 {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kTileN = 16;
constexpr int kTileK = 128;
constexpr int kTileBytes = 1024;

// status codes shared with the C ABI
constexpr int kOk = 0;
constexpr int kErrInvalid = 1;
constexpr int kErrUnsupported = 2;
constexpr int kErrHip = 3;

enum DType { kBF16 = 0, kF16 = 1, kF32 = 2 };
// kScaleE4M3: NVFP4's e4m3 block scales (group 16), times a per-output-channel f32 global that
// rides the zeros slot (e2m1 weights have no zero points)
enum ScaleFmt { kScaleF16 = 0, kScaleE8M0 = 1, kScaleE4M3 = 2 };
enum WFmt { kInt4 = 0, kE2M1 = 1 };

// e4m3 constants
constexpr uint32_t kE4M3Half4 = 0x30303030u;  // +0.5 in every byte

// fp8 x fp8 MFMA, unit scales.
__device__ __forceinline__ v4f mfma_f8f8(const v8i& a, const v8i& b, const v4f& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}
// fp8 x fp8 with a per-lane B block scale (E8M0 byte in the low byte of sb).
__device__ __forceinline__ v4f mfma_f8f8_sb(const v8i& a, const v8i& b, const v4f& c, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, sb);
}
// fp8 (A) x fp4 e2m1 (B) with a per-lane B block scale.
__device__ __forceinline__ v4f mfma_f8f4_sb(const v8i& a, const v8i& b, const v4f& c, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 4, 0, 127, 0, sb);
}

// Sign-magnitude int4 code -> e4m3 bytes. LUT magnitudes (t + 0.5), t = 0..7:
// 0.5 1.5 2.5 3.5 4.5 5.5 6.5 7.5 -> 30 3C 42 46 49 4B 4D 4F.
__device__ __forceinline__ void unpack_sm4(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t L0 = 0x46423C30u, L1 = 0x4F4D4B49u;
  uint32_t t0 = __builtin_amdgcn_perm(L1, L0, w & 0x07070707u);
  lo = ((w << 4) & 0x80808080u) | t0;
  uint32_t t1 = __builtin_amdgcn_perm(L1, L0, (w >> 4) & 0x07070707u);
  hi = (w & 0x80808080u) | t1;
}

// 16 stored bytes (uint4) -> 8-VGPR fp8 operand.
__device__ __forceinline__ v8i unpack_tile_int4(const uint4& raw) {
  v8i b;
  uint32_t lo, hi;
  unpack_sm4(raw.x, lo, hi); b[0] = (int)lo; b[1] = (int)hi;
  unpack_sm4(raw.y, lo, hi); b[2] = (int)lo; b[3] = (int)hi;
  unpack_sm4(raw.z, lo, hi); b[4] = (int)lo; b[5] = (int)hi;
  unpack_sm4(raw.w, lo, hi); b[6] = (int)lo; b[7] = (int)hi;
  return b;
}

__device__ __forceinline__ v8i fp4_operand(const uint4& raw) {
  v8i b;
  b[0] = (int)raw.x; b[1] = (int)raw.y; b[2] = (int)raw.z; b[3] = (int)raw.w;
  b[4] = 0; b[5] = 0; b[6] = 0; b[7] = 0;
  return b;
}

__device__ __forceinline__ v8i splat8(uint32_t v) {
  v8i b;
#pragma unroll
  for (int i = 0; i < 8; ++i) b[i] = (int)v;
  return b;
}

// bf16 / fp16 scalar helpers (RNE)
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }
// Round to nearest even; a NaN keeps its sign and top payload bits and is made quiet ((u >> 16) |
// 0x40). gfx950's v_cvt_pk_bf16_f32, which the __bf16 conversion compiles to, gives exactly these
// bits: checked on the GPU against the integer form ((u + 0x7fff + ((u >> 16) & 1)) >> 16, the NaN
// select) over all 65536 upper halves with 8 lower halves each (ties, subnormals, NaN payloads) and
// 2^25 random patterns, no difference. One instruction instead of six. The empty asm pins f as an
// f32 value, as for fp16 below.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// The empty asm pins f as an f32 value: without it the compiler may contract a producing f32
// multiply and this conversion into one mixed-precision op (v_mad_mixlo_f16) with a single
// rounding, where the f32 product and then the f16 conversion round twice.
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float load_act(const uint16_t* p, int dtype) {
  return dtype == kBF16 ? bf16_to_f32(*p) : f16_to_f32(*p);
}
__device__ __forceinline__ uint16_t to_dtype(float v, int dtype) {
  return dtype == kBF16 ? f32_to_bf16(v) : f32_to_f16(v);
}
__device__ __forceinline__ float from_dtype(uint16_t h, int dtype) {
  return dtype == kBF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

// ---- buffer loads: wave-uniform base and size in a resource descriptor (SGPRs), 32-bit per-lane
// offset, and a scalar offset that the compiler computes with SALU. Loads past `bytes` return 0.
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t BufRsrc;

__device__ __forceinline__ BufRsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload128(BufRsrc r, uint32_t voff, uint32_t soff) {
  const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ v4u bload128v(BufRsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
__device__ __forceinline__ uint2 bload64(BufRsrc r, uint32_t voff, uint32_t soff) {
  typedef unsigned int v2u __attribute__((ext_vector_type(2)));
  const v2u v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
  return make_uint2(v.x, v.y);
}
// streaming (non-temporal) variant for data read exactly once, such as weight tiles
__device__ __forceinline__ uint4 bload128_nt(BufRsrc r, uint32_t voff, uint32_t soff) {
  const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t bload32(BufRsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
__device__ __forceinline__ uint16_t bload16(BufRsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}
__device__ __forceinline__ uint8_t bload8(BufRsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, voff, soff, 0);
}

// LDS-DMA (buffer_load ... lds) of 16 (or 4) bytes per lane into lds + lane * 16 (lane * 4): the
// buffer unit writes LDS directly, no VGPR holds the data, and the wave's vmcnt tracks completion.
// The generic-to-LDS pointer cast only exists for the device target, so the host pass (which only
// needs the kernels' launch stubs) compiles an empty body.
__device__ __forceinline__ void lds_dma16(BufRsrc r, unsigned char* lds, uint32_t voff, uint32_t soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
#endif
}
// (an LDS-DMA lane always lands 4 bytes at lds + lane * 4, whatever the load size: E8M0 bytes
// travel as dwords)
__device__ __forceinline__ void lds_dma4(BufRsrc r, unsigned char* lds, uint32_t voff, uint32_t soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4, voff, soff, 0, 0);
#endif
}

// ---- per-token fp8 activation quant pieces (shared by the act-quant kernel and the decode GEMV's
// fused prologue, so both produce the same codes bit for bit)
//
// Wave reductions: four DPP steps (lanes xor 1, xor 2, then the 8- and 16-lane mirrors) leave every
// lane of each 16-lane row with the row's result, then four readlanes combine the rows. DPP moves
// are plain VALU operands, so this costs tens of cycles where a shuffle (ds_bpermute) costs an
// LDS round trip per step. All lanes must be active (uniform control flow).
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppRowMirror = 0x140, kDppHalfMirror = 0x141;
template <int CTRL> __device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations, not for its global
// loads and stores in flight (__syncthreads waits for every outstanding memory operation of the
// wave, which would drain a window of weight loads issued ahead of it). Register results of global
// loads are still waited for where they are used, as always. For data shared through LDS only; the
// memory clobber keeps the compiler from moving memory operations across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// max is exact and order-free: every lane returns the same bits whatever the order
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppRowMirror>(v));
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// f32 sum in a fixed tree order; every lane returns the same bits
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  v += dpp_f<kDppRowMirror>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

// 8 bf16/fp16 values (one 16-byte load) -> f32
__device__ __forceinline__ void unpack8(const uint4& u, int dtype, float* f) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = from_dtype((uint16_t)(w[i] & 0xffffu), dtype);
    f[2 * i + 1] = from_dtype((uint16_t)(w[i] >> 16), dtype);
  }
}

__device__ __forceinline__ float amax8(const uint4& u, int dtype) {
  float f[8];
  unpack8(u, dtype, f);
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(f[i]));
  return m;
}

// s = max(amax / 448, 1e-8) (IEEE f32 division)
__device__ __forceinline__ float act_row_scale(float amax) {
  float s = amax / 448.0f;
  if (s < 1e-8f) s = 1e-8f;
  return s;
}

// 8 values times inv, to e4m3 with round-to-nearest-even (v_cvt_pk_fp8_f32), packed little-endian
__device__ __forceinline__ uint2 quant8(const float* f, float inv) {
  uint32_t lo = 0, hi = 0;
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[0] * inv, f[1] * inv, lo, false);
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[2] * inv, f[3] * inv, lo, true);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[4] * inv, f[5] * inv, hi, false);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[6] * inv, f[7] * inv, hi, true);
  return make_uint2(lo, hi);
}

// A operand: row pointer (already offset to the tile's K start), valid K extent in bytes from
// the tile start (multiple of 16). Rows with a null pointer give zeros.
__device__ __forceinline__ v8i load_a_operand(const uint8_t* row, int kvalid, int lane) {
  v8i a;
  const int q = lane >> 4;
  uint4 lo = make_uint4(0, 0, 0, 0), hi = make_uint4(0, 0, 0, 0);
  if (row) {
    if (16 * q < kvalid) lo = *reinterpret_cast<const uint4*>(row + 16 * q);
    if (64 + 16 * q < kvalid) hi = *reinterpret_cast<const uint4*>(row + 64 + 16 * q);
  }
  a[0] = (int)lo.x; a[1] = (int)lo.y; a[2] = (int)lo.z; a[3] = (int)lo.w;
  a[4] = (int)hi.x; a[5] = (int)hi.y; a[6] = (int)hi.z; a[7] = (int)hi.w;
  return a;
}

// Per-lane B scale that keeps only the K blocks of sub-group `sg` (of width 128/gpt) for
// groups narrower than a tile: 127 (x1) for the lane's block inside the sub-group, 0 (x2^-127,
// i.e. far below one f32 ulp of any accumulated value) outside it.
__device__ __forceinline__ int subgroup_mask_scale(int lane, int gpt, int sg) {
  const int blk = lane >> 4;           // K block (32 wide) the lane's scale governs
  if (gpt == 8) return (blk == (sg >> 1)) ? 127 : 0;  // 16-wide groups: half a block each
  const int per = 4 / gpt;             // blocks per sub-group
  return (blk / per == sg) ? 127 : 0;
}

// 16-wide sub-group sg of an e2m1 operand (8 groups per 128-element tile): a lane's 16 bytes hold
// its block's elements 0..31 in order, two per byte, so the other half of the block is zeroed
__device__ __forceinline__ v8i fp4_half_operand(const v8i& b, int sg) {
  v8i h = b;
  if (sg & 1) { h[0] = 0; h[1] = 0; }
  else { h[2] = 0; h[3] = 0; }
  return h;
}

__device__ __forceinline__ float load_scale(const void* scales, int fmt, int64_t idx) {
  if (fmt == kScaleF16) return f16_to_f32(reinterpret_cast<const uint16_t*>(scales)[idx]);
  uint32_t s = reinterpret_cast<const uint8_t*>(scales)[idx];
  if (fmt == kScaleE4M3) return __builtin_amdgcn_cvt_f32_fp8((int)s, 0);
  return s == 0 ? 5.877471754111438e-39f : __uint_as_float(s << 23);
}

// group scale of output channel n: the stored scale, times the NVFP4 global (zeros slot, f32 bits)
// when zeros is given (kernels that apply the global in their epilogue pass null)
__device__ __forceinline__ float group_scale(const void* scales, int fmt, int64_t idx, const int32_t* zeros, int64_t n) {
  const float s = load_scale(scales, fmt, idx);
  return (fmt == kScaleE4M3 && zeros) ? s * __int_as_float(zeros[n]) : s;
}

}  // namespace w4a8

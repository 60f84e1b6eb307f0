/*
 * w4a8_oracle.c -- CPU restatement of minisglang-rdna4's W4A8 quantized-linear arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker for the HIP path: it is linked by
 * tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and by nothing else.
 * The product path (the package's C-ABI library) never calls it and has no CPU fallback.
 *
 * Every function cites the reference file:line whose behaviour it restates (paths relative to the
 * reference repository root). The reference's kernels live in an external repository that is not
 * part of the reference tree, so the contracts below are restated from the Python provider layer,
 * its docstrings and its parity harnesses.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   e4m3 codec      -- torch's float8_e4m3fn cast (RNE) over every code, every midpoint, +-1 ulp
 *                      around each midpoint and random values; closed-form decode of all 256 codes.
 *   act_quant       -- closed form per row (amax/448 floor 1e-8, reciprocal multiply, RNE) checked
 *                      against a numpy restatement built on torch's cast; special rows (all-zero,
 *                      single outlier, amax exactly 448, subnormal-only rows).
 *   e2m1 / e8m0     -- the LUT of python/minisgl/quant/mxfp4.py:37-38 and the shift decode of
 *                      tests/mxfp4_e8m0_test.py:23-42 over every code.
 *   gemm            -- brute force on tiny inputs against a dequantize-then-matmul numpy path,
 *                      and the invariants M-invariance / row-split / linearity in the weights.
 *   moe align       -- the worked example in python/minisgl/moe/fused.py:80-97.
 *   w4a16 moe       -- composition of pinned pieces: a single routed expert with weight 1 equals the
 *                      dense chain w4a16_gemm -> silu_mul -> w4a16_gemm (numpy f64 matmuls over
 *                      w4o_dequant); linearity in the top-k weights; dropped slots contribute 0.
 *   w4a16 split     -- the identity x == sum_t scale_t * e4m3(code_t) (exact for every bf16 value
 *                      and every fp16 value whose scaled magnitude is >= 2^-6), the scale being the
 *                      smallest power of two with amax/scale <= 448 (checked against frexp), and
 *                      each term's code being the RNE e4m3 of its residual (torch's cast).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

/* ------------------------------------------------------------------------------------------ */
/* bf16 / fp16 scalar conversions (IEEE RNE), used for activations and outputs.                 */
/* ------------------------------------------------------------------------------------------ */
static inline float u32_as_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_as_u32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float w4o_bf16_to_f32(uint16_t h) { return u32_as_f32(((uint32_t)h) << 16); }

uint16_t w4o_f32_to_bf16(float f) {
  uint32_t u = f32_as_u32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

float w4o_f16_to_f32(uint16_t h) {
  uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m | 1024u), (int)e - 25);
  return s ? -v : v;
}

uint16_t w4o_f32_to_f16(float f) {
  /* via double: every f16 value and midpoint is exact in double, so RNE on the double is RNE. */
  uint32_t u = f32_as_u32(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  float a = fabsf(f);
  if (isnan(f)) return (uint16_t)(sign | 0x7e00u);
  if (a >= 65520.0f) return (uint16_t)(sign | 0x7c00u);
  if (a < ldexpf(1.0f, -14)) {
    double q = (double)a * 16777216.0; /* units of 2^-24 */
    double r = nearbyint(q);           /* default rounding mode: ties-to-even */
    return (uint16_t)(sign | (uint16_t)r);
  }
  int e;
  double m = frexp((double)a, &e); /* a = m * 2^e, m in [0.5,1) */
  double q = ldexp(m, 11);         /* [1024, 2048) */
  double r = nearbyint(q);
  if (r >= 2048.0) { r = 1024.0; e += 1; }
  int be = e - 1 + 15;
  if (be >= 31) return (uint16_t)(sign | 0x7c00u);
  return (uint16_t)(sign | (uint16_t)(be << 10) | ((uint16_t)r & 1023u));
}

/* ------------------------------------------------------------------------------------------ */
/* OCP fp8 e4m3fn codec.                                                                        */
/* Restates the "UNCLAMPED f32_to_e4m3" with round-to-nearest-even that the reference's act-quant */
/* uses (python/minisgl/quant/kernels.py:1703-1712; RNE per docs/journal/PERF_NOTES.md:53).       */
/* Format: 1 sign, 4 exponent (bias 7), 3 mantissa; no infinities; S.1111.111 is NaN; max 448.   */
/* Overflow (|v| >= 464, the midpoint above 448) encodes NaN, like torch's float8_e4m3fn cast.    */
/* ------------------------------------------------------------------------------------------ */
float w4o_e4m3_to_f32(uint8_t c) {
  int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
  float v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf((float)(8 + m), e - 10);
  return s ? -v : v;
}

uint8_t w4o_f32_to_e4m3(float f) {
  uint8_t sign = (uint8_t)((f32_as_u32(f) >> 24) & 0x80u);
  if (isnan(f)) return (uint8_t)(sign | 0x7f);
  double a = fabs((double)f);
  if (a >= 464.0) return (uint8_t)(sign | 0x7f);
  if (a < ldexp(1.0, -6)) {
    /* subnormal range: multiples of 2^-9; RNE on the quotient (exact in double). */
    double r = nearbyint(a * 512.0);
    /* r == 8 is the smallest normal (2^-6), which has code 0x08: same bit pattern. */
    return (uint8_t)(sign | (uint8_t)r);
  }
  int e;
  double m = frexp(a, &e);  /* a = m*2^e, m in [0.5,1) */
  double q = ldexp(m, 4);   /* [8,16): 8 + mantissa */
  double r = nearbyint(q);  /* ties-to-even on the 3-bit mantissa */
  if (r >= 16.0) { r = 8.0; e += 1; }
  int be = e - 1 + 7;       /* a = (r/8) * 2^(e-1) */
  if (be > 15 || (be == 15 && r == 15.0)) return (uint8_t)(sign | 0x7f);
  return (uint8_t)(sign | (uint8_t)(be << 3) | (uint8_t)((int)r - 8));
}

/* ------------------------------------------------------------------------------------------ */
/* Per-token activation quant.                                                                 */
/* Restates python/minisgl/quant/kernels.py:1703-1712 (amax/448 with a 1e-8 floor, reciprocal-  */
/* multiply, unclamped RNE e4m3) and python/minisgl/layers/norm.py:27-46 (the producer emits the */
/* same pair over the already-rounded output row). The floor is applied to the scale:            */
/*   amax = max_k |x[m,k]|; s = max(amax / 448, 1e-8); q = e4m3(x * (1/s)).                      */
/* (Floor placement and the f32 reciprocal are the chosen reading of that prose: parity with the */
/* external kernel at the floor is unpinned.)                                                     */
/* dtype: 0 = bf16, 1 = fp16.                                                                     */
/* ------------------------------------------------------------------------------------------ */
void w4o_act_quant(const uint16_t* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* q,
                   float* scales) {
  for (int64_t m = 0; m < M; ++m) {
    const uint16_t* row = x + m * ldx;
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      float v = dtype == 0 ? w4o_bf16_to_f32(row[k]) : w4o_f16_to_f32(row[k]);
      float a = fabsf(v);
      if (a > amax) amax = a;
    }
    volatile float s = amax / 448.0f;
    if (s < 1e-8f) s = 1e-8f;
    volatile float inv = 1.0f / s;
    for (int64_t k = 0; k < K; ++k) {
      float v = dtype == 0 ? w4o_bf16_to_f32(row[k]) : w4o_f16_to_f32(row[k]);
      volatile float t = v * inv;
      q[m * K + k] = w4o_f32_to_e4m3(t);
    }
    scales[m] = s;
  }
}

/* ------------------------------------------------------------------------------------------ */
/* 4-bit weight decode.                                                                         */
/* E2M1 LUT: python/minisgl/quant/mxfp4.py:37-38. E8M0 decode 2^(s-127), s=0 -> 2^-127:          */
/* tests/mxfp4_e8m0_test.py:23-42. int4: w = code - zero, zero=8 when no zeros tensor is given   */
/* (symmetric uint4b8, tools/moe_parity.py:24-27); zeros packed 8 channels per int32 along N,    */
/* zero(g,n) = (z[g*(N/8) + n/8] >> 4*(n%8)) & 0xF (python/minisgl/quant/kernels.py:286-291).    */
/* ------------------------------------------------------------------------------------------ */
static const float E2M1_LUT[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                   -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

float w4o_e2m1_to_f32(uint8_t code) { return E2M1_LUT[code & 15]; }

double w4o_e8m0_to_f64(uint8_t s) {
  if (s == 255) return INFINITY; /* the (s << 23) shift decode lands on +inf */
  return ldexp(1.0, (int)s - 127);
}

static inline int code_at(const int32_t* w_packed, int64_t K, int64_t n, int64_t k) {
  uint32_t word = (uint32_t)w_packed[n * (K / 8) + k / 8];
  return (int)((word >> (4 * (k % 8))) & 15u);
}

/* Weight value (before the group scale) for op-layout element (n, k).
 * fmt: 0 = int4 with fp16 group scale, 1 = e2m1 (codes) */
static inline double weight_val(const int32_t* w_packed, const int32_t* zeros, int64_t N, int64_t K,
                                int64_t group, int e2m1, int64_t n, int64_t k) {
  int c = code_at(w_packed, K, n, k);
  if (e2m1) return (double)E2M1_LUT[c];
  int z = 8;
  if (zeros) {
    int64_t g = k / group;
    uint32_t zw = (uint32_t)zeros[g * (N / 8) + n / 8];
    z = (int)((zw >> (4 * (n % 8))) & 15u);
  }
  return (double)(c - z);
}

/* scale_fmt 2 (NVFP4, python/minisgl/quant/nvfp4.py:1-60 and quant/kernels.py:518-559): an e4m3
 * block scale times the per-output-channel f32 global multiplier, which rides the zeros slot. */
static inline double scale_val(const void* scales, int scale_fmt, int64_t N, int64_t g, int64_t n,
                               const int32_t* zeros) {
  if (scale_fmt == 1) return w4o_e8m0_to_f64(((const uint8_t*)scales)[g * N + n]);
  if (scale_fmt == 2) {
    float glob;
    memcpy(&glob, &zeros[n], 4);
    return (double)w4o_e4m3_to_f32(((const uint8_t*)scales)[g * N + n]) * (double)glob;
  }
  return (double)w4o_f16_to_f32(((const uint16_t*)scales)[g * N + n]);
}

/* ------------------------------------------------------------------------------------------ */
/* Dense W4A8 GEMM: restates the op contract of python/minisgl/quant/kernels.py:1686-1734        */
/* (mmq_fp8_gemm): y[m,n] = s_m * sum_g scale[g,n] * sum_{k in g} e4m3(q[m,k]) * w(n,k), with      */
/* scales GROUP-MAJOR (K/g, N) (kernels.py:265-268). Accumulated in f64 (exact per group).        */
/* w_packed: (N, K/8) int32, nibble j of word k/8 holds k%8 (kernels.py:279-281).                 */
/* scale_fmt: 0 fp16, 1 E8M0 uint8. zeros: (K/g, N/8) int32 or NULL.                               */
/* ------------------------------------------------------------------------------------------ */
void w4o_gemm(const uint8_t* xq, const float* act_scales, int64_t M, int64_t K,
              const int32_t* w_packed, int64_t N, const void* scales, int scale_fmt,
              const int32_t* zeros, int e2m1, int64_t group, double* out) {
  int64_t G = K / group;
  double* xv = (double*)malloc(sizeof(double) * (size_t)(M * K));
  for (int64_t i = 0; i < M * K; ++i) xv[i] = (double)w4o_e4m3_to_f32(xq[i]);
#pragma omp parallel
  {
    double* wrow = (double*)malloc(sizeof(double) * (size_t)K);
    double* sc = (double*)malloc(sizeof(double) * (size_t)G);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      for (int64_t k = 0; k < K; ++k) wrow[k] = weight_val(w_packed, zeros, N, K, group, e2m1, n, k);
      for (int64_t g = 0; g < G; ++g) sc[g] = scale_val(scales, scale_fmt, N, g, n, zeros);
      for (int64_t m = 0; m < M; ++m) {
        const double* xr = xv + m * K;
        double acc = 0.0;
        for (int64_t g = 0; g < G; ++g) {
          double part = 0.0;
          for (int64_t k = g * group; k < (g + 1) * group; ++k) part += xr[k] * wrow[k];
          acc += sc[g] * part;
        }
        out[m * N + n] = (double)act_scales[m] * acc;
      }
    }
    free(sc);
    free(wrow);
  }
  free(xv);
}

/* Dequantized weight (N, K) in f64 -- the "dequantize W" half of the reference's CPU path
 * (tools/moe_parity.py:24-27, python/minisgl/quant/mxfp4.py:262-275). */
void w4o_dequant(const int32_t* w_packed, int64_t N, int64_t K, const void* scales, int scale_fmt,
                 const int32_t* zeros, int e2m1, int64_t group, double* out) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k)
      out[n * K + k] = scale_val(scales, scale_fmt, N, k / group, n, zeros) *
                       weight_val(w_packed, zeros, N, K, group, e2m1, n, k);
}

/* ------------------------------------------------------------------------------------------ */
/* MoE routing: softmax over f32 logits, top-k with EXACT TIES KEEPING THE LOWER EXPERT INDEX     */
/* (python/minisgl/layers/moe.py:1218-1227), renormalised by sum + 1e-8                           */
/* (python/minisgl/moe/fused.py:52-53, tools/moe_parity.py:31-33). Selection is on the logits,   */
/* which orders experts exactly as the softmax does.                                             */
/* logits: (T, E) f32. tw: (T, k) f32; ids: (T, k) int32.                                         */
/* ------------------------------------------------------------------------------------------ */
void w4o_moe_route(const float* logits, int64_t T, int64_t E, int64_t top_k, int renormalize,
                   float* tw, int32_t* ids) {
  double* p = (double*)malloc(sizeof(double) * (size_t)E);
  char* used = (char*)malloc((size_t)E);
  for (int64_t t = 0; t < T; ++t) {
    const float* l = logits + t * E;
    double mx = -INFINITY;
    for (int64_t e = 0; e < E; ++e) if (l[e] > mx) mx = l[e];
    double sum = 0.0;
    for (int64_t e = 0; e < E; ++e) { p[e] = exp((double)l[e] - mx); sum += p[e]; }
    for (int64_t e = 0; e < E; ++e) p[e] /= sum;
    memset(used, 0, (size_t)E);
    double wsum = 0.0;
    for (int64_t j = 0; j < top_k; ++j) {
      int64_t best = -1;
      for (int64_t e = 0; e < E; ++e) {
        if (used[e]) continue;
        if (best < 0 || l[e] > l[best]) best = e; /* strict '>' keeps the lower index on ties */
      }
      used[best] = 1;
      ids[t * top_k + j] = (int32_t)best;
      tw[t * top_k + j] = (float)p[best];
      wsum += p[best];
    }
    if (renormalize)
      for (int64_t j = 0; j < top_k; ++j)
        tw[t * top_k + j] = (float)((double)tw[t * top_k + j] / (wsum + 1e-8));
  }
  free(used);
  free(p);
}

/* ------------------------------------------------------------------------------------------ */
/* moe_align_block_size: restates python/minisgl/moe/fused.py:120-176.                           */
/* sorted_ids has capacity P = T*k + (E+1)*(bm-1) (fused.py:94), pre-filled with the sentinel    */
/* T*k; each expert's slots in increasing flat index order (stable), padded to a multiple of bm;  */
/* expert_ids[b] = owning expert of block b, blocks past the end clamp to E-1; ntp = padded sum. */
/* Returns P. inv_pos (optional, T*k) gets each slot's position in sorted_ids. Ids outside       */
/* [0, E) (experts an expert-parallel rank does not hold) are dropped slots: not placed,         */
/* inv_pos -1.                                                                                   */
/* ------------------------------------------------------------------------------------------ */
int64_t w4o_moe_align(const int32_t* ids, int64_t numel, int64_t E, int64_t bm, int32_t* sorted_ids,
                      int32_t* expert_ids, int32_t* ntp, int32_t* inv_pos) {
  int64_t P = numel + (E + 1) * (bm - 1);
  int64_t nblocks = (P + bm - 1) / bm;
  int64_t* cnt = (int64_t*)calloc((size_t)E, sizeof(int64_t));
  int64_t* start = (int64_t*)calloc((size_t)E, sizeof(int64_t));
  int64_t* fill = (int64_t*)calloc((size_t)E, sizeof(int64_t));
  for (int64_t i = 0; i < numel; ++i)
    if (ids[i] >= 0 && ids[i] < E) cnt[ids[i]]++;
  int64_t pos = 0;
  for (int64_t e = 0; e < E; ++e) {
    start[e] = pos;
    pos += (cnt[e] + bm - 1) / bm * bm;
  }
  for (int64_t i = 0; i < P; ++i) sorted_ids[i] = (int32_t)numel;
  for (int64_t i = 0; i < numel; ++i) {
    int64_t e = ids[i];
    if (e < 0 || e >= E) {
      if (inv_pos) inv_pos[i] = -1;
      continue;
    }
    int64_t d = start[e] + fill[e]++;
    sorted_ids[d] = (int32_t)i;
    if (inv_pos) inv_pos[i] = (int32_t)d;
  }
  for (int64_t b = 0; b < nblocks; ++b) {
    int64_t owner = E - 1;
    for (int64_t e = 0; e < E; ++e) {
      int64_t nb = (cnt[e] + bm - 1) / bm;
      if (nb > 0 && b * bm >= start[e] && b * bm < start[e] + nb * bm) { owner = e; break; }
    }
    expert_ids[b] = (int32_t)owner;
  }
  *ntp = (int32_t)pos;
  free(cnt); free(start); free(fill);
  return P;
}

/* SiLU-and-mul epilogue of the fused gate_up GEMM, restating the replica in
 * tools/w4a8_gemm_silu_parity.py:52-54: round gate/up to the output dtype, silu in f32, round,
 * multiply in the dtype (i.e. f32 product rounded once). dtype: 0 bf16, 1 fp16. */
static inline uint16_t to_dt(float v, int dtype) { return dtype == 0 ? w4o_f32_to_bf16(v) : w4o_f32_to_f16(v); }
static inline float from_dt(uint16_t h, int dtype) { return dtype == 0 ? w4o_bf16_to_f32(h) : w4o_f16_to_f32(h); }

uint16_t w4o_silu_mul(double gate, double up, int dtype) {
  float g = from_dt(to_dt((float)gate, dtype), dtype);
  float u = from_dt(to_dt((float)up, dtype), dtype);
  volatile float den = 1.0f + expf(-g);
  volatile float sg = g / den;
  float sh = from_dt(to_dt(sg, dtype), dtype);
  volatile float prod = sh * u;
  return to_dt(prod, dtype);
}

/* ------------------------------------------------------------------------------------------ */
/* Grouped W4A8 MoE forward: restates python/minisgl/quant/kernels.py:562-882 (route -> align -> */
/* gemm1 + fused silu*up (output in x.dtype) -> per-row act-quant of the (P, inter) buffer ->     */
/* gemm2 -> top-k weighted combine in f32, cast to x.dtype); the combine order and the f32        */
/* accumulator follow mmq_fp8_moe_gather_reduce (kernels.py:876-882). round_y2 != 0: each slot's   */
/* gemm2 row is rounded to x.dtype before the combine, as the reference's unfused gemm2 hands it   */
/* over ((P, K) in the activation dtype: tools/vhip_patches/moe_experts.py:874-880); 0: the row   */
/* enters the combine unrounded, as in the fused gemm2 + gather-reduce (kernels.py:831-850).     */
/* Weights in op layout:                                                                          */
/* w13 (E, 2I, H/8), s13 (E, H/g, 2I), z13 (E, H/g, 2I/8) or NULL; w2 (E, H, I/8), s2 (E, I/g, H).*/
/* Uses the caller's route (tw, ids) and align (sorted_ids, expert_ids, ntp).                    */
/* out: (T, H) f64 before the final dtype cast.                                                   */
/* ------------------------------------------------------------------------------------------ */
void w4o_moe_forward(const uint16_t* x, int dtype, int64_t T, int64_t H, int64_t I, int64_t E,
                     int64_t top_k, const float* tw, const int32_t* sorted_ids,
                     const int32_t* expert_ids, int32_t ntp, int64_t bm,
                     const int32_t* w13, const void* s13, const int32_t* z13,
                     const int32_t* w2, const void* s2, const int32_t* z2,
                     int scale_fmt, int e2m1, int64_t g1, int64_t g2, double* out,
                     uint16_t* buf2_out /* optional (ntp, I) */, int round_y2) {
  int64_t N1 = 2 * I;
  uint8_t* xq = (uint8_t*)malloc((size_t)(T * H));
  float* xs = (float*)malloc(sizeof(float) * (size_t)T);
  w4o_act_quant(x, dtype, T, H, H, xq, xs);
  double* h = (double*)malloc(sizeof(double) * (size_t)N1);
  uint16_t* b2 = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)I);
  uint8_t* b2q = (uint8_t*)malloc((size_t)I);
  double* y2 = (double*)malloc(sizeof(double) * (size_t)H);
  int64_t sz13 = N1 * (H / 8), szs13 = (H / g1) * N1, szz13 = (H / g1) * (N1 / 8);
  int64_t sz2 = H * (I / 8), szs2 = (I / g2) * H, szz2 = (I / g2) * (H / 8);
  /* NVFP4: the zeros slot is the (E, N) f32 global (python/minisgl/quant/kernels.py:547-559) */
  if (scale_fmt == 2) { szz13 = N1; szz2 = H; }
  int sb = scale_fmt == 0 ? 2 : 1;
  memset(out, 0, sizeof(double) * (size_t)(T * H));
  for (int64_t p = 0; p < ntp; ++p) {
    int32_t r = sorted_ids[p];
    if (r >= T * top_k) continue;
    int64_t t = r / top_k;
    int64_t e = expert_ids[p / bm];
    float s2v;
    w4o_gemm(xq + t * H, xs + t, 1, H, w13 + e * sz13, N1, (const char*)s13 + e * szs13 * sb,
             scale_fmt, z13 ? z13 + e * szz13 : NULL, e2m1, g1, h);
    for (int64_t i = 0; i < I; ++i) b2[i] = w4o_silu_mul(h[i], h[I + i], dtype);
    if (buf2_out) memcpy(buf2_out + p * I, b2, sizeof(uint16_t) * (size_t)I);
    w4o_act_quant(b2, dtype, 1, I, I, b2q, &s2v);
    w4o_gemm(b2q, &s2v, 1, I, w2 + e * sz2, H, (const char*)s2 + e * szs2 * sb, scale_fmt,
             z2 ? z2 + e * szz2 : NULL, e2m1, g2, y2);
    double wgt = (double)tw[r];
    if (round_y2)
      for (int64_t j = 0; j < H; ++j) y2[j] = (double)from_dt(to_dt((float)y2[j], dtype), dtype);
    for (int64_t j = 0; j < H; ++j) out[t * H + j] += wgt * y2[j];
  }
  free(y2); free(b2q); free(b2); free(h); free(xs); free(xq);
}

/* ------------------------------------------------------------------------------------------ */
/* Grouped W4A16 MoE forward: restates python/minisgl/quant/kernels.py:899-1012 (w4a16_moe: x in */
/* the activation dtype, never quantized -> gemm1 -> silu(gate) * up rounded to the dtype as the  */
/* fused silu arms round (w4o_silu_mul) -> gemm2 on those unquantized values -> top-k weighted     */
/* sum) and :1015-1122 (w4a16_moe_decode, the same chain for NVFP4 weights). Both GEMMs are exact  */
/* f64 products of the decoded activations with the dequantized weights (w4o_dequant); out is the */
/* f64 weighted sum before the final dtype cast. Slots are taken from the route directly (the     */
/* align only orders work). ids: (T, top_k) int32, ids outside [0, E) are dropped slots.         */
/* Weights in op layout as in w4o_moe_forward. h_out (optional): (T*top_k, I) dtype bits.        */
/* ------------------------------------------------------------------------------------------ */
void w4o_w4a16_moe_forward(const uint16_t* x, int dtype, int64_t T, int64_t H, int64_t I, int64_t E,
                           int64_t top_k, const float* tw, const int32_t* ids,
                           const int32_t* w13, const void* s13, const int32_t* z13,
                           const int32_t* w2, const void* s2, const int32_t* z2,
                           int scale_fmt, int e2m1, int64_t g1, int64_t g2, double* out, uint16_t* h_out) {
  int64_t N1 = 2 * I;
  int64_t sz13 = N1 * (H / 8), szs13 = (H / g1) * N1, szz13 = (H / g1) * (N1 / 8);
  int64_t sz2 = H * (I / 8), szs2 = (I / g2) * H, szz2 = (I / g2) * (H / 8);
  if (scale_fmt == 2) { szz13 = N1; szz2 = H; }
  int sb = scale_fmt == 0 ? 2 : 1;
  double* d13 = (double*)malloc(sizeof(double) * (size_t)(N1 * H));
  double* d2 = (double*)malloc(sizeof(double) * (size_t)(H * I));
  double* xv = (double*)malloc(sizeof(double) * (size_t)H);
  double* hv = (double*)malloc(sizeof(double) * (size_t)I);
  double* y1 = (double*)malloc(sizeof(double) * (size_t)N1);
  memset(out, 0, sizeof(double) * (size_t)(T * H));
  for (int64_t e = 0; e < E; ++e) {
    int used = 0;
    for (int64_t s = 0; s < T * top_k && !used; ++s) used = ids[s] == e;
    if (!used) continue;
    w4o_dequant(w13 + e * sz13, N1, H, (const char*)s13 + e * szs13 * sb, scale_fmt,
                z13 ? z13 + e * szz13 : NULL, e2m1, g1, d13);
    w4o_dequant(w2 + e * sz2, H, I, (const char*)s2 + e * szs2 * sb, scale_fmt,
                z2 ? z2 + e * szz2 : NULL, e2m1, g2, d2);
    for (int64_t s = 0; s < T * top_k; ++s) {
      if (ids[s] != e) continue;
      int64_t t = s / top_k;
      for (int64_t k = 0; k < H; ++k) xv[k] = (double)from_dt(x[t * H + k], dtype);
      for (int64_t n = 0; n < N1; ++n) {
        double acc = 0.0;
        for (int64_t k = 0; k < H; ++k) acc += xv[k] * d13[n * H + k];
        y1[n] = acc;
      }
      for (int64_t i = 0; i < I; ++i) {
        uint16_t hb = w4o_silu_mul(y1[i], y1[I + i], dtype);
        if (h_out) h_out[s * I + i] = hb;
        hv[i] = (double)from_dt(hb, dtype);
      }
      double wgt = (double)tw[s];
      for (int64_t n = 0; n < H; ++n) {
        double acc = 0.0;
        for (int64_t i = 0; i < I; ++i) acc += hv[i] * d2[n * I + i];
        out[t * H + n] += wgt * acc;
      }
    }
  }
  free(y1); free(hv); free(xv); free(d2); free(d13);
}

/* ------------------------------------------------------------------------------------------ */
/* RMSNorm (+ residual add) producer: restates python/minisgl/layers/norm.py:9-24 (the torch   */
/* decomposition: f32-widened mean of squares, rsqrt(var + eps), rounded to dtype, times the   */
/* gain in dtype; plus_one uses dtype(weight + 1); no weight = unweighted) and :134-138 / :145- */
/* 168 (rms_norm_add: residual <- x + residual in dtype, normed over the sum). The fp8 pair of  */
/* rms_norm_quant is w4o_act_quant over the rounded output (norm.py:27-46,                      */
/* tools/w4a8_producer_actquant.py:113-136).                                                    */
/* The f32 sum of squares follows a fixed order (the order is this build's; the external       */
/* kernel's is unpinned): NT partial sums (NT = 256 for K <= 2048, 512 for K <= 4096, else      */
/* 1024), partial t accumulating elements (c*NT + t)*8 + i for c = 0, 1, ... and i = 0..7 with  */
/* fmaf; each 64-partial wave summed pairwise by lane xor 1, xor 2, then the 8- and 16-lane     */
/* mirrors, then (row 0 + row 1) + (row 2 + row 3); the NT/64 wave sums in a balanced pairwise  */
/* tree. mean = sum / K; rstd = 1 / sqrt(mean + eps).                                            */
/* residual (in/out) and weight may be NULL. out may be x.                                      */
/* ------------------------------------------------------------------------------------------ */
static float wave_sum64(const float* in) {
  float v[64], t[64];
  memcpy(v, in, sizeof v);
  for (int l = 0; l < 64; ++l) t[l] = v[l] + v[l ^ 1];
  memcpy(v, t, sizeof v);
  for (int l = 0; l < 64; ++l) t[l] = v[l] + v[l ^ 2];
  memcpy(v, t, sizeof v);
  for (int l = 0; l < 64; ++l) t[l] = v[l] + v[(l & ~7) | (7 - (l & 7))];
  memcpy(v, t, sizeof v);
  for (int l = 0; l < 64; ++l) t[l] = v[l] + v[(l & ~15) | (15 - (l & 15))];
  memcpy(v, t, sizeof v);
  return (v[0] + v[16]) + (v[32] + v[48]);
}

void w4o_rms_norm(const uint16_t* x, uint16_t* residual, const uint16_t* weight, int plus_one, float eps,
                  int dtype, int64_t M, int64_t K, uint16_t* out) {
  float* row = (float*)malloc(sizeof(float) * (size_t)K);
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t k = 0; k < K; ++k) {
      float v = from_dt(x[m * K + k], dtype);
      if (residual) {
        uint16_t s = to_dt(v + from_dt(residual[m * K + k], dtype), dtype);
        residual[m * K + k] = s;
        v = from_dt(s, dtype);
      }
      row[k] = v;
    }
    const int NT = K <= 2048 ? 256 : K <= 4096 ? 512 : 1024, NW = NT / 64;
    float part[1024];
    for (int t = 0; t < NT; ++t) {
      float ss = 0.0f;
      for (int64_t c = 0; c * NT * 8 < K; ++c)
        for (int i = 0; i < 8; ++i) {
          int64_t k = (c * NT + t) * 8 + i;
          float f = k < K ? row[k] : 0.0f;
          ss = fmaf(f, f, ss);
        }
      part[t] = ss;
    }
    float w[16];
    for (int q = 0; q < NW; ++q) w[q] = wave_sum64(part + 64 * q);
    for (int st = 1; st < NW; st <<= 1)
      for (int q = 0; q + st < NW; q += 2 * st) w[q] = w[q] + w[q + st];
    volatile float sum = w[0];
    volatile float mean = sum / (float)K;
    volatile float den = sqrtf(mean + eps);
    volatile float rstd = 1.0f / den;
    for (int64_t k = 0; k < K; ++k) {
      volatile float nv = row[k] * rstd;
      float o = from_dt(to_dt(nv, dtype), dtype);
      if (weight) {
        float g = from_dt(weight[k], dtype);
        if (plus_one) g = from_dt(to_dt(g + 1.0f, dtype), dtype);
        volatile float prod = o * g;
        o = from_dt(to_dt(prod, dtype), dtype);
      }
      out[m * K + k] = to_dt(o, dtype);
    }
  }
  free(row);
}

/* ------------------------------------------------------------------------------------------ */
/* W4A16 activation split. The reference's W4A16 arm (python/minisgl/quant/kernels.py:1125-1178) */
/* reads bf16/fp16 x unrounded; this build feeds the fp8 GEMM an exact fp8 expansion of x:       */
/* T terms (2 for bf16, 3 for fp16), term t = e4m3(r_t) with r_0 = x / 2^E,                      */
/* r_{t+1} = 16 (r_t - e4m3(r_t)), scale 2^(E - 4t), 2^E the smallest power of two with          */
/* amax / 2^E <= 448 (E = 0 for a zero row). Rows of token m are T*m + t.                        */
/* ------------------------------------------------------------------------------------------ */
static int split_exponent(float amax) {
  if (!(amax > 0.0f)) return 0;
  int e;
  const float m = 2.0f * frexpf(amax, &e);
  e -= 1;
  return m <= 1.75f ? e - 8 : e - 7;
}

void w4o_act_split(const uint16_t* x, int dtype, int64_t M, int64_t K, uint8_t* q, float* scales) {
  const int T = dtype == 0 ? 2 : 3;
  for (int64_t m = 0; m < M; ++m) {
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float v = fabsf(dtype == 0 ? w4o_bf16_to_f32(x[m * K + k]) : w4o_f16_to_f32(x[m * K + k]));
      amax = v > amax ? v : amax;
    }
    const int E = split_exponent(amax);
    for (int64_t k = 0; k < K; ++k) {
      float r = ldexpf(dtype == 0 ? w4o_bf16_to_f32(x[m * K + k]) : w4o_f16_to_f32(x[m * K + k]), -E);
      for (int t = 0; t < T; ++t) {
        const uint8_t c = w4o_f32_to_e4m3(r);
        q[(T * m + t) * K + k] = c;
        r = (r - w4o_e4m3_to_f32(c)) * 16.0f;
      }
    }
    for (int t = 0; t < T; ++t) scales[T * m + t] = ldexpf(1.0f, E - 4 * t);
  }
}

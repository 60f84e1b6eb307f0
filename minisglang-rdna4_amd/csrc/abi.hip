// extern "C" entry points of libw4a8_mi355x.so (declared in include/w4a8_mi355x.h).
//
// Every entry point validates its arguments on the host and returns a status code; the message of
// the last failure on the calling thread is available from w4a8_last_error(). No entry point
// allocates device memory: outputs and workspaces come from the caller.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include "gemm_args.h"
#include "../../include/w4a8_mi355x.h"

namespace w4a8 {
int launch_act_quant(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* q,
                     int64_t ldq, float* scales, const int32_t* row_count, hipStream_t stream);
int launch_repack(const int32_t* w, int64_t N, int64_t K, int wfmt, void* out, hipStream_t stream);
int launch_gemv(GemmArgs p, int64_t row_blocks, bool quant_src, hipStream_t stream);
bool gemv_can_fuse_quant(const GemmArgs& p, int64_t row_blocks);
bool moe_gemm2_combine_fits(int64_t K, int scale_fmt, bool has_zeros, int wfmt, int64_t group, int top_k);
int launch_moe_gemm2_combine(const GemmArgs& p, int64_t row_blocks, const uint16_t* a, int64_t lda, int adtype,
                             const int32_t* inv_pos, const int32_t* ids, const float* tw, int64_t T, int E,
                             int row_dtype, hipStream_t stream);
size_t gemv_workspace_bytes(int64_t M, int64_t N, int64_t K, int grouped, int64_t row_blocks);
int launch_prefill(const GemmArgs& p, int64_t rows_to_cover, int bm_rows, hipStream_t stream);
int launch_prefill_lds(const GemmArgs& p, int64_t rows_to_cover, int bm_rows, hipStream_t stream);
int launch_prefill_dma(const GemmArgs& p, int64_t rows_to_cover, int bm_rows, hipStream_t stream);
int launch_moe_route(const void* logits, int dtype, int64_t T, int E, int top_k, int renorm, float* tw,
                     int32_t* ids, hipStream_t stream);
int launch_moe_align(const int32_t* ids, int64_t numel, int E, int bm, int64_t P, int32_t* sorted_ids,
                     int32_t* expert_ids, int32_t* ntp, int32_t* inv_pos, hipStream_t stream);
int launch_moe_combine(const void* y, int ydt, int64_t ldy, const int32_t* inv_pos, const float* tw, int64_t T,
                       int top_k, int64_t H, void* out, int dtype, hipStream_t stream);
bool moe_prep_fits(int64_t T, int top_k);
int launch_moe_route_quant(const void* logits, int ldtype, int64_t T, int E, int top_k, int renorm, float* tw,
                           int32_t* ids, const void* x, int xdtype, int64_t K, int64_t ldx, uint8_t* xq, int64_t ldq,
                           float* xs, hipStream_t stream);
int launch_moe_route_gemm1(const GemmArgs& p, int64_t row_blocks, hipStream_t stream);
int launch_gelu_tanh_mul(const void* y, int64_t ldy, int64_t rows, int64_t inter, int dtype, void* out, int64_t ldo,
                         const int32_t* row_count, hipStream_t stream);
int launch_rms_norm(const void* x, int64_t ldx, void* res, int64_t ldr, const void* weight, int plus_one, float eps,
                    int64_t M, int64_t K, int dtype, void* out, int64_t ldo, uint8_t* q, int64_t ldq, float* scales,
                    hipStream_t stream);
int w4a16_terms(int dtype);
int launch_act_split(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* q, int64_t ldq,
                     float* scales, hipStream_t stream);
int launch_act_tile(const uint8_t* q, int64_t ldq, int64_t M, int64_t K, uint8_t* qt, float* seeds,
                    int64_t seeds_ld, hipStream_t stream);
int launch_act_quant_tiled(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* qt, float* scales,
                           float* seeds, int64_t seeds_ld, const int32_t* row_count, hipStream_t stream);
int launch_tsum(const float* y, int64_t N, int64_t M, int dtype, void* out, int64_t ldo, int silu, hipStream_t st);
int64_t w4a16_moe_max_inter();
int launch_moe_silu_split(const float* y, int64_t ldy, const int32_t* inv_pos, int64_t T, int top_k, int64_t I,
                          int dtype, uint8_t* q, int64_t ldq, float* scales, void* h, int64_t ldh, hipStream_t st);
int launch_moe_prep(const void* logits, int ldtype, int64_t T, int E, int top_k, int renorm, float* tw,
                    int32_t* ids, int bm, int64_t P, int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntp,
                    int32_t* inv_pos, const void* x, int xdtype, int64_t K, int64_t ldx, uint8_t* xq, int64_t ldq,
                    float* xs, int slots, hipStream_t stream);
}  // namespace w4a8

using namespace w4a8;

static thread_local char g_err[512];

static int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

static int hip_status(int rc, const char* what) {
  if (rc == kOk) return kOk;
  hipError_t e = hipGetLastError();
  return fail(kErrHip, "%s: HIP launch failed (%s)", what, hipGetErrorString(e));
}

namespace w4a8 {
// the library's error slot, for entry points defined in other units
int set_last_error(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace w4a8

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static const int kGemvMaxRows = 16;

// Dense symmetric int4 prefill calls of at least W4A8_PREFILL_TILED rows (default 1024; 0 turns it
// off) that the DMA-staged kernel takes (its own checks, launch_prefill_dma) have their codes in
// that kernel's operand order with the row-sum seeds, which it then reads instead of computing them.
// w4a8_linear quantizes x straight into that order (act_quant_tiled_lds_kernel, one launch as the
// row-major quant) on weights of at least W4A8_PREFILL_TILED_N output channels (default 2048:
// M=8192 qkv 299 -> 279 us, o_proj 205 -> 193, down 711 -> 695, gate_up unchanged within the runs'
// spread, M=2048 within +-1% but o_proj 58.6 -> 56.6); the producer pair (w4a8_gemm) needs a rewrite
// launch of the caller's codes (act_tile_kernel), which pays only on weights of 16384+ channels
// (M=2048 / 8192, K=4096: N=28672 5-7% faster, N=4096 and 6144 1-5% slower).
static int64_t tiled_min_rows() {
  static const int64_t min_rows = [] {
    const char* e = getenv("W4A8_PREFILL_TILED");
    return e ? (int64_t)atoll(e) : (int64_t)1024;
  }();
  return min_rows;
}
static int64_t tiled_min_n() {
  static const int64_t n = [] {
    const char* e = getenv("W4A8_PREFILL_TILED_N");
    return e ? (int64_t)atoll(e) : (int64_t)2048;
  }();
  return n;
}
static bool dma_tiled_ok(const GemmArgs& p, int64_t min_n = 16384) {
  const int64_t min_rows = tiled_min_rows();
  const bool sym4 = p.wfmt == kInt4 && p.sfmt == kScaleF16 && p.group % 128 == 0 && !p.zeros;
  const bool mx = p.wfmt == kE2M1 && p.sfmt == kScaleE8M0 && p.group == 32;  // MXFP4: A layout only, no seeds
  return min_rows > 0 && p.M >= min_rows && p.N >= min_n && (sym4 || mx) && p.K % 128 == 0 && p.KT >= 3 && !(p.silu && (p.N / 16) % 2) &&
         p.N * p.KT * 64 < ((int64_t)1 << 31) && p.M * p.K < ((int64_t)1 << 31);
}

// Bound on align blocks that can hold routed rows: every expert with rows contributes
// ceil(rows/bm) blocks, so at most numel/bm + min(E, numel) of them are non-empty.
static int64_t moe_max_blocks(int64_t numel, int64_t E, int bm, int64_t P) {
  int64_t bound = numel / bm + (E < numel ? E : numel);
  int64_t cap = (P + bm - 1) / bm;
  return bound < cap ? bound : cap;
}

static int check_weights(const char* who, int64_t N, int64_t K, int scale_fmt, const void* zeros, int wfmt,
                         int64_t group) {
  if (N <= 0 || K <= 0) return fail(kErrInvalid, "%s: N=%lld K=%lld must be positive", who, (long long)N, (long long)K);
  if (N % 16) return fail(kErrInvalid, "%s: N=%lld must be a multiple of 16", who, (long long)N);
  if (K % 32) return fail(kErrInvalid, "%s: K=%lld must be a multiple of 32", who, (long long)K);
  if (wfmt != kInt4 && wfmt != kE2M1) return fail(kErrInvalid, "%s: unknown weight format %d", who, wfmt);
  if (scale_fmt != kScaleF16 && scale_fmt != kScaleE8M0 && scale_fmt != kScaleE4M3)
    return fail(kErrInvalid, "%s: unknown scale format %d", who, scale_fmt);
  // 16-wide groups: NVFP4 (e4m3 block scales) and e2m1 with fp16 group scales
  const bool g16 = group == 16 && wfmt == kE2M1;
  if (!(g16 || group == 32 || group == 64 || (group >= 128 && (group & (group - 1)) == 0)))
    return fail(kErrUnsupported, "%s: group_size=%lld unsupported (32, 64 or a power of two >= 128; 16 for e2m1)", who,
                (long long)group);
  if (K % group) return fail(kErrInvalid, "%s: K=%lld is not a multiple of group_size=%lld", who, (long long)K, (long long)group);
  if (scale_fmt == kScaleE4M3 && (wfmt != kE2M1 || !zeros))
    return fail(kErrInvalid, "%s: e4m3 (NVFP4) block scales need e2m1 weights and the per-output-channel f32 global "
                "in the zeros slot", who);
  if (wfmt == kE2M1 && zeros && scale_fmt != kScaleE4M3)
    return fail(kErrInvalid, "%s: e2m1 weights are symmetric; w_zeros must be empty (it carries only the NVFP4 global)", who);
  if (scale_fmt == kScaleE8M0 && wfmt != kE2M1)
    return fail(kErrInvalid, "%s: E8M0 (uint8) scales are only defined for e2m1 weights", who);
  if (scale_fmt == kScaleE8M0 && group != 32)
    return fail(kErrInvalid, "%s: E8M0 scales are per 32-element block (group_size=32), got %lld", who, (long long)group);
  return kOk;
}

// w4a8_linear's workspace: the row-major codes and scales of x (what every call needs), then for
// the calls that may take the tiled prefill (tiled_min_rows) the codes of whole 16-row blocks in
// the GEMM's operand order and one row-sum seed per row and K tile. A workspace of only the first
// part is accepted; such calls run the row-major GEMM, with the same results.
static int64_t round256(int64_t b);
static int64_t linear_ws_rowmajor(int64_t M, int64_t K) { return round256(M * K) + round256(M * 4); }
static int64_t linear_ws_tiled(int64_t M, int64_t K) {
  const int64_t min_rows = tiled_min_rows();
  if (min_rows <= 0 || M < min_rows) return 0;
  const int64_t Mp = (M + 15) / 16 * 16, KT = (K + 127) / 128;
  return round256(Mp * K) + round256(KT * Mp * 4);
}
namespace w4a8 {
int64_t linear_workspace_min(int64_t M, int64_t K) { return M < 0 || K <= 0 ? -1 : linear_ws_rowmajor(M, K); }
}  // namespace w4a8

extern "C" {

int w4a8_abi_version(void) { return W4A8_ABI_VERSION; }

const char* w4a8_last_error(void) { return g_err; }

int w4a8_act_quant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* x_fp8, int64_t ldq,
                   float* act_scales, const int32_t* row_count, void* stream) {
  if (x_dtype != kBF16 && x_dtype != kF16) return fail(kErrInvalid, "act_quant: x must be bf16 or fp16");
  if (M < 0 || K <= 0 || K % 8) return fail(kErrInvalid, "act_quant: K=%lld must be a positive multiple of 8", (long long)K);
  if (ldx < K || ldx % 8 || ldq < K || ldq % 8)
    return fail(kErrInvalid, "act_quant: row strides must be >= K and multiples of 8 (ldx=%lld ldq=%lld)",
                (long long)ldx, (long long)ldq);
  if (!aligned16(x) || !aligned16(x_fp8)) return fail(kErrInvalid, "act_quant: x and x_fp8 must be 16-byte aligned");
  return hip_status(launch_act_quant(x, x_dtype, M, K, ldx, x_fp8, ldq, act_scales, row_count, (hipStream_t)stream),
                    "act_quant");
}

int w4a8_rms_norm(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, void* residual, int64_t ldr,
                  const void* weight, int plus_one, float eps, void* out, int64_t ldo, uint8_t* x_fp8, int64_t ldq,
                  float* act_scales, void* stream) {
  if (x_dtype != kBF16 && x_dtype != kF16) return fail(kErrInvalid, "rms_norm: x must be bf16 or fp16");
  if (M < 0 || K <= 0 || K % 8) return fail(kErrInvalid, "rms_norm: K=%lld must be a positive multiple of 8", (long long)K);
  if (K > 32768) return fail(kErrUnsupported, "rms_norm: rows of K=%lld > 32768 elements", (long long)K);
  if (ldx < K || ldx % 8 || ldo < K || ldo % 8 || (residual && (ldr < K || ldr % 8)) || (x_fp8 && (ldq < K || ldq % 8)))
    return fail(kErrInvalid, "rms_norm: row strides must be >= K and multiples of 8");
  if (!aligned16(x) || !aligned16(out) || (residual && !aligned16(residual)) || (weight && !aligned16(weight)) ||
      (x_fp8 && !aligned16(x_fp8)))
    return fail(kErrInvalid, "rms_norm: x, out, residual, weight and x_fp8 must be 16-byte aligned");
  if (!x_fp8 != !act_scales) return fail(kErrInvalid, "rms_norm: x_fp8 and act_scales must be supplied TOGETHER");
  if (residual && (residual == x || residual == out))
    return fail(kErrInvalid, "rms_norm: residual must not share storage with x or out");
  if (!(eps >= 0.0f)) return fail(kErrInvalid, "rms_norm: eps must be >= 0");
  return hip_status(launch_rms_norm(x, ldx, residual, ldr, weight, plus_one, eps, M, K, x_dtype, out, ldo, x_fp8, ldq,
                                    act_scales, (hipStream_t)stream), "rms_norm");
}

int64_t w4a8_tile_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || N % 16) return -1;
  return (N / 16) * ((K + 127) / 128) * 1024;
}

int w4a8_repack_weights(const int32_t* w_packed, int64_t N, int64_t K, int wfmt, void* w_tile, void* stream) {
  if (N <= 0 || N % 16) return fail(kErrInvalid, "repack: rows=%lld must be a positive multiple of 16", (long long)N);
  if (K <= 0 || K % 32) return fail(kErrInvalid, "repack: K=%lld must be a positive multiple of 32", (long long)K);
  if (wfmt != kInt4 && wfmt != kE2M1) return fail(kErrInvalid, "repack: unknown weight format %d", wfmt);
  if (!aligned16(w_tile)) return fail(kErrInvalid, "repack: output must be 16-byte aligned");
  return hip_status(launch_repack(w_packed, N, K, wfmt, w_tile, (hipStream_t)stream), "repack");
}

int64_t w4a8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int kernel) {
  if (M < 0 || N <= 0 || K <= 0) return -1;
  // prefill: room for the codes rewritten in the GEMM's operand order with their row-sum seeds,
  // which wide symmetric int4 weights take (the call runs without it too, on the row-major codes)
  if (kernel == 2 || (kernel == 0 && M > kGemvMaxRows)) return N >= 16384 ? linear_ws_tiled(M, K) : 0;
  return (int64_t)gemv_workspace_bytes(M, N, K, 0, (M + 15) / 16);
}

}  // extern "C"

// Checks shared by w4a8_gemm and w4a8_linear; fills the dense GEMM arguments (A fields left empty).
static int dense_args(const char* who, int64_t M, const void* w_tile, int64_t N, int64_t K, const void* scales,
                      int scale_fmt, const int32_t* zeros, int wfmt, int64_t group_size, void* out, int out_dtype,
                      int64_t ldo, int silu, int kernel, GemmArgs& p) {
  int rc = check_weights(who, N, K, scale_fmt, zeros, wfmt, group_size);
  if (rc) return rc;
  if (M < 0) return fail(kErrInvalid, "%s: M=%lld", who, (long long)M);
  if (out_dtype != kBF16 && out_dtype != kF16 && out_dtype != kF32)
    return fail(kErrInvalid, "%s: unknown output dtype %d", who, out_dtype);
  if (silu && (N % 32)) return fail(kErrInvalid, "%s: fused silu needs N=2*inter with inter %% 16 == 0 (N=%lld)", who, (long long)N);
  if (silu && out_dtype == kF32) return fail(kErrInvalid, "%s: fused silu rounds through bf16/fp16; f32 output unsupported", who);
  const int64_t nout = silu ? N / 2 : N;
  if (ldo < nout) return fail(kErrInvalid, "%s: ldo=%lld < output width %lld", who, (long long)ldo, (long long)nout);
  if (!aligned16(w_tile)) return fail(kErrInvalid, "%s: weight tiles must be 16-byte aligned", who);
  if (kernel < 0 || kernel > 2) return fail(kErrInvalid, "%s: kernel must be 0 (auto), 1 (decode) or 2 (prefill)", who);
  p = GemmArgs{};
  p.M = M;
  p.N = N; p.K = K; p.KT = (K + 127) / 128;
  p.wt = reinterpret_cast<const uint4*>(w_tile);
  p.scales = scales; p.sfmt = scale_fmt; p.zeros = zeros; p.group = (int)group_size; p.wfmt = wfmt;
  p.out = out; p.out_dtype = out_dtype; p.ldo = ldo; p.silu = silu;
  p.top_k = 1; p.bm = 16;
  return kOk;
}

static int run_dense(const char* who, GemmArgs& p, int kernel, hipStream_t stream) {
  const bool decode = kernel == 1 || (kernel == 0 && p.M <= kGemvMaxRows);
  char what[96];
  snprintf(what, sizeof what, "%s(%s)", who, decode ? "decode" : "prefill");
  if (decode) return hip_status(launch_gemv(p, (p.M + 15) / 16, false, stream), what);
  // LDS-staged kernel for int4 groups of 128+ and MXFP4; the per-wave kernel for the rest
  int rc = launch_prefill_lds(p, p.M, 0, stream);
  if (rc == kErrUnsupported) rc = launch_prefill(p, p.M, 128, stream);
  return hip_status(rc, what);
}

static int64_t round256(int64_t b) { return (b + 255) / 256 * 256; }

extern "C" {

int w4a8_gemm(const uint8_t* x_fp8, int64_t ldx, const float* act_scales, int64_t M, const void* w_tile, int64_t N,
              int64_t K, const void* scales, int scale_fmt, const int32_t* zeros, int wfmt, int64_t group_size,
              void* out, int out_dtype, int64_t ldo, int silu, void* workspace, int64_t workspace_bytes, int kernel,
              void* stream) {
  GemmArgs p;
  int rc = dense_args("w4a8_gemm", M, w_tile, N, K, scales, scale_fmt, zeros, wfmt, group_size, out, out_dtype, ldo,
                      silu, kernel, p);
  if (rc) return rc;
  if (M == 0) return kOk;
  if (ldx < K || ldx % 16 || !aligned16(x_fp8))
    return fail(kErrInvalid, "w4a8_gemm: x_fp8 rows must be 16-byte aligned with stride >= K (ldx=%lld)", (long long)ldx);
  p.xq = x_fp8; p.ldx = ldx; p.act_scales = act_scales;
  const hipStream_t st = (hipStream_t)stream;
  const bool decode = kernel == 1 || (kernel == 0 && M <= kGemvMaxRows);
  if (!decode && dma_tiled_ok(p) && workspace && aligned16(workspace) && workspace_bytes >= linear_ws_tiled(M, K)) {
    // the caller's codes rewritten in the GEMM's operand order with their seeds (as w4a8_linear)
    const int64_t Mp = (M + 15) / 16 * 16;
    uint8_t* xt = reinterpret_cast<uint8_t*>(workspace);
    float* seeds = reinterpret_cast<float*>(xt + round256(Mp * K));
    rc = launch_act_tile(x_fp8, ldx, M, K, xt, seeds, Mp, st);
    if (rc) return hip_status(rc, "w4a8_gemm(act tile)");
    GemmArgs q = p;
    q.xq = xt; q.ldx = K; q.a_tiled = 1; q.seeds = seeds; q.seeds_ld = Mp;
    rc = launch_prefill_dma(q, M, 0, st);
    if (rc != kErrUnsupported) return hip_status(rc, "w4a8_gemm(prefill, tiled)");
  }
  return run_dense("w4a8_gemm", p, kernel, st);
}

int64_t w4a8_linear_workspace_bytes(int64_t M, int64_t K) {
  if (M < 0 || K <= 0) return -1;
  return linear_ws_rowmajor(M, K) + linear_ws_tiled(M, K);
}

int w4a8_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* w_tile, int64_t N,
                const void* scales, int scale_fmt, const int32_t* zeros, int wfmt, int64_t group_size, void* out,
                int out_dtype, int64_t ldo, int silu, void* workspace, int64_t workspace_bytes, int kernel,
                void* stream) {
  GemmArgs p;
  int rc = dense_args("w4a8_linear", M, w_tile, N, K, scales, scale_fmt, zeros, wfmt, group_size, out, out_dtype,
                      ldo, silu, kernel, p);
  if (rc) return rc;
  if (M == 0) return kOk;
  if (x_dtype != kBF16 && x_dtype != kF16) return fail(kErrInvalid, "w4a8_linear: x must be bf16 or fp16 (dtype %d)", x_dtype);
  if (ldx < K || ldx % 8 || !aligned16(x))
    return fail(kErrInvalid, "w4a8_linear: x rows must be 16-byte aligned with stride >= K (ldx=%lld)", (long long)ldx);
  const bool decode = kernel == 1 || (kernel == 0 && M <= kGemvMaxRows);
  const hipStream_t st = (hipStream_t)stream;
  p.xsrc = reinterpret_cast<const uint16_t*>(x); p.ldxs = ldx; p.xdtype = x_dtype;
  if (decode && gemv_can_fuse_quant(p, (M + 15) / 16))
    return hip_status(launch_gemv(p, (M + 15) / 16, true, st), "w4a8_linear(decode, fused quant)");
  // quantize into the workspace, then the fp8 GEMM
  const int64_t need = linear_ws_rowmajor(M, K);
  if (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))
    return fail(kErrInvalid, "w4a8_linear: needs a 16-byte aligned workspace of %lld bytes, got %lld", (long long)need,
                (long long)workspace_bytes);
  uint8_t* xq = reinterpret_cast<uint8_t*>(workspace);
  float* xs = reinterpret_cast<float*>(xq + round256(M * K));
  if (!decode && dma_tiled_ok(p, tiled_min_n()) && workspace_bytes >= need + linear_ws_tiled(M, K)) {
    // prefill on the DMA-staged kernel: x quantized straight into its operand order, with the seeds
    const int64_t Mp = (M + 15) / 16 * 16;
    uint8_t* xt = reinterpret_cast<uint8_t*>(xs) + round256(M * 4);
    float* seeds = reinterpret_cast<float*>(xt + round256(Mp * K));
    rc = launch_act_quant_tiled(x, x_dtype, M, K, ldx, xt, xs, seeds, Mp, nullptr, st);
    if (rc) return hip_status(rc, "w4a8_linear(act quant, tiled)");
    GemmArgs q = p;
    q.xsrc = nullptr;
    q.xq = xt; q.ldx = K; q.act_scales = xs;
    q.a_tiled = 1; q.seeds = seeds; q.seeds_ld = Mp;
    rc = launch_prefill_dma(q, M, 0, st);
    if (rc != kErrUnsupported) return hip_status(rc, "w4a8_linear(prefill, tiled)");
  }
  rc = launch_act_quant(x, x_dtype, M, K, ldx, xq, K, xs, nullptr, st);
  if (rc) return hip_status(rc, "w4a8_linear(act quant)");
  p.xsrc = nullptr;
  p.xq = xq; p.ldx = K; p.act_scales = xs;
  return run_dense("w4a8_linear", p, kernel, st);
}

extern "C" {

int w4a8_linear_launch_count(int64_t M, int64_t N, int64_t K, int x_dtype, int scale_fmt, int has_zeros, int wfmt,
                             int64_t group_size, int silu, int kernel) {
  // the planner reads shapes and formats only: stand-in pointers (aligned, never dereferenced)
  const void* fake = reinterpret_cast<const void*>(static_cast<uintptr_t>(256));
  GemmArgs p;
  int rc = dense_args("w4a8_linear_launch_count", M, fake, N, K, fake, scale_fmt,
                      has_zeros ? reinterpret_cast<const int32_t*>(fake) : nullptr, wfmt, group_size,
                      const_cast<void*>(fake), x_dtype, N, silu, kernel, p);
  if (rc) return -rc;
  if (x_dtype != kBF16 && x_dtype != kF16) return -fail(kErrInvalid, "w4a8_linear_launch_count: x must be bf16 or fp16");
  if (M == 0) return 0;
  const bool decode = kernel == 1 || (kernel == 0 && M <= kGemvMaxRows);
  p.xsrc = reinterpret_cast<const uint16_t*>(fake); p.ldxs = K; p.xdtype = x_dtype;
  return decode && gemv_can_fuse_quant(p, (M + 15) / 16) ? 1 : 2;
}

}  // extern "C"

// ---- W4A16: unquantized bf16/fp16 activations, split exactly into fp8 terms (w4a16.hip)
static int64_t round16(int64_t b) { return (b + 15) / 16 * 16; }

extern "C" {

int64_t w4a16_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int x_dtype) {
  if (M < 0 || N <= 0 || K <= 0 || (x_dtype != kBF16 && x_dtype != kF16)) return -1;
  const int64_t T = w4a16_terms(x_dtype);
  return round256(T * M * round16(K)) + round256(T * M * 4) + round256(T * M * N * 4);
}

int w4a16_act_split(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* x_fp8, int64_t ldq,
                    float* scales, void* stream) {
  if (x_dtype != kBF16 && x_dtype != kF16) return fail(kErrInvalid, "w4a16_act_split: x must be bf16 or fp16");
  if (M < 0 || K <= 0 || K % 8) return fail(kErrInvalid, "w4a16_act_split: K=%lld must be a positive multiple of 8", (long long)K);
  if (ldx < K || ldx % 8 || !aligned16(x))
    return fail(kErrInvalid, "w4a16_act_split: x rows must be 16-byte aligned with stride >= K (ldx=%lld)", (long long)ldx);
  if (ldq < K || ldq % 8 || (reinterpret_cast<uintptr_t>(x_fp8) & 7u) || !scales)
    return fail(kErrInvalid, "w4a16_act_split: x_fp8 rows must be 8-byte aligned with stride >= K (ldq=%lld), scales non-null",
                (long long)ldq);
  return hip_status(launch_act_split(x, x_dtype, M, K, ldx, x_fp8, ldq, scales, (hipStream_t)stream), "w4a16_act_split");
}

int w4a16_moe_silu_split(const float* y, int64_t ldy, const int32_t* inv_pos, int64_t T, int top_k, int64_t inter,
                         int dtype, uint8_t* a_fp8, int64_t lda, float* a_scales, void* h, int64_t ldh, void* stream) {
  if (dtype != kBF16 && dtype != kF16) return fail(kErrInvalid, "w4a16_moe_silu_split: dtype must be bf16 or fp16");
  if (T < 0 || top_k <= 0) return fail(kErrInvalid, "w4a16_moe_silu_split: T=%lld top_k=%d", (long long)T, top_k);
  if (inter <= 0 || inter % 8 || inter > w4a16_moe_max_inter())
    return fail(kErrInvalid, "w4a16_moe_silu_split: inter=%lld must be a positive multiple of 8 up to %lld",
                (long long)inter, (long long)w4a16_moe_max_inter());
  if (ldy < 2 * inter || ldy % 4 || !aligned16(y) || !inv_pos)
    return fail(kErrInvalid, "w4a16_moe_silu_split: y rows must be 16-byte aligned with stride >= 2*inter (ldy=%lld)",
                (long long)ldy);
  if (lda < inter || lda % 8 || (reinterpret_cast<uintptr_t>(a_fp8) & 7u) || !a_scales)
    return fail(kErrInvalid, "w4a16_moe_silu_split: a_fp8 rows must be 8-byte aligned with stride >= inter (lda=%lld)",
                (long long)lda);
  if (h && (ldh < inter || ldh % 8 || !aligned16(h)))
    return fail(kErrInvalid, "w4a16_moe_silu_split: h rows must be 16-byte aligned with stride >= inter (ldh=%lld)",
                (long long)ldh);
  return hip_status(launch_moe_silu_split(y, ldy, inv_pos, T, top_k, inter, dtype, a_fp8, lda, a_scales, h, ldh,
                                          (hipStream_t)stream), "w4a16_moe_silu_split");
}

int w4a16_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* w_tile, int64_t N,
                 const void* scales, int scale_fmt, const int32_t* zeros, int wfmt, int64_t group_size, void* out,
                 int64_t ldo, int silu, void* workspace, int64_t workspace_bytes, int kernel, void* stream) {
  GemmArgs p;
  // the GEMM writes the terms' f32 rows into the workspace (out set below); the sum kernel
  // rounds, and applies silu * up for the fused arm
  int rc = dense_args("w4a16_linear", M, w_tile, N, K, scales, scale_fmt, zeros, wfmt, group_size, workspace, kF32, N, 0,
                      kernel, p);
  if (rc) return rc;
  if (x_dtype != kBF16 && x_dtype != kF16) return fail(kErrInvalid, "w4a16_linear: x must be bf16 or fp16 (dtype %d)", x_dtype);
  if (silu && (N % 32)) return fail(kErrInvalid, "w4a16_linear: fused silu needs N=2*inter with inter %% 16 == 0 (N=%lld)", (long long)N);
  const int64_t nout = silu ? N / 2 : N;
  if (ldo < nout) return fail(kErrInvalid, "w4a16_linear: ldo=%lld < output width %lld", (long long)ldo, (long long)nout);
  if (M == 0) return kOk;
  if (K % 8 || ldx < K || ldx % 8 || !aligned16(x))
    return fail(kErrInvalid, "w4a16_linear: x rows must be 16-byte aligned with stride >= K, K %% 8 == 0 (ldx=%lld)", (long long)ldx);
  const int64_t need = w4a16_linear_workspace_bytes(M, N, K, x_dtype);
  if (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))
    return fail(kErrInvalid, "w4a16_linear: needs a 16-byte aligned workspace of %lld bytes, got %lld", (long long)need,
                (long long)workspace_bytes);
  const hipStream_t st = (hipStream_t)stream;
  const int64_t T = w4a16_terms(x_dtype), ldq = round16(K);
  uint8_t* xq = reinterpret_cast<uint8_t*>(workspace);
  float* xs = reinterpret_cast<float*>(xq + round256(T * M * ldq));
  float* y = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(xs) + round256(T * M * 4));
  rc = launch_act_split(x, x_dtype, M, K, ldx, xq, ldq, xs, st);
  if (rc) return hip_status(rc, "w4a16_linear(act split)");
  p.M = T * M;
  p.xq = xq; p.ldx = ldq; p.act_scales = xs;
  p.out = y; p.ldo = N;
  // the kernel choice follows the token count, as the reference's arm does
  const bool decode = kernel == 1 || (kernel == 0 && M <= kGemvMaxRows);
  if (decode) {
    rc = hip_status(launch_gemv(p, (p.M + 15) / 16, false, st), "w4a16_linear(decode)");
  } else if (x_dtype == kBF16 && aligned16(out) && ldo % 8 == 0) {
    // bf16 on the DMA-staged kernel: its epilogue sums each row's two terms (and applies silu)
    // and writes the bf16 rows itself, the same arithmetic as the f32 rows + sum kernel below
    GemmArgs q = p;
    q.out = out; q.ldo = ldo; q.out_dtype = kBF16; q.silu = silu; q.tsum2 = 1;
    if (dma_tiled_ok(q)) {
      // wide symmetric int4: the terms' codes rewritten in the GEMM's operand order with their
      // row-sum seeds, into the f32 rows' space that this path leaves unused
      const int64_t Mp = round16(q.M), KT = q.KT;
      uint8_t* xt = reinterpret_cast<uint8_t*>(y);
      float* seeds = reinterpret_cast<float*>(xt + round256(Mp * K));
      if (round256(Mp * K) + round256(KT * Mp * 4) <= round256(T * M * N * 4)) {
        rc = launch_act_tile(xq, ldq, q.M, K, xt, seeds, Mp, st);
        if (rc) return hip_status(rc, "w4a16_linear(act tile)");
        q.xq = xt; q.ldx = K; q.a_tiled = 1; q.seeds = seeds; q.seeds_ld = Mp;
      }
    }
    rc = launch_prefill_dma(q, q.M, 0, st);
    if (rc != kErrUnsupported) return hip_status(rc, "w4a16_linear(prefill, term sum)");
    rc = launch_prefill_lds(p, p.M, 0, st);
    if (rc == kErrUnsupported) rc = launch_prefill(p, p.M, 128, st);
    rc = hip_status(rc, "w4a16_linear(prefill)");
  } else {
    rc = launch_prefill_lds(p, p.M, 0, st);
    if (rc == kErrUnsupported) rc = launch_prefill(p, p.M, 128, st);
    rc = hip_status(rc, "w4a16_linear(prefill)");
  }
  if (rc) return rc;
  return hip_status(launch_tsum(y, N, M, x_dtype, out, ldo, silu, st), "w4a16_linear(sum)");
}

}  // extern "C"

static int check_route(const char* who, int logits_dtype, int64_t E, int top_k) {
  if (logits_dtype != kBF16 && logits_dtype != kF16 && logits_dtype != kF32)
    return fail(kErrInvalid, "%s: logits must be bf16, fp16 or f32", who);
  if (E <= 0 || E > 512) return fail(kErrUnsupported, "%s: num_experts=%lld outside [1, 512]", who, (long long)E);
  if (top_k <= 0 || top_k > E || top_k > 64) return fail(kErrInvalid, "%s: top_k=%d invalid for E=%lld", who, top_k, (long long)E);
  return kOk;
}

static int check_align(const char* who, int64_t numel, int64_t E, int block_m, int64_t P) {
  if (E <= 0 || E > 512) return fail(kErrUnsupported, "%s: num_experts=%lld outside [1, 512]", who, (long long)E);
  if (block_m <= 0 || block_m % 16) return fail(kErrInvalid, "%s: block_m=%d must be a positive multiple of 16", who, block_m);
  if (P < numel + (E + 1) * (block_m - 1))
    return fail(kErrInvalid, "%s: capacity P=%lld < numel + (E+1)*(block_m-1)", who, (long long)P);
  if (numel > 0x7fffffff || P > 0x7fffffff) return fail(kErrInvalid, "%s: slots and padded rows must be below 2^31", who);
  return kOk;
}

int w4a8_moe_route(const void* logits, int logits_dtype, int64_t T, int64_t E, int top_k, int renormalize,
                   float* topk_w, int32_t* topk_ids, void* stream) {
  if (int rc = check_route("moe_route", logits_dtype, E, top_k)) return rc;
  return hip_status(launch_moe_route(logits, logits_dtype, T, (int)E, top_k, renormalize, topk_w, topk_ids,
                                     (hipStream_t)stream), "moe_route");
}

static int check_route_x(const char* what, const void* x, int x_dtype, int64_t K, int64_t ldx, const void* x_fp8,
                         int64_t ldq, const float* x_scales) {
  if (!x) return kOk;
  if (x_dtype != kBF16 && x_dtype != kF16) return fail(kErrInvalid, "%s: x must be bf16 or fp16", what);
  if (K <= 0 || K % 8) return fail(kErrInvalid, "%s: K=%lld must be a positive multiple of 8", what, (long long)K);
  if (ldx < K || ldx % 8 || ldq < K || ldq % 8)
    return fail(kErrInvalid, "%s: row strides must be >= K and multiples of 8 (ldx=%lld ldq=%lld)", what,
                (long long)ldx, (long long)ldq);
  if (!aligned16(x) || !aligned16(x_fp8) || !x_scales)
    return fail(kErrInvalid, "%s: x and x_fp8 must be 16-byte aligned and x_scales given", what);
  return kOk;
}

int w4a8_moe_route_align(const void* logits, int logits_dtype, int64_t T, int64_t E, int top_k, int renormalize,
                         int block_m, int64_t P, float* topk_w, int32_t* topk_ids, int32_t* sorted_ids,
                         int32_t* expert_ids, int32_t* ntp, int32_t* inv_pos, const void* x, int x_dtype, int64_t K,
                         int64_t ldx, uint8_t* x_fp8, int64_t ldq, float* x_scales, void* stream) {
  if (int rc = check_route("moe_route_align", logits_dtype, E, top_k)) return rc;
  if (T < 0) return fail(kErrInvalid, "moe_route_align: T=%lld negative", (long long)T);
  if (int rc = check_align("moe_route_align", T * top_k, E, block_m, P)) return rc;
  if (int rc = check_route_x("moe_route_align", x, x_dtype, K, ldx, x_fp8, ldq, x_scales)) return rc;
  const hipStream_t st = (hipStream_t)stream;
  if (moe_prep_fits(T, top_k))
    return hip_status(launch_moe_prep(logits, logits_dtype, T, (int)E, top_k, renormalize, topk_w, topk_ids, block_m, P,
                                      sorted_ids, expert_ids, ntp, inv_pos, x, x_dtype, K, ldx, x_fp8, ldq, x_scales,
                                      0, st), "moe_route_align");
  // route and the quant of x in one launch where the rows allow it, then the align
  int rc = x ? launch_moe_route_quant(logits, logits_dtype, T, (int)E, top_k, renormalize, topk_w, topk_ids, x, x_dtype,
                                      K, ldx, x_fp8, ldq, x_scales, st)
             : kErrUnsupported;
  const bool quantized = rc == kOk && x;
  if (rc == kErrUnsupported) rc = launch_moe_route(logits, logits_dtype, T, (int)E, top_k, renormalize, topk_w, topk_ids, st);
  if (!rc) rc = launch_moe_align(topk_ids, T * top_k, (int)E, block_m, P, sorted_ids, expert_ids, ntp, inv_pos, st);
  if (!rc && x && !quantized) rc = launch_act_quant(x, x_dtype, T, K, ldx, x_fp8, ldq, x_scales, nullptr, st);
  return hip_status(rc, "moe_route_align");
}

int w4a8_moe_route_slots(const void* logits, int logits_dtype, int64_t T, int64_t E, int top_k, int renormalize,
                         int block_m, int64_t P, float* topk_w, int32_t* topk_ids, int32_t* sorted_ids,
                         int32_t* expert_ids, int32_t* ntp, int32_t* inv_pos, const void* x, int x_dtype, int64_t K,
                         int64_t ldx, uint8_t* x_fp8, int64_t ldq, float* x_scales, void* stream) {
  if (int rc = check_route("moe_route_slots", logits_dtype, E, top_k)) return rc;
  if (T < 0) return fail(kErrInvalid, "moe_route_slots: T=%lld negative", (long long)T);
  if (int rc = check_align("moe_route_slots", T * top_k, E, block_m, P)) return rc;
  if (int rc = check_route_x("moe_route_slots", x, x_dtype, K, ldx, x_fp8, ldq, x_scales)) return rc;
  // the grouped GEMMs size their grids for numel / block_m + min(E, numel) blocks: no more slots
  // than experts
  if (!moe_prep_fits(T, top_k) || T * top_k * block_m > P || T * top_k > E || !inv_pos)
    return fail(kErrInvalid, "moe_route_slots: T*top_k=%lld slots of %d rows must fit P=%lld, E=%lld and the "
                "one-launch prep, with inv_pos given", (long long)(T * top_k), block_m, (long long)P, (long long)E);
  return hip_status(launch_moe_prep(logits, logits_dtype, T, (int)E, top_k, renormalize, topk_w, topk_ids, block_m, P,
                                    sorted_ids, expert_ids, ntp, inv_pos, x, x_dtype, K, ldx, x_fp8, ldq, x_scales, 1,
                                    (hipStream_t)stream), "moe_route_slots");
}

int64_t w4a8_moe_padded_capacity(int64_t numel, int64_t E, int block_m) {
  return numel + (E + 1) * (block_m - 1);
}

int w4a8_moe_align(const int32_t* topk_ids, int64_t numel, int64_t E, int block_m, int64_t P, int32_t* sorted_ids,
                   int32_t* expert_ids, int32_t* ntp, int32_t* inv_pos, void* stream) {
  if (int rc = check_align("moe_align", numel, E, block_m, P)) return rc;
  return hip_status(launch_moe_align(topk_ids, numel, (int)E, block_m, P, sorted_ids, expert_ids, ntp, inv_pos,
                                     (hipStream_t)stream), "moe_align");
}

// Validation and arguments of a grouped GEMM call (w4a8_moe_gemm, w4a8_moe_gemm_quant).
static int moe_gemm_setup(const char* who, const uint8_t* a_fp8, int64_t lda, const float* a_scales, int a_by_token,
                          const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* ntp, int64_t numel,
                          int top_k, int block_m, int64_t P, const void* w_tile, int64_t E, int64_t N, int64_t K,
                          const void* scales, int scale_fmt, const int32_t* zeros, int wfmt, int64_t group_size,
                          void* out, int out_dtype, int64_t ldo, int silu, int kernel, GemmArgs& p, bool& decode) {
  int rc = check_weights(who, N, K, scale_fmt, zeros, wfmt, group_size);
  if (rc) return rc;
  if (E <= 0 || E > 512) return fail(kErrUnsupported, "%s: num_experts=%lld outside [1, 512]", who, (long long)E);
  if (block_m <= 0 || block_m % 16) return fail(kErrInvalid, "%s: block_m=%d must be a multiple of 16", who, block_m);
  if (numel < 0 || numel > 0x7fffffff || P > 0x7fffffff)
    return fail(kErrInvalid, "%s: slots (%lld) and padded rows (%lld) must be below 2^31", who, (long long)numel,
                (long long)P);
  if (a_by_token && top_k <= 0) return fail(kErrInvalid, "%s: top_k=%d must be positive", who, top_k);
  if (lda < K || lda % 16 || !aligned16(a_fp8)) return fail(kErrInvalid, "%s: A rows must be 16-byte aligned, stride >= K", who);
  if (out_dtype != kBF16 && out_dtype != kF16 && out_dtype != kF32) return fail(kErrInvalid, "%s: unknown output dtype", who);
  if (silu && (N % 32 || out_dtype == kF32)) return fail(kErrInvalid, "%s: fused silu needs N %% 32 == 0 and bf16/fp16 output", who);
  const int64_t nout = silu ? N / 2 : N;
  if (ldo < nout) return fail(kErrInvalid, "%s: ldo=%lld < output width %lld", who, (long long)ldo, (long long)nout);
  if (kernel < 0 || kernel > 2) return fail(kErrInvalid, "%s: kernel must be 0, 1 or 2", who);
  decode = kernel == 1 || (kernel == 0 && block_m < 64);
  if (!decode && block_m % 64) return fail(kErrInvalid, "%s: the prefill arm needs block_m %% 64 == 0 (got %d)", who, block_m);

  p = GemmArgs{};
  p.xq = a_fp8; p.ldx = lda; p.act_scales = a_scales; p.M = P;
  p.N = N; p.K = K; p.KT = (K + 127) / 128;
  p.wt = reinterpret_cast<const uint4*>(w_tile);
  p.scales = scales; p.sfmt = scale_fmt; p.zeros = zeros; p.group = (int)group_size; p.wfmt = wfmt;
  p.sorted_ids = sorted_ids; p.expert_ids = expert_ids; p.ntp = ntp; p.top_k = top_k; p.num_slots = numel;
  p.bm = block_m; p.a_by_token = a_by_token;
  p.w_expert_tiles = (N / 16) * p.KT;
  p.s_expert_stride = (K / group_size) * N;
  // the NVFP4 global is one f32 per output channel per expert; zero words are (K/g, N/8) per expert
  p.z_expert_stride = scale_fmt == kScaleE4M3 ? N : (K / group_size) * (N / 8);
  p.out = out; p.out_dtype = out_dtype; p.ldo = ldo; p.silu = silu;
  return kOk;
}

// The grouped GEMM's launch on row-major fp8 rows: the decode GEMV below 64-row blocks, else the
// MFMA kernels on 64- or 128-row tiles.
static int moe_gemm_run(const char* who, GemmArgs& p, bool decode, int64_t E, void* workspace,
                        int64_t workspace_bytes, hipStream_t stream) {
  const int64_t nblk = moe_max_blocks(p.num_slots, E, p.bm, p.M);
  if (decode) {
    const int64_t rb = nblk * p.bm / 16;
    const size_t need = gemv_workspace_bytes(p.M, p.N, p.K, 1, rb);
    if (need > 0 && (workspace == nullptr || (size_t)workspace_bytes < need))
      return fail(kErrInvalid, "%s: decode split-K needs a %zu-byte workspace, got %lld", who, need,
                  (long long)workspace_bytes);
    p.partial = reinterpret_cast<float*>(workspace);
    return hip_status(launch_gemv(p, rb, false, stream), "w4a8_moe_gemm(decode)");
  }
  const int bm_rows = p.bm % 128 == 0 ? 128 : 64;
  int rc = launch_prefill_lds(p, nblk * p.bm, bm_rows, stream);
  if (rc == kErrUnsupported) rc = launch_prefill(p, nblk * p.bm, bm_rows, stream);
  return hip_status(rc, "w4a8_moe_gemm(prefill)");
}

// w4a8_moe_gemm_quant's codes: row-major (P, K), or for the tiled gemm2 the codes of whole 16-row
// blocks in operand order and one row-sum seed per row and K tile, whichever is larger
static int64_t moe_quant_code_bytes(int64_t P, int64_t K) {
  const int64_t Pp = (P + 15) / 16 * 16, KT = (K + 127) / 128;
  const int64_t rm = round256(P * K), tl = round256(Pp * K) + round256(KT * Pp * 4);
  return rm > tl ? rm : tl;
}

int64_t w4a8_moe_gemm_workspace_bytes(int64_t numel, int64_t E, int block_m, int64_t P, int64_t N, int64_t K,
                                      int kernel) {
  const bool decode = kernel == 1 || (kernel == 0 && block_m < 64);
  if (!decode) return 0;
  const int64_t rb = moe_max_blocks(numel, E, block_m, P) * block_m / 16;
  return (int64_t)gemv_workspace_bytes(P, N, K, 1, rb);
}

int w4a8_moe_gemm(const uint8_t* a_fp8, int64_t lda, const float* a_scales, int a_by_token, const int32_t* sorted_ids,
                  const int32_t* expert_ids, const int32_t* ntp, int64_t numel, int top_k, int block_m, int64_t P,
                  const void* w_tile, int64_t E, int64_t N, int64_t K, const void* scales, int scale_fmt,
                  const int32_t* zeros, int wfmt, int64_t group_size, void* out, int out_dtype, int64_t ldo, int silu,
                  void* workspace, int64_t workspace_bytes, int kernel, void* stream) {
  GemmArgs p;
  bool decode;
  int rc = moe_gemm_setup("w4a8_moe_gemm", a_fp8, lda, a_scales, a_by_token, sorted_ids, expert_ids, ntp, numel, top_k,
                          block_m, P, w_tile, E, N, K, scales, scale_fmt, zeros, wfmt, group_size, out, out_dtype, ldo,
                          silu, kernel, p, decode);
  if (rc || numel == 0) return rc;
  return moe_gemm_run("w4a8_moe_gemm", p, decode, E, workspace, workspace_bytes, (hipStream_t)stream);
}

int64_t w4a8_moe_gemm_quant_workspace_bytes(int64_t P, int64_t K) {
  if (P < 0 || K <= 0) return -1;
  return moe_quant_code_bytes(P, K) + round256(P * 4);
}

int w4a8_moe_gemm_quant(const void* a, int a_dtype, int64_t lda, const int32_t* sorted_ids, const int32_t* expert_ids,
                        const int32_t* ntp, int64_t numel, int block_m, int64_t P, const void* w_tile, int64_t E,
                        int64_t N, int64_t K, const void* scales, int scale_fmt, const int32_t* zeros, int wfmt,
                        int64_t group_size, void* out, int out_dtype, int64_t ldo, void* workspace,
                        int64_t workspace_bytes, int kernel, void* stream) {
  const char* who = "w4a8_moe_gemm_quant";
  if (a_dtype != kBF16 && a_dtype != kF16) return fail(kErrInvalid, "%s: a must be bf16 or fp16 (dtype %d)", who, a_dtype);
  if (lda < K || lda % 8 || !aligned16(a))
    return fail(kErrInvalid, "%s: a rows must be 16-byte aligned with stride >= K (lda=%lld)", who, (long long)lda);
  const int64_t need = w4a8_moe_gemm_quant_workspace_bytes(P, K);
  if (need < 0 || workspace == nullptr || workspace_bytes < need || !aligned16(workspace))
    return fail(kErrInvalid, "%s: needs a 16-byte aligned workspace of %lld bytes, got %lld", who, (long long)need,
                (long long)workspace_bytes);
  uint8_t* codes = reinterpret_cast<uint8_t*>(workspace);
  float* xs = reinterpret_cast<float*>(codes + moe_quant_code_bytes(P, K));
  GemmArgs p;
  bool decode;
  int rc = moe_gemm_setup(who, codes, K, xs, 0, sorted_ids, expert_ids, ntp, numel, 1, block_m, P, w_tile, E, N, K,
                          scales, scale_fmt, zeros, wfmt, group_size, out, out_dtype, ldo, 0, kernel, p, decode);
  if (rc || numel == 0) return rc;
  const hipStream_t st = (hipStream_t)stream;
  // rows that can hold data (the grid bound; *ntp bounds the work on the device)
  const int64_t nblk = moe_max_blocks(numel, E, block_m, P);
  const int64_t rows = nblk * block_m < P ? nblk * block_m : P;
  const bool sym4 = wfmt == kInt4 && scale_fmt == kScaleF16 && group_size % 128 == 0 && !zeros;
  if (!decode && sym4 && tiled_min_rows() > 0 && K % 128 == 0 && p.KT >= 3 && N * p.KT * 64 < ((int64_t)1 << 31)) {
    // the padded rows quantized straight into the DMA GEMM's operand order with the row-sum seeds
    const int64_t Pp = (P + 15) / 16 * 16;
    float* seeds = reinterpret_cast<float*>(codes + round256(Pp * K));
    rc = launch_act_quant_tiled(a, a_dtype, rows, K, lda, codes, xs, seeds, Pp, ntp, st);
    if (rc) return hip_status(rc, "w4a8_moe_gemm_quant(act quant, tiled)");
    GemmArgs q = p;
    q.a_tiled = 1; q.seeds = seeds; q.seeds_ld = Pp;
    rc = launch_prefill_dma(q, nblk * block_m, block_m % 128 == 0 ? 128 : 64, st);
    if (rc != kErrUnsupported) return hip_status(rc, "w4a8_moe_gemm_quant(prefill, tiled)");
  }
  const int64_t Pp = (P + 15) / 16 * 16;
  if (decode && tiled_min_rows() > 0 && numel >= 16 * E && K % 128 == 0 && Pp * K < ((int64_t)1 << 31)) {
    // the grouped GEMV reads each 16-row block's codes in operand order: per tile two 1 KiB runs
    // instead of 16 rows' 64-byte pieces (any weight format; the seeds go unused). Only where the
    // blocks are about full (16+ slots per expert): a block's rows without data read row 0's
    // pieces in the row-major form, one cache line, but whole runs in this one (configs[4] gemm2
    // T=512 177.5 -> 170.6 us whole call, T=256 120.1 -> 119.2; T=32 gemm2 23.6 -> 27.4 us)
    float* seeds = reinterpret_cast<float*>(codes + round256(Pp * K));
    rc = launch_act_quant_tiled(a, a_dtype, rows, K, lda, codes, xs, seeds, Pp, ntp, st);
    if (rc) return hip_status(rc, "w4a8_moe_gemm_quant(act quant, tiled)");
    GemmArgs q = p;
    q.a_tiled = 1;
    return moe_gemm_run(who, q, decode, E, nullptr, 0, st);
  }
  rc = launch_act_quant(a, a_dtype, rows, K, lda, codes, K, xs, ntp, st);
  if (rc) return hip_status(rc, "w4a8_moe_gemm_quant(act quant)");
  return moe_gemm_run(who, p, decode, E, nullptr, 0, st);
}

int w4a8_moe_gelu_tanh_mul(const void* y, int dtype, int64_t ldy, int64_t rows, int64_t inter, void* out, int64_t ldo,
                           const int32_t* row_count, void* stream) {
  const char* who = "w4a8_moe_gelu_tanh_mul";
  if (dtype != kBF16 && dtype != kF16) return fail(kErrInvalid, "%s: y must be bf16 or fp16", who);
  if (rows < 0 || inter <= 0 || inter % 8)
    return fail(kErrInvalid, "%s: rows=%lld, inter=%lld (a positive multiple of 8)", who, (long long)rows, (long long)inter);
  if (ldy < 2 * inter || ldy % 8 || ldo < inter || ldo % 8)
    return fail(kErrInvalid, "%s: row strides ldy=%lld (>= 2*inter) and ldo=%lld (>= inter), multiples of 8", who,
                (long long)ldy, (long long)ldo);
  if (!aligned16(y) || !aligned16(out)) return fail(kErrInvalid, "%s: y and out must be 16-byte aligned", who);
  return hip_status(launch_gelu_tanh_mul(y, ldy, rows, inter, dtype, out, ldo, row_count, (hipStream_t)stream), who);
}

int w4a8_moe_gemm2_combine_supported(int64_t K, int scale_fmt, int has_zeros, int wfmt, int64_t group_size, int top_k) {
  return moe_gemm2_combine_fits(K, scale_fmt, has_zeros != 0, wfmt, group_size, top_k) ? 1 : 0;
}

int w4a8_moe_gemm2_combine(const void* a, int a_dtype, int64_t lda, const int32_t* topk_ids, const float* topk_w,
                           const int32_t* inv_pos, int64_t T, int top_k, int block_m, int64_t P, const void* w_tile,
                           int64_t E, int64_t N, int64_t K, const void* scales, int scale_fmt, const int32_t* zeros,
                           int wfmt, int64_t group_size, void* out, int out_dtype, int64_t ldo, int row_dtype,
                           void* stream) {
  const char* who = "w4a8_moe_gemm2_combine";
  int rc = check_weights(who, N, K, scale_fmt, zeros, wfmt, group_size);
  if (rc) return rc;
  if (E <= 0 || E > 512) return fail(kErrUnsupported, "%s: num_experts=%lld outside [1, 512]", who, (long long)E);
  if (block_m <= 0 || block_m % 16 || block_m >= 64)
    return fail(kErrInvalid, "%s: the decode arm needs block_m in {16, 32, 48} (got %d)", who, block_m);
  if (a_dtype != kBF16 && a_dtype != kF16) return fail(kErrInvalid, "%s: the gemm1 buffer must be bf16 or fp16", who);
  if (lda < K || lda % 8 || !aligned16(a))
    return fail(kErrInvalid, "%s: gemm1 buffer rows must be 16-byte aligned with stride >= K (lda=%lld)", who, (long long)lda);
  if (out_dtype != kBF16 && out_dtype != kF16 && out_dtype != kF32) return fail(kErrInvalid, "%s: unknown output dtype", who);
  if (ldo < N) return fail(kErrInvalid, "%s: ldo=%lld < N=%lld", who, (long long)ldo, (long long)N);
  if (row_dtype != kBF16 && row_dtype != kF16 && row_dtype != kF32)
    return fail(kErrInvalid, "%s: unknown row dtype %d", who, row_dtype);
  if (T < 0 || T > 65535 || top_k <= 0) return fail(kErrInvalid, "%s: T=%lld (at most 65535) top_k=%d", who, (long long)T, top_k);
  const int64_t numel = T * top_k;
  if (int rc2 = check_align(who, numel, E, block_m, P)) return rc2;
  if (!topk_ids || !topk_w || !inv_pos) return fail(kErrInvalid, "%s: topk_ids, topk_w and inv_pos are required", who);
  if (!moe_gemm2_combine_fits(K, scale_fmt, zeros != nullptr, wfmt, group_size, top_k))
    return fail(kErrUnsupported, "%s: K=%lld, group %lld, formats %d/%d, top_k %d take the unfused path", who,
                (long long)K, (long long)group_size, wfmt, scale_fmt, top_k);
  if (numel == 0) return kOk;
  // the grouped gemm2 this call replaces, for its K split
  GemmArgs p = {};
  p.M = P; p.N = N; p.K = K; p.KT = (K + 127) / 128;
  p.wt = reinterpret_cast<const uint4*>(w_tile);
  p.scales = scales; p.sfmt = scale_fmt; p.zeros = zeros; p.group = (int)group_size; p.wfmt = wfmt;
  p.sorted_ids = topk_ids;  // non-null marks the grouped plan; the plan reads no array
  p.top_k = top_k; p.num_slots = numel; p.bm = block_m;
  p.w_expert_tiles = (N / 16) * p.KT;
  p.s_expert_stride = (K / group_size) * N;
  p.z_expert_stride = scale_fmt == kScaleE4M3 ? N : (K / group_size) * (N / 8);
  p.out = out; p.out_dtype = out_dtype; p.ldo = ldo;
  const int64_t rb = moe_max_blocks(numel, E, block_m, P) * block_m / 16;
  return hip_status(launch_moe_gemm2_combine(p, rb, reinterpret_cast<const uint16_t*>(a), lda, a_dtype, inv_pos,
                                             topk_ids, topk_w, T, (int)E, row_dtype, (hipStream_t)stream), who);
}

int w4a8_moe_route_gemm1(const void* logits, int logits_dtype, int64_t T, int64_t E, int top_k, int renormalize,
                         const void* x, int x_dtype, int64_t ldx, int block_m, int64_t P, const void* w_tile, int64_t N,
                         int64_t K, const void* scales, int scale_fmt, const int32_t* zeros, int wfmt,
                         int64_t group_size, float* topk_w, int32_t* topk_ids, int32_t* sorted_ids,
                         int32_t* expert_ids, int32_t* ntp, int32_t* inv_pos, void* out, int out_dtype, int64_t ldo,
                         void* stream) {
  const char* who = "w4a8_moe_route_gemm1";
  if (int rc = check_route(who, logits_dtype, E, top_k)) return rc;
  if (int rc = check_weights(who, N, K, scale_fmt, zeros, wfmt, group_size)) return rc;
  if (T < 0) return fail(kErrInvalid, "%s: T=%lld negative", who, (long long)T);
  const int64_t numel = T * top_k;
  if (int rc = check_align(who, numel, E, block_m, P)) return rc;
  if (x_dtype != kBF16 && x_dtype != kF16) return fail(kErrInvalid, "%s: x must be bf16 or fp16", who);
  if (K % 8 || ldx < K || ldx % 8 || !aligned16(x))
    return fail(kErrInvalid, "%s: x rows must be 16-byte aligned with stride >= K (K=%lld ldx=%lld)", who,
                (long long)K, (long long)ldx);
  if (out_dtype != kBF16 && out_dtype != kF16) return fail(kErrInvalid, "%s: the gemm1 buffer must be bf16 or fp16", who);
  if (N % 32 || ldo < N / 2) return fail(kErrInvalid, "%s: N=%lld must be a multiple of 32, ldo >= N/2", who, (long long)N);
  if (!topk_w || !topk_ids || !sorted_ids || !expert_ids || !ntp || !inv_pos || !out)
    return fail(kErrInvalid, "%s: every route output and the gemm1 buffer are required", who);
  // one 16-row block per slot (block_m < 64), the slots within the capacity and no more than the
  // experts (the grouped gemm2 sizes its grid for numel / block_m + min(E, numel) blocks), experts
  // within the in-kernel router's reach
  if (block_m >= 64 || numel * block_m > P || numel > E || E > kRouteMaxExperts || numel > 64)
    return fail(kErrUnsupported, "%s: %lld slots, E=%lld, block_m=%d take the route + slots launch", who,
                (long long)numel, (long long)E, block_m);
  if (numel == 0) return kOk;
  GemmArgs p = {};
  p.xsrc = reinterpret_cast<const uint16_t*>(x); p.ldxs = ldx; p.xdtype = x_dtype; p.M = P;
  p.N = N; p.K = K; p.KT = (K + 127) / 128;
  p.wt = reinterpret_cast<const uint4*>(w_tile);
  p.scales = scales; p.sfmt = scale_fmt; p.zeros = zeros; p.group = (int)group_size; p.wfmt = wfmt;
  p.sorted_ids = sorted_ids;  // non-null marks the grouped plan; the routed kernel writes it, reads none
  p.top_k = top_k; p.num_slots = numel; p.bm = block_m; p.a_by_token = 1;
  p.w_expert_tiles = (N / 16) * p.KT;
  p.s_expert_stride = (K / group_size) * N;
  p.z_expert_stride = scale_fmt == kScaleE4M3 ? N : (K / group_size) * (N / 8);
  p.logits = logits; p.ldtype = logits_dtype; p.num_experts = (int)E; p.renorm = renormalize;
  p.tw_out = topk_w; p.ids_out = topk_ids; p.inv_out = inv_pos; p.sorted_out = sorted_ids; p.eid_out = expert_ids;
  p.ntp_out = ntp;
  p.out = out; p.out_dtype = out_dtype; p.ldo = ldo; p.silu = 1;
  const int64_t rb = moe_max_blocks(numel, E, block_m, P) * block_m / 16;
  const int rc = launch_moe_route_gemm1(p, rb, (hipStream_t)stream);
  if (rc == kErrUnsupported)
    return fail(kErrUnsupported, "%s: formats %d/%d, group %lld, K=%lld take the route + slots launch", who, wfmt,
                scale_fmt, (long long)group_size, (long long)K);
  return hip_status(rc, who);
}

int w4a8_moe_combine(const void* y, int y_dtype, int64_t ldy, const int32_t* inv_pos, const float* topk_w, int64_t T,
                     int top_k, int64_t H, void* out, int out_dtype, void* stream) {
  if (out_dtype != kBF16 && out_dtype != kF16 && out_dtype != kF32) return fail(kErrInvalid, "moe_combine: unknown dtype");
  if (y_dtype != kBF16 && y_dtype != kF16 && y_dtype != kF32) return fail(kErrInvalid, "moe_combine: unknown y dtype");
  if (ldy < H) return fail(kErrInvalid, "moe_combine: ldy < H");
  const uintptr_t ymask = y_dtype == kF32 ? 15u : 7u;
  if (H % 4 || ldy % 4 || (reinterpret_cast<uintptr_t>(y) & ymask) ||
      (reinterpret_cast<uintptr_t>(out) & (out_dtype == kF32 ? 15u : 7u)))
    return fail(kErrInvalid, "moe_combine: H and ldy must be multiples of 4 with y %d-byte and out %d-byte aligned",
                y_dtype == kF32 ? 16 : 8, out_dtype == kF32 ? 16 : 8);
  return hip_status(launch_moe_combine(y, y_dtype, ldy, inv_pos, topk_w, T, top_k, H, out, out_dtype,
                                       (hipStream_t)stream),
                    "moe_combine");
}

}  // extern "C"

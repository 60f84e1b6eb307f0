// Decode GEMV: launch planning, and the launch unit for A read per tile from global memory
// (the kernel template lives in gemv.h; the staged and fused A sources are compiled in
// gemv_staged.hip and gemv_fused.hip so the three units build in parallel).
#include "gemv.h"

namespace w4a8 {

// Shape policy (from launch-shape sweeps on MI355X at the Llama-3-8B decode shapes, M = 1..16).
//   * nstr: blocks of more than 4 rows read A per tile from global memory and share each A
//     fragment between two strips when the weight has 384+ strips; smaller blocks, and narrower
//     dense weights (whose two-strip grid would leave CUs idle), run one strip per wave.
//   * waves x tpw: up to 8 waves per workgroup owning at least 4 K tiles each (many short waves
//     keep more loads in flight than few long ones); wide weights whose grid would pass ~8192
//     waves get fewer, longer waves instead (a grid that large runs in several rounds). Dense
//     calls plan this from (N, K) alone (see plan_gemv).
//   * A source: up to 4 rows are staged in LDS (fp8 codes, one barrier). A one-row call on
//     bf16/fp16 input, or a two-row call on a narrow weight, quantizes its rows in the GEMV itself
//     (one launch instead of two); larger blocks re-read and re-quantize too many rows per
//     workgroup, so they take the act-quant kernel first.
// The per-channel arithmetic depends only on (waves, tpw). For dense calls they come from (N, K)
// alone, planned as for a one-row call, so a row's output bits do not depend on how many rows share
// the call (rows[0:m] alone == rows[0:m] inside a 16-row call); the fused-silu arm, the plain arm
// and every A source agree bit for bit. Grouped (MoE) calls plan from their grid.
//
// K split of a grid of `groups` workgroups: up to 8 waves owning at least 4 K tiles each; grids
// that would pass ~8192 waves get fewer, longer waves; grids of under ~2 waves per SIMD (the MoE
// decode calls over a handful of experts, narrow dense weights) halve the tiles per wave, down to
// 2 and up to 8 waves, so more of the weight bytes are in flight at once. wmax caps the waves.
static void plan_ksplit(int64_t KT, int64_t groups, int64_t wmax, int64_t& waves, int64_t& tpw) {
  int64_t w = (KT + 3) / 4;
  if (w > wmax) w = wmax;
  if (w < 1) w = 1;
  // a power of two: 4 waves (two walking sets) rather than 5-7 (K=2560 N=9728 M=16 12.7 -> 10.5 us,
  // M=1 8.5 -> 7.5; K=2816 N=4096 M=1 6.2 -> 5.4 on gemv_kernel)
  while (w & (w - 1)) --w;
  while (w > 1 && groups * w > 8192 && (KT + w - 1) / w < 8) w = (w + 1) / 2;
  int64_t t = (KT + w - 1) / w;
  w = (KT + t - 1) / t;
  while (groups * w < 2048 && w < 8) {
    const int64_t t2 = (t + 1) / 2;
    const int64_t w2 = (KT + t2 - 1) / t2;
    if (t2 < 2 || w2 > 8) break;
    t = t2;
    w = w2;
  }
  waves = w;
  tpw = t;
}

// Wave cap of a call's K split, from (N, K, format) alone. Dense NVFP4 on wide weights (1024+
// strips) splits K over at most 4 waves of longer ranges: the 8 scaled MFMAs and 8 scale-byte loads
// of every NVFP4 tile make short waves pay their prologue and reduction more often than the extra
// loads in flight return. K=8192 N=28672, 8 -> 4 waves: M=1 42.6 -> 37.2 us, M=2 40.2 -> 36.2,
// M=16 57.7 -> 46.1; on K=28672 N=8192 (512 strips) 4 waves lose (M=1 38.7 -> 41.5), so it keeps 8.
static int64_t ksplit_wmax(const GemmArgs& p, int64_t strips) {
  return gemv_nvfp4(p) && !p.sorted_ids && strips >= 1024 ? 4 : 8;
}

GemvPlan plan_gemv(const GemmArgs& p, int64_t row_blocks, bool quant_src) {
  GemvPlan pl;
  const int64_t KT = (p.K + kTileK - 1) / kTileK;
  const int64_t rows = p.sorted_ids ? 16 : (p.M < 16 ? p.M : 16);
  const int64_t strips = p.N / kTileN;
  // two strips per workgroup only where that still leaves about a workgroup per CU (384+ strips);
  // narrower dense weights (o_proj, down at 4096 channels) run one strip each, twice the grid
  // (grouped MoE calls keep two: their grids already span the routed experts, except for decode
  // batches of at most 64 slots, whose few blocks hold a row or two each: one strip there, twice
  // the grid; configs[4] T=1 21.0 -> 19.7 us, T=2 25.4 -> 23.0, T=8 46.7 -> 45.8; and gemm1 (the
  // silu arm) up to 256 slots, whose blocks hold a few rows: T=16 66.1 -> 62.1 us, T=32 83.7 ->
  // 80.6, where T=256 measured 126.8 -> 130.8 with one strip)
  pl.nstr = rows > 4 && (p.sorted_ids || strips >= 384) ? 2 : 1;
  if (p.sorted_ids && (p.num_slots <= 64 || (p.silu && p.num_slots <= 256))) pl.nstr = 1;
  // dense: the one-row grid (one strip per workgroup, one row block); grouped: the launched grid
  const int64_t split_groups = p.sorted_ids ? (strips + pl.nstr - 1) / pl.nstr * row_blocks : strips;
  int64_t w, tpw;
  plan_ksplit(KT, split_groups, ksplit_wmax(p, strips), w, tpw);
  pl.waves = (int)w;
  pl.tpw = (int)tpw;

  const bool fast = (p.wfmt == kInt4 && p.group % kTileK == 0) || (p.wfmt == kE2M1 && p.sfmt == kScaleE8M0) ||
                    gemv_nvfp4(p);
  const int64_t lbytes = rows * (int64_t)stage_stride((int)KT);
  const bool lds_ok = fast && !p.sorted_ids && rows <= 4 && lbytes <= kStageLdsMax;
  const bool fuse_ok = rows == 1 || (rows == 2 && strips <= 512 && p.K <= 8192);
  const int64_t threads = (int64_t)pl.waves * 64;
  const int64_t qchunks = rows * KT * (kTileK / 8), schunks = rows * KT * (kTileK / 16);  // 16-byte loads
  pl.amode = kAGlobal;
  if (lds_ok && quant_src && fuse_ok && qchunks <= kStageMax * threads) pl.amode = kAQuant;
  else if (lds_ok && !quant_src && schunks <= kStageMax * threads) pl.amode = kAStage;
  // wide weights (1024+ strips): one-row fused-quant calls run 4 strips per workgroup (the silu arm
  // 2 gate + 2 up strips), a quarter of the grid, so each CU runs about two workgroups instead of
  // seven and quantizes the activation row twice instead of seven times: with seven, the workgroups
  // that had their row issued weight loads that the others' row loads then queued behind (their
  // A phase spread from 2 to 9 us); gate_up M=1 14.7 -> 13.8 us, MXFP4 K=8192 N=28672 25.8 -> 22.5
  // us. Three strips (an uneven grid) and seven (one workgroup of 4 waves per CU) were slower. The
  // K split is unchanged, so the output bits are too. NVFP4 (eight MFMAs per tile) keeps one strip
  // per workgroup: K=8192 N=28672 M=1 40.6 us against 50.6 with four.
  const bool nv = gemv_nvfp4(p);
  if (pl.amode == kAQuant && !p.sorted_ids && rows == 1 && strips >= 1024 && !nv) pl.nstr = p.silu ? 2 : 4;
  const int64_t chunks = pl.amode == kAQuant ? qchunks : schunks;
  // staging loads per thread: exact depths for the fused quant, 4 or 8 for fp8 staging
  pl.sm = chunks <= threads ? 1 : chunks <= 2 * threads ? 2 : chunks <= 4 * threads ? 4 : 8;
  if (pl.amode == kAStage && pl.sm < 4) pl.sm = 4;
  pl.stage_bytes = pl.amode == kAGlobal ? 0 : (size_t)((lbytes + 15) / 16) * 16;
  // Window order. One-row fused-quant calls on narrow weights (K <= 8192, at most 512 strips: about
  // a workgroup per CU) quantize A before issuing any weight load, so the row's loads meet no
  // weight load on their way (qkv M=1 7.1 against 7.7 us with the weights issued first). Every
  // other fused-quant call issues its first window right behind the A loads and quantizes while
  // the weights are in flight: o_proj M=2 7.15 -> 6.95 us, down M=1 (K = 14336, with a 4-tile
  // window) 11.2 -> 10.5 us, and the wide calls above. Staged fp8 A waits for the window before
  // its LDS writes (equal or up to 2% faster than staging on arrival at the sweep's staged calls).
  if (pl.amode == kAQuant)
    pl.af = rows == 1 && p.K <= 8192 && (strips <= 512 || nv) ? kWinAFirst : kWinAfterA;
  else
    pl.af = pl.amode == kAStage ? kWinWaitAll : kWinAfterA;
  pl.ch = pl.amode == kAQuant && p.wfmt == kInt4 && pl.af == kWinAfterA && p.K > 8192 ? 4 : 3;
  return pl;
}

// The strip-walking GEMV (gemv_walk.hip) for one row block of bf16/fp16 rows, int4 with groups of
// 128+ or MXFP4. Its cost over the weight stream is the row phase, where every workgroup quantizes
// all M x K values, vpt of them per thread of its 8 waves. Measured on MI355X against act quant +
// gemv_kernel (configs[1] shapes, configs[0], configs[5] and a few odd shapes; outputs equal bit for
// bit):
//   * vpt <= 96: the walk is faster or ties at every shape (K=4096 N=4096 M=4 6.0 against 8.2 us,
//     K=4096 N=6144 M=8 8.1 against 9.0, K=14336 N=4096 M=2 10.0 against 11.9, K=2560 N=9728 asym
//     M=16 10.5 against 12.7, one-row calls too: K=4096 N=28672 M=1 12.7 against 13.9);
//   * vpt <= 128 still pays where a workgroup streams more than 64 KiB of weights (K=4096 N=28672
//     M=16 17.9 against 19.7, K=14336 N=4096 M=4 11.3 against 12.0); on less it ties or loses
//     (K=4096 N=6144 M=16 10.0 against 9.8);
//   * above that it loses (K=14336 N=4096 M=8 15.3 against 13.4), and one-row calls on wide MXFP4
//     weights keep the 4-strip fused-quant kernel (K=8192 N=28672 M=1 22.4 against 23.6).
// Grid: 256 workgroups (one per CU) of 8 waves: two walking sets where the one-row plan has 4 or
// fewer waves (twice the weight bytes in flight: K=4096 N=28672 M=1 12.7 against 18.0 us with one
// set), the rest helper waves of the row phase; a window of 4 tiles per wave (8 and 16 measured
// slower: their loads delay the rows').
bool plan_gemv_walk(const GemmArgs& p, int64_t row_blocks, WalkPlan& wp) {
  if (p.sorted_ids || row_blocks != 1 || p.M < 1 || p.M > 16 || !p.xsrc) return false;
  const bool i4 = p.wfmt == kInt4 && p.group % kTileK == 0;
  const bool e8 = p.wfmt == kE2M1 && p.sfmt == kScaleE8M0;
  const bool nv = gemv_nvfp4(p);
  if (!i4 && !e8 && !nv) return false;
  const int64_t KT = p.KT, strips = p.N / kTileN;
  if (e8 && p.M == 1 && strips >= 1024) return false;
  // NVFP4 (8 MFMAs and 8 scale-byte loads per tile) walks only where the other path reads A per tile
  // (more than 4 rows): K=8192 N=28672 M=8 48.0 against 52.3 us, but M=4 45.5 against 43.2, M=1 43.2
  // against 39.3
  if (nv && p.M <= 4) return false;
  int64_t w, tpw;
  plan_ksplit(KT, strips, ksplit_wmax(p, strips), w, tpw);  // the one-row plan: the output bits of gemv_kernel's one-row call
  const int ns = p.silu ? 2 : 1;
  const int64_t ngroups = p.silu ? strips / 2 : strips;
  int64_t rp = 1;
  while (rp < p.M) rp <<= 1;
  const int64_t G = ngroups < 256 ? ngroups : 256;
  const int64_t ngmax = (ngroups + G - 1) / G;
  const int64_t sets = (2 * w <= 8 && ngmax >= 2) ? 2 : 1;
  // helper waves fill the workgroup to 8 waves for the row phase (K=2560 N=9728 M=16 with one set
  // of 5 waves: 13.9 -> 11.8 us)
  const int64_t bw = 8;
  // threads per row: the largest power of two that fits
  int tpr_log = 0;
  while ((int64_t)(2 << tpr_log) * rp <= bw * 64) ++tpr_log;
  const int64_t tpr = (int64_t)1 << tpr_log;
  if (tpr < 16) return false;
  const int64_t smn = (KT * (kTileK / 8) + tpr - 1) / tpr;
  if (smn > 16) return false;  // 32 row loads per thread spill (and only odd row counts reach them)
  const int64_t vpt = p.M * KT * kTileK / (tpr * rp);
  const int64_t wg_weight_bytes = ngmax * ns * KT * kTileBytes;
  if (vpt > 128 || (vpt > 96 && wg_weight_bytes <= 64 * 1024)) return false;
  const size_t a_bytes = (size_t)((p.M * stage_stride((int)KT) + 15) / 16) * 16;
  const size_t red = (size_t)(ngmax * w * ns * p.M * 16 * 4);
  if (a_bytes + red > (size_t)kWalkLdsMax) return false;
  wp.grid = (int)G;
  wp.waves = (int)w;
  wp.sets = (int)sets;
  wp.block_waves = (int)bw;
  wp.tpw = (int)tpw;
  wp.ngroups = (int)ngroups;
  wp.ngmax = (int)ngmax;
  wp.tpr_log = tpr_log;
  wp.sm = smn <= 1 ? 1 : smn <= 2 ? 2 : smn <= 4 ? 4 : smn <= 8 ? 8 : 16;
  wp.lds = a_bytes + red;
  return true;
}

// A read per tile, int4 with groups of 128+: a window of 2 tiles per wave. These calls (dense
// blocks of 5+ rows, every grouped MoE call) hold an A fragment per tile besides the weights, so the
// window sets their registers and occupancy (NS=4: 160 VGPRs with 4 tiles, 104 with 2; 3 and 4
// waves per SIMD become 4 and 6), and more resident waves keep more loads in flight than a longer
// window per wave. Measured on MI355X against the 4-tile window, outputs equal bit for bit (the
// window does not change the summation order): configs[4] MoE whole call T=16 60.7 -> 56.3 us,
// T=32 79.4 -> 72.4, T=256 118.8 -> 110.2, T=512 171.0 -> 155.6 (3 tiles: between the two; 1
// tile: 1-2 us slower than 2 at T <= 64); dense K=14336 N=4096 M=16 16.4 -> 15.3 us, K=4096
// N=4096 M=16 8.48 -> 8.25, the other decode-sweep calls within 0.5%.
constexpr int kGemvChunkGlobalI4 = 2;
bool launch_gemv_global(const GemmArgs& p, dim3 grid, const GemvPlan& pl, hipStream_t stream) {
  const int ns = p.silu ? 2 * pl.nstr : pl.nstr;
  bool ok = false;
  if (p.wfmt == kInt4 && p.group % kTileK == 0) {
    if (ns == 1) return gemv_launch_fmt<kAGlobal, 1, kGemvChunkGlobalI4, kWinAfterA, true, false>(p, grid, stream, pl);
    if (ns == 2) return gemv_launch_fmt<kAGlobal, 2, kGemvChunkGlobalI4, kWinAfterA, true, false>(p, grid, stream, pl);
    if (ns == 4) return gemv_launch_fmt<kAGlobal, 4, kGemvChunkGlobalI4, kWinAfterA, true, false>(p, grid, stream, pl);
    return false;
  }
  if (ns == 1) ok = gemv_launch_fmt<kAGlobal, 1, kGemvChunk, kWinAfterA, false, true>(p, grid, stream, pl);
  else if (ns == 2) ok = gemv_launch_fmt<kAGlobal, 2, kGemvChunk, kWinAfterA, false, true>(p, grid, stream, pl);
  else if (ns == 4) ok = gemv_launch_fmt<kAGlobal, 4, kGemvChunk, kWinAfterA, false, true>(p, grid, stream, pl);
  else return false;
  // the sub-tile-group formats (int4 group 32/64, e2m1 with fp16 scales)
  return ok || launch_gemv_generic(p, grid, pl, stream);
}

// row_blocks: number of 16-row blocks to launch (dense: ceil(M/16); grouped: a bound on the
// padded rows that can hold data). quant_src: p.xsrc holds bf16/fp16 rows; returns kErrUnsupported
// when the fused quant does not apply (the caller then quantizes first).
int launch_gemv(GemmArgs p, int64_t row_blocks, bool quant_src, hipStream_t stream) {
  WalkPlan wp;
  if (quant_src && plan_gemv_walk(p, row_blocks, wp)) {
    if (!launch_gemv_walk(p, wp, stream)) return kErrInvalid;
    return hipGetLastError() == hipSuccess ? kOk : kErrHip;
  }
  const GemvPlan pl = plan_gemv(p, row_blocks, quant_src);
  if (quant_src && pl.amode != kAQuant) return kErrUnsupported;
  const int64_t nstrips = p.N / kTileN;
  const int64_t sg = ((p.silu ? nstrips / 2 : nstrips) + pl.nstr - 1) / pl.nstr;
  const dim3 grid((unsigned)sg, 1, (unsigned)row_blocks);
  bool ok;
  if (pl.amode == kAQuant) ok = launch_gemv_fused(p, grid, pl, stream);
  else if (pl.amode == kAStage) ok = launch_gemv_staged(p, grid, pl, stream);
  else ok = launch_gemv_global(p, grid, pl, stream);
  if (!ok) return kErrInvalid;
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

// K split (waves, tpw) the grouped GEMV runs for these arguments and row blocks; the fused gemm2 +
// combine reproduces it so that its per-slot rows equal the grouped gemm2's bit for bit.
void gemv_ksplit(const GemmArgs& p, int64_t row_blocks, int& waves, int& tpw) {
  const GemvPlan pl = plan_gemv(p, row_blocks, false);
  waves = pl.waves;
  tpw = pl.tpw;
}

// True when launch_gemv can quantize bf16/fp16 rows itself for this call.
bool gemv_can_fuse_quant(const GemmArgs& p, int64_t row_blocks) {
  WalkPlan wp;
  if (plan_gemv_walk(p, row_blocks, wp)) return true;
  return plan_gemv(p, row_blocks, true).amode == kAQuant;
}


// The decode kernel reduces inside the workgroup: no workspace.
size_t gemv_workspace_bytes(int64_t, int64_t, int64_t, int, int64_t) { return 0; }

}  // namespace w4a8

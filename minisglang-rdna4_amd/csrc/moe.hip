// MoE routing, token-slot alignment and top-k combine for the grouped W4A8 FFN.
//
// route: restates the softmax + top-k + renormalize half of moe_hip.moe_route_align
//   (python/minisgl/quant/kernels.py:423-447): softmax over f32-widened logits, top-k with exact
//   ties keeping the LOWER expert index (python/minisgl/layers/moe.py:1218-1227), weights
//   renormalised by sum + 1e-8 (python/minisgl/moe/fused.py:52-53). One wave per token; experts
//   are selected on the logits, which orders them exactly as the softmax does.
// align: restates moe_align_block_size (python/minisgl/moe/fused.py:120-176): slots sorted by
//   expert, stable in slot order, each expert padded to a multiple of block_m with the sentinel
//   numel, per-block expert id (blocks past the end clamp to E-1), padded total ntp. A single
//   workgroup builds it deterministically: an LDS histogram, a scan, then chunks of slots ranked
//   with per-wave lane masks and per-expert prefix sums over the waves.
// combine: out[t] = sum_j tw[t,j] * y[pos(t,j)] in f32, j in slot order, cast to the activation
//   dtype (mmq_fp8_moe_gather_reduce, kernels.py:876-882).
#include <cstdlib>

#include "act_quant.h"
#include "moe_route.h"

namespace w4a8 {

constexpr int kMaxExperts = 512;

__device__ __forceinline__ float load_logit(const void* p, int dtype, int64_t i) {
  if (dtype == kF32) return reinterpret_cast<const float*>(p)[i];
  return from_dtype(reinterpret_cast<const uint16_t*>(p)[i], dtype);
}

template <int PER>
__global__ void __launch_bounds__(256)
moe_route_kernel(const void* __restrict__ logits, int dtype, int64_t T, int E, int top_k, int renorm,
                 float* __restrict__ tw, int32_t* __restrict__ ids) {
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;  // whole waves leave together
  route_token<PER>(logits, dtype, t, E, top_k, renorm, tw, ids, nullptr);
}

// Align of numel slots by one workgroup of NT threads (E <= EMAX): an LDS histogram, a scan of the
// padded counts, then chunks of NT slots. In a chunk every wave marks its lanes in a per-wave,
// per-expert 64-bit lane mask (LDS atomic OR): a lane's rank among the wave's lanes holding its
// expert is the popcount of the mask below it, and per-expert prefix sums of the mask popcounts
// over the waves give each wave's offset, so the order is stable in slot order. ids may point to
// global memory or LDS. With HELD > 0 the histogram pass, which reads every id once with
// independent loads, also keeps the first HELD ids in LDS as 16-bit values, so the chunk loop waits
// on no global load. Every output element is written by exactly one thread (slots by the scatter,
// padding and the tail by the fill), so no global store has to land before another: the barriers
// only order LDS traffic and never drain the stores in flight.
template <int NT, int EMAX, int HELD>
__device__ __forceinline__ void align_block(const int32_t* ids, int64_t numel, int E, int bm, int64_t P,
                                            int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
                                            int32_t* __restrict__ ntp_out, int32_t* __restrict__ inv_pos) {
  constexpr int NW = NT / 64;
  static_assert(NT >= EMAX, "one scan pass: a thread per expert");
  __shared__ int cnt[EMAX];
  __shared__ int base[EMAX];
  __shared__ unsigned long long mask[NW][EMAX];
  __shared__ int pre[NW][EMAX];
  __shared__ int wsums[NW];
  __shared__ int total_s;
  __shared__ uint16_t held[HELD > 0 ? HELD : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < EMAX; e += NT) cnt[e] = 0;
  for (int i = tid; i < NW * EMAX; i += NT) (&mask[0][0])[i] = 0ull;
  lds_barrier();
  // eight independent loads in flight per thread per batch
  for (int64_t i0 = 0; i0 < numel; i0 += 8 * NT) {
    int ev[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t i = i0 + u * NT + tid;
      ev[u] = i < numel ? ids[i] : -1;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t i = i0 + u * NT + tid;
      int e = ev[u];
      if (e < 0 || e >= E) e = -1;
      if (HELD > 0 && i < HELD && i < numel) held[i] = (uint16_t)e;  // -1 is kept as 0xffff
      if (e >= 0) atomicAdd(&cnt[e], 1);
    }
  }
  lds_barrier();
  // exclusive scan of padded counts over experts (one expert per thread)
  const int padded = tid < E ? (cnt[tid] + bm - 1) / bm * bm : 0;
  int incl = padded;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int n = __shfl_up(incl, o, 64);
    if (lane >= o) incl += n;
  }
  if (lane == 63) wsums[wave] = incl;
  lds_barrier();
  if (tid == 0) {
    int run = 0;
    for (int w = 0; w < NW; ++w) {
      const int s = wsums[w];
      wsums[w] = run;
      run += s;
    }
    total_s = run;
  }
  lds_barrier();
  if (tid < E) base[tid] = incl - padded + wsums[wave];
  const int total = total_s;
  lds_barrier();
  // padding rows of each expert and the tail [ntp, P) hold the sentinel numel
  for (int64_t x = tid; x < (int64_t)E * (bm - 1); x += NT) {
    const int e = (int)(x / (bm - 1)), j = (int)(x - (int64_t)e * (bm - 1));
    const int c = cnt[e];
    if (c + j < (c + bm - 1) / bm * bm) sorted_ids[base[e] + c + j] = (int32_t)numel;
  }
  for (int64_t i = total + tid; i < P; i += NT) sorted_ids[i] = (int32_t)numel;
  // block owners; blocks past the end clamp to E-1
  if (tid < E) {
    const int b0 = base[tid] / bm, nb = (cnt[tid] + bm - 1) / bm;
    for (int b = 0; b < nb; ++b) expert_ids[b0 + b] = tid;
  }
  const int64_t nblocks = (P + bm - 1) / bm;
  for (int64_t b = total / bm + tid; b < nblocks; b += NT) expert_ids[b] = E - 1;
  if (tid == 0) *ntp_out = total;
  // stable scatter in chunks of NT slots
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  for (int64_t c0 = 0; c0 < numel; c0 += NT) {
    const int64_t i = c0 + tid;
    int e = -1;
    if (i < numel) {
      if (HELD > 0 && i < HELD) {
        const uint16_t h = held[i];
        e = h == 0xffffu ? -1 : (int)h;
      } else {
        e = ids[i];
        if (e >= E) e = -1;
      }
    }
    if (e >= 0) atomicOr(&mask[wave][e], 1ull << lane);
    lds_barrier();
    const uint64_t m = e >= 0 ? mask[wave][e] : 0ull;
    if (tid < E) {
      // per-expert offsets of the waves: exclusive prefix of the mask popcounts, from base
      int run = base[tid];
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const int c = __popcll(mask[w][tid]);
        pre[w][tid] = run;
        run += c;
      }
      base[tid] = run;
    }
    lds_barrier();
    if (e >= 0) {
      const int off = pre[wave][e] + __popcll(m & below);
      sorted_ids[off] = (int32_t)i;
      if (inv_pos) inv_pos[i] = off;
      if (lane == __ffsll((long long)m) - 1) mask[wave][e] = 0ull;  // the wave's lowest lane clears
    } else if (i < numel && inv_pos) {
      inv_pos[i] = -1;  // dropped slot: the combine skips it
    }
  }
}

constexpr int kAlignHeld = 32768;  // slots whose ids the histogram pass keeps in LDS (64 KiB)
static int64_t align_multi_min() {
  const char* e = getenv("W4A8_ALIGN_MULTI_MIN");
  return e ? atoll(e) : 4096;
}
static const int64_t kAlignMultiMin = align_multi_min();  // slots above which the align spans workgroups

// Align by ceil(numel / NT) workgroups, workgroup b owning slots [b*NT, b*NT + NT): every workgroup
// reads all ids for the per-expert totals (and the counts of the slots before its own), scans the
// padded totals exactly as align_block does, and places its own slots at expert start + slots of
// that expert before the chunk + rank inside the chunk (the per-wave lane masks of align_block), so
// the order is the same stable slot order and every output equals align_block's. The padding
// sentinels, the tail, the block owners and ntp are split over the workgroups; every output element
// is written by exactly one thread. No workgroup depends on another (no workspace, no flags).
template <int NT, int EMAX>
__global__ void __launch_bounds__(NT)
moe_align_multi_kernel(const int32_t* __restrict__ ids, int64_t numel, int E, int bm, int64_t P,
                       int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
                       int32_t* __restrict__ ntp_out, int32_t* __restrict__ inv_pos) {
  constexpr int NW = NT / 64;
  static_assert(NT >= EMAX, "one scan pass: a thread per expert");
  __shared__ int cnt[EMAX];
  __shared__ int before[EMAX];
  __shared__ int base[EMAX];
  __shared__ unsigned long long mask[NW][EMAX];
  __shared__ int pre[NW][EMAX];
  __shared__ int wsums[NW];
  __shared__ int total_s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t nb = gridDim.x, b = blockIdx.x;
  const int64_t c0 = b * NT;
  for (int e = tid; e < EMAX; e += NT) {
    cnt[e] = 0;
    before[e] = 0;
  }
  for (int i = tid; i < NW * EMAX; i += NT) (&mask[0][0])[i] = 0ull;
  lds_barrier();
  for (int64_t i0 = 0; i0 < numel; i0 += 8 * NT) {
    int ev[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t i = i0 + u * NT + tid;
      ev[u] = i < numel ? ids[i] : -1;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t i = i0 + u * NT + tid;
      const int e = ev[u];
      if (e < 0 || e >= E) continue;
      atomicAdd(&cnt[e], 1);
      if (i < c0) atomicAdd(&before[e], 1);
    }
  }
  lds_barrier();
  // exclusive scan of padded counts over experts (one expert per thread)
  const int padded = tid < E ? (cnt[tid] + bm - 1) / bm * bm : 0;
  int incl = padded;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int n = __shfl_up(incl, o, 64);
    if (lane >= o) incl += n;
  }
  if (lane == 63) wsums[wave] = incl;
  lds_barrier();
  if (tid == 0) {
    int run = 0;
    for (int w = 0; w < NW; ++w) {
      const int sw = wsums[w];
      wsums[w] = run;
      run += sw;
    }
    total_s = run;
  }
  lds_barrier();
  const int start = tid < E ? incl - padded + wsums[wave] : 0;
  const int total = total_s;
  if (tid < E) base[tid] = start;
  lds_barrier();
  // this workgroup's share of the padding sentinels, the tail, the block owners and ntp
  const int64_t stride = nb * NT;
  for (int64_t x = b * NT + tid; x < (int64_t)E * (bm - 1); x += stride) {
    const int e = (int)(x / (bm - 1)), j = (int)(x - (int64_t)e * (bm - 1));
    const int c = cnt[e];
    if (c + j < (c + bm - 1) / bm * bm) sorted_ids[base[e] + c + j] = (int32_t)numel;
  }
  for (int64_t i = total + b * NT + tid; i < P; i += stride) sorted_ids[i] = (int32_t)numel;
  if (tid < E && tid % nb == b) {
    const int b0 = start / bm, nbl = (cnt[tid] + bm - 1) / bm;
    for (int k = 0; k < nbl; ++k) expert_ids[b0 + k] = tid;
  }
  const int64_t nblocks = (P + bm - 1) / bm;
  for (int64_t k = total / bm + b * NT + tid; k < nblocks; k += stride) expert_ids[k] = E - 1;
  if (b == 0 && tid == 0) *ntp_out = total;
  // stable scatter of this workgroup's slots
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int64_t i = c0 + tid;
  int e = -1;
  if (i < numel) {
    e = ids[i];
    if (e >= E) e = -1;
  }
  if (e >= 0) atomicOr(&mask[wave][e], 1ull << lane);
  lds_barrier();
  const uint64_t m = e >= 0 ? mask[wave][e] : 0ull;
  if (tid < E) {
    int run = start + before[tid];
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      pre[w][tid] = run;
      run += __popcll(mask[w][tid]);
    }
  }
  lds_barrier();
  if (e >= 0) {
    const int off = pre[wave][e] + __popcll(m & below);
    sorted_ids[off] = (int32_t)i;
    if (inv_pos) inv_pos[i] = off;
  } else if (i < numel && inv_pos) {
    inv_pos[i] = -1;  // dropped slot: the combine skips it
  }
}

// E <= 256: 1024 threads; E <= 512: 512 threads (the per-wave masks and offsets scale with both)
template <int NT, int EMAX>
__global__ void __launch_bounds__(NT)
moe_align_kernel(const int32_t* __restrict__ ids, int64_t numel, int E, int bm, int64_t P,
                 int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
                 int32_t* __restrict__ ntp_out, int32_t* __restrict__ inv_pos) {
  align_block<NT, EMAX, kAlignHeld>(ids, numel, E, bm, P, sorted_ids, expert_ids, ntp_out, inv_pos);
}

// Small-batch route + align (+ per-token act quant of x) in one launch. Workgroup 0 routes the T
// tokens (one wave per token, 16 at a time), keeping the ids in LDS, then aligns them; workgroups
// 1..T each quantize one token row of x (quant_row, the act-quant kernel's arithmetic) in parallel
// with it.
constexpr int kPrepThreads = 1024;
constexpr int kPrepMaxSlots = 256;

// Align of the prep launch's slots (at most 256): one wave counts, ranks, scans and places the
// slots with no LDS barrier, then (align_fill, after one barrier) the workgroup writes the padding
// sentinels, the tail and the block owners. Lane l owns slots l + 64c (c < 4) and experts l + 64k
// (k < EPL). A slot's position is its expert's start plus the number of earlier slots of that
// expert, so every output equals align_block's. That rank is found per 64-slot chunk: each slot
// sets its lane's bit in its expert's LDS mask, the bits below its own count the chunk's earlier
// slots and the expert's LDS count those of the earlier chunks; the lowest lane of each expert
// then adds the chunk's slots to the count and clears the mask. The wave's LDS operations complete
// in issue order (volatile keeps the compiler to that order), so no barrier separates the steps.
// ids in LDS; base_s, cnt_s, mask_s, total_s: LDS for the expert starts, the counts, the chunk
// masks and ntp. Against align_block (which the prep launch ran past 64 slots, where a loop over
// every slot per lane counted the experts): configs[4] T=16 prep launch 8.1 -> 7.6 us.
template <int EPL>
__device__ __forceinline__ void align_wave(const int32_t* ids, int numel, int E, int bm, int64_t P,
                                           int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids,
                                           int32_t* __restrict__ ntp_out, int32_t* __restrict__ inv_pos, int* base_s,
                                           int* cnt_s, unsigned long long* mask_s, int* total_s) {
  constexpr int kChunks = kPrepMaxSlots / 64;
  const int lane = threadIdx.x & 63;
  volatile int* vcnt = cnt_s;
  volatile unsigned long long* vmask = mask_s;
#pragma unroll
  for (int k = 0; k < EPL; ++k) {
    vcnt[lane + 64 * k] = 0;
    vmask[lane + 64 * k] = 0ull;
  }
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int ev[kChunks], rank[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int sl = 64 * c + lane;
    int e = sl < numel ? ids[sl] : -1;
    e = (e >= 0 && e < E) ? e : -1;
    ev[c] = e;
    rank[c] = 0;
    if (64 * c < numel) {  // uniform
      if (e >= 0) atomicOr(const_cast<unsigned long long*>(&vmask[e]), 1ull << lane);
      const uint64_t m = e >= 0 ? vmask[e] : 0ull;
      const int before = e >= 0 ? vcnt[e] : 0;
      rank[c] = before + __popcll(m & below);
      if (e >= 0 && (m & below) == 0ull) {
        vcnt[e] = before + __popcll(m);
        vmask[e] = 0ull;
      }
    }
  }
  // exclusive scan of the padded counts over experts in order
  int run = 0;
#pragma unroll
  for (int k = 0; k < EPL; ++k) {
    const int e = lane + 64 * k;
    const int padded = e < E ? (vcnt[e] + bm - 1) / bm * bm : 0;
    int incl = padded;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int n = __shfl_up(incl, o, 64);
      if (lane >= o) incl += n;
    }
    if (e < E) base_s[e] = run + incl - padded;
    run += __shfl(incl, 63, 64);
  }
  const int total = run;
  volatile int* vbase = base_s;
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int sl = 64 * c + lane;
    if (ev[c] >= 0) {
      const int off = vbase[ev[c]] + rank[c];
      sorted_ids[off] = sl;
      if (inv_pos) inv_pos[sl] = off;
    } else if (sl < numel && inv_pos) {
      inv_pos[sl] = -1;  // dropped slot: the combine skips it
    }
  }
  if (lane == 0) {
    *ntp_out = total;
    *total_s = total;
  }
}

// The rest of the align after align_wave, spread over the NT threads of the workgroup (after a
// barrier): padding rows of each expert, the tail [total, P) and the block owners.
template <int NT>
__device__ __forceinline__ void align_fill(int numel, int E, int bm, int64_t P, int32_t* __restrict__ sorted_ids,
                                           int32_t* __restrict__ expert_ids, const int* base_s, const int* cnt_s,
                                           int total) {
  const int tid = threadIdx.x;
  const int pad = bm - 1;
  for (int x = tid; x < E * pad; x += NT) {
    const int e = x / pad, j = x - e * pad;
    const int c = cnt_s[e];
    if (c + j < (c + bm - 1) / bm * bm) sorted_ids[base_s[e] + c + j] = numel;
  }
  for (int e = tid; e < E; e += NT) {
    const int nb = (cnt_s[e] + bm - 1) / bm, b0 = base_s[e] / bm;
    for (int b = 0; b < nb; ++b) expert_ids[b0 + b] = e;
  }
  for (int i = total + tid; i < (int)P; i += NT) sorted_ids[i] = numel;
  const int nblocks = (int)((P + bm - 1) / bm);
  for (int b = total / bm + tid; b < nblocks; b += NT) expert_ids[b] = E - 1;
}


// slots: instead of the align, give every slot a block of its own (slot s: padded row s*bm, the
// block's other rows sentinels, block owner its expert; ntp = slots * bm). Only [0, ntp) of
// sorted_ids and the first `slots` blocks of expert_ids are written: the grouped GEMMs read no row
// at or past ntp, and the combine reads inv_pos.
template <int PER, int CPT>
__global__ void __launch_bounds__(kPrepThreads)
moe_prep_kernel(const void* __restrict__ logits, int ldtype, int64_t T, int E, int top_k, int renorm,
                float* __restrict__ tw, int32_t* __restrict__ ids, int bm, int64_t P,
                int32_t* __restrict__ sorted_ids, int32_t* __restrict__ expert_ids, int32_t* __restrict__ ntp,
                int32_t* __restrict__ inv_pos, const uint16_t* __restrict__ x, int xdtype, int64_t K, int64_t ldx,
                uint8_t* __restrict__ xq, int64_t ldq, float* __restrict__ xs, int slots) {
  if (blockIdx.x > 0) {
    __shared__ float red[kPrepThreads / 64];
    const int64_t m = blockIdx.x - 1;
    quant_row<CPT, kPrepThreads>(x + m * ldx, K, xdtype, xq + m * ldq, xs + m, red);
    return;
  }
  __shared__ int32_t ids_s[kPrepMaxSlots];
  // one token per wave, 16 at a time; past 16 tokens with 16-bit logits two per wave (token t and
  // t + 16), whose routes run interleaved
  constexpr int kW = kPrepThreads / 64;
  for (int64_t t = threadIdx.x >> 6; t < T; t += 2 * kW) {
    if (t + kW < T && ldtype != kF32) {
      route_token_pair<PER>(logits, ldtype, t, t + kW, E, top_k, renorm, tw, ids, ids_s);
    } else {
      route_token<PER>(logits, ldtype, t, E, top_k, renorm, tw, ids, ids_s);
      if (t + kW < T) route_token<PER>(logits, ldtype, t + kW, E, top_k, renorm, tw, ids, ids_s);
    }
  }
  lds_barrier();
  if (slots) {
    const int S = (int)(T * top_k);
    // a slot left without an expert (NaN logits leave none to choose) is dropped, as the align
    // drops it: sentinel rows only, a valid block owner for the weight addresses, inv_pos -1
    auto eok = [&](int s) { return ids_s[s] >= 0 && ids_s[s] < E; };
    for (int i = threadIdx.x; i < S * bm; i += kPrepThreads) sorted_ids[i] = (i % bm == 0 && eok(i / bm)) ? i / bm : S;
    if (threadIdx.x < S) {
      const bool ok = eok(threadIdx.x);
      expert_ids[threadIdx.x] = ok ? ids_s[threadIdx.x] : E - 1;
      inv_pos[threadIdx.x] = ok ? (int32_t)threadIdx.x * bm : -1;
    }
    if (threadIdx.x == 0) *ntp = S * bm;
    return;
  }
  // one wave counts, ranks, scans and places the slots, then the workgroup fills
  __shared__ int base_s[64 * PER], cnt_s[64 * PER], total_s;
  __shared__ unsigned long long mask_s[64 * PER];
  if (threadIdx.x < 64)
    align_wave<PER>(ids_s, (int)(T * top_k), E, bm, P, sorted_ids, expert_ids, ntp, inv_pos, base_s, cnt_s, mask_s,
                    &total_s);
  lds_barrier();
  align_fill<kPrepThreads>((int)(T * top_k), E, bm, P, sorted_ids, expert_ids, base_s, cnt_s, total_s);
}

// Route of T tokens and the per-token quant of x in one launch, for batches past the one-launch
// prep (more than 256 slots) with rows the wave quant covers (K <= 4096): workgroups
// [0, route_blocks) route four tokens each (a wave per token, route_token), the rest quantize four
// rows each (a wave per row, quant_row_wave: the act-quant kernel's arithmetic). The halves share
// nothing, so they run side by side where they were two launches; the align follows it.
template <int PER, int CPW>
__global__ void __launch_bounds__(256)
moe_route_quant_kernel(const void* __restrict__ logits, int ldtype, int64_t T, int E, int top_k, int renorm,
                       float* __restrict__ tw, int32_t* __restrict__ ids, int64_t route_blocks,
                       const uint16_t* __restrict__ x, int xdtype, int64_t K, int64_t ldx, uint8_t* __restrict__ xq,
                       int64_t ldq, float* __restrict__ xs) {
  const int64_t w = threadIdx.x >> 6;  // whole waves leave together below
  if ((int64_t)blockIdx.x < route_blocks) {
    const int64_t t = (int64_t)blockIdx.x * 4 + w;
    if (t < T) route_token<PER>(logits, ldtype, t, E, top_k, renorm, tw, ids, nullptr);
    return;
  }
  const int64_t m = ((int64_t)blockIdx.x - route_blocks) * 4 + w;
  if (m < T) quant_row_wave<CPW>(x + m * ldx, K, xdtype, xq + m * ldq, xs + m, threadIdx.x & 63);
}

// Four channels per thread: 16-byte (f32 y) or 8-byte (bf16/fp16 y) loads of y, one 8-byte (or
// 16-byte f32) store. YF32: y holds f32 rows; else rows in ydt (bf16/fp16), widened exactly.
template <bool YF32>
__global__ void __launch_bounds__(256)
moe_combine_kernel(const void* __restrict__ yv, int ydt, int64_t ldy, const int32_t* __restrict__ inv_pos,
                   const float* __restrict__ tw, int64_t T, int top_k, int64_t H, void* __restrict__ out, int dtype) {
  const int64_t h = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (h >= H) return;
  for (int64_t t = blockIdx.y; t < T; t += gridDim.y) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = 0; j < top_k; ++j) {
      const int64_t pos = inv_pos[t * top_k + j];
      if (pos >= 0) {
        const float w = tw[t * top_k + j];
        float4 v;
        if constexpr (YF32) {
          v = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(yv) + pos * ldy + h);
        } else {
          const uint2 r = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(yv) + pos * ldy + h);
          v = make_float4(from_dtype((uint16_t)(r.x & 0xffffu), ydt), from_dtype((uint16_t)(r.x >> 16), ydt),
                          from_dtype((uint16_t)(r.y & 0xffffu), ydt), from_dtype((uint16_t)(r.y >> 16), ydt));
        }
        // one FMA per slot, in slot order (the fused gemm2 + combine does the same)
        acc.x = fmaf(w, v.x, acc.x);
        acc.y = fmaf(w, v.y, acc.y);
        acc.z = fmaf(w, v.z, acc.z);
        acc.w = fmaf(w, v.w, acc.w);
      }
    }
    if (dtype == kF32) {
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + t * H + h) = acc;
    } else {
      const uint32_t lo = (uint32_t)to_dtype(acc.x, dtype) | ((uint32_t)to_dtype(acc.y, dtype) << 16);
      const uint32_t hi = (uint32_t)to_dtype(acc.z, dtype) | ((uint32_t)to_dtype(acc.w, dtype) << 16);
      *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + t * H + h) = make_uint2(lo, hi);
    }
  }
}

// Eight channels per thread for 16-bit y rows (H and ldy multiples of 8, 16-byte aligned y and
// out): one 16-byte load per slot row and 16-byte stores, where the four-channel kernel above moves
// 8 bytes per load. Each channel's FMA chain is the four-channel kernel's, so the bits are too.
__global__ void __launch_bounds__(256)
moe_combine8_kernel(const uint16_t* __restrict__ y, int ydt, int64_t ldy, const int32_t* __restrict__ inv_pos,
                    const float* __restrict__ tw, int64_t T, int top_k, int64_t H, void* __restrict__ out, int dtype) {
  const int64_t h = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (h >= H) return;
  for (int64_t t = blockIdx.y; t < T; t += gridDim.y) {
    float acc[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = 0.f;
    for (int j = 0; j < top_k; ++j) {
      const int64_t pos = inv_pos[t * top_k + j];
      if (pos >= 0) {
        const float w = tw[t * top_k + j];
        const uint4 r = *reinterpret_cast<const uint4*>(y + pos * ldy + h);
        const uint32_t wd[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] = fmaf(w, from_dtype((uint16_t)(wd[q] & 0xffffu), ydt), acc[2 * q]);
          acc[2 * q + 1] = fmaf(w, from_dtype((uint16_t)(wd[q] >> 16), ydt), acc[2 * q + 1]);
        }
      }
    }
    if (dtype == kF32) {
      float4* o = reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + t * H + h);
      o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
      o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    } else {
      uint32_t pk[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        pk[q] = (uint32_t)to_dtype(acc[2 * q], dtype) | ((uint32_t)to_dtype(acc[2 * q + 1], dtype) << 16);
      *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(out) + t * H + h) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    }
  }
}

template <template <int> class F, typename... A>
static void with_per(int E, A... a) {
  if (E <= 64) F<1>::run(a...);
  else if (E <= 128) F<2>::run(a...);
  else if (E <= 256) F<4>::run(a...);
  else F<8>::run(a...);
}

template <int PER> struct RouteLaunch {
  static void run(const void* logits, int dtype, int64_t T, int E, int top_k, int renorm, float* tw, int32_t* ids,
                  hipStream_t stream) {
    const int per_block = 4;
    hipLaunchKernelGGL(moe_route_kernel<PER>, dim3((unsigned)((T + per_block - 1) / per_block)), dim3(per_block * 64),
                       0, stream, logits, dtype, T, E, top_k, renorm, tw, ids);
  }
};

int launch_moe_route(const void* logits, int dtype, int64_t T, int E, int top_k, int renorm, float* tw,
                     int32_t* ids, hipStream_t stream) {
  if (T <= 0) return kOk;
  with_per<RouteLaunch>(E, logits, dtype, T, E, top_k, renorm, tw, ids, stream);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

int launch_moe_align(const int32_t* ids, int64_t numel, int E, int bm, int64_t P, int32_t* sorted_ids,
                     int32_t* expert_ids, int32_t* ntp, int32_t* inv_pos, hipStream_t stream) {
  // one workgroup per 1024 (E > 256: 512) slots above kAlignMultiMin slots; below, the one-workgroup
  // kernel, which keeps the ids it reads in LDS
  if (numel > kAlignMultiMin) {
    if (E <= 256)
      hipLaunchKernelGGL((moe_align_multi_kernel<1024, 256>), dim3((unsigned)((numel + 1023) / 1024)), dim3(1024), 0,
                         stream, ids, numel, E, bm, P, sorted_ids, expert_ids, ntp, inv_pos);
    else
      hipLaunchKernelGGL((moe_align_multi_kernel<512, 512>), dim3((unsigned)((numel + 511) / 512)), dim3(512), 0,
                         stream, ids, numel, E, bm, P, sorted_ids, expert_ids, ntp, inv_pos);
    return hipGetLastError() == hipSuccess ? kOk : kErrHip;
  }
  if (E <= 256)
    hipLaunchKernelGGL((moe_align_kernel<1024, 256>), dim3(1), dim3(1024), 0, stream, ids, numel, E, bm, P, sorted_ids,
                       expert_ids, ntp, inv_pos);
  else
    hipLaunchKernelGGL((moe_align_kernel<512, 512>), dim3(1), dim3(512), 0, stream, ids, numel, E, bm, P, sorted_ids,
                       expert_ids, ntp, inv_pos);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

template <int PER> struct PrepLaunch {
  template <int CPT>
  static void go(dim3 grid, hipStream_t stream, const void* logits, int ldtype, int64_t T, int E, int top_k,
                 int renorm, float* tw, int32_t* ids, int bm, int64_t P, int32_t* sorted_ids, int32_t* expert_ids,
                 int32_t* ntp, int32_t* inv_pos, const uint16_t* x, int xdtype, int64_t K, int64_t ldx, uint8_t* xq,
                 int64_t ldq, float* xs, int slots) {
    hipLaunchKernelGGL((moe_prep_kernel<PER, CPT>), grid, dim3(kPrepThreads), 0, stream, logits, ldtype, T, E, top_k,
                       renorm, tw, ids, bm, P, sorted_ids, expert_ids, ntp, inv_pos, x, xdtype, K, ldx, xq, ldq, xs,
                       slots);
  }
  static void run(int cpt, const void* logits, int ldtype, int64_t T, int E, int top_k, int renorm, float* tw,
                  int32_t* ids, int bm, int64_t P, int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntp,
                  int32_t* inv_pos, const void* x, int xdtype, int64_t K, int64_t ldx, uint8_t* xq, int64_t ldq,
                  float* xs, int slots, hipStream_t stream) {
    const dim3 grid((unsigned)(1 + (x ? T : 0)));
    const uint16_t* xp = reinterpret_cast<const uint16_t*>(x);
#define W4A8_PREP(C) go<C>(grid, stream, logits, ldtype, T, E, top_k, renorm, tw, ids, bm, P, sorted_ids, expert_ids, \
                           ntp, inv_pos, xp, xdtype, K, ldx, xq, ldq, xs, slots)
    if (cpt == 1) W4A8_PREP(1);
    else if (cpt == 2) W4A8_PREP(2);
    else if (cpt == 4) W4A8_PREP(4);
    else W4A8_PREP(0);
#undef W4A8_PREP
  }
};

template <int PER> struct RouteQuantLaunch {
  static void run(int cpw, const void* logits, int ldtype, int64_t T, int E, int top_k, int renorm, float* tw,
                  int32_t* ids, const uint16_t* x, int xdtype, int64_t K, int64_t ldx, uint8_t* xq, int64_t ldq,
                  float* xs, hipStream_t stream) {
    const int64_t rb = (T + 3) / 4;
    const dim3 grid((unsigned)(2 * rb));
#define W4A8_RQ(C) hipLaunchKernelGGL((moe_route_quant_kernel<PER, C>), grid, dim3(256), 0, stream, logits, ldtype, T, E, \
                                      top_k, renorm, tw, ids, rb, x, xdtype, K, ldx, xq, ldq, xs)
    if (cpw <= 1) W4A8_RQ(1);
    else if (cpw <= 2) W4A8_RQ(2);
    else if (cpw <= 4) W4A8_RQ(4);
    else W4A8_RQ(8);
#undef W4A8_RQ
  }
};

// Route + per-token quant of x as one launch (rows of K <= 4096 elements); kErrUnsupported for
// longer rows, which take the route and act-quant kernels.
int launch_moe_route_quant(const void* logits, int ldtype, int64_t T, int E, int top_k, int renorm, float* tw,
                           int32_t* ids, const void* x, int xdtype, int64_t K, int64_t ldx, uint8_t* xq, int64_t ldq,
                           float* xs, hipStream_t stream) {
  if (T <= 0) return kOk;
  if (K > 64 * 8 * 8 || T > (int64_t)1 << 30) return kErrUnsupported;
  const int cpw = (int)((K + 511) / 512);
  with_per<RouteQuantLaunch>(E, cpw, logits, ldtype, T, E, top_k, renorm, tw, ids,
                             reinterpret_cast<const uint16_t*>(x), xdtype, K, ldx, xq, ldq, xs, stream);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

bool moe_prep_fits(int64_t T, int top_k) { return T * top_k <= kPrepMaxSlots; }

// Route + align (+ act quant of x when x is given) of a small batch in one launch; the caller
// checks moe_prep_fits first.
int launch_moe_prep(const void* logits, int ldtype, int64_t T, int E, int top_k, int renorm, float* tw,
                    int32_t* ids, int bm, int64_t P, int32_t* sorted_ids, int32_t* expert_ids, int32_t* ntp,
                    int32_t* inv_pos, const void* x, int xdtype, int64_t K, int64_t ldx, uint8_t* xq, int64_t ldq,
                    float* xs, int slots, hipStream_t stream) {
  if (T <= 0) return kOk;
  const int c = quant_row_cpt(K, kPrepThreads);
  const int cpt = c >= 1 && c <= 4 ? c : 0;
  with_per<PrepLaunch>(E, cpt, logits, ldtype, T, E, top_k, renorm, tw, ids, bm, P, sorted_ids, expert_ids, ntp,
                       inv_pos, x, xdtype, K, ldx, xq, ldq, xs, slots, stream);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

int launch_moe_combine(const void* y, int ydt, int64_t ldy, const int32_t* inv_pos, const float* tw, int64_t T,
                       int top_k, int64_t H, void* out, int dtype, hipStream_t stream) {
  if (T <= 0) return kOk;
  const unsigned gy = (unsigned)(T < 65535 ? T : 65535);
  if (ydt != kF32 && H % 8 == 0 && ldy % 8 == 0 && ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(out)) & 15) == 0) {
    hipLaunchKernelGGL(moe_combine8_kernel, dim3((unsigned)((H / 8 + 255) / 256), gy), dim3(256), 0, stream,
                       reinterpret_cast<const uint16_t*>(y), ydt, ldy, inv_pos, tw, T, top_k, H, out, dtype);
    return hipGetLastError() == hipSuccess ? kOk : kErrHip;
  }
  dim3 grid((unsigned)((H / 4 + 255) / 256), gy);
  if (ydt == kF32)
    hipLaunchKernelGGL(moe_combine_kernel<true>, grid, dim3(256), 0, stream, y, ydt, ldy, inv_pos, tw, T, top_k, H,
                       out, dtype);
  else
    hipLaunchKernelGGL(moe_combine_kernel<false>, grid, dim3(256), 0, stream, y, ydt, ldy, inv_pos, tw, T, top_k, H,
                       out, dtype);
  return hipGetLastError() == hipSuccess ? kOk : kErrHip;
}

}  // namespace w4a8

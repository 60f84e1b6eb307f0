/*
 * w4a8_mi355x.h -- C ABI of libw4a8_mi355x.so, the MI355X (gfx950) W4A8 quantized-linear path.
 *
 * Drop-in boundary for minisglang-rdna4's W4A8 hot path. The reference calls three external HIP
 * packages from its Python provider (python/minisgl/quant/kernels.py): fp8_wmma (GEMM/GEMV core),
 * moe_hip (route + align) and tail_hip (act-quant epilogues). Each entry point below names the
 * reference interface it replaces. Conventions:
 *   - plain device pointers, sizes and a hipStream_t passed as void*; no framework types;
 *   - every function returns 0 on success, otherwise a status code, and w4a8_last_error() returns
 *     the message of the calling thread's last failure (argument errors are detected on the host
 *     before any launch);
 *   - no entry point allocates: outputs and workspaces come from the caller, so every launch is
 *     capturable into a HIP graph as long as its pointers stay fixed;
 *   - dtype codes: 0 = bf16, 1 = fp16, 2 = f32. Scale formats: 0 = fp16 group scales,
 *     1 = E8M0 (uint8) 32-element block scales, 2 = NVFP4 e4m3 (uint8) 16-element block scales
 *     with the per-output-channel f32 global in the zeros slot (its bits as int32; (N,) per
 *     matrix, (E, N) for experts). Weight formats: 0 = int4 codes, 1 = e2m1 codes.
 *
 * Data layouts (all row-major):
 *   x_fp8 (M, ldx) uint8 e4m3fn codes; act_scales (M,) f32.
 *   w_packed (N, K/8) int32 -- the reference op layout: nibble j of word k/8 is input k.
 *   w_tile: the W4 tile layout written by w4a8_repack_weights, w4a8_tile_bytes(N, K) bytes.
 *   scales (K/group, N) group-major; zeros (K/group, N/8) int32, 8 channels per word, or NULL
 *   (symmetric, zero point 8). MoE weights stack experts on the leading dimension.
 */
#ifndef W4A8_MI355X_H
#define W4A8_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W4A8_OK 0
#define W4A8_ERR_INVALID 1
#define W4A8_ERR_UNSUPPORTED 2
#define W4A8_ERR_HIP 3

#define W4A8_SCALE_F16 0
#define W4A8_SCALE_E8M0 1
#define W4A8_SCALE_E4M3 2

/* ABI revision of this header. A client checks w4a8_abi_version() == W4A8_ABI_VERSION at load:
 * revision 3 inserted y_dtype as w4a8_moe_combine's second argument, revision 4 added
 * w4a8_linear_launch_count, w4a8_moe_gelu_tanh_mul and w4a8_moe_gemm2_combine's row_dtype,
 * revision 5 added w4a8_moe_gemm_quant. */
#define W4A8_ABI_VERSION 5
int w4a8_abi_version(void);

/* Message of the calling thread's last failed call. */
const char* w4a8_last_error(void);

/* Per-token fp8-e4m3 activation quant: s = max(amax/448, 1e-8), q = e4m3_rne(x/s).
 * Replaces fp8_wmma's in-op compute_act_fp8_and_scales_kernel (python/minisgl/quant/kernels.py:
 * 1512-1515, contract :1703-1712) and the (x_fp8, act_scales) pair tail_hip.rms_norm_quant emits
 * (python/minisgl/layers/norm.py:27-46). row_count: optional device int32 bounding the rows done
 * (rows at and past it are left untouched), for graph-captured MoE launches. */
int w4a8_act_quant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* x_fp8, int64_t ldq,
                   float* act_scales, const int32_t* row_count, void* stream);

/* Bytes of the W4 tile layout for an (N, K) weight (N % 16 == 0); -1 on bad sizes. */
int64_t w4a8_tile_bytes(int64_t N, int64_t K);

/* Load-time repack of op-layout codes (rows = N, or E*N for a stacked MoE weight) into W4 tiles.
 * Replaces the layout half of awq_to_op_layout / gptq_to_op_layout (python/minisgl/quant/
 * kernels.py:255-346) and mxfp4.convert_mxfp4_weight / convert_mxfp4_moe_e8m0
 * (python/minisgl/quant/mxfp4.py:134-206), whose (N, K/8) int32 output is this call's input. */
int w4a8_repack_weights(const int32_t* w_packed, int64_t N, int64_t K, int wfmt, void* w_tile, void* stream);

/* Workspace bytes w4a8_gemm may use for (M, N, K) and a kernel choice (0 auto, 1 decode, 2 prefill);
 * -1 on bad sizes. Prefill calls of 1024 rows or more on 16384+ output channels: room for the codes
 * rewritten in the GEMM's operand order with one row-sum seed per row and 128 inputs, which symmetric
 * int4 and MXFP4 weights take (a launch before the GEMM); without it the GEMM reads the row-major
 * codes, with the same outputs. */
int64_t w4a8_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int kernel);

/* Dense W4A8 GEMM: out[m, n] = act_scales[m] * sum_g scale[g, n] * sum_{k in g} e4m3(x[m,k]) * w(n,k).
 * Replaces fp8_wmma.mmq_fp8_gemm (python/minisgl/quant/kernels.py:1686-1734; arms decode_gemv and
 * wmma_tiled_tuned chosen by _pick_dense_kernel :1456-1632) and, with silu = 1,
 * fp8_wmma.mmq_fp8_gemm_silu (kernels.py:1737-1753): N = 2*inter with gate rows first, output
 * (M, inter) = silu(gate) * up rounded as in tools/w4a8_gemm_silu_parity.py:52-54.
 * kernel: 0 auto (M <= 16 decode, else prefill), 1 decode, 2 prefill. */
int w4a8_gemm(const uint8_t* x_fp8, int64_t ldx, const float* act_scales, int64_t M, const void* w_tile, int64_t N,
              int64_t K, const void* scales, int scale_fmt, const int32_t* zeros, int wfmt, int64_t group_size,
              void* out, int out_dtype, int64_t ldo, int silu, void* workspace, int64_t workspace_bytes, int kernel,
              void* stream);

/* Workspace bytes w4a8_linear may need for M rows of K inputs (the fp8 codes and scales of x when
 * they are not produced inside the GEMM kernel; for prefill calls of 1024 rows or more, also the
 * codes again in the GEMM's operand order with one row-sum seed per row and 128 inputs, which
 * symmetric int4 and MXFP4 weights of 2048+ output channels use, x quantized straight into it);
 * -1 on bad sizes. w4a8_linear also accepts a workspace of just the codes and scales (M * K and
 * 4 * M bytes, each rounded up to 256): such calls run the GEMM on the row-major codes, with the
 * same outputs. */
int64_t w4a8_linear_workspace_bytes(int64_t M, int64_t K);

/* Dense W4A8 linear on bf16/fp16 activations x (M, ldx): per-token fp8 quant of x, then the GEMM of
 * w4a8_gemm, with the same outputs bit for bit as w4a8_act_quant followed by w4a8_gemm. This is
 * fp8_wmma.mmq_fp8_gemm / mmq_fp8_gemm_silu called without a producer pair, which quantize in-op
 * (python/minisgl/quant/kernels.py:1686-1753, in-op quant :1703-1712). Decode calls (M <= 16) whose
 * rows the GEMV can quantize itself (int4 with groups of 128+ and MXFP4, up to 64 values per thread
 * of its row phase, 128 on weights of over 64 KiB per workgroup: at K = 4096 up to 8 rows, 16 on
 * the wide gate_up shape; see w4a8_linear_launch_count) are a single launch; otherwise one act-quant
 * launch writes the workspace (w4a8_linear_workspace_bytes, 16-byte aligned) first. */
int w4a8_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* w_tile, int64_t N,
                const void* scales, int scale_fmt, const int32_t* zeros, int wfmt, int64_t group_size, void* out,
                int out_dtype, int64_t ldo, int silu, void* workspace, int64_t workspace_bytes, int kernel,
                void* stream);

/* Kernel launches a w4a8_linear call of these shapes and formats makes: 1 when the per-token quant
 * runs inside the GEMV (decode calls whose rows the GEMV quantizes itself), 2 when an act-quant
 * launch comes first; 0 for M = 0; minus the status code on bad arguments. Host-only (no device
 * call), for callers that budget launches per step. No counterpart in the reference, whose in-op
 * quant is always a separate launch (python/minisgl/quant/kernels.py:1512-1515). */
int w4a8_linear_launch_count(int64_t M, int64_t N, int64_t K, int x_dtype, int scale_fmt, int has_zeros, int wfmt,
                             int64_t group_size, int silu, int kernel);

/* w4a8_linear for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). No counterpart in the reference: its ops
 * allocate their act-quant buffers in-op. Same arguments and results as w4a8_linear, bit for bit,
 * minus the workspace: the act-quant staging (w4a8_linear_workspace_bytes(M, K)) lives in a static
 * device array of w4a8_linear_noalloc_max_bytes() = 64 MiB that each GPU holds from its first call
 * until the process ends. Larger M*K is refused (kErrInvalid, message names the limit). Calls on
 * one GPU share that array, so calls that overlap on one GPU (several streams or threads) race.
 * The entry point calls no allocator. */
int64_t w4a8_linear_noalloc_max_bytes(void);
int w4a8_linear_noalloc(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* w_tile, int64_t N,
                        const void* scales, int scale_fmt, const int32_t* zeros, int wfmt, int64_t group_size,
                        void* out, int out_dtype, int64_t ldo, int silu, int kernel, void* stream);

/* Softmax + top-k (ties keep the lower expert index) + optional renormalisation. Replaces the
 * route half of moe_hip.moe_route_align (python/minisgl/quant/kernels.py:423-447; tie rule
 * python/minisgl/layers/moe.py:1218-1227). E <= 512. */
int w4a8_moe_route(const void* logits, int logits_dtype, int64_t T, int64_t E, int top_k, int renormalize,
                   float* topk_w, int32_t* topk_ids, void* stream);

/* Route + align in one call: replaces moe_hip.moe_route_align (python/minisgl/quant/kernels.py:423-447),
 * with the outputs of w4a8_moe_route and w4a8_moe_align (numel = T*top_k). When x is non-NULL it also
 * quantizes x (T, K) per token into x_fp8 / x_scales, as w4a8_act_quant does (the act-quant the grouped
 * gemm1 needs, kernels.py:1703-1712). Up to 256 slots (T*top_k) run as a single launch: one workgroup
 * routes and aligns while the others quantize the token rows. Past that, rows of K <= 4096 are
 * quantized in the routing launch (a wave per token routes, a wave per row quantizes) and the align
 * follows: two launches. */
int w4a8_moe_route_align(const void* logits, int logits_dtype, int64_t T, int64_t E, int top_k, int renormalize,
                         int block_m, int64_t P, float* topk_w, int32_t* topk_ids, int32_t* sorted_ids,
                         int32_t* expert_ids, int32_t* ntp, int32_t* inv_pos, const void* x, int x_dtype, int64_t K,
                         int64_t ldx, uint8_t* x_fp8, int64_t ldq, float* x_scales, void* stream);

/* Route (+ the per-token quant of x) as w4a8_moe_route_align, but instead of the align every slot gets a
 * block of its own: slot s's padded row is s*block_m, the block's other rows are sentinels
 * (T*top_k), expert_ids[s] is its expert, inv_pos[s] = s*block_m, ntp = T*top_k*block_m. Only
 * [0, ntp) of sorted_ids and the first T*top_k blocks of expert_ids are written. No counterpart in
 * the reference: w4a8_moe uses it for calls of up to 8 tokens on the decode arm (a token's experts
 * are distinct, and a few tokens share few), where the align's sort and its padding fills are a
 * third of the routing launch and the grouped GEMMs read no row past ntp. Needs T*top_k <= 256,
 * T*top_k <= E (the grouped GEMMs size their grids for numel/block_m + min(E, numel) blocks),
 * T*top_k*block_m <= P and inv_pos. */
int w4a8_moe_route_slots(const void* logits, int logits_dtype, int64_t T, int64_t E, int top_k, int renormalize,
                         int block_m, int64_t P, float* topk_w, int32_t* topk_ids, int32_t* sorted_ids,
                         int32_t* expert_ids, int32_t* ntp, int32_t* inv_pos, const void* x, int x_dtype, int64_t K,
                         int64_t ldx, uint8_t* x_fp8, int64_t ldq, float* x_scales, void* stream);

/* Route + slots + gemm1 of a decode-sized MoE batch in one launch: the outputs of
 * w4a8_moe_route_slots (topk_w, topk_ids, sorted_ids, expert_ids, ntp, inv_pos; slots whose token
 * has no expert left to choose, NaN logits, get inv_pos -1 and a sentinel block) and of
 * w4a8_moe_gemm on them (decode arm, silu, gemm1 of x: out (P, N/2) at rows s*block_m), bit for
 * bit, without the per-token quant of x in memory. Fuses the reference's moe_hip.moe_route_align
 * (python/minisgl/quant/kernels.py:423-447) with the gemm1 of mmq_fp8_moe_gemm1_silu
 * (kernels.py:744-773) for the calls where w4a8_moe gives every slot a block of its own; the
 * router runs inside every workgroup of the GEMV. x: (T, K) bf16/fp16, 16-byte aligned rows.
 * Needs block_m < 64, T*top_k <= min(E, 64), T*top_k*block_m <= P, E <= 256 and the GEMV's fast
 * formats (int4 with groups of 128+, MXFP4, NVFP4), else kErrUnsupported (2): the caller then runs
 * w4a8_moe_route_slots and w4a8_moe_gemm. */
int w4a8_moe_route_gemm1(const void* logits, int logits_dtype, int64_t T, int64_t E, int top_k, int renormalize,
                         const void* x, int x_dtype, int64_t ldx, int block_m, int64_t P, const void* w_tile, int64_t N,
                         int64_t K, const void* scales, int scale_fmt, const int32_t* zeros, int wfmt,
                         int64_t group_size, float* topk_w, int32_t* topk_ids, int32_t* sorted_ids,
                         int32_t* expert_ids, int32_t* ntp, int32_t* inv_pos, void* out, int out_dtype, int64_t ldo,
                         void* stream);

/* RMSNorm producer with the per-token fp8 quant of its output as an epilogue. Replaces tail_hip's
 * rms_norm / rms_norm_add / rms_norm_quant / rms_norm_add_quant (python/minisgl/layers/norm.py:9-58,
 * 134-168): with residual non-NULL, residual <- x + residual (in place, in the activation dtype) and
 * the norm runs over that sum; out = dtype(dtype(v * rsqrt(mean(v^2) + eps)) * g), g = weight,
 * dtype(weight + 1) with plus_one, none with weight NULL. With x_fp8/act_scales non-NULL it also
 * writes the pair w4a8_act_quant(out) would give, bit for bit, for a w4a8 linear to consume. out may
 * be x; K <= 32768. */
int w4a8_rms_norm(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, void* residual, int64_t ldr,
                  const void* weight, int plus_one, float eps, void* out, int64_t ldo, uint8_t* x_fp8, int64_t ldq,
                  float* act_scales, void* stream);

/* Padded capacity numel + (E+1)*(block_m-1) of sorted_ids (python/minisgl/moe/fused.py:94). */
int64_t w4a8_moe_padded_capacity(int64_t numel, int64_t E, int block_m);

/* moe_align_block_size: replaces moe_hip.moe_align and the align half of moe_route_align
 * (python/minisgl/quant/kernels.py:686-695; contract python/minisgl/moe/fused.py:120-176).
 * Writes sorted_ids (P), expert_ids (ceil(P/block_m)), ntp (1) and, if non-NULL, inv_pos (numel):
 * the position of every slot in sorted_ids. Deterministic. */
int w4a8_moe_align(const int32_t* topk_ids, int64_t numel, int64_t E, int block_m, int64_t P, int32_t* sorted_ids,
                   int32_t* expert_ids, int32_t* ntp, int32_t* inv_pos, void* stream);

/* Workspace bytes w4a8_moe_gemm needs. */
int64_t w4a8_moe_gemm_workspace_bytes(int64_t numel, int64_t E, int block_m, int64_t P, int64_t N, int64_t K,
                                      int kernel);

/* Grouped W4A8 GEMM over align blocks. a_by_token = 1: row p reads A row sorted_ids[p]/top_k
 * (gemm1, with silu = 1 the fused gate/up epilogue of fp8_wmma.mmq_fp8_moe_gemm1_silu[_flag],
 * python/minisgl/quant/kernels.py:744-765); a_by_token = 0: row p reads A row p (gemm2,
 * fp8_wmma.mmq_fp8_moe_gemm[_flag], kernels.py:851-874). Rows at or past *ntp and padding slots
 * are skipped. kernel: 0 auto (block_m < 64 decode), 1 decode, 2 prefill (block_m % 64 == 0). */
int w4a8_moe_gemm(const uint8_t* a_fp8, int64_t lda, const float* a_scales, int a_by_token, const int32_t* sorted_ids,
                  const int32_t* expert_ids, const int32_t* ntp, int64_t numel, int top_k, int block_m, int64_t P,
                  const void* w_tile, int64_t E, int64_t N, int64_t K, const void* scales, int scale_fmt,
                  const int32_t* zeros, int wfmt, int64_t group_size, void* out, int out_dtype, int64_t ldo, int silu,
                  void* workspace, int64_t workspace_bytes, int kernel, void* stream);

/* Workspace bytes of w4a8_moe_gemm_quant: the codes of (P, K) rows (row-major, or in 16-row blocks of
 * the DMA GEMM's operand order with one row-sum seed per row and K tile) and P f32 row scales. */
int64_t w4a8_moe_gemm_quant_workspace_bytes(int64_t P, int64_t K);

/* gemm2 of the grouped FFN on the gemm1 buffer in its activation dtype, as the reference's prefill
 * gemm2 takes it (fp8_wmma.mmq_fp8_moe_gemm on the bf16/fp16 rows, python/minisgl/quant/kernels.py:
 * 851-874): a (P, K) bf16/fp16 at padded positions (row stride lda elements, 16-byte aligned) is
 * quantized per row as w4a8_act_quant does (rows at or past *ntp skipped) into the workspace, then
 * multiplied as w4a8_moe_gemm with a_by_token = 0 does; the outputs are those of that pair, bit for
 * bit. On the prefill arm with symmetric int4 weights (groups of 128+, K % 128 == 0, K >= 384) the
 * codes go straight into the DMA GEMM's operand order with their row-sum seeds. Two launches. */
int w4a8_moe_gemm_quant(const void* a, int a_dtype, int64_t lda, const int32_t* sorted_ids, const int32_t* expert_ids,
                        const int32_t* ntp, int64_t numel, int block_m, int64_t P, const void* w_tile, int64_t E,
                        int64_t N, int64_t K, const void* scales, int scale_fmt, const int32_t* zeros, int wfmt,
                        int64_t group_size, void* out, int out_dtype, int64_t ldo, void* workspace,
                        int64_t workspace_bytes, int kernel, void* stream);

/* Top-k weighted combine: out[t] = sum_j topk_w[t, j] * y[inv_pos[t*top_k + j]] in f32 over the slots
 * in order, cast to out_dtype. y rows are f32, or bf16/fp16 (y_dtype), as the reference's unfused gemm2
 * hands them over ((P, K) in the activation dtype, tools/vhip_patches/moe_experts.py:874-880). H and
 * ldy multiples of 4; y 16-byte (f32) or 8-byte aligned, out 8-byte (16-byte for f32) aligned.
 * Replaces fp8_wmma.mmq_fp8_moe_gather_reduce (python/minisgl/quant/kernels.py:876-882). */
int w4a8_moe_combine(const void* y, int y_dtype, int64_t ldy, const int32_t* inv_pos, const float* topk_w, int64_t T,
                     int top_k, int64_t H, void* out, int out_dtype, void* stream);

/* Gated tanh-GELU between the unfused gemm1 and gemm2 of the MoE FFN (experts declaring HF
 * gelu_pytorch_tanh): out[r, i] = gelu_tanh(y[r, i]) * y[r, inter + i] in f32, rounded once to the
 * dtype of y (bf16/fp16). Replaces the reference's torch gelu_tanh_and_mul that w4a8_moe runs on its
 * unfused gemm1 output (python/minisgl/layers/activation.py:47-64, python/minisgl/quant/kernels.py:
 * 777-783). y (rows, ldy >= 2*inter), out (rows, ldo >= inter); row_count: optional device int32
 * bounding the rows done (the align's ntp). */
int w4a8_moe_gelu_tanh_mul(const void* y, int dtype, int64_t ldy, int64_t rows, int64_t inter, void* out, int64_t ldo,
                           const int32_t* row_count, void* stream);

/* Fused gemm2 + top-k weighted combine of the MoE FFN for decode-sized batches: replaces
 * fp8_wmma.mmq_fp8_moe_gemm2_gather_reduce (python/minisgl/quant/kernels.py:831-850), one launch for
 * the per-row act quant of the gemm1 buffer, gemm2 and the combine. a: the gemm1 buffer (P, K)
 * bf16/fp16 at padded positions (row stride lda elements, 16-byte aligned); slot s = t*top_k + j of
 * token t reads row inv_pos[s] (inv_pos < 0: dropped slot) with expert topk_ids[s], quantized per
 * row as w4a8_act_quant does, bit for bit. out (T, N) = sum_j topk_w[t, j] * gemm2(row of slot
 * (t, j)) in f32 over the slots in order, cast to out_dtype, each slot's gemm2 row first rounded
 * to row_dtype (2 = f32: not rounded, as the reference's fused gemm2 + gather-reduce sums them;
 * 0/1: bf16/fp16, as its unfused gemm2 hands them over): the same bits as w4a8_act_quant +
 * w4a8_moe_gemm (decode arm, block_m, row_dtype out) + w4a8_moe_combine. Deterministic; no
 * workspace, no atomics.
 * Formats: int4 with groups of 128+, MXFP4 (E8M0) and NVFP4; K % 128 == 0, K <= 2048, top_k <= 16,
 * NVFP4 and zero-point int4 with K > 1024 only for top_k <= 8 (w4a8_moe_gemm2_combine_supported),
 * else kErrUnsupported (2). Revision 4 added row_dtype. */
int w4a8_moe_gemm2_combine_supported(int64_t K, int scale_fmt, int has_zeros, int wfmt, int64_t group_size, int top_k);
int w4a8_moe_gemm2_combine(const void* a, int a_dtype, int64_t lda, const int32_t* topk_ids, const float* topk_w,
                           const int32_t* inv_pos, int64_t T, int top_k, int block_m, int64_t P, const void* w_tile,
                           int64_t E, int64_t N, int64_t K, const void* scales, int scale_fmt, const int32_t* zeros,
                           int wfmt, int64_t group_size, void* out, int out_dtype, int64_t ldo, int row_dtype,
                           void* stream);

/* ---- W4A16: the same 4-bit weights against unquantized bf16/fp16 activations. */

/* Exact split of bf16/fp16 rows into fp8-e4m3 terms with power-of-two scales: row t of token m
 * (x_fp8 row T*m + t, T = 2 for bf16, 3 for fp16) holds e4m3(16^t r_t), scale 2^(E-4t), where
 * 2^E is the smallest power of two with max|x_m| / 2^E <= 448, r_0 = x / 2^E and
 * r_{t+1} = 16 r_t - e4m3(r_t); x = sum_t scale_t * code_t exactly for scaled magnitudes of at
 * least 2^-6. No counterpart in the reference (whose W4A16 kernels read x directly); it is the
 * activation side of w4a16_linear, exposed for testing and for callers that run the GEMM
 * themselves. x rows 16-byte aligned, K % 8 == 0; x_fp8 rows 8-byte aligned. */
int w4a16_act_split(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, uint8_t* x_fp8, int64_t ldq,
                    float* scales, void* stream);

/* Workspace of w4a16_linear: the split rows (T*M x K rounded to 16), their scales and the terms'
 * f32 GEMM rows (T*M x N); -1 on bad sizes. */
int64_t w4a16_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int x_dtype);

/* Dense W4A16 linear: y = x @ W^T with x never rounded (f32 accumulation), out in x's dtype, same
 * weights and scale formats as w4a8_gemm (int4 with fp16 group scales and optional zeros, e2m1 with
 * E8M0 or fp16 scales). silu != 0: the fused gate_up arm, out (M, N/2) = silu(gate) * up with gate
 * and up rounded to the dtype first. Replaces fp8_wmma.mmq_regdirect_w4a16_gemv /
 * mmq_w4a16_tiled / mmq_regdirect_w4a16_gemv_silu (python/minisgl/quant/kernels.py:1125-1178,
 * 1756-1786): the kernel arm follows M (decode GEMV up to 16 tokens, the tiled GEMM above), the
 * activations go through w4a16_act_split and the W4A8 GEMM, and one sum kernel adds each token's
 * terms in order and rounds once. */
int w4a16_linear(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, const void* w_tile, int64_t N,
                 const void* scales, int scale_fmt, const int32_t* zeros, int wfmt, int64_t group_size, void* out,
                 int64_t ldo, int silu, void* workspace, int64_t workspace_bytes, int kernel, void* stream);

/* Middle step of the grouped W4A16 MoE: replaces the silu_and_mul tail between
 * fp8_wmma.mmq_regdirect_w4a16_moe's two GEMMs (python/minisgl/quant/kernels.py:957-975) and feeds
 * gemm2 unquantized activations. The caller runs gemm1 (w4a8_moe_gemm, f32 out, no silu) over the
 * w4a16_act_split rows of x under a virtual route of Tt = 2 (bf16) or 3 (fp16) tokens per token:
 * virtual token Tt*m + t has token m's expert ids and reads split row Tt*m + t. y: that gemm1's
 * (P, 2*inter) f32 output (row stride ldy); inv_pos: its align's (T*Tt*top_k,) inverse positions.
 * For slot (m, j): gate|up = sum over t in order of y[inv_pos[(Tt*m + t)*top_k + j]], h =
 * silu(gate) * up rounded as the fused silu arms round (gate and up to the dtype, silu in f32,
 * rounded, times up, rounded), then h is split as w4a16_act_split splits a row, term t written to
 * row inv_pos[(Tt*m + t)*top_k + j] of a_fp8 with its scale in a_scales at that index, so gemm2
 * (w4a8_moe_gemm, a_by_token 0) over the same route reads the slot's terms by padded position.
 * h (optional, may be NULL): h at row m*top_k + j. Dropped slots (inv_pos < 0) are skipped.
 * inter % 8 == 0 and inter <= 32768; y 16-byte, a_fp8 8-byte, h 16-byte aligned rows. */
int w4a16_moe_silu_split(const float* y, int64_t ldy, const int32_t* inv_pos, int64_t T, int top_k, int64_t inter,
                         int dtype, uint8_t* a_fp8, int64_t lda, float* a_scales, void* h, int64_t ldh, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* W4A8_MI355X_H */

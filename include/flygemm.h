/* flygemm -- C ABI of the gfx950 (MI355X) quantized preshuffle GEMM library.
 *
 * Replaces, for the preshuffle GEMM path, the launch boundary the reference reaches through
 * its JIT: the JIT'd host entry `void entry(void** args)` that packs
 * (c, a, b, scale_a, scale_b, i32 M, i32 N, stream) and calls hipModuleLaunchKernel
 * (reference python/flydsl/compiler/jit_executor.py:105-121, jit_function.py:593-617,
 * lib/Runtime/FlyRocmRuntimeWrappers.cpp:58-67).
 *
 * Conventions shared by every entry point:
 *  - All pointers are device pointers the caller allocated.  Launches are asynchronous on
 *    `stream` (a hipStream_t, NULL = default stream).  Callers keep buffers alive until the
 *    stream has finished.  Nothing is allocated, freed or synchronized here, and every GEMM is
 *    one kernel launch (a K split over the waves of a workgroup is summed in LDS;
 *    flygemm_preshuffle_quant_a launches the quant kernel and then the GEMM), so every entry
 *    point may be captured into a HIP graph on any stream.
 *  - A is row-major [M][K] bytes.  B is the preshuffled [N][K] buffer produced by the
 *    reference's `shuffle_weight(b, layout=(16, 16))` (tests/utils.py:76-96): element
 *    (n, k) at byte (n/16)*16*K + (k/16)*256 + (n%16)*16 + (k%16).  INT4 B is that buffer
 *    packed two values per byte as in tests/kernels/test_preshuffle_gemm.py:165-174.
 *    bf16/fp16 B uses the same rule on each row's bytes (8 elements per 16-byte chunk), which
 *    is what shuffle_weight produces for 2-byte elements.
 *  - Requirements: N % 16 == 0, K % 64 == 0 (K % 32 == 0 for bf16/fp16: K tiles of 128 bytes, the
 *    last one 64 bytes when K * elem_bytes % 128 == 64; blockscale K % 128), M >= 0 (M == 0 is
 *    a no-op), every operand below 2^31 bytes.  Violations return nonzero without launching.
 *  - Return value: 0 on success, otherwise a hipError_t code; flygemm_last_error() gives
 *    the message of the calling thread's last failure.
 *  - `variant`: -1 picks the kernel from the built-in table; 0..flygemm_num_variants()-1
 *    forces one (for tests and tuning); every variant accepts every M.
 */
#ifndef FLYGEMM_H
#define FLYGEMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FLYGEMM_IN_FP8 = 0,  /* OCP e4m3fn (torch.float8_e4m3fn) */
  FLYGEMM_IN_INT8 = 1, /* int8 A and B */
  FLYGEMM_IN_INT4 = 2, /* int8 A, packed signed int4 B */
  FLYGEMM_IN_BF16 = 3, /* bf16 A and B, no scaling (scale pointers ignored) */
  FLYGEMM_IN_FP16 = 4, /* fp16 A and B, no scaling (scale pointers ignored) */
  FLYGEMM_IN_FP4 = 5,  /* MXFP4: flygemm_mxfp4 only (and flygemm_select_variant) */
  FLYGEMM_IN_INT4_BF16 = 6,  /* MoE only: bf16 activations, packed int4 weights (W4A16) */
  FLYGEMM_IN_INT8_SMOOTH = 7 /* MoE only: int8, stage-1 activations per route, slot-major */
};
enum { FLYGEMM_OUT_BF16 = 0, FLYGEMM_OUT_FP16 = 1, FLYGEMM_OUT_F32 = 2 /* flygemm_mxfp4 only */ };

/* C[M][N] = out_dtype((acc[m][n] * scale_a[m]) * scale_b[n]),
 * acc = sum_k A[m][k] * B[n][k] in fp32 (fp8, bf16, fp16) or int32 (int8/int4);
 * bf16/fp16 inputs are not scaled: C = out_dtype(acc) (reference preshuffle_gemm.py:804-806).
 * scale_a: fp32 [M] per token; scale_b: fp32 [N] per output channel.
 * int4 weights take K < 131072 (here, in flygemm_accumulators and flygemm_preshuffle_quant_a).
 * Replaces the launcher returned by compile_preshuffle_gemm_a8
 * (reference kernels/preshuffle_gemm.py:39-57, launch_gemm :1268-1301; epilogue :863-883). */
int flygemm_preshuffle(void* c, const void* a, const void* b, const float* scale_a, const float* scale_b,
                       int32_t M, int32_t N, int32_t K, int32_t in_dtype, int32_t out_dtype,
                       int32_t variant, void* stream);

/* FP8 blockscale GEMM: C[m][n] = out_dtype(sum_kb (sum_{k in kb} A*B) * x_scale_t[kb][m]
 *                                                 * w_scale[n/128][kb]),
 * x_scale_t: fp32 [K/128][M] (K-block major), w_scale: fp32 [ceil(N/128)][K/128].
 * scale_block_k must be 128.  Replaces the launcher of compile_blockscale_preshuffle_gemm,
 * whose contract is its call site tests/kernels/test_blockscale_preshuffle_gemm.py:173-204
 * and oracle :86-109 (the kernel source is absent from the reference snapshot). */
int flygemm_blockscale(void* c, const void* a, const void* b, const float* x_scale_t, const float* w_scale,
                       int32_t M, int32_t N, int32_t K, int32_t scale_block_k, int32_t out_dtype,
                       int32_t variant, void* stream);

/* Raw accumulators, no scaling: int32 [M][N] for int8/int4, fp32 [M][N] for fp8/bf16/fp16.
 * Exposes the value the reference's kernels hold before their epilogue
 * (kernels/preshuffle_gemm.py:643-797) so integer paths can be checked bit-exactly. */
int flygemm_accumulators(void* acc, const void* a, const void* b, int32_t M, int32_t N, int32_t K,
                         int32_t in_dtype, int32_t variant, void* stream);

/* MXFP4 GEMM: C[m][n] = out_dtype(sum_k a[m][k] * sa[m][k/32] * b[n][k] * sb[n][k/32]),
 * fp32 accumulation; a, b OCP e2m1 (two per byte, element 2j in the low nibble), sa, sb E8M0.
 * a: row-major [M][K/2] bytes.  b: [N][K/2] bytes after the reference's
 * shuffle_weight_w4(b, 16, False, False) (tests/kernels/utils/fp4_utils.py:578-621), which
 * is the 1-byte preshuffle rule on rows of K/2 bytes.  scale_a / scale_b: E8M0 bytes
 * [round_up(M, 32)][K/32] / [N][K/32] after shuffle_scale_w4(s, 1, False) (:624-653).
 * K % 256 == 0, N % 32 == 0.  out_dtype bf16, fp16 or fp32.  A forced variant of 64x64
 * tiles is rejected (its 16-column wave tiles would split a 32-column scale group; the
 * library's own choice never takes it for MXFP4).  Replaces the launcher of
 * compile_preshuffle_gemm_w4 (reference kernels/preshuffle_gemm.py:1306-1337, MFMA use
 * :692-732; harness tests/kernels/test_preshuffle_gemm.py:261-379). */
int flygemm_mxfp4(void* c, const void* a, const void* b, const void* scale_a, const void* scale_b, int32_t M,
                  int32_t N, int32_t K, int32_t out_dtype, int32_t variant, void* stream);

/* Per-row (per-token) quantization of activations, the producer of A and scale_a:
 *   scale[m] = max_n |in[m][n]| / qmax (qmax 127 int8, 448 fp8), 1 where that is 0;
 *   out[m][n] = cast(in[m][n] / scale[m]), or cast(in[m][n] * (1 / scale[m])).
 * mode FLYGEMM_QMODE_RECIP_TRUNC: the reference's device kernel
 *   (tests/kernels/test_quant.py:81-265: fp16 in, int8 out, fptosi of the product with the
 *   reciprocal); inputs must be finite.
 * mode FLYGEMM_QMODE_DIV_TRUNC / _DIV_NEAREST: the reference's pertoken_quant
 *   (tests/utils.py:29-73): NaN -> 0, +-inf -> +-qmax, then the quotient is cast, truncating
 *   (int8, as torch's .to(int8)) or rounding half to even (int8 clamped to +-127; fp8
 *   e4m3fn always uses _DIV_NEAREST, like torch's cast).
 * in: [M][N] fp16/bf16/fp32 (16-byte aligned), out: [M][N] bytes (8-byte aligned),
 * scales: fp32 [M].  N % 8 == 0.  Nothing is allocated; asynchronous on `stream`. */
enum { FLYGEMM_QIN_F16 = 0, FLYGEMM_QIN_BF16 = 1, FLYGEMM_QIN_F32 = 2 };
enum { FLYGEMM_QOUT_FP8 = 0, FLYGEMM_QOUT_INT8 = 1 };
enum { FLYGEMM_QMODE_RECIP_TRUNC = 0, FLYGEMM_QMODE_DIV_TRUNC = 1, FLYGEMM_QMODE_DIV_NEAREST = 2 };
int flygemm_quant_rows(void* out, float* scales, const void* in, int32_t M, int32_t N, int32_t in_dtype,
                       int32_t out_dtype, int32_t mode, void* stream);

/* The GEMM of activations quantized per row on the way in, in one call:
 *   flygemm_quant_rows(a_q, scale_a, x, M, K, x_dtype, fp8 or int8 codes, mode), then
 *   flygemm_preshuffle(c, a_q, b, scale_a, scale_b, M, N, K, in_dtype, out_dtype, variant)
 * on `stream` (the quant kernel of tests/kernels/test_quant.py:81-265 or pertoken_quant of
 * tests/utils.py:29-73, then the launcher of kernels/preshuffle_gemm.py:1268-1301).  x: [M][K]
 * FLYGEMM_QIN_* activations, 16-byte aligned; in_dtype FLYGEMM_IN_FP8 (mode must be
 * _DIV_NEAREST), _INT8 or _INT4 (int8 codes); mode and scale_b as for those entries; a_q [M][K]
 * (8-byte aligned) and scale_a [M] receive the codes and the row scales and are required.
 * No allocation; asynchronous on `stream`.  Every check runs before the first launch. */
int flygemm_preshuffle_quant_a(void* c, void* a_q, float* scale_a, const void* x, const void* b, const float* scale_b,
                               int32_t M, int32_t N, int32_t K, int32_t x_dtype, int32_t in_dtype, int32_t mode,
                               int32_t out_dtype, int32_t variant, void* stream);

/* MoE 2-stage GEMM over routing metadata sorted by expert (the reference's moe_sorting,
 * tests/kernels/test_moe_gemm.py:97-162):
 *   sorted_token_ids int32 [>= num_valid_ids[0]]: (slot << 24) | token, each expert's run
 *     padded to a multiple of tile_m with entries whose token is >= tokens;
 *   sorted_expert_ids int32 [size_expert_ids]: the expert of each tile_m-row block (-1: none);
 *   sorted_weights fp32, aligned with sorted_token_ids (read only when doweight != 0);
 *   num_valid_ids int32 [1]: padded row count; blocks at or past it do nothing.
 * in_dtype (the reference's in_dtype strings, kernels/moe_gemm_2stage.py:110-121):
 *   FLYGEMM_IN_FP8 / _INT8: per-token scale_x, per-row scale_w;
 *   FLYGEMM_IN_INT8_SMOOTH ("int8smooth"): int8 whose stage-1 activations are given per route,
 *     x [topk*tokens][model_dim] with row s*tokens + t (slot-major) and scale_x [topk*tokens] in
 *     the same order; stage 2 is plain int8;
 *   FLYGEMM_IN_INT4 ("int4", W4A8): int8 activations, weights packed two int4 per byte exactly as
 *     the dense int4 B (the preshuffled int8 bytes, then packed), per-row scale_w; K < 131072;
 *   FLYGEMM_IN_INT4_BF16 ("int4_bf16", W4A16): bf16 activations (no scale_x), the same packed int4
 *     weights, converted to bf16 in registers; scale_w per weight row when group_size <= 0, or
 *     group scales [experts][K/32][rows of the expert's weight] (w[n][k] * scale[e][k/32][n],
 *     tests/kernels/test_ref.py:44-50,117-123) when group_size == 32;
 *   FLYGEMM_IN_BF16 / _FP16: unscaled (scale pointers ignored).
 * group_size: -1 (or 0) for per-row weight scales; 32 only with FLYGEMM_IN_INT4_BF16.
 * Weights preshuffled as B everywhere here.
 * tile_m (16, 32, 64) is the routing block size the metadata was built with; tile_n (64, 128,
 * 256, or 0 to choose) must divide the output width.  K % 128 == 0 (K % 64 for 16-bit).
 *
 * Stage 1: out [tokens][topk][inter_dim] (fp16 or bf16) =
 *   silu((x[t].W1[e*2I+n]) * sx[t] * sw[e*2I+n]) * ((x[t].W1[e*2I+I+n]) * sx[t] * sw[e*2I+I+n])
 *   (* sorted_weights if doweight_stage1); x [tokens][model_dim], W1 [experts*2*inter_dim]
 *   [model_dim], scale_x [tokens], scale_w [experts*2*inter_dim].  Rows no route writes are
 *   left untouched.  Replaces the launcher of compile_moe_gemm1
 *   (reference kernels/moe_gemm_2stage.py:93-1264; oracle tests/kernels/test_ref.py:7-75). */
int flygemm_moe_gemm1(void* out, const void* x, const void* w, const float* scale_x, const float* scale_w,
                      const int32_t* sorted_token_ids, const int32_t* sorted_expert_ids, const float* sorted_weights,
                      const int32_t* num_valid_ids, int32_t tokens, int32_t inter_dim, int32_t model_dim,
                      int32_t size_expert_ids, int32_t experts, int32_t topk, int32_t tile_m, int32_t tile_n,
                      int32_t in_dtype, int32_t out_dtype, int32_t doweight_stage1, int32_t group_size,
                      void* stream);

/* Stage 2, per route r = (t, s) of expert e: y_r[n] = (a2[t*topk+s].W2[e*D+n]) * sa[t*topk+s]
 *   * sw[e*D+n] (* sorted_weights if doweight_stage2); a2 [tokens*topk][inter_dim], W2
 *   [experts*model_dim][inter_dim], scale_a2 [tokens*topk], scale_w [experts*model_dim].
 *   accumulate != 0: out [tokens][model_dim] += sum over the token's routes, with device atomics
 *     (the caller zeroes `out` first; the order of the additions is unspecified); out_dtype
 *     fp16, bf16 or fp32.
 *   accumulate == 0: out [tokens*topk][model_dim] row t*topk+s = y_r, plain stores (rows no
 *     route writes are left untouched); out_dtype fp16 or bf16; flygemm_moe_reduce sums them.
 *   Replaces the launcher of compile_moe_gemm2(accumulate=True/False)
 *   (reference kernels/moe_gemm_2stage.py:1267-2481; oracle tests/kernels/test_ref.py:78-141). */
int flygemm_moe_gemm2(void* out, const void* a2, const void* w, const float* scale_a2, const float* scale_w,
                      const int32_t* sorted_token_ids, const int32_t* sorted_expert_ids, const float* sorted_weights,
                      const int32_t* num_valid_ids, int32_t tokens, int32_t model_dim, int32_t inter_dim,
                      int32_t size_expert_ids, int32_t experts, int32_t topk, int32_t tile_m, int32_t tile_n,
                      int32_t in_dtype, int32_t out_dtype, int32_t doweight_stage2, int32_t accumulate,
                      int32_t group_size, void* stream);

/* Blockscale MoE (fp8, per-block scales, ScaleBlockM = 1, N = K = 128): each 128-deep K block's
 * partial product is scaled before it is accumulated,
 *   acc[r][n] = sum_kb (sum_{k in kb} a[r][k] * w[n][k]) * a_scale_t[kb][r] * w_scale[n/128][kb],
 * with r the A row (stage 1: token t; stage 2: t*topk + s) and n the weight row of the expert
 * slab (e*2I + n / e*2I + I + n in stage 1, e*D + n in stage 2).  a_scale_t fp32 [K/128][rows of
 * A] (K-block major); w_scale fp32 [rows of W / 128][K/128].  Then stage 1: out = silu(gate) * up
 * (* sorted_weights if doweight); stage 2 as flygemm_moe_gemm2 (atomic or per-route rows).
 * scale_block_k must be 128; 2*inter_dim (stage 1) / model_dim (stage 2) a multiple of 128.
 * Replaces the launchers of compile_moe_blockscale_gemm1 / _gemm2 (reference
 * kernels/moe_blockscale_2stage.py:75-1217, :1220-2445; oracle
 * tests/kernels/test_moe_blockscale.py:64-133). */
int flygemm_moe_blockscale_gemm1(void* out, const void* x, const void* w, const float* x_scale_t,
                                 const float* w_scale, const int32_t* sorted_token_ids,
                                 const int32_t* sorted_expert_ids, const float* sorted_weights,
                                 const int32_t* num_valid_ids, int32_t tokens, int32_t inter_dim, int32_t model_dim,
                                 int32_t size_expert_ids, int32_t experts, int32_t topk, int32_t tile_m,
                                 int32_t tile_n, int32_t scale_block_k, int32_t out_dtype, int32_t doweight_stage1,
                                 void* stream);
int flygemm_moe_blockscale_gemm2(void* out, const void* a2, const void* w, const float* a2_scale_t,
                                 const float* w_scale, const int32_t* sorted_token_ids,
                                 const int32_t* sorted_expert_ids, const float* sorted_weights,
                                 const int32_t* num_valid_ids, int32_t tokens, int32_t model_dim, int32_t inter_dim,
                                 int32_t size_expert_ids, int32_t experts, int32_t topk, int32_t tile_m,
                                 int32_t tile_n, int32_t scale_block_k, int32_t out_dtype, int32_t doweight_stage2,
                                 int32_t accumulate, void* stream);

/* The MoE launchers' tile choice for a call with these sizes (they treat tile_n as a hint):
 * *runs = routing blocks per workgroup (1: single-block tiles; more: runs of 128 rows in stage
 * 1, 256 in stage 2, and 256 in stage 1 of routings with large experts, blockscale included) and *tile_n_out =
 * output columns per tile.  Stage 2 values are those of accumulating calls; per-route-row calls
 * (accumulate = 0) of 1-byte, int4 (int8 activations) and 16-bit weights with inter_dim of 1, 2
 * or 4 128-byte K steps run 64-column tiles instead: single routing blocks (two for tile_m 16)
 * with 1 to 32 routes per expert on average, 128-row runs from 128 routes per expert (int4: 256;
 * from 32 for tile_m 16).  n is the GEMM's output width and k its depth (stage 1: inter_dim and
 * model_dim; stage 2: model_dim and inter_dim); in_dtype as for flygemm_moe_gemm1/2; blockscale
 * != 0 for the blockscale MoE.  Validates like the launchers; touches no device.  Counterpart of
 * the reference's compile-time tile arguments (kernels/moe_gemm_2stage.py:93-121), for tests and
 * tuning, like flygemm_select_variant. */
int flygemm_moe_select_tile(int32_t stage, int32_t tokens, int32_t n, int32_t k, int32_t experts, int32_t topk,
                            int32_t tile_m, int32_t tile_n, int32_t in_dtype, int32_t blockscale, int32_t* runs,
                            int32_t* tile_n_out);

/* Reduce mode, second step: y [tokens][model_dim] = sum over k < topk of x [tokens][topk]
 * [model_dim] (only slots with valid_mask[t*topk+k] != 0 when valid_mask, int8 [tokens*topk], is
 * given), fp32 sums; dtype fp16, bf16 or fp32 for both x and y; model_dim a multiple of 8 (4 for
 * fp32); x and y 16-byte aligned.  Replaces the launcher of compile_moe_reduction (reference
 * kernels/moe_gemm_2stage.py:2484-2604). */
int flygemm_moe_reduce(void* y, const void* x, const void* valid_mask, int32_t tokens, int32_t topk,
                       int32_t model_dim, int32_t dtype, void* stream);

/* Stage 2 in reduce mode in one call that allocates nothing: flygemm_moe_gemm2 with
 * accumulate = 0 into per-route rows [tokens*topk][model_dim] (fp16 or bf16), zeroed first when
 * zero_intermediate != 0 and valid_mask is NULL, then flygemm_moe_reduce of those rows into out
 * [tokens][model_dim]; the arguments mean what they mean there, and out equals what those two
 * calls give.  No counterpart in the reference: it is for callers that cannot allocate (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc), where the
 * reference's reduce mode takes its rows from torch's allocator.  The rows live in a static
 * device array of FLYGEMM_MOE_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends);
 * larger tokens*topk*model_dim*2 is rejected.  Every call on one GPU shares that array: calls
 * that overlap on one GPU (other streams, other threads) race.  The first call on each device
 * resolves the array's address and must not run under graph capture. */
#define FLYGEMM_MOE_NOALLOC_SCRATCH_BYTES (64L << 20)
int flygemm_moe_gemm2_reduce_noalloc(void* out, const void* a2, const void* w, const float* scale_a2,
                                     const float* scale_w, const int32_t* sorted_token_ids,
                                     const int32_t* sorted_expert_ids, const float* sorted_weights,
                                     const int32_t* num_valid_ids, int32_t tokens, int32_t model_dim,
                                     int32_t inter_dim, int32_t size_expert_ids, int32_t experts, int32_t topk,
                                     int32_t tile_m, int32_t tile_n, int32_t in_dtype, int32_t out_dtype,
                                     int32_t doweight_stage2, int32_t group_size, const void* valid_mask,
                                     int32_t zero_intermediate, void* stream);

/* Kernel variant table (replaces the reference's per-call tile kwargs,
 * kernels/preshuffle_gemm.py:39-53, with a static table). */
int32_t flygemm_num_variants(void);
const char* flygemm_variant_name(int32_t variant);
int32_t flygemm_select_variant(int32_t M, int32_t N, int32_t K, int32_t in_dtype, int32_t blockscale);

/* The launch that flygemm_preshuffle (blockscale == 0), flygemm_blockscale (blockscale != 0) or
 * flygemm_mxfp4 (in_dtype FLYGEMM_IN_FP4) would make for these sizes and variant (-1: the
 * table's choice), on the current device: the variant index, the workgroup count, threads per
 * workgroup and the work items the grid walks (output tiles for the large-M kernel, which is
 * persistent: one workgroup takes tiles w, w + grid, ...; workgroups for the others, one item
 * each).  K counts elements as in those entry points.  Launches nothing; it queries the
 * device's CU count and occupancy.  Counterpart of the grid the reference's launcher computes
 * (kernels/preshuffle_gemm.py:1268-1301), for tests and tuning. */
int flygemm_launch_shape(int32_t M, int32_t N, int32_t K, int32_t in_dtype, int32_t blockscale, int32_t variant,
                         int32_t* variant_out, int32_t* grid, int32_t* threads, int32_t* items);

/* Message of the calling thread's last failure ("" if none).  The reference prints HIP
 * errors instead of returning them (lib/Runtime/FlyRocmRuntimeWrappers.cpp:22-30). */
const char* flygemm_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* FLYGEMM_H */

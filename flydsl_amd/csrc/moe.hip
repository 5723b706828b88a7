// C-ABI of the MoE 2-stage GEMM (declarations: include/flygemm.h).  Host-side validation,
// tile dispatch and launch; the kernels are in moe.h.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>

#include "../../include/flygemm.h"
#include "abi_error.h"
#include "moe.h"

using namespace flygemm;

// Kernel tables (stage 2 lives in moe_stage2.hip and the stage-1 stream kernel of 1-byte,
// 16-bit and W4A8 weights in moe_stream.hip, compiled in parallel).  Here: stage 1 of W4A16 and
// of blockscale fp8 -- runs of one routing block (R = 1, 4 waves) for every (tile_m, tile_n).
namespace flygemm {
MoeKernel moe_stage2_kernel(int kind, int tm, int r, int tn, bool f32, bool bs);
MoeKernel moe_stage1_stream_kernel(int kind, int tm);
MoeKernel moe_stage2_stream_kernel(int kind, int tm, int nk, bool single);
}

namespace {

template <int KIND, bool BS>
MoeKernel moe_stage1_tile(int tm, int r, int tn) {
#define T(M_, R_, N_, WM_, WN_)        \
  if (tm == M_ && r == R_ && tn == N_) \
    return MoeKernel{moe_gemm_kernel<1, KIND, M_, R_, N_, WM_, WN_, false, BS>, WM_ * WN_ * 64};
  // (64 or 128 columns: the launcher never takes 256 for these single-block stage-1 tiles)
  T(16, 1, 64, 1, 4) T(16, 1, 128, 1, 4) T(32, 1, 64, 1, 4) T(32, 1, 128, 1, 4) T(64, 1, 64, 1, 4) T(64, 1, 128, 1, 4)
  // runs of 256 rows (four 64-row, eight 32-row or sixteen 16-row blocks), 128 columns (128 gate
  // + 128 up weight rows): routings with large experts (see moe_tiles)
  if constexpr (!BS && moe_big_kind(KIND)) {
    T(64, 4, 128, 2, 4) T(32, 8, 128, 2, 4) T(16, 16, 128, 2, 4)
  }
  if constexpr (KIND == KIND_W4A16) {
    T(64, 4, 128, 2, 4) T(32, 8, 128, 2, 4)
  }
  // blockscale with 16-row blocks: runs of 256 rows, 64 columns (see moe_tiles)
  if constexpr (BS) {
    T(16, 16, 64, 2, 4)
  }
#undef T
  return MoeKernel{nullptr, 0};
}

// Stage 1 of fp8, int8 (int8smooth included), int4 weights with int8 activations (W4A8), bf16
// and fp16 runs the stream kernel (moe_stream.h) for every routing but large experts (moe_tiles): DS-TP8 dims (128 experts, model_dim 7168, inter_dim 256),
// fp8, graph-timed against the kernels it replaced (64-column single-block tiles for 64-row
// blocks, 128-row run tiles with weights in LDS for 16- and 32-row blocks), bit-equal outputs:
// 64-row blocks 2048 / 4096 / 8192 / 16384 tokens 134 / 181 / 298 / 527 us against 160 / 216 /
// 424 / 722; 32-row 146 / 198 / 307 / 528 against 164 / 264 / 518 / 1728; 16-row 146 / 200 / 313
// / 549 against 211 / 313 / 525 / 1743; decode-sized routings (16 to 1024 tokens) level or up
// to 10% faster.
bool moe_stream_stage1(int stage, int kind, bool bs) {
  return stage == 1 && !bs &&
         (kind == KIND_FP8 || kind == KIND_INT8 || kind == KIND_INT4 || kind == KIND_BF16 || kind == KIND_F16);
}

MoeKernel moe_stage1_kernel(int kind, int tm, int r, int tn, bool bs) {
  if (bs) return kind == KIND_FP8 ? moe_stage1_tile<KIND_FP8, true>(tm, r, tn) : MoeKernel{nullptr, 0};
  if (r * tm == 256 && !bs) {
    switch (kind) {
      case KIND_FP8: return moe_stage1_tile<KIND_FP8, false>(tm, r, tn);
      case KIND_INT8: return moe_stage1_tile<KIND_INT8, false>(tm, r, tn);
      case KIND_BF16: return moe_stage1_tile<KIND_BF16, false>(tm, r, tn);
      case KIND_F16: return moe_stage1_tile<KIND_F16, false>(tm, r, tn);
      case KIND_INT4: return moe_stage1_tile<KIND_INT4, false>(tm, r, tn);
      case KIND_W4A16: return moe_stage1_tile<KIND_W4A16, false>(tm, r, tn);
      default: return MoeKernel{nullptr, 0};
    }
  }
  if (moe_stream_stage1(1, kind, bs))
    return r * tm == 128 && tn == 64 ? moe_stage1_stream_kernel(kind, tm) : MoeKernel{nullptr, 0};
  return kind == KIND_W4A16 ? moe_stage1_tile<KIND_W4A16, false>(tm, r, tn) : MoeKernel{nullptr, 0};
}

// Estimated runs (workgroups before column splitting): routing blocks grouped R at a time, plus
// one partial run per expert that has routes.
long est_runs(int tokens, int topk, int experts, int tm, int r) {
  const long routes = (long)tokens * topk;
  return routes / ((long)tm * r) + (routes < experts ? routes : experts);
}

// Column tile when the caller leaves it open (tile_n <= 0): the widest of 256/128/64 that
// divides N and still gives about two workgroups per CU.
int pick_tile_n(int N, long runs) {
  for (int tn : {256, 128})
    if (N % tn == 0 && runs * (N / tn) >= 512) return tn;
  return 64;
}

// Tile of a call: runs of R routing blocks per workgroup and tile_n output columns (the
// caller's tile_n, already validated, is a hint).  atomics: a stage-2 call that accumulates
// (per-route-row calls take the stream kernel's tiles where it applies).
int moe_tiles(int stage, int tokens, int N, int K, int experts, int topk, int tile_m, int tile_n, int kind, bool bs,
              bool atomics, const char* what, int* r_out, int* tn_out, bool wgroup = false) {
  const long routes = (long)tokens * topk;
  const int inter = stage == 1 ? N : K;
  // Blockscale on large experts (inter_dim of at least 1024): runs of 256 rows, 128 columns in
  // stage 2 (16- and 32-row blocks from 128 routes per expert, 64-row blocks from 512) and 64 in
  // stage 1 (16-row blocks only).  Graph-timed, DS-V3 prefill dims (7168 x 2048, 256 experts,
  // top-8), single-block tiles against runs (µs): 16-row blocks, 16384 tokens stage 1 15736 ->
  // 13737, stage 2 17192 -> 6105; 4096 tokens 4868 -> 4067 / 4495 -> 2036; 32-row blocks stage 2
  // 8812 -> 5908 at 16384 tokens, 2453 -> 2032 at 4096, slower at 2048 (1386 -> 1713); 64-row
  // blocks stage 2 7054 -> 5748 at 16384 tokens, level at 4096 (2032 / 2012); stage 1 slower on
  // runs for 32- and 64-row blocks (9239 -> 12862), as is inter_dim 256 (8192 tokens, 16-row
  // blocks, stage 2 909 -> 1196).
  if (bs && inter >= 1024) {
    if (stage == 2 && N % 128 == 0 &&
        (tile_m == 64 ? routes >= 512L * experts : routes >= 128L * experts)) {
      *r_out = 256 / tile_m;
      *tn_out = 128;
      return 0;
    }
    if (stage == 1 && tile_m == 16 && routes >= 128L * experts && N % 64 == 0) {
      *r_out = 16;
      *tn_out = 64;
      return 0;
    }
  }
  // Large experts (fp8, int8, bf16, fp16, int4; inter_dim of at least 1024, at least 512 routes per
  // expert on average; stage 1 with model_dim of at least 4096): runs of 256 rows (four 64-row,
  // eight 32-row or sixteen 16-row blocks)
  // on 2 x 4 waves with both operands staged through LDS -- 128 output columns in stage 1 (128
  // gate + 128 up weight rows), 256 in stage 2 -- the bytes per flop of the dense kernel's large
  // tiles, where the stream kernel's 128 x 64 tiles (stage 1) and single-block tiles (stage 2)
  // move two to four times as many.  Graph-timed on MI355X (µs, stage 1 / stage 2 with atomics,
  // former choice against runs): the reference's benchmark shape 32768 tokens, 8192 x 8192, 16
  // experts, top-4: 29190 -> 18376 / 25441 -> 8885; the same at 4096 tokens 3538 -> 2477 / 3119
  // -> 1276; 8192 tokens, 4096 x 14336, 8 experts, top-2: 2931 -> 2015 / 2405 -> 1306, at 2048
  // tokens 906 -> 709 / 582 -> 391; 8192 tokens, 4096 x 1536, 64 experts, top-8: 972 -> 851 / 910
  // -> 747; 16384 tokens, 7168 x 2048, 256 experts, top-8: 5393 -> 4419 / 4562 -> 3060.  Not for
  // DS-TP8 (inter_dim 256: 289 -> 336 / 731 -> 838) nor inter_dim 768 (270 -> 270 / 282 -> 324).
  // int8, bf16 and fp16 alike (8192 tokens, 4096 x 14336, 8 experts, top-2: int8 3089 -> 2013 /
  // 2496 -> 1311, bf16 6574 -> 4106 / 5592 -> 2711; 4096 tokens, 8192 x 8192, 16 experts, top-4:
  // bf16 7303 -> 4782 / 6984 -> 2494; stage-1 outputs bit-equal), and 32- / 16-row blocks too
  // (8192 tokens, 4096 x 14336, 8 experts, top-2, fp8: 32-row 3000 -> 2007 / 4920 -> 1199, 16-row
  // stage 1 3117 -> 2195, its stage 2 already on runs; bf16 32-row 4096 tokens, 8192 x 8192, 16
  // experts, top-4: 7313 -> 5109 / 12150 -> 2549).  int4 (W4A8), whose weights move half the
  // bytes, from inter_dim 4096 (4096 tokens, 8192 x 8192, 16 experts, top-4: 2353 -> 1935 / 1769
  // -> 1085; 8192 tokens, 4096 x 14336: 2062 -> 1787 / 1371 -> 1168; at 4096 x 1536, 64 experts:
  // 765 -> 744 / 671 -> 731).  Not W4A16 (its group scales ride the two-slot pipeline) nor
  // blockscale.
  // With inter_dim of at least 4096 (not int4) from 256 routes per expert already (1024 tokens,
  // 4096 x 14336, 8 experts, top-2: 485 -> 361 / 358 -> 199; 1024 tokens, 8192 x 8192, 16
  // experts, top-4: 1148 -> 906 / 816 -> 478), not at 1536 (2048 tokens, 64 experts, top-8, stage
  // 2 256 -> 265) nor with fewer routes (128 per expert, 4096 x 1536: 198 -> 216 / 155 -> 210).
  const bool big = kind == KIND_INT4 ? inter >= 4096 && routes >= 512L * experts
                                     : (inter >= 1024 && routes >= 512L * experts) ||
                                           (inter >= 4096 && routes >= 256L * experts);
  // W4A16 with per-row weight scales (no group scales, which ride the two-slot pipeline) takes
  // them as bf16 does, for 32- and 64-row blocks (4096 tokens, 8192 x 8192, 16 experts, top-4:
  // 6994 -> 5431 / 3271 -> 2392; 8192 tokens, 4096 x 14336, 8 experts, top-2: 6213 -> 4603 / 2780
  // -> 2815).
  const bool w4a16_runs = kind == KIND_W4A16 && !wgroup && tile_m >= 32 &&
                          ((inter >= 1024 && routes >= 512L * experts) || (inter >= 4096 && routes >= 256L * experts));
  if ((moe_big_kind(kind) && !bs && big) || w4a16_runs) {
    if (stage == 1 && K >= 4096 && N % 128 == 0) {
      *r_out = 256 / tile_m;
      *tn_out = 128;
      return 0;
    }
    if (stage == 2 && N % 256 == 0) {
      *r_out = 256 / tile_m;
      *tn_out = 256;
      return 0;
    }
  }
  // Stage 1 of 1-byte, 16-bit and W4A8 weights: the stream kernel, 128-row runs of 64 columns
  // (every N here is a multiple of 64: tile_n, checked by the callers, divides it).  The
  // caller's tile_n is a hint throughout: tiling does not change results.
  if (moe_stream_stage1(stage, kind, bs)) {
    *r_out = 128 / tile_m;
    *tn_out = 64;
    return 0;
  }
  // Stage 2 of 16-row blocks: runs of 256 rows x 256 columns on 2 x 4 waves when experts hold two
  // or more blocks on average.  Not for blockscale nor W4A16 (their scales do not fit next to the
  // run tiles); stage 1 of those two kinds uses single-block tiles.
  // Stage 2 of 32- and 64-row blocks keeps single-block tiles (128 columns, below): with three
  // workgroups per CU their epilogues and row stores overlap each other's MFMAs.  DS-TP8 dims
  // (128 experts, model_dim 7168, inter_dim 256), fp8, graph-timed: 64-row blocks, reduce mode
  // 2048 / 4096 / 8192 / 16384 tokens 167 / 296 / 610 / 1153 us against 247 / 363 / 711 / 1508
  // for 256-row runs, atomics 270 / 435 / 846 / 1539 against 341 / 457 / 937 / 2167; 32-row
  // blocks reduce 189 / 381 / 702 / 1369 against 277 / 374 / 723 / 1512, atomics 254 / 502 /
  // 835 / 1701 against 385 / 454 / 991 / 2185.  16-row blocks keep the runs (reduce mode 1.0-1.3x
  // slower single-block from 4096 tokens).
  int R = 1;
  if (stage == 2 && tile_m == 16 && !bs && kind != KIND_W4A16 && routes >= 2L * tile_m * experts && N % 256 == 0 &&
      tile_n != 64) {
    R = 256 / tile_m;
    tile_n = 256;
  }
  if (tile_n <= 0) tile_n = pick_tile_n(N, est_runs(tokens, topk, experts, tile_m, R));
  // Few runs (decode): narrower column tiles until there are workgroups for every CU (each
  // workgroup streams its own weight columns, so parallelism is bandwidth here).
  if (R == 1 && (tile_n == 128 || tile_n == 256)) {
    const long runs1 = est_runs(tokens, topk, experts, tile_m, 1);
    while (tile_n > 64 && runs1 * (N / tile_n) < 256 && N % (tile_n / 2) == 0) tile_n /= 2;
    // decode-sized routings (stage 2 up to 512 routes, stage 1 up to 256): 64-column tiles,
    // whose short weight streams finish together (DS-V3 dims, top-8: stage 2 at 8 tokens 19.8
    // µs against 27.2 with 256 columns, at 32 tokens 71.8 against 76.6; stage 1 at 32 tokens
    // 101 against 115; from 128 tokens on the wider tiles are within +-7%)
    if (routes <= (stage == 2 ? 512 : 256) && N % 64 == 0) tile_n = 64;
    // stage 2 with more routes but still single-block tiles: 128 columns (1024-2048 routes:
    // 0-11% faster than 256 for fp8 and blockscale, never slower), so stage 2 never runs
    // single-block tiles of 256 columns
    else if (stage == 2 && tile_n == 256 && N % 128 == 0) tile_n = 128;
    // stage 2 with atomics on prefill routings (16+ routes per expert) of 32- and 64-row blocks:
    // 64 columns (DS-TP8 dims, 64-row blocks: fp8 2048 / 8192 tokens 194.6 / 727.6 us against
    // 206.3 / 749.4 for 128, W4A16 8192 tokens 806.9 against 861.9; 32-row int4 2048 tokens
    // level); per-route rows and fewer routes keep 128 (fp8 rows at 1024 tokens: 88.2 against
    // 114.9; DS-TP8 decode dims 128 tokens, W4A16 atomics: 80.5 against 87.5)
    if (stage == 2 && atomics && tile_m >= 32 && routes >= 16L * experts && tile_n == 128 && N % 64 == 0)
      tile_n = 64;
    // stage 1 (W4A16, blockscale): 128 columns where that gives about three workgroups per CU,
    // else 64, never 256.  Graph-timed against the caller's 256: W4A16 DS-TP8 prefill dims,
    // 64-row blocks at 2048 tokens 220 us (128) against 387, 32-row blocks at 512 tokens 91.8
    // (64) against 117.5 (128) and 161 (256); DS-V3 decode dims at 64 tokens 127.5 (64) / 124.4
    // (128) against 162; blockscale DS-V3-M128 dims at 1024 tokens 244.5 (128) against 268 (64)
    // and 324, at 128 tokens 157.9 (64) against 160.4 (128) and 162.
    else if (stage == 1 && N % 128 == 0)
      tile_n = runs1 * (N / 128) >= 768 ? 128 : 64;
  }
  if (tile_n != 64 && tile_n != 128 && tile_n != 256)
    return fail(hipErrorInvalidValue, "%s: tile_n=%d must be 64, 128 or 256", what, tile_n);
  if (N % tile_n != 0) return fail(hipErrorInvalidValue, "%s: N=%d must be a multiple of tile_n=%d", what, N, tile_n);
  *r_out = R;
  *tn_out = tile_n;
  return 0;
}

// in_dtype -> kernel kind (and whether stage-1 activations come per route); -1 if unknown
int moe_kind(int in_dtype, int stage, bool* token_slot) {
  *token_slot = false;
  switch (in_dtype) {
    case FLYGEMM_IN_FP8: return KIND_FP8;
    case FLYGEMM_IN_INT8: return KIND_INT8;
    case FLYGEMM_IN_INT8_SMOOTH: *token_slot = stage == 1; return KIND_INT8;
    case FLYGEMM_IN_INT4: return KIND_INT4;
    case FLYGEMM_IN_INT4_BF16: return KIND_W4A16;
    case FLYGEMM_IN_BF16: return KIND_BF16;
    case FLYGEMM_IN_FP16: return KIND_F16;
    default: return -1;
  }
}

// A validated MoE GEMM launch; kernel null when there is nothing to launch (no tokens or blocks).
struct MoePlan {
  MoeKernel kernel;
  long grid;
  MoeArgs args;
};

// Every check of a MoE GEMM call and its launch parameters, without launching anything.
int moe_plan(int stage, void* out, const void* a, const void* w, const float* sa, const float* sw,
             const int32_t* sorted_ids, const int32_t* expert_ids, const float* sorted_w, const int32_t* num_valid,
             int tokens, int N, int K, int blocks, int experts, int topk, int tile_m, int tile_n, int in_dtype,
             int out_dtype, int doweight, int accumulate, bool bs, int group_size, MoePlan* pl) {
  pl->kernel = MoeKernel{nullptr, 0};
  const char* what = bs ? (stage == 1 ? "moe_blockscale_gemm1" : "moe_blockscale_gemm2")
                        : (stage == 1 ? "moe_gemm1" : "moe_gemm2");
  if (tokens < 0 || N <= 0 || K <= 0 || blocks < 0 || experts <= 0)
    return fail(hipErrorInvalidValue, "%s: invalid sizes tokens=%d N=%d K=%d blocks=%d experts=%d", what, tokens, N, K,
                blocks, experts);
  if (topk < 1 || topk > 255) return fail(hipErrorInvalidValue, "%s: topk=%d must be in [1, 255]", what, topk);
  if (tokens >= (1 << 24)) return fail(hipErrorInvalidValue, "%s: tokens=%d must be below 2^24", what, tokens);
  if (tile_m != 16 && tile_m != 32 && tile_m != 64)
    return fail(hipErrorInvalidValue, "%s: tile_m=%d must be 16, 32 or 64", what, tile_m);
  // the caller's tile is checked as the reference checks it, before the choices below
  if (tile_n > 0 && tile_n != 64 && tile_n != 128 && tile_n != 256)
    return fail(hipErrorInvalidValue, "%s: tile_n=%d must be 64, 128 or 256", what, tile_n);
  if (tile_n > 0 && N % tile_n != 0)
    return fail(hipErrorInvalidValue, "%s: N=%d must be a multiple of tile_n=%d", what, N, tile_n);
  bool token_slot = false;
  const int kind = moe_kind(in_dtype, stage, &token_slot);
  if (kind < 0) return fail(hipErrorInvalidValue, "%s: in_dtype %d not supported", what, in_dtype);
  if (bs && kind != KIND_FP8) return fail(hipErrorInvalidValue, "%s: blockscale takes fp8", what);
  if (kind == KIND_INT4 && K >= kInt4KLimit)
    return fail(hipErrorInvalidValue, "%s: K=%d: int4 weights take K < %d (int32 accumulators of 16x the dot product)",
                what, K, kInt4KLimit);
  // group scales: W4A16 only, 32-element groups along K (reference tests/utils.py:99-120)
  if (group_size > 0 && (kind != KIND_W4A16 || group_size != 32))
    return fail(hipErrorInvalidValue, "%s: group_size=%d: group scales are for int4_bf16 with group_size 32", what,
                group_size);
  int R = 1;
  if (int rc = moe_tiles(stage, tokens, N, K, experts, topk, tile_m, tile_n, kind, bs, stage == 2 && accumulate != 0,
                         what, &R, &tile_n, group_size > 0))
    return rc;
  const bool is16 = moe_a_16bit(kind);      // 2-byte activations (bf16, fp16, W4A16)
  const long kb = is16 ? 2L * K : (long)K;  // activation bytes per row
  if (kb % 128 != 0)
    return fail(hipErrorInvalidValue, "%s: K=%d must be a multiple of %d (128-byte K tile)", what, K, is16 ? 64 : 128);
  const long a_rows = stage == 1 && !token_slot ? tokens : (long)tokens * topk;
  const long w_rows = stage == 1 ? 2L * N : (long)N;
  const long wb = moe_w_int4(kind) ? K / 2 : kb;  // weight bytes per row
  if (a_rows * kb >= (1L << 31) || w_rows * wb >= (1L << 31))
    return fail(hipErrorInvalidValue, "%s: activation or per-expert weight above 2^31 bytes", what);
  int mout;
  const bool rows = stage == 2 && !accumulate;
  if (out_dtype == FLYGEMM_OUT_FP16) mout = rows ? MOE_OUT_F16_ROWS : MOE_OUT_F16;
  else if (out_dtype == FLYGEMM_OUT_BF16) mout = rows ? MOE_OUT_BF16_ROWS : MOE_OUT_BF16;
  else if (out_dtype == FLYGEMM_OUT_F32 && stage == 2 && accumulate) mout = MOE_OUT_F32;
  else return fail(hipErrorInvalidValue, "%s: out_dtype %d not supported%s", what, out_dtype,
                   rows ? " without accumulation (fp16 or bf16)" : "");
  if (tokens == 0 || blocks == 0) return 0;
  if (!out || !a || !w || !sorted_ids || !expert_ids || !num_valid)
    return fail(hipErrorInvalidValue, "%s: null tensor pointer", what);
  const bool need_sa = !is16, need_sw = !kind_is_16bit(kind);
  if ((need_sa && !sa) || (need_sw && !sw)) return fail(hipErrorInvalidValue, "%s: null scale pointer", what);
  if (doweight && !sorted_w) return fail(hipErrorInvalidValue, "%s: null sorted_weights with doweight", what);

  const long out_bytes = (stage == 1 || !accumulate) ? (long)tokens * topk * N * 2
                                                     : (long)tokens * N * (mout == MOE_OUT_F32 ? 4 : 2);
  if (out_bytes > 0xFFFFFF00L) return fail(hipErrorInvalidValue, "%s: output above 4 GB", what);

  if (bs && (2L * N) % (stage == 1 ? 128 : 256) != 0)
    return fail(hipErrorInvalidValue, "%s: %s=%d must be a multiple of 128 (weight scale blocks)", what,
                stage == 1 ? "2*inter_dim" : "model_dim", stage == 1 ? 2 * N : N);
  MoeKernel k = stage == 1 ? moe_stage1_kernel(kind, tile_m, R, tile_n, bs)
                           : moe_stage2_kernel(kind, tile_m, R, tile_n, mout == MOE_OUT_F32, bs);
  // Stage 2 per-route rows (the reduce mode's GEMM) of 1-byte and 16-bit weights with inter_dim
  // of 1, 2 or 4 128-byte K steps: the stream kernel (moe_stream.h), 64-column tiles, A resident,
  // the next tile's weights loaded before this tile's stores.  With 1 to 32 routes per expert on
  // average it runs single routing blocks (32 rows for 16-row blocks), each workgroup walking
  // about 64 KB of weights (four 64-column tiles of fp8 at inter_dim 256, two of bf16); with a
  // full 128-row run per expert on average (and for 16-row blocks from 32 routes per expert,
  // wherever the kernel above takes 256-row runs) runs of 128 rows.  Graph-timed, bit-equal,
  // reduce mode (GEMM + reduction), fp8, inter_dim 256, model_dim 7168: DS-TP8 decode dims (256
  // experts, 32-row blocks) 32 / 128 / 256 / 512 tokens 49.0 / 98.5 / 106.7 / 117.4 us against
  // 59.0 / 117.3 / 123.6 / 124.5 (single-block kernel above), 8 tokens level (20 us); bf16 2
  // tiles per workgroup, 9-16% faster from 32 tokens; DS-TP8 prefill dims (128 experts) 128 / 512
  // tokens 42.3 / 60.1 against 46.7 / 80.5 (16-row blocks, the latter against 128-row runs),
  // 43.1 / 59.4 against 51.3 / 61.6 (64-row blocks); at 64 routes per expert (1024 tokens) single
  // blocks were 3-6% slower for 16- and 64-row blocks, and 128-row runs win from 128 (64-row
  // blocks 2048 / 4096 / 8192 tokens 146 / 246 / 438 us against 164 / 279 / 586 for the kernel
  // above).  Fewer routes than experts (8 tokens top-8 of 256): the kernel above.
  bool stream2 = false, single2 = false;
  const long routes_all = (long)tokens * topk;
  if (stage == 2 && rows && !bs && kb <= 512 && routes_all >= experts) {
    single2 = routes_all <= 32L * experts;
    // (int4 weights, half the bytes per tile: 128-row runs from 256 routes per expert for 32- and
    // 64-row blocks -- DS-TP8 prefill 4096 / 8192 tokens 232 / 443 us against 266 / 566 for the
    // kernel above, at 2048 149 against 128)
    const long runs_from = kind == KIND_INT4 ? 256L : 128L;
    if (single2 || routes_all >= runs_from * experts || (tile_m == 16 && routes_all >= 32L * experts)) {
      const MoeKernel k2 = moe_stage2_stream_kernel(kind, tile_m, (int)(kb / 128), single2);
      if (k2.fn) {
        k = k2;
        R = single2 ? (tile_m == 16 ? 2 : 1) : 128 / tile_m;
        tile_n = 64;
        stream2 = true;
      }
    }
  }
  if (!k.fn) return fail(hipErrorInvalidValue, "%s: no kernel for tile %dx%d (runs of %d)", what, tile_m, tile_n, R);

  // column ranges per run: about 1024 workgroups in all (the stream kernel: one column tile each)
  const long ntn = N / tile_n;
  const long runs = est_runs(tokens, topk, experts, tile_m, R);
  long nsplit = (1024 + runs - 1) / runs;
  nsplit = nsplit < 1 ? 1 : (nsplit > ntn ? ntn : nsplit);
  if (moe_stream_stage1(stage, kind, bs)) nsplit = ntn;
  // stage 2 with atomics: at least half as many column ranges as tiles (two tiles of 128 columns
  // or 256 per workgroup, at most; about 1024 workgroups leave few runs long walks whose atomic
  // epilogues queue behind each other).  Graph-timed, fp8 (blockscale for DS-V3-M128), the
  // former about-1024 rule against this: DS-TP8 prefill 64-row blocks 2048 / 4096 / 8192 tokens
  // 269 / 437 / 861 us against 208 / 387 / 749, 32-row 2048 tokens 260 against 210, 16-row
  // (256-row runs) 8192 tokens 899 against 859; DS-TP8 decode dims 32 / 128 tokens 64.7 / 112.6
  // against 51.5 / 97.2; DS-V3-M128 blockscale 95.6 against 84.1.  Fewer routes than experts
  // (decode, 8 tokens top-8 of 256: 19.0 against 19.5) and the per-route rows keep the rule
  // above (level or faster there).
  if (stage == 2 && !rows && routes_all >= experts && ntn / 2 > nsplit) nsplit = ntn / 2;
  // the stage-2 stream kernel: 4 column ranges per run (DS-TP8 prefill, 2 / 3 / 4 / 6 / 8: 574 /
  // 470 / 438 / 468 / 444 us), more when the runs are few (about 1024 workgroups; 1024 tokens,
  // 32-row blocks: 16 ranges 111 us against 117 for 4)
  if (stream2) nsplit = std::min(ntn, std::max(4L, (1024 + runs - 1) / runs));
  // single blocks: about 64 KB of weights per workgroup (DS-TP8 decode dims, 32 tokens: fp8 28
  // ranges of four tiles 49.0 us, 4 ranges 52.6, 56 ranges 52.6; bf16 56 ranges of two 105.8
  // against 107.9 for 28)
  if (stream2 && single2) {
    const long per = std::max(1L, 65536L / ((long)tile_n * kb));
    nsplit = (ntn + per - 1) / per;
  }
  MoeArgs args{out,      (const uint8_t*)a, (const uint8_t*)w, sa,  sw,      sorted_ids, expert_ids,
               sorted_w, num_valid,         tokens,            topk, N,      (int)kb,    experts,
               doweight ? 1 : 0, blocks, (int)nsplit, mout, (uint32_t)out_bytes, token_slot ? 1 : 0,
               group_size > 0 ? group_size : 0};
  // grid (N / tile_n, blocks) in the reference; here one dimension over (block, column range),
  // rounded up to a multiple of 8 for the kernel's XCD-aware order (the extra workgroups and
  // those that do not start a run exit at once)
  const long g = (nsplit * blocks + 7) / 8 * 8;
  if (g >= (1L << 31)) return fail(hipErrorInvalidValue, "%s: grid too large", what);
  pl->kernel = k;
  pl->grid = g;
  pl->args = args;
  return 0;
}

int moe_run(const MoePlan& pl, const char* what, hipStream_t stream) {
  if (!pl.kernel.fn) return 0;
  hipLaunchKernelGGL(pl.kernel.fn, dim3((unsigned)pl.grid), dim3(pl.kernel.threads), 0, stream, pl.args);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(e, "launch of %s failed: %s", what, hipGetErrorString(e));
  return 0;
}

int moe_launch(int stage, void* out, const void* a, const void* w, const float* sa, const float* sw,
               const int32_t* sorted_ids, const int32_t* expert_ids, const float* sorted_w,
               const int32_t* num_valid, int tokens, int N, int K, int blocks, int experts, int topk, int tile_m,
               int tile_n, int in_dtype, int out_dtype, int doweight, int accumulate, bool bs, int group_size,
               hipStream_t stream) {
  MoePlan pl;
  if (int rc = moe_plan(stage, out, a, w, sa, sw, sorted_ids, expert_ids, sorted_w, num_valid, tokens, N, K, blocks,
                        experts, topk, tile_m, tile_n, in_dtype, out_dtype, doweight, accumulate, bs, group_size, &pl))
    return rc;
  return moe_run(pl, bs ? (stage == 1 ? "moe_blockscale_gemm1" : "moe_blockscale_gemm2")
                        : (stage == 1 ? "moe_gemm1" : "moe_gemm2"),
                 stream);
}

// Per-route rows of flygemm_moe_gemm2_reduce_noalloc: a device array of the library's own, so
// that entry point allocates nothing.  Each GPU holds one copy at its own address until the
// process ends, shared by every call on that GPU (calls that overlap on one GPU race).  In host
// code the name is a stand-in, not a device address: kernels and fills get the address
// hipGetSymbolAddress returns for the current device.
constexpr long kNoAllocScratchBytes = FLYGEMM_MOE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, resolved once per device.  The first
// resolution on a device must not happen while `stream` is being captured into a graph (the
// symbol lookup is not a stream operation and may invalidate the capture): that call fails
// with a message instead.
int noalloc_scratch(void** out, const char* what, hipStream_t stream) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(e, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(hipErrorInvalidDevice, "%s: device %d out of range", what, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) return fail(e, "%s: hipStreamIsCapturing failed: %s", what, hipGetErrorString(e));
    if (cs != hipStreamCaptureStatusNone)
      return fail(hipErrorStreamCaptureUnsupported,
                  "%s: the first call on device %d is under graph capture; make one eager call on this device "
                  "first (it resolves the scratch address)", what, dev);
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "%s: hipGetSymbolAddress of the scratch failed: %s",
                  what, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

// Zero fill in place of hipMemsetAsync, so the call can be captured in a graph.
__global__ void __launch_bounds__(256) zero_fill_kernel(uint4* p, long n) {
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) p[i] = uint4{0, 0, 0, 0};
}

}  // namespace

extern "C" {

int flygemm_moe_gemm1(void* out, const void* x, const void* w, const float* scale_x, const float* scale_w,
                      const int32_t* sorted_token_ids, const int32_t* sorted_expert_ids, const float* sorted_weights,
                      const int32_t* num_valid_ids, int32_t tokens, int32_t inter_dim, int32_t model_dim,
                      int32_t size_expert_ids, int32_t experts, int32_t topk, int32_t tile_m, int32_t tile_n,
                      int32_t in_dtype, int32_t out_dtype, int32_t doweight_stage1, int32_t group_size,
                      void* stream) {
  return moe_launch(1, out, x, w, scale_x, scale_w, sorted_token_ids, sorted_expert_ids, sorted_weights, num_valid_ids,
                    tokens, inter_dim, model_dim, size_expert_ids, experts, topk, tile_m, tile_n, in_dtype, out_dtype,
                    doweight_stage1, 1, false, group_size, (hipStream_t)stream);
}

int flygemm_moe_gemm2(void* out, const void* a2, const void* w, const float* scale_a2, const float* scale_w,
                      const int32_t* sorted_token_ids, const int32_t* sorted_expert_ids, const float* sorted_weights,
                      const int32_t* num_valid_ids, int32_t tokens, int32_t model_dim, int32_t inter_dim,
                      int32_t size_expert_ids, int32_t experts, int32_t topk, int32_t tile_m, int32_t tile_n,
                      int32_t in_dtype, int32_t out_dtype, int32_t doweight_stage2, int32_t accumulate,
                      int32_t group_size, void* stream) {
  return moe_launch(2, out, a2, w, scale_a2, scale_w, sorted_token_ids, sorted_expert_ids, sorted_weights,
                    num_valid_ids, tokens, model_dim, inter_dim, size_expert_ids, experts, topk, tile_m, tile_n,
                    in_dtype, out_dtype, doweight_stage2, accumulate, false, group_size, (hipStream_t)stream);
}

int flygemm_moe_blockscale_gemm1(void* out, const void* x, const void* w, const float* x_scale_t,
                                 const float* w_scale, const int32_t* sorted_token_ids,
                                 const int32_t* sorted_expert_ids, const float* sorted_weights,
                                 const int32_t* num_valid_ids, int32_t tokens, int32_t inter_dim, int32_t model_dim,
                                 int32_t size_expert_ids, int32_t experts, int32_t topk, int32_t tile_m,
                                 int32_t tile_n, int32_t scale_block_k, int32_t out_dtype, int32_t doweight_stage1,
                                 void* stream) {
  if (scale_block_k != 128)
    return fail(hipErrorInvalidValue, "moe_blockscale_gemm1: scale_block_k=%d: only 128 is supported", scale_block_k);
  return moe_launch(1, out, x, w, x_scale_t, w_scale, sorted_token_ids, sorted_expert_ids, sorted_weights,
                    num_valid_ids, tokens, inter_dim, model_dim, size_expert_ids, experts, topk, tile_m, tile_n,
                    FLYGEMM_IN_FP8, out_dtype, doweight_stage1, 1, true, -1, (hipStream_t)stream);
}

int flygemm_moe_blockscale_gemm2(void* out, const void* a2, const void* w, const float* a2_scale_t,
                                 const float* w_scale, const int32_t* sorted_token_ids,
                                 const int32_t* sorted_expert_ids, const float* sorted_weights,
                                 const int32_t* num_valid_ids, int32_t tokens, int32_t model_dim, int32_t inter_dim,
                                 int32_t size_expert_ids, int32_t experts, int32_t topk, int32_t tile_m,
                                 int32_t tile_n, int32_t scale_block_k, int32_t out_dtype, int32_t doweight_stage2,
                                 int32_t accumulate, void* stream) {
  if (scale_block_k != 128)
    return fail(hipErrorInvalidValue, "moe_blockscale_gemm2: scale_block_k=%d: only 128 is supported", scale_block_k);
  return moe_launch(2, out, a2, w, a2_scale_t, w_scale, sorted_token_ids, sorted_expert_ids, sorted_weights,
                    num_valid_ids, tokens, model_dim, inter_dim, size_expert_ids, experts, topk, tile_m, tile_n,
                    FLYGEMM_IN_FP8, out_dtype, doweight_stage2, accumulate, true, -1, (hipStream_t)stream);
}

int flygemm_moe_reduce(void* y, const void* x, const void* valid_mask, int32_t tokens, int32_t topk,
                       int32_t model_dim, int32_t dtype, void* stream) {
  if (tokens < 0 || topk < 1 || model_dim <= 0)
    return fail(hipErrorInvalidValue, "moe_reduce: invalid sizes tokens=%d topk=%d model_dim=%d", tokens, topk,
                model_dim);
  if (dtype != FLYGEMM_OUT_FP16 && dtype != FLYGEMM_OUT_BF16 && dtype != FLYGEMM_OUT_F32)
    return fail(hipErrorInvalidValue, "moe_reduce: dtype %d not supported", dtype);
  const int ve = dtype == FLYGEMM_OUT_F32 ? 4 : 8;
  if (model_dim % ve != 0)
    return fail(hipErrorInvalidValue, "moe_reduce: model_dim=%d must be a multiple of %d (16-byte vectors)",
                model_dim, ve);
  if (tokens == 0) return 0;
  if (!y || !x) return fail(hipErrorInvalidValue, "moe_reduce: null tensor pointer");
  if (((uintptr_t)y | (uintptr_t)x) & 15) return fail(hipErrorInvalidValue, "moe_reduce: misaligned pointer");
  const long n = (long)tokens * (model_dim / ve);
  const long g = (n + 255) / 256;
  if (g >= (1L << 31)) return fail(hipErrorInvalidValue, "moe_reduce: too large");
  void (*fn)(void*, const void*, const int8_t*, int, int, int) =
      dtype == FLYGEMM_OUT_FP16 ? moe_reduce_kernel<0> : dtype == FLYGEMM_OUT_BF16 ? moe_reduce_kernel<1>
                                                                                   : moe_reduce_kernel<2>;
  hipLaunchKernelGGL(fn, dim3((unsigned)g), dim3(256), 0, (hipStream_t)stream, y, x, (const int8_t*)valid_mask,
                     tokens, topk, model_dim);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(e, "launch of moe_reduce failed: %s", hipGetErrorString(e));
  return 0;
}

int flygemm_moe_select_tile(int32_t stage, int32_t tokens, int32_t n, int32_t k, int32_t experts, int32_t topk,
                            int32_t tile_m, int32_t tile_n, int32_t in_dtype, int32_t blockscale, int32_t* runs,
                            int32_t* tile_n_out) {
  const char* what = "moe_select_tile";
  if (stage != 1 && stage != 2) return fail(hipErrorInvalidValue, "%s: stage %d must be 1 or 2", what, stage);
  if (tokens < 0 || n <= 0 || k <= 0 || experts <= 0 || topk < 1 || topk > 255)
    return fail(hipErrorInvalidValue, "%s: invalid sizes tokens=%d n=%d k=%d experts=%d topk=%d", what, tokens, n, k,
                experts, topk);
  if (tile_m != 16 && tile_m != 32 && tile_m != 64)
    return fail(hipErrorInvalidValue, "%s: tile_m=%d must be 16, 32 or 64", what, tile_m);
  if (tile_n > 0 && ((tile_n != 64 && tile_n != 128 && tile_n != 256) || n % tile_n != 0))
    return fail(hipErrorInvalidValue, "%s: tile_n=%d must be 64, 128 or 256 and divide n=%d", what, tile_n, n);
  if (!runs || !tile_n_out) return fail(hipErrorInvalidValue, "%s: null output pointer", what);
  bool token_slot = false;
  const int kind = moe_kind(in_dtype, stage, &token_slot);
  if (kind < 0) return fail(hipErrorInvalidValue, "%s: in_dtype %d not supported", what, in_dtype);
  int r = 1, tn = 0;
  if (int rc = moe_tiles(stage, tokens, n, k, experts, topk, tile_m, tile_n, kind, blockscale != 0, stage == 2, what, &r,
                         &tn))
    return rc;
  *runs = r;
  *tile_n_out = tn;
  return 0;
}

int flygemm_moe_gemm2_reduce_noalloc(void* out, const void* a2, const void* w, const float* scale_a2,
                                     const float* scale_w, const int32_t* sorted_token_ids,
                                     const int32_t* sorted_expert_ids, const float* sorted_weights,
                                     const int32_t* num_valid_ids, int32_t tokens, int32_t model_dim,
                                     int32_t inter_dim, int32_t size_expert_ids, int32_t experts, int32_t topk,
                                     int32_t tile_m, int32_t tile_n, int32_t in_dtype, int32_t out_dtype,
                                     int32_t doweight_stage2, int32_t group_size, const void* valid_mask,
                                     int32_t zero_intermediate, void* stream) {
  const char* what = "moe_gemm2_reduce_noalloc";
  if (out_dtype != FLYGEMM_OUT_FP16 && out_dtype != FLYGEMM_OUT_BF16)
    return fail(hipErrorInvalidValue, "%s: out_dtype %d not supported (fp16 or bf16)", what, out_dtype);
  if (tokens < 0 || topk < 1 || model_dim <= 0)
    return fail(hipErrorInvalidValue, "%s: invalid sizes tokens=%d topk=%d model_dim=%d", what, tokens, topk,
                model_dim);
  if (model_dim % 8 != 0)
    return fail(hipErrorInvalidValue, "%s: model_dim=%d must be a multiple of 8", what, model_dim);
  const long need = (long)tokens * topk * model_dim * 2;
  if (need > kNoAllocScratchBytes)
    return fail(hipErrorInvalidValue, "%s: tokens*topk*model_dim*2 = %ld bytes exceeds the static scratch of %ld bytes",
                what, need, kNoAllocScratchBytes);
  if (tokens == 0) return 0;
  // every check comes before the first launch: a rejected call queues nothing on the stream
  if (!out) return fail(hipErrorInvalidValue, "%s: null output pointer", what);
  if ((uintptr_t)out & 15) return fail(hipErrorInvalidValue, "%s: misaligned output (16 bytes needed)", what);
  hipStream_t s = (hipStream_t)stream;
  // the GEMM's checks run with `out` standing in for the scratch (both are non-null); the
  // scratch address goes into the arguments once resolved
  MoePlan pl;
  if (int rc = moe_plan(2, out, a2, w, scale_a2, scale_w, sorted_token_ids, sorted_expert_ids, sorted_weights,
                        num_valid_ids, tokens, model_dim, inter_dim, size_expert_ids, experts, topk, tile_m, tile_n,
                        in_dtype, out_dtype, doweight_stage2, 0, false, group_size, &pl))
    return rc;
  void* inter = nullptr;
  if (int rc = noalloc_scratch(&inter, what, s)) return rc;
  pl.args.out = inter;
  if (zero_intermediate && !valid_mask) {
    const long n = need / 16;
    const long g = (n + 255) / 256 < 2048 ? (n + 255) / 256 : 2048;
    hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)g), dim3(256), 0, s, (uint4*)inter, n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(e, "%s: launch of the zero fill failed: %s", what, hipGetErrorString(e));
  }
  if (int rc = moe_run(pl, what, s)) return rc;
  return flygemm_moe_reduce(out, inter, valid_mask, tokens, topk, model_dim, out_dtype, stream);
}

}  // extern "C"

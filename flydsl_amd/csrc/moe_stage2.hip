// Kernel table of MoE stage 2 (the down projection), in a translation unit of its own so the
// library's sources compile in parallel.
#include <hip/hip_runtime.h>

#include "moe.h"

namespace flygemm {

namespace {
template <int KIND, bool F32, bool BS>
MoeKernel stage2_tile(int tm, int r, int tn) {
#define T(M_, R_, N_, WM_, WN_)        \
  if (tm == M_ && r == R_ && tn == N_) \
    return MoeKernel{moe_gemm_kernel<2, KIND, M_, R_, N_, WM_, WN_, F32, BS>, WM_ * WN_ * 64};
  // single-block tiles of 64 and 128 columns: the launcher never gives stage 2 single-block
  // tiles of 256 columns (it narrows them to 128 or 64)
  T(16, 1, 64, 1, 4) T(16, 1, 128, 1, 4) T(32, 1, 64, 1, 4) T(32, 1, 128, 1, 4) T(64, 1, 64, 1, 4)
  T(64, 1, 128, 1, 4)
  // run tiles of 256 rows: for 16-row blocks only (32- and 64-row blocks keep single-block
  // tiles in stage 2); not for blockscale (its partials and factors do not fit next to them)
  // nor W4A16 (its group scales ride the two-slot pipeline)
  if constexpr (!BS && KIND != KIND_W4A16) {
    T(16, 16, 256, 2, 4)
  }
  // runs of 256 rows (four 64-row or eight 32-row blocks), 256 columns: routings with large
  // experts (see moe_tiles)
  if constexpr (!BS && (moe_big_kind(KIND) || KIND == KIND_W4A16)) {
    T(64, 4, 256, 2, 4) T(32, 8, 256, 2, 4)
  }
  // blockscale: runs of 256 rows, 128 columns (the per-K-block partials and factors fit next to
  // 128-column accumulators), for large experts (see moe_tiles)
  if constexpr (BS) {
    T(64, 4, 128, 2, 4) T(32, 8, 128, 2, 4) T(16, 16, 128, 2, 4)
  }
#undef T
  return MoeKernel{nullptr, 0};
}

template <int KIND>
MoeKernel stage2_kind(int tm, int r, int tn, bool f32) {
  return f32 ? stage2_tile<KIND, true, false>(tm, r, tn) : stage2_tile<KIND, false, false>(tm, r, tn);
}
}  // namespace

MoeKernel moe_stage2_kernel(int kind, int tm, int r, int tn, bool f32, bool bs) {
  if (bs)
    return kind != KIND_FP8 ? MoeKernel{nullptr, 0}
                            : (f32 ? stage2_tile<KIND_FP8, true, true>(tm, r, tn)
                                   : stage2_tile<KIND_FP8, false, true>(tm, r, tn));
  switch (kind) {
    case KIND_FP8: return stage2_kind<KIND_FP8>(tm, r, tn, f32);
    case KIND_INT8: return stage2_kind<KIND_INT8>(tm, r, tn, f32);
    case KIND_INT4: return stage2_kind<KIND_INT4>(tm, r, tn, f32);
    case KIND_W4A16: return stage2_kind<KIND_W4A16>(tm, r, tn, f32);
    case KIND_BF16: return stage2_kind<KIND_BF16>(tm, r, tn, f32);
    case KIND_F16: return stage2_kind<KIND_F16>(tm, r, tn, f32);
    default: return MoeKernel{nullptr, 0};
  }
}

}  // namespace flygemm

// Kernel table of the MoE stage-2 per-route-rows stream kernel (moe_stream.h), in a
// translation unit of its own so the library's sources compile in parallel.
#include <hip/hip_runtime.h>

#include "moe_stream.h"

namespace flygemm {

namespace {
template <int KIND, int NK>
MoeKernel stream2_tile(int tm, bool single) {
  if (single) {
    switch (tm) {   // one routing block (two of 16 rows)
      case 16: return MoeKernel{moe_stream2_kernel<KIND, 16, 2, NK>, 256};
      case 32: return MoeKernel{moe_stream2_kernel<KIND, 32, 1, NK>, 256};
      case 64: return MoeKernel{moe_stream2_kernel<KIND, 64, 1, NK>, 256};
      default: return MoeKernel{nullptr, 0};
    }
  }
  switch (tm) {   // runs of 128 rows
    case 16: return MoeKernel{moe_stream2_kernel<KIND, 16, 8, NK>, 256};
    case 32: return MoeKernel{moe_stream2_kernel<KIND, 32, 4, NK>, 256};
    case 64: return MoeKernel{moe_stream2_kernel<KIND, 64, 2, NK>, 256};
    default: return MoeKernel{nullptr, 0};
  }
}

template <int KIND>
MoeKernel stream2_kind(int tm, int nk, bool single) {
  switch (nk) {
    case 1: return stream2_tile<KIND, 1>(tm, single);
    case 2: return stream2_tile<KIND, 2>(tm, single);
    case 4: return stream2_tile<KIND, 4>(tm, single);
    default: return MoeKernel{nullptr, 0};
  }
}
}  // namespace

// nk: 128-byte K steps of inter_dim (1, 2 or 4); single: runs of one routing block (32 rows for
// 16-row blocks) instead of 128 rows; null for other kinds and depths
MoeKernel moe_stage2_stream_kernel(int kind, int tm, int nk, bool single) {
  switch (kind) {
    case KIND_FP8: return stream2_kind<KIND_FP8>(tm, nk, single);
    case KIND_INT8: return stream2_kind<KIND_INT8>(tm, nk, single);
    case KIND_INT4: return stream2_kind<KIND_INT4>(tm, nk, single);
    case KIND_BF16: return stream2_kind<KIND_BF16>(tm, nk, single);
    case KIND_F16: return stream2_kind<KIND_F16>(tm, nk, single);
    default: return MoeKernel{nullptr, 0};
  }
}

}  // namespace flygemm

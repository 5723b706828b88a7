// Kernel table of the MoE stage-1 stream kernel (moe_stream.h), in a translation unit of its own
// so the library's sources compile in parallel.
#include <hip/hip_runtime.h>

#include "moe_stream.h"

namespace flygemm {

namespace {
template <int KIND>
MoeKernel stream_tile(int tm) {
  // runs of 128 rows; D = 3 weight register sets (weights two steps ahead): 3, 4 and 6 sets
  // within 1% of each other on DS-TP8 prefill (fp8, 8192 tokens: 293 / 294 / 297 us)
  switch (tm) {
    case 16: return MoeKernel{moe_stream_kernel<KIND, 16, 8, 3>, 256};
    case 32: return MoeKernel{moe_stream_kernel<KIND, 32, 4, 3>, 256};
    case 64: return MoeKernel{moe_stream_kernel<KIND, 64, 2, 3>, 256};
    default: return MoeKernel{nullptr, 0};
  }
}
}  // namespace

MoeKernel moe_stage1_stream_kernel(int kind, int tm) {
  switch (kind) {
    case KIND_FP8: return stream_tile<KIND_FP8>(tm);
    case KIND_INT8: return stream_tile<KIND_INT8>(tm);
    case KIND_INT4: return stream_tile<KIND_INT4>(tm);
    case KIND_BF16: return stream_tile<KIND_BF16>(tm);
    case KIND_F16: return stream_tile<KIND_F16>(tm);
    default: return MoeKernel{nullptr, 0};
  }
}

}  // namespace flygemm

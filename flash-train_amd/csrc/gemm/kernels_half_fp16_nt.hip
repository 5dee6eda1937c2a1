// FP16 half-precision MFMA tiles for row-major a, column-major b (see gemm/half_tile.hpp).
// One translation unit per type and layout keeps the build parallel.
#include "half_tile.hpp"

namespace ftrain::gemm {

const void* halfKernelFp16NT(int tile) { return hdev::halfKernel<false, false, true>(tile); }

const void* groupedHalfKernelFp16NT(int which) { return hdev::groupedHalfKernel<false, false, true>(which); }

}  // namespace ftrain::gemm

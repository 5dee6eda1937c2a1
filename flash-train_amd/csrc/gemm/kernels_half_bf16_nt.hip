// BF16 half-precision MFMA tiles for row-major a, column-major b (see gemm/half_tile.hpp).
// One translation unit per type and layout keeps the build parallel.
#include "half_tile.hpp"

namespace ftrain::gemm {

const void* halfKernelBf16NT(int tile) { return hdev::halfKernel<true, false, true>(tile); }

const void* groupedHalfKernelBf16NT(int which) { return hdev::groupedHalfKernel<true, false, true>(which); }

}  // namespace ftrain::gemm

// BF16 half-precision MFMA tiles for column-major a, row-major b (see gemm/half_tile.hpp).
// One translation unit per type and layout keeps the build parallel.
#include "half_tile.hpp"

namespace ftrain::gemm {

const void* halfKernelBf16TN(int tile) { return hdev::halfKernel<true, true, false>(tile); }

const void* groupedHalfKernelBf16TN(int which) { return hdev::groupedHalfKernel<true, true, false>(which); }

}  // namespace ftrain::gemm

// BF16 half-precision MFMA tiles for column-major a and b (see gemm/half_tile.hpp).
// One translation unit per type and layout keeps the build parallel.
#include "half_tile.hpp"

namespace ftrain::gemm {

const void* halfKernelBf16TT(int tile) { return hdev::halfKernel<true, true, true>(tile); }

const void* groupedHalfKernelBf16TT(int which) { return hdev::groupedHalfKernel<true, true, true>(which); }

}  // namespace ftrain::gemm

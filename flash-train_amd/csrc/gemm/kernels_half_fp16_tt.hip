// FP16 half-precision MFMA tiles for column-major a and b (see gemm/half_tile.hpp).
// One translation unit per type and layout keeps the build parallel.
#include "half_tile.hpp"

namespace ftrain::gemm {

const void* halfKernelFp16TT(int tile) { return hdev::halfKernel<false, true, true>(tile); }

const void* groupedHalfKernelFp16TT(int which) { return hdev::groupedHalfKernel<false, true, true>(which); }

}  // namespace ftrain::gemm

// FP16 half-precision MFMA tiles for row-major a and b (see gemm/half_tile.hpp).
// One translation unit per type and layout keeps the build parallel.
#include "half_tile.hpp"

namespace ftrain::gemm {

const void* halfKernelFp16NN(int tile) { return hdev::halfKernel<false, false, false>(tile); }

const void* groupedHalfKernelFp16NN(int which) { return hdev::groupedHalfKernel<false, false, false>(which); }

}  // namespace ftrain::gemm

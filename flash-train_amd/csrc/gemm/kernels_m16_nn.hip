// FP32 16x16x4 MFMA tiles for one operand orientation (see gemm/mfma16_tile.hpp).
// One translation unit per layout keeps the build parallel.
#include "mfma16_tile.hpp"

namespace ftrain::gemm {

const void* mfma16KernelNN(int which) { return m16::mfma16Kernel<false, false>(which); }

}  // namespace ftrain::gemm

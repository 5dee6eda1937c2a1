// MFMA tile instantiations for row-major a, column-major b (see gemm/mfma_tile.hpp).
// One translation unit per layout keeps the build parallel.
#include "mfma_tile.hpp"

namespace ftrain::gemm {

const void* layoutKernelNT(Variant v) { return dev::layoutKernel<false, true>(v); }

const void* groupedKernelNT(int which) { return dev::groupedLayoutKernel<false, true>(which); }

}  // namespace ftrain::gemm

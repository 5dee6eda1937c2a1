// MFMA tile instantiations for column-major a, row-major b (see gemm/mfma_tile.hpp).
// One translation unit per layout keeps the build parallel.
#include "mfma_tile.hpp"

namespace ftrain::gemm {

const void* layoutKernelTN(Variant v) { return dev::layoutKernel<true, false>(v); }

const void* groupedKernelTN(int which) { return dev::groupedLayoutKernel<true, false>(which); }

}  // namespace ftrain::gemm

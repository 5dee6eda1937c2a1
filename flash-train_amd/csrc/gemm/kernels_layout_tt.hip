// MFMA tile instantiations for column-major a and b (see gemm/mfma_tile.hpp).
// One translation unit per layout keeps the build parallel.
#include "mfma_tile.hpp"

namespace ftrain::gemm {

const void* layoutKernelTT(Variant v) { return dev::layoutKernel<true, true>(v); }

const void* groupedKernelTT(int which) { return dev::groupedLayoutKernel<true, true>(which); }

}  // namespace ftrain::gemm

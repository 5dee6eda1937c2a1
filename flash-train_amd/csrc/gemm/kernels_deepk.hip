// The deep-k fp32 kernel (gemm/deepk_tile.hpp) and its counter reset.
#include "deepk_tile.hpp"

namespace ftrain::gemm {

const void* deepkKernel() { return reinterpret_cast<const void*>(&deepk::deepk_gemm); }
const void* deepkClearKernel() { return reinterpret_cast<const void*>(&deepk::deepk_clear_counters); }

}  // namespace ftrain::gemm

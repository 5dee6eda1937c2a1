// FP32 256x256 tile with LDS staging by DMA, row-major a and b (see gemm/dma32_tile.hpp).
#include "dma32_tile.hpp"

namespace ftrain::gemm {

const void* dma32Kernel() { return reinterpret_cast<const void*>(&d32::fp32_gemm_dma); }

}  // namespace ftrain::gemm

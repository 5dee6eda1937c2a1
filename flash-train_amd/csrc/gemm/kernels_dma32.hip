// FP32 256x256 tiles with LDS staging by DMA, row-major a and b, plain and grouped (see gemm/dma32_tile.hpp).
#include "dma32_tile.hpp"

namespace ftrain::gemm {

const void* dma32Kernel() { return reinterpret_cast<const void*>(&d32::fp32_gemm_dma); }

const void* groupedDma32Kernel() { return reinterpret_cast<const void*>(&d32::grouped_fp32_gemm_dma); }

}  // namespace ftrain::gemm

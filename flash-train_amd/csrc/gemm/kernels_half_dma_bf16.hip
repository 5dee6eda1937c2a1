// BF16 256x256 tiles with LDS staging by DMA, every operand orientation (see gemm/dma_tile.hpp).
#include "dma_tile.hpp"

namespace ftrain::gemm {

const void* dmaKernelBf16(bool ta, bool tb) { return ddev::dmaKernel<true>(ta, tb); }

const void* groupedDmaKernelBf16(bool ta, bool tb) { return ddev::groupedDmaKernel<true>(ta, tb); }

}  // namespace ftrain::gemm

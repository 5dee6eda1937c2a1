// FP16 256x256 tiles with LDS staging by DMA, every operand orientation (see gemm/dma_tile.hpp).
#include "dma_tile.hpp"

namespace ftrain::gemm {

const void* dmaKernelFp16(bool ta, bool tb) { return ddev::dmaKernel<false>(ta, tb); }

const void* groupedDmaKernelFp16(bool ta, bool tb) { return ddev::groupedDmaKernel<false>(ta, tb); }

}  // namespace ftrain::gemm

// FP16 256x256 tiles with LDS staging by DMA, every operand orientation (see gemm/dma_tile.hpp).
#include "dma_tile.hpp"

namespace ftrain::gemm {

const void* dmaKernelFp16(bool ta, bool tb, bool prefetch_b) { return ddev::dmaKernel<false>(ta, tb, prefetch_b); }

const void* groupedDmaKernelFp16(bool ta, bool tb, bool prefetch_b) {
    return prefetch_b ? ddev::groupedDmaKernel<false, 256, ddev::kLargeBPrefetch>(ta, tb) : ddev::groupedDmaKernel<false>(ta, tb);
}

const void* groupedDma128KernelFp16(bool ta, bool tb) { return ddev::groupedDmaKernel<false, 128>(ta, tb); }

const void* dma64x128KernelFp16(bool ta, bool tb) { return ddev::dma64x128Kernel<false>(ta, tb); }

const void* dma128KernelFp16(bool ta, bool tb, bool split) {
    return split ? ddev::dma128Kernel<false, true>(ta, tb) : ddev::dma128Kernel<false, false>(ta, tb);
}

}  // namespace ftrain::gemm

// BF16 256x256 tiles with LDS staging by DMA, every operand orientation (see gemm/dma_tile.hpp).
#include "dma_tile.hpp"

namespace ftrain::gemm {

const void* dmaKernelBf16(bool ta, bool tb, bool prefetch_b) { return ddev::dmaKernel<true>(ta, tb, prefetch_b); }

const void* groupedDmaKernelBf16(bool ta, bool tb, bool prefetch_b) {
    return prefetch_b ? ddev::groupedDmaKernel<true, 256, ddev::kLargeBPrefetch>(ta, tb) : ddev::groupedDmaKernel<true>(ta, tb);
}

const void* groupedDma128KernelBf16(bool ta, bool tb) { return ddev::groupedDmaKernel<true, 128>(ta, tb); }

const void* dma64x128KernelBf16(bool ta, bool tb) { return ddev::dma64x128Kernel<true>(ta, tb); }

const void* dma128KernelBf16(bool ta, bool tb, bool split) {
    return split ? ddev::dma128Kernel<true, true>(ta, tb) : ddev::dma128Kernel<true, false>(ta, tb);
}

}  // namespace ftrain::gemm

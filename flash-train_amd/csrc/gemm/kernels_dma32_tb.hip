// FP32 tiles with LDS staging by DMA, row-major a and column-major b (see gemm/dma32_tile.hpp).
// The 256x256 tiles are not instantiated for column-major b: their register budget spills there.
#include "dma32_tile.hpp"

namespace ftrain::gemm {

const void* dma32KernelTB(Variant v) {
    switch (v) {
        case Variant::kMfma16Dma128x128: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<128, 128, 2, 2, 2, false, true>);
        case Variant::kMfma16Dma128x128S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<128, 128, 2, 2, 2, true, true>);
        case Variant::kMfma16Dma64x256S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<64, 256, 1, 4, 2, true, true>);
        case Variant::kMfma16Dma256x64S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<256, 64, 4, 1, 2, true, true>);
        case Variant::kMfma16Dma64x128S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<64, 128, 2, 2, 2, true, true>);
        case Variant::kMfma16Dma128x64S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<128, 64, 4, 1, 2, true, true>);
        case Variant::kMfma16Dma64x64S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<64, 64, 4, 1, 2, true, true>);
        case Variant::kMfma16Dma64x128: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<64, 128, 2, 2, 2, false, true>);
        case Variant::kMfma16Dma128x64: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<128, 64, 4, 1, 2, false, true>);
        default: return nullptr;
    }
}

}  // namespace ftrain::gemm

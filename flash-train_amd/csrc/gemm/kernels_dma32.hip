// FP32 tiles with LDS staging by DMA, row-major a and b, plain and grouped (see gemm/dma32_tile.hpp).
#include "dma32_tile.hpp"

namespace ftrain::gemm {

const void* dma32Kernel(Variant v) {
    switch (v) {
        case Variant::kMfma16Dma256x256: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<256, 256, 2, 2, 1, false>);
        case Variant::kMfma16Dma256x256S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<256, 256, 2, 2, 1, true>);
        case Variant::kMfma16Dma128x128: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<128, 128, 2, 2, 2, false>);
        case Variant::kMfma16Dma128x128S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<128, 128, 2, 2, 2, true>);
        case Variant::kMfma16Dma64x256S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<64, 256, 1, 4, 2, true>);
        case Variant::kMfma16Dma256x64S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<256, 64, 4, 1, 2, true>);
        case Variant::kMfma16Dma64x128S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<64, 128, 2, 2, 2, true>);
        case Variant::kMfma16Dma128x64S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<128, 64, 4, 1, 2, true>);
        case Variant::kMfma16Dma64x64S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<64, 64, 4, 1, 2, true>);
        case Variant::kMfma16Dma64x128: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<64, 128, 2, 2, 2, false>);
        case Variant::kMfma16Dma128x64: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<128, 64, 4, 1, 2, false>);
        default: return nullptr;
    }
}

const void* groupedDma32Kernel() {
    return reinterpret_cast<const void*>(&d32::grouped_fp32_gemm_dma<256, 256, 2, 2, 1, false, false>);
}

const void* groupedDma32Kernel64x128(bool tb) {
    using namespace d32;
    return tb ? reinterpret_cast<const void*>(&grouped_fp32_gemm_dma<64, 128, 2, 2, 2, true, false>)
              : reinterpret_cast<const void*>(&grouped_fp32_gemm_dma<64, 128, 2, 2, 2, false, false>);
}

const void* groupedDma32Kernel128(bool ta, bool tb) {
    using namespace d32;
    if (ta) return tb ? reinterpret_cast<const void*>(&grouped_fp32_gemm_dma<128, 128, 2, 2, 2, true, true>)
                      : reinterpret_cast<const void*>(&grouped_fp32_gemm_dma<128, 128, 2, 2, 2, false, true>);
    return tb ? reinterpret_cast<const void*>(&grouped_fp32_gemm_dma<128, 128, 2, 2, 2, true, false>)
              : reinterpret_cast<const void*>(&grouped_fp32_gemm_dma<128, 128, 2, 2, 2, false, false>);
}

}  // namespace ftrain::gemm

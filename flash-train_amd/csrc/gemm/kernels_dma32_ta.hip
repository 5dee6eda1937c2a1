// FP32 tiles with LDS staging by DMA, column-major a and either b (see gemm/dma32_tile.hpp).  Only
// the tiles whose wave rows come in runs of 64 (the row interleave of a column-major a) have one.
#include "dma32_tile.hpp"

namespace ftrain::gemm {

namespace {
template <bool TB>
const void* ta_kernel(Variant v) {
    switch (v) {
        case Variant::kMfma16Dma128x128: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<128, 128, 2, 2, 2, false, TB, true>);
        case Variant::kMfma16Dma128x128S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<128, 128, 2, 2, 2, true, TB, true>);
        case Variant::kMfma16Dma64x256S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<64, 256, 1, 4, 2, true, TB, true>);
        case Variant::kMfma16Dma256x64S: return reinterpret_cast<const void*>(&d32::fp32_gemm_dma<256, 64, 4, 1, 2, true, TB, true>);
        default: return nullptr;
    }
}
}  // namespace

const void* dma32KernelTA(Variant v, bool tb) { return tb ? ta_kernel<true>(v) : ta_kernel<false>(v); }

}  // namespace ftrain::gemm

// Static description of every kernel variant: its Primitive name, tile
// geometry and the figures the Finder's cost model uses.
#include "ft/gemm_kernels.hpp"

namespace ftrain::gemm {
namespace {

// name, bm, bn, bk, threads, occupancy, vec, split, gemv, simt, efficiency
constexpr VariantInfo kInfo[] = {
    {"Fp32MfmaGemm_256x256", 256, 256, 16, 256, 1, true, false, false, false, 0.80},
    {"Fp32MfmaGemm_256x256_SplitK", 256, 256, 16, 256, 1, true, true, false, false, 0.78},
    {"Fp32MfmaGemm_128x128", 128, 128, 16, 256, 2, true, false, false, false, 0.70},
    {"Fp32MfmaGemm_128x128_SplitK", 128, 128, 16, 256, 2, true, true, false, false, 0.68},
    {"Fp32MfmaGemm_64x256", 64, 256, 16, 256, 2, true, false, false, false, 0.62},
    {"Fp32MfmaGemm_64x256_SplitK", 64, 256, 16, 256, 2, true, true, false, false, 0.60},
    {"Fp32MfmaGemm_256x64", 256, 64, 16, 256, 2, true, false, false, false, 0.62},
    {"Fp32MfmaGemm_256x64_SplitK", 256, 64, 16, 256, 2, true, true, false, false, 0.60},
    {"Fp32MfmaGemm_128x128_Unaligned", 128, 128, 16, 256, 2, false, false, false, false, 0.50},
    {"Fp32MfmaGemm_128x128_Unaligned_SplitK", 128, 128, 16, 256, 2, false, true, false, false, 0.48},
    {"Fp32Gemv_SplitK", kGemvRows, kGemvCols, 1, 256, 8, true, true, true, false, 0.0},
    {"Fp32Gemv_Unaligned_SplitK", kGemvRows, kGemvCols, 1, 256, 8, false, true, true, false, 0.0},
    {"Fp32Gemm", 64, 64, 16, 256, 2, false, false, false, true, 0.20},
};
static_assert(sizeof(kInfo) / sizeof(kInfo[0]) == static_cast<int>(Variant::kCount), "catalog");

}  // namespace

const VariantInfo& info(Variant v) { return kInfo[static_cast<int>(v)]; }

}  // namespace ftrain::gemm

// Static description of every kernel variant: its Primitive name, tile
// geometry and the figures the Finder's cost model uses.
#include "ft/gemm_kernels.hpp"

namespace ftrain::gemm {
namespace {

// name, bm, bn, bk, threads, occupancy, vec, split, gemv, simt, layouts, efficiency
constexpr SplitKind N = SplitKind::kNone, P = SplitKind::kPartial, A = SplitKind::kAtomic;
constexpr VariantInfo kInfo[] = {
    {"Fp32MfmaGemm_256x256", 256, 256, 16, 256, 1, true, N, false, false, false, 0.85},
    {"Fp32MfmaGemm_256x256_SplitK", 256, 256, 16, 256, 1, true, P, false, false, false, 0.25},
    {"Fp32MfmaGemm_256x128", 256, 128, 16, 256, 2, true, N, false, false, false, 0.84},
    {"Fp32MfmaGemm_128x128", 128, 128, 16, 256, 3, true, N, false, false, true, 0.865},
    {"Fp32MfmaGemm_128x128_SplitK", 128, 128, 16, 256, 3, true, P, false, false, true, 0.55},
    {"Fp32MfmaGemm_64x256", 64, 256, 16, 256, 2, true, N, false, false, false, 0.76},
    {"Fp32MfmaGemm_64x256_SplitK", 64, 256, 16, 256, 2, true, P, false, false, false, 0.55},
    {"Fp32MfmaGemm_256x64", 256, 64, 16, 256, 2, true, N, false, false, false, 0.76},
    {"Fp32MfmaGemm_256x64_SplitK", 256, 64, 16, 256, 2, true, P, false, false, false, 0.55},
    {"Fp32MfmaGemm_64x64", 64, 64, 16, 256, 4, true, N, false, false, true, 0.50},
    {"Fp32MfmaGemm_64x64_SplitK", 64, 64, 16, 256, 4, true, P, false, false, true, 0.50},
    {"Fp32MfmaGemm_128x128_Unaligned", 128, 128, 16, 256, 2, false, N, false, false, true, 0.70},
    {"Fp32MfmaGemm_128x128_Unaligned_SplitK", 128, 128, 16, 256, 2, false, P, false, false, true, 0.45},
    {"Fp32MfmaGemm_64x64_Unaligned", 64, 64, 16, 256, 4, false, N, false, false, true, 0.45},
    {"Fp32Gemv_SplitK", kGemvRows, kGemvCols, 1, 256, 8, true, A, true, false, false, 0.0},
    {"Fp32Gemv_Unaligned_SplitK", kGemvRows, kGemvCols, 1, 256, 8, false, A, true, false, false, 0.0},
    {"Fp32Gemm", 64, 64, 16, 256, 2, false, N, false, true, true, 0.20},
};
static_assert(sizeof(kInfo) / sizeof(kInfo[0]) == static_cast<int>(Variant::kCount), "catalog");

}  // namespace

const VariantInfo& info(Variant v) { return kInfo[static_cast<int>(v)]; }

}  // namespace ftrain::gemm

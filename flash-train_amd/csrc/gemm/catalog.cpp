// Static description of every kernel variant: its Primitive name, tile
// geometry and the figures the Finder's cost model uses.
#include "ft/gemm_kernels.hpp"

namespace ftrain::gemm {
namespace {

// name, bm, bn, bk, threads, occupancy, vec, split, gemv, simt, layouts, efficiency, input type,
// MFMA FLOP/clk/CU (fp32 256; bf16/fp16 4096, the 2.5 PFLOP/s dense peak over 256 CUs at 2.4 GHz),
// efficiency with one resident workgroup.  The fp32 efficiencies are fitted to Primitive timings
// on MI355X (every applicable Primitive over 25 shapes from 64x4096x4096 to 16384x14336x4096,
// random N(0,1) inputs, best of 3 interleaved passes): the squared log error of the modelled
// time of every Primitive within 1.35x of a shape's best, plus the time lost by the top pick
// (the headline and skinny shapes weighted 3x).  The DMA tiles' figures were then refitted with
// the split-k Primitives also timed at forced split counts 2 .. 128 on 18 skinny, deep-k and square
// shapes (the reduction reading every split's slice in flight, non-temporal partial stores): the
// top pick, with its own split count, loses 0.8% on average against the fastest measured
// (Primitive, split count) and 5.2% at most (512x512x8192), against 2.2% and 10.8% before.
// The 16-bit efficiencies are set by hand so that the ranking matches measured timings from
// 1024^3 to 8192^3 in every layout (the 64x64 tile loses to 128x128 from 1024^3 on, 128x128
// to the 256x256 tiles from 3072^3 on), in grouped MoE shapes with 8 and 64 experts, and in
// deep-k shapes where split-k wins (384x4096x4096, 512x512x8192, 1536x1536x8192); the 128x128
// DMA tiles' figures pick the fastest Primitive on each of 14 bf16 shapes from 64x4096x4096 to
// 16384x14336x4096 (one box).
constexpr SplitKind N = SplitKind::kNone, P = SplitKind::kPartial, F = SplitKind::kFused;
constexpr FTrainNumericType FP32 = FTRAIN_NUMERIC_TYPE_FP32, BF16 = FTRAIN_NUMERIC_TYPE_BF16,
                            FP16 = FTRAIN_NUMERIC_TYPE_FP16;
constexpr VariantInfo kInfo[] = {
    {"Fp32Mfma16Gemm_256x256_Dma", 256, 256, 32, 256, 1, true, N, false, false, false, 0.965, FP32, 256.0, 0.965},
    {"Fp32Mfma16Gemm_256x256_Dma_SplitK", 256, 256, 32, 256, 1, true, P, false, false, false, 0.957, FP32, 256.0, 0.957},
    {"Fp32Mfma16Gemm_128x128_Dma", 128, 128, 32, 256, 2, true, N, false, false, false, 0.982, FP32, 256.0, 0.956},
    {"Fp32Mfma16Gemm_128x128_Dma_SplitK", 128, 128, 32, 256, 2, true, P, false, false, false, 0.990, FP32, 256.0, 0.974},
    {"Fp32Mfma16Gemm_64x256_Dma_SplitK", 64, 256, 32, 256, 2, true, P, false, false, false, 0.958, FP32, 256.0, 0.915},
    {"Fp32Mfma16Gemm_256x64_Dma_SplitK", 256, 64, 32, 256, 2, true, P, false, false, false, 0.984, FP32, 256.0, 0.984},
    {"Fp32Mfma16Gemm_64x128_Dma_SplitK", 64, 128, 32, 256, 3, true, P, false, false, false, 0.961, FP32, 256.0, 0.893},
    {"Fp32Mfma16Gemm_128x64_Dma_SplitK", 128, 64, 32, 256, 3, true, P, false, false, false, 0.939, FP32, 256.0, 0.957},
    {"Fp32Mfma16Gemm_64x64_Dma_SplitK", 64, 64, 32, 256, 5, true, P, false, false, false, 0.964, FP32, 256.0, 0.846},
    {"Fp32Mfma16Gemm_64x128_Dma", 64, 128, 32, 256, 3, true, N, false, false, false, 0.966, FP32, 256.0, 0.933},
    {"Fp32Mfma16Gemm_128x64_Dma", 128, 64, 32, 256, 3, true, N, false, false, false, 0.933, FP32, 256.0, 0.934},
    {"Fp32Mfma16Gemm_256x256", 256, 256, 16, 256, 1, true, N, false, false, true, 0.903, FP32, 256.0, 0.903},
    {"Fp32Mfma16Gemm_256x256_SplitK", 256, 256, 16, 256, 1, true, P, false, false, true, 0.842, FP32, 256.0, 0.842},
    {"Fp32Mfma16Gemm_256x128", 256, 128, 16, 256, 2, true, N, false, false, true, 0.891, FP32, 256.0, 0.821},
    {"Fp32Mfma16Gemm_256x128_SplitK", 256, 128, 16, 256, 2, true, P, false, false, true, 0.905, FP32, 256.0, 0.836},
    {"Fp32Mfma16Gemm_128x256", 128, 256, 16, 256, 2, true, N, false, false, true, 0.892, FP32, 256.0, 0.819},
    {"Fp32Mfma16Gemm_64x256", 64, 256, 16, 256, 2, true, N, false, false, true, 0.861, FP32, 256.0, 0.789},
    {"Fp32Mfma16Gemm_64x256_SplitK", 64, 256, 16, 256, 2, true, P, false, false, true, 0.829, FP32, 256.0, 0.810},
    {"Fp32Mfma16Gemm_256x64", 256, 64, 16, 256, 2, true, N, false, false, true, 0.869, FP32, 256.0, 0.776},
    {"Fp32Mfma16Gemm_256x64_SplitK", 256, 64, 16, 256, 2, true, P, false, false, true, 0.854, FP32, 256.0, 0.747},
    {"Fp32MfmaGemm_256x256", 256, 256, 16, 256, 1, true, N, false, false, false, 0.853, FP32, 256.0, 0.853},
    {"Fp32MfmaGemm_256x256_SplitK", 256, 256, 16, 256, 1, true, P, false, false, false, 0.848, FP32, 256.0, 0.848},
    {"Fp32MfmaGemm_256x128", 256, 128, 16, 256, 2, true, N, false, false, false, 0.854, FP32, 256.0, 0.791},
    {"Fp32MfmaGemm_128x128", 128, 128, 16, 256, 3, true, N, false, false, true, 0.867, FP32, 256.0, 0.749},
    {"Fp32MfmaGemm_128x128_SplitK", 128, 128, 16, 256, 3, true, P, false, false, true, 0.888, FP32, 256.0, 0.792},
    {"Fp32MfmaGemm_64x256", 64, 256, 16, 256, 2, true, N, false, false, false, 0.791, FP32, 256.0, 0.640},
    {"Fp32MfmaGemm_64x256_SplitK", 64, 256, 16, 256, 2, true, P, false, false, false, 0.782, FP32, 256.0, 0.687},
    {"Fp32MfmaGemm_256x64", 256, 64, 16, 256, 2, true, N, false, false, false, 0.812, FP32, 256.0, 0.735},
    {"Fp32MfmaGemm_256x64_SplitK", 256, 64, 16, 256, 2, true, P, false, false, false, 0.787, FP32, 256.0, 0.720},
    {"Fp32MfmaGemm_64x64", 64, 64, 16, 256, 4, true, N, false, false, true, 0.720, FP32, 256.0, 0.571},
    {"Fp32MfmaGemm_64x64_SplitK", 64, 64, 16, 256, 4, true, P, false, false, true, 0.704, FP32, 256.0, 0.632},
    {"Fp32MfmaGemm_128x128_Unaligned", 128, 128, 16, 256, 2, false, N, false, false, true, 0.654, FP32, 256.0, 0.658},
    {"Fp32MfmaGemm_128x128_Unaligned_SplitK", 128, 128, 16, 256, 2, false, P, false, false, true, 0.683, FP32, 256.0, 0.590},
    {"Fp32MfmaGemm_64x64_Unaligned", 64, 64, 16, 256, 4, false, N, false, false, true, 0.678, FP32, 256.0, 0.469},
    {"Fp32Gemv", kGemvRows, kGemvPassCols, 1, 1024, 1, true, N, true, false, false, 0, FP32, 256.0, 0},
    {"Fp32Gemv_SplitK", kGemvRows, kGemvCols, 1, 256, 8, true, P, true, false, false, 0, FP32, 256.0, 0},
    {"Fp32Gemv_Unaligned_SplitK", kGemvRows, kGemvCols, 1, 256, 8, false, P, true, false, false, 0, FP32, 256.0, 0},
    {"Fp32Mfma16Gemm_64x64_DeepK", 64, 64, 32, 256, 1, true, F, false, false, false, 0.698, FP32, 256.0, 0.698},
    {"Fp32Gemm", 64, 64, 16, 256, 2, false, N, false, true, true, 0.2, FP32, 256.0, 0.2},
    {"Bf16MfmaGemm_256x256", 256, 256, 64, 512, 1, true, N, false, false, true, 0.6, BF16, 4096.0, 0.6},
    {"Bf16MfmaGemm_128x128", 128, 128, 64, 256, 2, true, N, false, false, true, 0.4, BF16, 4096.0, 0.4},
    {"Bf16MfmaGemm_128x128_SplitK", 128, 128, 64, 256, 2, true, P, false, false, true, 0.42, BF16, 4096.0, 0.3},
    {"Bf16MfmaGemm_64x64_Unaligned", 64, 64, 32, 256, 2, false, N, false, false, true, 0.08, BF16, 4096.0, 0.08},
    {"Fp16MfmaGemm_256x256", 256, 256, 64, 512, 1, true, N, false, false, true, 0.6, FP16, 4096.0, 0.6},
    {"Fp16MfmaGemm_128x128", 128, 128, 64, 256, 2, true, N, false, false, true, 0.4, FP16, 4096.0, 0.4},
    {"Fp16MfmaGemm_128x128_SplitK", 128, 128, 64, 256, 2, true, P, false, false, true, 0.42, FP16, 4096.0, 0.3},
    {"Fp16MfmaGemm_64x64_Unaligned", 64, 64, 32, 256, 2, false, N, false, false, true, 0.08, FP16, 4096.0, 0.08},
    {"Bf16MfmaGemm_256x256_Dma", 256, 256, 64, 256, 1, true, N, false, false, true, 0.66, BF16, 4096.0, 0.66},
    {"Fp16MfmaGemm_256x256_Dma", 256, 256, 64, 256, 1, true, N, false, false, true, 0.66, FP16, 4096.0, 0.66},
    {"Bf16MfmaGemm_128x128_Dma", 128, 128, 64, 256, 2, true, N, false, false, true, 0.48, BF16, 4096.0, 0.45},
    {"Bf16MfmaGemm_128x128_Dma_SplitK", 128, 128, 64, 256, 2, true, P, false, false, true, 0.55, BF16, 4096.0, 0.45},
    {"Fp16MfmaGemm_128x128_Dma", 128, 128, 64, 256, 2, true, N, false, false, true, 0.48, FP16, 4096.0, 0.45},
    {"Fp16MfmaGemm_128x128_Dma_SplitK", 128, 128, 64, 256, 2, true, P, false, false, true, 0.55, FP16, 4096.0, 0.45},
    // Applicable to m of at most 64 only.  The low single-workgroup figure makes the model spread
    // such a problem over 8 splits (one workgroup per CU), as measured (64x4096x4096: 4 splits
    // leave half the CUs idle).
    {"Bf16MfmaGemm_64x128_Dma_SplitK", 64, 128, 64, 256, 2, true, P, false, false, true, 0.52, BF16, 4096.0, 0.35},
    {"Fp16MfmaGemm_64x128_Dma_SplitK", 64, 128, 64, 256, 2, true, P, false, false, true, 0.52, FP16, 4096.0, 0.35},
    {"Bf16Gemv", kGemvHalfRows, kGemvHalfCols, 1, 1024, 1, true, N, true, false, false, 0, BF16, 4096.0, 0},
    {"Fp16Gemv", kGemvHalfRows, kGemvHalfCols, 1, 1024, 1, true, N, true, false, false, 0, FP16, 4096.0, 0},
};
static_assert(sizeof(kInfo) / sizeof(kInfo[0]) == static_cast<int>(Variant::kCount), "catalog");

}  // namespace

const VariantInfo& info(Variant v) { return kInfo[static_cast<int>(v)]; }

}  // namespace ftrain::gemm

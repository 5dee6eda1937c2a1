// Kernel catalog shared by the HIP translation unit (which defines the
// kernels) and the host Primitives (which launch them).
//
// Every kernel computes d = alpha * (a @ b) + beta * c on fp32 matrices
// (a: m x k, b: k x n, c/d: m x n), the semantics of the reference kernel
// (src/primitive/hygon/gemm/fp32_gemm.hip:18-31): with a null c the beta term
// is dropped, with a non-null c it is always evaluated (so 0 * NaN
// propagates).  The reference takes row-major contiguous matrices only;
// here a and b may each be row- or column-major with a leading dimension,
// and c and d row-major with their own row strides (a column-major d is
// computed as d^T = b^T a^T by the host).
#pragma once

#include <cstdint>

#include <flash_train/common.h>

namespace ftrain::gemm {

// Kernel parameters, passed by value.  Dimensions are 32-bit (Primitives
// that launch these kernels require m, n, k < 2^31); element offsets are
// computed in 64 bits inside the kernels.
struct GemmParams {
    const float* a;
    const float* b;
    const float* c;  // may be null
    float* d;
    float alpha;
    float beta;
    int32_t m, n, k;
    int32_t k_chunk;  // reduction depth per split (a multiple of the kernel's BK); == k when not split
    int32_t tiles_m, tiles_n;
    // Leading dimensions in elements: the stride between rows of a row-major
    // matrix or between columns of a column-major one (the kernel's TA / TB
    // template flags say which).  c and d are row-major.
    int64_t lda, ldb, ldc, ldd;
};

// 64-bit parameters for the general SIMT kernel.  Element (i, j) of a sits at
// a[i*a_rs + j*a_cs], likewise b; c and d are row-major with row strides ldc
// and ldd.
struct WideParams {
    const float* a;
    const float* b;
    const float* c;
    float* d;
    float alpha;
    float beta;
    uint64_t m, n, k;
    int64_t a_rs, a_cs, b_rs, b_cs, ldc, ldd;
};

// Parameters of the bf16 / fp16 MFMA kernels (inputs a, b in the variant's
// 16-bit type, fp32 accumulation; c and d in fp32 or the input type).
struct HalfGemmParams {
    const void* a;
    const void* b;
    const void* c;  // may be null
    void* d;        // d, or the fp32 partial slices of a split-k variant
    float alpha;
    float beta;
    int32_t m, n, k;
    int32_t k_chunk;
    int32_t tiles_m, tiles_n;
    int64_t lda, ldb, ldc, ldd;  // as in GemmParams
    int32_t cd_half;             // c and d hold the input type (else fp32)
};

// Parameters of the deep-k kernel (gemm/deepk_tile.hpp): the tile problem,
// and for splits > 1 the partial slots (splits x tiles x 4096 floats) and
// one arrival counter per output tile (0 when a launch starts; each launch
// leaves them 0).
struct DeepKParams {
    GemmParams g;
    float* partials;
    unsigned int* counters;
    int32_t splits;
};

// Grouped GEMM launch arguments: a device table of per-group parameters
// (non-empty groups only) and each group's first workgroup, ascending.
struct GroupedGemmArgs {
    const GemmParams* params;
    const int32_t* tile_start;
    int32_t groups;
};
struct GroupedHalfArgs {
    const HalfGemmParams* params;
    const int32_t* tile_start;
    int32_t groups;
};

// Element type of c and d in the split-k reduction.
enum CdType : int32_t { kCdFp32 = 0, kCdBf16 = 1, kCdFp16 = 2 };

// Parameters of the split-k reduction (d = alpha * sum_z partials[z] + beta*c).
struct ReduceParams {
    const float* partials;  // splits dense m x n fp32 slices of count elements
    const void* c;          // may be null; element type cd_type
    void* d;                // element type cd_type
    float alpha;
    float beta;
    uint64_t count;  // m * n
    uint64_t n;      // columns (the row length of a partial slice)
    int64_t ldc, ldd;
    int32_t splits;
    int32_t cd_type;  // CdType
};

// Skinny-m kernel geometry: at most kGemvRows rows of a, kGemvCols output
// columns per workgroup.
constexpr int kGemvRows = 8;
constexpr int kGemvCols = 256;
// Columns per workgroup of the one-pass skinny kernels (128 bytes of a b
// row): fp32 and 16-bit inputs.
constexpr int kGemvPassCols = 32;
constexpr int kGemvHalfCols = 64;
// Rows of a the 16-bit one-pass kernel takes.  Measured on MI355X, bf16, us, against the
// 64x128 DMA split-k tile: one row 9.0 / 4.6 / 23.9 against 9.1 / 7.3 / 25.4 (4096^2, 2048^2,
// 8192^2), two rows 10.7 / 5.8 / 26.2 against 9.1 / 7.2 / 25.8, four rows 17.9 / 10.1 / 31.0
// against 9.2 / 7.5 / 26.5.
constexpr int kGemvHalfRows = 2;

enum class Variant : int {
    // v_mfma_f32_16x16x4_f32 256x256 tiles, 4 waves of 128x128 (one per
    // SIMD), 128-bit loads, every operand orientation; whole-k and split-k.
    // fp32 tiles with operands staged into LDS by DMA (global_load_lds_dwordx4),
    // v_mfma_f32_16x16x4_f32: row-major a and b, k a multiple of 32, any m and
    // n; 256x256 (one workgroup per CU) and 128x128 whole-k, and split-k forms.
    kMfma16Dma256x256,
    kMfma16Dma256x256S,
    kMfma16Dma128x128,
    kMfma16Dma128x128S,
    kMfma16Dma64x256S,
    kMfma16Dma256x64S,
    kMfma16Dma64x128S,
    kMfma16Dma128x64S,
    kMfma16Dma64x64S,
    kMfma16Dma64x128,
    kMfma16Dma128x64,
    kMfma16_256x256,
    kMfma16_256x256S,
    // Same instruction, 256x128 tiles of 4 waves of 128x64, two workgroups
    // per CU, plain stage loop.
    kMfma16_256x128,
    kMfma16_256x128S,
    // 128x256 tiles of 4 waves of 64x128 (m padded to 128 rows only).
    kMfma16_128x256,
    // Skinny 64x256 / 256x64 tiles (4 waves of 64x64, two workgroups per CU),
    // whole-k and split-k.
    kMfma16_64x256,
    kMfma16_64x256S,
    kMfma16_256x64,
    kMfma16_256x64S,
    // MFMA tiles, 128-bit global loads (needs k % 4 == 0, n % 4 == 0 and
    // 16-byte aligned a/b/c/d).  Suffix S = split-k: per-split partial tiles
    // to a workspace, then a deterministic reduction kernel.
    kMfma256x256,
    kMfma256x256S,
    kMfma256x128,
    kMfma128x128,
    kMfma128x128S,
    kMfma64x256,
    kMfma64x256S,
    kMfma256x64,
    kMfma256x64S,
    kMfma64x64,
    kMfma64x64S,
    // MFMA tiles with per-element loads/stores: any shape, 4-byte alignment.
    kMfma128x128U,
    kMfma128x128US,
    kMfma64x64U,
    // Skinny m (<= 8), 128-bit loads of b: one pass, 32 columns per
    // workgroup over all of k, reduced in the workgroup in a fixed order.
    kGemv,
    // Skinny m (<= 8): streaming split-k, partial slices reduced by
    // splitk_reduce in a fixed order.
    kGemvS,
    kGemvUS,
    // Deep-k 64x64 tiles (v_mfma_f32_16x16x4_f32, 4 waves splitting k,
    // operands streamed from global memory into registers), split-k reduced
    // inside the launch by the last-arriving workgroup of each tile.
    // Row-major a and b only.
    kDeepK64x64,
    // General SIMT kernel with 64-bit indexing.
    kSimt,
    // bf16 and fp16 inputs, fp32 accumulation (v_mfma_f32_32x32x16_*):
    // 16-byte loads (k, leading dimensions and contiguous extents multiples
    // of 8), except the _Unaligned tile (per-element loads, any shape).
    kBf16Mfma256x256,
    kBf16Mfma128x128,
    kBf16Mfma128x128S,
    kBf16Mfma64x64U,
    kFp16Mfma256x256,
    kFp16Mfma128x128,
    kFp16Mfma128x128S,
    kFp16Mfma64x64U,
    // bf16 / fp16 256x256 tiles with operands staged into LDS by DMA
    // (global_load_lds_dwordx4): k a multiple of 64, any m and n.
    kBf16MfmaDma256x256,
    kFp16MfmaDma256x256,
    // bf16 / fp16 128x128 DMA-staged tiles (two workgroups per CU), whole-k and split-k.
    kBf16MfmaDma128x128,
    kBf16MfmaDma128x128S,
    kFp16MfmaDma128x128,
    kFp16MfmaDma128x128S,
    // bf16 / fp16 64x128 DMA-staged split-k tiles (m of at most 64; row-major a).
    kBf16MfmaDma64x128S,
    kFp16MfmaDma64x128S,
    // One-pass skinny-m kernels (m <= 8, row-major b) for bf16 / fp16 inputs.
    kBf16Gemv,
    kFp16Gemv,
    kCount
};

// Tile index of a half-precision variant inside its type's group (the
// order of the four variants above): 0 = 256x256, 1 = 128x128,
// 2 = 128x128 split-k, 3 = 64x64 per-element.
constexpr int kHalfTiles = 4;

enum class SplitKind : int {
    kNone,     // one workgroup owns each output tile's whole reduction
    kPartial,  // partial tiles to a workspace, then splitk_reduce (fixed order)
    kFused,    // partial tiles to a workspace, summed by the tile's last workgroup in the same launch
};

struct VariantInfo {
    const char* name;  // Primitive name (the FTRAIN_*_PRIMITIVES filter key)
    int bm, bn, bk;    // output tile and reduction step (gemv: bm = max rows, bn = columns per workgroup)
    int threads;       // workgroup size
    int occupancy;     // workgroups expected to share one CU
    bool vec;          // needs 16-byte alignment and n % 4 == 0, k % 4 == 0
    SplitKind split;
    bool gemv;
    bool simt;
    bool layouts;       // instantiated for column-major a and b as well (else row-major a and b only)
    double efficiency;        // sustained fraction of the MFMA rate with `occupancy` workgroups resident per CU
    FTrainNumericType input;  // element type of a and b
    double flop_per_clk;      // dense MFMA FLOP per clock per CU for that type
    double solo_efficiency;   // the same with a single resident workgroup (equal to efficiency when occupancy is 1)
};

// Largest split-k workspace (partial tiles) a Primitive will use.
constexpr uint64_t kMaxPartialBytes = 256ull << 20;

// Every split-k buffer (a Plan's own, a caller's workspace, the device
// scratch array) starts with this many bytes of per-tile arrival counters
// for the kFused kernels; partial tiles follow.  The split kernels of every
// kind leave the region alone, so a buffer shared by several Primitives
// keeps its counters.
constexpr uint64_t kCounterBytes = 16384;
constexpr uint64_t kMaxFusedTiles = kCounterBytes / 4;

const VariantInfo& info(Variant v);

// Device entry points (host-side stubs registered by the HIP TUs).
// kernelFor: the variant's kernel for a column-major (ta) or row-major a and
// a column-major (tb) or row-major b; null when that layout is not
// instantiated for the variant (see VariantInfo::layouts).
// prefetch_b: the 256x256 16-bit DMA tiles take their form that prefetches b into L2 ahead of its
// DMA (prefetchB decides).
const void* kernelFor(Variant v, bool ta = false, bool tb = false, bool prefetch_b = false);
// The one-pass skinny kernels (Variant::kGemv, kBf16Gemv, kFp16Gemv) for m
// rows of a (up to the variant's row limit) and a row-major (ta false) or,
// fp32 only, column-major a; null otherwise.  `threads` receives the
// workgroup size, gemvPassThreads(m).  b is row-major.
int gemvPassThreads(int m);
const void* gemvKernel(Variant v, int m, bool ta, int& threads);
const void* gemvHalfKernel(bool bf16, int m);
// Per-layout instantiations of the layout-capable MFMA variants (one HIP TU
// each); null for other variants.
const void* layoutKernelTN(Variant v);  // column-major a, row-major b
const void* layoutKernelNT(Variant v);  // row-major a, column-major b
const void* layoutKernelTT(Variant v);  // both column-major
// FP32 16x16x4 tiles (0 = whole-k, 1 = split-k) per operand orientation.
const void* mfma16KernelNN(int which);
const void* mfma16KernelTN(int which);
const void* mfma16KernelNT(int which);
const void* mfma16KernelTT(int which);
// Half-precision tiles (index 0..kHalfTiles-1) per input type and operand
// orientation, one HIP TU each.
const void* halfKernelBf16NN(int tile);
const void* halfKernelBf16TN(int tile);
const void* halfKernelBf16NT(int tile);
const void* halfKernelBf16TT(int tile);
const void* halfKernelFp16NN(int tile);
const void* halfKernelFp16TN(int tile);
const void* halfKernelFp16NT(int tile);
const void* halfKernelFp16TT(int tile);
// The DMA-staged 256x256 tiles per input type and operand orientation.
const void* dma32Kernel(Variant v);
const void* groupedDma32Kernel();
const void* groupedDma32Kernel128(bool ta, bool tb);  // grouped 128x128 DMA tile, any orientation
const void* groupedDma32Kernel64x128(bool tb);        // grouped 64x128 DMA tile, row-major a
const void* dma32KernelTB(Variant v);  // column-major b
const void* dma32KernelTA(Variant v, bool tb);  // column-major a
// prefetch_b: the form that prefetches b into L2 ahead of its DMA.
const void* dmaKernelBf16(bool ta, bool tb, bool prefetch_b);
const void* dmaKernelFp16(bool ta, bool tb, bool prefetch_b);
const void* dma128KernelBf16(bool ta, bool tb, bool split);
const void* dma128KernelFp16(bool ta, bool tb, bool split);
const void* dma64x128KernelBf16(bool ta, bool tb);  // null for a column-major a
const void* dma64x128KernelFp16(bool ta, bool tb);
const void* groupedDmaKernelBf16(bool ta, bool tb, bool prefetch_b);
const void* groupedDmaKernelFp16(bool ta, bool tb, bool prefetch_b);
const void* groupedDma128KernelBf16(bool ta, bool tb);
const void* groupedDma128KernelFp16(bool ta, bool tb);
// Grouped kernels: element type (FTRAIN_NUMERIC_TYPE_FP32 / BF16 / FP16),
// tile (0 = 128x128 with 16-byte loads, 1 = 64x64 per-element, 2 = the
// family's large tile: fp32 16x16x4 256x128, bf16/fp16 256x256; 3 = fp32
// 16x16x4 128x256) and operand
// orientation.
const void* groupedKernelFor(FTrainNumericType input, int which, bool ta, bool tb, bool prefetch_b = false);

// When the 256x256 16-bit DMA tiles prefetch b into L2 (bf16, MI355X, against the same tile
// without it): b (every group's together for a grouped launch) larger than the 256 MB MALL, and k
// at most kPrefetchMaxK; a grouped launch also needs at least a band of 8 tile rows per group on
// average.  Measured: plain 2048x114688x4096 -8%, 4096x65536x4096 -7.5%, 1024x131072x4096 -9.5%,
// 8192x32768x4096, 16384x16384x8192 and 8192x65536x2048 within 1%, but 4096x4096x65536 +4%;
// grouped 8 experts of 2048 rows (k 4096) -1 to -2.5%, 16 or more experts (4 tile rows or fewer
// each) +2 to +35%, 8 experts of 4096 rows at k 14336 +5%.
constexpr uint64_t kLargeBBytes  = 256ull << 20;
constexpr uint64_t kPrefetchMaxK = 8192;
inline bool prefetchB(uint64_t b_bytes, uint64_t max_k, double tile_rows_per_group = 8.0) {
    return b_bytes > kLargeBBytes && max_k <= kPrefetchMaxK && tile_rows_per_group >= 8.0;
}
const void* groupedKernelNN(int which);
const void* groupedKernelTN(int which);
const void* groupedKernelNT(int which);
const void* groupedKernelTT(int which);
const void* groupedHalfKernelBf16NN(int which);
const void* groupedHalfKernelBf16TN(int which);
const void* groupedHalfKernelBf16NT(int which);
const void* groupedHalfKernelBf16TT(int which);
const void* groupedHalfKernelFp16NN(int which);
const void* groupedHalfKernelFp16TN(int which);
const void* groupedHalfKernelFp16NT(int which);
const void* groupedHalfKernelFp16TT(int which);
// Split-k reduction (ReduceParams); wide: one thread per output unit (outputs
// with at least kWideReduceUnits units, or at most 8 splits), else 16 threads
// per unit.
const void* reduceKernel(bool vec, bool wide);
constexpr uint64_t kWideReduceUnits = 256 * 1024;
const void* deepkKernel();              // kDeepK64x64 (DeepKParams)
const void* deepkClearKernel();         // zeroes (unsigned*, int n) arrival counters

}  // namespace ftrain::gemm

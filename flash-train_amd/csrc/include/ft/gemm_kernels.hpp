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

// 64-bit parameters for the general SIMT kernel, the skinny kernel's
// operand reads and the elementwise prologue.  Element (i, j) of a sits at
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

// Parameters of the split-k reduction (d = alpha * sum_z partials[z] + beta*c).
struct ReduceParams {
    const float* partials;  // splits dense m x n slices of count floats
    const float* c;         // may be null
    float* d;
    float alpha;
    float beta;
    uint64_t count;  // m * n
    uint64_t n;      // columns (the row length of a partial slice)
    int64_t ldc, ldd;
    int32_t splits;
};

// Skinny-m kernel geometry: at most kGemvRows rows of a, kGemvCols output
// columns per workgroup.
constexpr int kGemvRows = 8;
constexpr int kGemvCols = 256;

enum class Variant : int {
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
    // Skinny m (<= 8): streaming GEMV-style split-k with atomic accumulation.
    kGemvS,
    kGemvUS,
    // General SIMT kernel with 64-bit indexing.
    kSimt,
    kCount
};

enum class SplitKind : int {
    kNone,     // one workgroup owns each output tile's whole reduction
    kPartial,  // partial tiles to a workspace, then splitk_reduce
    kAtomic,   // beta*c prologue, then fp32 atomic adds
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
    double efficiency;  // fraction of the FP32 matrix peak the tile sustains (cost model)
};

// Largest split-k workspace (partial tiles) a Primitive will use.
constexpr uint64_t kMaxPartialBytes = 256ull << 20;

const VariantInfo& info(Variant v);

// Device entry points (host-side stubs registered by the HIP TUs).
// kernelFor: the variant's kernel for a column-major (ta) or row-major a and
// a column-major (tb) or row-major b; null when that layout is not
// instantiated for the variant (see VariantInfo::layouts).
const void* kernelFor(Variant v, bool ta = false, bool tb = false);
// Per-layout instantiations of the layout-capable MFMA variants (one HIP TU
// each); null for other variants.
const void* layoutKernelTN(Variant v);  // column-major a, row-major b
const void* layoutKernelNT(Variant v);  // row-major a, column-major b
const void* layoutKernelTT(Variant v);  // both column-major
const void* prologueKernel();            // d = c ? beta*c : 0 over m*n elements (WideParams)
const void* reduceKernel(bool vec);      // split-k reduction (ReduceParams)

}  // namespace ftrain::gemm

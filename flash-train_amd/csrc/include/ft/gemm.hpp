// The GEMM family: problem description and validation, the supported
// Pattern, the Primitive catalog and the shape-ranking Finder.
//
// Reference counterparts:
//   GemmProblem            src/family/gemm/problem.cpp:13-91, src/include/flash_train/family/gemm/problem.hpp:35-118
//   GemmFamily             src/include/flash_train/family/gemm/family.hpp:20-72, src/family/gemm/family.cpp:13-15
//   Finder                 src/include/flash_train/family/gemm/finder.hpp:21-26 (placeholder there)
//   Fp32Gemm applicability src/primitive/hygon/gemm/fp32_gemm.cpp:27-62
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "ft/engine.hpp"
#include "ft/gemm_kernels.hpp"

namespace ftrain {

struct GemmShape {
    uint64_t m, n, k;
};

// How a rank-2 matrix view is laid out in memory: element (i, j) sits at
// i*ld + j (row-major) or i + j*ld (column-major).
struct MatrixLayout {
    bool col_major = false;
    int64_t ld     = 0;
};

// Returns nullptr and fills `out` when the view is a layout the kernels can
// read: FTRAIN_INDEX_TYPE_CONTINUOUS (row-major, ld = columns), or explicit
// non-negative strides with a unit stride in one dimension and a leading
// dimension that covers the other.  Otherwise returns the UNSUPPORTED reason.
// Explicit strides that restate the continuous layout are rejected, as the
// reference rejects every explicit-stride view
// (src/primitive/hygon/gemm/fp32_gemm.cpp:39-46): callers name that layout
// with the index type.
const char* matrixLayout(const StorageView& view, MatrixLayout& out);

// The problem rewritten for the kernels: a and b in either orientation, c
// and d row-major.  A column-major d is computed as d^T = b^T a^T (m and n
// swap, a and b swap and flip orientation).
struct GemmLaunch {
    GemmShape shape;
    const void* a;
    const void* b;
    const void* c;
    void* d;
    bool ta, tb;  // a / b column-major
    int64_t lda, ldb, ldc, ldd;
};

class GemmProblem {
  public:
    // Validates structure: rank-2 a/b/c/d, scalar alpha/beta, a/b/c/d in
    // device memory and alpha/beta in host memory (INVALID_ARGUMENT);
    // a.cols == b.rows, c and d shaped m x n (INVALID_ARGUMENT); every
    // matrix byte count fits uint64 (OVERFLOW).
    GemmProblem(Tensor a, Tensor b, Tensor c, Tensor d, Tensor alpha, Tensor beta, FTrainNumericType compute_type);

    GemmShape shape() const noexcept {
        return {static_cast<uint64_t>(a_.view.dims()[0]), static_cast<uint64_t>(b_.view.dims()[1]),
                static_cast<uint64_t>(a_.view.dims()[1])};
    }
    bool emptyOutput() const noexcept { return shape().m == 0 || shape().n == 0; }
    FTrainNumericType computeType() const noexcept { return compute_type_; }

    // Ports in the order a, b, c, d, alpha, beta.
    const StorageView& port(int i) const noexcept;
    const StorageView& a() const noexcept { return a_.view; }
    const StorageView& b() const noexcept { return b_.view; }
    const StorageView& c() const noexcept { return c_.view; }
    const StorageView& d() const noexcept { return d_.view; }
    const StorageView& alpha() const noexcept { return alpha_.view; }
    const StorageView& beta() const noexcept { return beta_.view; }
    bool inPlace() const noexcept { return c_.view.memory() == d_.view.memory(); }

    // Fills `out` and returns nullptr, or returns the UNSUPPORTED reason
    // (a matrix layout the kernels cannot read, or c and d in different
    // orientations).
    const char* launch(GemmLaunch& out) const;

    // Selection-cache tokens: everything that can change applicability or
    // the Finder's ranking -- per port: numeric type, index type, null-ness,
    // address modulo 16 (covers the 4-byte and 16-byte alignment rules),
    // rank, dims, strides -- then compute type and in-place.  Raw addresses
    // never enter.  Each field is preceded by a running field number and
    // variable-length fields by their length, so encodings cannot alias.
    std::vector<uint64_t> key() const;

  private:
    Tensor a_, b_, c_, d_, alpha_, beta_;
    FTrainNumericType compute_type_;
};

// Supported Pattern: six Tensors and one Gemm(a, b, c, alpha, beta -> d).
struct GemmFamily {
    using Problem = GemmProblem;
    struct Roles {
        Pattern pattern;
        uint64_t a, b, c, d, alpha, beta, gemm;
    };
    static const Roles& roles();
    static Pattern makePattern() { return roles().pattern; }
    static std::vector<std::shared_ptr<const Primitive<GemmProblem>>> makeRecords();
    static GemmProblem makeProblem(const Args& args);
};

// Ranks the catalog by a roofline cost model of each variant on the
// problem's shape (see gemm/finder.cpp).  Name: "ShapeCost".
struct ShapeCostFinder {
    static const char* name() { return "ShapeCost"; }
    static std::vector<std::string> candidates(const GemmProblem& problem, const Constraints& constraints);
};

namespace gemm {

// Split count a split-k variant uses for a shape on a device with `cus`
// compute units (>= 2), or 0 when the reduction is too shallow to split.
uint32_t chooseSplits(Variant v, const GemmShape& s, int cus);
// Test hook: with s > 0, every split-k variant takes s splits (clamped to what
// its workspace, counters and k allow) instead of the modelled choice; 0
// restores the model.  Process-wide.
void forceSplits(uint32_t s);

// Modelled execution time in microseconds (lower is better).
double estimateMicros(Variant v, const GemmShape& s, bool has_c, int cus);

// Compute units of `device` (cached; 256 when HIP cannot be queried).
int computeUnits(FTrainDeviceId device);

// Modelled microseconds of one grouped launch over the groups' (kernel-
// orientation) shapes with tile variant v.
double groupedMicros(Variant v, const std::vector<GemmShape>& shapes, bool has_c, int cus);

}  // namespace gemm

using GemmEngine = OpsEngine<GemmFamily, ShapeCostFinder>;

}  // namespace ftrain

// The grouped GEMM families: GroupedABCDGemm, GroupedBCDGemm, GroupedABGemm.
//
// Reference counterparts: the operation kinds and their operand storage
// families (src/include/flash_train/operation/gemm.hpp:80-150), the
// GroupedTensor value (src/include/flash_train/tensor.hpp:40-71) and its
// addressing rule (include/flash_train/common.h:397-425): element index[d]
// of group g sits offsets[g] + sum(index[d] * strides[d][g]) elements from
// data.memory, 0 <= index[d] < dim_sizes[d][g].  The reference ships no
// engine for these kinds.
//
// Here every group is one GEMM, d_g = alpha * (a_g @ b_g) + beta * c_g, with
// the element types, orientations and alpha/beta rules of the Gemm family.
// Operand forms:
//   GroupedABCDGemm: a, b, c, d GroupedTensors;
//   GroupedBCDGemm:  a a TensorList (one matrix per group), b, c, d grouped;
//   GroupedABGemm:   a, b grouped, c and d TensorLists.
// A GroupedTensor operand of a GEMM has rank-two data.  Its descriptor
// arrays are read at Plan creation and must be rank-one host arrays of
// int32, uint32, int64 or uint64:
//   dim_sizes: rows and columns of each group; absent: data.dims for every
//              group;
//   strides:   row and column strides of each group; absent: row-major,
//              contiguous (columns, 1);
//   offsets:   first element of each group; absent: the groups follow each
//              other contiguously (offset_g = sum of rows_h * cols_h, h < g).
// A GroupedTensor c with null data memory, or null TensorList c entries,
// drop the beta term for those groups.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "ft/engine.hpp"
#include "ft/gemm.hpp"

namespace ftrain {

enum class GroupedKind { kABCD, kBCD, kAB };

// One group's matrix: address, shape and layout.
struct GroupMatrix {
    const void* memory = nullptr;
    int64_t rows = 0, cols = 0;
    MatrixLayout layout;
};

// One operand over all groups.
struct GroupOperand {
    FTrainNumericType type = FTRAIN_NUMERIC_TYPE_INVALID;
    std::vector<GroupMatrix> groups;
};

class GroupedGemmProblem {
  public:
    // Expands the operands into per-group matrices and validates them:
    // INVALID_ARGUMENT for structural errors (group counts, ranks, per-group
    // shapes, placement, descriptor lengths or values), UNSUPPORTED for
    // descriptor placement or types this build cannot read, or a matrix
    // layout the kernels cannot read.
    GroupedGemmProblem(GroupedKind kind, const OperandValue& a, const OperandValue& b, const OperandValue& c,
                       const OperandValue& d, Tensor alpha, Tensor beta, FTrainNumericType compute_type);

    GroupedKind kind() const noexcept { return kind_; }
    uint32_t groups() const noexcept { return groups_; }
    const GroupOperand& a() const noexcept { return a_; }
    const GroupOperand& b() const noexcept { return b_; }
    const GroupOperand& c() const noexcept { return c_; }
    const GroupOperand& d() const noexcept { return d_; }
    const StorageView& alpha() const noexcept { return alpha_.view; }
    const StorageView& beta() const noexcept { return beta_.view; }
    FTrainNumericType computeType() const noexcept { return compute_type_; }
    bool emptyOutput(uint32_t g) const noexcept { return d_.groups[g].rows == 0 || d_.groups[g].cols == 0; }

    // Group g rewritten for the kernels as in GemmProblem::launch (a column-
    // major d becomes d^T = b^T a^T).  nullptr, or the UNSUPPORTED reason.
    const char* launch(uint32_t g, GemmLaunch& out) const;

    // Selection-cache tokens: kind, group count, element types, compute type,
    // and per group every shape, orientation, leading dimension, address
    // alignment and null-ness (never raw addresses).
    std::vector<uint64_t> key() const;

  private:
    GroupedKind kind_;
    uint32_t groups_ = 0;
    GroupOperand a_, b_, c_, d_;
    Tensor alpha_, beta_;
    FTrainNumericType compute_type_;
};

template <GroupedKind K>
struct GroupedGemmFamily {
    using Problem = GroupedGemmProblem;
    struct Roles {
        Pattern pattern;
        uint64_t a, b, c, d, alpha, beta, op;
    };
    static const Roles& roles();
    static Pattern makePattern() { return roles().pattern; }
    static std::vector<std::shared_ptr<const Primitive<GroupedGemmProblem>>> makeRecords();
    static GroupedGemmProblem makeProblem(const Args& args);
};

// Ranks the grouped variants of a's element type by the roofline model of
// one launch over all groups (gemm::groupedMicros).  Name: "GroupedCost".
struct GroupedCostFinder {
    static const char* name() { return "GroupedCost"; }
    static std::vector<std::string> candidates(const GroupedGemmProblem& problem, const Constraints& constraints);
};

// The three grouped engines (registered beside the Gemm engine).
std::vector<std::shared_ptr<OpsEngineBase>> groupedEngines();

}  // namespace ftrain

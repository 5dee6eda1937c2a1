// Argument values bound into Args: StorageView (one tensor's address and
// metadata), and the three operand storage families Tensor, TensorList,
// GroupedTensor.
//
// Validation rules follow the reference: StorageView
// (src/storage_view.cpp:9-52), GroupedTensor (src/tensor.cpp:9-62).  None of
// these types owns device or host memory.
#pragma once

#include <cstdint>
#include <optional>
#include <variant>
#include <vector>

#include <flash_train/common.h>

namespace ftrain {

class StorageView {
  public:
    // Copies dims/strides out of `view` after checking it.  Throws
    // INVALID_ARGUMENT when the numeric type is INVALID or out of range, the
    // index type is out of range, a scalar has null memory, dims is null for
    // a non-scalar, a dimension is negative, or strides and index_type do not
    // describe exactly one layout.
    explicit StorageView(const FTrainStorageView& view);

    void* memory() const noexcept { return memory_; }
    const std::vector<int64_t>& dims() const noexcept { return dims_; }
    const std::vector<int64_t>& strides() const noexcept { return strides_; }
    FTrainNumericType numericType() const noexcept { return numeric_type_; }
    FTrainIndexType indexType() const noexcept { return index_type_; }
    bool isHost() const noexcept { return is_host_; }
    std::size_t rank() const noexcept { return dims_.size(); }

  private:
    void* memory_;
    std::vector<int64_t> dims_;
    std::vector<int64_t> strides_;
    FTrainNumericType numeric_type_;
    FTrainIndexType index_type_;
    bool is_host_;
};

struct Tensor {
    StorageView view;
};

struct TensorList {
    std::vector<StorageView> views;
};

class GroupedTensor {
  public:
    // `dim_sizes` and `strides` are empty (not supplied) or hold rank(data)
    // rank-one views of num_groups entries; `offsets`, when present, is a
    // rank-one view of num_groups entries.  Violations throw
    // INVALID_ARGUMENT.
    GroupedTensor(uint32_t num_groups, StorageView data, std::optional<StorageView> offsets,
                  std::vector<StorageView> dim_sizes, std::vector<StorageView> strides);

    uint32_t numGroups() const noexcept { return num_groups_; }
    const StorageView& data() const noexcept { return data_; }
    const std::optional<StorageView>& offsets() const noexcept { return offsets_; }
    const std::vector<StorageView>& dimSizes() const noexcept { return dim_sizes_; }
    const std::vector<StorageView>& strides() const noexcept { return strides_; }

  private:
    uint32_t num_groups_;
    StorageView data_;
    std::optional<StorageView> offsets_;
    std::vector<StorageView> dim_sizes_;
    std::vector<StorageView> strides_;
};

// Storage family of a Pattern operand; the alternative index of
// OperandValue follows this order.
enum class OperandKind : uint8_t { kTensor = 0, kTensorList = 1, kGroupedTensor = 2 };
using OperandValue = std::variant<Tensor, TensorList, GroupedTensor>;

// Operation kinds and their per-call attributes (all four carry only a
// compute type, reference src/include/flash_train/operation/gemm.hpp:16-60).
enum class OperationKind : uint16_t { kGemm = 0, kGroupedABCDGemm = 1, kGroupedBCDGemm = 2, kGroupedABGemm = 3 };
struct OperationAttributes {
    OperationKind kind;
    FTrainNumericType compute_type;
};

}  // namespace ftrain

#include "ft/values.hpp"

#include "ft/error.hpp"

namespace ftrain {

StorageView::StorageView(const FTrainStorageView& view)
    : memory_(view.memory), numeric_type_(view.numeric_type), index_type_(view.index_type),
      is_host_(view.is_host_memory) {
    if (numeric_type_ == FTRAIN_NUMERIC_TYPE_INVALID || numeric_type_ >= FTRAIN_NUMERIC_TYPE_COUNT)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "StorageView numeric_type %u is invalid",
                        unsigned(numeric_type_));
    if (index_type_ >= FTRAIN_INDEX_TYPE_COUNT)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "StorageView index_type %u is unknown", unsigned(index_type_));
    const std::size_t rank = view.num_dims;
    if (rank == 0 && view.memory == nullptr)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "StorageView memory must not be null for a scalar");
    if (rank != 0 && view.dims == nullptr)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "StorageView dims must not be null when num_dims is %zu",
                        rank);
    const bool has_strides = view.strides != nullptr;
    const bool predefined  = index_type_ != FTRAIN_INDEX_TYPE_INVALID;
    if (!has_strides && !predefined)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "StorageView requires strides or a non-invalid index_type");
    if (has_strides && predefined)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                        "StorageView strides must be null when index_type %u defines a predefined layout",
                        unsigned(index_type_));
    for (std::size_t i = 0; i < rank; ++i) {
        if (view.dims[i] < 0)
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "StorageView dimension %zu must be non-negative, got %lld",
                            i, static_cast<long long>(view.dims[i]));
    }
    if (rank == 0) return;
    dims_.assign(view.dims, view.dims + rank);
    if (has_strides) strides_.assign(view.strides, view.strides + rank);
}

namespace {

void checkGroupArray(const StorageView& view, uint32_t num_groups, const char* what, std::size_t index) {
    if (view.rank() != 1)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "GroupedTensor %s[%zu] rank %zu must be 1", what, index,
                        view.rank());
    if (view.dims()[0] != static_cast<int64_t>(num_groups))
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "GroupedTensor %s[%zu] length %lld must match num_groups %u",
                        what, index, static_cast<long long>(view.dims()[0]), num_groups);
}

}  // namespace

GroupedTensor::GroupedTensor(uint32_t num_groups, StorageView data, std::optional<StorageView> offsets,
                             std::vector<StorageView> dim_sizes, std::vector<StorageView> strides)
    : num_groups_(num_groups), data_(std::move(data)), offsets_(std::move(offsets)),
      dim_sizes_(std::move(dim_sizes)), strides_(std::move(strides)) {
    const std::size_t rank = data_.rank();
    if (!dim_sizes_.empty() && dim_sizes_.size() != rank)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                        "GroupedTensor dim_sizes count %zu must be zero or match data rank %zu", dim_sizes_.size(),
                        rank);
    if (!strides_.empty() && strides_.size() != rank)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                        "GroupedTensor strides count %zu must be zero or match data rank %zu", strides_.size(), rank);
    if (offsets_) checkGroupArray(*offsets_, num_groups_, "offsets", 0);
    for (std::size_t d = 0; d < dim_sizes_.size(); ++d) checkGroupArray(dim_sizes_[d], num_groups_, "dim_sizes", d);
    for (std::size_t d = 0; d < strides_.size(); ++d) checkGroupArray(strides_[d], num_groups_, "strides", d);
}

}  // namespace ftrain

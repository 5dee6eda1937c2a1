#include <hip/hip_runtime_api.h>

#include "ft/primitive.hpp"

namespace ftrain {

FTrainDeviceId getCurrentDeviceId() {
    int device         = 0;
    const hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess)
        raise(FTRAIN_STATUS_INTERNAL_ERROR, "hipGetDevice failed: %s", hipGetErrorString(e));
    return static_cast<FTrainDeviceId>(device);
}

Plan::Plan(std::vector<std::unique_ptr<PrimitiveBase>> primitives, FTrainDeviceId device)
    : device_(device), primitives_(std::move(primitives)) {
    if (primitives_.empty()) raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Plan requires at least one Primitive");
    for (const auto& p : primitives_)
        if (!p) raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Plan Primitive must not be null");
}

void Plan::prepare() {
    for (std::size_t i = 0; i < primitives_.size(); ++i) primitives_[i]->prepare(i == 0);
}

PrimitiveBase& Plan::at(uint64_t index) const {
    if (index >= primitives_.size())
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Plan primitive index %llu is out of range for %llu primitives",
                        static_cast<unsigned long long>(index),
                        static_cast<unsigned long long>(primitives_.size()));
    return *primitives_[index];
}

void Plan::execute(uint64_t index, void* workspace, uint64_t workspace_bytes, FTrainStream stream,
                   bool counters_clear) {
    const FTrainDeviceId current = getCurrentDeviceId();
    if (current != device_)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                        "Plan was created for device %d but the calling thread uses device %d", int(device_),
                        int(current));
    at(index).execute(Resources{workspace, workspace_bytes, stream, counters_clear});
}

}  // namespace ftrain

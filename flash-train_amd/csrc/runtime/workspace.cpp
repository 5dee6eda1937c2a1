#include "ft/workspace.hpp"

#include <cstdint>
#include <limits>
#include <mutex>

#include "ft/error.hpp"

namespace ftrain {
namespace {

constexpr int kMaxDevices = 64;

// Pool per device, created on first use; never destroyed (the process owns it).
hipMemPool_t poolFor(int device) {
    static std::mutex mutex;
    static hipMemPool_t pools[kMaxDevices] = {};
    if (device < 0 || device >= kMaxDevices)
        raise(FTRAIN_STATUS_INTERNAL_ERROR, "device %d is outside the workspace pool table", device);
    std::lock_guard<std::mutex> lock(mutex);
    if (pools[device] == nullptr) {
        hipMemPoolProps props{};
        props.allocType     = hipMemAllocationTypePinned;
        props.handleTypes   = hipMemHandleTypeNone;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id   = device;
        hipMemPool_t pool   = nullptr;
        hipError_t e        = hipMemPoolCreate(&pool, &props);
        if (e != hipSuccess)
            raise(FTRAIN_STATUS_INTERNAL_ERROR, "hipMemPoolCreate failed: %s", hipGetErrorString(e));
        // Keep released memory in the pool across synchronizations.
        uint64_t keep = std::numeric_limits<uint64_t>::max();
        e             = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
        if (e != hipSuccess)
            raise(FTRAIN_STATUS_INTERNAL_ERROR, "hipMemPoolSetAttribute failed: %s", hipGetErrorString(e));
        pools[device] = pool;
    }
    return pools[device];
}

}  // namespace

void* acquireWorkspace(uint64_t bytes, hipStream_t stream) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) raise(FTRAIN_STATUS_INTERNAL_ERROR, "hipGetDevice failed: %s", hipGetErrorString(e));
    void* p = nullptr;
    e       = hipMallocFromPoolAsync(&p, bytes, poolFor(device), stream);
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();
        raise(FTRAIN_STATUS_OUT_OF_MEMORY, "split-k workspace of %llu bytes: %s",
                        static_cast<unsigned long long>(bytes), hipGetErrorString(e));
    }
    if (e != hipSuccess)
        raise(FTRAIN_STATUS_INTERNAL_ERROR, "hipMallocFromPoolAsync failed: %s", hipGetErrorString(e));
    return p;
}

void releaseWorkspace(void* buffer, hipStream_t stream) {
    if (buffer == nullptr) return;
    const hipError_t e = hipFreeAsync(buffer, stream);
    if (e != hipSuccess) raise(FTRAIN_STATUS_INTERNAL_ERROR, "hipFreeAsync failed: %s", hipGetErrorString(e));
}

}  // namespace ftrain

// Device scratch array for ftrainGemmNoAlloc (see ft/scratch.hpp).
//
// The array is a file-scope __device__ variable, so each GPU the library's
// code object is loaded on holds its own copy, from load until the process
// ends.  In host code `scratch` names a host-side stand-in, not device
// memory: only the address hipGetSymbolAddress returns for the current
// device may be handed to kernels or copies.
#include <hip/hip_runtime.h>

#include <mutex>

#include "ft/error.hpp"
#include "ft/scratch.hpp"

namespace ftrain {
namespace {

static __device__ __align__(256) unsigned char scratch[kDeviceScratchBytes];

constexpr int kMaxDevices = 64;

struct Slot {
    std::once_flag once;
    void* address = nullptr;
    hipError_t error = hipSuccess;
};

Slot& slotFor(int device) {
    static Slot slots[kMaxDevices];
    return slots[device];
}

}  // namespace

DeviceScratch deviceScratch() {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) raise(FTRAIN_STATUS_INTERNAL_ERROR, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (device < 0 || device >= kMaxDevices)
        raise(FTRAIN_STATUS_INTERNAL_ERROR, "device %d is outside the scratch table (%d devices)", device, kMaxDevices);
    Slot& slot = slotFor(device);
    // Once per device, with that device current (it is: hipGetDevice above).
    std::call_once(slot.once, [&] {
        void* p = nullptr;
        slot.error = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (slot.error == hipSuccess) slot.address = p;
    });
    if (slot.error != hipSuccess || slot.address == nullptr)
        raise(FTRAIN_STATUS_INTERNAL_ERROR, "hipGetSymbolAddress of the device scratch array failed on device %d: %s",
              device, hipGetErrorString(slot.error));
    return DeviceScratch{slot.address, kDeviceScratchBytes};
}

}  // namespace ftrain

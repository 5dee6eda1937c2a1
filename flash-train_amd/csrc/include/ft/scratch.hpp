// The library's fixed device scratch array, for ftrainGemmNoAlloc: callers
// that cannot allocate device memory (code under HIP graph capture, serving
// loops, harnesses that forbid hipMalloc) run split-k Primitives with their
// partial tiles in this array instead of a Plan-owned or caller buffer.
#pragma once

#include <cstdint>

namespace ftrain {

struct DeviceScratch {
    void* memory;    // the array's address on the calling thread's device
    uint64_t bytes;  // its size
};

// Bytes of the array on every device (fixed at build time).
constexpr uint64_t kDeviceScratchBytes = 64ull << 20;

// The array on the calling thread's current device.  The first call on a
// device looks its address up (hipGetSymbolAddress, with that device
// current) and keeps it; nothing is allocated.  The array starts with the
// split-k arrival counters (kCounterBytes, zero at load); every kernel
// leaves them zero, and no kernel writes partial tiles over them.  INTERNAL_ERROR when HIP
// fails.  Every use on one device shares the array: executions that
// overlap on one device race.
DeviceScratch deviceScratch();

}  // namespace ftrain

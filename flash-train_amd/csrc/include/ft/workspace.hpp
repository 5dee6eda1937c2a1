// Transient device buffers for Primitives that need scratch space but
// advertise no caller workspace (so the convenience path, which passes none,
// can run them).  Buffers come from a library-owned, per-device,
// stream-ordered memory pool: acquire/release are ordered on the execution
// stream, so concurrent executions on different streams never share a
// buffer, nothing synchronizes, and freed memory stays in the pool for the
// next call.
#pragma once

#include <cstdint>

#include <hip/hip_runtime_api.h>

namespace ftrain {

// Returns `bytes` of device memory on the calling thread's current device,
// usable by work enqueued on `stream` after this call.  Throws
// OUT_OF_MEMORY or INTERNAL_ERROR.
void* acquireWorkspace(uint64_t bytes, hipStream_t stream);

// Returns a buffer from acquireWorkspace once the work already enqueued on
// `stream` has used it.
void releaseWorkspace(void* buffer, hipStream_t stream);

}  // namespace ftrain

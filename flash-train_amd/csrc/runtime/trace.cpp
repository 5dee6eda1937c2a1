#include "ft/trace.hpp"

#include <roctracer/roctx.h>

namespace ftrain {

TraceRange::TraceRange(const char* name) noexcept { open_ = roctxRangePushA(name) >= 0; }

TraceRange::~TraceRange() noexcept {
    if (open_) (void)roctxRangePop();
}

}  // namespace ftrain

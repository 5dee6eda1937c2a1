// roctx ranges around the C API entry points, visible in rocprofv3 traces
// (--marker-trace).  Same use sites as the reference
// (src/trace.cpp:14-36; src/api/plan_api.cpp:13,87; src/api/gemm_api.cpp:57).
#pragma once

namespace ftrain {

class TraceRange {
  public:
    explicit TraceRange(const char* name) noexcept;
    ~TraceRange() noexcept;
    TraceRange(const TraceRange&)            = delete;
    TraceRange& operator=(const TraceRange&) = delete;

  private:
    bool open_ = false;
};

}  // namespace ftrain

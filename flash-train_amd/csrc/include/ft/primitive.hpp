// Primitive contract, execution resources, runtime constraints and Plan.
//
// Contract follows the reference:
//   PrimitiveBase/Primitive<Problem>  src/include/flash_train/primitive.hpp:24-76,
//                                     src/primitive.cpp:12-25
//   Resources                         src/include/flash_train/resources.hpp:17-36
//   Constraints, getCurrentDeviceId   src/include/flash_train/constraints.hpp:15-40,
//                                     src/constraints.cpp:15-26
//   Plan                              src/include/flash_train/plan.hpp:21-57,
//                                     src/plan.cpp:12-55
#pragma once

#include <cstdint>
#include <memory>
#include <vector>

#include <flash_train/common.h>

#include "ft/error.hpp"

namespace ftrain {

// The calling thread's current HIP device; INTERNAL_ERROR when HIP fails.
FTrainDeviceId getCurrentDeviceId();

struct Resources {
    void* workspace;
    uint64_t workspace_bytes;
    FTrainStream stream;
    // The workspace's split-k arrival counters are known to be 0 (the
    // library's device scratch array: zero at load, left zero by every
    // launch).  A caller's workspace has arbitrary contents.
    bool counters_clear = false;
};

// Everything outside the Problem that can change a selection.  Encoded into
// the selection-cache key.
class Constraints {
  public:
    explicit Constraints(FTrainDeviceId device) noexcept : device_(device) {}
    FTrainDeviceId device() const noexcept { return device_; }
    std::vector<uint64_t> key() const { return {static_cast<uint64_t>(static_cast<uint32_t>(device_))}; }

  private:
    FTrainDeviceId device_;
};

// One implementation.  Engines keep unconfigured prototypes; each Plan owns
// configured clones.  A configured clone keeps everything it needs (pointers,
// scalar values, launch geometry) so Args and Ops can be destroyed.
class PrimitiveBase {
  public:
    virtual ~PrimitiveBase() = default;
    virtual const char* name() const noexcept                   = 0;
    virtual std::unique_ptr<PrimitiveBase> clone() const        = 0;
    virtual uint64_t requiredWorkspaceBytes() const noexcept    = 0;

    // Device memory beyond the operands that one execution writes and reads
    // back (split-k partial tiles), whoever provides it.
    virtual uint64_t scratchBytes() const noexcept { return 0; }

    // Acquires the device resources the Primitive keeps for its Plan's
    // lifetime, on the Plan's device, once, at Plan creation (never during
    // an execution).  `default_slot` is true for Primitive 0, the one
    // ftrainGemm runs without a workspace.
    virtual void prepare(bool default_slot) { (void)default_slot; }

    // Checks the workspace against the requirement (INVALID_ARGUMENT) and
    // enqueues the work on resources.stream without synchronizing.
    void execute(const Resources& resources) {
        const uint64_t need = requiredWorkspaceBytes();
        if (resources.workspace_bytes < need)
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Primitive requires %llu workspace bytes but received %llu",
                            static_cast<unsigned long long>(need),
                            static_cast<unsigned long long>(resources.workspace_bytes));
        if (need != 0 && resources.workspace == nullptr)
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Primitive requires a non-null workspace for %llu bytes",
                            static_cast<unsigned long long>(need));
        run(resources);
    }

  protected:
    PrimitiveBase()                                = default;
    PrimitiveBase(const PrimitiveBase&)            = default;
    PrimitiveBase& operator=(const PrimitiveBase&) = default;
    virtual void run(const Resources& resources)   = 0;
};

template <typename Problem>
class Primitive : public PrimitiveBase {
  public:
    // Success, or UNSUPPORTED with a reason the engine reports.  Must be safe
    // for concurrent const calls.
    virtual Result isApplicable(const Problem& problem, const Constraints& constraints) const = 0;
    virtual void configure(const Problem& problem)                                            = 0;
};

class Plan {
  public:
    // INVALID_ARGUMENT when `primitives` is empty or holds a null entry.
    Plan(std::vector<std::unique_ptr<PrimitiveBase>> primitives, FTrainDeviceId device);

    uint64_t size() const noexcept { return primitives_.size(); }
    FTrainDeviceId device() const noexcept { return device_; }
    const char* primitiveName(uint64_t index) const { return at(index).name(); }
    uint64_t requiredWorkspaceBytes(uint64_t index) const { return at(index).requiredWorkspaceBytes(); }
    uint64_t scratchBytes(uint64_t index) const { return at(index).scratchBytes(); }

    // Runs every Primitive's prepare() (Primitive 0 as the default slot).
    void prepare();

    // Device check (calling thread's device must be the Plan's), index check,
    // then the Primitive's workspace check and launch.
    // `counters_clear`: see Resources.
    void execute(uint64_t index, void* workspace, uint64_t workspace_bytes, FTrainStream stream,
                 bool counters_clear = false);

  private:
    PrimitiveBase& at(uint64_t index) const;
    FTrainDeviceId device_;
    std::vector<std::unique_ptr<PrimitiveBase>> primitives_;
};

}  // namespace ftrain

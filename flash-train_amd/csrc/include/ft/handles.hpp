// Definitions behind the opaque C handles (reference
// src/include/flash_train/api.hpp:68-88).
#pragma once

#include <exception>
#include <new>

#include <flash_train/common.h>

#include "ft/engine.hpp"

struct FTrainPatternStruct {
    ftrain::PatternBuilder builder;
};
struct FTrainOpsStruct {
    ftrain::Ops ops;
};
struct FTrainArgsStruct {
    ftrain::Args args;
};
struct FTrainPlanStruct {
    ftrain::Plan plan;
};

namespace ftrain {
// The calling thread's last result (shared by the C API and test hooks).
Result& lastResult() noexcept;

// Plans made by ftrainGemm / ftrainGemmNoAlloc that are still alive (held by
// a thread's convenience cache or by a graph that captured them), after
// destroying those whose last graph is gone.
long conveniencePlansAlive();

// Runs `body` at the C boundary: success clears the thread's last result;
// Failure -> its own status and message, std::bad_alloc -> OUT_OF_MEMORY,
// any other exception -> INTERNAL_ERROR.  Never throws.
template <typename F>
inline FTrainStatus guarded(F&& body) noexcept {
    try {
        body();
        lastResult().clear();
        return FTRAIN_STATUS_SUCCESS;
    } catch (const Failure& e) {
        lastResult() = e.result();
        return e.result().getStatus();
    } catch (const std::bad_alloc& e) {
        lastResult().set(FTRAIN_STATUS_OUT_OF_MEMORY, e.what());
        return FTRAIN_STATUS_OUT_OF_MEMORY;
    } catch (const std::exception& e) {
        lastResult().set(FTRAIN_STATUS_INTERNAL_ERROR, e.what());
        return FTRAIN_STATUS_INTERNAL_ERROR;
    } catch (...) {
        lastResult().set(FTRAIN_STATUS_INTERNAL_ERROR, "a non-standard exception reached the C entry point");
        return FTRAIN_STATUS_INTERNAL_ERROR;
    }
}

}  // namespace ftrain

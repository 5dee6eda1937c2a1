// Host-only test hooks, linked into libflash_train_testing.so only (never
// into libflash_train.so).  They expose internals that need no GPU -- the
// Finder's ranking and cost model, the selection cache, the environment-list
// parsing, and Plan creation for an explicit device id -- so the CPU test
// suite can pin them.  Not part of the product ABI.
#include <cstring>
#include <string>

#include "ft/gemm.hpp"
#include "ft/handles.hpp"

#define FTRAIN_TESTING_API extern "C" __attribute__((visibility("default")))

using namespace ftrain;

namespace {

void copyOut(const std::string& s, char* out, size_t cap) {
    if (out == nullptr || cap == 0) return;
    const size_t n = std::min(s.size(), cap - 1);
    std::memcpy(out, s.data(), n);
    out[n] = '\0';
}

const GemmEngine& gemmEngine() {
    static const GemmEngine engine;
    return engine;
}

}  // namespace

// Plan creation as ftrainPlanCreate does it, but for `device` instead of
// the calling thread's current device (lets CPU hosts exercise validation,
// selection and configuration).
FTRAIN_TESTING_API FTrainStatus ftrainTestingPlanCreateOnDevice(FTrainPlan* plan, FTrainArgs args, int32_t device) {
    return guarded([&] {
        if (plan == nullptr || args == nullptr) raise(FTRAIN_STATUS_INVALID_ARGUMENT, "null argument");
        const auto engine = globalHandle().find(args->args.key());
        if (!engine) raise(FTRAIN_STATUS_INTERNAL_ERROR, "OpsEngine registered for Args is unavailable");
        *plan = new FTrainPlanStruct{Plan(engine->createPrimitives(args->args, Constraints(device)), device)};
    });
}

// Ranked Primitive names (comma separated) the engine selects for a Gemm
// given its six port views, on a device with id `device` -- without
// configuring or caching.
FTRAIN_TESTING_API FTrainStatus ftrainTestingRankGemm(const FTrainStorageView views[6], FTrainNumericType compute_type,
                                                      int32_t device, char* out, size_t cap) {
    return guarded([&] {
        const GemmProblem problem(Tensor{StorageView(views[0])}, Tensor{StorageView(views[1])},
                                  Tensor{StorageView(views[2])}, Tensor{StorageView(views[3])},
                                  Tensor{StorageView(views[4])}, Tensor{StorageView(views[5])}, compute_type);
        std::string joined;
        for (const std::string& n : gemmEngine().rank(problem, Constraints(device))) {
            if (!joined.empty()) joined += ",";
            joined += n;
        }
        copyOut(joined, out, cap);
    });
}

FTRAIN_TESTING_API int ftrainTestingVariantCount(void) { return static_cast<int>(gemm::Variant::kCount); }

FTRAIN_TESTING_API const char* ftrainTestingVariantName(int v) {
    return v >= 0 && v < ftrainTestingVariantCount() ? gemm::info(static_cast<gemm::Variant>(v)).name : nullptr;
}

FTRAIN_TESTING_API double ftrainTestingEstimateMicros(int v, uint64_t m, uint64_t n, uint64_t k, bool has_c, int cus) {
    return gemm::estimateMicros(static_cast<gemm::Variant>(v), GemmShape{m, n, k}, has_c, cus);
}

FTRAIN_TESTING_API uint32_t ftrainTestingChooseSplits(int v, uint64_t m, uint64_t n, uint64_t k, int cus) {
    return gemm::chooseSplits(static_cast<gemm::Variant>(v), GemmShape{m, n, k}, cus);
}

FTRAIN_TESTING_API void ftrainTestingForceSplits(uint32_t s) { gemm::forceSplits(s); }

// Convenience Plans still alive (cached per thread or owned by captured graphs).
FTRAIN_TESTING_API long ftrainTestingConveniencePlansAlive(void) { return conveniencePlansAlive(); }

// ---- selection cache ----

FTRAIN_TESTING_API void* ftrainTestingCacheCreate(uint64_t max_entries, uint64_t shards) {
    void* cache = nullptr;
    if (guarded([&] { cache = new SelectionCache(max_entries, shards); }) != FTRAIN_STATUS_SUCCESS) return nullptr;
    return cache;
}

FTRAIN_TESTING_API void ftrainTestingCacheDestroy(void* cache) { delete static_cast<SelectionCache*>(cache); }

FTRAIN_TESTING_API FTrainStatus ftrainTestingCachePublish(void* cache, const uint64_t* ct, size_t nct,
                                                          const uint64_t* pt, size_t npt, const uint64_t* pos,
                                                          size_t npos) {
    return guarded([&] {
        std::vector<std::size_t> p(pos, pos + npos);
        static_cast<SelectionCache*>(cache)->publish(
            CacheKey(std::vector<uint64_t>(ct, ct + nct), std::vector<uint64_t>(pt, pt + npt)), std::move(p));
    });
}

// Returns the number of positions found (-1 on a miss), writing up to `cap`.
FTRAIN_TESTING_API int64_t ftrainTestingCacheFind(void* cache, const uint64_t* ct, size_t nct, const uint64_t* pt,
                                                  size_t npt, uint64_t* out, size_t cap) {
    const auto hit = static_cast<SelectionCache*>(cache)->find(
        CacheKey(std::vector<uint64_t>(ct, ct + nct), std::vector<uint64_t>(pt, pt + npt)));
    if (!hit) return -1;
    for (size_t i = 0; i < hit->size() && i < cap; ++i) out[i] = (*hit)[i];
    return static_cast<int64_t>(hit->size());
}

FTRAIN_TESTING_API uint64_t ftrainTestingCacheSize(void* cache) { return static_cast<SelectionCache*>(cache)->size(); }

// ---- environment parsing ----

FTRAIN_TESTING_API void ftrainTestingParseNameList(const char* value, char* out, size_t cap) {
    const auto names = parseNameList(value);
    std::vector<std::string> sorted(names.begin(), names.end());
    std::sort(sorted.begin(), sorted.end());
    std::string joined;
    for (const auto& n : sorted) joined += (joined.empty() ? "" : "|") + n;
    copyOut(joined, out, cap);
}

FTRAIN_TESTING_API bool ftrainTestingParseSwitch(const char* value) { return parseSwitch(value); }

// Raises a failure whose message is `length` repetitions of 'x' (formatted
// when `formatted`, literal otherwise) through the C boundary, so the
// last-message capacity can be checked.
FTRAIN_TESTING_API FTrainStatus ftrainTestingFailWithLength(FTrainStatus status, size_t length, bool formatted) {
    return guarded([&] {
        const std::string text(length, 'x');
        if (formatted) raise(status, "%s", text.c_str());
        Result r(status, text.c_str());
        throw Failure(r);
    });
}

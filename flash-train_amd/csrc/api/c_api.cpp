// The exported C ABI: the 29 ftrain* entry points of the reference
// (include/flash_train/common.h:162-589, include/flash_train/flash_train.h:46-48;
// implementations src/api/{common,pattern,ops_args,plan,gemm}_api.cpp).
//
// Each entry point runs its body through `guarded`, which maps exceptions to
// status codes (Failure -> its status, bad_alloc -> OUT_OF_MEMORY, any
// other exception -> INTERNAL_ERROR) and records the status and message as
// the thread's last result (reference src/include/flash_train/api.hpp:37-62).
#include <algorithm>
#include <atomic>
#include <cstring>
#include <exception>
#include <mutex>
#include <new>
#include <optional>
#include <utility>

#include <flash_train/flash_train.h>

#include "ft/handles.hpp"
#include "ft/scratch.hpp"
#include "ft/trace.hpp"

namespace ftrain {

Result& lastResult() noexcept {
    static thread_local Result r;
    return r;
}

namespace {

[[noreturn]] void invalid(const char* message) { raise(FTRAIN_STATUS_INVALID_ARGUMENT, "%s", message); }

template <typename T>
void requireNonNull(const T* p, const char* message) {
    if (p == nullptr) invalid(message);
}

OpNode gemmNode(OperationKind kind, uint64_t a, uint64_t b, uint64_t c, uint64_t d, uint64_t alpha, uint64_t beta) {
    return OpNode{kind, {a, b, c, alpha, beta}, {d}};
}

template <typename Id>
FTrainStatus addOperand(FTrainPattern pattern, Id* out, OperandKind kind, const char* fn) {
    return guarded([&] {
        if (pattern == nullptr) raise(FTRAIN_STATUS_INVALID_ARGUMENT, "%s: pattern must not be null", fn);
        if (out == nullptr) raise(FTRAIN_STATUS_INVALID_ARGUMENT, "%s: output must not be null", fn);
        *out = Id{pattern->builder.addOperand(kind)};
    });
}

template <typename Id>
FTrainStatus addGemmLike(FTrainPattern pattern, Id* op, OperationKind kind, uint64_t a, uint64_t b, uint64_t c,
                         uint64_t d, uint64_t alpha, uint64_t beta, const char* fn) {
    return guarded([&] {
        if (pattern == nullptr) raise(FTRAIN_STATUS_INVALID_ARGUMENT, "%s: pattern must not be null", fn);
        if (op == nullptr) raise(FTRAIN_STATUS_INVALID_ARGUMENT, "%s: op output must not be null", fn);
        *op = Id{pattern->builder.addOperation(gemmNode(kind, a, b, c, d, alpha, beta))};
    });
}

FTrainStatus setOperation(FTrainArgs args, uint64_t op, OperationKind kind, FTrainNumericType compute_type,
                          const char* fn) {
    return guarded([&] {
        if (args == nullptr) raise(FTRAIN_STATUS_INVALID_ARGUMENT, "%s: args handle must not be null", fn);
        if (compute_type == FTRAIN_NUMERIC_TYPE_INVALID || compute_type >= FTRAIN_NUMERIC_TYPE_COUNT)
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "%s: compute_type %u is invalid", fn,
                            unsigned(compute_type));
        args->args.setOperation(op, OperationAttributes{kind, compute_type});
    });
}

// A convenience Plan shared by its cache entry and by every graph that
// captured one of its executions (the graph's kernels point at the Plan's
// split-k buffer).  The last owner to let go destroys the Plan.  A graph lets
// go through a HIP user object whose destructor HIP runs when the graph and
// every executable graph made from it are destroyed; that destructor must not
// call HIP, so it only queues the Plan, and the next convenience call destroys
// it on an ordinary thread.
struct SharedPlan {
    FTrainPlan plan;
    std::atomic<int> owners{1};
};

// Never destroyed: HIP may run a graph's user-object destructor while the
// process tears down its statics.
std::mutex& releasedMutex() {
    static auto* m = new std::mutex();
    return *m;
}
std::vector<FTrainPlan>& releasedPlans() {
    static auto* v = new std::vector<FTrainPlan>();
    return *v;
}
std::atomic<long>& livePlans() {
    static std::atomic<long> n{0};
    return n;
}

void destroyPlan(FTrainPlan plan) {
    delete plan;
    livePlans().fetch_sub(1);
}

// Destroys the Plans whose last graph has been destroyed.
void destroyReleasedPlans() {
    std::vector<FTrainPlan> batch;
    {
        std::lock_guard<std::mutex> lock(releasedMutex());
        if (releasedPlans().empty()) return;
        batch.swap(releasedPlans());
    }
    for (FTrainPlan p : batch) destroyPlan(p);
}

void dropOwner(SharedPlan* s, bool may_call_hip) {
    if (s->owners.fetch_sub(1) != 1) return;
    FTrainPlan plan = s->plan;
    delete s;
    if (may_call_hip) {
        destroyPlan(plan);
    } else {
        std::lock_guard<std::mutex> lock(releasedMutex());
        releasedPlans().push_back(plan);
    }
}

void graphReleased(void* shared) { dropOwner(static_cast<SharedPlan*>(shared), false); }

// Makes the graph `stream` is capturing into an owner of `s`.  When HIP
// cannot attach the user object, the Plan is kept until the process ends
// instead (the graph may still replay it).
void ownByCapturingGraph(SharedPlan* s, FTrainStream stream) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    hipGraph_t graph              = nullptr;
    s->owners.fetch_add(1);
    if (hipStreamGetCaptureInfo_v2(stream, &status, nullptr, &graph, nullptr, nullptr) == hipSuccess &&
        status == hipStreamCaptureStatusActive && graph != nullptr) {
        hipUserObject_t object = nullptr;
        if (hipUserObjectCreate(&object, s, graphReleased, 1, hipUserObjectNoDestructorSync) == hipSuccess) {
            if (hipGraphRetainUserObject(graph, object, 1, hipGraphUserObjectMove) == hipSuccess) return;
            s->owners.fetch_add(1);                 // the graph may replay the Plan: never let go
            (void)hipUserObjectRelease(object, 1);  // runs graphReleased for the reference just taken
        }
    }
    (void)hipGetLastError();
}

// Plans created by ftrainGemm, kept per thread and reused when a later call
// describes exactly the same problem: the same six views (addresses, dims,
// strides, types, placement), the same host alpha/beta values, compute type
// and device.  A Plan binds exactly those values, so reuse is
// indistinguishable from creating it again.  Least recently used entries are
// released beyond kCapacity (destroyed, unless a graph still owns them).
// Skipped when FTRAIN_DISABLE_CACHE is set.
class ConveniencePlans {
  public:
    static constexpr std::size_t kCapacity = 32;

    // One cache per thread for each convenience entry point: ftrainGemm's
    // Plans are prepared (they own split-k buffers), ftrainGemmNoAlloc's are
    // not.
    static ConveniencePlans& local(bool no_alloc) {
        static thread_local ConveniencePlans cache[2];
        return cache[no_alloc ? 1 : 0];
    }

    // Host scalars must be readable fp32 values of rank 0 for the key.
    static bool describable(const FTrainStorageView* const views[6]) {
        for (int i = 4; i < 6; ++i) {
            const FTrainStorageView& v = *views[i];
            if (v.memory == nullptr || v.num_dims != 0 || !v.is_host_memory ||
                v.numeric_type != FTRAIN_NUMERIC_TYPE_FP32)
                return false;
        }
        for (int i = 0; i < 4; ++i)
            if (views[i]->num_dims != 0 && views[i]->dims == nullptr) return false;
        return true;
    }

    static std::vector<uint64_t> describe(const FTrainStorageView* const views[6], FTrainNumericType compute_type,
                                          int device, FTrainStream stream) {
        std::vector<uint64_t> k;
        k.reserve(48);
        k.push_back(uint64_t(uint32_t(device)));
        // A split-k Plan keeps its partial tiles in a buffer of its own, so
        // calls on different streams, which may overlap on the device, get
        // Plans of their own.
        k.push_back(reinterpret_cast<uintptr_t>(stream));
        k.push_back(compute_type);
        for (int i = 0; i < 6; ++i) {
            const FTrainStorageView& v = *views[i];
            k.push_back(reinterpret_cast<uintptr_t>(v.memory));
            k.push_back(uint64_t(v.num_dims) | uint64_t(v.numeric_type) << 8 | uint64_t(v.index_type) << 16 |
                        uint64_t(v.is_host_memory) << 24 | uint64_t(v.strides != nullptr) << 25);
            for (uint8_t j = 0; j < v.num_dims; ++j) k.push_back(uint64_t(v.dims[j]));
            if (v.strides != nullptr)
                for (uint8_t j = 0; j < v.num_dims; ++j) k.push_back(uint64_t(v.strides[j]));
            if (i >= 4) {
                uint32_t bits;
                std::memcpy(&bits, v.memory, sizeof(bits));
                k.push_back(bits);
            }
        }
        return k;
    }

    SharedPlan* find(const std::vector<uint64_t>& key) {
        for (std::size_t i = 0; i < entries_.size(); ++i) {
            if (entries_[i].key == key) {
                if (i != 0) std::rotate(entries_.begin(), entries_.begin() + i, entries_.begin() + i + 1);
                return entries_.front().shared;
            }
        }
        return nullptr;
    }

    SharedPlan* insert(std::vector<uint64_t> key, FTrainPlan plan) {
        auto* shared = new SharedPlan{plan};
        entries_.insert(entries_.begin(), Entry{std::move(key), shared});
        while (entries_.size() > kCapacity) {
            dropOwner(entries_.back().shared, true);
            entries_.pop_back();
        }
        return shared;
    }

    ~ConveniencePlans() {
        for (auto& e : entries_) dropOwner(e.shared, true);
    }

  private:
    struct Entry {
        std::vector<uint64_t> key;
        SharedPlan* shared;
    };

    std::vector<Entry> entries_;  // most recent first
};

bool streamCapturing(FTrainStream stream) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &status) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return status != hipStreamCaptureStatusNone;
}

// A Plan as ftrainPlanCreate makes it, minus Plan::prepare: no Primitive
// acquires device memory of its own.
FTrainStatus createUnpreparedPlan(FTrainPlan* plan, FTrainArgs args) {
    return guarded([&] {
        const auto engine = globalHandle().find(args->args.key());
        if (!engine) raise(FTRAIN_STATUS_INTERNAL_ERROR, "OpsEngine registered for Args is unavailable");
        *plan = new FTrainPlanStruct{engine->createPlan(args->args)};
    });
}

// Runs a convenience Plan.  With `scratch` set (ftrainGemmNoAlloc) the first
// Primitive whose split-k partials fit the scratch array runs with the array
// as its workspace.  Otherwise, with `fit_bytes` nonzero (a Plan made under
// capture, without a buffer of its own), the first Primitive whose workspace
// requirement is below `fit_bytes` runs; else Primitive 0.
FTrainStatus executeConvenience(FTrainPlan plan, uint64_t fit_bytes, void* workspace, uint64_t workspace_bytes,
                                FTrainStream stream, const DeviceScratch* scratch) {
    if (scratch == nullptr && fit_bytes == 0)
        return ftrainPlanExecutePrimitive(plan, 0, workspace, workspace_bytes, stream);
    uint64_t index = 0;
    const FTrainStatus s = guarded([&] {
        const uint64_t n = plan->plan.size();
        if (scratch != nullptr) {
            while (index < n && plan->plan.scratchBytes(index) > scratch->bytes) ++index;
            if (index == n)
                raise(FTRAIN_STATUS_UNSUPPORTED,
                      "ftrainGemmNoAlloc: every Primitive of the Plan needs more than the %llu-byte device scratch "
                      "array (Primitive 0, %s, needs %llu bytes)",
                      static_cast<unsigned long long>(scratch->bytes), plan->plan.primitiveName(0),
                      static_cast<unsigned long long>(plan->plan.scratchBytes(0)));
        } else {
            while (index < n && plan->plan.requiredWorkspaceBytes(index) >= fit_bytes) ++index;
            if (index == n)
                raise(FTRAIN_STATUS_UNSUPPORTED,
                      "ftrainGemm under stream capture: the problem is not in the calling thread's Plan cache and "
                      "every Primitive needs more than the %llu-byte workspace given (Primitive 0, %s, needs %llu "
                      "bytes); call ftrainGemm once before the capture, pass a workspace, or use ftrainGemmNoAlloc",
                      static_cast<unsigned long long>(fit_bytes - 1), plan->plan.primitiveName(0),
                      static_cast<unsigned long long>(plan->plan.requiredWorkspaceBytes(0)));
        }
    });
    if (s != FTRAIN_STATUS_SUCCESS) return s;
    if (scratch == nullptr) return ftrainPlanExecutePrimitive(plan, index, workspace, workspace_bytes, stream);
    // The scratch array's split-k arrival counters are 0 (zero at load, left
    // zero by every launch), so no clearing launch is needed.
    return guarded([&] { plan->plan.execute(index, scratch->memory, scratch->bytes, stream, true); });
}

// The convenience path behind ftrainGemm and ftrainGemmNoAlloc.  With
// `scratch` null (ftrainGemm) the Plan is made by ftrainPlanCreate and its
// Primitive 0 runs.  With `scratch` set (ftrainGemmNoAlloc) the Plan is made
// without preparation, so nothing is allocated on the device, and the first
// Primitive in rank order whose scratch need fits the library's device
// scratch array runs with that array as its workspace.
FTrainStatus convenienceGemm(const FTrainStorageView* const views[6], FTrainNumericType compute_type, void* workspace,
                             uint64_t workspace_bytes, FTrainStream stream, const DeviceScratch* scratch) {
    const FTrainStorageView &a = *views[0], &b = *views[1], &c = *views[2], &d = *views[3], &alpha = *views[4],
                            &beta = *views[5];
    // One Ops for the Gemm Pattern per process, built through the staged API
    // (reference src/api/gemm_api.cpp:28-49).
    struct Entry {
        FTrainOps ops = nullptr;
        FTrainTensorId a{}, b{}, c{}, d{}, alpha{}, beta{};
        FTrainGemmOpId gemm{};
        FTrainStatus status = FTRAIN_STATUS_SUCCESS;
    };
    static const Entry entry = [] {
        Entry e;
        FTrainPattern p = nullptr;
        FTrainStatus s  = ftrainPatternCreate(&p);
        for (FTrainTensorId* id : {&e.a, &e.b, &e.c, &e.alpha, &e.beta, &e.d})
            if (s == FTRAIN_STATUS_SUCCESS) s = ftrainPatternAddTensor(p, id);
        if (s == FTRAIN_STATUS_SUCCESS) s = ftrainPatternAddGemm(p, &e.gemm, e.a, e.b, e.c, e.d, e.alpha, e.beta);
        if (s == FTRAIN_STATUS_SUCCESS) s = ftrainOpsCreate(&e.ops, p);
        if (p != nullptr) ftrainPatternDestroy(p);
        e.status = s;
        return e;
    }();
    if (entry.status != FTRAIN_STATUS_SUCCESS) return entry.status;

    destroyReleasedPlans();
    const bool no_alloc  = scratch != nullptr;
    const bool capturing = streamCapturing(stream);
    const bool cacheable = !selectionCacheDisabled() && ConveniencePlans::describable(views);
    int device           = -1;
    std::vector<uint64_t> key;
    if (cacheable && hipGetDevice(&device) == hipSuccess) {
        key = ConveniencePlans::describe(views, compute_type, device, stream);
        if (SharedPlan* cached = ConveniencePlans::local(no_alloc).find(key)) {
            const FTrainStatus s = executeConvenience(cached->plan, 0, workspace, workspace_bytes, stream, scratch);
            if (s == FTRAIN_STATUS_SUCCESS && capturing) ownByCapturingGraph(cached, stream);
            return s;
        }
    } else {
        (void)hipGetLastError();
    }

    // Under capture ftrainGemm makes its new Plan without preparation
    // (Plan::prepare allocates and clears device memory, which a capture
    // forbids) and runs the first Primitive that needs no more than the
    // caller's workspace.  That Plan is owned by the graph alone and not
    // cached: uncaptured calls expect Primitive 0 to run without a workspace.
    const bool fit_workspace = capturing && !no_alloc;
    FTrainArgs args          = nullptr;
    FTrainPlan plan          = nullptr;
    FTrainStatus s           = ftrainArgsCreate(&args, entry.ops);
    const std::pair<FTrainTensorId, const FTrainStorageView*> ports[] = {
        {entry.a, &a}, {entry.b, &b}, {entry.c, &c}, {entry.d, &d}, {entry.alpha, &alpha}, {entry.beta, &beta}};
    for (const auto& port : ports)
        if (s == FTRAIN_STATUS_SUCCESS) s = ftrainArgsSetTensor(args, port.first, *port.second);
    if (s == FTRAIN_STATUS_SUCCESS) s = ftrainArgsSetGemm(args, entry.gemm, compute_type);
    if (s == FTRAIN_STATUS_SUCCESS)
        s = no_alloc || fit_workspace ? createUnpreparedPlan(&plan, args) : ftrainPlanCreate(&plan, args);
    if (s == FTRAIN_STATUS_SUCCESS) livePlans().fetch_add(1);
    if (s == FTRAIN_STATUS_SUCCESS)
        s = executeConvenience(plan, fit_workspace ? workspace_bytes + 1 : 0, workspace, workspace_bytes, stream,
                               scratch);
    // Keep the failing step's diagnostic across the clean-up calls.
    const Result failure = s != FTRAIN_STATUS_SUCCESS ? lastResult() : Result{};
    if (plan != nullptr) {
        if (s != FTRAIN_STATUS_SUCCESS) {
            destroyPlan(plan);
        } else if (!key.empty() && !fit_workspace) {
            SharedPlan* shared = ConveniencePlans::local(no_alloc).insert(std::move(key), plan);  // the cache owns it
            if (capturing) ownByCapturingGraph(shared, stream);
        } else if (capturing) {
            auto* shared = new SharedPlan{plan};
            ownByCapturingGraph(shared, stream);
            dropOwner(shared, true);  // the graph is now its only owner
        } else {
            destroyPlan(plan);
        }
    }
    if (args != nullptr) ftrainArgsDestroy(args);
    if (s != FTRAIN_STATUS_SUCCESS) lastResult() = failure;
    return s;
}

}  // namespace

long conveniencePlansAlive() {
    destroyReleasedPlans();
    return livePlans().load();
}

}  // namespace ftrain

using namespace ftrain;

extern "C" {

FTrainStatus ftrainGetLastStatus(void) { return lastResult().getStatus(); }
const char* ftrainGetLastMessage(void) { return lastResult().getMessage(); }

// ---------------------------------------------------------------- Pattern

FTrainStatus ftrainPatternCreate(FTrainPattern* pattern) {
    return guarded([&] {
        requireNonNull(pattern, "ftrainPatternCreate: pattern output must not be null");
        *pattern = new FTrainPatternStruct();
    });
}

FTrainStatus ftrainPatternDestroy(FTrainPattern pattern) {
    return guarded([&] {
        requireNonNull(pattern, "ftrainPatternDestroy: pattern must not be null");
        delete pattern;
    });
}

FTrainStatus ftrainPatternAddTensor(FTrainPattern pattern, FTrainTensorId* tensor) {
    return addOperand(pattern, tensor, OperandKind::kTensor, "ftrainPatternAddTensor");
}

FTrainStatus ftrainPatternAddTensorList(FTrainPattern pattern, FTrainTensorListId* tensor_list) {
    return addOperand(pattern, tensor_list, OperandKind::kTensorList, "ftrainPatternAddTensorList");
}

FTrainStatus ftrainPatternAddGroupedTensor(FTrainPattern pattern, FTrainGroupedTensorId* grouped_tensor) {
    return addOperand(pattern, grouped_tensor, OperandKind::kGroupedTensor, "ftrainPatternAddGroupedTensor");
}

FTrainStatus ftrainPatternAddGemm(FTrainPattern pattern, FTrainGemmOpId* op, FTrainTensorId a, FTrainTensorId b,
                                  FTrainTensorId c, FTrainTensorId d, FTrainTensorId alpha, FTrainTensorId beta) {
    return addGemmLike(pattern, op, OperationKind::kGemm, a.opaque, b.opaque, c.opaque, d.opaque, alpha.opaque,
                       beta.opaque, "ftrainPatternAddGemm");
}

FTrainStatus ftrainPatternAddGroupedABCDGemm(FTrainPattern pattern, FTrainGroupedABCDGemmOpId* op,
                                             FTrainGroupedTensorId a, FTrainGroupedTensorId b, FTrainGroupedTensorId c,
                                             FTrainGroupedTensorId d, FTrainTensorId alpha, FTrainTensorId beta) {
    return addGemmLike(pattern, op, OperationKind::kGroupedABCDGemm, a.opaque, b.opaque, c.opaque, d.opaque,
                       alpha.opaque, beta.opaque, "ftrainPatternAddGroupedABCDGemm");
}

FTrainStatus ftrainPatternAddGroupedBCDGemm(FTrainPattern pattern, FTrainGroupedBCDGemmOpId* op, FTrainTensorListId a,
                                            FTrainGroupedTensorId b, FTrainGroupedTensorId c, FTrainGroupedTensorId d,
                                            FTrainTensorId alpha, FTrainTensorId beta) {
    return addGemmLike(pattern, op, OperationKind::kGroupedBCDGemm, a.opaque, b.opaque, c.opaque, d.opaque,
                       alpha.opaque, beta.opaque, "ftrainPatternAddGroupedBCDGemm");
}

FTrainStatus ftrainPatternAddGroupedABGemm(FTrainPattern pattern, FTrainGroupedABGemmOpId* op, FTrainGroupedTensorId a,
                                           FTrainGroupedTensorId b, FTrainTensorListId c, FTrainTensorListId d,
                                           FTrainTensorId alpha, FTrainTensorId beta) {
    return addGemmLike(pattern, op, OperationKind::kGroupedABGemm, a.opaque, b.opaque, c.opaque, d.opaque,
                       alpha.opaque, beta.opaque, "ftrainPatternAddGroupedABGemm");
}

// ---------------------------------------------------------------- Ops

FTrainStatus ftrainOpsCreate(FTrainOps* ops, FTrainPattern pattern) {
    TraceRange trace("ftrainOpsCreate");
    return guarded([&] {
        requireNonNull(ops, "ftrainOpsCreate: ops output must not be null");
        requireNonNull(pattern, "ftrainOpsCreate: pattern must not be null");
        const Pattern user = pattern->builder.build();
        const auto engine  = globalHandle().find(user.key());
        if (!engine)
            raise(FTRAIN_STATUS_UNSUPPORTED,
                            "ftrainOpsCreate: PatternBuilder does not match any registered OpsEngine");
        *ops = new FTrainOpsStruct{Ops(user, engine->pattern())};
    });
}

FTrainStatus ftrainOpsDestroy(FTrainOps ops) {
    return guarded([&] {
        requireNonNull(ops, "ftrainOpsDestroy: ops handle must not be null");
        delete ops;
    });
}

// ---------------------------------------------------------------- Args

FTrainStatus ftrainArgsCreate(FTrainArgs* args, FTrainOps ops) {
    TraceRange trace("ftrainArgsCreate");
    return guarded([&] {
        requireNonNull(args, "ftrainArgsCreate: args output must not be null");
        requireNonNull(ops, "ftrainArgsCreate: ops handle must not be null");
        *args = new FTrainArgsStruct{ops->ops.makeArgs()};
    });
}

FTrainStatus ftrainArgsDestroy(FTrainArgs args) {
    return guarded([&] {
        requireNonNull(args, "ftrainArgsDestroy: args handle must not be null");
        delete args;
    });
}

FTrainStatus ftrainArgsSetTensor(FTrainArgs args, FTrainTensorId tensor, FTrainStorageView storage_view) {
    return guarded([&] {
        requireNonNull(args, "ftrainArgsSetTensor: args handle must not be null");
        args->args.setOperand(tensor.opaque, OperandValue(Tensor{StorageView(storage_view)}));
    });
}

FTrainStatus ftrainArgsSetTensorList(FTrainArgs args, FTrainTensorListId tensor_list,
                                     const FTrainStorageView storage_views[], uint32_t num_storage_views) {
    return guarded([&] {
        requireNonNull(args, "ftrainArgsSetTensorList: args handle must not be null");
        if (storage_views == nullptr && num_storage_views != 0)
            raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                            "ftrainArgsSetTensorList: storage_views must not be null when num_storage_views is %u",
                            num_storage_views);
        TensorList list;
        list.views.reserve(num_storage_views);
        for (uint32_t i = 0; i < num_storage_views; ++i) list.views.emplace_back(storage_views[i]);
        args->args.setOperand(tensor_list.opaque, OperandValue(std::move(list)));
    });
}

FTrainStatus ftrainArgsSetGroupedTensor(FTrainArgs args, FTrainGroupedTensorId grouped_tensor, uint32_t num_groups,
                                        FTrainStorageView data, const FTrainStorageView* offsets,
                                        const FTrainStorageView dim_sizes[], const FTrainStorageView strides[]) {
    return guarded([&] {
        requireNonNull(args, "ftrainArgsSetGroupedTensor: args handle must not be null");
        StorageView data_view(data);
        std::optional<StorageView> offsets_view;
        if (offsets != nullptr) offsets_view.emplace(*offsets);
        std::vector<StorageView> sizes, steps;
        if (dim_sizes != nullptr)
            for (std::size_t d = 0; d < data.num_dims; ++d) sizes.emplace_back(dim_sizes[d]);
        if (strides != nullptr)
            for (std::size_t d = 0; d < data.num_dims; ++d) steps.emplace_back(strides[d]);
        args->args.setOperand(grouped_tensor.opaque,
                              OperandValue(GroupedTensor(num_groups, std::move(data_view), std::move(offsets_view),
                                                         std::move(sizes), std::move(steps))));
    });
}

FTrainStatus ftrainArgsSetGemm(FTrainArgs args, FTrainGemmOpId op, FTrainNumericType compute_type) {
    return setOperation(args, op.opaque, OperationKind::kGemm, compute_type, "ftrainArgsSetGemm");
}

FTrainStatus ftrainArgsSetGroupedABCDGemm(FTrainArgs args, FTrainGroupedABCDGemmOpId op,
                                          FTrainNumericType compute_type) {
    return setOperation(args, op.opaque, OperationKind::kGroupedABCDGemm, compute_type,
                        "ftrainArgsSetGroupedABCDGemm");
}

FTrainStatus ftrainArgsSetGroupedBCDGemm(FTrainArgs args, FTrainGroupedBCDGemmOpId op, FTrainNumericType compute_type) {
    return setOperation(args, op.opaque, OperationKind::kGroupedBCDGemm, compute_type, "ftrainArgsSetGroupedBCDGemm");
}

FTrainStatus ftrainArgsSetGroupedABGemm(FTrainArgs args, FTrainGroupedABGemmOpId op, FTrainNumericType compute_type) {
    return setOperation(args, op.opaque, OperationKind::kGroupedABGemm, compute_type, "ftrainArgsSetGroupedABGemm");
}

// ---------------------------------------------------------------- Plan

FTrainStatus ftrainPlanCreate(FTrainPlan* plan, FTrainArgs args) {
    TraceRange trace("ftrainPlanCreate");
    return guarded([&] {
        requireNonNull(plan, "ftrainPlanCreate: plan output must not be null");
        requireNonNull(args, "ftrainPlanCreate: args handle must not be null");
        const auto engine = globalHandle().find(args->args.key());
        if (!engine) raise(FTRAIN_STATUS_INTERNAL_ERROR, "OpsEngine registered for Args is unavailable");
        auto made = std::make_unique<FTrainPlanStruct>(FTrainPlanStruct{engine->createPlan(args->args)});
        made->plan.prepare();
        *plan = made.release();
    });
}

FTrainStatus ftrainPlanDestroy(FTrainPlan plan) {
    return guarded([&] {
        requireNonNull(plan, "ftrainPlanDestroy: plan handle must not be null");
        delete plan;
    });
}

FTrainStatus ftrainPlanGetNumPrimitives(FTrainPlan plan, uint64_t* num_primitives) {
    return guarded([&] {
        requireNonNull(plan, "ftrainPlanGetNumPrimitives: plan handle must not be null");
        requireNonNull(num_primitives, "ftrainPlanGetNumPrimitives: num_primitives output must not be null");
        *num_primitives = plan->plan.size();
    });
}

FTrainStatus ftrainPlanGetPrimitiveName(FTrainPlan plan, uint64_t primitive_index, const char** name) {
    return guarded([&] {
        requireNonNull(plan, "ftrainPlanGetPrimitiveName: plan handle must not be null");
        requireNonNull(name, "ftrainPlanGetPrimitiveName: name output must not be null");
        *name = plan->plan.primitiveName(primitive_index);
    });
}

FTrainStatus ftrainPlanGetPrimitiveRequiredWorkspaceBytes(FTrainPlan plan, uint64_t primitive_index,
                                                          uint64_t* workspace_bytes) {
    return guarded([&] {
        requireNonNull(plan, "ftrainPlanGetPrimitiveRequiredWorkspaceBytes: plan handle must not be null");
        requireNonNull(workspace_bytes,
                       "ftrainPlanGetPrimitiveRequiredWorkspaceBytes: workspace_bytes output must not be null");
        *workspace_bytes = plan->plan.requiredWorkspaceBytes(primitive_index);
    });
}

FTrainStatus ftrainPlanExecutePrimitive(FTrainPlan plan, uint64_t primitive_index, void* workspace,
                                        uint64_t workspace_bytes, FTrainStream stream) {
    TraceRange trace("ftrainPlanExecutePrimitive");
    return guarded([&] {
        requireNonNull(plan, "ftrainPlanExecutePrimitive: plan handle must not be null");
        plan->plan.execute(primitive_index, workspace, workspace_bytes, stream);
    });
}

// ---------------------------------------------------------------- convenience

FTrainStatus ftrainGemm(FTrainStorageView a, FTrainStorageView b, FTrainStorageView c, FTrainStorageView d,
                        FTrainStorageView alpha, FTrainStorageView beta, FTrainNumericType compute_type,
                        void* workspace, uint64_t workspace_bytes, FTrainStream stream) {
    TraceRange trace("ftrainGemm");
    const FTrainStorageView* views[6] = {&a, &b, &c, &d, &alpha, &beta};
    return convenienceGemm(views, compute_type, workspace, workspace_bytes, stream, nullptr);
}

FTrainStatus ftrainGemmNoAlloc(FTrainStorageView a, FTrainStorageView b, FTrainStorageView c, FTrainStorageView d,
                               FTrainStorageView alpha, FTrainStorageView beta, FTrainNumericType compute_type,
                               FTrainStream stream) {
    TraceRange trace("ftrainGemmNoAlloc");
    DeviceScratch scratch{};
    const FTrainStatus s = guarded([&] { scratch = deviceScratch(); });
    if (s != FTRAIN_STATUS_SUCCESS) return s;
    const FTrainStorageView* views[6] = {&a, &b, &c, &d, &alpha, &beta};
    return convenienceGemm(views, compute_type, nullptr, 0, stream, &scratch);
}

}  // extern "C"

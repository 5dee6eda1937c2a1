// GEMM Primitives: one Primitive per kernel variant of the catalog.
//
// The applicability checklist starts with the reference Fp32Gemm's rules
// (src/primitive/hygon/gemm/fp32_gemm.cpp:27-62), with the same reason
// strings, then adds each variant's own limits.  configure() turns the
// problem into a ready launch (kernel, grid, packed parameters, host-side
// alpha/beta values) so run() is one or two hipLaunchKernel calls.
#include <limits>

#include <hip/hip_runtime.h>

#include "ft/gemm.hpp"

namespace ftrain {
namespace {

using gemm::GemmParams;
using gemm::HalfGemmParams;
using gemm::ReduceParams;
using gemm::SplitKind;
using gemm::Variant;
using gemm::VariantInfo;
using gemm::WideParams;

uint64_t ceilDiv(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

bool floatAligned(const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % alignof(float) == 0; }
bool vecAligned(const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0; }
bool aligned(const void* p, uintptr_t n) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % n == 0; }

uintptr_t elementBytes(FTrainNumericType t) { return t == FTRAIN_NUMERIC_TYPE_FP32 ? 4 : 2; }

// Element types a variant takes.  fp32 variants: the reference Fp32Gemm's
// rule, every port fp32 (fp32_gemm.cpp:28-37).  bf16 / fp16 variants: a and
// b in that type, c and d both fp32 or both that type, alpha and beta fp32.
Result typeChecks(const GemmProblem& p, FTrainNumericType input) {
    if (p.computeType() != FTRAIN_NUMERIC_TYPE_FP32) return Result(FTRAIN_STATUS_UNSUPPORTED, "compute type is not fp32");
    if (input == FTRAIN_NUMERIC_TYPE_FP32) {
        for (int i = 0; i < 6; ++i)
            if (p.port(i).numericType() != FTRAIN_NUMERIC_TYPE_FP32)
                return Result(FTRAIN_STATUS_UNSUPPORTED, "an operand is not fp32");
        return Result{};
    }
    const bool bf16 = input == FTRAIN_NUMERIC_TYPE_BF16;
    if (p.a().numericType() != input || p.b().numericType() != input)
        return Result(FTRAIN_STATUS_UNSUPPORTED, bf16 ? "a or b is not bf16" : "a or b is not fp16");
    const FTrainNumericType cd = p.d().numericType();
    // A null c (no beta term) carries no data; its declared type is not checked.
    if ((cd != FTRAIN_NUMERIC_TYPE_FP32 && cd != input) || (p.c().memory() != nullptr && p.c().numericType() != cd))
        return Result(FTRAIN_STATUS_UNSUPPORTED, bf16 ? "c and d must both be fp32 or both bf16"
                                                      : "c and d must both be fp32 or both fp16");
    if (p.alpha().numericType() != FTRAIN_NUMERIC_TYPE_FP32 || p.beta().numericType() != FTRAIN_NUMERIC_TYPE_FP32)
        return Result(FTRAIN_STATUS_UNSUPPORTED, "alpha or beta is not fp32");
    return Result{};
}

// Rules every variant shares (reference fp32_gemm.cpp:27-62), for the
// variant's input type.
Result commonChecks(const GemmProblem& p, FTrainNumericType input) {
    if (Result r = typeChecks(p, input); !r.isSuccess()) return r;
    // alpha and beta: continuous scalars.  a, b, c, d: continuous, or
    // explicit strides with one unit dimension (GemmProblem::launch).
    for (int i = 4; i < 6; ++i)
        if (p.port(i).indexType() != FTRAIN_INDEX_TYPE_CONTINUOUS)
            return Result(FTRAIN_STATUS_UNSUPPORTED, "an operand is not continuously indexed");
    GemmLaunch g;
    if (const char* why = p.launch(g)) return Result(FTRAIN_STATUS_UNSUPPORTED, why);
    for (int i = 0; i < 6; ++i)
        if (!aligned(p.port(i).memory(), elementBytes(p.port(i).numericType())))
            return Result(FTRAIN_STATUS_UNSUPPORTED, input == FTRAIN_NUMERIC_TYPE_FP32
                                                         ? "an operand address is not float-aligned"
                                                         : "an operand address is not aligned to its element size");
    if (p.emptyOutput()) return Result{};
    const GemmShape s = p.shape();
    if (p.d().memory() == nullptr || (s.k != 0 && (p.a().memory() == nullptr || p.b().memory() == nullptr)))
        return Result(FTRAIN_STATUS_UNSUPPORTED, "a required operand address is null");
    return Result{};
}

// The launch's workgroup size must equal the kernel's launch bounds (every
// kernel here declares its exact size: a larger launch fails, a smaller one
// would leave part of each tile uncomputed).  Checked when HIP can describe
// the kernel, i.e. on a host with a device.
void checkBlockSize(const void* kernel, int threads, const char* name) {
    hipFuncAttributes attr{};
    if (hipFuncGetAttributes(&attr, kernel) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    if (attr.maxThreadsPerBlock != threads)
        raise(FTRAIN_STATUS_INTERNAL_ERROR, "%s: workgroup size %d does not match the kernel's launch bounds %d",
                        name, threads, attr.maxThreadsPerBlock);
}

void check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        raise(FTRAIN_STATUS_INTERNAL_ERROR, "%s launch failed: %s", what, hipGetErrorString(e));
}

class GemmPrimitive final : public Primitive<GemmProblem> {
  public:
    explicit GemmPrimitive(Variant v)
        : v_(v), info_(&gemm::info(v)), half_(gemm::info(v).input != FTRAIN_NUMERIC_TYPE_FP32) {}

    const char* name() const noexcept override { return info_->name; }
    std::unique_ptr<PrimitiveBase> clone() const override { return std::make_unique<GemmPrimitive>(*this); }
    // Split-k partial tiles: Primitive 0 of a Plan made by ftrainPlanCreate
    // owns its buffer (allocated at Plan creation), so it needs none; any
    // other split Primitive needs its partial bytes from the caller.
    uint64_t requiredWorkspaceBytes() const noexcept override { return owned_ ? 0 : partial_bytes_; }
    uint64_t scratchBytes() const noexcept override { return partial_bytes_; }

    void prepare(bool default_slot) override {
        if (!default_slot || partial_bytes_ == 0 || owned_) return;
        void* q = nullptr;
        if (hipMalloc(&q, partial_bytes_) != hipSuccess) {
            (void)hipGetLastError();
            raise(FTRAIN_STATUS_OUT_OF_MEMORY, "%s: split-k partial buffer of %llu bytes", info_->name,
                  static_cast<unsigned long long>(partial_bytes_));
        }
        owned_.reset(q, [](void* x) { (void)hipFree(x); });
        // The arrival counters start at 0; every launch leaves them 0.
        if (hipMemset(q, 0, gemm::kCounterBytes) != hipSuccess) {
            (void)hipGetLastError();
            raise(FTRAIN_STATUS_INTERNAL_ERROR, "%s: clearing the split-k counters failed", info_->name);
        }
    }

    Result isApplicable(const GemmProblem& p, const Constraints& constraints) const override {
        Result r = commonChecks(p, info_->input);
        if (!r.isSuccess() || p.emptyOutput()) return r;
        GemmLaunch g;
        (void)p.launch(g);  // succeeded in commonChecks
        const GemmShape s = g.shape;
        if (gemm::kernelFor(v_, g.ta, g.tb) == nullptr)
            return Result(FTRAIN_STATUS_UNSUPPORTED, "this variant has no kernel for these operand orientations");
        if (!info_->simt) {
            constexpr uint64_t kMax = std::numeric_limits<int32_t>::max();
            if (s.m > kMax || s.n > kMax || s.k > kMax)
                return Result(FTRAIN_STATUS_UNSUPPORTED, "a dimension exceeds the 32-bit kernel limit");
            if (ceilDiv(s.m, info_->bm) * ceilDiv(s.n, info_->bn) > kMax)
                return Result(FTRAIN_STATUS_UNSUPPORTED, "the tile count exceeds the grid limit");
        }
        if (info_->vec && half_) {
            // 16-byte accesses (8 elements) along a's and b's contiguous
            // dimensions; c and d are accessed per element.
            const uint64_t a_run = g.ta ? s.m : s.k, b_run = g.tb ? s.k : s.n;
            if (a_run % 8 != 0 || b_run % 8 != 0)
                return Result(FTRAIN_STATUS_UNSUPPORTED,
                              "a contiguous extent of a or b is not a multiple of 8 (16-byte loads)");
            if (g.lda % 8 != 0 || g.ldb % 8 != 0)
                return Result(FTRAIN_STATUS_UNSUPPORTED, "a leading dimension of a or b is not a multiple of 8");
            if (!vecAligned(g.a) || !vecAligned(g.b))
                return Result(FTRAIN_STATUS_UNSUPPORTED, "a or b is not 16-byte aligned");
        } else if (info_->vec) {
            // 128-bit accesses along each matrix's contiguous dimension:
            // that extent and every leading dimension a multiple of 4.
            const uint64_t a_run = g.ta ? s.m : s.k, b_run = g.tb ? s.k : s.n;
            if (s.n % 4 != 0 || a_run % 4 != 0 || b_run % 4 != 0)
                return Result(FTRAIN_STATUS_UNSUPPORTED,
                              "n or a contiguous matrix extent is not a multiple of 4 (128-bit loads)");
            if (g.lda % 4 != 0 || g.ldb % 4 != 0 || g.ldc % 4 != 0 || g.ldd % 4 != 0)
                return Result(FTRAIN_STATUS_UNSUPPORTED, "a leading dimension is not a multiple of 4 (128-bit loads)");
            for (int i = 0; i < 4; ++i)
                if (!vecAligned(p.port(i).memory()))
                    return Result(FTRAIN_STATUS_UNSUPPORTED, "a matrix address is not 16-byte aligned");
        }
        if (v_ >= Variant::kMfma16Dma256x256 && v_ <= Variant::kMfma16Dma128x64 &&
            (s.k == 0 || g.lda >= (int64_t(1) << 22) || g.ldb >= (int64_t(1) << 22) || g.ldc >= (int64_t(1) << 21) ||
             g.ldd >= (int64_t(1) << 21)))
            return Result(FTRAIN_STATUS_UNSUPPORTED,
                          "needs k positive, leading dimensions of a and b below 2^22 and of c and d below 2^21 "
                          "(DMA stages, 32-bit offsets)");
        if (v_ >= Variant::kBf16MfmaDma256x256 && v_ <= Variant::kFp16MfmaDma64x128S &&
            (s.k == 0 || g.lda >= (int64_t(1) << 23) || g.ldb >= (int64_t(1) << 23) || g.ldc >= (int64_t(1) << 21) ||
             g.ldd >= (int64_t(1) << 21)))
            return Result(FTRAIN_STATUS_UNSUPPORTED,
                          "needs k positive, leading dimensions of a and b below 2^23 and of c and d below 2^21 "
                          "(DMA stages, 32-bit offsets)");
        if ((v_ == Variant::kBf16MfmaDma128x128S || v_ == Variant::kFp16MfmaDma128x128S ||
             v_ == Variant::kBf16MfmaDma64x128S || v_ == Variant::kFp16MfmaDma64x128S) &&
            s.n >= (uint64_t(1) << 21))
            return Result(FTRAIN_STATUS_UNSUPPORTED, "n of 2^21 or more (32-bit offsets into the partial slices)");
        if ((v_ == Variant::kBf16MfmaDma64x128S || v_ == Variant::kFp16MfmaDma64x128S) && s.m > 64)
            return Result(FTRAIN_STATUS_UNSUPPORTED, "m above 64 (the 64-row tile is for shapes one tile high)");
        if (info_->gemv && s.m > uint64_t(info_->bm))
            return Result(FTRAIN_STATUS_UNSUPPORTED, "m exceeds the skinny-kernel row limit");
        if (info_->split == SplitKind::kPartial &&
            gemm::chooseSplits(v_, s, gemm::computeUnits(constraints.device())) == 0)
            return Result(FTRAIN_STATUS_UNSUPPORTED, "reduction depth too shallow to split");
        if (info_->split == SplitKind::kFused &&
            ceilDiv(s.m, info_->bm) * ceilDiv(s.n, info_->bn) > gemm::kMaxFusedTiles)
            return Result(FTRAIN_STATUS_UNSUPPORTED, "more output tiles than the deep-k kernel's arrival counters");
        return Result{};
    }

    void configure(const GemmProblem& p) override {
        owned_.reset();
        empty_ = p.emptyOutput();
        if (empty_) return;
        GemmLaunch g;
        if (const char* why = p.launch(g)) raise(FTRAIN_STATUS_UNSUPPORTED, "%s", why);
        const GemmShape s = g.shape;
        const float alpha = *static_cast<const float*>(p.alpha().memory());
        const float beta  = *static_cast<const float*>(p.beta().memory());
        const auto* a     = static_cast<const float*>(g.a);
        const auto* b     = static_cast<const float*>(g.b);
        const auto* c     = static_cast<const float*>(g.c);
        auto* d           = static_cast<float*>(g.d);
        const int64_t a_rs = g.ta ? 1 : g.lda, a_cs = g.ta ? g.lda : 1;
        const int64_t b_rs = g.tb ? 1 : g.ldb, b_cs = g.tb ? g.ldb : 1;
        wide_ = WideParams{a, b, c, d, alpha, beta, s.m, s.n, s.k, a_rs, a_cs, b_rs, b_cs, g.ldc, g.ldd};

        int threads = info_->threads;
        const bool prefetch_b = gemm::prefetchB(s.k * s.n * (half_ ? 2 : 4), s.k);
        kernel_     = info_->gemv && info_->split == SplitKind::kNone ? gemm::gemvKernel(v_, int(s.m), g.ta, threads)
                                                                  : gemm::kernelFor(v_, g.ta, g.tb, prefetch_b);
        checkBlockSize(kernel_, threads, info_->name);
        block_  = dim3(threads);
        if (info_->simt) {
            const uint64_t tiles = ceilDiv(s.m, 64) * ceilDiv(s.n, 64);
            grid_                = dim3(static_cast<uint32_t>(std::min<uint64_t>(tiles, 1u << 20)));
            return;
        }
        const int cus   = gemm::computeUnits(getCurrentDeviceIdOr(0));
        const bool split = info_->split != SplitKind::kNone;
        uint32_t splits = split ? gemm::chooseSplits(v_, s, cus) : 1;
        uint64_t chunk  = s.k;
        if (split) {
            const uint64_t step = info_->gemv ? 1 : uint64_t(info_->bk);
            chunk               = ceilDiv(ceilDiv(s.k, splits), step) * step;
            splits              = chunk == 0 ? 1 : static_cast<uint32_t>(ceilDiv(s.k, chunk));
        }
        params_ = GemmParams{a,      b,      c,     d,     alpha, beta,   int32_t(s.m), int32_t(s.n), int32_t(s.k),
                             int32_t(chunk), 0, 0, g.lda, g.ldb, g.ldc, g.ldd};
        const bool cd_half = p.d().numericType() != FTRAIN_NUMERIC_TYPE_FP32;
        half_params_       = HalfGemmParams{g.a,          g.b,          g.c,          g.d,   alpha, beta,
                                      int32_t(s.m), int32_t(s.n), int32_t(s.k), int32_t(chunk),
                                      0,            0,            g.lda,        g.ldb, g.ldc, g.ldd,
                                      int32_t(cd_half)};
        if (info_->gemv) {
            grid_ = dim3(static_cast<uint32_t>(ceilDiv(s.n, uint64_t(info_->bn))), 1, splits);
        } else {
            params_.tiles_m = half_params_.tiles_m = int32_t(ceilDiv(s.m, info_->bm));
            params_.tiles_n = half_params_.tiles_n = int32_t(ceilDiv(s.n, info_->bn));
            grid_           = dim3(uint32_t(params_.tiles_m) * uint32_t(params_.tiles_n), 1, splits);
        }
        const uint64_t count = s.m * s.n;
        if (info_->split == SplitKind::kFused) {
            // One launch of tiles x splits workgroups (grid x); with splits >
            // 1 the buffer holds the tiles' arrival counters, then the
            // partial tiles.
            const uint64_t tiles = uint64_t(params_.tiles_m) * uint64_t(params_.tiles_n);
            grid_          = dim3(uint32_t(tiles * splits));
            deepk_         = gemm::DeepKParams{params_, nullptr, nullptr, int32_t(splits)};
            partial_bytes_ = splits > 1 ? gemm::kCounterBytes + uint64_t(splits) * tiles * info_->bm * info_->bn * sizeof(float) : 0;
            fused_tiles_   = int32_t(tiles);
        }
        if (info_->split == SplitKind::kPartial) {
            partial_bytes_ = gemm::kCounterBytes + uint64_t(splits) * count * sizeof(float);
            const int32_t cd_type = !cd_half ? gemm::kCdFp32
                                    : p.d().numericType() == FTRAIN_NUMERIC_TYPE_BF16 ? gemm::kCdBf16
                                                                                     : gemm::kCdFp16;
            reduce_ = ReduceParams{nullptr, g.c, g.d, alpha, beta, count, s.n, g.ldc, g.ldd, int32_t(splits), cd_type};
            // isApplicable guaranteed n, ldc, ldd % 4 == 0 and 16-byte bases
            // for the fp32 vec variants; the half variants reduce four at a
            // time when c and d are fp32 and meet the same conditions.
            const auto a16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
            reduce_vec_ = info_->vec && (!half_ || (!cd_half && s.n % 4 == 0 && g.ldd % 4 == 0 && a16(g.d) &&
                                                    (g.c == nullptr || (g.ldc % 4 == 0 && a16(g.c)))));
            const uint64_t units = reduce_vec_ ? count / 4 : count;
            // One thread per unit also when there are few splits: the 16-thread form then idles
            // most of its threads (measured on MI355X, 65536 float4 units: 2.6 against 2.9 us at
            // 4 splits, 3.3 at 8).
            reduce_wide_         = units >= gemm::kWideReduceUnits || splits <= 8;
            // splitk_reduce: 16 output units per block (16 threads each); the
            // wide form 256 units per block.
            aux_grid_ = dim3(static_cast<uint32_t>(std::min<uint64_t>(ceilDiv(units, reduce_wide_ ? 256 : 16), 65535)));
        }
    }

  protected:
    void run(const Resources& r) override {
        if (empty_) return;
        if (info_->simt) {
            void* args[] = {&wide_};
            check(hipLaunchKernel(kernel_, grid_, block_, args, 0, r.stream), info_->name);
            return;
        }
        GemmParams params          = params_;
        HalfGemmParams half_params = half_params_;
        void* args[]               = {half_ ? static_cast<void*>(&half_params) : static_cast<void*>(&params)};
        switch (info_->split) {
            case SplitKind::kNone:
                check(hipLaunchKernel(kernel_, grid_, block_, args, 0, r.stream), info_->name);
                break;
            case SplitKind::kPartial: {
                // Partial tiles go to the caller's workspace when it is large
                // and aligned enough, else to the buffer this Primitive got
                // at Plan creation.  Nothing is allocated here, so every
                // execution, the first included, can be captured.  Executions
                // of one Plan are serialised by the caller (reference
                // common.h:576), so they may share the owned buffer.
                const bool caller = r.workspace != nullptr && r.workspace_bytes >= partial_bytes_ &&
                                    reinterpret_cast<uintptr_t>(r.workspace) % 16 == 0;
                void* ws = caller ? r.workspace : owned_.get();
                if (ws == nullptr)
                    raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                          "%s requires a 16-byte aligned workspace of %llu bytes for its split-k partial tiles",
                          info_->name, static_cast<unsigned long long>(partial_bytes_));
                char* const partials = static_cast<char*>(ws) + gemm::kCounterBytes;
                params.d           = reinterpret_cast<float*>(partials);
                half_params.d      = partials;
                ReduceParams red   = reduce_;
                red.partials       = reinterpret_cast<const float*>(partials);
                void* rargs[]      = {&red};
                hipError_t e       = hipLaunchKernel(kernel_, grid_, block_, args, 0, r.stream);
                if (e == hipSuccess)
                    e = hipLaunchKernel(gemm::reduceKernel(reduce_vec_, reduce_wide_), aux_grid_, dim3(256), rargs, 0, r.stream);
                check(e, info_->name);
                break;
            }
            case SplitKind::kFused: {
                gemm::DeepKParams dp = deepk_;
                void* dargs[]  = {&dp};
                if (dp.splits > 1) {
                    // Counters and partials in the buffer the kPartial case
                    // would use.  A caller's workspace starts with arbitrary
                    // contents: its counters are cleared first (a kernel,
                    // not a memset, so the launch pair can be captured).
                    const bool caller = r.workspace != nullptr && r.workspace_bytes >= partial_bytes_ &&
                                        reinterpret_cast<uintptr_t>(r.workspace) % 16 == 0;
                    void* ws = caller ? r.workspace : owned_.get();
                    if (ws == nullptr)
                        raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                              "%s requires a 16-byte aligned workspace of %llu bytes for its split-k partial tiles",
                              info_->name, static_cast<unsigned long long>(partial_bytes_));
                    dp.counters = static_cast<unsigned int*>(ws);
                    dp.partials = reinterpret_cast<float*>(static_cast<char*>(ws) + gemm::kCounterBytes);
                    if (caller && !r.counters_clear) {
                        unsigned int* counters = dp.counters;
                        int n                  = fused_tiles_;
                        void* cargs[]          = {&counters, &n};
                        check(hipLaunchKernel(gemm::deepkClearKernel(), dim3(uint32_t(ceilDiv(uint64_t(n), 256))),
                                              dim3(256), cargs, 0, r.stream),
                              info_->name);
                    }
                }
                check(hipLaunchKernel(kernel_, grid_, block_, dargs, 0, r.stream), info_->name);
                break;
            }
        }
    }

  public:
    // clone() copies; the launch argument arrays must then point at the
    // copy's own parameter blocks.
    GemmPrimitive(const GemmPrimitive&) = default;
    GemmPrimitive& operator=(const GemmPrimitive&) = delete;

  private:
    static FTrainDeviceId getCurrentDeviceIdOr(FTrainDeviceId fallback) {
        int dev = 0;
        return hipGetDevice(&dev) == hipSuccess ? dev : fallback;
    }

    Variant v_;
    const VariantInfo* info_;
    bool half_;  // bf16 / fp16 inputs (HalfGemmParams)
    bool empty_         = true;
    const void* kernel_ = nullptr;
    dim3 grid_, block_, aux_grid_;
    GemmParams params_{};
    HalfGemmParams half_params_{};
    WideParams wide_{};
    ReduceParams reduce_{};
    gemm::DeepKParams deepk_{};
    int32_t fused_tiles_ = 0;
    bool reduce_vec_        = false;
    bool reduce_wide_       = false;
    uint64_t partial_bytes_ = 0;
    std::shared_ptr<void> owned_;  // split-k partials of Primitive 0 (shared by clones)
};

}  // namespace

// Registration order is the engine's fallback preference when no Finder
// contributes (e.g. FTRAIN_DISABLED_FINDERS=ShapeCost): general large tiles
// first, the universal SIMT kernel last.
std::vector<std::shared_ptr<const Primitive<GemmProblem>>> GemmFamily::makeRecords() {
    std::vector<std::shared_ptr<const Primitive<GemmProblem>>> records;
    for (int i = 0; i < static_cast<int>(Variant::kCount); ++i)
        records.push_back(std::make_shared<GemmPrimitive>(static_cast<Variant>(i)));
    return records;
}

}  // namespace ftrain

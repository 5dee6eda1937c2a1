// Grouped GEMM families: operand expansion and validation, selection key,
// Patterns, and the grouped Primitives (one launch over every group's
// tiles).  See ft/grouped.hpp for the operand forms; the addressing rule
// follows include/flash_train/common.h:397-425 of the reference.
#include "ft/grouped.hpp"

#include <algorithm>
#include <limits>

#include <hip/hip_runtime.h>

#include "ft/gemm_kernels.hpp"

namespace ftrain {
namespace {

using gemm::GemmParams;
using gemm::GroupedGemmArgs;
using gemm::GroupedHalfArgs;
using gemm::HalfGemmParams;

const char* groupName(int i) {
    static const char* const names[] = {"a", "b", "c", "d"};
    return names[i];
}

// Values of a rank-one descriptor array of `groups` integers in host memory.
std::vector<int64_t> readIndexArray(const StorageView& v, uint32_t groups, const char* operand, const char* what) {
    if (!v.isHost())
        raise(FTRAIN_STATUS_UNSUPPORTED, "grouped %s: %s must be in host memory", operand, what);
    std::vector<int64_t> out(groups);
    if (groups == 0) return out;
    if (v.memory() == nullptr)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "grouped %s: %s memory is null", operand, what);
    const void* m = v.memory();
    for (uint32_t g = 0; g < groups; ++g) {
        switch (v.numericType()) {
            case FTRAIN_NUMERIC_TYPE_INT64: out[g] = static_cast<const int64_t*>(m)[g]; break;
            case FTRAIN_NUMERIC_TYPE_INT32: out[g] = static_cast<const int32_t*>(m)[g]; break;
            case FTRAIN_NUMERIC_TYPE_UINT32: out[g] = static_cast<const uint32_t*>(m)[g]; break;
            case FTRAIN_NUMERIC_TYPE_UINT64: {
                const uint64_t x = static_cast<const uint64_t*>(m)[g];
                if (x > static_cast<uint64_t>(std::numeric_limits<int64_t>::max()))
                    raise(FTRAIN_STATUS_INVALID_ARGUMENT, "grouped %s: %s[%u] is out of range", operand,
                                    what, g);
                out[g] = static_cast<int64_t>(x);
                break;
            }
            default:
                raise(FTRAIN_STATUS_UNSUPPORTED, "grouped %s: %s must hold int32, uint32, int64 or uint64",
                                operand, what);
        }
    }
    return out;
}

// Layout of a rows x cols matrix with element strides (s0, s1): row-major
// (unit column stride) or column-major (unit row stride) with a leading
// dimension covering the other extent.
const char* groupLayout(int64_t rows, int64_t cols, int64_t s0, int64_t s1, MatrixLayout& out) {
    if (s0 < 0 || s1 < 0) return "a group stride is negative";
    const bool unit_cols = cols <= 1 || s1 == 1;
    const bool unit_rows = rows <= 1 || s0 == 1;
    constexpr int64_t max_off = std::numeric_limits<int64_t>::max() / 8;
    const auto span       = [](int64_t n, int64_t s) { return n <= 1 ? 0 : (s > max_off / (n - 1) ? max_off : (n - 1) * s); };
    if (span(rows, s0) >= max_off || span(cols, s1) >= max_off || span(rows, s0) + span(cols, s1) >= max_off)
        return "a group extent overflows the address range";
    if (unit_cols && (rows <= 1 || s0 >= cols)) {
        out = MatrixLayout{false, rows <= 1 ? std::max<int64_t>(cols, 1) : s0};
        return nullptr;
    }
    if (unit_rows && (cols <= 1 || s1 >= rows)) {
        out = MatrixLayout{true, cols <= 1 ? std::max<int64_t>(rows, 1) : s1};
        return nullptr;
    }
    return "group strides need a unit stride in one dimension and a non-overlapping leading dimension";
}

size_t elementBytes(FTrainNumericType t) {
    switch (t) {
        case FTRAIN_NUMERIC_TYPE_FP64:
        case FTRAIN_NUMERIC_TYPE_INT64:
        case FTRAIN_NUMERIC_TYPE_UINT64: return 8;
        case FTRAIN_NUMERIC_TYPE_FP32:
        case FTRAIN_NUMERIC_TYPE_INT32:
        case FTRAIN_NUMERIC_TYPE_UINT32: return 4;
        case FTRAIN_NUMERIC_TYPE_FP16:
        case FTRAIN_NUMERIC_TYPE_BF16:
        case FTRAIN_NUMERIC_TYPE_INT16:
        case FTRAIN_NUMERIC_TYPE_UINT16: return 2;
        default: return 1;
    }
}

GroupOperand expandGrouped(const GroupedTensor& gt, int which) {
    const char* name     = groupName(which);
    const StorageView& v = gt.data();
    if (v.rank() != 2)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "grouped Gemm operand %s needs rank-two data, got rank %zu",
                        name, v.rank());
    if (v.isHost())
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "grouped Gemm operand %s must be in device memory", name);
    const uint32_t G = gt.numGroups();
    std::vector<int64_t> rows(G, v.dims()[0]), cols(G, v.dims()[1]);
    if (!gt.dimSizes().empty()) {
        rows = readIndexArray(gt.dimSizes()[0], G, name, "dim_sizes[0]");
        cols = readIndexArray(gt.dimSizes()[1], G, name, "dim_sizes[1]");
    }
    for (uint32_t g = 0; g < G; ++g)
        if (rows[g] < 0 || cols[g] < 0)
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "grouped %s: group %u has a negative size", name, g);
    std::vector<int64_t> s0(G), s1(G, 1);
    if (!gt.strides().empty()) {
        s0 = readIndexArray(gt.strides()[0], G, name, "strides[0]");
        s1 = readIndexArray(gt.strides()[1], G, name, "strides[1]");
    } else {
        for (uint32_t g = 0; g < G; ++g) s0[g] = cols[g];
    }
    // Element offsets stay below this bound, with each group's extent, so
    // that byte addresses cannot overflow.
    constexpr int64_t max_off = std::numeric_limits<int64_t>::max() / 8;
    std::vector<int64_t> off(G, 0);
    if (gt.offsets()) {
        off = readIndexArray(*gt.offsets(), G, name, "offsets");
    } else {
        int64_t run = 0;
        for (uint32_t g = 0; g < G; ++g) {
            off[g] = run;
            if (rows[g] != 0 && cols[g] > (max_off - run) / rows[g])
                raise(FTRAIN_STATUS_OVERFLOW, "grouped %s: packed group offsets overflow", name);
            run += rows[g] * cols[g];
        }
    }
    GroupOperand out;
    out.type = v.numericType();
    out.groups.resize(G);
    const size_t eb = elementBytes(out.type);
    for (uint32_t g = 0; g < G; ++g) {
        if (off[g] < 0) raise(FTRAIN_STATUS_INVALID_ARGUMENT, "grouped %s: offsets[%u] is negative", name, g);
        if (off[g] >= max_off)
            raise(FTRAIN_STATUS_OVERFLOW, "grouped %s: offsets[%u] overflows the address range", name, g);
        GroupMatrix& m = out.groups[g];
        m.rows = rows[g];
        m.cols = cols[g];
        m.memory = v.memory() == nullptr ? nullptr : static_cast<const char*>(v.memory()) + static_cast<size_t>(off[g]) * eb;
        if (const char* why = groupLayout(rows[g], cols[g], s0[g], s1[g], m.layout))
            raise(FTRAIN_STATUS_UNSUPPORTED, "grouped %s, group %u: %s", name, g, why);
        // The group's last element: offset plus its (already bounded) extent.
        const int64_t extent = (rows[g] <= 1 ? 0 : (rows[g] - 1) * s0[g]) + (cols[g] <= 1 ? 0 : (cols[g] - 1) * s1[g]);
        if (extent > max_off - off[g])
            raise(FTRAIN_STATUS_OVERFLOW, "grouped %s, group %u: offset plus extent overflows the address range",
                            name, g);
    }
    return out;
}

GroupOperand expandList(const TensorList& tl, int which) {
    const char* name = groupName(which);
    GroupOperand out;
    out.groups.resize(tl.views.size());
    for (size_t g = 0; g < tl.views.size(); ++g) {
        const StorageView& v = tl.views[g];
        if (v.rank() != 2)
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Gemm TensorList %s[%zu] must be rank two, got rank %zu",
                            name, g, v.rank());
        if (v.isHost())
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Gemm TensorList %s[%zu] must be in device memory", name, g);
        if (g == 0)
            out.type = v.numericType();
        else if (v.numericType() != out.type)
            raise(FTRAIN_STATUS_UNSUPPORTED, "Gemm TensorList %s elements differ in numeric type", name);
        GroupMatrix& m = out.groups[g];
        m.rows         = v.dims()[0];
        m.cols         = v.dims()[1];
        m.memory       = v.memory();
        if (const char* why = matrixLayout(v, m.layout))
            raise(FTRAIN_STATUS_UNSUPPORTED, "Gemm TensorList %s[%zu]: %s", name, g, why);
    }
    return out;
}

GroupOperand expand(const OperandValue& value, int which) {
    if (const auto* gt = std::get_if<GroupedTensor>(&value)) return expandGrouped(*gt, which);
    if (const auto* tl = std::get_if<TensorList>(&value)) return expandList(*tl, which);
    raise(FTRAIN_STATUS_INVALID_ARGUMENT, "grouped Gemm operand %s has the wrong storage family",
                    groupName(which));
}

bool nullOperand(const GroupOperand& o) {
    return std::all_of(o.groups.begin(), o.groups.end(), [](const GroupMatrix& m) { return m.memory == nullptr; });
}

}  // namespace

GroupedGemmProblem::GroupedGemmProblem(GroupedKind kind, const OperandValue& a, const OperandValue& b,
                                       const OperandValue& c, const OperandValue& d, Tensor alpha, Tensor beta,
                                       FTrainNumericType compute_type)
    : kind_(kind), alpha_(std::move(alpha)), beta_(std::move(beta)), compute_type_(compute_type) {
    if (alpha_.view.rank() != 0 || beta_.view.rank() != 0)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Gemm requires scalar alpha and beta Tensors");
    if (!alpha_.view.isHost() || !beta_.view.isHost())
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Gemm requires alpha and beta in host memory");
    a_      = expand(a, 0);
    b_      = expand(b, 1);
    c_      = expand(c, 2);
    d_      = expand(d, 3);
    groups_ = static_cast<uint32_t>(d_.groups.size());
    const GroupOperand* ops[4] = {&a_, &b_, &c_, &d_};
    for (int i = 0; i < 4; ++i)
        if (ops[i]->groups.size() != groups_)
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "grouped Gemm operand %s has %zu groups, d has %u",
                            groupName(i), ops[i]->groups.size(), groups_);
    const bool has_c = !nullOperand(c_);
    for (uint32_t g = 0; g < groups_; ++g) {
        const GroupMatrix &ma = a_.groups[g], &mb = b_.groups[g], &mc = c_.groups[g], &md = d_.groups[g];
        if (ma.cols != mb.rows)
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "group %u: a column count %lld does not match b row count %lld",
                            g, static_cast<long long>(ma.cols), static_cast<long long>(mb.rows));
        if (md.rows != ma.rows || md.cols != mb.cols)
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "group %u: d must be m-by-n", g);
        if (has_c && mc.memory != nullptr && (mc.rows != md.rows || mc.cols != md.cols))
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "group %u: c must be m-by-n", g);
        constexpr uint64_t max_elems = std::numeric_limits<uint64_t>::max() / sizeof(double);
        const auto over          = [](int64_t x, int64_t y) {
            return y != 0 && static_cast<uint64_t>(x) > max_elems / static_cast<uint64_t>(y);
        };
        if (over(ma.rows, ma.cols) || over(mb.rows, mb.cols) || over(md.rows, md.cols))
            raise(FTRAIN_STATUS_OVERFLOW, "group %u: matrix byte size overflows uint64_t", g);
    }
}

const char* GroupedGemmProblem::launch(uint32_t g, GemmLaunch& out) const {
    const GroupMatrix &ma = a_.groups[g], &mb = b_.groups[g], &mc = c_.groups[g], &md = d_.groups[g];
    const GemmShape s{static_cast<uint64_t>(ma.rows), static_cast<uint64_t>(mb.cols), static_cast<uint64_t>(ma.cols)};
    MatrixLayout lc = mc.layout;
    const MatrixLayout& ld = md.layout;
    const bool has_c = mc.memory != nullptr;
    if (has_c && lc.col_major != ld.col_major) {
        if (s.m <= 1 || s.n <= 1)
            lc = MatrixLayout{ld.col_major, ld.col_major ? std::max<int64_t>(int64_t(s.m), 1) : std::max<int64_t>(int64_t(s.n), 1)};
        else
            return "c and d must share one orientation";
    }
    if (!ld.col_major)
        out = GemmLaunch{s, ma.memory, mb.memory, mc.memory, const_cast<void*>(md.memory),
                         ma.layout.col_major, mb.layout.col_major, ma.layout.ld, mb.layout.ld, lc.ld, ld.ld};
    else
        out = GemmLaunch{GemmShape{s.n, s.m, s.k}, mb.memory, ma.memory, mc.memory, const_cast<void*>(md.memory),
                         !mb.layout.col_major, !ma.layout.col_major, mb.layout.ld, ma.layout.ld, lc.ld, ld.ld};
    if (!has_c) out.ldc = out.ldd;
    return nullptr;
}

std::vector<uint64_t> GroupedGemmProblem::key() const {
    std::vector<uint64_t> k;
    k.reserve(8 + groups_ * 40);
    k.insert(k.end(), {uint64_t(kind_), groups_, a_.type, b_.type, c_.type, d_.type, alpha_.view.numericType(),
                       beta_.view.numericType(), compute_type_, uint64_t(alpha_.view.indexType()),
                       uint64_t(beta_.view.indexType())});
    for (uint32_t g = 0; g < groups_; ++g)
        for (const GroupOperand* o : {&a_, &b_, &c_, &d_}) {
            const GroupMatrix& m = o->groups[g];
            k.insert(k.end(), {uint64_t(m.rows), uint64_t(m.cols), uint64_t(m.layout.col_major), uint64_t(m.layout.ld),
                               uint64_t(m.memory != nullptr), uint64_t(reinterpret_cast<uintptr_t>(m.memory) % 16)});
        }
    return k;
}

// ---------------------------------------------------------------- Primitives

namespace {

struct GroupedVariant {
    const char* name;
    FTrainNumericType input;
    int which;             // kernel index for groupedKernelFor
    gemm::Variant tile;    // the plain variant with the same tile: geometry and cost-model figures
};

// Registration order is also the fallback order when the GroupedCost Finder
// is disabled: largest tiles first.
constexpr GroupedVariant kGroupedVariants[] = {
    {"GroupedFp32Mfma16Gemm_256x256_Dma", FTRAIN_NUMERIC_TYPE_FP32, 4, gemm::Variant::kMfma16Dma256x256},
    {"GroupedFp32Mfma16Gemm_128x128_Dma", FTRAIN_NUMERIC_TYPE_FP32, 5, gemm::Variant::kMfma16Dma128x128},
    {"GroupedFp32Mfma16Gemm_64x128_Dma", FTRAIN_NUMERIC_TYPE_FP32, 6, gemm::Variant::kMfma16Dma64x128},
    {"GroupedFp32Mfma16Gemm_256x128", FTRAIN_NUMERIC_TYPE_FP32, 2, gemm::Variant::kMfma16_256x128},
    {"GroupedFp32Mfma16Gemm_128x256", FTRAIN_NUMERIC_TYPE_FP32, 3, gemm::Variant::kMfma16_128x256},
    {"GroupedFp32MfmaGemm_128x128", FTRAIN_NUMERIC_TYPE_FP32, 0, gemm::Variant::kMfma128x128},
    {"GroupedFp32MfmaGemm_64x64_Unaligned", FTRAIN_NUMERIC_TYPE_FP32, 1, gemm::Variant::kMfma64x64U},
    {"GroupedBf16MfmaGemm_256x256_Dma", FTRAIN_NUMERIC_TYPE_BF16, 3, gemm::Variant::kBf16MfmaDma256x256},
    {"GroupedBf16MfmaGemm_128x128_Dma", FTRAIN_NUMERIC_TYPE_BF16, 4, gemm::Variant::kBf16MfmaDma128x128},
    {"GroupedBf16MfmaGemm_256x256", FTRAIN_NUMERIC_TYPE_BF16, 2, gemm::Variant::kBf16Mfma256x256},
    {"GroupedBf16MfmaGemm_128x128", FTRAIN_NUMERIC_TYPE_BF16, 0, gemm::Variant::kBf16Mfma128x128},
    {"GroupedBf16MfmaGemm_64x64_Unaligned", FTRAIN_NUMERIC_TYPE_BF16, 1, gemm::Variant::kBf16Mfma64x64U},
    {"GroupedFp16MfmaGemm_256x256_Dma", FTRAIN_NUMERIC_TYPE_FP16, 3, gemm::Variant::kFp16MfmaDma256x256},
    {"GroupedFp16MfmaGemm_128x128_Dma", FTRAIN_NUMERIC_TYPE_FP16, 4, gemm::Variant::kFp16MfmaDma128x128},
    {"GroupedFp16MfmaGemm_256x256", FTRAIN_NUMERIC_TYPE_FP16, 2, gemm::Variant::kFp16Mfma256x256},
    {"GroupedFp16MfmaGemm_128x128", FTRAIN_NUMERIC_TYPE_FP16, 0, gemm::Variant::kFp16Mfma128x128},
    {"GroupedFp16MfmaGemm_64x64_Unaligned", FTRAIN_NUMERIC_TYPE_FP16, 1, gemm::Variant::kFp16Mfma64x64U},
};

// Workgroup slots of a group: its tiles rounded up to a multiple of 8, so
// that every group starts on an XCD boundary of the workgroup ids.
uint64_t groupSlots(uint64_t tiles) { return (tiles + 7) / 8 * 8; }

bool aligned(const void* p, uintptr_t n) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % n == 0; }
uint64_t ceilDiv(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

void check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        raise(FTRAIN_STATUS_INTERNAL_ERROR, "%s launch failed: %s", what, hipGetErrorString(e));
}

class GroupedGemmPrimitive final : public Primitive<GroupedGemmProblem> {
  public:
    explicit GroupedGemmPrimitive(const GroupedVariant& v) : v_(&v) {}

    const char* name() const noexcept override { return v_->name; }
    std::unique_ptr<PrimitiveBase> clone() const override { return std::make_unique<GroupedGemmPrimitive>(*v_); }
    uint64_t requiredWorkspaceBytes() const noexcept override { return 0; }

    Result isApplicable(const GroupedGemmProblem& p, const Constraints&) const override {
        if (p.computeType() != FTRAIN_NUMERIC_TYPE_FP32) return Result(FTRAIN_STATUS_UNSUPPORTED, "compute type is not fp32");
        const bool half = v_->input != FTRAIN_NUMERIC_TYPE_FP32;
        if (p.alpha().numericType() != FTRAIN_NUMERIC_TYPE_FP32 || p.beta().numericType() != FTRAIN_NUMERIC_TYPE_FP32)
            return Result(FTRAIN_STATUS_UNSUPPORTED, "alpha or beta is not fp32");
        if (p.alpha().indexType() != FTRAIN_INDEX_TYPE_CONTINUOUS || p.beta().indexType() != FTRAIN_INDEX_TYPE_CONTINUOUS)
            return Result(FTRAIN_STATUS_UNSUPPORTED, "an operand is not continuously indexed");
        if (!half) {
            for (const GroupOperand* o : {&p.a(), &p.b(), &p.c(), &p.d()})
                if (o->type != FTRAIN_NUMERIC_TYPE_FP32 && !o->groups.empty())
                    return Result(FTRAIN_STATUS_UNSUPPORTED, "an operand is not fp32");
        } else {
            const bool bf16 = v_->input == FTRAIN_NUMERIC_TYPE_BF16;
            if (p.a().type != v_->input || p.b().type != v_->input)
                return Result(FTRAIN_STATUS_UNSUPPORTED, bf16 ? "a or b is not bf16" : "a or b is not fp16");
            const FTrainNumericType cd = p.d().type;
            if ((cd != FTRAIN_NUMERIC_TYPE_FP32 && cd != v_->input) || (!nullOperand(p.c()) && p.c().type != cd))
                return Result(FTRAIN_STATUS_UNSUPPORTED, bf16 ? "c and d must both be fp32 or both bf16"
                                                              : "c and d must both be fp32 or both fp16");
        }
        const uintptr_t ea = half ? 2 : 4, ed = p.d().type == FTRAIN_NUMERIC_TYPE_FP32 ? 4 : 2;
        uint64_t tiles = 0;
        constexpr uint64_t kMax = std::numeric_limits<int32_t>::max();
        for (uint32_t g = 0; g < p.groups(); ++g) {
            if (p.emptyOutput(g)) continue;
            GemmLaunch l;
            if (const char* why = p.launch(g, l)) return Result(FTRAIN_STATUS_UNSUPPORTED, why);
            if (l.shape.k != 0 && (l.a == nullptr || l.b == nullptr))
                return Result(FTRAIN_STATUS_UNSUPPORTED, "a required operand address is null");
            if (l.d == nullptr) return Result(FTRAIN_STATUS_UNSUPPORTED, "a required operand address is null");
            const bool reads_ab = l.shape.k != 0;  // a k = 0 group reads neither a nor b
            if ((reads_ab && (!aligned(l.a, ea) || !aligned(l.b, ea))) || !aligned(l.c, ed) || !aligned(l.d, ed))
                return Result(FTRAIN_STATUS_UNSUPPORTED, "an operand address is not aligned to its element size");
            if (l.shape.m > kMax || l.shape.n > kMax || l.shape.k > kMax)
                return Result(FTRAIN_STATUS_UNSUPPORTED, "a dimension exceeds the 32-bit kernel limit");
            if (gemm::info(v_->tile).vec) {
                // 16-byte accesses along each matrix's contiguous dimension.
                const uint64_t w = half ? 8 : 4;
                const uint64_t a_run = l.ta ? l.shape.m : l.shape.k, b_run = l.tb ? l.shape.k : l.shape.n;
                if (reads_ab &&
                    (a_run % w != 0 || b_run % w != 0 || uint64_t(l.lda) % w != 0 || uint64_t(l.ldb) % w != 0))
                    return Result(FTRAIN_STATUS_UNSUPPORTED, "a group's contiguous extent or leading dimension does not fit 16-byte loads");
                if (reads_ab && (!aligned(l.a, 16) || !aligned(l.b, 16)))
                    return Result(FTRAIN_STATUS_UNSUPPORTED, "a group's a or b is not 16-byte aligned");
                if (!half && (l.shape.n % 4 != 0 || uint64_t(l.ldc) % 4 != 0 || uint64_t(l.ldd) % 4 != 0 ||
                              !aligned(l.c, 16) || !aligned(l.d, 16)))
                    return Result(FTRAIN_STATUS_UNSUPPORTED, "a group's c or d does not fit 128-bit stores");
            }
            if (v_->tile == gemm::Variant::kMfma16Dma256x256 &&
                (l.ta || l.tb || l.lda >= (int64_t(1) << 22) || l.ldb >= (int64_t(1) << 22) ||
                 l.ldc >= (int64_t(1) << 21) || l.ldd >= (int64_t(1) << 21)))
                return Result(FTRAIN_STATUS_UNSUPPORTED,
                              "a group is not row-major a and b with leading dimensions that fit 32-bit offsets (fp32 "
                              "DMA tiles)");
            if (v_->tile == gemm::Variant::kMfma16Dma64x128 && l.ta)
                return Result(FTRAIN_STATUS_UNSUPPORTED, "a group's a is column-major (the 64x128 DMA tile takes row-major a)");
            if ((v_->tile == gemm::Variant::kMfma16Dma128x128 || v_->tile == gemm::Variant::kMfma16Dma64x128) &&
                (l.lda >= (int64_t(1) << 22) || l.ldb >= (int64_t(1) << 22) || l.ldc >= (int64_t(1) << 21) ||
                 l.ldd >= (int64_t(1) << 21)))
                return Result(FTRAIN_STATUS_UNSUPPORTED,
                              "a group's leading dimension is too large for 32-bit offsets (fp32 DMA tiles)");
            if ((v_->tile == gemm::Variant::kBf16MfmaDma256x256 || v_->tile == gemm::Variant::kFp16MfmaDma256x256 ||
                 v_->tile == gemm::Variant::kBf16MfmaDma128x128 || v_->tile == gemm::Variant::kFp16MfmaDma128x128) &&
                (l.lda >= (int64_t(1) << 23) || l.ldb >= (int64_t(1) << 23) || l.ldc >= (int64_t(1) << 21) ||
                 l.ldd >= (int64_t(1) << 21)))
                return Result(FTRAIN_STATUS_UNSUPPORTED,
                              "a group's leading dimension is too large for 32-bit offsets (DMA tiles)");
            const gemm::VariantInfo& vi = gemm::info(v_->tile);
            tiles += groupSlots(ceilDiv(l.shape.m, vi.bm) * ceilDiv(l.shape.n, vi.bn));
            if (tiles > kMax) return Result(FTRAIN_STATUS_UNSUPPORTED, "the tile count exceeds the grid limit");
        }
        return Result{};
    }

    void configure(const GroupedGemmProblem& p) override {
        const float alpha  = *static_cast<const float*>(p.alpha().memory());
        const float beta   = *static_cast<const float*>(p.beta().memory());
        const bool half    = v_->input != FTRAIN_NUMERIC_TYPE_FP32;
        const bool cd_half = p.d().type != FTRAIN_NUMERIC_TYPE_FP32;
        for (Bucket& bk : buckets_) bk = Bucket{};
        // Per bucket: every group's b (the launch streams them all), the deepest k, the tile rows and
        // the groups, for the L2 prefetch of b (gemm::prefetchB).
        uint64_t b_bytes[4] = {0, 0, 0, 0}, max_k[4] = {0, 0, 0, 0}, tile_rows[4] = {0, 0, 0, 0}, groups[4] = {0, 0, 0, 0};
        for (uint32_t g = 0; g < p.groups(); ++g) {
            if (p.emptyOutput(g)) continue;
            GemmLaunch l;
            if (const char* why = p.launch(g, l)) raise(FTRAIN_STATUS_UNSUPPORTED, "%s", why);
            // Groups are launched per operand orientation (one kernel
            // instantiation each); a degenerate matrix may read as either.
            const int o      = (l.ta ? 1 : 0) + (l.tb ? 2 : 0);
            Bucket& bk       = buckets_[o];
            b_bytes[o] += l.shape.k * l.shape.n * (half ? 2 : 4);
            max_k[o] = std::max<uint64_t>(max_k[o], l.shape.k);
            const gemm::VariantInfo& vi = gemm::info(v_->tile);
            const int32_t tm = int32_t(ceilDiv(l.shape.m, vi.bm)), tn = int32_t(ceilDiv(l.shape.n, vi.bn));
            tile_rows[o] += uint64_t(tm);
            groups[o] += 1;
            bk.tile_start.push_back(bk.tiles);
            bk.tiles += int32_t(groupSlots(uint64_t(tm) * uint64_t(tn)));
            const int32_t m = int32_t(l.shape.m), n = int32_t(l.shape.n), k = int32_t(l.shape.k);
            if (half)
                bk.half_params.push_back(HalfGemmParams{l.a, l.b, l.c, l.d, alpha, beta, m, n, k, k, tm, tn, l.lda,
                                                        l.ldb, l.ldc, l.ldd, int32_t(cd_half)});
            else
                bk.params.push_back(GemmParams{static_cast<const float*>(l.a), static_cast<const float*>(l.b),
                                               static_cast<const float*>(l.c), static_cast<float*>(l.d), alpha, beta,
                                               m, n, k, k, tm, tn, l.lda, l.ldb, l.ldc, l.ldd});
        }
        for (int o = 0; o < 4; ++o)
            if (buckets_[o].tiles > 0) {
                buckets_[o].kernel  = gemm::groupedKernelFor(v_->input, v_->which, o & 1, o & 2,
                                                              gemm::prefetchB(b_bytes[o], max_k[o],
                                                                              double(tile_rows[o]) / double(groups[o])));
                buckets_[o].threads = gemm::info(v_->tile).threads;
            }
        table_.reset();
    }

    // The per-group parameter tables live on the device for the Plan's
    // lifetime.  They are uploaded here, at Plan creation, with blocking
    // copies, so executions on any stream find them complete and every
    // execution, the first included, only launches kernels (and can be
    // captured).  Layout per orientation bucket: parameters, then tile
    // starts (16-byte aligned sections).
    void prepare(bool) override {
        if (table_) return;
        const bool half = v_->input != FTRAIN_NUMERIC_TYPE_FP32;
        size_t total = 0;
        for (Bucket& bk : buckets_) {
            if (bk.tiles == 0) continue;
            bk.param_off = total;
            total += ((half ? bk.half_params.size() * sizeof(HalfGemmParams) : bk.params.size() * sizeof(GemmParams)) + 15) / 16 * 16;
            bk.start_off = total;
            total += (bk.tile_start.size() * sizeof(int32_t) + 15) / 16 * 16;
        }
        if (total == 0) return;
        void* buf = nullptr;
        if (hipMalloc(&buf, total) != hipSuccess) {
            (void)hipGetLastError();
            raise(FTRAIN_STATUS_OUT_OF_MEMORY, "%s: device parameter table of %zu bytes", v_->name, total);
        }
        std::shared_ptr<void> table(buf, [](void* q) { (void)hipFree(q); });
        for (const Bucket& bk : buckets_) {
            if (bk.tiles == 0) continue;
            const void* host = half ? static_cast<const void*>(bk.half_params.data()) : static_cast<const void*>(bk.params.data());
            const size_t bytes = half ? bk.half_params.size() * sizeof(HalfGemmParams) : bk.params.size() * sizeof(GemmParams);
            check(hipMemcpy(static_cast<char*>(buf) + bk.param_off, host, bytes, hipMemcpyHostToDevice), v_->name);
            check(hipMemcpy(static_cast<char*>(buf) + bk.start_off, bk.tile_start.data(),
                            bk.tile_start.size() * sizeof(int32_t), hipMemcpyHostToDevice),
                  v_->name);
        }
        table_ = std::move(table);
    }

  protected:
    void run(const Resources& r) override {
        const bool half = v_->input != FTRAIN_NUMERIC_TYPE_FP32;
        bool any = false;
        for (const Bucket& bk : buckets_) any = any || bk.tiles > 0;
        if (!any) return;
        if (!table_)
            raise(FTRAIN_STATUS_INTERNAL_ERROR, "%s: the Plan's device parameter table was never uploaded", v_->name);
        char* base = static_cast<char*>(table_.get());
        for (const Bucket& bk : buckets_) {
            if (bk.tiles == 0) continue;
            const auto* start    = reinterpret_cast<const int32_t*>(base + bk.start_off);
            const int32_t groups = static_cast<int32_t>(bk.tile_start.size());
            if (!half) {
                GroupedGemmArgs args{reinterpret_cast<const GemmParams*>(base + bk.param_off), start, groups};
                void* kargs[] = {&args};
                check(hipLaunchKernel(bk.kernel, dim3(uint32_t(bk.tiles)), dim3(uint32_t(bk.threads)), kargs, 0, r.stream), v_->name);
            } else {
                GroupedHalfArgs args{reinterpret_cast<const HalfGemmParams*>(base + bk.param_off), start, groups};
                void* kargs[] = {&args};
                check(hipLaunchKernel(bk.kernel, dim3(uint32_t(bk.tiles)), dim3(uint32_t(bk.threads)), kargs, 0, r.stream), v_->name);
            }
        }
    }

  private:
    // Non-empty groups of one operand orientation (index ta + 2*tb).
    struct Bucket {
        std::vector<GemmParams> params;
        std::vector<HalfGemmParams> half_params;
        std::vector<int32_t> tile_start;
        int32_t tiles       = 0;
        const void* kernel  = nullptr;
        int threads         = 256;
        size_t param_off    = 0;
        size_t start_off    = 0;
    };
    const GroupedVariant* v_;
    Bucket buckets_[4];
    std::shared_ptr<void> table_;
};

OperandKind kindA(GroupedKind k) { return k == GroupedKind::kBCD ? OperandKind::kTensorList : OperandKind::kGroupedTensor; }
OperandKind kindCD(GroupedKind k) { return k == GroupedKind::kAB ? OperandKind::kTensorList : OperandKind::kGroupedTensor; }
OperationKind opKind(GroupedKind k) {
    return k == GroupedKind::kABCD ? OperationKind::kGroupedABCDGemm
           : k == GroupedKind::kBCD ? OperationKind::kGroupedBCDGemm
                                    : OperationKind::kGroupedABGemm;
}

}  // namespace

template <GroupedKind K>
const typename GroupedGemmFamily<K>::Roles& GroupedGemmFamily<K>::roles() {
    // Operands in the reference's port order (operation/gemm.hpp:80-150):
    // inputs a, b, c, alpha, beta; output d.
    static const Roles r = [] {
        PatternBuilder pb;
        const uint64_t a     = pb.addOperand(kindA(K));
        const uint64_t b     = pb.addOperand(OperandKind::kGroupedTensor);
        const uint64_t c     = pb.addOperand(kindCD(K));
        const uint64_t alpha = pb.addOperand(OperandKind::kTensor);
        const uint64_t beta  = pb.addOperand(OperandKind::kTensor);
        const uint64_t d     = pb.addOperand(kindCD(K));
        const uint64_t op    = pb.addOperation(OpNode{opKind(K), {a, b, c, alpha, beta}, {d}});
        return Roles{pb.build(), a, b, c, d, alpha, beta, op};
    }();
    return r;
}

template <GroupedKind K>
std::vector<std::shared_ptr<const Primitive<GroupedGemmProblem>>> GroupedGemmFamily<K>::makeRecords() {
    std::vector<std::shared_ptr<const Primitive<GroupedGemmProblem>>> records;
    for (const GroupedVariant& v : kGroupedVariants) records.push_back(std::make_shared<GroupedGemmPrimitive>(v));
    return records;
}

template <GroupedKind K>
GroupedGemmProblem GroupedGemmFamily<K>::makeProblem(const Args& args) {
    const Roles& r = roles();
    auto tensor    = [&](uint64_t id) { return std::get<Tensor>(*args.operand(id)); };
    return GroupedGemmProblem(K, *args.operand(r.a), *args.operand(r.b), *args.operand(r.c), *args.operand(r.d),
                              tensor(r.alpha), tensor(r.beta), args.operation(r.op)->compute_type);
}

template struct GroupedGemmFamily<GroupedKind::kABCD>;
template struct GroupedGemmFamily<GroupedKind::kBCD>;
template struct GroupedGemmFamily<GroupedKind::kAB>;

std::vector<std::string> GroupedCostFinder::candidates(const GroupedGemmProblem& problem,
                                                       const Constraints& constraints) {
    std::vector<GemmShape> shapes;
    bool has_c = false;
    for (uint32_t g = 0; g < problem.groups(); ++g) {
        if (problem.emptyOutput(g)) continue;
        GemmLaunch l;
        if (problem.launch(g, l) != nullptr) continue;
        shapes.push_back(l.shape);
        has_c = has_c || l.c != nullptr;
    }
    const int cus = gemm::computeUnits(constraints.device());
    std::vector<std::pair<double, const char*>> ranked;
    for (const GroupedVariant& v : kGroupedVariants)
        if (v.input == problem.a().type) ranked.emplace_back(gemm::groupedMicros(v.tile, shapes, has_c, cus), v.name);
    std::stable_sort(ranked.begin(), ranked.end(), [](const auto& x, const auto& y) { return x.first < y.first; });
    std::vector<std::string> names;
    for (const auto& r : ranked) names.emplace_back(r.second);
    return names;
}

std::vector<std::shared_ptr<OpsEngineBase>> groupedEngines() {
    return {std::make_shared<OpsEngine<GroupedGemmFamily<GroupedKind::kABCD>, GroupedCostFinder>>(),
            std::make_shared<OpsEngine<GroupedGemmFamily<GroupedKind::kBCD>, GroupedCostFinder>>(),
            std::make_shared<OpsEngine<GroupedGemmFamily<GroupedKind::kAB>, GroupedCostFinder>>()};
}

}  // namespace ftrain
